"""CPU fp32 restatement of the reference's batch-1 Qwen3 decode step.

TEST INFRASTRUCTURE ONLY. This module is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The product path (``qwen0.6b_amd/``) never imports or calls it.

The reference has no CPU or fp32 path of its own: its only correctness check
(Model/benchmark.py:128-246) compares the CUDA megakernel with HuggingFace
Qwen3 on real weights. This module restates that arithmetic in plain fp32 on
the CPU, on the fp16-valued weights the GPU path uses, following:

* op order of one token step: Tools/megakernel/megakernel.cu:763-920
  (embedding gather 791-796, input RMSNorm 807-847, QKV 242-291, q/k RMSNorm
  *before* RoPE 345-434, GQA attention with kv head = q head // 2 479,
  residual + o_proj 581-610, post-attention RMSNorm 617-638, SiLU(gate)*up
  643-675, down + residual 682-707, final RMSNorm 893-919, tied lm_head +
  argmax 1001-1144);
* RMSNorm ``x * rsqrt(mean(x^2) + eps) * w`` with eps = 1e-6
  (Tools/megakernel/megakernel.cu:79; HF Qwen3RMSNorm);
* rotate-half RoPE over the fp16 cos/sin tables the reference builds in
  Model/Qwen06B_architecture.py:134-142 (dims i and i+64 share a frequency,
  Tools/megakernel/megakernel.cu:363-381);
* attention scale 1/sqrt(128) (Model/Qwen06B_architecture.py:229), softmax
  over positions 0..pos inclusive (cache_len = position + 1,
  Tools/megakernel/megakernel.cu:859);
* greedy argmax over the tied embedding (Model/Qwen06B_architecture.py:167);
  exact ties resolve to the lowest index (torch.argmax).

Where the reference rounds intermediates to fp16 (s_norm, q/k/v, attn_out,
the residual stream) this restatement keeps fp32: it is the fp32 reference
the device path is measured against, with the tolerances stated in the tests.

``Oracle.forward`` runs a whole id sequence at once (a causal prefill): the
same per-position arithmetic as ``Oracle.step``, batched over positions, which
is what the reference's prefill computes one ``step`` at a time
(Model/Qwen06B_architecture.py:346-347).

Pinned by tests/test_oracle.py: closed forms for every function below, float64
brute force for the MLP block and the top-2 gap, and an end-to-end comparison
with the third-party HuggingFace ``Qwen3ForCausalLM`` (transformers, present in
the image) on a small configuration, for both ``step`` and ``forward``.
"""

from __future__ import annotations

import math

import numpy as np
import torch

EPS = 1e-6


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """RMSNorm over the last dim (Tools/megakernel/megakernel.cu:807-847, 617-638, 893-919)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: torch.Tensor, cos_row: torch.Tensor, sin_row: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE for one position (Tools/megakernel/megakernel.cu:363-381).

    ``out[i] = x[i] c[i] - x[i+64] s[i]`` for i < 64 and
    ``out[i] = x[i] c[i] + x[i-64] s[i]`` for i >= 64.
    """
    return x * cos_row + rotate_half(x) * sin_row


def gqa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Decode attention for one query position (Tools/megakernel/megakernel.cu:457-552).

    q: [Hq, D]; k, v: [Hkv, T, D] holding positions 0..T-1. Query head h reads
    kv head ``h // (Hq // Hkv)`` (megakernel.cu:479). Returns [Hq, D].
    """
    hq, d = q.shape
    hkv = k.shape[0]
    group = hq // hkv
    kk = k.repeat_interleave(group, dim=0)  # [Hq, T, D]
    vv = v.repeat_interleave(group, dim=0)
    scores = torch.einsum("hd,htd->ht", q, kk) * scale
    p = torch.softmax(scores, dim=-1)
    return torch.einsum("ht,htd->hd", p, vv)


def swiglu_mlp(x: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, wd: torch.Tensor) -> torch.Tensor:
    """``down(silu(gate x) * up x)`` (Tools/megakernel/megakernel.cu:643-707)."""
    g = wg @ x
    u = wu @ x
    return wd @ (torch.nn.functional.silu(g) * u)


def mlp_block(x, post_norm_w, wg, wu, wd, eps: float = EPS):
    """One MLP half-layer with its residual: ``x + mlp(rmsnorm(x))``.

    The isolated MLP workload: RMSNorm, gate/up GEMV, SiLU*up, down GEMV and
    the residual add (Tools/megakernel/megakernel.cu:617-707).
    """
    h = rms_norm(x, post_norm_w, eps)
    return x + swiglu_mlp(h, wg, wu, wd)


def lm_head_logits(w: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    """``W h`` in fp32 (Tools/megakernel/megakernel.cu:1001-1060). h: [H] or [H, B]."""
    return w @ h


def argmax_lowest(logits: torch.Tensor) -> int:
    """Greedy token: first index of the maximum (NaN never wins)."""
    x = torch.nan_to_num(logits, nan=-math.inf)
    return int(torch.argmax(x))


def top2_gap(logits: torch.Tensor) -> float:
    """Largest logit minus the second largest (0 for an exact tie). Decides which
    greedy steps are near-ties (gap < 1e-2) and exempt from the token check."""
    v = torch.topk(logits.float(), 2).values
    return float(v[0] - v[1])


class Oracle:
    """Stateful fp32 decoder over one synthetic model (host memory).

    ``hw`` is a ``qwen_weights.HostWeights``. ``rope="fp16"`` uses the fp16
    cos/sin tables the reference hands to its kernel; ``rope="fp32"`` rebuilds
    them in fp32 (used to compare against HuggingFace, which never rounds them).
    """

    def __init__(self, hw, rope: str = "fp16"):
        s = hw.shape
        self.shape = s
        f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).float()
        self.embed = f32(hw.embed)
        lm = getattr(hw, "lm_head", None)
        self.lm_head = self.embed if lm is None else f32(lm)
        self.layers = [[f32(t) for t in layer] for layer in hw.layers]
        self.final_norm = f32(hw.final_norm)
        if rope == "fp16":
            self.cos = f32(hw.cos)
            self.sin = f32(hw.sin)
        else:
            inv_freq = 1.0 / (s.rope_theta ** (torch.arange(0, s.head_dim, 2, dtype=torch.float32) / s.head_dim))
            freqs = torch.outer(torch.arange(s.max_seq, dtype=torch.float32), inv_freq)
            self.cos = torch.cos(freqs).repeat(1, 2)
            self.sin = torch.sin(freqs).repeat(1, 2)
        self.scale = 1.0 / math.sqrt(s.head_dim)
        self.k_cache = torch.zeros(s.layers, s.kv_heads, s.max_seq, s.head_dim)
        self.v_cache = torch.zeros_like(self.k_cache)

    def reset(self) -> None:
        self.k_cache.zero_()
        self.v_cache.zero_()

    @torch.no_grad()
    def step(self, token: int, pos: int, want_logits: bool = True) -> dict:
        """One decode step at ``pos``; writes K/V at ``pos`` and returns
        ``logits`` [V], ``hidden`` (final-layer residual before the final norm),
        ``norm_out`` (final-normed vector) and the greedy ``token``. With
        ``want_logits=False`` only the KV cache and ``hidden`` are produced."""
        s = self.shape
        assert 0 <= pos < s.max_seq
        x = self.embed[token].clone()
        cos, sin = self.cos[pos], self.sin[pos]
        for li, (w_in, wq, wk, wv, w_qn, w_kn, wo, w_post, wg, wu, wd) in enumerate(self.layers):
            h = rms_norm(x, w_in)
            q = (wq @ h).view(s.q_heads, s.head_dim)
            k = (wk @ h).view(s.kv_heads, s.head_dim)
            v = (wv @ h).view(s.kv_heads, s.head_dim)
            q = apply_rope(rms_norm(q, w_qn), cos, sin)
            k = apply_rope(rms_norm(k, w_kn), cos, sin)
            self.k_cache[li, :, pos] = k
            self.v_cache[li, :, pos] = v
            attn = gqa_attention(q, self.k_cache[li, :, : pos + 1], self.v_cache[li, :, : pos + 1], self.scale)
            x = x + wo @ attn.reshape(-1)
            x = x + swiglu_mlp(rms_norm(x, w_post), wg, wu, wd)
        if not want_logits:
            return dict(hidden=x)
        norm_out = rms_norm(x, self.final_norm)
        logits = lm_head_logits(self.lm_head, norm_out)
        return dict(logits=logits, hidden=x, norm_out=norm_out, token=argmax_lowest(logits))

    @torch.no_grad()
    def forward(self, ids: list, start: int = 0, logits_at=()) -> dict:
        """Causal forward of ``ids`` at positions ``start .. start + n - 1`` in one batch
        (every position attends to the cache at positions ``< start`` and to the ids
        before it). Writes K/V at those positions, as ``n`` calls of ``step`` would.

        Returns ``hidden`` [n, H] (each position's final-layer residual before the final
        norm) and, for the positions listed in ``logits_at``, ``logits`` [m, V],
        ``norm_out`` [m, H] and the greedy ``tokens``."""
        s = self.shape
        n = len(ids)
        assert n >= 1 and start >= 0 and start + n <= s.max_seq
        pos = torch.arange(start, start + n)
        x = self.embed[torch.tensor(ids, dtype=torch.long)].clone()  # [n, H]
        cos, sin = self.cos[pos][:, None, :], self.sin[pos][:, None, :]  # [n, 1, D]
        total = start + n
        # query i (position start + i) sees keys 0 .. start + i
        mask = torch.arange(total)[None, :] > pos[:, None]  # [n, total]
        group = s.q_heads // s.kv_heads
        for li, (w_in, wq, wk, wv, w_qn, w_kn, wo, w_post, wg, wu, wd) in enumerate(self.layers):
            h = rms_norm(x, w_in)
            q = (h @ wq.T).view(n, s.q_heads, s.head_dim)
            k = (h @ wk.T).view(n, s.kv_heads, s.head_dim)
            v = (h @ wv.T).view(n, s.kv_heads, s.head_dim)
            q = apply_rope(rms_norm(q, w_qn), cos, sin)
            k = apply_rope(rms_norm(k, w_kn), cos, sin)
            self.k_cache[li, :, start:total] = k.transpose(0, 1)
            self.v_cache[li, :, start:total] = v.transpose(0, 1)
            kk = self.k_cache[li, :, :total].repeat_interleave(group, dim=0)  # [Hq, total, D]
            vv = self.v_cache[li, :, :total].repeat_interleave(group, dim=0)
            sc = torch.matmul(q.transpose(0, 1), kk.transpose(1, 2)) * self.scale  # [Hq, n, total]
            sc = sc.masked_fill(mask[None], float("-inf"))
            attn = torch.matmul(torch.softmax(sc, dim=-1), vv)  # [Hq, n, D]
            x = x + attn.transpose(0, 1).reshape(n, s.q_size) @ wo.T
            hh = rms_norm(x, w_post)
            x = x + (torch.nn.functional.silu(hh @ wg.T) * (hh @ wu.T)) @ wd.T
        out = dict(hidden=x)
        idx = [int(p) - start for p in logits_at]
        if idx:
            assert all(0 <= i < n for i in idx)
            norm_out = rms_norm(x[idx], self.final_norm)
            logits = norm_out @ self.lm_head.T
            out.update(norm_out=norm_out, logits=logits, tokens=[argmax_lowest(r) for r in logits])
        return out

    def greedy(self, prompt: list, n_new: int, start: int = 0) -> dict:
        """Prefill ``prompt[:-1]`` step by step, then ``n_new`` greedy steps
        starting from ``prompt[-1]`` (Model/Qwen06B_architecture.py:343-382).

        Returns per generated step the input token, the output token, the
        top-2 gap and the step's outputs (logits, hidden, norm_out)."""
        pos = start
        for t in prompt[:-1]:
            self.step(t, pos, want_logits=False)
            pos += 1
        tok = prompt[-1]
        steps = []
        for _ in range(n_new):
            out = self.step(tok, pos)
            out["input"] = tok
            out["pos"] = pos
            out["gap"] = top2_gap(out["logits"])
            steps.append(out)
            tok = out["token"]
            pos += 1
        return dict(steps=steps, tokens=[o["token"] for o in steps])
