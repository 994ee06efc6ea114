"""Pins the CPU oracle before anything is compared with it.

Each oracle function is checked against something that does not restate its
own formula: closed forms and invariants (RMSNorm of constant vectors, RoPE
identity/isometry/relative-position property, attention with one position or
identical keys, a planted argmax row), float64 brute force on tiny shapes, and
an end-to-end comparison with the third-party HuggingFace Qwen3ForCausalLM.
The reference itself ships no golden vectors usable here: its only published
tokens (README.md:452-461) need the real checkpoint.
"""

import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import qwen3_oracle as orc
import qwen_weights as qw

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TINY = qw.QwenShape(hidden=64, inter=192, layers=3, q_heads=4, kv_heads=2, head_dim=16, vocab=512, max_seq=64)


def test_rms_norm_closed_forms():
    n = 1024
    w = torch.ones(n)
    for c in (3.0, -0.25, 1e-2):
        out = orc.rms_norm(torch.full((n,), c), w)
        expect = math.copysign(1.0, c) / math.sqrt(1.0 + orc.EPS / (c * c))
        assert torch.allclose(out, torch.full((n,), expect), rtol=1e-6, atol=0)
    assert torch.count_nonzero(orc.rms_norm(torch.zeros(n), w)) == 0
    # unit RMS output and weight applied elementwise
    x = torch.randn(n, generator=torch.Generator().manual_seed(0)) * 5
    out = orc.rms_norm(x, w)
    assert abs(float(out.pow(2).mean()) - 1.0) < 1e-5
    w2 = torch.arange(n, dtype=torch.float32)
    assert torch.allclose(orc.rms_norm(x, w2), out * w2, rtol=1e-6)
    # per-row normalisation over the last dim only (q/k heads)
    h = torch.randn(4, 128)
    rows = orc.rms_norm(h, torch.ones(128))
    for r in range(4):
        assert torch.allclose(rows[r], orc.rms_norm(h[r], torch.ones(128)))


def test_rope_tables_match_float64_math():
    cos, sin = qw.rope_tables_fp16(2048, 128, 1e6)
    pos = np.arange(2048, dtype=np.float64)[:, None]
    inv = 1.0 / (1e6 ** (np.arange(0, 128, 2, dtype=np.float64) / 128))
    ang = np.concatenate([pos * inv, pos * inv], axis=1)
    # fp32 angle math vs float64: within one fp16 ulp of [-1, 1] values (~1e-3);
    # a wrong theta (1e4) or a non-repeated half would be off by O(1).
    assert np.max(np.abs(cos.float().numpy() - np.cos(ang))) < 1.5e-3
    assert np.max(np.abs(sin.float().numpy() - np.sin(ang))) < 1.5e-3
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)
    assert torch.equal(cos[:, :64], cos[:, 64:])


def test_rope_identity_isometry_and_relative_position():
    d = 128
    g = torch.Generator().manual_seed(1)
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float64) / d))

    def tab(p):
        a = torch.cat([p * inv, p * inv])
        return torch.cos(a), torch.sin(a)

    q = torch.randn(d, generator=g, dtype=torch.float64)
    k = torch.randn(d, generator=g, dtype=torch.float64)
    c0, s0 = tab(0)
    assert torch.allclose(orc.apply_rope(q, c0, s0), q)
    c, s = tab(777)
    rq = orc.apply_rope(q, c, s)
    # each (i, i+64) pair is rotated: pair norms are preserved
    assert torch.allclose(rq[:64] ** 2 + rq[64:] ** 2, q[:64] ** 2 + q[64:] ** 2)
    # explicit rotation on a basis vector: e_i -> (cos, +sin) on (i, i+64)
    e = torch.zeros(d, dtype=torch.float64)
    e[5] = 1
    r = orc.apply_rope(e, c, s)
    assert abs(r[5] - c[5]) < 1e-12 and abs(r[69] - s[5]) < 1e-12
    # <R_m q, R_n k> depends only on m - n
    def dot(m, n):
        cm, sm = tab(m)
        cn, sn = tab(n)
        return float(orc.apply_rope(q, cm, sm) @ orc.apply_rope(k, cn, sn))

    assert abs(dot(10, 3) - dot(1007, 1000)) < 1e-9
    assert abs(dot(10, 3) - dot(3, 10)) > 1e-6  # and is not symmetric


def test_attention_closed_forms_and_gqa_mapping():
    g = torch.Generator().manual_seed(2)
    hq, hkv, d = 4, 2, 16
    q = torch.randn(hq, d, generator=g, dtype=torch.float64)
    # one position: output is v of the mapped kv head
    k1 = torch.randn(hkv, 1, d, generator=g, dtype=torch.float64)
    v1 = torch.randn(hkv, 1, d, generator=g, dtype=torch.float64)
    out = orc.gqa_attention(q, k1, v1, 0.25)
    for h in range(hq):
        assert torch.allclose(out[h], v1[h // 2, 0])
    # identical keys: uniform weights -> mean of V
    T = 9
    kk = torch.randn(hkv, 1, d, generator=g, dtype=torch.float64).expand(hkv, T, d).contiguous()
    vv = torch.randn(hkv, T, d, generator=g, dtype=torch.float64)
    out = orc.gqa_attention(q, kk, vv, 0.1)
    for h in range(hq):
        assert torch.allclose(out[h], vv[h // 2].mean(0))
    # brute force softmax in float64 with explicit loops
    kr = torch.randn(hkv, T, d, generator=g, dtype=torch.float64)
    out = orc.gqa_attention(q, kr, vv, 0.3)
    for h in range(hq):
        sc = [float(q[h] @ kr[h // 2, t]) * 0.3 for t in range(T)]
        m = max(sc)
        e = [math.exp(x - m) for x in sc]
        ref = sum(e[t] * vv[h // 2, t] for t in range(T)) / sum(e)
        assert torch.allclose(out[h], ref)


def test_swiglu_and_mlp_block_brute_force():
    g = torch.Generator().manual_seed(3)
    h, i = 8, 12
    x = torch.randn(h, generator=g, dtype=torch.float64)
    wg = torch.randn(i, h, generator=g, dtype=torch.float64)
    wu = torch.randn(i, h, generator=g, dtype=torch.float64)
    wd = torch.randn(h, i, generator=g, dtype=torch.float64)
    ref = torch.zeros(h, dtype=torch.float64)
    for r in range(h):
        acc = 0.0
        for j in range(i):
            gj = sum(float(wg[j, c] * x[c]) for c in range(h))
            uj = sum(float(wu[j, c] * x[c]) for c in range(h))
            acc += float(wd[r, j]) * (gj / (1.0 + math.exp(-gj))) * uj
        ref[r] = acc
    assert torch.allclose(orc.swiglu_mlp(x, wg, wu, wd), ref)
    w = torch.ones(h, dtype=torch.float64)
    assert torch.allclose(orc.mlp_block(x, w, wg, wu, wd), x + orc.swiglu_mlp(orc.rms_norm(x, w), wg, wu, wd))


def test_argmax_planted_ties_and_nan():
    g = torch.Generator().manual_seed(4)
    W = torch.randn(5000, 64, generator=g)
    for row in (0, 17, 4999):
        h = W[row] * 10
        assert orc.argmax_lowest(orc.lm_head_logits(W, h)) == row
    x = torch.tensor([1.0, 3.0, 3.0, 2.0])
    assert orc.argmax_lowest(x) == 1
    x = torch.tensor([float("nan"), 1.0, float("nan"), 0.5])
    assert orc.argmax_lowest(x) == 1


def _hf_model(hw, shape):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen3Config(
        vocab_size=shape.vocab,
        hidden_size=shape.hidden,
        intermediate_size=shape.inter,
        num_hidden_layers=shape.layers,
        num_attention_heads=shape.q_heads,
        num_key_value_heads=shape.kv_heads,
        head_dim=shape.head_dim,
        max_position_embeddings=shape.max_seq,
        rms_norm_eps=shape.eps,
        rope_parameters={"rope_type": "default", "rope_theta": shape.rope_theta},
        tie_word_embeddings=True,
        attention_bias=False,
    )
    model = transformers.Qwen3ForCausalLM(cfg).float().eval()
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).float()
    sd = {"model.embed_tokens.weight": f32(hw.embed), "model.norm.weight": f32(hw.final_norm)}
    names = ["input_layernorm", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
             "self_attn.q_norm", "self_attn.k_norm", "self_attn.o_proj", "post_attention_layernorm",
             "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
    for li, layer in enumerate(hw.layers):
        for n, t in zip(names, layer):
            sd[f"model.layers.{li}.{n}.weight"] = f32(t)
    sd["lm_head.weight"] = sd["model.embed_tokens.weight"]
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("lm_head" in m for m in missing)
    return model


@pytest.mark.parametrize("std", [0.02, 0.2])
def test_oracle_matches_huggingface_qwen3(std):
    """End-to-end: the oracle's step-by-step decode equals HF Qwen3's causal
    forward over the same ids (fp32 both, fp32 RoPE tables), and greedy tokens
    agree. Non-unit norm weights exercise every norm's weight multiply."""
    hw = qw.host_weights(seed=7, std=std, shape=TINY)
    rng = np.random.default_rng(11)
    for layer in hw.layers:
        for f in qw.NORM_FIELDS:
            layer[f] = (1.0 + 0.5 * rng.standard_normal(layer[f].shape)).astype(np.float16)
    hw.final_norm = (1.0 + 0.5 * rng.standard_normal(hw.final_norm.shape)).astype(np.float16)
    prompt = qw.synthetic_prompt(6, seed=5, vocab=TINY.vocab)
    oracle = orc.Oracle(hw, rope="fp32")
    run = oracle.greedy(prompt, n_new=10)
    ids = prompt + run["tokens"][:-1]
    model = _hf_model(hw, TINY)
    with torch.no_grad():
        logits = model(torch.tensor([ids])).logits[0]
    for i, st in enumerate(run["steps"]):
        ref = logits[len(prompt) - 1 + i]
        assert torch.allclose(st["logits"], ref, atol=2e-5, rtol=1e-5), (i, float((st["logits"] - ref).abs().max()))
        assert st["token"] == int(torch.argmax(ref))


def test_fp16_rope_tables_stay_close_to_fp32():
    hw = qw.host_weights(seed=7, std=0.2, shape=TINY)
    prompt = qw.synthetic_prompt(6, seed=5, vocab=TINY.vocab)
    a = orc.Oracle(hw, rope="fp16").greedy(prompt, 4)
    b = orc.Oracle(hw, rope="fp32").greedy(prompt, 4)
    for sa, sb in zip(a["steps"], b["steps"]):
        d = float((sa["logits"] - sb["logits"]).abs().max())
        assert 0 < d < 5e-2


def test_tiny_golden_fixture():
    """Regression pin: the committed tiny-config greedy run."""
    with open(os.path.join(GOLDEN, "tiny_decode.json")) as f:
        gold = json.load(f)
    hw = qw.host_weights(seed=gold["seed"], std=gold["std"], shape=TINY)
    assert hw.digest() == gold["weights_sha256"]
    run = orc.Oracle(hw).greedy(gold["prompt"], gold["n_new"])
    assert run["tokens"] == gold["tokens"]
    for st, top in zip(run["steps"], gold["top5"]):
        vals, idx = torch.topk(st["logits"], 5)
        assert idx.tolist() == top["idx"]
        assert np.allclose(vals.numpy(), top["val"], atol=1e-5)


@pytest.mark.slow
def test_full_model_golden_fixture():
    """Regression pin of the full-size synthetic model (seed 0) and the
    16-token-prompt greedy run of the end-to-end parity workload."""
    with open(os.path.join(GOLDEN, "c0_decode.json")) as f:
        gold = json.load(f)
    hw = qw.host_weights(seed=0, std=0.02)
    assert hw.digest() == gold["weights_sha256"]
    prompt = qw.synthetic_prompt(16, seed=1)
    assert prompt == gold["prompt"]
    n = gold["n_check"]
    run = orc.Oracle(hw).greedy(prompt, n)
    assert run["tokens"] == gold["tokens"][:n]
    for st, g in zip(run["steps"], gold["steps"][:n]):
        assert abs(st["gap"] - g["gap"]) < 1e-4
        vals, idx = torch.topk(st["logits"], 4)
        assert idx.tolist() == g["top4_idx"]
        assert np.allclose(vals.numpy(), g["top4_val"], atol=1e-4)
        assert np.allclose(st["hidden"][:16].numpy(), g["hidden16"], atol=1e-4)
