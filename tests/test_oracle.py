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


def test_mlp_block_brute_force_nonunit_norm_and_residual():
    """The isolated-MLP oracle against explicit float64 loops: RMSNorm written out
    (sum of squares, eps inside the root, per-element gain), SiLU as g / (1 + e^-g),
    the down projection and the residual add. A dropped gain, a missing residual or
    eps outside the root fails this."""
    g = torch.Generator().manual_seed(13)
    h, i = 16, 24
    x = torch.randn(h, generator=g, dtype=torch.float64) * 3
    wn = 1.0 + 0.5 * torch.randn(h, generator=g, dtype=torch.float64)
    wg = torch.randn(i, h, generator=g, dtype=torch.float64) * 0.3
    wu = torch.randn(i, h, generator=g, dtype=torch.float64) * 0.3
    wd = torch.randn(h, i, generator=g, dtype=torch.float64) * 0.3
    xs = [float(v) for v in x]
    rms = math.sqrt(sum(v * v for v in xs) / h + orc.EPS)
    hn = [xs[c] / rms * float(wn[c]) for c in range(h)]
    inter = []
    for j in range(i):
        gj = sum(float(wg[j, c]) * hn[c] for c in range(h))
        uj = sum(float(wu[j, c]) * hn[c] for c in range(h))
        inter.append(gj / (1.0 + math.exp(-gj)) * uj)
    ref = [xs[r] + sum(float(wd[r, j]) * inter[j] for j in range(i)) for r in range(h)]
    out = orc.mlp_block(x, wn, wg, wu, wd)
    assert torch.allclose(out, torch.tensor(ref, dtype=torch.float64), rtol=1e-12, atol=1e-12)
    # the gain is really applied: unit gain gives a different answer
    assert float((out - orc.mlp_block(x, torch.ones(h, dtype=torch.float64), wg, wu, wd)).abs().max()) > 1e-3


def test_top2_gap_closed_forms():
    """The near-tie exemption's gap: an exact tie is 0, otherwise max minus the
    runner-up (not minus the minimum, not the top-2 of the absolute values)."""
    assert orc.top2_gap(torch.tensor([1.0, 3.0, 3.0, 2.0])) == 0.0
    assert orc.top2_gap(torch.tensor([5.0, 1.0, 2.0])) == 3.0
    assert orc.top2_gap(torch.tensor([-1.0, -4.0])) == 3.0
    assert orc.top2_gap(torch.tensor([-7.0, 0.5, -0.25, 0.0])) == 0.5
    x = torch.randn(100000, generator=torch.Generator().manual_seed(6))
    x[4242] = float(x.max()) + 0.25
    ranked = sorted(x.tolist(), reverse=True)
    assert abs(orc.top2_gap(x) - (ranked[0] - ranked[1])) < 1e-6
    assert abs(orc.top2_gap(x) - 0.25) < 1e-6


def test_forward_matches_steps_and_is_chunkable():
    """The batched causal forward (prefill) against n single steps of the oracle on a
    model with non-unit norms and an untied lm_head: same K/V cache, hidden states
    and logits; and a forward split in two chunks equals one forward over all ids."""
    hw = qw.host_weights(seed=7, std=0.2, shape=TINY, norms="random", untied=True)
    ids = qw.synthetic_prompt(30, seed=5, vocab=TINY.vocab)
    a, b, c = orc.Oracle(hw), orc.Oracle(hw), orc.Oracle(hw)
    steps = [a.step(t, p) for p, t in enumerate(ids)]
    whole = b.forward(ids, logits_at=range(len(ids)))
    c.forward(ids[:11])
    tail = c.forward(ids[11:], start=11, logits_at=range(11, len(ids)))
    for p, st in enumerate(steps):
        # fp32 sums in another order: relative agreement of ~1e-6 on values of O(10)
        assert torch.allclose(whole["hidden"][p], st["hidden"], rtol=1e-5, atol=1e-4), p
        assert torch.allclose(whole["logits"][p], st["logits"], rtol=1e-5, atol=1e-4), p
        assert whole["tokens"][p] == st["token"]
    assert torch.allclose(a.k_cache, b.k_cache, rtol=1e-5, atol=1e-4)
    assert torch.allclose(a.v_cache, b.v_cache, rtol=1e-5, atol=1e-4)
    assert torch.allclose(b.k_cache, c.k_cache, rtol=1e-5, atol=1e-4)
    assert torch.allclose(tail["logits"], whole["logits"][11:], rtol=1e-5, atol=1e-4)
    # the untied lm_head is the one used: the tied embedding gives other logits
    tied = orc.lm_head_logits(b.embed, whole["norm_out"][-1])
    assert float((tied - whole["logits"][-1]).abs().max()) > 1e-2


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
    tied = hw.lm_head is None
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
        tie_word_embeddings=tied,
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
    sd["lm_head.weight"] = sd["model.embed_tokens.weight"] if tied else f32(hw.lm_head)
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("lm_head" in m for m in missing)
    if not tied:
        assert not missing
        assert torch.equal(model.lm_head.weight, f32(hw.lm_head))
    return model


@pytest.mark.parametrize("std,untied", [(0.02, False), (0.2, False), (0.2, True)])
def test_oracle_matches_huggingface_qwen3(std, untied):
    """End-to-end: the oracle's step-by-step decode and its batched forward both equal
    HF Qwen3's causal forward over the same ids (fp32 both, fp32 RoPE tables), and
    greedy tokens agree. Non-unit norm weights (distinct per layer and field) exercise
    every norm's weight multiply; the untied case, HF's separate lm_head."""
    hw = qw.host_weights(seed=7, std=std, shape=TINY, norms="random", untied=untied)
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
    fwd = orc.Oracle(hw, rope="fp32").forward(ids, logits_at=range(len(ids)))
    assert torch.allclose(fwd["logits"], logits, atol=2e-5, rtol=1e-5), float((fwd["logits"] - logits).abs().max())


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
