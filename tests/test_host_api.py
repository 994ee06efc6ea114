"""Host-side logic of the Qwen06B_architecture mirror, on the CPU.

A stub ``qwen_megakernel_C`` (test-only) stands in for the compiled module: its
decode / generate_nosync / generate_ex run the CPU oracle on a small model, so
position bookkeeping, prefill/generate sequencing, EOS handling, the pointer
table and the import-time ABI gate are checked without a GPU.
"""

import importlib.util
import os
import sys
import types

import numpy as np
import pytest
import torch

import qwen_weights as qw
from oracle import qwen3_oracle as orc
from oracle import sampling as sp

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MOD = os.path.join(REPO, "qwen0.6b_amd", "Qwen06B_architecture.py")
SMALL = qw.QwenShape(hidden=64, inter=192, layers=2, q_heads=4, kv_heads=2, head_dim=16, vocab=512, max_seq=2048)


def _load(stub, name):
    saved = sys.modules.get("qwen_megakernel_C")
    sys.modules["qwen_megakernel_C"] = stub
    try:
        spec = importlib.util.spec_from_file_location(name, MOD)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        return mod
    finally:
        if saved is None:
            sys.modules.pop("qwen_megakernel_C", None)
        else:
            sys.modules["qwen_megakernel_C"] = saved


class OracleStub(types.ModuleType):
    """Test double of the extension backed by the CPU oracle (small model)."""

    def __init__(self, hw):
        super().__init__("qwen_megakernel_C")
        self.oracle = orc.Oracle(hw)
        self.calls = []

    def abi_version(self):
        return 2

    def last_error(self):
        return 0

    def decode(self, token, *args):
        num_layers, position, max_seq, scale = args[-4:]
        self.calls.append(("decode", token, position))
        return torch.tensor([self.oracle.step(token, position)["token"]], dtype=torch.int32)

    def generate_nosync(self, first, n, *args):
        num_layers, start, max_seq, scale = args[-4:]
        self.calls.append(("generate_nosync", first, start, n))
        out, tok = [], first
        for s in range(n):
            tok = self.oracle.step(tok, start + s)["token"]
            out.append(tok)
        return torch.tensor(out, dtype=torch.int32)

    def generate_until(self, first, n, eos, *args):
        num_layers, start, max_seq, scale = args[-4:]
        self.calls.append(("generate_until", first, start, n, eos))
        out, tok = [], first
        for s in range(n):
            tok = self.oracle.step(tok, start + s)["token"]
            out.append(tok)
            if tok == eos:
                break
        count = len(out)
        return torch.tensor(out + [-1] * (n - count), dtype=torch.int32), torch.tensor([count], dtype=torch.int32)

    def generate_ex(self, first, n, forced, *args):
        num_layers, start, max_seq, scale = args[-4:]
        self.calls.append(("generate_ex", first, start, n))
        ids = forced.tolist()
        out = [self.oracle.step(ids[s], start + s)["token"] for s in range(n)]
        return torch.tensor(out, dtype=torch.int32)

    def generate_sampled(self, first, n, eos, *args):
        num_layers, start, max_seq, scale, temperature, top_k, top_p, seed = args[-8:]
        self.calls.append(("generate_sampled", first, start, n, eos))
        out, tok = [], first
        for s in range(n):
            logits = self.oracle.step(tok, start + s)["logits"].numpy()
            tok = sp.sample(logits, temperature, top_k, top_p, seed, start + s)
            out.append(tok)
            if tok == eos:
                break
        count = len(out)
        return torch.tensor(out + [-1] * (n - count), dtype=torch.int32), torch.tensor([count], dtype=torch.int32)

    def prefill(self, ids, *args):
        num_layers, start, max_seq, scale = args[-4:]
        ids = ids.tolist()
        self.calls.append(("prefill", start, len(ids)))
        self.oracle.forward(ids, start=start)


@pytest.fixture(scope="module")
def small_hw():
    return qw.host_weights(seed=3, std=0.2, shape=SMALL)


@pytest.fixture()
def qa_cpu(small_hw):
    stub = OracleStub(small_hw)
    mod = _load(stub, "qa_cpu_under_test")
    mod.DEVICE = "cpu"
    return mod, stub


def _weights(mod):
    # placeholder tensors: the stub ignores them; the Decoder only packs pointers
    lw = [torch.zeros(16, dtype=torch.float16) for _ in range(28 * 11)]
    e = torch.zeros(16, dtype=torch.float16)
    return dict(embed_weight=e, layer_weights=lw, final_norm_weight=e, lm_head_weight=e, cos_table=e, sin_table=e)


def test_import_gate_rejects_wrong_abi():
    stub = types.ModuleType("qwen_megakernel_C")
    stub.abi_version = lambda: 1
    stub.built_torch_version = lambda: "9.9"
    stub.decode = lambda *a: None
    with pytest.raises(RuntimeError, match="Expected ABI 2, got 1"):
        _load(stub, "qa_bad_abi")


def test_import_fails_loudly_without_decode_op():
    stub = types.ModuleType("qwen_megakernel_C")
    stub.abi_version = lambda: 2
    stub.generate_nosync = lambda *a: None
    with pytest.raises(RuntimeError, match="op 'decode' is unavailable.*Available extension ops: generate_nosync"):
        _load(stub, "qa_no_decode")


def test_pack_layer_weights(qa_cpu):
    mod, _ = qa_cpu
    lw = [torch.zeros(8, dtype=torch.float16) for _ in range(2 * 11)]
    t = mod._pack_layer_weights(lw)
    assert t.dtype == torch.int64 and t.numel() == 24 and t.data_ptr() % 16 == 0
    for li in range(2):
        for j in range(11):
            assert int(t[li * 12 + j]) == lw[li * 11 + j].data_ptr()
        assert int(t[li * 12 + 11]) == 0
    with pytest.raises(AssertionError, match="Expected 33 weight tensors .* got 42"):
        mod._pack_layer_weights(lw[:-1] + lw[:-1])  # 42 tensors: not a multiple of 11


def test_step_positions_and_tokens(qa_cpu, small_hw):
    mod, stub = qa_cpu
    dec = mod.Decoder(weights=_weights(mod), verbose=False)
    ref = orc.Oracle(small_hw).greedy([5, 9, 17], 4)
    assert dec.position == 0
    for t in (5, 9):
        dec.step(t)
    tok = 17
    got = []
    for _ in range(4):
        tok = dec.step(tok)
        got.append(tok)
    assert got == ref["tokens"]
    assert dec.position == 6
    assert [c[2] for c in stub.calls] == list(range(6))
    dec.reset()
    assert dec.position == 0 and int(dec._k_cache.abs().sum()) == 0


def test_generate_ids_prefill_then_nosync(qa_cpu, small_hw):
    mod, stub = qa_cpu
    dec = mod.Decoder(weights=_weights(mod), verbose=False)
    prompt = [3, 1, 4, 1, 5]
    out = dec.generate_ids(prompt, 6)
    ref = orc.Oracle(small_hw).greedy(prompt, 6)
    assert out == ref["tokens"]
    # prefill covers positions 0..n-2 in one batched launch, generation starts at n-1
    assert stub.calls == [("prefill", 0, 4), ("generate_nosync", 5, 4, 6)]
    assert dec.position == len(prompt) - 1 + 6


def test_prefill_returns_token_after_prompt(qa_cpu, small_hw):
    """prefill(ids): the batched launch over ids[:-1], then one decode step of ids[-1]
    whose greedy token is returned; batched=False teacher forces every id instead."""
    mod, stub = qa_cpu
    prompt = [7, 2, 9, 4, 4, 1]
    ref = orc.Oracle(small_hw).greedy(prompt, 1)["tokens"][0]
    dec = mod.Decoder(weights=_weights(mod), verbose=False)
    stub.calls.clear()
    assert dec.prefill(prompt) == ref
    assert stub.calls == [("prefill", 0, 5), ("generate_ex", 1, 5, 1)]
    assert dec.position == len(prompt)
    stub.oracle.reset()
    dec.reset()
    stub.calls.clear()
    assert dec.prefill(prompt, batched=False) == ref
    assert stub.calls == [("generate_ex", 7, 0, 6)]
    assert dec.position == len(prompt)


def test_generate_text_truncates_at_eos(qa_cpu, small_hw):
    mod, stub = qa_cpu
    ref = orc.Oracle(small_hw).greedy([7, 8], 5)["tokens"]

    class Tok:
        eos_token_id = ref[2]

        def encode(self, text, add_special_tokens=True):
            return [7, 8]

        def decode(self, ids, skip_special_tokens=True):
            return ",".join(map(str, ids))

    dec = mod.Decoder(weights=_weights(mod), tokenizer=Tok(), verbose=False)
    first = ref.index(ref[2])
    assert dec.generate("hi", 5) == ",".join(map(str, ref[:first]))


def test_generate_ids_stops_at_eos(qa_cpu, small_hw):
    mod, stub = qa_cpu
    prompt = [3, 1, 4, 1, 5]
    ref = orc.Oracle(small_hw).greedy(prompt, 8)["tokens"]
    k = next(i for i in range(2, 8) if ref[i] not in ref[:i])
    dec = mod.Decoder(weights=_weights(mod), verbose=False)
    out = dec.generate_ids(prompt, 8, eos_token_id=ref[k])
    assert out == ref[:k + 1]
    assert stub.calls[-1] == ("generate_until", 5, 4, 8, ref[k])
    assert dec.position == len(prompt) - 1 + k + 1


def _sampled_ref(hw, prompt, n, eos=None, **kw):
    o = orc.Oracle(hw)
    o.forward(prompt[:-1])
    out, tok = [], prompt[-1]
    for s in range(n):
        pos = len(prompt) - 1 + s
        tok = sp.sample(o.step(tok, pos)["logits"].numpy(), kw["temperature"], kw["top_k"], kw["top_p"],
                        kw["seed"], pos)
        out.append(tok)
        if tok == eos:
            break
    return out


def test_generate_ids_sampled_one_call_and_eos(qa_cpu, small_hw):
    """temperature > 0 goes to generate_sampled as one call for every parameter set (top-p
    alone, top-k with and without top-p, a top-k above the single-kernel fast path,
    temperature alone): the device draws the tokens and stops after the eos, which ends the
    list; the position advances by the tokens drawn. Greedy settings take the greedy path."""
    mod, stub = qa_cpu
    prompt = [3, 1, 4, 1, 5]
    dec = mod.Decoder(weights=_weights(mod), verbose=False)
    for kw in (dict(temperature=1.3, top_k=0, top_p=0.9, seed=77), dict(temperature=1.3, top_k=20, top_p=0.9, seed=77),
               dict(temperature=1.1, top_k=300, top_p=1.0, seed=3), dict(temperature=1.3, top_k=0, top_p=1.0, seed=5)):
        ref = _sampled_ref(small_hw, prompt, 10, **kw)
        stub.oracle.reset()
        stub.calls.clear()
        assert dec.generate_ids(prompt, 10, **kw) == ref
        assert stub.calls[-1] == ("generate_sampled", 5, 4, 10, -1)
        k = next(i for i in range(4, 10) if ref[i] not in ref[:i])
        stub.oracle.reset()
        stub.calls.clear()
        assert dec.generate_ids(prompt, 10, eos_token_id=ref[k], **kw) == ref[:k + 1]
        assert dec.position == len(prompt) - 1 + k + 1
        assert [c for c in stub.calls if c[0] == "generate_sampled"] == [("generate_sampled", 5, 4, 10, ref[k])]
    # greedy settings take the greedy path
    stub.calls.clear()
    stub.oracle.reset()
    dec.generate_ids(prompt, 4, temperature=0.7, top_k=1)
    assert stub.calls[-1][0] == "generate_nosync"
    with pytest.raises(ValueError):
        dec.generate_sampled(1, 2, temperature=1.0, top_k=-3)


def test_positions_past_the_cache_raise(qa_cpu):
    mod, _ = qa_cpu
    dec = mod.Decoder(weights=_weights(mod), verbose=False)
    with pytest.raises(RuntimeError, match="exceed"):
        dec.generate_nosync(1, mod.MAX_SEQ_LEN + 1)
    dec._position = mod.MAX_SEQ_LEN
    with pytest.raises(RuntimeError, match="MAX_SEQ_LEN"):
        dec.step(1)


def test_load_weights_needs_local_directory(qa_cpu, tmp_path):
    mod, _ = qa_cpu
    with pytest.raises(RuntimeError, match="not a local checkpoint directory"):
        mod.load_weights("Qwen/Qwen3-0.6B")
    with pytest.raises(RuntimeError, match="no .safetensors"):
        mod.load_weights(str(tmp_path))


def test_load_weights_reads_safetensors(qa_cpu, tmp_path):
    """A local checkpoint in HF naming loads into LDGLayerWeight order, fp16, tied lm_head."""
    from safetensors.torch import save_file

    mod, _ = qa_cpu
    rng = np.random.default_rng(0)
    state = {"model.embed_tokens.weight": torch.from_numpy(rng.standard_normal((8, 4)).astype(np.float32)),
             "model.norm.weight": torch.ones(4, dtype=torch.bfloat16)}
    for i in range(mod.NUM_LAYERS):
        for j, key in enumerate(mod._LAYER_KEYS):
            state[f"model.layers.{i}.{key}"] = torch.full((2,), float(i * 11 + j), dtype=torch.float32)
    save_file(state, str(tmp_path / "model.safetensors"))
    w, tok = mod.load_weights(str(tmp_path), verbose=False)
    assert len(w["layer_weights"]) == 28 * 11
    for i in (0, 27):
        for j in range(11):
            t = w["layer_weights"][i * 11 + j]
            assert t.dtype == torch.float16 and float(t[0]) == float(i * 11 + j)
    assert w["lm_head_weight"] is w["embed_weight"]
    assert w["cos_table"].shape == (mod.MAX_SEQ_LEN, mod.HEAD_DIM) and w["cos_table"].dtype == torch.float16


def test_bench_cpu_baseline_stays_inside_the_cache(monkeypatch):
    """bench.py's CPU baseline times oracle decode steps from position PREFILL + 1 until its time
    budget or step limit, and never past the cache's last position (2047), however fast the host."""
    import bench

    monkeypatch.setattr(bench, "PREFILL", 2040)
    hw = qw.host_weights(seed=0, std=0.02)
    r = bench.cpu_baseline(hw, budget_s=300.0, max_steps=400)
    assert r["sample"].startswith("7 greedy decode steps") and "positions 2041..2047" in r["sample"], r
