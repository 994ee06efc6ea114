"""Weight loading and high-level decode API for Qwen3-0.6B on MI355X.

Mirror of the reference's Model/Qwen06B_architecture.py: same module name,
constants, ``EXTENSION_ABI_VERSION``, import-time extension gate
(``_assert_extension_compatibility`` / ``_require_megakernel_op``, lines
32-94), ``load_weights``, ``_pack_layer_weights`` (the 12-pointer
``LDGLayerWeight`` table, lines 177-202) and ``Decoder`` with
``step``/``generate``/``reset``/``position`` (lines 205-382). Every call goes
to the compiled ``qwen_megakernel_C`` module next to this file; importing this
module without it raises, exactly as the reference does.

Differences from the reference, all additive:
* ``load_weights`` reads a local Hugging Face checkpoint directory
  (safetensors) instead of downloading; ``qwen_weights.synthetic_weights``
  builds seeded random weights in the same dictionary layout;
* ``Decoder.prefill`` / ``generate_ids`` run a prompt and greedy generation on
  token ids (no tokenizer needed); the prompt is prefilled in one launch of the
  batched (MFMA) prefill kernel instead of one launch and host sync per token;
* positions beyond ``MAX_SEQ_LEN`` raise instead of silently skipping
  attention (Tools/megakernel/megakernel.cu:330-333);
* device-side errors are checked after every synchronising call.
"""

import math
import os

import numpy as np
import torch

try:
    import qwen_megakernel_C
except ImportError:
    qwen_megakernel_C = None

EXTENSION_ABI_VERSION = 2

NUM_LAYERS = 28
NUM_KV_HEADS = 8
HEAD_DIM = 128
HIDDEN_SIZE = 1024
INTERMEDIATE_SIZE = 3072
Q_SIZE = 16 * HEAD_DIM  # 2048
KV_SIZE = 8 * HEAD_DIM  # 1024
MAX_SEQ_LEN = 2048
VOCAB_SIZE = 151936
ROPE_THETA = 1_000_000.0  # Qwen3-0.6B config.json "rope_theta"
DEVICE = "cuda"  # where Decoder allocates its state; the engine itself needs the GPU

_OPS = ("decode", "generate_nosync", "generate_until")



def _require_megakernel_op(op_name: str):
    """Return an op from the extension module or the torch.ops namespace."""
    if qwen_megakernel_C is not None and hasattr(qwen_megakernel_C, op_name):
        return getattr(qwen_megakernel_C, op_name)
    namespace = getattr(torch.ops, "qwen_megakernel_C", None)
    if namespace is not None and hasattr(namespace, op_name):
        return getattr(namespace, op_name)
    available = []
    if qwen_megakernel_C is not None:
        available.extend(op for op in _OPS if hasattr(qwen_megakernel_C, op))
    text = ", ".join(sorted(set(available))) or "none"
    raise RuntimeError(
        f"qwen_megakernel_C op '{op_name}' is unavailable: the HIP extension is not built or not on sys.path. "
        "Build it with `python qwen0.6b_amd/build.py` (gfx950). "
        f"torch {torch.__version__}. Available extension ops: {text}."
    )


def _assert_extension_compatibility() -> None:
    """Fail fast on an extension whose pointer-table ABI differs from this module's."""
    if qwen_megakernel_C is None:
        return
    ext_abi = None
    if hasattr(qwen_megakernel_C, "abi_version"):
        try:
            ext_abi = int(qwen_megakernel_C.abi_version())
        except Exception:
            ext_abi = None
    if ext_abi != EXTENSION_ABI_VERSION:
        built = "unknown"
        if hasattr(qwen_megakernel_C, "built_torch_version"):
            try:
                built = str(qwen_megakernel_C.built_torch_version())
            except Exception:
                built = "unknown"
        raise RuntimeError(
            "Incompatible qwen_megakernel_C extension binary detected. "
            f"Expected ABI {EXTENSION_ABI_VERSION}, got {ext_abi}. The Python code and the extension are out of "
            f"sync (the pointer packing changed). Rebuild qwen_megakernel_C for torch {torch.__version__} "
            f"(extension was built against {built})."
        )


_assert_extension_compatibility()
_decode = _require_megakernel_op("decode")


def _synchronize() -> None:
    if torch.device(DEVICE).type == "cuda":
        torch.cuda.synchronize()


_DEVICE_ERRORS = {
    4: "a cross-workgroup wait exceeded its deadline",
    5: "a forced token id outside the vocabulary reached the device",
}


def _check_device_errors() -> None:
    fn = getattr(qwen_megakernel_C, "last_error", None)
    if fn is None:
        return
    rc = int(fn())
    if rc != 0:
        why = _DEVICE_ERRORS.get(rc, "unknown error")
        raise RuntimeError(
            f"qwen_megakernel_C device-side error {rc}: {why} "
            "(the engine state was reset; call Decoder.reset() before continuing)"
        )


def rope_tables(device=None):
    """fp16 cos/sin tables [MAX_SEQ_LEN, HEAD_DIM] built in fp32 (reference lines 134-142)."""
    inv_freq = 1.0 / (ROPE_THETA ** (torch.arange(0, HEAD_DIM, 2, dtype=torch.float32) / HEAD_DIM))
    positions = torch.arange(MAX_SEQ_LEN, dtype=torch.float32)
    freqs = torch.outer(positions, inv_freq)
    device = device or DEVICE
    cos_table = torch.cos(freqs).repeat(1, 2).to(torch.float16).to(device).contiguous()
    sin_table = torch.sin(freqs).repeat(1, 2).to(torch.float16).to(device).contiguous()
    return cos_table, sin_table


_LAYER_KEYS = (
    "input_layernorm.weight",
    "self_attn.q_proj.weight",
    "self_attn.k_proj.weight",
    "self_attn.v_proj.weight",
    "self_attn.q_norm.weight",
    "self_attn.k_norm.weight",
    "self_attn.o_proj.weight",
    "post_attention_layernorm.weight",
    "mlp.gate_proj.weight",
    "mlp.up_proj.weight",
    "mlp.down_proj.weight",
)


def load_weights(model_name="Qwen/Qwen3-0.6B", verbose: bool = True):
    """Load Qwen3-0.6B weights from a local Hugging Face checkpoint directory.

    ``model_name`` must be a directory holding ``*.safetensors`` (and, for text
    generation, the tokenizer files). Tensors are cast to fp16 on the GPU and
    returned in the reference's dictionary layout (reference lines 97-174):
    11 per-layer tensors in ``LDGLayerWeight`` order; the lm_head is the
    embedding (tied, as Qwen3-0.6B) unless the checkpoint has ``lm_head.weight``.
    """
    if not os.path.isdir(model_name):
        raise RuntimeError(
            f"load_weights: '{model_name}' is not a local checkpoint directory. This build does not download "
            "weights; pass a directory with the Qwen3-0.6B safetensors, or use "
            "qwen_weights.synthetic_weights() for seeded random weights."
        )
    from safetensors.torch import load_file

    state = {}
    files = sorted(f for f in os.listdir(model_name) if f.endswith(".safetensors"))
    if not files:
        raise RuntimeError(f"load_weights: no .safetensors files in {model_name}")
    for f in files:
        state.update(load_file(os.path.join(model_name, f)))
    if verbose:
        print(f"Loaded {len(state)} tensors from {model_name}")

    def dev(name):
        return state[name].to(device=DEVICE, dtype=torch.float16).contiguous()

    layer_weights = []
    for i in range(NUM_LAYERS):
        for key in _LAYER_KEYS:
            layer_weights.append(dev(f"model.layers.{i}.{key}"))
    embed_weight = dev("model.embed_tokens.weight")
    cos_table, sin_table = rope_tables(DEVICE)
    weights = dict(
        embed_weight=embed_weight,
        layer_weights=layer_weights,
        final_norm_weight=dev("model.norm.weight"),
        lm_head_weight=dev("lm_head.weight") if "lm_head.weight" in state else embed_weight,
        cos_table=cos_table,
        sin_table=sin_table,
    )
    tokenizer = None
    try:
        from transformers import AutoTokenizer

        tokenizer = AutoTokenizer.from_pretrained(model_name, local_files_only=True)
    except Exception:
        tokenizer = None
    return weights, tokenizer


def _pack_layer_weights(layer_weights: list) -> torch.Tensor:
    """Pack 11 device pointers per layer plus one zero pad into a 16-B aligned
    int64 device tensor (reference lines 177-202)."""
    N = 11  # [0] input_layernorm, [1] q, [2] k, [3] v, [4] q_norm, [5] k_norm, [6] o, [7] post_attn_norm,
    #         [8] gate, [9] up, [10] down
    n_layers = len(layer_weights) // N
    assert len(layer_weights) == n_layers * N, (
        f"Expected {n_layers * N} weight tensors ({N} per layer x {n_layers} layers), got {len(layer_weights)}. "
        "Check that the loader appends exactly 11 tensors per layer in LDGLayerWeight field order."
    )
    all_ptrs = []
    for li in range(n_layers):
        for j in range(N):
            all_ptrs.append(layer_weights[li * N + j].data_ptr())
        all_ptrs.append(0)  # padding: the struct is 12 pointers (96 bytes)
    t = torch.zeros(len(all_ptrs) + 2, dtype=torch.int64, device=DEVICE)
    offset_elems = ((16 - (t.data_ptr() % 16)) % 16) // 8
    t_aligned = t[offset_elems : offset_elems + len(all_ptrs)]
    t_aligned.copy_(torch.tensor(all_ptrs, dtype=torch.int64))
    assert t_aligned.data_ptr() % 16 == 0, "Alignment failed!"
    return t_aligned


class Decoder:
    """Stateful decoder over the MI355X decode engine (reference lines 205-382)."""

    def __init__(self, weights=None, tokenizer=None, model_name="Qwen/Qwen3-0.6B", verbose: bool = True):
        if weights is None:
            weights, tokenizer = load_weights(model_name, verbose=verbose)
        self.tokenizer = tokenizer
        self._position = 0
        self._weights = weights  # keep alive: the pointer table refers to this memory
        self._embed_weight = weights["embed_weight"]
        self._final_norm_weight = weights["final_norm_weight"]
        self._lm_head_weight = weights["lm_head_weight"]
        self._cos_table = weights["cos_table"]
        self._sin_table = weights["sin_table"]
        self._num_layers = len(weights["layer_weights"]) // 11
        self._layer_weights_packed = _pack_layer_weights(weights["layer_weights"])
        self._check_weight_alignment(weights["layer_weights"], verbose)
        self._attn_scale = 1.0 / math.sqrt(HEAD_DIM)

        self._k_cache = torch.zeros(self._num_layers, NUM_KV_HEADS, MAX_SEQ_LEN, HEAD_DIM,
                                    dtype=torch.float16, device=DEVICE)
        self._v_cache = torch.zeros_like(self._k_cache)

        f16 = dict(dtype=torch.float16, device=DEVICE)
        f32 = dict(dtype=torch.float32, device=DEVICE)
        i32 = dict(dtype=torch.int32, device=DEVICE)
        self._hidden = torch.empty(HIDDEN_SIZE, **f16)
        self._act = torch.empty(Q_SIZE, **f32)
        self._res = torch.empty(HIDDEN_SIZE, **f32)
        self._q = torch.empty(Q_SIZE, **f16)
        self._k = torch.empty(KV_SIZE, **f16)
        self._v = torch.empty(KV_SIZE, **f16)
        self._attn_out = torch.empty(Q_SIZE, **f16)
        self._mlp_inter = torch.empty(INTERMEDIATE_SIZE, **f32)
        self._norm_out = torch.empty(HIDDEN_SIZE, **f32)
        self._fmax_vals = torch.empty(4096, **f32)
        self._fmax_idxs = torch.empty(4096, **i32)
        self._out_token = torch.empty(1, **i32)

    def _check_weight_alignment(self, layer_weights_list, verbose=True):
        names = ["input_layernorm", "q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "o_proj",
                 "post_attn_norm", "gate_proj", "up_proj", "down_proj"]
        bad = []
        for li in range(self._num_layers):
            for j in range(11):
                ptr = layer_weights_list[li * 11 + j].data_ptr()
                if ptr % 16 != 0:
                    bad.append(f"  Layer {li} [{names[j]}]: ptr={ptr:#x}, rem={ptr % 16}")
        if bad:
            raise RuntimeError("misaligned weight tensors (16-byte alignment required):\n" + "\n".join(bad))

    def _tensors(self):
        return (
            self._embed_weight, self._layer_weights_packed, self._final_norm_weight, self._lm_head_weight,
            self._cos_table, self._sin_table, self._k_cache, self._v_cache, self._hidden, self._act, self._res,
            self._q, self._k, self._v, self._attn_out, self._mlp_inter, self._norm_out, self._fmax_vals,
            self._fmax_idxs,
        )

    def step(self, input_token_id) -> int:
        """Decode one token at the current position; returns the greedy next token."""
        if self._position >= MAX_SEQ_LEN:
            raise RuntimeError(f"position {self._position} reached MAX_SEQ_LEN {MAX_SEQ_LEN}; call reset()")
        result_tensor = _decode(int(input_token_id), *self._tensors(), self._num_layers, self._position,
                                MAX_SEQ_LEN, self._attn_scale)
        _synchronize()
        _check_device_errors()
        self._out_token.copy_(result_tensor)
        self._position += 1
        return int(result_tensor.item())

    def reset(self):
        self._position = 0
        self._k_cache.zero_()
        self._v_cache.zero_()

    @property
    def position(self) -> int:
        return self._position

    def generate_nosync(self, first_token_id: int, num_steps: int) -> torch.Tensor:
        """``num_steps`` greedy steps in one launch from the current position; returns the
        device int32 tensor of generated ids. Advances the position by ``num_steps``."""
        if self._position + num_steps > MAX_SEQ_LEN:
            raise RuntimeError(f"positions {self._position}..{self._position + num_steps} exceed {MAX_SEQ_LEN}")
        gen = _require_megakernel_op("generate_nosync")
        out = gen(int(first_token_id), int(num_steps), *self._tensors(), self._num_layers, self._position,
                  MAX_SEQ_LEN, self._attn_scale)
        self._position += num_steps
        return out

    def _prefill_kv(self, ids) -> None:
        """Write the K/V cache of ``ids`` at positions ``position ..`` in one batched launch
        (MFMA prefill kernel) and advance the position; no greedy token."""
        if not ids:
            return
        if self._position + len(ids) > MAX_SEQ_LEN:
            raise RuntimeError(f"prefill of {len(ids)} ids at position {self._position} exceeds {MAX_SEQ_LEN}")
        # through numpy: half the host time of torch.tensor on a long Python list
        t = torch.from_numpy(np.fromiter(ids, dtype=np.int32, count=len(ids))).to(DEVICE)
        qwen_megakernel_C.prefill(t, self._embed_weight, self._layer_weights_packed, self._cos_table,
                                  self._sin_table, self._k_cache, self._v_cache, self._hidden, self._num_layers,
                                  self._position, MAX_SEQ_LEN, self._attn_scale)
        self._position += len(ids)

    def prefill(self, ids, batched: bool = True) -> int:
        """Run every id in ``ids`` through the model at consecutive positions; returns the
        greedy token after the last id (the reference prefills with one ``step`` per id,
        lines 346-347). ``batched``: all but the last id in one launch of the batched
        (MFMA) prefill kernel, then one decode step of the last id; otherwise every id
        teacher forced through the decode kernel in one launch."""
        ids = [int(t) for t in ids]
        if not ids:
            raise ValueError("prefill needs at least one id")
        if self._position + len(ids) > MAX_SEQ_LEN:
            raise RuntimeError(f"prefill of {len(ids)} ids at position {self._position} exceeds {MAX_SEQ_LEN}")
        if batched:
            self._prefill_kv(ids[:-1])
            ids = ids[-1:]
        forced = torch.tensor(ids, dtype=torch.int32, device=DEVICE)
        out = qwen_megakernel_C.generate_ex(
            ids[0], len(ids), forced, self._embed_weight, self._layer_weights_packed, self._final_norm_weight,
            self._lm_head_weight, self._cos_table, self._sin_table, self._k_cache, self._v_cache, self._hidden,
            self._norm_out, None, None, self._num_layers, self._position, MAX_SEQ_LEN, self._attn_scale)
        self._position += len(ids)
        last = int(out[-1].item())
        _check_device_errors()
        return last

    def generate_until(self, first_token_id: int, max_tokens: int, eos_token_id: int) -> list:
        """Up to ``max_tokens`` greedy steps in one launch that end on the device after the
        first ``eos_token_id`` (included in the result); advances the position by the
        number of steps run."""
        if self._position + max_tokens > MAX_SEQ_LEN:
            raise RuntimeError(f"positions {self._position}..{self._position + max_tokens} exceed {MAX_SEQ_LEN}")
        gen = _require_megakernel_op("generate_until")
        out, count = gen(int(first_token_id), int(max_tokens), int(eos_token_id), self._embed_weight,
                         self._layer_weights_packed, self._final_norm_weight, self._lm_head_weight, self._cos_table,
                         self._sin_table, self._k_cache, self._v_cache, self._hidden, self._norm_out,
                         self._num_layers, self._position, MAX_SEQ_LEN, self._attn_scale)
        n = int(count.item())
        _check_device_errors()
        self._position += n
        return out[:n].cpu().tolist()

    def generate_sampled(self, first_token_id: int, max_tokens: int, temperature: float, top_k: int = 0,
                         top_p: float = 1.0, seed: int = 0, eos_token_id=None) -> list:
        """Up to ``max_tokens`` sampled steps from the current position in one launch of the
        decode kernel, with no host synchronisation until the end: each step's next token is
        drawn on the device from its logits (temperature, then top-k, then top-p, then a draw
        seeded by ``seed`` and the step's position; temperature <= 0 or top_k == 1 is greedy).
        With ``eos_token_id`` the device ends the generation after that id (which ends the
        list); advances the position by the number of steps run."""
        if self._position + max_tokens > MAX_SEQ_LEN:
            raise RuntimeError(f"positions {self._position}..{self._position + max_tokens} exceed {MAX_SEQ_LEN}")
        if top_k < 0 or not 0.0 <= top_p or temperature != temperature:
            raise ValueError(f"invalid sampling parameters temperature={temperature} top_k={top_k} top_p={top_p}")
        gen = _require_megakernel_op("generate_sampled")
        eos = -1 if eos_token_id is None else int(eos_token_id)
        ids, count = gen(int(first_token_id), max_tokens, eos, self._embed_weight, self._layer_weights_packed,
                         self._final_norm_weight, self._lm_head_weight, self._cos_table, self._sin_table,
                         self._k_cache, self._v_cache, self._hidden, self._norm_out, self._num_layers, self._position,
                         MAX_SEQ_LEN, self._attn_scale, float(temperature), int(top_k), float(top_p),
                         int(seed) & 0xFFFFFFFFFFFFFFFF)
        n = int(count.item())
        _check_device_errors()
        self._position += n
        return ids[:n].cpu().tolist()

    def generate_ids(self, ids, max_tokens: int = 100, eos_token_id=None, temperature: float = 0.0,
                     top_k: int = 0, top_p: float = 1.0, seed: int = 0) -> list:
        """Generation on token ids (reference ``generate`` without the tokenizer): prefill
        ids[:-1], then ``max_tokens`` on-device steps from ids[-1]; with ``eos_token_id``
        the device stops after that id (which ends the list). Greedy by default, as the
        reference; ``temperature`` > 0 samples (see ``generate_sampled``)."""
        self.reset()
        ids = [int(t) for t in ids]
        self._prefill_kv(ids[:-1])
        if temperature > 0 and top_k != 1:
            return self.generate_sampled(ids[-1], max_tokens, temperature, top_k, top_p, seed, eos_token_id)
        if eos_token_id is not None:
            return self.generate_until(ids[-1], max_tokens, eos_token_id)
        out = self.generate_nosync(ids[-1], max_tokens).cpu().tolist()
        _check_device_errors()
        return out

    def generate(self, prompt: str, max_tokens: int = 100, temperature: float = 0.0, top_k: int = 0,
                 top_p: float = 1.0, seed: int = 0) -> str:
        if self.tokenizer is None:
            raise RuntimeError("generate(prompt) needs a tokenizer; use generate_ids() for token ids")
        ids = self.tokenizer.encode(prompt, add_special_tokens=True)
        eos = self.tokenizer.eos_token_id
        out = self.generate_ids(ids, max_tokens, eos_token_id=eos, temperature=temperature, top_k=top_k,
                                top_p=top_p, seed=seed)
        if eos in out:
            out = out[: out.index(eos)]
        return self.tokenizer.decode(out, skip_special_tokens=True)


def generate(prompt: str, max_tokens: int = 50, verbose: bool = True, model_name="Qwen/Qwen3-0.6B",
             temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0, seed: int = 0) -> str:
    """One-shot convenience: load model, generate (greedy unless temperature > 0), return text."""
    return Decoder(model_name=model_name, verbose=verbose).generate(prompt, max_tokens, temperature, top_k,
                                                                    top_p, seed)
