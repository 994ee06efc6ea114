"""Seeded synthetic Qwen3-0.6B weights and the RoPE tables.

The reference loads real weights with ``AutoModelForCausalLM.from_pretrained``
(Model/Qwen06B_architecture.py:97-174), which needs the network. This module
builds the same dictionary (``embed_weight``, ``layer_weights`` as 11 tensors
per layer in the ``LDGLayerWeight`` field order of Model/Qwen06B_architecture.py:148-160,
``final_norm_weight``, tied ``lm_head_weight``, ``cos_table``, ``sin_table``)
from a seeded, version-stable generator, so every run on every machine sees the
same fp16 values:

* each tensor ``i`` is drawn from its own ``numpy`` PCG64 stream seeded with
  ``SeedSequence([seed, i])`` as ``standard_normal(float32) * std`` and rounded
  once to fp16 (round-to-nearest-even);
* tensor ids: 0 = embedding, ``1 + 11*layer + field`` for the per-layer fields;
  the embedding is drawn in blocks of ``EMBED_BLOCK_ROWS`` rows, block ``c``
  from ``SeedSequence([seed, 0, c + 1])``, so it can be drawn in parallel;
* RMSNorm weights (fields 0, 4, 5, 7 and the final norm) are all 1.0 with
  ``norms="ones"`` (the default workload); with ``norms="random"`` each is
  ``1 + 0.5 * N(0, 1)`` from its own stream (tensor id of its field; the final
  norm is id ``1 + 11 * layers``), so every layer and every field differs, as
  real checkpoints do;
* ``untied=True`` adds a separate lm_head matrix (``N(0, std)``, tensor id
  ``(0, 0)``) in place of the tied embedding.

The RoPE tables follow Model/Qwen06B_architecture.py:134-142: ``inv_freq`` and
the angle table are built in fp32, ``cos``/``sin`` are taken in fp32, repeated
to the full head dimension (rotate-half pairing of dims ``i`` and ``i+64``) and
then rounded to fp16.
"""

from __future__ import annotations

import hashlib
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field

import numpy as np

# Field order of one layer's 11 tensors (Model/Qwen06B_architecture.py:148-160,
# Tools/megakernel/megakernel.cu:87-100).
LAYER_FIELDS = (
    "input_layernorm",
    "q_proj",
    "k_proj",
    "v_proj",
    "q_norm",
    "k_norm",
    "o_proj",
    "post_attention_layernorm",
    "gate_proj",
    "up_proj",
    "down_proj",
)
NORM_FIELDS = frozenset({0, 4, 5, 7})
EMBED_BLOCK_ROWS = 8192


@dataclass(frozen=True)
class QwenShape:
    """Model dimensions (Model/Qwen06B_architecture.py:14-29)."""

    hidden: int = 1024
    inter: int = 3072
    layers: int = 28
    q_heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 151936
    max_seq: int = 2048
    rope_theta: float = 1_000_000.0
    eps: float = 1e-6

    @property
    def q_size(self) -> int:
        return self.q_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.kv_heads * self.head_dim

    def field_shape(self, f: int) -> tuple:
        h, i, q, kv, d = self.hidden, self.inter, self.q_size, self.kv_size, self.head_dim
        return {
            0: (h,), 1: (q, h), 2: (kv, h), 3: (kv, h), 4: (d,), 5: (d,),
            6: (h, q), 7: (h,), 8: (i, h), 9: (i, h), 10: (h, i),
        }[f]


QWEN3_0_6B = QwenShape()


def _normal_fp16(seed, tensor_id, shape: tuple, std: float) -> np.ndarray:
    key = [seed] + (list(tensor_id) if isinstance(tensor_id, tuple) else [tensor_id])
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence(key)))
    x = rng.standard_normal(int(np.prod(shape)), dtype=np.float32)
    x *= np.float32(std)
    return x.astype(np.float16).reshape(shape)


def rope_tables_fp16(max_seq: int, head_dim: int, theta: float):
    """fp16 ``[max_seq, head_dim]`` cos/sin tables (Model/Qwen06B_architecture.py:134-142)."""
    import torch

    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    positions = torch.arange(max_seq, dtype=torch.float32)
    freqs = torch.outer(positions, inv_freq)
    cos = torch.cos(freqs).repeat(1, 2).to(torch.float16).contiguous()
    sin = torch.sin(freqs).repeat(1, 2).to(torch.float16).contiguous()
    return cos, sin


@dataclass
class HostWeights:
    """fp16 numpy copies of one synthetic model (host memory)."""

    shape: QwenShape
    embed: np.ndarray
    layers: list = field(default_factory=list)  # layers[l][f] -> np.ndarray fp16
    final_norm: np.ndarray = None
    cos: np.ndarray = None
    sin: np.ndarray = None
    lm_head: np.ndarray = None  # None: tied to the embedding (Model/Qwen06B_architecture.py:167)

    @property
    def lm_head_or_embed(self) -> np.ndarray:
        return self.embed if self.lm_head is None else self.lm_head

    def digest(self) -> str:
        """sha256 over every tensor's fp16 bytes in tensor-id order."""
        h = hashlib.sha256()
        h.update(np.ascontiguousarray(self.embed).view(np.uint16).tobytes())
        for layer in self.layers:
            for t in layer:
                h.update(np.ascontiguousarray(t).view(np.uint16).tobytes())
        h.update(np.ascontiguousarray(self.final_norm).view(np.uint16).tobytes())
        if self.lm_head is not None:
            h.update(np.ascontiguousarray(self.lm_head).view(np.uint16).tobytes())
        return h.hexdigest()


def _norm_fp16(seed, tensor_id, shape: tuple) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, tensor_id])))
    x = rng.standard_normal(int(np.prod(shape)), dtype=np.float32)
    return (np.float32(1.0) + np.float32(0.5) * x).astype(np.float16).reshape(shape)


def host_weights(seed: int = 0, std: float = 0.02, shape: QwenShape = QWEN3_0_6B, norms: str = "ones",
                 untied: bool = False) -> HostWeights:
    """Draw one synthetic model into host fp16 arrays (``norms``: "ones" or "random")."""
    if norms not in ("ones", "random"):
        raise ValueError(f"norms must be 'ones' or 'random', not {norms!r}")
    jobs = []
    for c, r0 in enumerate(range(0, shape.vocab, EMBED_BLOCK_ROWS)):
        jobs.append(((0, c + 1), (min(EMBED_BLOCK_ROWS, shape.vocab - r0), shape.hidden)))
    if untied:
        for c, r0 in enumerate(range(0, shape.vocab, EMBED_BLOCK_ROWS)):
            jobs.append(((0, 0, c + 1), (min(EMBED_BLOCK_ROWS, shape.vocab - r0), shape.hidden)))
    for layer in range(shape.layers):
        for f in range(len(LAYER_FIELDS)):
            if f not in NORM_FIELDS:
                jobs.append((1 + 11 * layer + f, shape.field_shape(f)))
    # Each tensor has its own stream, so drawing them concurrently is deterministic.
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        drawn = dict(zip([j[0] for j in jobs], ex.map(lambda j: _normal_fp16(seed, j[0], j[1], std), jobs)))
    nblk = (shape.vocab + EMBED_BLOCK_ROWS - 1) // EMBED_BLOCK_ROWS
    embed = np.concatenate([drawn[(0, c + 1)] for c in range(nblk)])
    lm_head = np.concatenate([drawn[(0, 0, c + 1)] for c in range(nblk)]) if untied else None

    def norm(tensor_id, shp):
        return np.ones(shp, dtype=np.float16) if norms == "ones" else _norm_fp16(seed, tensor_id, shp)

    layers = []
    for layer in range(shape.layers):
        fields = []
        for f in range(len(LAYER_FIELDS)):
            shp = shape.field_shape(f)
            if f in NORM_FIELDS:
                fields.append(norm(1 + 11 * layer + f, shp))
            else:
                fields.append(drawn[1 + 11 * layer + f])
        layers.append(fields)
    cos, sin = rope_tables_fp16(shape.max_seq, shape.head_dim, shape.rope_theta)
    return HostWeights(
        shape=shape,
        embed=embed,
        layers=layers,
        final_norm=norm(1 + 11 * shape.layers, (shape.hidden,)),
        cos=cos.numpy(),
        sin=sin.numpy(),
        lm_head=lm_head,
    )


def synthetic_prompt(n: int, seed: int = 1, vocab: int = 151936) -> list:
    """``n`` prompt ids uniform in ``[0, vocab)`` from PCG64(seed)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return [int(t) for t in rng.integers(0, vocab, size=n)]


def device_weights(hw: HostWeights, device: str = "cuda") -> dict:
    """Upload host weights into the dictionary layout ``Decoder`` consumes.

    Every tensor is a separate contiguous device allocation (the caching
    allocator aligns each to at least 512 B), so all pointers in the packed
    table are 16-byte aligned as the device code requires.
    """
    import torch

    def up(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(device)

    embed = up(hw.embed)
    lm_head = embed if hw.lm_head is None else up(hw.lm_head)
    layer_weights = []
    for layer in hw.layers:
        for t in layer:
            layer_weights.append(up(t))
    return dict(
        embed_weight=embed,
        layer_weights=layer_weights,
        final_norm_weight=up(hw.final_norm),
        lm_head_weight=lm_head,  # tied unless the model has its own (Model/Qwen06B_architecture.py:167)
        cos_table=up(hw.cos),
        sin_table=up(hw.sin),
    )


def synthetic_weights(seed: int = 0, std: float = 0.02, device: str = "cuda", shape: QwenShape = QWEN3_0_6B):
    """Seeded synthetic weights on ``device`` in the ``load_weights`` layout."""
    return device_weights(host_weights(seed, std, shape), device)
