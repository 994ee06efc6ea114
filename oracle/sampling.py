"""CPU restatement of the engine's token sampler (temperature, top-k, top-p, seeded draw).

TEST INFRASTRUCTURE ONLY, like the rest of ``oracle/``: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import it.

The reference decodes greedily only (Model/Qwen06B_architecture.py:343-382,
README.md:688-692); sampling is an addition, so the semantics restated here are
those of the usual logits processors (HuggingFace ``TemperatureLogitsWarper``,
``TopKLogitsWarper``, ``TopPLogitsWarper`` applied in that order, then a draw
from the softmax), with two choices fixed where they leave freedom:

* ties at a top-k or top-p boundary are all kept (HuggingFace keeps top-k ties
  too; its top-p boundary among equal logits depends on its sort order);
* the draw is a Gumbel-max pick, ``argmax_j l_j / T + g_j`` over the kept
  tokens, with ``g_j = -log(-log(u_j))`` and ``u_j`` from Philox4x32-10
  (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as easy as 1, 2, 3",
  SC'11) of counter ``(j, step, 0, 0)`` under key ``(seed & 0xffffffff,
  seed >> 32)``: ``u = ((x0 >> 9) + 0.5) / 2^23``, exact in fp32 and inside
  [2^-24, 1 - 2^-24].

Top-p works on integer masses, ``trunc(exp((l - M) / T) * 2^40)`` in fp32 (M
the largest logit), so its sums do not depend on the order of additions: the
kept set is every token whose key is >= the key of the token at which the
descending cumulative mass first reaches ``ceil(total * top_p)``.

Pinned by tests/test_sampling_oracle.py: Philox against the published
known-answer vectors of the Random123 distribution, the kept sets against the
HuggingFace warpers (transformers, present in the image) away from exact
boundary ties, and the draw against the softmax by a chi-square test.
"""

from __future__ import annotations

import math

import numpy as np

PHILOX_M0, PHILOX_M1 = 0xD2511F53, 0xCD9E8D57
PHILOX_W0, PHILOX_W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = 0xFFFFFFFF
MASS_SCALE = np.float32(2.0 ** 40)


def philox4x32_10(ctr, key):
    """Philox4x32 with 10 rounds over arrays: ``ctr`` 4 arrays, ``key`` 2 arrays of 32-bit
    values (any integer dtype); returns 4 uint64 arrays holding 32-bit words."""
    c = [np.asarray(x, dtype=np.uint64) & MASK32 for x in ctr]
    k0, k1 = (np.asarray(x, dtype=np.uint64) & MASK32 for x in key)
    for _ in range(10):
        p0 = np.uint64(PHILOX_M0) * c[0]
        p1 = np.uint64(PHILOX_M1) * c[2]
        c = [(p1 >> np.uint64(32)) ^ c[1] ^ k0, p1 & np.uint64(MASK32),
             (p0 >> np.uint64(32)) ^ c[3] ^ k1, p0 & np.uint64(MASK32)]
        k0 = (k0 + np.uint64(PHILOX_W0)) & np.uint64(MASK32)
        k1 = (k1 + np.uint64(PHILOX_W1)) & np.uint64(MASK32)
    return c


def word_to_uniform(x0) -> np.ndarray:
    """fp32 u in (0, 1) from a 32-bit word: (x0 >> 9) + 0.5 is exact in fp32 and so is the
    scaling by 2^-23."""
    x0 = np.asarray(x0, dtype=np.uint64)
    return ((x0 >> np.uint64(9)).astype(np.float32) + np.float32(0.5)) * np.float32(1.0 / 8388608.0)


def uniforms(seed: int, step: int, n: int) -> np.ndarray:
    """u_j in (0, 1) (fp32) for tokens j = 0 .. n-1 at ``step``."""
    j = np.arange(n, dtype=np.uint64)
    z = np.zeros(n, dtype=np.uint64)
    x0 = philox4x32_10((j, np.full(n, step & MASK32, np.uint64), z, z),
                       (np.full(n, seed & MASK32, np.uint64), np.full(n, (seed >> 32) & MASK32, np.uint64)))[0]
    return word_to_uniform(x0)


def gumbel(seed: int, step: int, n: int) -> np.ndarray:
    """Gumbel(0, 1) noise g_j = -log(-log(u_j)), evaluated in float64 and rounded to fp32."""
    u = uniforms(seed, step, n).astype(np.float64)
    return (-np.log(-np.log(u))).astype(np.float32)


def fkey(logits: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 key of fp32 values (larger value, larger key); NaN -> 0."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    b = x.view(np.uint32)
    key = np.where(b & np.uint32(0x80000000), ~b, b | np.uint32(0x80000000)).astype(np.uint32)
    key[np.isnan(x)] = 0
    return key


def masses(logits: np.ndarray, m: np.float32, temperature: float) -> np.ndarray:
    """trunc(exp((l - M) / T) * 2^40) as uint64, fp32 arithmetic; NaN -> 0."""
    x = np.asarray(logits, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp((x - np.float32(m)) / np.float32(temperature)).astype(np.float32) * MASS_SCALE
    e = np.where(np.isnan(x), np.float32(0), e)
    return e.astype(np.uint64)


def argmax_lowest(v: np.ndarray) -> int:
    """Index of the largest non-NaN value, lowest index on ties; 0 if every value is NaN."""
    v = np.asarray(v, dtype=np.float32)
    ok = ~np.isnan(v)
    if not ok.any():
        return 0
    best = v[ok].max()
    return int(np.flatnonzero(ok & (v == best))[0])


def kept_set(logits: np.ndarray, temperature: float, top_k: int = 0, top_p: float = 1.0):
    """The tokens the draw chooses from (bool mask) and the details of the top-p cut:
    ``(mask, info)`` with info = {"lo": key threshold, "total", "target", "cum_at_cut"}."""
    x = np.asarray(logits, dtype=np.float32)
    n = x.size
    keys = fkey(x)
    m = np.float32(x[argmax_lowest(x)])
    lo = np.uint32(0)
    info = {"lo": 0, "total": None, "target": None, "cum_before": None, "cum_at_cut": None}
    if 1 < top_k < n:
        lo = np.sort(keys)[::-1][top_k - 1]
    if top_p < 1.0:
        sel = keys >= lo
        w = np.where(sel, masses(x, m, temperature), np.uint64(0))
        total = int(w.sum(dtype=np.uint64))
        tgt = float(total) * float(np.float32(max(top_p, 0.0)))
        target = int(tgt)
        if target < tgt:
            target += 1
        target = min(max(target, 1), total)
        order = np.argsort(keys, kind="stable")[::-1]
        cum = np.cumsum(w[order], dtype=np.uint64)
        i = int(np.searchsorted(cum, np.uint64(target), side="left"))
        lo = max(lo, keys[order[i]])
        info.update(total=total, target=target, cum_at_cut=int(cum[i]),
                    cum_before=int(cum[i - 1]) if i > 0 else 0)
    info["lo"] = int(lo)
    mask = (keys >= lo) & (x > -np.inf) & ~np.isnan(x)
    return mask, info


def sample(logits: np.ndarray, temperature: float, top_k: int = 0, top_p: float = 1.0, seed: int = 0,
           step: int = 0, details: bool = False):
    """The sampled token id; with ``details`` also the perturbed scores' top-2 gap and the
    kept-set info (the quantities near which an fp32 rounding difference could change it)."""
    x = np.asarray(logits, dtype=np.float32)
    greedy = argmax_lowest(x)
    m = np.float32(x[greedy])
    if not (temperature > 0) or top_k == 1 or not np.isfinite(m):
        return (greedy, {"gap": math.inf, "greedy": True}) if details else greedy
    mask, info = kept_set(x, temperature, top_k, top_p)
    with np.errstate(invalid="ignore"):
        score = x / np.float32(temperature) + gumbel(seed, step, x.size)
    score = np.where(mask, score, np.float32(-np.inf)).astype(np.float32)
    tok = argmax_lowest(np.where(mask, score, np.float32(np.nan)))
    if not details:
        return tok
    s = np.sort(score[mask])[::-1]
    info["gap"] = float(s[0] - s[1]) if s.size > 1 else math.inf
    info["greedy"] = False
    info["kept"] = int(mask.sum())
    return tok, info


def kept_probs(logits: np.ndarray, temperature: float, top_k: int = 0, top_p: float = 1.0) -> np.ndarray:
    """The distribution the draw follows: softmax(l / T) renormalised over the kept set (float64)."""
    x = np.asarray(logits, dtype=np.float64)
    mask, _ = kept_set(logits, temperature, top_k, top_p)
    z = np.where(mask, (x - x[mask].max()) / temperature, -np.inf)
    p = np.exp(z)
    return p / p.sum()
