"""Writes the oracle's golden fixtures (run from the repo root):

    python tests/golden/make_golden.py

* tiny_decode.json - a 3-layer 64-wide model (seed 7, std 0.2), 6-id prompt,
  12 greedy tokens: ids, top-5 logits per step, weight digest.
* c0_decode.json   - the full-size synthetic Qwen3-0.6B (seed 0, std 0.02,
  norms 1.0), 16-id prompt (seed 1), 32 greedy tokens: ids, top-2 gap, top-4
  logits, the first 16 hidden values per step, and the weight digest.

The fixtures come from the CPU oracle (oracle/qwen3_oracle.py), which
tests/test_oracle.py pins independently (closed forms + HuggingFace Qwen3).
"""

import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "qwen0.6b_amd"))

import qwen_weights as qw  # noqa: E402
from oracle import qwen3_oracle as orc  # noqa: E402

TINY = qw.QwenShape(hidden=64, inter=192, layers=3, q_heads=4, kv_heads=2, head_dim=16, vocab=512, max_seq=64)


def tiny():
    seed, std, n_new = 7, 0.2, 12
    hw = qw.host_weights(seed=seed, std=std, shape=TINY)
    prompt = qw.synthetic_prompt(6, seed=5, vocab=TINY.vocab)
    run = orc.Oracle(hw).greedy(prompt, n_new)
    top5 = []
    for st in run["steps"]:
        v, i = torch.topk(st["logits"], 5)
        top5.append(dict(idx=i.tolist(), val=[round(float(x), 7) for x in v]))
    out = dict(seed=seed, std=std, prompt=prompt, n_new=n_new, tokens=run["tokens"],
               weights_sha256=hw.digest(), top5=top5)
    with open(os.path.join(HERE, "tiny_decode.json"), "w") as f:
        json.dump(out, f, indent=1)


def c0():
    hw = qw.host_weights(seed=0, std=0.02)
    prompt = qw.synthetic_prompt(16, seed=1)
    run = orc.Oracle(hw).greedy(prompt, 32)
    steps = []
    for st in run["steps"]:
        v, i = torch.topk(st["logits"], 4)
        steps.append(dict(pos=st["pos"], input=st["input"], token=st["token"], gap=round(st["gap"], 7),
                          top4_idx=i.tolist(), top4_val=[round(float(x), 6) for x in v],
                          hidden16=[round(float(x), 6) for x in st["hidden"][:16]]))
    out = dict(seed=0, std=0.02, prompt=prompt, n_new=32, n_check=32, tokens=run["tokens"],
               weights_sha256=hw.digest(), steps=steps)
    with open(os.path.join(HERE, "c0_decode.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    torch.set_num_threads(os.cpu_count() or 1)
    tiny()
    c0()
    print("golden fixtures written")
