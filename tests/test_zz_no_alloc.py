"""qwen_generate_nosync_noalloc (the entry point that allocates nothing) against
launch_ldg_generate_nosync, both through the C-ABI (ctypes).

Two calls of the no-allocation entry point in a row, the second smaller (fewer
steps, another first token), are compared bit for bit with the allocating
entry point on the same inputs: generated ids, the final hidden state,
norm_out and the whole K/V cache. The device's free memory is the same before
and after those two calls (their output buffers are made first). A one-step
call comes first: it makes the library's per-device set-up (a placement probe
written into the fixed array, no allocation by the library) and, in a fresh
process, the HIP runtime's one-time load of the library's device code and
static arrays (the fixed array among them) at its first kernel launch, which
changes the device's free memory once (14 MiB measured; every later call of
the entry point, of any size, changes nothing). Run after the other GPU tests
(the usual order), both have already happened. Under stream capture the entry
point is refused.
"""

import ctypes
import math
import os

import pytest
import torch

import qwen_weights as qw

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MAX_SEQ = 2048
SCALE = 1.0 / math.sqrt(128)
L = 28


def _bind():
    lib = ctypes.CDLL(os.path.join(REPO, "qwen0.6b_amd", "libqwen_megakernel.so"))
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    for name in ("launch_ldg_generate_nosync", "qwen_generate_nosync_noalloc"):
        fn = getattr(lib, name)
        fn.argtypes = [i32, i32] + [vp] * 19 + [vp, i32, i32, i32, f32, vp]
        fn.restype = i32
    lib.qwen_last_error.restype = i32
    return lib


class State:
    """Caller-owned buffers of one run (the reference's 19 tensors plus the output log)."""

    def __init__(self, w, packed, n):
        f16 = dict(dtype=torch.float16, device="cuda")
        f32 = dict(dtype=torch.float32, device="cuda")
        self.kc = torch.zeros(L, 8, MAX_SEQ, 128, **f16)
        self.vc = torch.zeros_like(self.kc)
        self.hidden = torch.zeros(1024, **f16)
        self.norm_out = torch.zeros(1024, **f32)
        self.unused = torch.zeros(4096, **f32)  # the scratch tensors the engine does not touch
        self.log = torch.full((n,), -1, dtype=torch.int32, device="cuda")
        u = self.unused.data_ptr()
        self.args = [w["embed_weight"].data_ptr(), packed.data_ptr(), w["final_norm_weight"].data_ptr(),
                     w["lm_head_weight"].data_ptr(), w["cos_table"].data_ptr(), w["sin_table"].data_ptr(),
                     self.kc.data_ptr(), self.vc.data_ptr(), self.hidden.data_ptr(), u, u, u, u, u, u, u,
                     self.norm_out.data_ptr(), u, u]


def _call(lib, name, st, first, n, stream=None):
    stream = torch.cuda.current_stream().cuda_stream if stream is None else stream
    return getattr(lib, name)(first, n, *st.args, st.log.data_ptr(), L, 0, MAX_SEQ, SCALE, stream)


def _run(lib, name, w, packed, first, n, st=None):
    st = State(w, packed, n) if st is None else st
    rc = _call(lib, name, st, first, n)
    assert rc == 0, f"{name} returned {rc}"
    torch.cuda.synchronize()
    assert lib.qwen_last_error() == 0
    return st


def test_noalloc_matches_generate_nosync_twice():
    import Qwen06B_architecture as qa

    lib = _bind()
    hw = qw.host_weights(seed=0, std=0.02)
    w = qw.device_weights(hw, "cuda")
    packed = qa._pack_layer_weights(w["layer_weights"])
    ids = qw.synthetic_prompt(2, seed=41)
    cases = [(ids[0], 24), (ids[1], 6)]  # the second call is smaller
    print(f"no-alloc: cases {cases}", flush=True)
    states = [State(w, packed, n) for _, n in cases]
    first = State(w, packed, 1)
    torch.cuda.synchronize()
    before_first = torch.cuda.mem_get_info()[0]
    _run(lib, "qwen_generate_nosync_noalloc", w, packed, ids[0], 1, first)  # set-up (see the module docstring)
    free0 = torch.cuda.mem_get_info()[0]
    print(f"no-alloc: device free memory change at the first call {before_first - free0} B", flush=True)
    got = [_run(lib, "qwen_generate_nosync_noalloc", w, packed, f, n, st) for (f, n), st in zip(cases, states)]
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, f"device free memory changed across the no-allocation calls: {free0} -> {free1}"
    ref = [_run(lib, "launch_ldg_generate_nosync", w, packed, f, n) for f, n in cases]
    for (f, n), a, b in zip(cases, got, ref):
        assert a.log.cpu().tolist() == b.log.cpu().tolist(), (f, n)
        assert int((a.log < 0).sum()) == 0
        assert torch.equal(a.hidden, b.hidden) and torch.equal(a.norm_out, b.norm_out)
        assert torch.equal(a.kc, b.kc) and torch.equal(a.vc, b.vc)
    # and once more after the allocating entry point ran in between
    again = _run(lib, "qwen_generate_nosync_noalloc", w, packed, *cases[1])
    assert again.log.cpu().tolist() == ref[1].log.cpu().tolist()
    assert torch.equal(again.kc, ref[1].kc)


def test_noalloc_refused_under_capture():
    """A replayed graph would reuse the launch's token epochs: the entry point refuses a capturing
    stream (QWEN_ERR_ARG = 1) and records nothing into the graph."""
    import Qwen06B_architecture as qa

    lib = _bind()
    hw = qw.host_weights(seed=0, std=0.02)
    w = qw.device_weights(hw, "cuda")
    packed = qa._pack_layer_weights(w["layer_weights"])
    st = State(w, packed, 2)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(g, stream=side):
        rcs.append(_call(lib, "qwen_generate_nosync_noalloc", st, 1, 2, stream=side.cuda_stream))
    torch.cuda.synchronize()
    assert rcs == [1]
    assert st.log.cpu().tolist() == [-1, -1]
    assert lib.qwen_last_error() == 0
