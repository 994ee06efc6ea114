"""Build recipe for the engine (run from anywhere: ``python qwen0.6b_amd/build.py``).

Produces, next to this file:
  libqwen_megakernel.so                  the HIP kernels + C-ABI (hipcc, gfx950)
  qwen_megakernel_C<ext-suffix>          the pybind11 module over that C-ABI
  layout_check                           host-side exhaustive index checker (run here)

All HIP code is compiled with ``-Xclang -target-feature -Xclang -packed-fp32-ops``
(packed fp32 instructions disabled). hipcc passes the flag to both of its
compiler passes; the x86 host pass prints "'-packed-fp32-ops' is not a
recognized feature for this target (ignoring feature)", the gfx950 device pass
applies it. ``audit_device_code`` enforces the result on every build: it reads
the gfx950 code object out of the built library, disassembles it and fails the
build if it holds a packed fp32 add, multiply or fma, or any use of ``m0`` other
than the ``s_mov_b32 m0`` that directly precedes each LDS-DMA load (the one
inline-asm sequence that sets it; hipcc warns about that clobber).
"""

import os
import re
import struct
import subprocess
import sys
import sysconfig
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INC = os.path.join(REPO, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# SimplifyCFG's common-code sinking merges the per-stage-type stores into the
# compute waves' weight prefetch buffer into one store through a phi of
# addresses, which pins that buffer in scratch memory: every prefetch then waits
# for its loads (vmcnt(0)) to spill them and every stage reloads them from
# memory. With sinking off the buffer stays in VGPRs.
NO_SINK = ["-mllvm", "-simplifycfg-sink-common=false"]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_kernels():
    out = os.path.join(HERE, "libqwen_megakernel.so")
    _run([HIPCC, f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared", f"-I{INC}", f"-I{CSRC}",
          *NO_PACKED_FP32, *NO_SINK, os.path.join(CSRC, "megakernel.hip"), "-o", out])
    audit_device_code(out)
    return out


def device_code_object(lib):
    """The gfx950 code object inside a hipcc-built shared library (an uncompressed
    clang offload bundle: 24-byte magic, entry count, then offset/size/triple per entry)."""
    data = open(lib, "rb").read()
    base = data.find(b"__CLANG_OFFLOAD_BUNDLE__")
    if base < 0:
        raise RuntimeError(f"{lib}: no offload bundle found")
    (n,) = struct.unpack_from("<Q", data, base + 24)
    o = base + 32
    for _ in range(n):
        off, size, tlen = struct.unpack_from("<QQQ", data, o)
        o += 24
        triple = data[o:o + tlen].decode()
        o += tlen
        if triple.endswith(ARCH):
            return data[base + off:base + off + size]
    raise RuntimeError(f"{lib}: no {ARCH} code object in the bundle")


def audit_device_code(lib):
    """Disassemble the library's gfx950 code and check two build invariants."""
    objdump = os.path.join(os.path.dirname(os.path.realpath(HIPCC)), "..", "llvm", "bin", "llvm-objdump")
    if not os.path.exists(objdump):
        objdump = "/opt/rocm/llvm/bin/llvm-objdump"
    with tempfile.TemporaryDirectory() as td:
        co = os.path.join(td, "kernel.co")
        with open(co, "wb") as f:
            f.write(device_code_object(lib))
        dis = subprocess.run([objdump, "-d", f"--mcpu={ARCH}", co], check=True, capture_output=True, text=True).stdout
    ins = [ln.split("//")[0].strip() for ln in dis.splitlines() if ln[:1] in ("\t", " ")]
    ins = [x for x in ins if x]
    packed = [x for x in ins if re.match(r"v_pk_(add|mul|fma)_f32\b", x)]
    if packed:
        raise RuntimeError(f"{lib}: {len(packed)} packed fp32 instructions, e.g. {packed[0]}")
    m0_uses = [k for k, x in enumerate(ins) if re.search(r"\bm0\b", x)]
    bad = [ins[k] for k in m0_uses
           if not (ins[k].startswith("s_mov_b32 m0,") and k + 1 < len(ins)
                   and ins[k + 1].startswith("global_load_lds_dwordx4"))]
    if bad:
        raise RuntimeError(f"{lib}: m0 used outside the LDS-DMA sequence: {bad[:3]}")
    print(f"device code audit: {len(ins)} instructions, no packed fp32, m0 set only before "
          f"{len(m0_uses)} LDS-DMA loads", flush=True)


def build_layout_check():
    out = os.path.join(HERE, "layout_check")
    _run(["g++", "-O2", "-std=c++17", f"-I{CSRC}", os.path.join(CSRC, "layout_check.cpp"), "-o", out])
    subprocess.run([out], check=True)
    return out


def build_binding():
    import torch
    from torch.utils import cpp_extension

    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(HERE, "qwen_megakernel_C" + suffix)
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], INC, "/opt/rocm/include"]
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           "-DTORCH_EXTENSION_NAME=qwen_megakernel_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{i}" for i in incs], os.path.join(CSRC, "qwen_ops.cpp"), "-o", out,
           f"-L{libdir}", f"-L{HERE}", "-L/opt/rocm/lib",
           "-lqwen_megakernel", "-ltorch_python", "-ltorch", "-ltorch_cpu", "-lc10_hip", "-lc10", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}", "-Wl,-rpath,/opt/rocm/lib"]
    _run(cmd)
    return out


def build_all():
    build_layout_check()
    build_kernels()
    build_binding()


if __name__ == "__main__":
    build_all()
    sys.exit(0)
