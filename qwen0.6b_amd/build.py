"""Build recipe for the engine (run from anywhere: ``python qwen0.6b_amd/build.py``).

Produces, next to this file:
  libqwen_megakernel.so                  the HIP kernels + C-ABI (hipcc, gfx950)
  qwen_megakernel_C<ext-suffix>          the pybind11 module over that C-ABI
  layout_check                           host-side exhaustive index checker (run here)

All HIP code is compiled with ``-Xclang -target-feature -Xclang -packed-fp32-ops``
(packed fp32 instructions disabled).
"""

import os
import subprocess
import sys
import sysconfig

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
    return out


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
