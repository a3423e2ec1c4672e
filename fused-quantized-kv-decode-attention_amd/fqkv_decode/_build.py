"""In-tree build of the two native libraries of the package.

* ``libfqkv_decode.so`` -- the gfx950 HIP kernels and the C ABI of
  ``include/fqkv_decode.h``, compiled with hipcc for gfx950 only. No PyTorch
  dependency.
* ``_fqkv_torch<ext>.so`` -- the pybind11 PyTorch binding (host C++ compiled
  with g++ against PyTorch's headers), linked to ``libfqkv_decode.so`` with
  an ``$ORIGIN`` rpath.

Both land next to this file so they travel with the source tree. Run
``python -m fqkv_decode._build`` (from the package's parent directory) or
call ``build()``.
"""

import os
import subprocess
import sys
import sysconfig

from ._paths import EXT_NAME, LIB_NAME, PKG_DIR, ext_filename

ROOT = os.path.dirname(PKG_DIR)  # fused-quantized-kv-decode-attention_amd/
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(os.path.dirname(ROOT), "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# Every HIP translation unit: gfx950 only, -O3, and no packed-fp32 VALU
# instructions (v_pk_{add,mul,fma}_f32 are disabled on this target).
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=" + ARCH,
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines()
                    if "is not a recognized feature for this target" not in l)
    if res.returncode != 0:
        raise RuntimeError("build step failed (%d): %s\n%s" % (res.returncode, " ".join(cmd), out))
    if verbose and out.strip():
        print(out, flush=True)


def build_hip_lib(verbose=False):
    """Compile the kernels and the C ABI into libfqkv_decode.so."""
    objs = []
    for src in ("decode_kernels.hip", "quant_kernels.hip", "probe_kernels.hip", "capi.cpp"):
        obj = os.path.join(PKG_DIR, "_obj_" + os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC] + HIP_FLAGS + ["-I", INCLUDE, "-I", CSRC, "-x", "hip",
                                     "-c", os.path.join(CSRC, src), "-o", obj]
        _run(cmd, verbose)
        objs.append(obj)
    out = os.path.join(PKG_DIR, LIB_NAME)
    tmp = out + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + objs
         + ["-Wl,-soname," + LIB_NAME], verbose)
    os.replace(tmp, out)
    for o in objs:
        os.remove(o)
    return out


def build_torch_ext(verbose=False):
    """Compile the pybind11 PyTorch binding against libfqkv_decode.so."""
    import torch
    from torch.utils import cpp_extension

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], INCLUDE,
                                            os.path.join(ROCM, "include")]
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    out = os.path.join(PKG_DIR, ext_filename())
    tmp = out + ".tmp"
    cmd = (["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
            "-D_GLIBCXX_USE_CXX11_ABI=%d" % abi,
            "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=" + EXT_NAME,
            "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-w"]
           + ["-I" + p for p in incs]
           + [os.path.join(CSRC, "torch_binding.cpp"), "-o", tmp,
              "-L" + libdir, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
              "-L" + PKG_DIR, "-lfqkv_decode", "-Wl,-rpath,$ORIGIN"])
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose=False):
    """Build both libraries (always recompiles)."""
    lib = build_hip_lib(verbose)
    ext = build_torch_ext(verbose)
    return lib, ext


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv):
        print("built", p)
