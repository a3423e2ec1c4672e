"""In-tree build of the native libraries of the package.

* ``libfqkv_decode.so`` -- the gfx950 HIP kernels and the C ABI of
  ``include/fqkv_decode.h``, compiled with hipcc for gfx950 only. No PyTorch
  dependency.
* ``_fqkv_torch<ext>.so`` -- the pybind11 PyTorch binding (host C++ compiled
  with g++ against PyTorch's headers), linked to ``libfqkv_decode.so`` with
  an ``$ORIGIN`` rpath.
* ``libfqkv_decode_timeline.so`` -- the same library with the decode
  kernel compiled with ``-DFQKV_TIMELINE``: each wave stamps the 100 MHz
  real-time counter at the kernel's stages (read back with
  ``fqkv_timeline_read``). A diagnostic build only: nothing in the package
  loads it; ``bench.py --timeline`` does.

All land next to this file so they travel with the source tree. The
translation units compile in parallel. Run
``python -m fqkv_decode._build`` (from the package's parent directory) or
call ``build()``.
"""

import os
import subprocess
import sys
import sysconfig

from ._paths import EXT_NAME, LIB_NAME, PKG_DIR, TIMELINE_LIB_NAME, ext_filename

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


def _filtered(text):
    # hipcc's host pass does not know the -packed-fp32-ops target feature: harmless
    return "\n".join(l for l in text.splitlines()
                     if "is not a recognized feature for this target" not in l)


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = _filtered(res.stdout)
    if res.returncode != 0:
        raise RuntimeError("build step failed (%d): %s\n%s" % (res.returncode, " ".join(cmd), out))
    if verbose and out.strip():
        print(out, flush=True)


def _run_all(cmds, verbose):
    """Run independent compile commands concurrently; raise on the first failure."""
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                            text=True)))
    failed = None
    for cmd, pr in procs:
        out = _filtered(pr.communicate()[0])
        if verbose and out.strip():
            print(out, flush=True)
        if pr.returncode != 0 and failed is None:
            failed = "build step failed (%d): %s\n%s" % (pr.returncode, " ".join(cmd), out)
    if failed:
        raise RuntimeError(failed)


SOURCES = ("decode_kernels.hip", "quant_kernels.hip", "probe_kernels.hip", "capi.cpp")


def _compile_cmd(src, obj, defines=()):
    return ([HIPCC] + HIP_FLAGS + list(defines) + ["-I", INCLUDE, "-I", CSRC, "-x", "hip",
                                                    "-c", os.path.join(CSRC, src), "-o", obj])


def _link(objs, name, verbose):
    out = os.path.join(PKG_DIR, name)
    tmp = out + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + objs
         + ["-Wl,-soname," + name], verbose)
    os.replace(tmp, out)
    return out


def _hip_plan(timeline):
    """(compile commands, objects of libfqkv_decode.so, timeline object or None)."""
    objs = [os.path.join(PKG_DIR, "_obj_" + os.path.splitext(src)[0] + ".o") for src in SOURCES]
    cmds = [_compile_cmd(src, obj) for src, obj in zip(SOURCES, objs)]
    tl_obj = None
    if timeline:
        tl_obj = os.path.join(PKG_DIR, "_obj_decode_kernels_timeline.o")
        cmds.append(_compile_cmd("decode_kernels.hip", tl_obj, ["-DFQKV_TIMELINE"]))
    return cmds, objs, tl_obj


def _link_hip(objs, tl_obj, verbose):
    out = _link(objs, LIB_NAME, verbose)
    if tl_obj:
        # the stamped decode kernel with the other objects of the library
        _link([tl_obj] + objs[1:], TIMELINE_LIB_NAME, verbose)
    return out


def _torch_plan():
    """(compile command, object, link command, output) of the PyTorch binding."""
    import torch
    from torch.utils import cpp_extension

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], INCLUDE,
                                            os.path.join(ROCM, "include")]
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    obj = os.path.join(PKG_DIR, "_obj_torch_binding.o")
    out = os.path.join(PKG_DIR, ext_filename())
    compile_cmd = (["g++", "-O2", "-std=c++17", "-fPIC", "-c",
                    "-D_GLIBCXX_USE_CXX11_ABI=%d" % abi,
                    "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=" + EXT_NAME,
                    "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-w"]
                   + ["-I" + p for p in incs]
                   + [os.path.join(CSRC, "torch_binding.cpp"), "-o", obj])
    link_cmd = (["g++", "-shared", obj, "-o", out + ".tmp",
                 "-L" + libdir, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
                 "-L" + PKG_DIR, "-lfqkv_decode", "-Wl,-rpath,$ORIGIN"])
    return compile_cmd, obj, link_cmd, out


def _remove(paths):
    for o in paths:
        if o and os.path.exists(o):
            os.remove(o)


def build_hip_lib(verbose=False, timeline=True):
    """Compile the kernels and the C ABI into libfqkv_decode.so and, with
    ``timeline``, the stamped decode kernel into libfqkv_decode_timeline.so
    (which shares the other objects)."""
    cmds, objs, tl_obj = _hip_plan(timeline)
    try:
        _run_all(cmds, verbose)
        return _link_hip(objs, tl_obj, verbose)
    finally:
        _remove(objs + [tl_obj])


def build_torch_ext(verbose=False):
    """Compile the pybind11 PyTorch binding against libfqkv_decode.so."""
    compile_cmd, obj, link_cmd, out = _torch_plan()
    try:
        _run(compile_cmd, verbose)
        _run(link_cmd, verbose)
        os.replace(out + ".tmp", out)
    finally:
        _remove([obj])
    return out


def build(verbose=False, timeline=True):
    """Build every library (always recompiles). All objects compile
    concurrently; the links follow, libfqkv_decode.so first."""
    cmds, objs, tl_obj = _hip_plan(timeline)
    t_compile, t_obj, t_link, ext = _torch_plan()
    try:
        _run_all(cmds + [t_compile], verbose)
        lib = _link_hip(objs, tl_obj, verbose)
        _run(t_link, verbose)
        os.replace(ext + ".tmp", ext)
    finally:
        _remove(objs + [tl_obj, t_obj])
    return lib, ext


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv):
        print("built", p)
