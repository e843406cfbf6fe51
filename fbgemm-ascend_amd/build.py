"""In-tree build of the HIP library and its torch binding (no cmake, no JIT cache).

  libtbe_hip.so    hand-written gfx950 kernels + the C ABIs of include/tbe_nbit.h,
                   include/tbe_pooled_ops.h and include/tbe_sparse_ops.h
  _tbe_torch.so    registers fbgemm::int_nbit_split_embedding_codegen_lookup_function
                   for HIP tensors; links libtbe_hip.so through $ORIGIN; also a Python
                   extension module (BoundLookup, the module's forward without the
                   dispatcher)

Both land next to this file so they travel with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO, "include")
HIP_LIB = os.path.join(PKG_DIR, "libtbe_hip.so")
TORCH_LIB = os.path.join(PKG_DIR, "_tbe_torch.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

# hipcc flags for device code: gfx950 only, no packed-fp32 instructions.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if out.strip():
        print(out, flush=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")


HIP_SOURCES = ["tbe_nbit.hip", "tbe_kern_int4.hip", "tbe_kern_int8.hip", "tbe_kern_int2.hip", "tbe_kern_fp8.hip",
               "tbe_kern_fp16.hip", "tbe_kern_fp32.hip", "pooled_ops.hip", "sparse_ops.hip"]
OBJ_DIR = os.path.join(PKG_DIR, "_build")


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer: every flag goes to the host
# compilation only (device code is built exactly as in the product library).
SANITIZE_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-g"]
ASAN_DIR = os.path.join(PKG_DIR, "_asan")
ASAN_LIB = os.path.join(ASAN_DIR, "libtbe_hip.so")


def asan_runtime() -> str:
    """clang's shared ASan runtime (holds the UBSan handlers too); preload it into the
    process that loads ASAN_LIB."""
    import glob
    hits = sorted(glob.glob(os.path.join(ROCM, "llvm", "lib", "clang", "*", "lib", "linux",
                                         "libclang_rt.asan-x86_64.so")))
    if not hits:
        raise FileNotFoundError("clang ASan runtime not found under " + ROCM)
    return hits[-1]


def build_hip_lib(sanitize: bool = False):
    """Compile every HIP source to an object (in parallel), then link one .so
    (sanitize: the host-sanitizer variant, into _asan/)."""
    from concurrent.futures import ThreadPoolExecutor

    obj_dir = OBJ_DIR + ("_asan" if sanitize else "")
    out = ASAN_LIB if sanitize else HIP_LIB
    extra = SANITIZE_FLAGS if sanitize else []
    os.makedirs(obj_dir, exist_ok=True)
    os.makedirs(os.path.dirname(out), exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    objs = [os.path.join(obj_dir, os.path.splitext(s)[0] + ".o") for s in HIP_SOURCES]
    cmds = [[hipcc, *HIP_FLAGS, *extra, "-c", f"-I{INCLUDE}", f"-I{CSRC}", os.path.join(CSRC, s), "-o", o]
            for s, o in zip(HIP_SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        for f in [ex.submit(_run, c) for c in cmds]:
            f.result()
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", *objs, "-o", out]
    if sanitize:
        link[2:2] = ["-fsanitize=address,undefined", "-shared-libsan"]
    _run(link)


def build_torch_binding():
    import torch
    from torch.utils import cpp_extension

    tdir = os.path.dirname(torch.__file__)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=_tbe_torch", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-I{INCLUDE}", f"-I{ROCM}/include", f"-I{sysconfig.get_paths()['include']}"]
    for inc in cpp_extension.include_paths():
        cmd.append(f"-I{inc}")
    cmd += [os.path.join(CSRC, "tbe_torch.cpp"), "-o", TORCH_LIB,
            f"-L{PKG_DIR}", "-ltbe_hip", "-Wl,-rpath,$ORIGIN",
            f"-L{os.path.join(tdir, 'lib')}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch",
            "-ltorch_python"]
    _run(cmd)


def build():
    build_hip_lib()
    build_torch_binding()


def build_sanitized():
    """The host-sanitizer library (_asan/libtbe_hip.so) and oracle (oracle/_build_asan/)."""
    build_hip_lib(sanitize=True)
    _run(["make", "-s", "-C", os.path.join(REPO, "oracle"), "asan"])


if __name__ == "__main__":
    if "--sanitize" in sys.argv[1:]:
        build_sanitized()
    else:
        build()
    sys.exit(0)
