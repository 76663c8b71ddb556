"""Builds the native parts in-tree.

* ``xdna_train/_lib/libxdna_hip.so``: the gfx950 kernels behind the C ABI of
  ``include/xdna_hip.h`` (hipcc, one object per ``csrc/*.hip``, linked together).
* ``xdna_train/_C*.so``: the PrivateUse1 ``xdna`` backend (C++ against the installed
  PyTorch, linked to libxdna_hip.so).

Usage: ``python pytorch-xdna2_amd/build_native.py [--hip-only] [-j N]``.  Every call
compiles (objects are rebuilt when their source or a header changed).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
NATIVE = PKG / "native"
BUILD = PKG / "_build"
LIBDIR = PKG / "xdna_train" / "_lib"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    # Packed-fp32 VALU forms have given silent wrong results on this pool: never emit them.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _digest(paths) -> str:
    h = hashlib.sha256()
    for p in sorted(paths):
        h.update(Path(p).read_bytes())
    h.update(" ".join(HIP_FLAGS).encode())
    return h.hexdigest()[:16]


def _compile_hip(src: Path, headers, force: bool = False) -> Path:
    obj = BUILD / (src.stem + ".o")
    stamp = BUILD / (src.stem + ".stamp")
    key = _digest([src, *headers])
    if not force and obj.exists() and stamp.exists() and stamp.read_text() == key:
        return obj
    cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    stamp.write_text(key)
    return obj


def build_hip(jobs: int = 8, force: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(parents=True, exist_ok=True)
    headers = list(CSRC.glob("*.h")) + [REPO / "include" / "xdna_hip.h"]
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: _compile_hip(s, headers, force), sources))
    out = LIBDIR / "libxdna_hip.so"
    tmp = LIBDIR / "libxdna_hip.so.tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libxdna_hip.so",
           *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build_ext(force: bool = False) -> Path | None:
    """The PrivateUse1 extension (C++ only; calls the kernels through the C ABI)."""
    sources = sorted(NATIVE.glob("*.cpp"))
    if not sources:
        return None
    import ctypes

    from torch.utils import cpp_extension

    # the extension links libxdna_hip.so through $ORIGIN/_lib, which only resolves once
    # it sits in xdna_train/; preload it for the import load() does from the build dir
    ctypes.CDLL(str(LIBDIR / "libxdna_hip.so"), mode=ctypes.RTLD_GLOBAL)
    name = "_C"
    build_dir = BUILD / "ext"
    if force and build_dir.exists():
        shutil.rmtree(build_dir)
    build_dir.mkdir(parents=True, exist_ok=True)
    torch_lib = Path(cpp_extension.library_paths()[0])
    extra_ldflags = [
        f"-L{LIBDIR}",
        "-lxdna_hip",
        "-Wl,-rpath,$ORIGIN/_lib",
        f"-L{torch_lib}",
        "-lc10_hip",
        "-ltorch_hip",
    ]
    mod = cpp_extension.load(
        name=name,
        sources=[str(s) for s in sources],
        extra_cflags=["-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
                      f"-I{REPO / 'include'}", "-I/opt/rocm/include"],
        extra_ldflags=extra_ldflags,
        build_directory=str(build_dir),
        with_cuda=False,
        is_python_module=True,
        verbose=False,
    )
    built = Path(mod.__file__)
    dst = PKG / "xdna_train" / built.name
    shutil.copy2(built, dst)
    return dst


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--hip-only", action="store_true")
    ap.add_argument("--force", action="store_true", help="recompile everything")
    ap.add_argument("-j", type=int, default=int(os.environ.get("MAX_JOBS", "8")))
    args = ap.parse_args()
    lib = build_hip(args.j, args.force)
    print(f"built {lib}")
    if not args.hip_only:
        ext = build_ext(args.force)
        if ext:
            print(f"built {ext}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
