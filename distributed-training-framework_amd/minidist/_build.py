"""Build libmdx.so (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: ``python -m minidist._build`` or ``minidist._build.build_native()``.
The library lands next to this file, where :mod:`minidist._native` loads it.
Cross-compiles for gfx950 on a machine without a GPU.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
PROJECT_DIR = PKG_DIR.parent
CSRC = PROJECT_DIR / "csrc"
INCLUDE = PROJECT_DIR.parent / "include"
BUILD_DIR = PROJECT_DIR / "_build"
LIB_PATH = PKG_DIR / "libmdx.so"

SOURCES = [
    "mdx_api.hip",
    "mdx_copy.hip",
    "mdx_reduce.hip",
    "mdx_allreduce_f32.hip",
    "mdx_allreduce_bf16.hip",
    "mdx_allreduce_f16.hip",
    "mdx_allreduce_wide.hip",
    "mdx_allreduce_wide_f16.hip",
    "mdx_allreduce_pack.hip",
    "mdx_allreduce_pack_wide.hip",
    "mdx_allreduce_op.hip",
    "mdx_share_fast.hip",
    "mdx_share_generic.hip",
    "mdx_share_generic_bf16.hip",
    "mdx_share_generic_f16.hip",
]
HEADERS = ["mdx_internal.h", "mdx_reduce_impl.h"]

ARCH = "gfx950"

# -ffp-contract=off: x*s + y must stay two roundings, as in the ATen chains.
# -packed-fp32-ops off: no v_pk_* fp32 forms anywhere in this library.
CXXFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: install ROCm or put hipcc on PATH")
    return exe


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *CXXFLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


HOST_HELPER_SRC = CSRC / "host_grad_ptrs.cpp"


def host_helper_path() -> Path:
    return PKG_DIR / ("_hostptrs" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_host_helper() -> Path:
    """Compile the ``_hostptrs`` CPython module (host-only, g++ against torch's headers)."""
    import torch
    import torch.utils.cpp_extension as ce

    libdir = ce.library_paths()[0]
    out = host_helper_path()
    tmp = out.with_suffix(".tmp")
    cmd = [
        shutil.which("g++") or "g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        *[f"-I{d}" for d in ce.include_paths()], f"-I{sysconfig.get_paths()['include']}",
        str(HOST_HELPER_SRC), "-o", str(tmp),
        f"-L{libdir}", f"-Wl,-rpath,{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
    ]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build of {out.name} failed:\n{res.stderr}")
    os.replace(tmp, out)
    return out


def _stale(src: Path, obj: Path) -> bool:
    """True when ``obj`` is missing or older than its source or any shared header."""
    if not obj.exists():
        return True
    deps = [src, *(CSRC / h for h in HEADERS), INCLUDE / "mdx.h"]
    return obj.stat().st_mtime < max(d.stat().st_mtime for d in deps)


def build_native(jobs: int | None = None, incremental: bool = False) -> Path:
    """Compile every translation unit for gfx950 and link ``libmdx.so``.

    ``incremental`` recompiles only the objects older than their source or a
    shared header (and skips the host helper when it exists); the default
    rebuilds everything."""
    BUILD_DIR.mkdir(exist_ok=True)
    objs = [BUILD_DIR / (Path(s).stem + ".o") for s in SOURCES]
    todo = [(s, o) for s, o in zip(SOURCES, objs) if not incremental or _stale(CSRC / s, o)]
    jobs = jobs or max(1, min(len(todo), os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        helper = None if incremental and host_helper_path().exists() else pool.submit(build_host_helper)
        list(pool.map(lambda so: _compile(CSRC / so[0], so[1]), todo))
        if helper is not None:
            helper.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of libmdx.so failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_native(incremental="--incremental" in sys.argv[1:]))
