"""Build the gfx950 attention library and the C++ host mirror, in-tree.

    python -m sketchpad_amd.build            # both
    python -m sketchpad_amd.build --lib      # only libsketchpad_attn.so

Outputs (git-ignored, but shipped with the tree to the GPU box):
    sketchpad_amd/lib/libsketchpad_attn.so   C-ABI kernels (include/sketchpad_attn.h)
    sketchpad_amd/lib/libsketchpad_host.so   C++ mirror of the reference's paged-cache API
The checkers (the CPU oracle and the C++ tests of the mirror) are built by
tests/build_checkers.py; __graft_entry__.build() builds everything.
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
LIBDIR = PKG / "lib"
OBJDIR = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-fp32 VALU ops (v_pk_add/mul/fma_f32) are switched off for every device pass: some of
# their forms have given silently wrong results on the target machines.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]

LIB_SOURCES = ["kv_cache.hip", "paged_decode.hip", "prefill.hip", "prefill_f32.hip", "rope_append.hip",
               "polar_cache.hip", "qjl.hip", "linear.hip", "capi.cpp"]
HOST_SOURCES = ["paged_attention.cpp", "ragged_batch.cpp"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _compile(src: Path, obj: Path, extra: list[str]) -> Path:
    obj.parent.mkdir(parents=True, exist_ok=True)
    lang = ["-x", "hip"] if src.suffix == ".cpp" else []
    _run([HIPCC, *DEVICE_FLAGS, *extra, *lang, "-c", str(src), "-o", str(obj)])
    return obj


def build_lib(jobs: int = 8) -> Path:
    """Compile the kernels + C ABI into lib/libsketchpad_attn.so."""
    LIBDIR.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(CSRC / s, OBJDIR / (s + ".o"), []), LIB_SOURCES))
    out = LIBDIR / "libsketchpad_attn.so"
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    tmp.replace(out)
    return out


def build_host(jobs: int = 8) -> Path | None:
    """C++ mirror of the reference's PagedKvCache / BlockTable API over the C ABI."""
    srcs = [HOST / s for s in HOST_SOURCES if (HOST / s).exists()]
    if not srcs:
        return None
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, OBJDIR / (s.name + ".o"), [f"-I{HOST}"]), srcs))
    out = LIBDIR / "libsketchpad_host.so"
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
          f"-L{LIBDIR}", "-lsketchpad_attn", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)])
    tmp.replace(out)
    return out


def build_all(jobs: int = 8) -> None:
    build_lib(jobs)
    build_host(jobs)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib", action="store_true", help="only the kernel library")
    ap.add_argument("-j", type=int, default=8)
    args = ap.parse_args()
    if args.lib:
        print(build_lib(args.j))
    else:
        build_all(args.j)


if __name__ == "__main__":
    main()
