"""Build the test checkers in-tree (test infrastructure, never part of the product):

    oracle/build/libsp_oracle.so           the CPU oracle (oracle/build.sh)
    tests/cpp/build/test_paged_attention   the C++ tests of the host mirror, checked against it

The product (sketchpad_amd/lib/*.so) must be built first (python -m sketchpad_amd.build);
__graft_entry__.build() runs both."""
from __future__ import annotations

from pathlib import Path

from sketchpad_amd import build as product

ROOT = Path(__file__).resolve().parent.parent
ORACLE = ROOT / "oracle"
CPP = Path(__file__).resolve().parent / "cpp"


def build_oracle() -> Path:
    product._run(["bash", str(ORACLE / "build.sh")])
    return ORACLE / "build" / "libsp_oracle.so"


def build_cpp_tests() -> Path:
    """The C++ tests link the host mirror, the kernel library and the oracle (their checker)."""
    srcs = [CPP / "test_paged_attention.cpp", CPP / "test_batching.cpp"]
    exe = CPP / "build" / "test_paged_attention"
    exe.parent.mkdir(parents=True, exist_ok=True)
    product._run([product.HIPCC, *product.DEVICE_FLAGS, f"-I{product.HOST}", f"-I{ORACLE}",
                  "-x", "hip", *map(str, srcs), "-o", str(exe),
                  f"-L{product.LIBDIR}", "-lsketchpad_host", "-lsketchpad_attn",
                  f"-L{ORACLE / 'build'}", "-lsp_oracle",
                  "-Wl,-rpath,$ORIGIN/../../../sketchpad_amd/lib",
                  "-Wl,-rpath,$ORIGIN/../../../oracle/build"])
    return exe


def build_checkers() -> None:
    build_oracle()
    build_cpp_tests()


if __name__ == "__main__":
    build_checkers()
