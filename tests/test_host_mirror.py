"""The C++ mirror of the reference's paged/flash attention API (sketchpad_amd/host/), through the
test binary tests/cpp/test_paged_attention: the restated reference unit tests of
paged_attention.rs (block table, memory-budget config, causal mask entries, Result errors) on the
CPU, and the device paths on the GPU: allocation and scheduler counts, store/gather round trips,
paged cache == concat cache, flash attention with its options, ragged-batch metadata, a serving
loop driven by a test-local schedule and a three-layer step, checked against the f64 oracle's
attention (oracle/, linked into the binary as its checker)."""
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "build" / "test_paged_attention"


def _run(args):
    if not BIN.exists():
        pytest.fail(f"{BIN} is missing: build it with `python -m tests.build_checkers` "
                    "(or __graft_entry__.build())")
    proc = subprocess.run([str(BIN), *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=300)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout


def test_mirror_reference_unit_tests_cpu():
    """test_block_table, test_config_from_memory_budget, causal mask entries and Result errors."""
    _run(["--cpu-only"])


@pytest.mark.gpu
def test_mirror_device_paths():
    """Every case of the binary, including the pool-backed reference tests and device paths."""
    _run([])
