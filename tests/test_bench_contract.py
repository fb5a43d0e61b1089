"""bench.py's contract on the CPU: more than one GPU is refused with a message (this build measures
one GPU), and the algorithmic figures its roofline fractions divide by come out at the sizes the
benchmark configurations define (Llama-3-8B decode and prefill, the Mistral window)."""
import subprocess
import sys
from pathlib import Path

import numpy as np

from sketchpad_amd import workloads as W

ROOT = Path(__file__).resolve().parent.parent


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr
    assert proc.stdout.strip() == ""  # no JSON line for an unmeasured configuration


def test_decode_bytes_c2_c5():
    """C2 reads every cached K/V row once (64 sequences, 8 KV heads, D 128, bf16) plus q, out,
    the table entries walked and the lengths; C5 reads only the 4,097-key window of each of its
    16 sequences. Both land at the sizes the configurations quote (~0.6 GB and ~0.269 GB)."""
    c2 = W.decode_c2()
    L = c2.context_lens.astype(np.int64)
    assert c2.num_seqs == 64 and (c2.hq, c2.hkv, c2.head_dim, c2.block_size) == (32, 8, 128, 16)
    assert L.min() >= 512 and L.max() <= 4096
    kv_rows = int(L.sum()) * 2 * 8              # K and V rows of all KV heads
    assert c2.decode_bytes() == kv_rows * 256 + 64 * 32 * 128 * 2 * 2 + \
        int(((L + 15) // 16).sum()) * 4 + 64 * 4
    assert 0.55e9 < c2.decode_bytes() < 0.65e9

    c5 = W.decode_c5()
    L5 = c5.context_lens.astype(np.int64)
    assert c5.window_left == 4096 and L5.min() >= 8192
    attended = np.minimum(L5, 4097)
    assert (attended == 4097).all()
    assert abs(c5.decode_bytes() - 0.269e9) < 0.002e9


def test_prefill_flops_c3():
    """C3 counts 4 * Hq * D flops per visible (query, key) pair, L(L+1)/2 pairs per causal
    sequence: ~105 GFLOP for 8 sequences of U[256, 2048] tokens (107.0 on the seeded draw)."""
    c3 = W.prefill_c3()
    assert c3.num_seqs == 8 and c3.lens.min() >= 256 and c3.lens.max() <= 2048
    pairs = sum(int(x) * (int(x) + 1) // 2 for x in c3.lens)
    assert c3.flops() == 4 * 32 * 128 * pairs
    assert 95e9 < c3.flops() < 115e9
    # a brute-force count of the causal mask's visible entries on a small sequence
    n = 37
    assert sum(1 for i in range(n) for j in range(n) if j <= i) == n * (n + 1) // 2
