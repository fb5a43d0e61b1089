"""Seeded random sweeps over the options of the paged paths, each case against the f64 oracle:
  - decode (sp_paged_decode / sp_paged_decode_softcap): dtype, head dim 64 / 128 / 256, GQA
    group, block size 1-64 (multiples of 16 or not), window, the logit soft cap at head dim 256,
    lengths 0-3,000;
  - chunked prefill (sp_paged_prefill / sp_paged_prefill_softcap): head dim, GQA group, block
    size, window, cap, chunk and context lengths, with and without a workspace (key splits);
  - both again at head dim 512 (16-bit), with their own seeds.
Every case prints its draw before the GPU step, so a failure names the parameters."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import announce, as_f64, assert_attention_close, host_array, oracle_dtype
from tests.test_gpu_prefill import run_chunked

pytestmark = pytest.mark.gpu

GROUPS = [(8, 8), (8, 4), (16, 4), (28, 4), (16, 8), (16, 2)]


def _draw_decode(seed, dims=(64, 128, 256)):
    rng = np.random.default_rng(seed)
    d = int(rng.choice(dims))
    dtype = str(rng.choice(["bf16", "f16"] if d >= 256 else ["f32", "bf16", "f16"]))
    hq, hkv = GROUPS[int(rng.integers(len(GROUPS)))]
    bs = int(rng.choice([1, 2, 3, 5, 8, 12, 16, 20, 24, 32, 48, 64]))
    window = int(rng.choice([-1, -1, 0, 7, 100, 1023]))
    cap = float(rng.choice([0.0, 0.0, 5.0, 50.0])) if d >= 256 else 0.0
    return d, dtype, hq, hkv, bs, window, cap, int(rng.integers(1, 9))


@pytest.mark.parametrize("seed", range(24))
def test_random_decode(seed):
    _decode_case(seed, 4000, 4100, (64, 128, 256))


@pytest.mark.parametrize("seed", range(12))
def test_random_decode_d512(seed):
    _decode_case(seed, 6000, 6100, (512,))


def _decode_case(seed, draw_base, data_base, dims):
    d, dtype, hq, hkv, bs, window, cap, nseq = _draw_decode(draw_base + seed, dims)
    w = W.random_decode(seed=data_base + seed, num_seqs=nseq, hq=hq, hkv=hkv, head_dim=d,
                        block_size=bs, dtype=dtype, min_len=0, max_len=3000, window_left=window)
    t = W.make_decode_tensors(w)
    if cap:
        t["q"].mul_(4.0)
    lay = w.layout()
    max_ctx = max(w.max_context_len, 1)
    announce(f"random decode seed={seed}: D={d} {dtype} Hq={hq} Hkv={hkv} BS={bs} window={window} "
             f"cap={cap} lens={list(w.context_lens)}")
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, max_ctx, window, lay)
    sp.paged_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                    t["context_lens"], max_ctx, d ** -0.5, window_left=window, workspace=ws,
                    softcap=cap)
    torch.cuda.synchronize()
    olay = O.make_layout(w.num_blocks, w.num_layers, w.layer, w.hkv, w.block_size, w.head_dim)
    ref = O.paged_decode_f64(host_array(t["q"]), host_array(t["k_pool"]), host_array(t["v_pool"]),
                             olay, w.block_tables, w.context_lens, scale=d ** -0.5,
                             window_left=window, dtype=oracle_dtype(t["q"]), softcap=cap)
    assert_attention_close(as_f64(t["out"]), ref, dtype, f"random decode {seed}")


@pytest.mark.parametrize("seed", range(16))
def test_random_chunked_prefill(seed):
    _chunked_case(seed, 5000, 5100, (64, 128, 256))


@pytest.mark.parametrize("seed", range(8))
def test_random_chunked_prefill_d512(seed):
    _chunked_case(seed, 7000, 7100, (512,))


def _chunked_case(seed, draw_base, data_base, dims):
    rng = np.random.default_rng(draw_base + seed)
    d = int(rng.choice(dims))
    hq, hkv = GROUPS[int(rng.integers(len(GROUPS)))]
    bs = int(rng.choice([4, 8, 12, 16, 24, 32, 64]))
    window = int(rng.choice([-1, -1, 50, 1023]))
    cap = float(rng.choice([0.0, 5.0, 50.0])) if d >= 256 else 0.0
    n = int(rng.integers(1, 5))
    chunks = rng.integers(1, 300, size=n).astype(np.int32)
    ctx = rng.integers(0, 2500, size=n).astype(np.int32)
    split = bool(rng.integers(2)) and d < 256
    w = W.ChunkedPrefillWorkload(f"random-chunked-{data_base + seed}", data_base + seed, chunks,
                                 ctx, hq, hkv, d, "bf16", block_size=bs, window_left=window)
    announce(f"random chunked prefill seed={seed}: D={d} Hq={hq} Hkv={hkv} BS={bs} window={window} "
             f"cap={cap} chunks={list(chunks)} ctx={list(ctx)} split={split}")
    if split:
        lay = sp.layout(1, 1, 0, hkv, bs, d)
        mb = int(((w.context_lens + bs - 1) // bs).max())
        ws = sp.alloc_paged_prefill_workspace(w.num_seqs, w.max_seqlen_q, hq, lay, mb)
        split = ws is not None
    run_chunked(w, split=split, softcap=cap, qscale=4.0 if cap else 1.0)
