"""GPU parity of the paged decode (sp_paged_decode) against the oracle's reference decode:
gather_kv per sequence (paged_attention.rs:313-378) then softmax((q k^T) * d^-1/2) v with no mask
(transformer.rs:227-243, llama.rs:255-260), optionally restricted to a Mistral window."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import announce, as_f64, assert_attention_close, host_array, oracle_dtype

pytestmark = pytest.mark.gpu


def run_step(w: W.DecodeWorkload):
    """Append the step's token, then decode; returns the device tensors."""
    t = W.make_decode_tensors(w)
    lay = w.layout()
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, max(w.max_context_len, 1), w.window_left, lay)
    sp.paged_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                    t["context_lens"], max(w.max_context_len, 1), w.head_dim ** -0.5,
                    window_left=w.window_left, workspace=ws)
    torch.cuda.synchronize()
    return t


def reference(w: W.DecodeWorkload, t) -> np.ndarray:
    olay = O.make_layout(w.num_blocks, w.num_layers, w.layer, w.hkv, w.block_size, w.head_dim)
    return O.paged_decode_f64(host_array(t["q"]), host_array(t["k_pool"]), host_array(t["v_pool"]),
                              olay, w.block_tables, w.context_lens, scale=w.head_dim ** -0.5,
                              window_left=w.window_left, dtype=oracle_dtype(t["q"]))


def check(w: W.DecodeWorkload):
    announce(f"decode {w.name} B={w.num_seqs} Hq={w.hq} Hkv={w.hkv} D={w.head_dim} "
             f"BS={w.block_size} {w.dtype} window={w.window_left} maxL={w.max_context_len}")
    t = run_step(w)
    assert_attention_close(as_f64(t["out"]), reference(w, t), w.dtype, w.name)
    return t


def test_decode_c1_f32():
    """The parity config: f32, 4 sequences, L = 17/64/129/250, tolerance 1e-5 relative."""
    check(W.decode_c1())


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (32, 8), (28, 4), (16, 2)])
@pytest.mark.parametrize("d", [64, 128])
def test_decode_random_shapes(dtype, hq, hkv, d):
    g = hq // hkv
    bs = 16
    w = W.random_decode(seed=hq * 131 + hkv * 7 + d, num_seqs=5, hq=hq, hkv=hkv, head_dim=d,
                        block_size=bs, dtype=dtype, min_len=1, max_len=300)
    check(w)


@pytest.mark.parametrize("window", [0, 1, 15, 16, 17, 100])
def test_decode_window(window):
    w = W.random_decode(seed=window + 1000, num_seqs=6, hq=32, hkv=8, head_dim=128,
                        block_size=16, dtype="bf16", min_len=1, max_len=400, window_left=window)
    check(w)


def test_decode_window_f32_tight():
    w = W.random_decode(seed=77, num_seqs=4, hq=8, hkv=8, head_dim=64, block_size=16,
                        dtype="f32", min_len=90, max_len=300, window_left=37)
    check(w)


def test_decode_edge_lengths():
    """Lengths on and around tile / block boundaries, including 1 (only the new token)."""
    lens = np.array([1, 2, 15, 16, 17, 31, 32, 33, 255, 256, 257, 1023, 1024, 1025], np.int32)
    rng = np.random.default_rng(5)
    nblk = int(((lens + 15) // 16).sum())
    tables = W._tables_from_pool(rng, lens, 16, nblk)
    w = W.DecodeWorkload("edge-lengths", 5, len(lens), 32, 8, 128, 16, "bf16", lens, tables, nblk)
    check(w)


def test_decode_zero_length_context_gives_zeros():
    """A sequence with no keys: the reference's matmul over an empty key axis gives zeros."""
    lens = np.array([0, 5, 0, 40], np.int32)
    rng = np.random.default_rng(6)
    nblk = int(((lens + 15) // 16).sum()) + 2
    tables = W._tables_from_pool(rng, np.maximum(lens, 1), 16, nblk)
    w = W.DecodeWorkload("zero-length", 6, 4, 8, 2, 64, 16, "bf16", lens, tables, nblk)
    announce("decode zero-length contexts")
    t = W.make_decode_tensors(w)
    lay = w.layout()
    ws = sp.alloc_decode_workspace(4, 8, 40, -1, lay)
    sp.paged_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                    t["context_lens"], 40, 0.125, workspace=ws)
    torch.cuda.synchronize()
    out = as_f64(t["out"])
    assert (out[0] == 0).all() and (out[2] == 0).all()
    assert_attention_close(out, reference(w, t), "bf16", "zero-length")


def test_decode_multi_layer_pool():
    """The reference's interleaved-layer pool [blocks, layers, Hkv, BS, D]: layer 2 of 4."""
    w = W.random_decode(seed=88, num_seqs=3, hq=16, hkv=4, head_dim=128, block_size=16,
                        dtype="bf16", min_len=20, max_len=200, num_layers=4, layer=2)
    check(w)


def test_decode_block_size_32():
    w = W.random_decode(seed=99, num_seqs=4, hq=32, hkv=8, head_dim=128, block_size=32,
                        dtype="bf16", min_len=1, max_len=700)
    check(w)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("bs", [1, 2, 3, 4, 8, 12, 24, 48])
def test_decode_block_sizes_off_the_tile(dtype, d, bs):
    """Block sizes that are not multiples of the 16-token tile (the reference's BlockTable takes
    any size; its own test uses 4, paged_attention.rs:568-598): every tile then spans several
    blocks of a shuffled table (1-12) or straddles a block edge (24, 48). Lengths cross many
    tile and block edges, and split the keys."""
    w = W.random_decode(seed=600 + bs * 10 + d + len(dtype), num_seqs=6, hq=16, hkv=4,
                        head_dim=d, block_size=bs, dtype=dtype, min_len=1, max_len=1500)
    check(w)


@pytest.mark.parametrize("bs", [4, 8, 12, 24])
def test_decode_block_sizes_off_the_tile_window(bs):
    w = W.random_decode(seed=700 + bs, num_seqs=5, hq=32, hkv=8, head_dim=128, block_size=bs,
                        dtype="bf16", min_len=50, max_len=900, window_left=200)
    check(w)


@pytest.mark.parametrize("bs", [4, 8, 12])
def test_decode_block_sizes_off_the_tile_out_of_pool_block(bs):
    """A block id outside the pool in the middle of a tile masks that block's rows only (the
    reference panics on such an id, "Block not allocated", paged_attention.rs:242; this build
    skips the rows): the output is attention over the sequence's other keys, computed here in
    float64 from the pool."""
    w = W.random_decode(seed=800 + bs, num_seqs=3, hq=8, hkv=2, head_dim=128, block_size=bs,
                        dtype="bf16", min_len=100, max_len=400)
    bad = 16 // bs + 1  # a block of the sequence's second tile (16 // bs + 1 = 2 at 12: keys 24-35)
    w.block_tables[1, bad] = -1
    announce(f"decode sub-tile blocks BS={bs} with block {bad} of sequence 1 outside the pool")
    t = run_step(w)
    got = as_f64(t["out"])
    kp = t["k_pool"].double().cpu().numpy()
    vp = t["v_pool"].double().cpu().numpy()
    q = t["q"].double().cpu().numpy()
    for s_ in range(w.num_seqs):
        L = int(w.context_lens[s_])
        pos = [p for p in range(L) if w.block_tables[s_, p // bs] >= 0]
        blk = [int(w.block_tables[s_, p // bs]) for p in pos]
        for h in range(w.hq):
            kvh = h // (w.hq // w.hkv)
            k = np.stack([kp[b_, 0, kvh, p % bs] for b_, p in zip(blk, pos)])
            v = np.stack([vp[b_, 0, kvh, p % bs] for b_, p in zip(blk, pos)])
            sc = k @ q[s_, h] * w.head_dim ** -0.5
            pr = np.exp(sc - sc.max())
            ref = pr @ v / pr.sum()
            assert np.abs(got[s_, h] - ref).max() <= 2e-2, (s_, h)


def test_decode_many_splits_and_repeat_calls():
    """Long contexts (many split-K partials); a second call on the same workspace matches."""
    w = W.random_decode(seed=321, num_seqs=3, hq=32, hkv=8, head_dim=128, block_size=16,
                        dtype="bf16", min_len=5000, max_len=9000)
    t = check(w)
    first = t["out"].clone()
    lay = w.layout()
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, w.max_context_len, -1, lay)
    sp.paged_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                    t["context_lens"], w.max_context_len, w.head_dim ** -0.5, workspace=ws)
    sp.paged_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                    t["context_lens"], w.max_context_len, w.head_dim ** -0.5, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(first, t["out"])


@pytest.mark.parametrize("name", ["C2", "C4", "C5"])
def test_decode_full_size_configs(name):
    """The decode benchmark configs (C1, C2, C4, C5) at full size against the f64 oracle."""
    check(W.DECODE_CONFIGS[name]())
