"""GPU parity of the fused decode step (sp_paged_append_decode): the append of each sequence's new
token (store_kv, paged_attention.rs:230-310, at the slot the block table gives position L-1) and
the decode attention (transformer.rs:227-243) in one call must give the same output and the same
pools, bit for bit, as sp_kv_append followed by sp_paged_decode, and match the f64 oracle."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import announce, as_f64, assert_attention_close, host_array, oracle_dtype

pytestmark = pytest.mark.gpu


def _slots(w: W.DecodeWorkload) -> np.ndarray:
    """The append's slot of each sequence's new token (position L-1); -1 (skipped) when L == 0
    or when the block id the table gives lies outside the pool."""
    lens = w.context_lens.astype(np.int64)
    pos = np.maximum(lens - 1, 0)
    blk = w.block_tables[np.arange(w.num_seqs), pos // w.block_size].astype(np.int64)
    ok = (lens > 0) & (blk >= 0) & (blk < w.num_blocks)
    return np.where(ok, blk * w.block_size + pos % w.block_size, -1).astype(np.int32)


def fused_vs_separate(w: W.DecodeWorkload, k_new=None, v_new=None, oracle=True, max_ctx=None,
                      softcap=0.0, qscale=1.0):
    """max_ctx: the max_context_len both calls get (default: the longest context); contexts past
    it are attended up to it, and their new token is still appended at position L - 1.
    softcap: the logit soft cap of both calls; qscale multiplies q."""
    announce(f"append+decode {w.name} B={w.num_seqs} Hq={w.hq} Hkv={w.hkv} D={w.head_dim} "
             f"BS={w.block_size} {w.dtype} window={w.window_left} maxL={w.max_context_len}")
    t = W.make_decode_tensors(w)
    if qscale != 1.0:
        t["q"].mul_(qscale)
    lay = w.layout()
    kn = t["k_new"] if k_new is None else k_new
    vn = t["v_new"] if v_new is None else v_new
    max_ctx = max(w.max_context_len, 1) if max_ctx is None else max_ctx
    scale = w.head_dim ** -0.5
    kp2, vp2 = t["k_pool"].clone(), t["v_pool"].clone()
    out2 = torch.empty_like(t["out"])
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, max_ctx, w.window_left, lay)
    ws2 = sp.alloc_decode_workspace(w.num_seqs, w.hq, max_ctx, w.window_left, lay)
    slots = torch.from_numpy(_slots(w)).cuda()
    # separate: append, then decode
    sp.kv_append(t["k_pool"], t["v_pool"], lay, kn, vn, slots,
                 token_stride=kn.stride(0), head_stride=kn.stride(1))
    sp.paged_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                    t["context_lens"], max_ctx, scale, window_left=w.window_left, workspace=ws,
                    softcap=softcap)
    # fused
    sp.paged_append_decode(out2, t["q"], kp2, vp2, lay, kn, vn, t["block_tables"],
                           t["context_lens"], max_ctx, scale, window_left=w.window_left,
                           workspace=ws2, softcap=softcap)
    torch.cuda.synchronize()
    assert torch.equal(t["k_pool"], kp2), "K pool differs"
    assert torch.equal(t["v_pool"], vp2), "V pool differs"
    assert torch.equal(t["out"], out2), "output differs from append + decode"
    if not oracle:  # block ids outside the pool: the reference panics, the oracle has no answer
        return t, out2
    olay = O.make_layout(w.num_blocks, w.num_layers, w.layer, w.hkv, w.block_size, w.head_dim)
    ref = O.paged_decode_f64(host_array(t["q"]), host_array(kp2), host_array(vp2), olay,
                             w.block_tables, np.minimum(w.context_lens, max_ctx), scale=scale,
                             window_left=w.window_left, dtype=oracle_dtype(t["q"]),
                             softcap=softcap)
    assert_attention_close(as_f64(out2), ref, w.dtype, w.name)
    return t, out2


def test_append_decode_c1_f32():
    fused_vs_separate(W.decode_c1())


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (32, 8), (28, 4)])
@pytest.mark.parametrize("d", [64, 128])
def test_append_decode_random_shapes(dtype, hq, hkv, d):
    w = W.random_decode(seed=hq * 17 + hkv * 3 + d + 5000, num_seqs=5, hq=hq, hkv=hkv,
                        head_dim=d, block_size=16, dtype=dtype, min_len=1, max_len=300)
    fused_vs_separate(w)


@pytest.mark.parametrize("window", [0, 15, 16, 100])
def test_append_decode_window(window):
    w = W.random_decode(seed=window + 5100, num_seqs=6, hq=32, hkv=8, head_dim=128,
                        block_size=16, dtype="bf16", min_len=1, max_len=400, window_left=window)
    fused_vs_separate(w)


def test_append_decode_edge_lengths():
    """The new token at every offset of a tile and a block, and alone (L = 1)."""
    lens = np.array([1, 2, 15, 16, 17, 31, 32, 33, 255, 256, 257, 1023, 1024, 1025], np.int32)
    rng = np.random.default_rng(51)
    nblk = int(((lens + 15) // 16).sum())
    tables = W._tables_from_pool(rng, lens, 16, nblk)
    w = W.DecodeWorkload("edge-lengths", 51, len(lens), 32, 8, 128, 16, "bf16", lens, tables, nblk)
    fused_vs_separate(w)


def test_append_decode_zero_length_and_out_of_pool_block():
    """L = 0 writes nothing and gives zeros; a last block id outside the pool skips the write
    and masks the tile, exactly as the separate append and decode do."""
    lens = np.array([0, 5, 40, 33, 0, 17], np.int32)
    rng = np.random.default_rng(52)
    nblk = int(((np.maximum(lens, 1) + 15) // 16).sum()) + 2
    tables = W._tables_from_pool(rng, np.maximum(lens, 1), 16, nblk)
    tables[2, (40 - 1) // 16] = -1        # sequence 2's last block: not a pool block
    tables[3, (33 - 1) // 16] = nblk      # sequence 3's last block: one past the pool
    w = W.DecodeWorkload("zero-len-oob", 52, 6, 8, 2, 64, 16, "bf16", lens, tables, nblk)
    _, out = fused_vs_separate(w, oracle=False)
    o = as_f64(out)
    assert (o[0] == 0).all() and (o[4] == 0).all()


def test_append_decode_context_past_max_context_len():
    """context_lens above max_context_len: both paths append the token at position L - 1 and
    attend the first max_context_len keys only, so the fused call writes no attended row (the
    token's slot lies past them) and matches the two calls bit for bit."""
    lens = np.array([40, 300, 129, 17, 300], np.int32)
    rng = np.random.default_rng(53)
    nblk = int(((lens + 15) // 16).sum())
    tables = W._tables_from_pool(rng, lens, 16, nblk)
    w = W.DecodeWorkload("past-max-ctx", 53, len(lens), 16, 4, 128, 16, "bf16", lens, tables, nblk)
    t, _ = fused_vs_separate(w, max_ctx=129)
    # sequence 1's new row landed at position 299, past the attended 129 keys
    kp = host_array(t["k_pool"])
    blk = int(tables[1, 299 // 16])
    assert np.array_equal(kp[blk, 0, :, 299 % 16], host_array(t["k_new"])[1])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("bs", [1, 4, 8, 12, 24])
def test_append_decode_block_sizes_off_the_tile(dtype, bs):
    """Tiles spanning several blocks or straddling a block edge: the new token's row comes from
    k_new / v_new whatever block of its tile holds it."""
    fused_vs_separate(W.random_decode(seed=5500 + bs + len(dtype), num_seqs=6, hq=16, hkv=4,
                                      head_dim=128, block_size=bs, dtype=dtype, min_len=1,
                                      max_len=600))


def test_append_decode_block_size_32_and_multi_layer():
    fused_vs_separate(W.random_decode(seed=5300, num_seqs=4, hq=32, hkv=8, head_dim=128,
                                      block_size=32, dtype="bf16", min_len=1, max_len=700))
    fused_vs_separate(W.random_decode(seed=5301, num_seqs=3, hq=16, hkv=4, head_dim=128,
                                      block_size=16, dtype="bf16", min_len=20, max_len=200,
                                      num_layers=4, layer=2))


def test_append_decode_strided_new_rows():
    """k_new / v_new as views with token and head strides of their own."""
    w = W.random_decode(seed=5400, num_seqs=5, hq=32, hkv=8, head_dim=128, block_size=16,
                        dtype="bf16", min_len=1, max_len=500)
    g = torch.Generator(device="cuda")
    g.manual_seed(5400)
    big = torch.randn(w.num_seqs, 3 * w.hkv, w.head_dim, generator=g, device="cuda").bfloat16()
    kn = big[:, 0::3]  # head stride 3 D, token stride 3 Hkv D
    vn = big[:, 1::3]
    assert not kn.is_contiguous()
    fused_vs_separate(w, kn, vn)


def test_append_decode_long_contexts_many_splits():
    fused_vs_separate(W.random_decode(seed=5500, num_seqs=3, hq=32, hkv=8, head_dim=128,
                                      block_size=16, dtype="bf16", min_len=5000, max_len=9000))


@pytest.mark.parametrize("name", ["C2", "C5"])
def test_append_decode_full_size_configs(name):
    fused_vs_separate(W.DECODE_CONFIGS[name]())


def test_append_decode_graph_capture():
    """The fused step captured into a HIP graph through torch: four replays, each after eager
    work that overwrites the output and clears the new rows' pool slots, each giving the eager
    call's output and pools bit for bit."""
    w = W.random_decode(seed=5600, num_seqs=6, hq=32, hkv=8, head_dim=128, block_size=16,
                        dtype="bf16", min_len=1, max_len=3000)
    t = W.make_decode_tensors(w)
    lay = w.layout()
    max_ctx = w.max_context_len
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, max_ctx, -1, lay)
    slots = torch.from_numpy(_slots(w)).long().cuda()

    def call(stream):
        sp.paged_append_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["k_new"],
                               t["v_new"], t["block_tables"], t["context_lens"], max_ctx,
                               w.head_dim ** -0.5, workspace=ws, stream=stream)

    blk, row = slots // w.block_size, slots % w.block_size

    def clear_new_slots():  # pools are [blocks, layers, Hkv, BS, D]
        for pool in (t["k_pool"], t["v_pool"]):
            pool[blk, 0, :, row, :] = 0

    announce("fused append + decode under graph capture")
    call(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = t["out"].clone()
    kp, vp = t["k_pool"].clone(), t["v_pool"].clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call(s.cuda_stream)
    torch.cuda.current_stream().wait_stream(s)
    for r in range(4):
        t["out"].fill_(float("nan"))
        clear_new_slots()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(t["out"], eager), f"replay {r}: output differs from the eager call"
        assert torch.equal(t["k_pool"], kp) and torch.equal(t["v_pool"], vp), \
            f"replay {r}: pools differ from the eager call"
