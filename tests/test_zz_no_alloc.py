"""sp_paged_decode_noalloc (the decode entry point that allocates nothing: its split partials live
in the library's per-GPU scratch) against sp_paged_decode with a caller-owned workspace, through
the C ABI: two calls in a row, the second on a smaller batch, so the second runs over the first
call's leftover scratch contents. Both entry points plan the same splits, so the outputs must be
bit-identical (stronger than the 2e-2 / 1e-5 attention bar); the first call is also checked
against the f64 oracle."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import announce, as_f64, assert_attention_close, host_array, oracle_dtype

pytestmark = pytest.mark.gpu


def _both(w: W.DecodeWorkload):
    t = W.make_decode_tensors(w)
    lay = w.layout()
    L = max(w.max_context_len, 1)
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])
    assert sp.paged_decode_workspace_size(w.num_seqs, w.hq, L, w.window_left, lay) > 0, \
        "the case must split its keys, so that the scratch holds partials"
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, L, w.window_left, lay)
    ref = torch.full_like(t["out"], float("nan"))
    got = torch.full_like(t["out"], float("nan"))
    announce(f"decode noalloc {w.name} B={w.num_seqs} Hq={w.hq} Hkv={w.hkv} maxL={L}")
    sp.paged_decode(ref, t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                    t["context_lens"], L, w.head_dim ** -0.5, window_left=w.window_left,
                    workspace=ws)
    sp.paged_decode_noalloc(got, t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                            t["context_lens"], L, w.head_dim ** -0.5, window_left=w.window_left)
    torch.cuda.synchronize()
    return t, ref, got


def test_noalloc_decode_matches_workspace_decode_twice():
    # call 1: C2 (64 sequences, Llama-3-8B heads, up to 4096 keys: 8 splits per sequence)
    w1 = W.decode_c2()
    t1, ref1, got1 = _both(w1)
    assert torch.equal(got1, ref1), "noalloc decode differs from sp_paged_decode on C2"
    olay = O.make_layout(w1.num_blocks, w1.num_layers, w1.layer, w1.hkv, w1.block_size,
                         w1.head_dim)
    rows = np.arange(0, w1.num_seqs, 9)
    oracle = O.paged_decode_f64(host_array(t1["q"][rows]), host_array(t1["k_pool"]),
                                host_array(t1["v_pool"]), olay, w1.block_tables[rows],
                                w1.context_lens[rows], scale=w1.head_dim ** -0.5,
                                dtype=oracle_dtype(t1["q"]))
    assert_attention_close(as_f64(got1[rows]), oracle, w1.dtype, "noalloc C2 rows")
    # call 2: a smaller batch (fewer sequences, a window) over the scratch call 1 left behind
    w2 = W.random_decode(seed=777, num_seqs=5, hq=28, hkv=4, head_dim=128, block_size=16,
                         dtype="bf16", min_len=600, max_len=3000, window_left=1500)
    _, ref2, got2 = _both(w2)
    assert torch.equal(got2, ref2), "noalloc decode differs from sp_paged_decode on call 2"


def test_noalloc_decode_rejects_batches_past_the_scratch():
    """256 sequences x 32 heads x 32k keys need 138 MB of partials (32 splits of 64 tiles):
    SP_ENOSPACE, no launch."""
    lay = sp.layout(16, 1, 0, 8, 16, 128)
    need = sp.paged_decode_workspace_size(256, 32, 32768, -1, lay)
    assert need > 32 << 20
    q = torch.zeros(256, 32, 128, dtype=torch.bfloat16, device="cuda")
    pool = torch.zeros(16, 1, 8, 16, 128, dtype=torch.bfloat16, device="cuda")
    tables = torch.zeros(256, 2048, dtype=torch.int32, device="cuda")
    lens = torch.ones(256, dtype=torch.int32, device="cuda")
    with pytest.raises(sp.SketchpadError) as e:
        sp.paged_decode_noalloc(torch.empty_like(q), q, pool, pool, lay, tables, lens, 32768,
                                128 ** -0.5)
    assert e.value.code == sp._lib.SP_ENOSPACE and "scratch" in e.value.message


def test_noalloc_decode_runs_where_only_the_polar_plan_passes_the_scratch():
    """sp_paged_decode_workspace_size covers both pool kinds, so it can exceed the 32 MiB scratch
    for a batch whose dense split plan fits it: 256 sequences x 16 query heads over one KV head
    with max_context_len 19,200 (1,200 tiles) plan 13 dense splits of 96 tiles (28.1 MB of
    partials) against 22 PolarQuant ones of 56 (47.6 MB). The no-allocation call runs such a
    batch (the scratch check is the dense plan's), bit-identical to sp_paged_decode with the
    workspace it asks for."""
    w = W.random_decode(seed=779, num_seqs=256, hq=16, hkv=1, head_dim=128, block_size=16,
                        dtype="bf16", min_len=1, max_len=300)
    max_ctx = 19200
    t = W.make_decode_tensors(w)
    lay = w.layout()
    need = sp.paged_decode_workspace_size(w.num_seqs, w.hq, max_ctx, -1, lay)
    assert need > 32 << 20, need
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, max_ctx, -1, lay)
    ref = torch.full_like(t["out"], float("nan"))
    got = torch.full_like(t["out"], float("nan"))
    # tables as wide as max_context_len needs; the columns past each context are unused (-1)
    tables = torch.full((w.num_seqs, max_ctx // w.block_size), -1, dtype=torch.int32,
                        device="cuda")
    tables[:, :t["block_tables"].shape[1]] = t["block_tables"]
    announce(f"decode noalloc past-polar-plan B={w.num_seqs} Hq={w.hq} maxL={max_ctx}")
    sp.paged_decode(ref, t["q"], t["k_pool"], t["v_pool"], lay, tables,
                    t["context_lens"], max_ctx, w.head_dim ** -0.5, workspace=ws)
    sp.paged_decode_noalloc(got, t["q"], t["k_pool"], t["v_pool"], lay, tables,
                            t["context_lens"], max_ctx, w.head_dim ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
