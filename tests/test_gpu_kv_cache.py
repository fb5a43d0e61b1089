"""GPU parity of the cache append (sp_kv_append) and gather (sp_kv_gather): bit-exact against
the oracle's store_kv / gather_kv (paged_attention.rs:230-378)."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import announce, host_array

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _pool(nb, nl, hkv, bs, d, dt, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(nb, nl, hkv, bs, d, generator=g, device="cuda").to(dt)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("layout_kind", ["token_major", "head_major"])
def test_append_bit_exact(dtype, layout_kind):
    nb, nl, layer, hkv, bs, d = 37, 3, 2, 4, 16, 64
    T = 50
    announce(f"append dtype={dtype} layout={layout_kind} T={T}")
    dt = DT[dtype]
    kp, vp = _pool(nb, nl, hkv, bs, d, dt, 1), _pool(nb, nl, hkv, bs, d, dt, 2)
    kp0, vp0 = host_array(kp).copy(), host_array(vp).copy()
    rng = np.random.default_rng(3)
    slots = rng.choice(nb * bs, size=T, replace=False).astype(np.int32)
    slots[[4, 17]] = -1  # skipped tokens
    g = torch.Generator(device="cuda").manual_seed(4)
    if layout_kind == "token_major":
        kn = torch.randn(T, hkv, d, generator=g, device="cuda").to(dt)
        vn = torch.randn(T, hkv, d, generator=g, device="cuda").to(dt)
        ts, hs = hkv * d, d
        k_rows = host_array(kn)                       # [T, Hkv, D]
        v_rows = host_array(vn)
    else:  # the reference's [Hkv, T, D]
        kn = torch.randn(hkv, T, d, generator=g, device="cuda").to(dt)
        vn = torch.randn(hkv, T, d, generator=g, device="cuda").to(dt)
        ts, hs = d, T * d
        k_rows = host_array(kn).transpose(1, 0, 2)
        v_rows = host_array(vn).transpose(1, 0, 2)
    lay = sp.layout(nb, nl, layer, hkv, bs, d)
    sp.kv_append(kp, vp, lay, kn, vn, torch.from_numpy(slots).cuda(), token_stride=ts,
                 head_stride=hs)
    torch.cuda.synchronize()
    # oracle: store each token through a one-block table built from its slot
    olay = O.make_layout(nb, nl, layer, hkv, bs, d)
    for t in range(T):
        if slots[t] < 0:
            continue
        blk, s = divmod(int(slots[t]), bs)
        k_t = np.ascontiguousarray(k_rows[t][:, None, :])   # [Hkv, 1, D]
        v_t = np.ascontiguousarray(v_rows[t][:, None, :])
        assert O.store_kv(kp0, vp0, olay, [blk], k_t, v_t, s) == 0
    np.testing.assert_array_equal(host_array(kp), kp0)
    np.testing.assert_array_equal(host_array(vp), vp0)


def test_append_skips_out_of_range_slots():
    nb, hkv, bs, d = 4, 2, 16, 128
    announce("append out-of-range slots")
    kp = torch.zeros(nb, 1, hkv, bs, d, dtype=torch.bfloat16, device="cuda")
    vp = torch.zeros_like(kp)
    kn = torch.ones(3, hkv, d, dtype=torch.bfloat16, device="cuda")
    slots = torch.tensor([nb * bs, nb * bs + 100, 5], dtype=torch.int32, device="cuda")
    sp.kv_append(kp, vp, sp.layout(nb, 1, 0, hkv, bs, d), kn, kn, slots)
    torch.cuda.synchronize()
    assert kp.float().sum().item() == hkv * d  # only slot 5 written
    assert (kp[0, 0, :, 5] == 1).all()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("seq_len", [1, 15, 16, 17, 250])
def test_gather_bit_exact(dtype, seq_len):
    nb, nl, layer, hkv, bs, d = 40, 2, 1, 8, 16, 64
    announce(f"gather dtype={dtype} seq_len={seq_len}")
    dt = DT[dtype]
    kp, vp = _pool(nb, nl, hkv, bs, d, dt, 5), _pool(nb, nl, hkv, bs, d, dt, 6)
    rng = np.random.default_rng(seq_len)
    nblk = -(-seq_len // bs)
    table = rng.permutation(nb)[:nblk].astype(np.int32)
    ko = torch.empty(hkv, seq_len, d, dtype=dt, device="cuda")
    vo = torch.empty_like(ko)
    lay = sp.layout(nb, nl, layer, hkv, bs, d)
    sp.kv_gather(ko, vo, kp, vp, lay, torch.from_numpy(table).cuda(), seq_len)
    torch.cuda.synchronize()
    olay = O.make_layout(nb, nl, layer, hkv, bs, d)
    kr, vr = O.gather_kv(host_array(kp), host_array(vp), olay, table, seq_len)
    np.testing.assert_array_equal(host_array(ko), kr)
    np.testing.assert_array_equal(host_array(vo), vr)


def test_append_then_gather_round_trip_c1():
    """C1: append the step's token of every sequence, then gather each sequence: the last row of
    every gathered sequence is the appended row and the rest is untouched pool content."""
    w = W.decode_c1()
    announce(f"append+gather round trip {w.name}")
    t = W.make_decode_tensors(w)
    before = host_array(t["k_pool"]).copy()
    lay = w.layout()
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])
    for s in range(w.num_seqs):
        L = int(w.context_lens[s])
        ko = torch.empty(w.hkv, L, w.head_dim, dtype=torch.float32, device="cuda")
        vo = torch.empty_like(ko)
        sp.kv_gather(ko, vo, t["k_pool"], t["v_pool"], lay, t["block_tables"][s], L)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host_array(ko)[:, L - 1], host_array(t["k_new"])[s])
        np.testing.assert_array_equal(host_array(vo)[:, L - 1], host_array(t["v_new"])[s])
        olay = O.make_layout(w.num_blocks, 1, 0, w.hkv, w.block_size, w.head_dim)
        kr, _ = O.gather_kv(before, before, olay, w.block_tables[s], L)
        np.testing.assert_array_equal(host_array(ko)[:, :L - 1], kr[:, :L - 1])
