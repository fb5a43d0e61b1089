"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the GPU path.

Each oracle function is checked against something that does not restate its own formula:
the reference's own unit-test known answers, a library routine (torch SDPA in float64),
closed forms, invariants, and brute force on tiny inputs.
"""
import numpy as np
import pytest
import torch

from oracle import np_oracle as N
from oracle import oracle as O

NEG = -np.inf


# ---------------------------------------------------------------------------------------------
# BlockTable / config arithmetic: the reference's known answers
# ---------------------------------------------------------------------------------------------

def test_block_table_kat():
    """paged_attention.rs:568-598 (test_block_table): BS=4, blocks [0, 5]."""
    bs = 4
    assert not O.needs_new_block(0, bs)          # empty table
    assert O.needs_new_block(4, bs)              # 4 % 4 == 0 -> next token needs a block
    table = [0]
    assert O.get_block(table, 0, bs) == 0
    assert O.get_block(table, 3, bs) == 0
    assert O.get_slot(0, bs) == 0 and O.get_slot(3, bs) == 3
    table = [0, 5]
    assert O.get_block(table, 4, bs) == 5
    assert O.get_block(table, 5, bs) == 5
    assert O.get_slot(4, bs) == 0 and O.get_slot(5, bs) == 1
    assert not O.needs_new_block(6, bs)
    assert O.get_block(table, 8, bs) is None     # past the table -> None


def test_blocks_needed_kat():
    """paged_attention.rs:623-645 (test_paged_scheduler): 3 tokens -> 1 block, 5 -> 2,
    so a 10-block pool has 10 - 3 = 7 free after both allocations."""
    assert O.blocks_needed(3, 4) == 1
    assert O.blocks_needed(5, 4) == 2
    assert 10 - O.blocks_needed(3, 4) - O.blocks_needed(5, 4) == 7
    assert O.blocks_needed(0, 4) == 0
    assert O.blocks_needed(4, 4) == 1


def test_memory_budget_kat():
    """paged_attention.rs:648-661: 1 GiB, 8 kv heads, D 128, 32 layers, BS 16 -> 256 blocks."""
    assert O.blocks_from_memory_budget(1 << 30, 8, 128, 32, 16) == 256


def test_slot_mapping_closed_form():
    rng = np.random.default_rng(7)
    for bs in (1, 4, 16, 32):
        table = rng.permutation(50)[:9].astype(np.int32)
        n = len(table) * bs
        sm = O.slot_mapping(table, 0, n, bs)
        pos = np.arange(n)
        np.testing.assert_array_equal(sm, table[pos // bs] * bs + pos % bs)
        assert O.slot_mapping(table, n - 1, 2, bs) is None  # second token has no block


# ---------------------------------------------------------------------------------------------
# masks: the reference's known entries, then C vs numpy vs brute force
# ---------------------------------------------------------------------------------------------

def test_causal_mask_kat():
    """transformer.rs:524-536."""
    m = O.causal_mask(4).ravel()
    assert m[0] == 0.0 and m[1] == NEG and m[2] == NEG and m[4] == 0.0 and m[5] == 0.0


def test_sliding_window_mask_kat():
    """transformer.rs:539-561: window 2 on 5x5."""
    m = O.sliding_window_mask(5, 2).ravel()
    assert m[0] == 0.0 and m[1] == NEG
    assert m[15] == NEG and m[16] == 0.0 and m[17] == 0.0 and m[18] == 0.0
    assert m[20] == NEG and m[21] == NEG and m[22] == 0.0 and m[23] == 0.0 and m[24] == 0.0


@pytest.mark.parametrize("n", [1, 2, 7, 33])
def test_masks_brute_force(n):
    np.testing.assert_array_equal(O.causal_mask(n), N.causal_mask(n))
    for w in (0, 1, 3, n + 2):
        np.testing.assert_array_equal(O.sliding_window_mask(n, w), N.sliding_window_mask(n, w))
    for new in range(1, n + 1):
        np.testing.assert_array_equal(O.prefill_causal_mask(new, n), N.prefill_causal_mask(new, n))
        for w in (1, 2, 5):
            np.testing.assert_array_equal(O.sliding_window_prefill_mask(new, n, w),
                                          N.sliding_window_prefill_mask(new, n, w))
    # prefill mask with no cached prefix is the plain causal mask (llama.rs:374-388)
    np.testing.assert_array_equal(O.prefill_causal_mask(n, n), O.causal_mask(n))
    # Gemma-4's window W keeps W keys, the Mistral window W keeps W + 1
    for w in (1, 2, 5):
        np.testing.assert_array_equal(O.sliding_window_prefill_mask(n, n, w + 1),
                                      O.sliding_window_mask(n, w))
    # visible count per row of the causal mask is i + 1
    assert ((O.causal_mask(n) == 0).sum(axis=1) == np.arange(1, n + 1)).all()


# ---------------------------------------------------------------------------------------------
# attention: library routine, closed forms, invariants
# ---------------------------------------------------------------------------------------------

def _rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


def _torch_sdpa_f64(q, k, v, scale, mask):
    """torch's SDPA on the CPU in float64, with repeat_kv done by repeat_interleave."""
    qt = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2)   # [Hq, Sq, D]
    kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2)
    vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2)
    rep = q.shape[1] // k.shape[1]
    kt = kt.repeat_interleave(rep, dim=0)
    vt = vt.repeat_interleave(rep, dim=0)
    am = None if mask is None else torch.from_numpy(mask.astype(np.float64))
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=am, scale=scale)
    return o.permute(1, 0, 2).numpy()


@pytest.mark.parametrize("sq,lk,hq,hkv,d", [(1, 1, 1, 1, 8), (1, 37, 8, 2, 64), (5, 5, 4, 4, 16),
                                            (6, 19, 6, 3, 32), (17, 40, 28, 4, 128)])
def test_attention_f64_vs_torch_sdpa(sq, lk, hq, hkv, d):
    rng = np.random.default_rng(sq * 1000 + lk)
    q, k, v = _rand(rng, sq, hq, d), _rand(rng, lk, hkv, d), _rand(rng, lk, hkv, d)
    scale = d ** -0.5
    # no mask
    np.testing.assert_allclose(O.attention_f64(q, k, v, scale=scale),
                               _torch_sdpa_f64(q, k, v, scale, None), rtol=0, atol=1e-12)
    # chunked-prefill causal (queries are the last sq positions) == prefill_causal_mask
    if sq <= lk:
        ref = _torch_sdpa_f64(q, k, v, scale, O.prefill_causal_mask(sq, lk))
        got = O.attention_f64(q, k, v, scale=scale, causal=True, q_pos0=lk - sq)
        np.testing.assert_allclose(got, ref, rtol=0, atol=1e-12)
        # window rule == explicit Mistral sliding-window mask rows
        w = 3
        full = O.sliding_window_mask(lk, w)[lk - sq:]
        ref = _torch_sdpa_f64(q, k, v, scale, full)
        got = O.attention_f64(q, k, v, scale=scale, causal=True, q_pos0=lk - sq, window_left=w)
        np.testing.assert_allclose(got, ref, rtol=0, atol=1e-12)
        # explicit additive mask path == rule path
        got2 = O.attention_f64(q, k, v, scale=scale, mask=full)
        np.testing.assert_allclose(got2, got, rtol=0, atol=1e-15)


def test_attention_closed_forms():
    rng = np.random.default_rng(3)
    d, hq, hkv = 16, 4, 2
    # one key: the output is that key's value row, whatever q is
    q, k, v = _rand(rng, 3, hq, d), _rand(rng, 1, hkv, d), _rand(rng, 1, hkv, d)
    o = O.attention_f64(q, k, v, scale=0.3)
    for h in range(hq):
        np.testing.assert_allclose(o[:, h], np.broadcast_to(v[0, h // 2], (3, d)), atol=1e-15)
    # identical keys: uniform softmax, output = mean of the values
    k = np.broadcast_to(_rand(rng, 1, hkv, d), (9, hkv, d)).copy()
    v = _rand(rng, 9, hkv, d)
    o = O.attention_f64(q, k, v, scale=0.3)
    for h in range(hq):
        np.testing.assert_allclose(o[:, h], np.broadcast_to(v[:, h // 2].astype(np.float64).mean(0),
                                                             (3, d)), atol=1e-12)
    # one dominant key: output is (numerically) its value row
    k = np.zeros((5, hkv, d), np.float32)
    k[2] = 1.0
    q = np.full((1, hq, d), 10.0, np.float32)
    o = O.attention_f64(q, k, v[:5], scale=1.0)
    for h in range(hq):
        np.testing.assert_allclose(o[0, h], v[2, h // 2], atol=1e-12)
    # no visible key -> zeros; no keys at all -> zeros
    o = O.attention_f64(q, k, v[:5], scale=1.0, causal=True, q_pos0=-1)
    assert (o == 0).all()
    o = O.attention_f64(q, k[:0], v[:0], scale=1.0)
    assert (o == 0).all()


@pytest.mark.parametrize("d,dv", [(40, 160), (64, 24), (16, 16 * 3)])
def test_attention_value_head_dim(d, dv):
    """V with a head dim of its own (flash_attention's val_dim, sketchpad-cubecl
    attention.rs:135-143): the output is linear in V column by column, so it equals the
    equal-dim oracle applied to V's columns in D-wide slices (the last slice zero-padded), and
    float64 SDPA (which takes any value dim) on the whole."""
    rng = np.random.default_rng(d * 10 + dv)
    q, k = _rand(rng, 7, 4, d), _rand(rng, 19, 2, d)
    v = _rand(rng, 19, 2, dv)
    got = O.attention_f64(q, k, v, scale=d ** -0.5, causal=True, q_pos0=12)
    assert got.shape == (7, 4, dv)
    for c0 in range(0, dv, d):
        w = min(d, dv - c0)
        vs = np.zeros((19, 2, d), np.float32)
        vs[:, :, :w] = v[:, :, c0:c0 + w]
        part = O.attention_f64(q, k, vs, scale=d ** -0.5, causal=True, q_pos0=12)
        np.testing.assert_array_equal(got[:, :, c0:c0 + w], part[:, :, :w])
    ref = _torch_sdpa_f64(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1), d ** -0.5,
                          O.prefill_causal_mask(7, 19))
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-12)


def test_attention_gqa_equals_repeated_mha():
    """repeat_kv (transformer.rs:257-271): query head h reads KV head h // (Hq/Hkv)."""
    rng = np.random.default_rng(5)
    q, k, v = _rand(rng, 4, 8, 32), _rand(rng, 11, 2, 32), _rand(rng, 11, 2, 32)
    gqa = O.attention_f64(q, k, v, scale=0.2, causal=True, q_pos0=7)
    mha = O.attention_f64(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), scale=0.2,
                          causal=True, q_pos0=7)
    np.testing.assert_array_equal(gqa, mha)


def test_attention_key_permutation_invariance():
    rng = np.random.default_rng(9)
    q, k, v = _rand(rng, 2, 2, 16), _rand(rng, 13, 1, 16), _rand(rng, 13, 1, 16)
    perm = rng.permutation(13)
    a = O.attention_f64(q, k, v, scale=0.25)
    b = O.attention_f64(q, k[perm], v[perm], scale=0.25)
    np.testing.assert_allclose(a, b, atol=1e-14)


def test_attention_numpy_cross_check_bf16():
    rng = np.random.default_rng(11)
    q, k, v = _rand(rng, 6, 8, 64), _rand(rng, 30, 2, 64), _rand(rng, 30, 2, 64)
    qb, kb, vb = N.f32_to_bf16_bits(q), N.f32_to_bf16_bits(k), N.f32_to_bf16_bits(v)
    got = O.attention_f64(qb, kb, vb, scale=0.125, causal=True, q_pos0=24)
    ref = N.attention(qb, kb, vb, 0.125, N.prefill_causal_mask(6, 30))
    np.testing.assert_allclose(got, ref, atol=1e-12)


def test_attention_f32_refops_within_f32_rounding():
    rng = np.random.default_rng(13)
    q, k, v = _rand(rng, 9, 8, 64), _rand(rng, 250, 8, 64), _rand(rng, 250, 8, 64)
    ref = O.attention_f64(q, k, v, scale=0.125, causal=True, q_pos0=241)
    got = O.attention_f32_refops(q, k, v, scale=0.125, mask=O.prefill_causal_mask(9, 250))
    err = np.abs(got - ref).max(axis=2) / np.abs(ref).max(axis=2)
    assert err.max() < 2e-6


# ---------------------------------------------------------------------------------------------
# store / gather
# ---------------------------------------------------------------------------------------------

def _layout(nb, nl, layer, hkv, bs, d):
    return O.make_layout(nb, nl, layer, hkv, bs, d)


@pytest.mark.parametrize("elem", [np.float32, np.uint16])
def test_store_gather_round_trip(elem):
    rng = np.random.default_rng(17)
    nb, nl, hkv, bs, d = 12, 3, 2, 4, 8
    k_pool = np.zeros((nb, nl, hkv, bs, d), elem)
    v_pool = np.zeros_like(k_pool)
    table = rng.permutation(nb)[:5].astype(np.int32)
    seq = 18
    k = rng.integers(1, 60000, size=(hkv, seq, d)).astype(elem)
    v = rng.integers(1, 60000, size=(hkv, seq, d)).astype(elem)
    lay = _layout(nb, nl, 1, hkv, bs, d)
    assert O.store_kv(k_pool, v_pool, lay, table, k[:, :7], v[:, :7], 0) == 0
    assert O.store_kv(k_pool, v_pool, lay, table, k[:, 7:], v[:, 7:], 7) == 0
    kg, vg = O.gather_kv(k_pool, v_pool, lay, table, seq)
    np.testing.assert_array_equal(kg, k)
    np.testing.assert_array_equal(vg, v)
    # other layers and unused blocks are untouched (pools start at zero, paged_attention.rs:165-185)
    assert (k_pool[:, 0] == 0).all() and (k_pool[:, 2] == 0).all()
    unused = np.setdiff1d(np.arange(nb), table)
    assert (k_pool[unused] == 0).all()
    # numpy restatement agrees on every pool byte
    kp2, vp2 = np.zeros_like(k_pool), np.zeros_like(v_pool)
    N.store_kv(kp2, vp2, 1, table, k, v, 0, bs)
    np.testing.assert_array_equal(kp2, k_pool)
    np.testing.assert_array_equal(vp2, v_pool)
    # concat-cache equivalence (KvCache::update, kv_cache.rs:108-130): prefix gathers are prefixes
    for L in (1, 4, 5, 13):
        kg, _ = O.gather_kv(k_pool, v_pool, lay, table, L)
        np.testing.assert_array_equal(kg, k[:, :L])


def test_store_past_table_fails_like_reference():
    """store_kv panics "Block not allocated" (paged_attention.rs:242) past the table."""
    lay = _layout(4, 1, 0, 1, 4, 4)
    kp = np.zeros((4, 1, 1, 4, 4), np.float32)
    vp = np.zeros_like(kp)
    k = np.ones((1, 6, 4), np.float32)
    assert O.store_kv(kp, vp, lay, [2], k, k, 0) == -1


def test_gather_empty():
    """paged_attention.rs:664-674: empty table -> [Hkv, 0, D]."""
    lay = _layout(10, 2, 0, 8, 4, 64)
    kp = np.zeros((10, 2, 8, 4, 64), np.float32)
    kg, vg = O.gather_kv(kp, kp, lay, [], 0)
    assert kg.shape == (8, 0, 64) and vg.shape == (8, 0, 64)


def test_paged_decode_reference_equals_dense():
    """Decode through the paged pool equals dense attention over the sequence's own rows."""
    rng = np.random.default_rng(23)
    nb, hkv, bs, d, hq = 40, 2, 16, 32, 4
    lens = [1, 16, 17, 70]
    perm = rng.permutation(nb).astype(np.int32)
    tables, off = np.full((4, 5), -1, np.int32), 0
    for s, L in enumerate(lens):
        n = -(-L // bs)
        tables[s, :n] = perm[off:off + n]
        off += n
    k_pool = _rand(rng, nb, 1, hkv, bs, d)
    v_pool = _rand(rng, nb, 1, hkv, bs, d)
    q = _rand(rng, 4, hq, d)
    lay = _layout(nb, 1, 0, hkv, bs, d)
    got = O.paged_decode_f64(q, k_pool, v_pool, lay, tables, np.array(lens), scale=0.2)
    for s, L in enumerate(lens):
        kg, vg = N.gather_kv(k_pool, v_pool, 0, tables[s], L, bs)
        ref = N.attention(q[s:s + 1], kg.transpose(1, 0, 2), vg.transpose(1, 0, 2), 0.2)
        np.testing.assert_allclose(got[s], ref[0], atol=1e-12)


# ---------------------------------------------------------------------------------------------
# the timed CPU baselines (bench.py's cpu_baseline legs) compute the same thing as the oracle
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("window", [-1, 20])
def test_cpu_decode_baseline_matches_oracle(window):
    """spo_cpu_decode_baseline = store the step's token (store_kv) + gather + repeat_kv +
    softmax((q k^T) * scale) v, in f32: within f32 rounding of the f64 oracle, and the append
    lands exactly where the slot mapping says."""
    rng = np.random.default_rng(29)
    nb, hkv, bs, d, hq = 48, 2, 16, 64, 8
    lens = np.array([1, 16, 17, 129, 250], np.int32)
    perm = rng.permutation(nb).astype(np.int32)
    tables, off = np.full((5, 16), -1, np.int32), 0
    for s, L in enumerate(lens):
        n = -(-L // bs)
        tables[s, :n] = perm[off:off + n]
        off += n
    k_pool = _rand(rng, nb, 1, hkv, bs, d).astype(np.float32)
    v_pool = _rand(rng, nb, 1, hkv, bs, d).astype(np.float32)
    q = _rand(rng, 5, hq, d).astype(np.float32)
    kn = _rand(rng, 5, hkv, d).astype(np.float32)
    vn = _rand(rng, 5, hkv, d).astype(np.float32)
    lay = _layout(nb, 1, 0, hkv, bs, d)
    out = np.zeros_like(q)
    kp, vp = k_pool.copy(), v_pool.copy()
    O.cpu_decode_baseline(out, q, kn, vn, kp, vp, lay, tables, lens, scale=d ** -0.5,
                          window_left=window, threads=2)
    # the appended row of every sequence is bit-exact, everything else untouched
    kp_ref, vp_ref = k_pool.copy(), v_pool.copy()
    for s, L in enumerate(lens):
        blk, slot = tables[s, (L - 1) // bs], (L - 1) % bs
        kp_ref[blk, 0, :, slot] = kn[s]
        vp_ref[blk, 0, :, slot] = vn[s]
    np.testing.assert_array_equal(kp, kp_ref)
    np.testing.assert_array_equal(vp, vp_ref)
    ref = O.paged_decode_f64(q, kp_ref, vp_ref, lay, tables, lens, scale=d ** -0.5,
                             window_left=window)
    err = np.abs(out - ref).max(axis=-1) / np.abs(ref).max(axis=-1)
    assert err.max() < 1e-5


def test_cpu_prefill_baseline_matches_oracle():
    """spo_cpu_prefill_baseline = per sequence repeat_kv + [Hq, L, L] scores + causal mask +
    softmax + matmul in f32: within f32 rounding of the f64 oracle."""
    rng = np.random.default_rng(31)
    hq, hkv, d = 8, 2, 32
    lens = [1, 7, 40, 65]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    q = _rand(rng, T, hq, d).astype(np.float32)
    k = _rand(rng, T, hkv, d).astype(np.float32)
    v = _rand(rng, T, hkv, d).astype(np.float32)
    out = np.zeros_like(q)
    O.cpu_prefill_baseline(out, q, k, v, cu, hq=hq, hkv=hkv, d=d, scale=d ** -0.5, threads=2)
    for s in range(len(lens)):
        a, b = cu[s], cu[s + 1]
        ref = O.attention_f64(q[a:b], k[a:b], v[a:b], scale=d ** -0.5, causal=True, q_pos0=0)
        err = np.abs(out[a:b] - ref).max(axis=-1) / np.abs(ref).max(axis=-1)
        assert err.max() < 1e-5, s
