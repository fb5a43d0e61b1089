"""GPU parity of the PolarQuant compressed paged cache (include/sketchpad_attn.h, sp_polar_*)
against the oracle's restatement of polar_quant_compress / polar_quant_decompress
(kv_cache.rs:437-532):
  - compression, encode-on-append and export are bit-exact: the records equal the oracle's bytes
    for the same f32 rows (bf16 / f16 inputs are converted exactly first);
  - decompression and the decompressing gather are bit-exact in f32 and equal the f32 value
    rounded once for bf16 / f16;
  - the pool layout documented in the header is read back on the host and equals the export;
  - decode attention on the codes matches float64 attention over the oracle-decompressed keys and
    values (the reference's CompressedKvCache + forward_cached): within 2e-2 absolute on
    unit-scale data, and on data with row norms spread over e^(0.5 N(0,1)) within a per-output
    bound derived from the kernel's rounding points (polar_error_bound), with the worst measured
    error and its ratio to the bound printed."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import LOWP_ABS_TOL, announce, as_f64

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _edge_rows(d: int) -> np.ndarray:
    """Rows that exercise every branch of the encoder (zero, one-hot, half-way codes, f32
    subnormal squares, underflow to zero, binary16 overflow / subnormal magnitudes)."""
    rows = [np.zeros(d), np.eye(1, d, d // 2)[0] * -3.0]
    if d >= 4:
        r = np.zeros(d)
        r[:4] = [5, 11, -5, 5]  # |x| = 14: 5 * (1/14) * 7 == 2.5 exactly -> code 3
        rows.append(r)
    rows += [np.full(d, 1e-20), np.full(d, 1e-30), np.full(d, 1e4), np.full(d, 3e-6),
             np.linspace(-1, 1, d) * 1e-3]
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("d", [3, 64, 128, 255])
def test_compress_bit_exact(dtype, d):
    announce(f"polar compress {dtype} D={d}")
    g = torch.Generator(device="cuda").manual_seed(d * 3 + len(dtype))
    x = torch.randn(700, d, generator=g, device="cuda") * torch.exp(
        torch.randn(700, 1, generator=g, device="cuda") * 3)
    if dtype == "f32":
        edge = _edge_rows(d)
        x[:len(edge)] = torch.from_numpy(edge).cuda()
    x = x.to(DT[dtype])
    rec = torch.empty(700, sp.polar_record_bytes(d), dtype=torch.uint8, device="cuda")
    sp.polar_compress(rec, x)
    torch.cuda.synchronize()
    want = O.polar_compress(x.float().cpu().numpy())
    got = rec.cpu().numpy()
    bad = np.nonzero((got != want).any(1))[0]
    assert bad.size == 0, (bad[:4], got[bad[:2]], want[bad[:2]])


def test_compress_nan_rows():
    announce("polar compress NaN rows")
    x = torch.randn(4, 64, device="cuda")
    x[0, 3] = float("nan")
    x[1, :] = float("nan")
    rec = torch.empty(4, 34, dtype=torch.uint8, device="cuda")
    sp.polar_compress(rec, x)
    torch.cuda.synchronize()
    r = rec.cpu().numpy()
    mag = r[:2, 0].astype(np.uint16) | (r[:2, 1].astype(np.uint16) << 8)
    assert ((mag & 0x7C00) == 0x7C00).all() and ((mag & 0x3FF) != 0).all()  # NaN magnitudes
    assert (r[:2, 2:] == 0).all()                                         # NaN codes map to 0
    assert (r[2:] == O.polar_compress(x[2:].cpu().numpy())).all()


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("d", [5, 64, 128])
def test_decompress_bit_exact(dtype, d):
    announce(f"polar decompress {dtype} D={d}")
    rng = np.random.default_rng(d + 17)
    n = 900
    rec = rng.integers(0, 256, size=(n, O.polar_record_bytes(d)), dtype=np.uint8)
    mags = np.concatenate([
        (rng.standard_normal(n - 6) * 10.0 ** rng.integers(-3, 4, n - 6)).astype(np.float16),
        np.array([0.0, -0.0, 6e-8, 1e-5, 65504.0, np.inf], np.float16)]).view(np.uint16)
    mags &= 0x7FFF  # a norm is never negative
    rec[:, 0] = mags & 0xFF
    rec[:, 1] = mags >> 8
    out = torch.empty(n, d, dtype=DT[dtype], device="cuda")
    sp.polar_decompress(out, torch.from_numpy(rec).cuda())
    torch.cuda.synchronize()
    want = torch.from_numpy(O.polar_decompress(rec, d))
    got = out.cpu()
    ref = want.to(DT[dtype])  # one rounding of the f32 value
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan].view(torch.int16 if dtype != "f32" else torch.int32),
                       ref[~nan].view(torch.int16 if dtype != "f32" else torch.int32))


def _read_pool_records(pool: np.ndarray, lay, blk: int, h: int, sl: int, which: str) -> np.ndarray:
    """A vector's record read from a pool per the layout in include/sketchpad_attn.h."""
    bs, d, hkv = lay.block_size, lay.head_dim, lay.num_kv_heads
    hb = d // 2
    region = bs * (hb + 2)
    base = ((blk * lay.num_layers + lay.layer) * hkv + h) * region
    if which == "k":
        codes = pool[base + sl * hb: base + (sl + 1) * hb]
    else:
        q0 = base + (sl // 4) * hb * 4 + sl % 4
        codes = pool[q0: q0 + 4 * hb: 4]
    mag = pool[base + bs * hb + 2 * sl: base + bs * hb + 2 * sl + 2]
    return np.concatenate([mag, codes])


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("d,bs,hkv,layers,layer", [(128, 16, 4, 1, 0), (64, 16, 2, 3, 1),
                                                   (64, 32, 1, 2, 1), (6, 4, 3, 1, 0)])
def test_append_export_gather(dtype, d, bs, hkv, layers, layer):
    announce(f"polar append/export/gather {dtype} D={d} BS={bs} Hkv={hkv} layer={layer}/{layers}")
    rng = np.random.default_rng(d * 7 + bs + hkv)
    num_blocks = 12
    seq_len = 5 * bs - 3
    table = rng.permutation(num_blocks)[:5].astype(np.int32)
    pos = np.arange(seq_len)
    slots = (table[pos // bs] * bs + pos % bs).astype(np.int32)
    T = seq_len + 2
    slots = np.concatenate([slots, [-1, num_blocks * bs]]).astype(np.int32)  # two skipped tokens
    order = rng.permutation(T)  # tokens arrive in any order
    g = torch.Generator(device="cuda").manual_seed(d + bs)
    k = (torch.randn(T, hkv, d, generator=g, device="cuda") * 2).to(DT[dtype])
    v = torch.randn(T, hkv, d, generator=g, device="cuda").to(DT[dtype])
    lay = sp.layout(num_blocks, layers, layer, hkv, bs, d)
    kp, vp = sp.alloc_polar_pools(lay)
    sp.polar_kv_append(kp, vp, lay, k[order].contiguous(), v[order].contiguous(),
                       torch.from_numpy(slots[order]).cuda())
    tab = torch.from_numpy(table).cuda()
    rb = sp.polar_record_bytes(d)
    kr = torch.zeros(hkv, seq_len, rb, dtype=torch.uint8, device="cuda")
    vr = torch.zeros_like(kr)
    sp.polar_kv_export(kr, vr, kp, vp, lay, tab, seq_len)
    kg = torch.empty(hkv, seq_len, d, dtype=DT[dtype], device="cuda")
    vg = torch.empty_like(kg)
    sp.polar_kv_gather(kg, vg, kp, vp, lay, tab, seq_len)
    torch.cuda.synchronize()
    # oracle records of the rows in sequence order, head-major [Hkv, seq_len, rb]
    want_k = O.polar_compress(k[:seq_len].float().cpu().numpy().transpose(1, 0, 2))
    want_v = O.polar_compress(v[:seq_len].float().cpu().numpy().transpose(1, 0, 2))
    assert (kr.cpu().numpy() == want_k).all()
    assert (vr.cpu().numpy() == want_v).all()
    # the documented layout, read on the host, holds the same records
    kpn, vpn = kp.cpu().numpy(), vp.cpu().numpy()
    for p in rng.choice(seq_len, 6, replace=False):
        blk, sl = int(table[p // bs]), int(p % bs)
        for h in range(hkv):
            assert (_read_pool_records(kpn, lay, blk, h, sl, "k") == want_k[h, p]).all()
            assert (_read_pool_records(vpn, lay, blk, h, sl, "v") == want_v[h, p]).all()
    # the skipped tokens wrote nothing: only the seq_len * hkv records are nonzero regions
    used = np.zeros(num_blocks, bool)
    used[table] = True
    per_block = kpn.reshape(num_blocks, -1)
    assert (per_block[~used] == 0).all() and (vpn.reshape(num_blocks, -1)[~used] == 0).all()
    # decompressing gather == oracle decompress, rounded once
    for got, want in ((kg, want_k), (vg, want_v)):
        ref = torch.from_numpy(O.polar_decompress(want, d)).to(DT[dtype])
        assert torch.equal(got.cpu(), ref)


def test_gather_out_of_pool_block_gives_zeros():
    announce("polar gather with an out-of-pool block id")
    lay = sp.layout(4, 1, 0, 2, 16, 64)
    kp, vp = sp.alloc_polar_pools(lay)
    kp.fill_(0x5A)
    vp.fill_(0x5A)
    tab = torch.tensor([1, 99], dtype=torch.int32, device="cuda")
    kr = torch.full((2, 32, 34), 7, dtype=torch.uint8, device="cuda")
    vr = torch.full_like(kr, 7)
    sp.polar_kv_export(kr, vr, kp, vp, lay, tab, 32)
    torch.cuda.synchronize()
    assert (kr[:, 16:].cpu() == 0).all() and (vr[:, 16:].cpu() == 0).all()
    assert (kr[:, :16].cpu() == 0x5A).all()


# --- decode on the codes ----------------------------------------------------------------------

def _polar_decode_case(seed, *, lens, hq, hkv, d, bs, dtype, window=-1, num_layers=1, layer=0,
                       spare_blocks=3, q_scale=1.0, row_spread=0.5):
    announce(f"polar decode seed={seed} B={len(lens)} Hq={hq} Hkv={hkv} D={d} BS={bs} {dtype} "
             f"window={window} maxL={max(lens)} layer={layer}/{num_layers}")
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    nblk = int(((np.maximum(lens, 1) + bs - 1) // bs).sum()) + spare_blocks
    tables = W._tables_from_pool(rng, np.maximum(lens, 1), bs, nblk)
    lay = sp.layout(nblk, num_layers, layer, hkv, bs, d)
    slots = np.concatenate([tables[s, np.arange(L) // bs] * bs + np.arange(L) % bs
                            for s, L in enumerate(lens)]).astype(np.int32)
    T = len(slots)
    g = torch.Generator(device="cuda").manual_seed(seed)
    dt = DT[dtype]
    k = (torch.randn(T, hkv, d, generator=g, device="cuda") *
         torch.exp(torch.randn(T, hkv, 1, generator=g, device="cuda") * row_spread)).to(dt)
    v = (torch.randn(T, hkv, d, generator=g, device="cuda") *
         torch.exp(torch.randn(T, hkv, 1, generator=g, device="cuda") * row_spread)).to(dt)
    q = (torch.randn(len(lens), hq, d, generator=g, device="cuda") * q_scale).to(dt)
    kp, vp = sp.alloc_polar_pools(lay)
    slot_d = torch.from_numpy(slots).cuda()
    sp.polar_kv_append(kp, vp, lay, k, v, slot_d)
    maxL = max(int(lens.max()), 1)
    ws = sp.alloc_decode_workspace(len(lens), hq, maxL, window, lay)
    out = torch.empty(len(lens), hq, d, dtype=dt, device="cuda")
    tab_d = torch.from_numpy(tables).cuda()
    sp.polar_paged_decode(out, q, kp, vp, lay, tab_d, torch.from_numpy(lens).cuda(), maxL,
                          d ** -0.5, window_left=window, workspace=ws)
    torch.cuda.synchronize()
    # reference: dense f32 pools of the oracle-decompressed rows, float64 attention
    kd = O.polar_decompress(O.polar_compress(k.float().cpu().numpy()), d)  # [T, Hkv, D]
    vd = O.polar_decompress(O.polar_compress(v.float().cpu().numpy()), d)
    kpool = np.zeros((nblk, num_layers, hkv, bs, d), np.float32)
    vpool = np.zeros_like(kpool)
    kpool[slots // bs, layer, :, slots % bs] = kd
    vpool[slots // bs, layer, :, slots % bs] = vd
    olay = O.make_layout(nblk, num_layers, layer, hkv, bs, d)
    ref = O.paged_decode_f64(q.float().cpu().numpy(), kpool, vpool, olay, tables, lens,
                             scale=d ** -0.5, window_left=window, dtype=O.F32)
    bound = polar_error_bound(q.float().cpu().numpy(), k.float().cpu().numpy(),
                              v.float().cpu().numpy(), kd, vd, lens, hq, window, dtype)
    return as_f64(out), ref, bound


def polar_error_bound(q, k, v, kd, vd, lens, hq, window, dtype):
    """Per-output bound [B, Hq, D] on |kernel - float64 attention over the decompressed K/V|,
    from the rounding points of polar_decode_kernel (tokens appended sequence by sequence):

      1. P'_j = p_j |v_j| is rounded to bf16 (unit roundoff 2^-8) before the PV MFMA; the bias
         row sums the same rounded P', so the error left is sum_j (P'_j~ - P'_j) n_jd / 7, at
         most 2^-8 * A_d with A_d = sum_j w_j |v_jd| (w the exact softmax weights).
      2. The raw score q . n_j is accumulated in fp32 from -136 sum(q) over D/32 MFMA steps, each
         partial sum below 143 sum|q|: |error| <= (D/32 + 2) * 2 * 2^-24 * 143 * sum|q|, then
         times |k_j|/7 * scale; the fp32 scale product, the exp2 and the offset add a few ulp.
         A score error eps moves each normalised weight by a factor within e^(+-2 eps).
      3. The PV accumulation in fp32 over L/64 + 16 MFMA steps of terms below P'_j * 143, the
         four-wave and split merges, and the f32 rounding of the oracle's decompressed values:
         (L/64 + 40) * 2^-24 * (143/7) * sum_j w_j |v_j|.
      4. The output is rounded once to the storage type (2^-8 bf16, 2^-11 f16).
    Norms are the vectors' binary16 norms (|x| rounded to binary16, times 1 + 2^-10)."""
    B, D = len(lens), q.shape[-1]
    hkv = k.shape[1]
    G = hq // hkv
    scale = D ** -0.5
    u32, u_p = 2.0 ** -24, 2.0 ** -8
    u_out = {"bf16": 2.0 ** -8, "f16": 2.0 ** -11}[dtype]
    knorm = np.float16(np.sqrt((k.astype(np.float64) ** 2).sum(-1))).astype(np.float64)
    vnorm = np.float16(np.sqrt((v.astype(np.float64) ** 2).sum(-1))).astype(np.float64)
    knorm *= 1 + 2.0 ** -10
    vnorm *= 1 + 2.0 ** -10
    offs = np.concatenate([[0], np.cumsum(lens)])
    bound = np.zeros((B, hq, D))
    for s in range(B):
        L = int(lens[s])
        if L == 0:
            continue
        lo = offs[s] + (0 if window < 0 else max(0, L - 1 - window))
        hi = offs[s] + L
        for h in range(hq):
            kh = h // G
            qh = q[s, h].astype(np.float64)
            sc = (kd[lo:hi, kh].astype(np.float64) @ qh) * scale
            w = np.exp(sc - sc.max())
            w /= w.sum()
            A = w @ np.abs(vd[lo:hi, kh].astype(np.float64))
            raw = (D / 32 + 2) * 2 * u32 * 143 * np.abs(qh).sum()
            eps = (raw * knorm[lo:hi, kh] / 7 * scale).max()
            eps += 8 * u32 * (np.abs(sc).max() + 1) + 4 * u32
            eps += 4 * u32 * scale * (np.abs(kd[lo:hi, kh]) @ np.abs(qh)).max()
            acc = (L / 64 + 40) * u32 * (143 / 7) * (w @ vnorm[lo:hi, kh])
            pre = u_p * A + np.expm1(2 * eps) * A + acc
            bound[s, h] = pre + u_out * (np.abs(w @ vd[lo:hi, kh].astype(np.float64)) + pre)
    return bound


def assert_within_bound(got, ref, bound, what):
    """|got - ref| <= bound for every output; prints the worst error and its ratio to the bound."""
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref)
    ratio = (err / np.maximum(bound, 1e-300)).max()
    print(f"[polar-bound] {what}: worst |err| {err.max():.3e}, worst err/bound {ratio:.3f}, "
          f"largest bound {bound.max():.3e}", flush=True)
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} outputs beyond the derived bound, e.g. "
                           f"err {err[bad][:4]} > bound {bound[bad][:4]}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 2), (32, 8), (28, 4), (16, 1)])
@pytest.mark.parametrize("d", [64, 128])
def test_polar_decode_shapes(dtype, hq, hkv, d):
    rng = np.random.default_rng(hq * 31 + hkv + d)
    lens = rng.integers(1, 300, 5)
    got, ref, bound = _polar_decode_case(hq * 31 + hkv + d, lens=lens, hq=hq, hkv=hkv, d=d,
                                        bs=16, dtype=dtype)
    assert_within_bound(got, ref, bound, f"polar decode {dtype} {hq}/{hkv} D={d}")


def test_polar_decode_edge_lengths_and_windows():
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 255, 256, 257, 1023, 1024, 1025]
    got, ref, bound = _polar_decode_case(5, lens=lens, hq=32, hkv=8, d=128, bs=16, dtype="bf16")
    assert_within_bound(got, ref, bound, "edge lengths")
    for window in (0, 15, 16, 100):
        got, ref, bound = _polar_decode_case(6 + window, lens=lens[::2], hq=16, hkv=4, d=128,
                                            bs=16, dtype="bf16", window=window)
        assert_within_bound(got, ref, bound, f"window {window}")


def test_polar_decode_long_contexts_many_splits():
    got, ref, bound = _polar_decode_case(11, lens=[5000, 9000, 7123], hq=32, hkv=8, d=128, bs=16,
                                        dtype="bf16")
    assert_within_bound(got, ref, bound, "long contexts")


def test_polar_decode_multi_layer_block32_and_zero_length():
    got, ref, bound = _polar_decode_case(12, lens=[0, 40, 700, 0, 33], hq=16, hkv=4, d=64, bs=32,
                                        dtype="f16", num_layers=3, layer=2)
    assert (got[0] == 0).all() and (got[3] == 0).all()
    assert_within_bound(got, ref, bound, "multi-layer / block 32 / empty")


def test_polar_decode_large_query_scale():
    """Sharp softmax (large scores): the bias removal happens before the scale, so the scores
    stay exact enough for a near-argmax distribution (the score term of the bound grows with
    sum|q|)."""
    got, ref, bound = _polar_decode_case(13, lens=[100, 333], hq=8, hkv=2, d=128, bs=16,
                                        dtype="bf16", q_scale=8.0)
    assert_within_bound(got, ref, bound, "sharp softmax")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (28, 4, 128), (16, 2, 64)])
def test_polar_decode_unit_scale_holds_abs_bar(dtype, hq, hkv, d):
    """Unit-scale K/V (N(0, 1) rows, no norm spread), C2's length range U[512, 4096] plus three
    short contexts: the plain 16-bit bar, 2e-2 absolute, on every output, besides the derived
    bound. (A one-token context is left to the bound: its output is one value row taken through
    two 16-bit roundings, bf16 P' and the output, up to 2^-7 of |v| ~ 3.)"""
    rng = np.random.default_rng(hq + d)
    lens = np.concatenate([[16, 17, 100], rng.integers(512, 4097, 13)])
    got, ref, bound = _polar_decode_case(40 + hq + d, lens=lens, hq=hq, hkv=hkv, d=d, bs=16,
                                         dtype=dtype, row_spread=0.0)
    assert_within_bound(got, ref, bound, f"unit scale {dtype} {hq}/{hkv} D={d}")
    err = np.abs(got - ref).max()
    assert err <= LOWP_ABS_TOL, f"unit scale: abs error {err:.3e} > {LOWP_ABS_TOL}"
