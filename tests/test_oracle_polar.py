"""Pins the PolarQuant oracle (oracle/sp_oracle.c spo_f32_to_f16_bits, spo_polar_compress /
spo_polar_decompress, restating crates/sketchpad-core/src/kv_cache.rs:437-532 and
KvQuantMethod::compression_ratio at :315-318) without running the reference:
  - the binary16 conversion against numpy's float16 conversion (a library routine), exhaustively
    on the decode side and on ties / overflow / subnormals / NaN on the encode side;
  - records derived by hand from the format (one-hot, negative, zero, odd head_dim, and a code
    that lands exactly on a half, which f32::round takes away from zero);
  - the nibble table: a magnitude of 7 makes the scale exactly 1, so decompression returns the
    codes themselves for every byte value;
  - decompress(compress(x)) within the closed-form bound |x_j - x'_j| <= |x|/14 + |n_j|/7 * |mag
    rounding|, and the codes equal round-half-away(7 x_j / |x|) computed in float64 wherever that
    value is not within float32 noise of a half;
  - record size against compression_ratio; NaN / infinity / underflowing rows.
Also checks that the product's record-size entry point (no GPU needed) agrees."""
import numpy as np
import pytest

from oracle import oracle as O


# --- binary16 conversion ----------------------------------------------------------------------

def test_f16_to_f32_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_bits_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    assert (got[~nan].view(np.uint32) == want[~nan].view(np.uint32)).all()


def _f32_to_f16_numpy(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return x.astype(np.float32).astype(np.float16).view(np.uint16)


def test_f32_to_f16_matches_numpy():
    rng = np.random.default_rng(0)
    f16 = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (f16[:-1] + f16[1:]) / 2  # exact ties between neighbouring binary16 values
    vals = np.concatenate([
        f16, mids, np.nextafter(mids, 0), np.nextafter(mids, np.inf),
        rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
        [65504.0, 65519.0, 65519.99, 65520.0, 65536.0, 1e6, 3e38, 2.0 ** -24, 2.0 ** -25,
         2.0 ** -25 * 1.0000001, 2.0 ** -26, 1e-30, 0.0, 6.0e-8, 6.1e-5, 2.0 ** -14],
    ]).astype(np.float32)
    vals = np.unique(np.concatenate([vals, -vals]))
    vals = np.concatenate([vals, np.array([np.inf, -np.inf], dtype=np.float32)])
    want = _f32_to_f16_numpy(vals)
    got = np.array([O.f32_to_f16_bits(float(v)) for v in vals], dtype=np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(vals[i]), hex(got[i]), hex(want[i])) for i in bad[:5]]


def test_f32_to_f16_nan_stays_nan():
    for v in (float("nan"), -float("nan")):
        h = O.f32_to_f16_bits(v)
        assert (h & 0x7C00) == 0x7C00 and (h & 0x03FF) != 0


# --- records derived by hand --------------------------------------------------------------------

def _rec(x, d=None):
    x = np.asarray([x], dtype=np.float32)
    return [int(b) for b in O.polar_compress(x)[0]]


def test_known_records():
    # [3, 0, 0, 0]: |x| = 3 = binary16 0x4200; codes (7, 0), (0, 0)
    assert _rec([3, 0, 0, 0]) == [0x00, 0x42, 0x70, 0x00]
    # [0, -5, 0, 0]: |x| = 5 = 0x4500; code -7 = nibble 0x9 in the low half of byte 0
    assert _rec([0, -5, 0, 0]) == [0x00, 0x45, 0x09, 0x00]
    # zero row: magnitude 0 and no codes
    assert _rec([0, 0, 0, 0]) == [0, 0, 0, 0]
    # odd head_dim 3: ceil(3/2) = 2 code bytes, the last low nibble stays 0
    assert _rec([0, 0, 2]) == [0x00, 0x40, 0x00, 0x70]
    # [1, 1, 1, 1]: |x| = 2 = 0x4000, each 0.5 * 7 = 3.5 -> 4
    assert _rec([1, 1, 1, 1]) == [0x00, 0x40, 0x44, 0x44]


def test_half_way_code_rounds_away_from_zero():
    """x = [5, 11, -5, 5]: |x| = 14 exactly and float32 5 * (1/14) * 7 evaluates to exactly 2.5
    (checked below), so f32::round gives 3 (ties-to-even would give 2). Codes (3, 6), (-3, 3);
    |x| = 14 = binary16 0x4B00."""
    inv = np.float32(1.0) / np.float32(14.0)
    assert np.float32(np.float32(5.0) * inv) * np.float32(7.0) == np.float32(2.5)
    assert _rec([5, 11, -5, 5]) == [0x00, 0x4B, 0x36, 0xD3]


def test_nibble_table_and_decompress_scale_one():
    """|x| = 7 (binary16 0x4700) makes mag / 7 exactly 1: every byte decodes to its two signed
    nibbles (high nibble first)."""
    recs = np.zeros((256, 3), dtype=np.uint8)
    recs[:, 1] = 0x47
    recs[:, 2] = np.arange(256)
    out = O.polar_decompress(recs, 2)
    hi = np.arange(256) >> 4
    lo = np.arange(256) & 15
    want = np.stack([np.where(hi > 7, hi - 16, hi), np.where(lo > 7, lo - 16, lo)], 1)
    assert (out == want.astype(np.float32)).all()


def test_decompress_known_and_zero_magnitude():
    out = O.polar_decompress(np.array([[0x00, 0x42, 0x70, 0x00]], np.uint8), 4)
    assert out.tolist() == [[3.0, 0.0, 0.0, 0.0]]
    # a zero magnitude gives zeros whatever the codes are (and no -0.0 from negative codes)
    out = O.polar_decompress(np.array([[0x00, 0x00, 0x9F, 0xF1]], np.uint8), 4)
    assert (out.view(np.uint32) == 0).all()


# --- closed-form properties -------------------------------------------------------------------

@pytest.mark.parametrize("d", [2, 7, 64, 128, 257])
@pytest.mark.parametrize("scale", [1e-3, 1.0, 300.0])
def test_round_trip_bound_and_codes(d, scale):
    rng = np.random.default_rng(d * 1000 + int(scale * 7))
    x = (rng.standard_normal((400, d)) * scale).astype(np.float32)
    x[0] = 0.0
    x[1, :] = 0.0
    x[1, d // 2] = -scale  # one-hot
    rec = O.polar_compress(x)
    assert rec.shape == (400, 2 + (d + 1) // 2)
    y = O.polar_decompress(rec, d)
    norm = np.sqrt((x.astype(np.float64) ** 2).sum(1))
    mag = rec[:, 0].astype(np.uint16) | (rec[:, 1].astype(np.uint16) << 8)
    mag = mag.view(np.float16).astype(np.float64)
    # the stored magnitude is |x| rounded to binary16 (relative 2^-11, plus f32 summation slop)
    assert (np.abs(mag - norm) <= norm * (2.0 ** -11 + 1e-6)).all()
    # codes: round half away from zero of 7 x_j / |x| away from ties
    codes = np.zeros((400, 2 * ((d + 1) // 2)), dtype=np.int64)
    codes[:, 0::2] = rec[:, 2:] >> 4
    codes[:, 1::2] = rec[:, 2:] & 15
    codes = np.where(codes > 7, codes - 16, codes)[:, :d]
    with np.errstate(invalid="ignore", divide="ignore"):
        t = 7.0 * x.astype(np.float64) / norm[:, None]
    t = np.nan_to_num(t)
    want = np.sign(t) * np.floor(np.abs(t) + 0.5)
    clear = np.abs(np.abs(t) - np.floor(np.abs(t)) - 0.5) > 1e-5
    assert (codes[clear] == want[clear]).all()
    assert (np.abs(codes) <= 7).all()
    # closed-form reconstruction bound
    err = np.abs(y.astype(np.float64) - x)
    bound = norm[:, None] / 14.0 * (1 + 1e-5) + np.abs(codes) / 7.0 * np.abs(mag - norm)[:, None]
    assert (err <= bound + 1e-30).all()
    # zero row stays zero, one-hot row comes back exactly up to the magnitude rounding
    assert (y[0] == 0).all()
    assert y[1, d // 2] == np.float32(-mag[1]) and (np.delete(y[1], d // 2) == 0).all()


def test_non_finite_and_underflowing_rows():
    x = np.array([[np.inf, 1, 0, 0],
                  [np.nan, 1, 0, 0],
                  [1e-30, 0, 0, 0],       # x^2 underflows to 0 in f32: magnitude 0, no codes
                  [1e-20, 0, 0, 0]],      # x^2 is an f32 subnormal: f32 magnitude 1e-20 (codes
                  np.float32)             # 7) but binary16 flushes it to 0
    rec = O.polar_compress(x)
    assert rec[0].tolist() == [0x00, 0x7C, 0x00, 0x00]  # +inf; inv = 0, codes 0 (inf*0 = NaN -> 0)
    mag1 = int(rec[1, 0]) | (int(rec[1, 1]) << 8)
    assert (mag1 & 0x7C00) == 0x7C00 and (mag1 & 0x3FF) and rec[1, 2:].tolist() == [0, 0]
    assert rec[2].tolist() == [0, 0, 0, 0]
    assert rec[3].tolist() == [0x00, 0x00, 0x70, 0x00]
    y = O.polar_decompress(rec, 4)
    assert (y[2:] == 0).all()                 # zero stored magnitude: zero rows
    assert np.isnan(y[0]).all()               # inf * 0 codes
    assert np.isnan(y[1]).all()


@pytest.mark.parametrize("d", [2, 8, 64, 96, 128, 256])
def test_record_size_matches_compression_ratio(d):
    assert O.polar_record_bytes(d) == 2 + d // 2
    assert O.polar_record_bytes(d) / (2 * d) == O.polar_compression_ratio(d)


def test_compression_ratio_values():
    assert O.polar_compression_ratio(128) == 66 / 256   # ~3.88x fewer bytes than f16
    assert O.polar_compression_ratio(64) == 34 / 128
    # odd head_dim: the reference's formula uses D/2 unrounded, records hold ceil(D/2) bytes
    assert O.polar_record_bytes(3) == 4 and O.polar_compression_ratio(3) == 3.5 / 6


def test_product_record_bytes_matches_oracle(sp_lib):
    for d in (1, 2, 3, 64, 127, 128, 255, 256):
        assert sp_lib.sp_polar_record_bytes(d) == O.polar_record_bytes(d)
    assert sp_lib.sp_polar_record_bytes(0) == -1
