"""Pinning the oracle's QJL restatement (KvQuantMethod::QJL, kv_cache.rs:300-324, :371-396,
:534-617) without running the reference: the LCG's integer sequence re-derived with Python
integers, its uniforms and Box-Muller values against float64 arithmetic, the reference's own QJL
tests (record size and compression ratio), closed forms of compression (zero, one-hot, scaled and
negated vectors) and decompression (all bits set, zero magnitude), and the Johnson-Lindenstrauss
property of the round trip. The product's host-side projection (sp_qjl_projection) must equal the
oracle's bit for bit."""
import ctypes
import math

import numpy as np
import pytest

from oracle import oracle as O
from sketchpad_amd import _lib

M64 = (1 << 64) - 1


def _lcg_uniforms(n_pairs):
    """(u1, u2) as the reference forms them: 64-bit wrapping LCG from 42, (state >> 11) rounded
    to float32 and divided by 2^53, u1 floored at 1e-10."""
    state, out = 42, []
    for _ in range(n_pairs):
        state = (state * 1664525 + 1013904223) & M64
        u1 = np.float32(np.float32(state >> 11) / np.float32(2.0 ** 53))
        u1 = max(u1, np.float32(1e-10))
        state = (state * 1664525 + 1013904223) & M64
        u2 = np.float32(np.float32(state >> 11) / np.float32(2.0 ** 53))
        out.append((u1, u2))
    return out


def test_lcg_normal_against_float64_box_muller():
    scale = np.float32(math.sqrt(1.0 / 16))
    got = O.qjl_lcg_normal(2000, float(scale))
    pairs = _lcg_uniforms(1000)
    ref = np.empty(2000)
    for i, (u1, u2) in enumerate(pairs):
        r = math.sqrt(-2.0 * math.log(float(u1))) * float(scale)
        t = 2.0 * math.pi * float(u2)
        ref[2 * i], ref[2 * i + 1] = r * math.cos(t), r * math.sin(t)
    # f32 evaluation of the same formula: a few ulp of the value, plus the f32 rounding of the
    # angle 2 pi u2, which moves the value by up to |r| * 2 pi * 2^-24 (~4e-7 |r|)
    radius = np.repeat([math.sqrt(-2.0 * math.log(float(u1))) * float(scale) for u1, _ in pairs], 2)
    tol = 8 * np.spacing(np.abs(ref).astype(np.float32)) + 4e-7 * radius
    assert (np.abs(got - ref) <= tol).all()


def test_lcg_first_value_is_the_floored_uniform():
    """The first uniform of the seed-42 LCG is ~5.9e-11, floored to 1e-10: the first normal is
    sqrt(-2 ln(1e-10)) * scale * cos(2 pi u2) (the reference's own first sample)."""
    (u1, u2), = _lcg_uniforms(1)
    assert u1 == np.float32(1e-10)
    v = O.qjl_lcg_normal(2, 1.0)
    r = math.sqrt(-2.0 * math.log(float(np.float32(1e-10))))
    assert abs(v[0] - r * math.cos(2 * math.pi * float(u2))) < 4 * np.spacing(np.float32(r))
    assert abs(v[1] - r * math.sin(2 * math.pi * float(u2))) < 4 * np.spacing(np.float32(r))


def test_projection_statistics_and_shape():
    R = O.qjl_projection(64, 128)
    assert R.shape == (64, 128) and R.dtype == np.float32
    # R ~ N(0, 1/proj_dim) (kv_cache.rs:417-421)
    assert abs(R.mean()) < 0.02
    assert abs(R.std() - math.sqrt(1 / 64)) < 0.01
    # odd counts end with the cosine half of a pair
    odd = O.qjl_lcg_normal(7, 1.0)
    assert np.array_equal(odd, O.qjl_lcg_normal(8, 1.0)[:7])


def test_reference_qjl_tests():
    # test_qjl_compressed_kv_cache_shape (kv_cache.rs:846-869): head_dim 32, proj_dim 8 -> 3 bytes
    assert O.qjl_record_bytes(8) == 3
    assert O.qjl_compress(np.ones((4, 32), np.float32), O.qjl_projection(8, 32)).shape == (4, 3)
    # test_qjl_compression_ratio (kv_cache.rs:871-876): (2 + 16/8) / (64*2) = 0.03125
    assert O.qjl_compression_ratio(16, 64) == 0.03125
    assert O.qjl_record_bytes(1) == 3 and O.qjl_record_bytes(9) == 4 and O.qjl_record_bytes(16) == 4


def _bits(rec, p):
    return np.array([(rec[2 + k // 8] >> (k % 8)) & 1 for k in range(p)])


def test_compress_closed_forms():
    P, D = 20, 16
    R = O.qjl_projection(P, D)
    zero = O.qjl_compress(np.zeros(D, np.float32), R)
    assert not zero.any()  # magnitude 0 and no sign bits
    for j in (0, 5, 15):
        e = np.zeros(D, np.float32)
        e[j] = 1.0
        rec = O.qjl_compress(e, R)
        assert rec[0] == 0x00 and rec[1] == 0x3C  # binary16 1.0, little-endian
        assert np.array_equal(_bits(rec, P), (R[:, j] >= 0).astype(int))
        assert rec[2 + P // 8] >> (P % 8) == 0    # unused high bits of the last byte stay 0
    rng = np.random.default_rng(1)
    x = rng.standard_normal((50, D)).astype(np.float32)
    dots = x.astype(np.float64) @ R.astype(np.float64).T
    clear = np.abs(dots) > 1e-4  # away from ties, the sign equals the float64 dot's
    rec = O.qjl_compress(x, R)
    for i in range(50):
        b = _bits(rec[i], P)
        assert np.array_equal(b[clear[i]], (dots[i] >= 0)[clear[i]].astype(int))
        neg = _bits(O.qjl_compress(-x[i], R), P)
        assert np.array_equal(neg[clear[i]], 1 - b[clear[i]])
        sc = O.qjl_compress(np.float32(4.0) * x[i], R)  # power-of-two scaling: same signs
        assert np.array_equal(_bits(sc, P), b)
        m = O.f16_bits_to_f32(int(rec[i][0]) | (int(rec[i][1]) << 8))
        assert abs(m - np.linalg.norm(x[i].astype(np.float64))) <= 1e-3 * m


def test_decompress_closed_forms():
    P, D = 12, 10
    R = O.qjl_projection(P, D)
    rec = np.zeros(O.qjl_record_bytes(P), np.uint8)
    rec[0], rec[1] = 0x00, 0x40  # binary16 2.0
    rec[2], rec[3] = 0xFF, 0x0F  # all 12 bits set
    got = O.qjl_decompress(rec, R)
    scale = 2.0 * np.float32(np.float32(math.pi / 2) / np.float32(P))
    ref = R.astype(np.float64).sum(axis=0) * float(scale)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    rec[0] = rec[1] = 0
    assert not O.qjl_decompress(rec, R).any()  # magnitude 0: zeros whatever the bits


def test_round_trip_preserves_direction():
    """QJL's estimate correlates with the input: cosine similarity of x and decompress(compress(x))
    is positive for every vector and concentrates as the projection grows."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((200, 64)).astype(np.float32)
    cos = []
    for p in (16, 256):
        R = O.qjl_projection(p, 64)
        y = O.qjl_decompress(O.qjl_compress(x, R), R)
        c = (x * y).sum(1) / np.linalg.norm(x, axis=1) / np.linalg.norm(y, axis=1)
        assert (c > 0).all()
        cos.append(c.mean())
    assert cos[1] > cos[0] > 0.3


@pytest.mark.parametrize("p,d", [(8, 32), (16, 64), (32, 128), (100, 37)])
def test_product_projection_equals_oracle(p, d):
    """sp_qjl_projection (the product's host-side generator) is the oracle's matrix bit for bit."""
    lib = _lib.load()
    out = np.zeros((p, d), np.float32)
    assert lib.sp_qjl_projection(out.ctypes.data_as(ctypes.c_void_p), p, d) == _lib.SP_OK
    assert np.array_equal(out.view(np.uint32), O.qjl_projection(p, d).view(np.uint32))
    assert lib.sp_qjl_record_bytes(p) == O.qjl_record_bytes(p)
