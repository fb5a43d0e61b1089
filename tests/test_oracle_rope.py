"""Pins the RoPE oracle (oracle/sp_oracle.c spo_rope_caches / spo_rope_apply, restating
crates/sketchpad-core/src/rope.rs:60-170) without running the reference: the reference's own
rope tests (rope.rs:180-230), exact values at position 0, float64 trigonometry for every table
entry, complex multiplication for the rotation, and the rotation's invariants. Also checks that
the product's host table builder (sp_rope_tables, no GPU needed) matches the restatement."""
import numpy as np
import pytest

from oracle import oracle as O
import sketchpad_amd as sp


def _ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in float32 units in the last place (same-sign, finite values)."""
    ai = a.astype(np.float32).view(np.int32).astype(np.int64)
    bi = b.astype(np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


@pytest.mark.parametrize("head_dim,base", [(4, 10000.0), (64, 10000.0), (128, 500000.0)])
def test_rope_caches_position_zero_and_pairs(head_dim, base):
    cos, sin = O.rope_caches(64, head_dim, base)
    # position 0: every angle is 0 -> cos 1, sin 0 exactly
    assert (cos[0] == 1.0).all() and (sin[0] == 0.0).all()
    # each pair's value is stored twice (repeat_interleave, rope.rs:95-102)
    assert (cos[:, 0::2] == cos[:, 1::2]).all() and (sin[:, 0::2] == sin[:, 1::2]).all()
    # pair 0 has inv_freq = base^0 = 1: angle = p, so cos / sin of the integer position
    p = np.arange(64, dtype=np.float64)
    assert _ulp_diff(cos[:, 0], np.cos(p).astype(np.float32)).max() <= 1
    assert _ulp_diff(sin[1:, 0], np.sin(p[1:]).astype(np.float32)).max() <= 1


@pytest.mark.parametrize("head_dim,base", [(64, 10000.0), (128, 10000.0), (128, 1e6)])
def test_rope_caches_match_float64_trigonometry(head_dim, base):
    """Every entry is cos / sin (float64, correctly rounded to f32) of the f32 angle the
    reference forms: inv_freq = 1 / base^(2i/d) in f32, angle = p * inv_freq in f32."""
    rows = 4096
    cos, sin = O.rope_caches(rows, head_dim, base)
    half = head_dim // 2
    i = np.arange(half)
    inv = (np.float32(1.0) / np.power(np.float32(base), (2 * i).astype(np.float32)
                                      / np.float32(head_dim))).astype(np.float32)
    ang = (np.arange(rows, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    ref_c = np.cos(ang.astype(np.float64))
    ref_s = np.sin(ang.astype(np.float64))
    # libm's powf may differ from numpy's float32 power by an ulp in inv_freq, which moves the
    # angle by up to ulp * p: allow that in absolute terms, plus 1 ulp of the result.
    slack = np.abs(ang.astype(np.float64)) * 2.0 ** -23 * 2 + 2.0 ** -24
    assert (np.abs(cos[:, 0::2] - ref_c) <= slack + 1e-7).all()
    assert (np.abs(sin[:, 0::2] - ref_s) <= slack + 1e-7).all()


def test_product_tables_equal_restatement():
    """sp_rope_tables (host part of the C ABI) builds the same fp32 values, one per pair."""
    for head_dim, base in ((64, 10000.0), (128, 10000.0), (128, 500000.0)):
        c_full, s_full = O.rope_caches(9000, head_dim, base)
        c, s = sp.rope_tables(9000, head_dim, base)
        assert np.array_equal(c, c_full[:, 0::2]) and np.array_equal(s, s_full[:, 0::2])


def test_rope_reference_tests():
    """rope.rs:180-230: shapes preserved, zeros stay zeros (with an offset), ones change."""
    cos, sin = O.rope_caches(256, 32)
    z = np.zeros((8, 4, 32), np.float32)
    out = O.rope_apply(z, np.arange(100, 108), cos, sin)
    assert out.shape == z.shape and (out == 0).all()
    cos4, sin4 = O.rope_caches(16, 4)
    ones = np.ones((4, 1, 4), np.float32)
    rot = O.rope_apply(ones, np.arange(4), cos4, sin4)
    assert (np.abs(rot - ones) > 1e-6).any()       # test_rope_modifies_values
    assert (rot[0] == ones[0]).all()               # position 0 is the identity exactly


def test_rope_is_complex_multiplication():
    """(y0 + i y1) = (x0 + i x1) (c + i s) in float64, within f32 rounding of the ops."""
    rng = np.random.default_rng(7)
    cos, sin = O.rope_caches(2048, 128)
    x = rng.standard_normal((64, 8, 128)).astype(np.float32)
    pos = rng.integers(0, 2048, 64).astype(np.int32)
    y = O.rope_apply(x, pos, cos, sin).astype(np.float64)
    z = (x[..., 0::2].astype(np.float64) + 1j * x[..., 1::2]) * \
        (cos[pos][:, None, 0::2].astype(np.float64) + 1j * sin[pos][:, None, 0::2])
    assert np.abs(y[..., 0::2] - z.real).max() < 4e-6
    assert np.abs(y[..., 1::2] - z.imag).max() < 4e-6


def test_rope_invariants():
    rng = np.random.default_rng(11)
    cos, sin = O.rope_caches(4096, 64)
    x = rng.standard_normal((32, 4, 64)).astype(np.float32)
    pos = rng.integers(0, 4096, 32).astype(np.int32)
    y = O.rope_apply(x, pos, cos, sin)
    # pair norms are preserved
    nx = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    ny = y.astype(np.float64)[..., 0::2] ** 2 + y.astype(np.float64)[..., 1::2] ** 2
    assert np.allclose(nx, ny, rtol=1e-5, atol=1e-6)
    # rotating by the negative angle restores x
    back = O.rope_apply(y, pos, cos, -sin)
    assert np.abs(back - x).max() < 1e-5
    # <R(m) q, R(n) k> depends only on m - n
    q = rng.standard_normal((1, 1, 64)).astype(np.float32)
    k = rng.standard_normal((1, 1, 64)).astype(np.float32)
    dots = []
    for m, n in ((10, 3), (107, 100), (2007, 2000)):
        a = O.rope_apply(q, [m], cos, sin).astype(np.float64)
        b = O.rope_apply(k, [n], cos, sin).astype(np.float64)
        dots.append(float((a * b).sum()))
    assert max(dots) - min(dots) < 1e-3


def test_rope_apply_numpy_restatement_bit_exact():
    """The apply step restated with numpy float32 elementwise ops (no contraction) matches."""
    rng = np.random.default_rng(5)
    cos, sin = O.rope_caches(512, 128)
    x = rng.standard_normal((40, 6, 128)).astype(np.float32)
    pos = rng.integers(0, 512, 40).astype(np.int32)
    y = O.rope_apply(x, pos, cos, sin)
    c = cos[pos][:, None, :]
    s = sin[pos][:, None, :]
    rot = np.empty_like(x)
    rot[..., 0::2] = -x[..., 1::2]
    rot[..., 1::2] = x[..., 0::2]
    ref = (x * c).astype(np.float32) + (rot * s).astype(np.float32)
    assert np.array_equal(y, ref)


def test_rope_apply_rejects_positions_outside_the_caches():
    cos, sin = O.rope_caches(8, 4)
    with pytest.raises(ValueError):
        O.rope_apply(np.ones((1, 1, 4), np.float32), [8], cos, sin)
