"""Pinning of the oracle's logit soft cap (spo_attention_f64_cap, Gemma-4's attention:
logits = cap * tanh(logits / cap) on the scaled product, before the mask and the softmax,
crates/sketchpad-llm/src/gemma4.rs:366-377). No reference output exists for it (Rust/Burn does
not run here), so it is pinned by what the mathematics fixes:
  - two keys: the weight of key 1 is 1 / (1 + exp(c tanh(l2/c) - c tanh(l1/c))), evaluated with
    math.tanh / math.exp on the logits l = (q . k) * scale;
  - saturation: logits far past +-c weigh exactly as e^{+c}, e^{-c} and e^{0};
  - a cap far above every logit gives the uncapped attention;
  - the cap comes before the mask: a key hidden by the window stays hidden, and an additive mask
    is added to the capped logit (c tanh(l/c) + m, not c tanh((l + m)/c));
  - the numpy restatement agrees on random GQA batches.
A dropped tanh, the cap applied before the scale, or the mask applied before the cap each fail
one of these."""
import math

import numpy as np
import pytest

from oracle import np_oracle as N
from oracle import oracle as O


def _rand(rng, *shape, s=1.0):
    return (rng.standard_normal(shape) * s).astype(np.float32)


@pytest.mark.parametrize("cap", [0.5, 3.0, 50.0])
def test_softcap_two_key_closed_form(cap):
    rng = np.random.default_rng(int(cap * 10))
    d = 8
    q = _rand(rng, 1, 1, d, s=3.0)
    k = _rand(rng, 2, 1, d, s=3.0)
    v = _rand(rng, 2, 1, d)
    scale = 0.37
    l1 = float(np.dot(q[0, 0].astype(np.float64), k[0, 0].astype(np.float64))) * scale
    l2 = float(np.dot(q[0, 0].astype(np.float64), k[1, 0].astype(np.float64))) * scale
    p1 = 1.0 / (1.0 + math.exp(cap * math.tanh(l2 / cap) - cap * math.tanh(l1 / cap)))
    want = p1 * v[0, 0].astype(np.float64) + (1.0 - p1) * v[1, 0].astype(np.float64)
    got = O.attention_f64(q, k, v, scale=scale, softcap=cap)[0, 0]
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-13)
    # and it is not the uncapped weight (the cap matters at these logits)
    p1_plain = 1.0 / (1.0 + math.exp(l2 - l1))
    if abs(p1_plain - p1) > 1e-3:
        plain = O.attention_f64(q, k, v, scale=scale)[0, 0]
        assert np.abs(plain - got).max() > 1e-4


def test_softcap_saturation():
    """Keys whose logits are +-1e4 and 0 under a cap of 5 weigh e^5 : e^-5 : 1."""
    d = 4
    q = np.zeros((1, 1, d), np.float32)
    q[0, 0, 0] = 100.0
    k = np.zeros((3, 1, d), np.float32)
    k[0, 0, 0], k[1, 0, 0], k[2, 0, 0] = 100.0, -100.0, 0.0
    v = np.eye(3, d, dtype=np.float32)[:, None, :]
    cap = 5.0
    got = O.attention_f64(q, k, v, scale=1.0, softcap=cap)[0, 0]
    w = np.array([math.exp(cap), math.exp(-cap), 1.0])
    np.testing.assert_allclose(got[:3], w / w.sum(), rtol=1e-14, atol=0)


def test_softcap_far_above_logits_is_no_cap():
    rng = np.random.default_rng(5)
    q, k, v = _rand(rng, 7, 4, 32), _rand(rng, 19, 2, 32), _rand(rng, 19, 2, 32)
    a = O.attention_f64(q, k, v, scale=32 ** -0.5, causal=True, q_pos0=12)
    b = O.attention_f64(q, k, v, scale=32 ** -0.5, causal=True, q_pos0=12, softcap=1e9)
    np.testing.assert_allclose(b, a, rtol=0, atol=1e-12)


def test_softcap_before_the_mask():
    rng = np.random.default_rng(6)
    sq, lk, d = 5, 23, 16
    q, k, v = _rand(rng, sq, 2, d, s=4.0), _rand(rng, lk, 1, d, s=4.0), _rand(rng, lk, 1, d)
    cap, scale, w = 2.0, 0.25, 6
    # the window rule equals its explicit mask, applied after the cap
    full = O.sliding_window_prefill_mask(sq, lk, w)
    rule = O.attention_f64(q, k, v, scale=scale, causal=True, q_pos0=lk - sq, window_left=w - 1,
                           softcap=cap)
    masked = O.attention_f64(q, k, v, scale=scale, mask=full, softcap=cap)
    np.testing.assert_allclose(masked, rule, rtol=0, atol=1e-13)
    # an additive mask adds to the capped logit: a shift of every logit of a row by the same
    # amount after the cap leaves the softmax unchanged, but not before the cap
    shift = np.full((sq, lk), 7.0, np.float32)
    a = O.attention_f64(q, k, v, scale=scale, softcap=cap)
    b = O.attention_f64(q, k, v, scale=scale, mask=shift, softcap=cap)
    np.testing.assert_allclose(b, a, rtol=0, atol=1e-13)


@pytest.mark.parametrize("cap", [1.0, 50.0])
def test_softcap_numpy_cross_check(cap):
    rng = np.random.default_rng(int(cap))
    q, k, v = _rand(rng, 9, 8, 64, s=3.0), _rand(rng, 30, 2, 64, s=3.0), _rand(rng, 30, 2, 64)
    mask = O.prefill_causal_mask(9, 30)
    got = O.attention_f64(q, k, v, scale=0.125, causal=True, q_pos0=21, softcap=cap)
    want = N.attention(q, k, v, 0.125, mask=mask, softcap=cap)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
