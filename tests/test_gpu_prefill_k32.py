"""GPU parity of prefill_k32_kernel, the kernel contiguous 16-bit prefills with head_dim 128 run
on once their grid holds at least 1,536 workgroups (query blocks of 128 x sequences x query heads;
kK32MinWorkgroups in sketchpad_amd/csrc/prefill.hip). The smaller shapes of test_gpu_prefill.py
and test_gpu_flash.py run on prefill_kernel, so every option is repeated here at a grid above the
threshold: many short sequences with many heads keep the f64 oracle's work small.

The masks are the reference's: causal_mask / prefill_causal_mask / sliding_window_mask
(crates/sketchpad-core/src/transformer.rs:415-451, crates/sketchpad-llm/src/llama.rs:374-388), the
flash-attention test oracle's top-left j > i (crates/sketchpad-cubecl/tests/correctness_cpu.rs:
1066-1074) and flash_attention_masked's additive mask (crates/sketchpad-cubecl/src/attention.rs:
119-128). Outputs within 2e-2 absolute of the f64 oracle (16-bit inputs, fp32 accumulation)."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from tests.helpers import announce
from tests.test_gpu_flash import _check
from tests.test_gpu_prefill import _score_range_inputs, run_varlen

pytestmark = pytest.mark.gpu

K32_MIN_WORKGROUPS = 1536
D = 128


def _lens(seed, n, lo, hi, fixed=()):
    rng = np.random.default_rng(seed)
    return [int(x) for x in fixed] + [int(x) for x in rng.integers(lo, hi + 1, size=n - len(fixed))]


def _assert_k32_grid(lens_q, hq):
    grid = (max(lens_q) + 127) // 128 * len(lens_q) * hq
    assert grid >= K32_MIN_WORKGROUPS, f"grid of {grid} workgroups runs on prefill_kernel"


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("hq,hkv", [(16, 16), (16, 4), (14, 2)])
def test_k32_varlen_causal(dtype, hq, hkv):
    """Self attention with every tile edge: lengths 1, 31-33, 127-129, 300 and random ones."""
    lens = _lens(100 + hq + hkv, 48, 1, 300, fixed=(1, 31, 32, 33, 127, 128, 129, 300))
    _assert_k32_grid(lens, hq)
    run_varlen(lens, lens, hq, hkv, D, dtype, sp.SP_CAUSAL_BOTTOM_RIGHT, -1, seed=hq * 7 + hkv)


@pytest.mark.parametrize("causal", [sp.SP_CAUSAL_NONE, sp.SP_CAUSAL_BOTTOM_RIGHT,
                                    sp.SP_CAUSAL_TOP_LEFT])
def test_k32_varlen_cross_lengths(causal):
    """Lq != Lk (prefill_causal_mask for bottom-right, j > i for top-left, none)."""
    lens_q = _lens(200 + causal, 48, 1, 260, fixed=(1, 3, 129, 260))
    lens_k = _lens(300 + causal, 48, 1, 420, fixed=(300, 1, 130, 77))
    _assert_k32_grid(lens_q, 16)
    run_varlen(lens_q, lens_k, 16, 4, D, "bf16", causal, -1, seed=17 + causal)


@pytest.mark.parametrize("window", [0, 1, 31, 100])
def test_k32_varlen_window(window):
    """Mistral's sliding_window_mask(W): keys [i - W, i]."""
    lens = _lens(400 + window, 48, 1, 300, fixed=(300, 7, 65))
    _assert_k32_grid(lens, 16)
    run_varlen(lens, lens, 16, 4, D, "bf16", sp.SP_CAUSAL_BOTTOM_RIGHT, window, seed=23 + window)


@pytest.mark.parametrize("mode", ["up", "down", "neg", "wide"])
def test_k32_varlen_score_range(mode):
    """The lazily raised maximum over scores far from N(0,1) (see _score_range_inputs)."""
    lens = _lens(500, 48, 1, 300, fixed=(1, 70, 200, 300))
    _assert_k32_grid(lens, 16)
    run_varlen(lens, lens, 16, 4, D, "bf16", sp.SP_CAUSAL_BOTTOM_RIGHT, -1, seed=43,
               inputs=_score_range_inputs(mode, 16, 4, D, seed=43))


def test_k32_varlen_empty_sequences():
    """Sequences without queries, or without keys (their queries get zeros)."""
    lens_q = _lens(600, 48, 0, 260, fixed=(0, 50, 0, 260))
    lens_k = list(lens_q)
    lens_k[5] = 0
    lens_q[5] = 0
    _assert_k32_grid(lens_q, 16)
    run_varlen(lens_q, lens_k, 16, 4, D, "bf16", sp.SP_CAUSAL_BOTTOM_RIGHT, -1, seed=31)


@pytest.mark.parametrize("causal", [False, True])
def test_k32_dense_out_dtypes(causal):
    """flash_attention_ex on [2, 48, 2048, 128] bf16: the f32 output against float64 (every row)
    and the oracle (sampled rows); the bf16 and f16 outputs are that fp32 result rounded once."""
    g = torch.Generator(device="cuda").manual_seed(61 + causal)
    q, k, v = (torch.randn(2, 48, 2048, D, generator=g, device="cuda").bfloat16()
               for _ in range(3))
    assert 2 * 48 * 2048 // 128 >= K32_MIN_WORKGROUPS
    o32 = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    obf = torch.empty_like(q)
    of16 = torch.empty(q.shape, dtype=torch.float16, device="cuda")
    announce(f"k32 dense bf16 -> f32 / bf16 / f16 causal={causal}")
    for o in (o32, obf, of16):
        sp.flash_attention_ex(o, q, k, v, D ** -0.5, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(obf, o32.to(torch.bfloat16))
    assert torch.equal(of16, o32.to(torch.float16))
    _check(obf, q, k, v, "k32 dense bf16", causal=causal, rows=(0, 31, 32, 1000, 2047))


@pytest.mark.parametrize("per_head", [False, True])
def test_k32_masked_16bit(per_head):
    """flash_attention_masked on [2, 48, 2048, 128] f16 with random biases, padded keys at -inf
    and a row half at -1e4."""
    B, H, S = 2, 48, 2048
    g = torch.Generator(device="cuda").manual_seed(73 + per_head)
    q, k, v = (torch.randn(B, H, S, D, generator=g, device="cuda").half() for _ in range(3))
    mask = 2.0 * torch.randn(*((B, H, S, S) if per_head else (S, S)), generator=g, device="cuda")
    mask[..., S - 9:] = float("-inf")
    mask[..., 5, S // 2:] = -1e4
    out = torch.full_like(q, float("nan"))
    announce(f"k32 flash_attention_masked f16 per_head={per_head}")
    sp.flash_attention_masked(out, q, k, v, mask, D ** -0.5)
    torch.cuda.synchronize()
    _check(out, q, k, v, "k32 masked f16", mask=mask, rows=(0, 5, 1000, 2047))
