"""Head dim 256 on the 16-bit paths: Gemma-4's sliding-window layers run head_dim_swa = 256 with
a window of W keys [p - W + 1, p] (crates/sketchpad-llm/src/gemma4.rs:94-102, the mask at
:1086-1108), i.e. window_left = W - 1; griffin uses 256 as well (griffin.rs:63). At the Gemma-4
shape (16 query / 8 KV heads, W = 1024), against the f64 oracle within 2e-2 absolute:
  - paged decode (sp_paged_decode) and the fused append + decode (sp_paged_append_decode);
  - varlen prefill (sp_varlen_prefill), causal with and without the window;
  - chunked prefill against a paged context (sp_paged_prefill), with the window;
  - a mixed ragged step (sp_ragged_paged_attention);
  - dense flash attention (sp_flash_attention_ex) with an f32 output."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from sketchpad_amd import workloads as W
from tests.helpers import announce
from tests.test_gpu_append_decode import fused_vs_separate
from tests.test_gpu_decode import check as check_decode
from tests.test_gpu_flash import _check as check_flash
from tests.test_gpu_prefill import run_chunked, run_varlen
from tests.test_gpu_ragged import _run as run_mixed

pytestmark = pytest.mark.gpu

D = 256
HQ, HKV = 16, 8
GEMMA_WINDOW = 1024  # W keys: window_left = W - 1


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("window", [-1, GEMMA_WINDOW - 1])
def test_d256_decode(dtype, window):
    w = W.random_decode(seed=900 + (window > 0) + len(dtype), num_seqs=8, hq=HQ, hkv=HKV,
                        head_dim=D, block_size=16, dtype=dtype, min_len=1, max_len=3000,
                        window_left=window)
    check_decode(w)


@pytest.mark.parametrize("bs", [8, 12, 16])
def test_d256_append_decode(bs):
    fused_vs_separate(W.random_decode(seed=910 + bs, num_seqs=6, hq=HQ, hkv=HKV, head_dim=D,
                                      block_size=bs, dtype="bf16", min_len=1, max_len=2500,
                                      window_left=GEMMA_WINDOW - 1))


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("window", [-1, 100, GEMMA_WINDOW - 1])
def test_d256_varlen_prefill(dtype, window):
    lens = [1, 31, 32, 33, 127, 128, 129, 700, 1500]
    run_varlen(lens, lens, HQ, HKV, D, dtype, sp.SP_CAUSAL_BOTTOM_RIGHT, window,
               seed=920 + max(window, 0) % 97 + len(dtype))


@pytest.mark.parametrize("window", [-1, GEMMA_WINDOW - 1])
@pytest.mark.parametrize("bs", [8, 16, 24, 32])
def test_d256_chunked_prefill(window, bs):
    w = W.ChunkedPrefillWorkload("d256-chunked", 930 + bs, np.array([1, 70, 300, 129], np.int32),
                                 np.array([0, 900, 2000, 40], np.int32), HQ, HKV, D, "bf16",
                                 block_size=bs, window_left=window)
    run_chunked(w)


def test_d256_mixed_step():
    w = W.MixedWorkload("d256-mixed", 940, np.array([200, 64], np.int32),
                        np.array([1500, 0], np.int32), np.array([2100, 17, 900], np.int32),
                        HQ, HKV, D, "bf16")
    run_mixed(w, window_left=GEMMA_WINDOW - 1, repeats=2)


@pytest.mark.parametrize("causal", [False, True])
def test_d256_flash_f32_out(causal):
    """flash_attention_ex on bf16 [2, 16, 600, 256] with an f32 output; the bf16 output is that
    fp32 result rounded once."""
    g = torch.Generator(device="cuda").manual_seed(950 + causal)
    q, k, v = (torch.randn(2, HQ, 600, D, generator=g, device="cuda").bfloat16()
               for _ in range(3))
    o32 = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    o16 = torch.empty_like(q)
    announce(f"d256 flash bf16 -> f32 causal={causal}")
    sp.flash_attention_ex(o32, q, k, v, D ** -0.5, causal=causal)
    sp.flash_attention_ex(o16, q, k, v, D ** -0.5, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(o16, o32.to(torch.bfloat16))
    check_flash(o16, q, k, v, "d256 flash", causal=causal, rows=(0, 31, 32, 599))
