"""Head dim 512 on the 16-bit paths: Gemma-4's global-attention layers run head_dim = 512 with 16
query / 8 KV heads and the logit soft cap of 50 (crates/sketchpad-llm/src/gemma4.rs:82-107; the
26B-A4B configuration's programmatic init builds every layer that way, :140-160), causal with no
window. Against the f64 oracle within 2e-2 absolute (16-bit inputs, fp32 accumulation):
  - paged decode (sp_paged_decode, *_softcap) at block sizes that are and are not multiples of
    the 16-token tile, windowed and not, GQA groups 1-16, one split and many;
  - the fused append + decode (sp_paged_append_decode), bit for bit against append + decode;
  - varlen prefill (sp_varlen_prefill, *_softcap), causal, with and without a window;
  - chunked prefill against a paged context (sp_paged_prefill) at block sizes 1-64, which take
    every tile-load path of the kernel (a base per block, per group of four rows, per row);
  - a mixed ragged step (sp_ragged_paged_attention) with the cap;
  - dense flash attention (sp_flash_attention_ex), with an f32 output and an additive mask."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import announce, as_f64, assert_attention_close, host_array, oracle_dtype
from tests.test_gpu_append_decode import fused_vs_separate
from tests.test_gpu_decode import check as check_decode
from tests.test_gpu_flash import _check as check_flash
from tests.test_gpu_prefill import run_chunked, run_varlen
from tests.test_gpu_ragged import _run as run_mixed

pytestmark = pytest.mark.gpu

D = 512
HQ, HKV = 16, 8
GEMMA_CAP = 50.0


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("window", [-1, 1023])
@pytest.mark.parametrize("bs", [16, 8, 12, 32])
def test_d512_decode(dtype, window, bs):
    w = W.random_decode(seed=2000 + bs + (window > 0) + len(dtype), num_seqs=8, hq=HQ, hkv=HKV,
                        head_dim=D, block_size=bs, dtype=dtype, min_len=0, max_len=3000,
                        window_left=window)
    check_decode(w)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (16, 4), (16, 2), (16, 1)])
def test_d512_decode_groups(hq, hkv):
    w = W.random_decode(seed=2100 + hq * 3 + hkv, num_seqs=5, hq=hq, hkv=hkv, head_dim=D,
                        block_size=16, dtype="bf16", min_len=1, max_len=1200)
    check_decode(w)


def test_d512_decode_many_splits():
    """Contexts to 9,000 tokens beside 1-token ones: sequences of one split and of many, merged
    by the combine at head dim 512."""
    lens = np.array([1, 9000, 17, 4096, 8191, 300], np.int32)
    rng = np.random.default_rng(2200)
    nblk = int(((lens + 15) // 16).sum()) + 2
    tables = W._tables_from_pool(rng, lens, 16, nblk)
    check_decode(W.DecodeWorkload("d512-many-splits", 2200, len(lens), HQ, HKV, D, 16, "bf16",
                                  lens, tables, nblk))


@pytest.mark.parametrize("cap,qscale", [(GEMMA_CAP, 8.0), (5.0, 2.0)])
@pytest.mark.parametrize("bs", [16, 12])
def test_d512_decode_softcap(cap, qscale, bs):
    w = W.random_decode(seed=2300 + bs + int(cap), num_seqs=8, hq=HQ, hkv=HKV, head_dim=D,
                        block_size=bs, dtype="bf16", min_len=1, max_len=3000)
    t = W.make_decode_tensors(w)
    t["q"].mul_(qscale)
    lay = w.layout()
    announce(f"d512 softcap decode cap={cap} qscale={qscale} BS={bs} maxL={w.max_context_len}")
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, w.max_context_len, -1, lay)
    sp.paged_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                    t["context_lens"], w.max_context_len, D ** -0.5, workspace=ws, softcap=cap)
    torch.cuda.synchronize()
    olay = O.make_layout(w.num_blocks, w.num_layers, w.layer, w.hkv, w.block_size, w.head_dim)
    args = (host_array(t["q"]), host_array(t["k_pool"]), host_array(t["v_pool"]), olay,
            w.block_tables, w.context_lens)
    kw = dict(scale=D ** -0.5, dtype=oracle_dtype(t["q"]))
    ref = O.paged_decode_f64(*args, softcap=cap, **kw)
    assert_attention_close(as_f64(t["out"]), ref, "bf16", w.name)
    plain = O.paged_decode_f64(*args, **kw)
    assert np.abs(ref - plain).max() > 0.1, "the cap does not change these outputs"


@pytest.mark.parametrize("bs,cap", [(16, 0.0), (8, GEMMA_CAP), (12, 0.0), (24, GEMMA_CAP)])
def test_d512_append_decode(bs, cap):
    fused_vs_separate(W.random_decode(seed=2400 + bs, num_seqs=6, hq=HQ, hkv=HKV, head_dim=D,
                                      block_size=bs, dtype="bf16", min_len=1, max_len=2500),
                      softcap=cap, qscale=8.0 if cap else 1.0)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("window", [-1, 100, 1023])
def test_d512_varlen_prefill(dtype, window):
    lens = [1, 15, 16, 17, 127, 128, 129, 300, 700]
    run_varlen(lens, lens, HQ, HKV, D, dtype, sp.SP_CAUSAL_BOTTOM_RIGHT, window,
               seed=2500 + max(window, 0) % 97 + len(dtype))


@pytest.mark.parametrize("causal", [sp.SP_CAUSAL_NONE, sp.SP_CAUSAL_TOP_LEFT])
def test_d512_varlen_prefill_modes(causal):
    """Query and key lengths that differ (a chunk over a longer context), non-causal and
    top-left causal."""
    run_varlen([1, 64, 200, 129], [40, 64, 500, 1000], HQ, HKV, D, "bf16", causal, -1,
               seed=2550 + causal)


@pytest.mark.parametrize("cap,qscale", [(GEMMA_CAP, 8.0), (5.0, 2.0)])
def test_d512_varlen_prefill_softcap(cap, qscale):
    lens = [1, 33, 129, 700, 1200]
    run_varlen(lens, lens, HQ, HKV, D, "bf16", sp.SP_CAUSAL_BOTTOM_RIGHT, -1,
               seed=2600 + int(cap), softcap=cap, qscale=qscale)


@pytest.mark.parametrize("bs", [1, 2, 4, 8, 12, 16, 32, 64])
def test_d512_chunked_prefill(bs):
    w = W.ChunkedPrefillWorkload("d512-chunked", 2700 + bs, np.array([1, 70, 300, 129], np.int32),
                                 np.array([0, 900, 1500, 40], np.int32), HQ, HKV, D, "bf16",
                                 block_size=bs)
    run_chunked(w)


@pytest.mark.parametrize("window,cap", [(1023, 0.0), (-1, GEMMA_CAP)])
def test_d512_chunked_prefill_options(window, cap):
    w = W.ChunkedPrefillWorkload("d512-chunked-opts", 2750 + window % 7,
                                 np.array([200, 17, 256], np.int32),
                                 np.array([1800, 3, 700], np.int32), HQ, HKV, D, "bf16",
                                 block_size=16, window_left=window)
    run_chunked(w, softcap=cap, qscale=8.0 if cap else 1.0)


def test_d512_mixed_step():
    w = W.MixedWorkload("d512-mixed", 2800, np.array([200, 64], np.int32),
                        np.array([1500, 0], np.int32), np.array([2100, 17, 900], np.int32),
                        HQ, HKV, D, "bf16")
    run_mixed(w, repeats=2, softcap=GEMMA_CAP, qscale=8.0)


@pytest.mark.parametrize("causal", [False, True])
def test_d512_flash_f32_out(causal):
    """flash_attention_ex on bf16 [2, 16, 300, 512] with an f32 output; the bf16 output is that
    fp32 result rounded once."""
    g = torch.Generator(device="cuda").manual_seed(2850 + causal)
    q, k, v = (torch.randn(2, HQ, 300, D, generator=g, device="cuda").bfloat16()
               for _ in range(3))
    o32 = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    o16 = torch.empty_like(q)
    announce(f"d512 flash bf16 -> f32 causal={causal}")
    sp.flash_attention_ex(o32, q, k, v, D ** -0.5, causal=causal)
    sp.flash_attention_ex(o16, q, k, v, D ** -0.5, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(o16, o32.to(torch.bfloat16))
    check_flash(o16, q, k, v, "d512 flash", causal=causal, rows=(0, 15, 16, 17, 299))


def test_d512_flash_masked():
    """An additive [Sq, Sk] mask broadcast over batch and heads (flash_attention_masked)."""
    g = torch.Generator(device="cuda").manual_seed(2870)
    q = torch.randn(1, HQ, 200, D, generator=g, device="cuda").bfloat16()
    k, v = (torch.randn(1, HQ, 333, D, generator=g, device="cuda").bfloat16() for _ in range(2))
    mask = torch.randn(200, 333, generator=g, device="cuda") * 3.0
    mask[:, 100:150] = float("-inf")
    out = torch.empty_like(q)
    announce("d512 flash bf16 masked [1, 16, 200 x 333, 512]")
    sp.flash_attention_ex(out, q, k, v, D ** -0.5, mask=mask)
    torch.cuda.synchronize()
    check_flash(out, q, k, v, "d512 flash masked", mask=mask, rows=(0, 1, 77, 199))
