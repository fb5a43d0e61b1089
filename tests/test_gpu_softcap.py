"""Gemma-4's logit soft cap through the *_softcap entry points: logits = cap * tanh(logits / cap)
on the scaled product, before the mask (crates/sketchpad-llm/src/gemma4.rs:366-377;
attn_logit_softcap = 50 at :96), at the shape of its sliding-window layers (head_dim 256, 16
query / 8 KV heads, a window of W = 1024 keys, window_left = W - 1; gemma4.rs:94-102,
:1086-1108). Against the f64 oracle's capped attention (spo_attention_f64_cap, pinned in
test_oracle_softcap.py) within 2e-2 absolute (16-bit inputs, fp32 accumulation).

q is scaled so that the logits reach the cap: x8 for the Gemma cap of 50 (logits of standard
deviation ~8) and x2 for a cap of 5. The decode tests also check that the capped and the
uncapped oracle outputs differ by far more than the tolerance at these inputs, so a kernel that
skipped the cap could not pass."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import announce, as_f64, assert_attention_close, host_array, oracle_dtype
from tests.test_gpu_append_decode import fused_vs_separate
from tests.test_gpu_prefill import run_chunked, run_varlen
from tests.test_gpu_ragged import _run as run_mixed

pytestmark = pytest.mark.gpu

D, HQ, HKV = 256, 16, 8
WINDOW_LEFT = 1023  # Gemma-4's W = 1024 keys
CAPS = [(50.0, 8.0), (5.0, 2.0)]  # (logit_softcap, q scale)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("cap,qscale", CAPS)
@pytest.mark.parametrize("bs", [16, 8])
def test_softcap_decode(dtype, cap, qscale, bs):
    w = W.random_decode(seed=1500 + bs + int(cap) + len(dtype), num_seqs=8, hq=HQ, hkv=HKV,
                        head_dim=D, block_size=bs, dtype=dtype, min_len=1, max_len=3000,
                        window_left=WINDOW_LEFT)
    t = W.make_decode_tensors(w)
    t["q"].mul_(qscale)
    lay = w.layout()
    announce(f"softcap decode cap={cap} qscale={qscale} BS={bs} {dtype} maxL={w.max_context_len}")
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])
    ws = sp.alloc_decode_workspace(w.num_seqs, w.hq, w.max_context_len, w.window_left, lay)
    sp.paged_decode(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                    t["context_lens"], w.max_context_len, D ** -0.5, window_left=w.window_left,
                    workspace=ws, softcap=cap)
    torch.cuda.synchronize()
    olay = O.make_layout(w.num_blocks, w.num_layers, w.layer, w.hkv, w.block_size, w.head_dim)
    args = (host_array(t["q"]), host_array(t["k_pool"]), host_array(t["v_pool"]), olay,
            w.block_tables, w.context_lens)
    kw = dict(scale=D ** -0.5, window_left=w.window_left, dtype=oracle_dtype(t["q"]))
    ref = O.paged_decode_f64(*args, softcap=cap, **kw)
    assert_attention_close(as_f64(t["out"]), ref, dtype, w.name)
    plain = O.paged_decode_f64(*args, **kw)
    assert np.abs(ref - plain).max() > 0.1, "the cap does not change these outputs"


@pytest.mark.parametrize("cap,qscale", CAPS)
@pytest.mark.parametrize("bs", [16, 8])
def test_softcap_append_decode(cap, qscale, bs):
    """sp_paged_append_decode_softcap = sp_kv_append + sp_paged_decode_softcap, bit for bit."""
    fused_vs_separate(W.random_decode(seed=1600 + bs + int(cap), num_seqs=6, hq=HQ, hkv=HKV,
                                      head_dim=D, block_size=bs, dtype="bf16", min_len=1,
                                      max_len=2500, window_left=WINDOW_LEFT),
                      softcap=cap, qscale=qscale)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("cap,qscale", CAPS)
@pytest.mark.parametrize("window", [-1, WINDOW_LEFT])
def test_softcap_varlen_prefill(dtype, cap, qscale, window):
    lens = [1, 31, 33, 129, 700, 1500]
    run_varlen(lens, lens, HQ, HKV, D, dtype, sp.SP_CAUSAL_BOTTOM_RIGHT, window,
               seed=1700 + int(cap) + max(window, 0) % 13 + len(dtype), softcap=cap,
               qscale=qscale)


@pytest.mark.parametrize("cap,qscale", CAPS)
@pytest.mark.parametrize("bs", [8, 16])
def test_softcap_chunked_prefill(cap, qscale, bs):
    w = W.ChunkedPrefillWorkload("softcap-chunked", 1800 + bs + int(cap),
                                 np.array([1, 70, 300, 129], np.int32),
                                 np.array([0, 900, 2000, 40], np.int32), HQ, HKV, D, "bf16",
                                 block_size=bs, window_left=WINDOW_LEFT)
    run_chunked(w, softcap=cap, qscale=qscale)


@pytest.mark.parametrize("cap,qscale", CAPS)
def test_softcap_mixed_step(cap, qscale):
    """Both halves of a mixed batch (chunks beside decode on the side stream) take the cap; the
    rows equal the two entry points' on their own, bit for bit, and the oracle's."""
    w = W.MixedWorkload("softcap-mixed", 1900 + int(cap), np.array([200, 64], np.int32),
                        np.array([1500, 0], np.int32), np.array([2100, 17, 900], np.int32),
                        HQ, HKV, D, "bf16")
    run_mixed(w, window_left=WINDOW_LEFT, repeats=2, softcap=cap, qscale=qscale)
