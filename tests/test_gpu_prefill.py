"""GPU parity of the prefill paths against the f64 oracle (attention per sequence with the
reference's masks: causal_mask / prefill_causal_mask / sliding_window_mask, transformer.rs:415-451,
llama.rs:374-388) and, at the full C3 / C4 sizes, against a float32 torch reference on the GPU plus
oracle rows sampled from every sequence."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import announce, assert_attention_close, host_array, oracle_dtype

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _rand(g, *shape, dt):
    return torch.randn(*shape, generator=g, device="cuda", dtype=torch.float32).to(dt)


def _oracle_varlen(q, k, v, cu_q, cu_k, scale, causal_mode, window, softcap=0.0):
    """Per-sequence f64 oracle over packed q [Tq, Hq, D], k/v [Tk, Hkv, D] (host arrays)."""
    out = np.zeros(q.shape, dtype=np.float64)
    dt = O.BF16 if q.dtype == np.uint16 else O.F32
    for s in range(len(cu_q) - 1):
        qa, qb, ka, kb = cu_q[s], cu_q[s + 1], cu_k[s], cu_k[s + 1]
        lq, lk = qb - qa, kb - ka
        if lq == 0:
            continue
        causal = causal_mode != sp.SP_CAUSAL_NONE
        pos0 = 0 if causal_mode == sp.SP_CAUSAL_TOP_LEFT else lk - lq
        out[qa:qb] = O.attention_f64(q[qa:qb], k[ka:kb], v[ka:kb], scale=scale, causal=causal,
                                     q_pos0=pos0, window_left=window, dtype=dt, softcap=softcap)
    return out


def _as_f64(t):
    return t.float().cpu().numpy().astype(np.float64)


def run_varlen(lens_q, lens_k, hq, hkv, d, dtype, causal, window, seed, inputs=None,
               f32_bar="abs", softcap=0.0, qscale=1.0):
    """f32_bar: "abs" checks f32 outputs at 1e-5 per row against the f64 oracle; "refops" (for
    inputs whose scores are so large that fp32 rounding of the scores alone exceeds that) bounds
    the worst and mean row error by twice those of the reference's own f32 op order.
    softcap: the logit soft cap (sp_varlen_prefill_softcap); qscale multiplies q (in its dtype)
    so that the logits reach the cap. Returns the oracle's output."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    dt = DT[dtype]
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lens_k)]).astype(np.int32)
    if inputs is None:
        q = _rand(g, int(cu_q[-1]), hq, d, dt=dt)
        k = _rand(g, int(cu_k[-1]), hkv, d, dt=dt)
        v = _rand(g, int(cu_k[-1]), hkv, d, dt=dt)
    else:
        q, k, v = (x.to(device="cuda", dtype=dt) for x in inputs(cu_q, cu_k))
    if qscale != 1.0:
        q.mul_(qscale)
    out = torch.full_like(q, float("nan"))
    announce(f"varlen prefill lens_q={list(lens_q)} lens_k={list(lens_k)} hq={hq} hkv={hkv} "
             f"d={d} {dtype} causal={causal} window={window} softcap={softcap}")
    sp.varlen_prefill(out, q, k, v, torch.from_numpy(cu_q).cuda(), torch.from_numpy(cu_k).cuda(),
                      int(max(lens_q)), d ** -0.5, causal=causal, window_left=window,
                      softcap=softcap)
    torch.cuda.synchronize()
    # the oracle reads 16-bit tensors as bf16 bits; f16 inputs are handed over as float32
    to_host = host_array if dtype == "bf16" else (lambda t: t.float().cpu().numpy())
    ref = _oracle_varlen(to_host(q), to_host(k), to_host(v), cu_q, cu_k, d ** -0.5, causal, window,
                         softcap)
    if dtype == "f32" and f32_bar == "refops":
        got = _as_f64(out)
        r32 = np.zeros_like(ref)
        qh, kh, vh = to_host(q), to_host(k), to_host(v)
        for s_ in range(len(cu_q) - 1):
            qa, qb, ka, kb = cu_q[s_], cu_q[s_ + 1], cu_k[s_], cu_k[s_ + 1]
            if qb == qa:
                continue
            pos0 = 0 if causal == sp.SP_CAUSAL_TOP_LEFT else (kb - ka) - (qb - qa)
            r32[qa:qb] = O.attention_f32_refops(qh[qa:qb], kh[ka:kb], vh[ka:kb], scale=d ** -0.5,
                                                causal=causal != sp.SP_CAUSAL_NONE, q_pos0=pos0,
                                                window_left=window)
        row = np.maximum(np.abs(ref).max(axis=-1, keepdims=True), 1e-30)
        ours = (np.abs(got - ref) / row).max(axis=-1)
        theirs = (np.abs(r32 - ref) / row).max(axis=-1)
        # per-row errors of two fp32 computations scatter independently, so the distributions
        # are compared: the worst and the mean row within twice the reference op order's
        assert ours.max() <= max(1e-5, 2 * theirs.max()), (
            f"f32 worst row {ours.max():.3e} vs reference op order {theirs.max():.3e}")
        assert ours.mean() <= max(1e-5, 2 * theirs.mean()), (
            f"f32 mean row {ours.mean():.3e} vs reference op order {theirs.mean():.3e}")
        return
    assert_attention_close(_as_f64(out), ref, dtype, "varlen prefill")
    return ref


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (7, 1)])
def test_varlen_causal_self(dtype, d, hq, hkv):
    lens = [1, 5, 16, 17, 64, 65, 127, 128, 129, 200, 300]
    run_varlen(lens, lens, hq, hkv, d, dtype, sp.SP_CAUSAL_BOTTOM_RIGHT, -1, seed=hq * 10 + d)


def test_varlen_llama_heads():
    lens = [256, 33, 513, 130]
    run_varlen(lens, lens, 32, 8, 128, "bf16", sp.SP_CAUSAL_BOTTOM_RIGHT, -1, seed=3)


@pytest.mark.parametrize("causal", [sp.SP_CAUSAL_NONE, sp.SP_CAUSAL_BOTTOM_RIGHT,
                                    sp.SP_CAUSAL_TOP_LEFT])
def test_varlen_cross_lengths(causal):
    """Lq != Lk: the bottom-right mask is prefill_causal_mask (queries are the last positions)."""
    lens_q = [3, 40, 130, 64, 1]
    lens_k = [10, 200, 130, 300, 77]
    run_varlen(lens_q, lens_k, 8, 4, 128, "bf16", causal, -1, seed=11 + causal)


@pytest.mark.parametrize("window", [0, 1, 31, 64, 100])
def test_varlen_sliding_window(window):
    """Mistral's sliding_window_mask(W): keys [i - W, i] (window_left = W)."""
    lens = [7, 150, 300, 65]
    run_varlen(lens, lens, 8, 2, 128, "bf16", sp.SP_CAUSAL_BOTTOM_RIGHT, window, seed=21 + window)


def _score_range_inputs(mode, hq, hkv, d, seed):
    """q/k/v whose scores sit far from the N(0,1) range: 'up' rises along every sequence's keys
    (x = score * scale * log2 e climbs to ~390, so the running maximum is raised tile after tile),
    'down' falls (the maximum is in the first tile, later weights underflow to zero), 'neg' sits
    near x = -390 for every key (weights would underflow without a maximum taken from the data),
    'wide' draws q and k from N(0, 4^2) (|x| up to ~100: peaked softmax, large exponents)."""
    def make(cu_q, cu_k):
        g = torch.Generator().manual_seed(seed)
        tq, tk = int(cu_q[-1]), int(cu_k[-1])
        v = torch.randn(tk, hkv, d, generator=g)
        if mode == "wide":
            return (4 * torch.randn(tq, hq, d, generator=g), 4 * torch.randn(tk, hkv, d, generator=g),
                    v)
        q = 2.0 + 0.5 * torch.randn(tq, hq, d, generator=g)
        level = torch.zeros(tk)
        for s in range(len(cu_k) - 1):
            a, b = int(cu_k[s]), int(cu_k[s + 1])
            ramp = torch.arange(b - a, dtype=torch.float32) / max(b - a, 1)
            level[a:b] = {"up": 12.0 * ramp, "down": 12.0 * (1 - ramp),
                          "neg": torch.full_like(ramp, -12.0)}[mode]
        k = level[:, None, None] + 0.5 * torch.randn(tk, hkv, d, generator=g)
        return q, k, v
    return make


@pytest.mark.parametrize("mode", ["up", "down", "neg", "wide"])
def test_varlen_score_range(mode):
    """The online softmax's maximum handling over score ranges far from N(0,1) inputs."""
    lens = [1, 70, 200, 333]
    run_varlen(lens, lens, 8, 2, 128, "bf16", sp.SP_CAUSAL_BOTTOM_RIGHT, -1, seed=41,
               inputs=_score_range_inputs(mode, 8, 2, 128, seed=41))


def test_varlen_score_range_window():
    """Rising scores under a sliding window: each query's maximum leaves the window."""
    lens = [150, 300]
    run_varlen(lens, lens, 4, 4, 64, "bf16", sp.SP_CAUSAL_BOTTOM_RIGHT, 40, seed=43,
               inputs=_score_range_inputs("up", 4, 4, 64, seed=43))


def test_varlen_empty_sequences():
    lens = [0, 50, 0, 3]
    run_varlen(lens, lens, 4, 2, 64, "bf16", sp.SP_CAUSAL_BOTTOM_RIGHT, -1, seed=31)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2)])
def test_varlen_f32(d, hq, hkv):
    """fp32 prefill (fp32 MFMA, fp32 P): within 1e-5 of the f64 oracle per output row."""
    lens = [1, 17, 31, 32, 33, 64, 127, 129, 300]
    run_varlen(lens, lens, hq, hkv, d, "f32", sp.SP_CAUSAL_BOTTOM_RIGHT, -1, seed=51 + d + hq)


@pytest.mark.parametrize("causal", [sp.SP_CAUSAL_NONE, sp.SP_CAUSAL_TOP_LEFT])
def test_varlen_f32_cross_lengths_and_window(causal):
    lens_q = [3, 40, 130, 1]
    lens_k = [10, 200, 130, 77]
    run_varlen(lens_q, lens_k, 8, 4, 64, "f32", causal, -1, seed=61 + causal)
    run_varlen([150, 300], [150, 300], 4, 2, 128, "f32", sp.SP_CAUSAL_BOTTOM_RIGHT, 40,
               seed=63)


@pytest.mark.parametrize("mode", ["neg", "wide"])
def test_varlen_f32_score_range(mode):
    lens = [1, 70, 200]
    run_varlen(lens, lens, 4, 2, 128, "f32", sp.SP_CAUSAL_BOTTOM_RIGHT, -1, seed=65,
               inputs=_score_range_inputs(mode, 4, 2, 128, seed=65), f32_bar="refops")


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk,d", [(77, 77, 64), (256, 256, 128), (40, 300, 64)])
def test_flash_attention_f32(causal, sq, sk, d):
    """flash_attention in f32, the element type the reference's flash_attention runs
    (sketchpad-cubecl attention.rs:21-25): [B, H, S, D], top-left causal, 1e-5 relative."""
    B, H = 2, 3
    g = torch.Generator(device="cuda").manual_seed(sq * 3 + sk + causal)
    q = _rand(g, B, H, sq, d, dt=torch.float32)
    k = _rand(g, B, H, sk, d, dt=torch.float32)
    v = _rand(g, B, H, sk, d, dt=torch.float32)
    out = torch.full_like(q, float("nan"))
    announce(f"flash_attention f32 sq={sq} sk={sk} d={d} causal={causal}")
    sp.flash_attention(out, q, k, v, d ** -0.5, causal=causal)
    torch.cuda.synchronize()
    qh, kh, vh = (x.cpu().numpy() for x in (q, k, v))
    ref = np.zeros((B, H, sq, d))
    for bi in range(B):
        r = O.attention_f64(qh[bi].transpose(1, 0, 2), kh[bi].transpose(1, 0, 2),
                            vh[bi].transpose(1, 0, 2), scale=d ** -0.5, causal=causal, q_pos0=0,
                            dtype=O.F32)
        ref[bi] = r.transpose(1, 0, 2)
    assert_attention_close(_as_f64(out), ref, "f32", "flash_attention f32")


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("per_head", [False, True])
def test_flash_attention_masked_f32(causal, per_head):
    """flash_attention_masked (sketchpad-cubecl attention.rs:119-128): additive f32 mask, either
    one [Sq, Sk] mask for every batch and head (as the reference's tests expand it) or a full
    [B, H, Sq, Sk] one; random biases, padded keys at -inf, 1e-5 per row vs the f64 oracle."""
    B, H, sq, sk, d = 2, 3, 90, 150, 64
    g = torch.Generator(device="cuda").manual_seed(71 + causal + 2 * per_head)
    q, k, v = (_rand(g, B, H, n, d, dt=torch.float32) for n in (sq, sk, sk))
    mshape = (B, H, sq, sk) if per_head else (sq, sk)
    mask = 2.0 * torch.randn(*mshape, generator=g, device="cuda")
    mask[..., sk - 7:] = float("-inf")   # padded keys
    # large finite negatives on half of a row, beside keys that stay visible (were they a row's
    # only keys, fp32 could not hold score differences next to -1e4, nor could the reference's)
    mask[..., 5, sk // 2:] = -1e4
    out = torch.full_like(q, float("nan"))
    announce(f"flash_attention_masked f32 per_head={per_head} causal={causal}")
    sp.flash_attention_masked(out, q, k, v, mask, d ** -0.5, causal=causal)
    torch.cuda.synchronize()
    qh, kh, vh = (x.cpu().numpy() for x in (q, k, v))
    mh = mask.expand(B, H, sq, sk).cpu().numpy()
    if causal:  # the oracle takes an explicit mask instead of its causal predicate: fold it in
        i, j = np.arange(sq)[:, None], np.arange(sk)[None, :]
        mh = mh + np.where(j > i, -np.inf, 0.0).astype(np.float32)
    ref = np.zeros((B, H, sq, d))
    for bi in range(B):
        for hi in range(H):
            ref[bi, hi] = O.attention_f64(qh[bi, hi][:, None], kh[bi, hi][:, None],
                                          vh[bi, hi][:, None], scale=d ** -0.5, mask=mh[bi, hi],
                                          q_pos0=0, dtype=O.F32)[:, 0]
    assert_attention_close(_as_f64(out), ref, "f32", "flash_attention_masked")


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk", [(16, 16), (64, 64), (130, 70), (33, 200)])
def test_flash_attention_dense(causal, sq, sk):
    """flash_attention on [B, H, S, D]; causal is the reference test oracle's j > i mask."""
    B, H, D = 2, 4, 64
    g = torch.Generator(device="cuda").manual_seed(sq + sk + causal)
    q = _rand(g, B, H, sq, D, dt=torch.bfloat16)
    k = _rand(g, B, H, sk, D, dt=torch.bfloat16)
    v = _rand(g, B, H, sk, D, dt=torch.bfloat16)
    out = torch.empty_like(q)
    announce(f"flash_attention dense sq={sq} sk={sk} causal={causal}")
    sp.flash_attention(out, q, k, v, D ** -0.5, causal=causal)
    torch.cuda.synchronize()
    qh, kh, vh = host_array(q), host_array(k), host_array(v)
    ref = np.zeros((B, H, sq, D))
    for bi in range(B):
        r = O.attention_f64(qh[bi].transpose(1, 0, 2), kh[bi].transpose(1, 0, 2),
                            vh[bi].transpose(1, 0, 2), scale=D ** -0.5, causal=causal, q_pos0=0,
                            dtype=O.BF16)
        ref[bi] = r.transpose(1, 0, 2)
    assert_attention_close(_as_f64(out), ref, "bf16", "flash_attention")


def run_chunked(w: W.ChunkedPrefillWorkload, sample_rows=None, split=False, shift=None,
                softcap=0.0, qscale=1.0):
    """split: hand sp_paged_prefill the workspace it asks for, so long contexts are split over
    several workgroups per query block (the test asserts that a split is planned).
    shift: (q_mean, k_mean) moves q and every cached / new key off N(0,1) (q = q_mean + x/2,
    k = k_mean + x/2), so the scores sit far from zero.
    softcap: the logit soft cap (sp_paged_prefill_softcap); qscale multiplies q."""
    t = W.make_chunked_tensors(w)
    if qscale != 1.0:
        t["q"].mul_(qscale)
    if shift is not None:
        qm, km = shift
        for name, m in (("q", qm), ("k_pool", km), ("k_new", km)):
            t[name].copy_((m + 0.5 * t[name].float()).to(t[name].dtype))
    lay = sp.layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
    ws = None
    if split:
        ws = sp.alloc_paged_prefill_workspace(w.num_seqs, w.max_seqlen_q, w.hq, lay,
                                              t["block_tables"].shape[1])
        assert ws is not None, "no key split planned for this shape"
    announce(f"chunked prefill {w.name} chunks={list(w.chunk_lens)} ctx={list(w.ctx_before)} "
             f"workspace={0 if ws is None else ws.numel()} softcap={softcap}")
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])
    sp.paged_prefill(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                     t["cu_seqlens_q"], t["context_lens"], w.max_seqlen_q, w.head_dim ** -0.5,
                     window_left=w.window_left, workspace=ws, softcap=softcap)
    torch.cuda.synchronize()
    olay = O.make_layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
    kp, vp, q = host_array(t["k_pool"]), host_array(t["v_pool"]), host_array(t["q"])
    got = _as_f64(t["out"])
    cu = w.cu_seqlens_q
    rng = np.random.default_rng(0)
    for s in range(w.num_seqs):
        L = int(w.context_lens[s])
        kg, vg = O.gather_kv(kp, vp, olay, w.block_tables_np[s] if hasattr(w, "block_tables_np")
                             else t["block_tables"][s].cpu().numpy(), L)
        kt = np.ascontiguousarray(kg.transpose(1, 0, 2))
        vt = np.ascontiguousarray(vg.transpose(1, 0, 2))
        lq = int(w.chunk_lens[s])
        rows = np.arange(lq) if sample_rows is None else np.unique(
            np.concatenate([[0, lq - 1], rng.choice(lq, size=min(lq, sample_rows), replace=False)]))
        # the chunk's queries sit at positions L - lq .. L - 1 (prefill_causal_mask)
        ref = O.attention_f64(q[cu[s]:cu[s] + lq], kt[:L], vt[:L], scale=w.head_dim ** -0.5,
                              causal=True, q_pos0=L - lq, window_left=w.window_left,
                              dtype=oracle_dtype(t["q"]), softcap=softcap)
        assert_attention_close(got[cu[s] + rows], ref[rows], w.dtype, f"{w.name} seq {s}")
    return t


def test_paged_prefill_small():
    w = W.ChunkedPrefillWorkload("chunked-small", 41, np.array([1, 17, 130, 64], np.int32),
                                 np.array([0, 40, 300, 5], np.int32), 8, 2, 128, "bf16")
    run_chunked(w)


def test_paged_prefill_window():
    w = W.ChunkedPrefillWorkload("chunked-window", 42, np.array([50, 129], np.int32),
                                 np.array([200, 90], np.int32), 8, 2, 64, "bf16", window_left=70)
    run_chunked(w)


@pytest.mark.parametrize("window", [-1, 50])
def test_paged_prefill_f32(window):
    """Chunked prefill on an f32 paged cache (the reference cache's default element type)."""
    w = W.ChunkedPrefillWorkload("chunked-f32", 53, np.array([1, 40, 130], np.int32),
                                 np.array([0, 300, 77], np.int32), 8, 2, 64, "f32",
                                 window_left=window)
    run_chunked(w)


def test_paged_prefill_block_size_32():
    w = W.ChunkedPrefillWorkload("chunked-bs32", 43, np.array([65, 100], np.int32),
                                 np.array([77, 31], np.int32), 4, 4, 128, "bf16", block_size=32)
    run_chunked(w)


@pytest.mark.parametrize("d,bs", [(128, 4), (128, 8), (128, 64), (64, 4), (64, 8), (64, 64),
                                  (128, 12), (128, 24), (64, 3), (64, 48)])
def test_paged_prefill_block_sizes(d, bs):
    """Block sizes on every tile-load path: blocks holding whole groups of four 1 KiB loads (one
    base per group), smaller blocks (one base per load), blocks smaller than one load and block
    sizes that do not divide the tile (per-lane addresses)."""
    w = W.ChunkedPrefillWorkload(f"chunked-d{d}-bs{bs}", 44 + bs + d, np.array([130, 61], np.int32),
                                 np.array([200, 7], np.int32), 8, 2, d, "bf16", block_size=bs)
    run_chunked(w)


@pytest.mark.parametrize("window", [-1, 1000])
def test_paged_prefill_split_keys(window):
    """Few query blocks over long contexts: the keys are split over workgroups (4 splits here)
    and the fp32 partials merged; every row checked against the f64 oracle."""
    w = W.ChunkedPrefillWorkload("chunked-split", 47, np.array([64, 200, 1], np.int32),
                                 np.array([3000, 2100, 5000], np.int32), 8, 2, 128, "bf16",
                                 window_left=window)
    run_chunked(w, split=True)


@pytest.mark.parametrize("shift", [None, (2.0, -12.0)])
def test_paged_prefill_split_with_empty_splits(shift):
    """A key split planned from the table width (one long context) over a batch that also holds
    a short context (48 keys) and a fresh 128-query chunk: their later splits see no key. With
    (2, -12) every score sits near x = q.k * scale * log2(e) = -390, so a split that saw no key
    must not lend its offset to the merge. Every row against the f64 oracle."""
    w = W.ChunkedPrefillWorkload("chunked-split-empty", 48, np.array([64, 32, 128], np.int32),
                                 np.array([3000, 16, 0], np.int32), 8, 2, 128, "bf16")
    run_chunked(w, split=True, shift=shift)


def test_chunked_prefill_c4_all_rows():
    """C4's four 512-token chunks on 2k-6.3k-token contexts: every row against the f64 oracle.
    (Its 448 workgroups fill most of one round of resident slots, so no key split is planned.)"""
    run_chunked(W.chunked_prefill_c4())


def test_chunked_prefill_long_context_split_all_rows():
    """One 512-token chunk of Qwen2.5-7B heads (28 / 4) on a 32k-token context: 112 workgroups,
    so the keys are split 4 ways and merged; every row against the f64 oracle."""
    w = W.ChunkedPrefillWorkload("chunked-32k", 49, np.array([512], np.int32),
                                 np.array([32256], np.int32), 28, 4, 128, "bf16")
    run_chunked(w, split=True)


def _torch_ref_causal(q, k, v, cu, scale):
    """float32 torch reference for causal self-attention over packed sequences (GPU)."""
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    hq, hkv = q.shape[1], k.shape[1]
    for s in range(len(cu) - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        qf = q[a:b].float().permute(1, 0, 2).contiguous()                       # [Hq, L, D]
        kf = k[a:b].float().permute(1, 0, 2).repeat_interleave(hq // hkv, 0)   # [Hq, L, D]
        vf = v[a:b].float().permute(1, 0, 2).repeat_interleave(hq // hkv, 0)
        sc = torch.matmul(qf, kf.transpose(1, 2).contiguous()) * scale
        L = b - a
        mask = torch.ones(L, L, dtype=torch.bool, device=q.device).triu(1)
        sc.masked_fill_(mask, float("-inf"))
        out[a:b] = torch.matmul(torch.softmax(sc, dim=-1), vf.contiguous()).permute(1, 0, 2)
    return out


def test_prefill_c3_full_size():
    """C3 at full size: every row against the f64 oracle and against a float32 torch reference,
    and the appended pool rows bit-exact."""
    w = W.prefill_c3()
    t = W.make_prefill_tensors(w)
    lay = sp.layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
    announce(f"prefill {w.name} lens={list(w.lens)}")
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k"], t["v"], t["slot_mapping"])
    sp.varlen_prefill(t["out"], t["q"], t["k"], t["v"], t["cu_seqlens"], t["cu_seqlens"],
                      w.max_seqlen, w.head_dim ** -0.5)
    torch.cuda.synchronize()
    ref = _torch_ref_causal(t["q"], t["k"], t["v"], w.cu_seqlens, w.head_dim ** -0.5)
    err = (t["out"].float() - ref).abs().max().item()
    assert err <= 2e-2, f"C3 vs fp32 torch: {err}"
    # every row of every sequence against the f64 oracle
    q, k, v = host_array(t["q"]), host_array(t["k"]), host_array(t["v"])
    got = _as_f64(t["out"])
    cu = w.cu_seqlens
    for s in range(w.num_seqs):
        a, b = int(cu[s]), int(cu[s + 1])
        r = O.attention_f64(q[a:b], k[a:b], v[a:b], scale=w.head_dim ** -0.5, causal=True,
                            q_pos0=0, dtype=O.BF16)
        assert_attention_close(got[a:b], r, "bf16", f"C3 seq {s}")
    # the append wrote every token's rows exactly
    tables, _ = w.pool_tables()
    kp = t["k_pool"]
    for s in range(w.num_seqs):
        L = int(w.lens[s])
        pos = torch.arange(L, device="cuda")
        blk = torch.from_numpy(tables[s]).cuda()[pos // w.block_size].long()
        rows = kp[blk, 0, :, pos % w.block_size, :]             # [L, Hkv, D]
        assert torch.equal(rows, t["k"][cu[s]:cu[s + 1]])
