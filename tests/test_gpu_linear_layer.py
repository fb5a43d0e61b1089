"""GPU parity of the projections around the path (sp_linear: burn's nn::Linear as
MultiHeadAttention applies it, transformer.rs:196-208, :249-253) and of a whole attention layer
composed through the C ABI: q/k/v projections, RoPE fused into the paged append, decode or chunked
prefill, o projection — MultiHeadAttention::forward_cached (transformer.rs:184-254) for a ragged
batch. References:
  - sp_linear: the float64 product of the same (exactly converted) inputs, rounded to the element
    type, plus the bias rounded again (matmul then + bias, as two ops): the kernel's fp32
    accumulation may move a result by one unit in the last place;
  - the layer: the same chain in float64 with the element-type rounding at the same points,
    using the oracle's RoPE restatement (rope.rs) and float64 attention (transformer.rs:227-243)."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from tests.helpers import announce

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
ULP = {"f32": 2.0 ** -23, "bf16": 2.0 ** -7, "f16": 2.0 ** -10}


def _round(a64: torch.Tensor, dtype: str) -> torch.Tensor:
    """float64 -> element type (round to nearest even) -> float64."""
    return a64.to(DT[dtype]).to(torch.float64)


def _linear_ref(x, w, b, dtype):
    prod = _round(x.double().cpu() @ w.double().cpu().t(), dtype)
    ref = _round(prod + b.double().cpu(), dtype) if b is not None else prod
    return prod, ref


def _linear_tol(x, w, prod, ref, dtype):
    # fp32 accumulation order: allow a couple of units in the last place of the product (which
    # may exceed the final value when the bias cancels part of it) and of the result, plus the
    # fp32 rounding of a K-term sum measured against the magnitude of its terms
    k = x.shape[-1]
    terms = x.double().abs().cpu() @ w.double().abs().cpu().t()
    return 2 * ULP[dtype] * torch.maximum(ref.abs(), prod.abs()) + 2 * k * 2.0 ** -24 * terms + 1e-30


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("m,k,n", [(1, 64, 32), (64, 4096, 6144), (7, 96, 40), (300, 512, 1024),
                                   (129, 136, 130), (65, 1024, 4096), (2, 8192, 1027),
                                   (512, 128, 256), (1000, 512, 523), (777, 1024, 1000),
                                   (1024, 4096, 1536), (1, 4096, 4096), (17, 2048, 2048),
                                   (64, 512, 3000), (33, 1024, 2050)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_linear(dtype, m, k, n, with_bias):
    """y = x . w^T (+ b) with w [out, in]; M/N tails, K not a multiple of the 32-deep stage,
    the 64-row (decode), 128-row and 256 x 256 (M >= 512) tiles, split K with partials."""
    announce(f"linear {dtype} M={m} K={k} N={n} bias={with_bias}")
    g = torch.Generator(device="cuda").manual_seed(m * 7 + k + n)
    x = torch.randn(m, k, generator=g, device="cuda").to(DT[dtype])
    w = (torch.randn(n, k, generator=g, device="cuda") * k ** -0.5).to(DT[dtype])
    b = torch.randn(n, generator=g, device="cuda").to(DT[dtype]) if with_bias else None
    y = torch.empty(m, n, dtype=DT[dtype], device="cuda")
    ws = sp.alloc_linear_workspace([(m, k, n)])
    sp.linear(y, x, w, b, workspace=ws)
    torch.cuda.synchronize()
    prod, ref = _linear_ref(x, w, b, dtype)
    got = y.double().cpu()
    bad = (got - ref).abs() > _linear_tol(x, w, prod, ref, dtype)
    assert not bad.any(), (int(bad.sum()), float((got - ref).abs().max()))


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_linear_split_counts_and_determinism(dtype):
    """A decode-shaped GEMM with the full split, a workspace for two splits, and none: each
    within the bound of the float64 product, and each bit-identical when repeated."""
    announce(f"linear split-K {dtype}")
    m, k, n = 16, 4096, 1024
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(m, k, generator=g, device="cuda").to(DT[dtype])
    w = (torch.randn(n, k, generator=g, device="cuda") * k ** -0.5).to(DT[dtype])
    b = torch.randn(n, generator=g, device="cuda").to(DT[dtype])
    full = sp.linear_workspace_size(m, k, n)
    assert full >= 2 * m * n * 4
    prod, ref = _linear_ref(x, w, b, dtype)
    tol = _linear_tol(x, w, prod, ref, dtype)
    for ws_bytes in (full, 2 * m * n * 4, 0):
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")[:ws_bytes] \
            if ws_bytes else None
        outs = []
        for _ in range(2):
            y = torch.empty(m, n, dtype=DT[dtype], device="cuda")
            sp.linear(y, x, w, b, workspace=ws)
            outs.append(y)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), ws_bytes
        bad = (outs[0].double().cpu() - ref).abs() > tol
        assert not bad.any(), (ws_bytes, int(bad.sum()))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("k,n", [(64, 32), (33, 70), (4096, 1024), (1, 5)])
def test_linear_weight_nk(dtype, k, n):
    """burn's [in, out] weight -> [out, in], bit-exact."""
    announce(f"linear weight transpose {dtype} K={k} N={n}")
    g = torch.Generator(device="cuda").manual_seed(k + n)
    w = torch.randn(k, n, generator=g, device="cuda").to(DT[dtype])
    got = sp.linear_weight_nk(w)
    torch.cuda.synchronize()
    assert got.shape == (n, k)
    assert torch.equal(got, w.t().contiguous())


def test_linear_without_workspace_and_validation():
    announce("linear without workspace")
    x = torch.randn(16, 128, device="cuda").to(torch.bfloat16)
    w = torch.randn(64, 128, device="cuda").to(torch.bfloat16)
    y = torch.empty(16, 64, dtype=torch.bfloat16, device="cuda")
    sp.linear(y, x, w)
    torch.cuda.synchronize()
    ref = _round(x.double().cpu() @ w.double().cpu().t(), "bf16")
    assert (y.double().cpu() - ref).abs().max() <= 4 * ULP["bf16"] * ref.abs().max()
    with pytest.raises(sp.SketchpadError):  # K not a multiple of 8
        sp.linear(y, x[:, :100].contiguous(), w[:, :100].contiguous())
    with pytest.raises(sp.SketchpadError):  # x not 16-byte aligned
        xs = torch.empty(16 * 128 + 1, dtype=torch.bfloat16, device="cuda")[1:].view(16, 128)
        sp.linear(y, xs, w)


def _layer_case(seed, *, new_lens, ctx_lens, hidden, hq, hkv, d, bs, dtype, bias):
    """One attention layer step of a ragged batch: sequence s has ctx_lens[s] cached tokens and
    appends new_lens[s] tokens (decode when all are 1)."""
    rng = np.random.default_rng(seed)
    B = len(new_lens)
    new_lens, ctx_lens = np.asarray(new_lens), np.asarray(ctx_lens)
    total = ctx_lens + new_lens
    nblk = int(((total + bs - 1) // bs).sum()) + 2
    perm = rng.permutation(nblk).astype(np.int32)
    maxb = int(((total + bs - 1) // bs).max())
    tables = np.zeros((B, maxb), np.int32)
    off = 0
    for s in range(B):
        nb = int((total[s] + bs - 1) // bs)
        tables[s, :nb] = perm[off:off + nb]
        off += nb
    dt = DT[dtype]
    g = torch.Generator(device="cuda").manual_seed(seed)
    T = int(new_lens.sum())
    x = torch.randn(T, hidden, generator=g, device="cuda").to(dt)
    # weights [out, in]
    wq = (torch.randn(hq * d, hidden, generator=g, device="cuda") * hidden ** -0.5).to(dt)
    wk = (torch.randn(hkv * d, hidden, generator=g, device="cuda") * hidden ** -0.5).to(dt)
    wv = (torch.randn(hkv * d, hidden, generator=g, device="cuda") * hidden ** -0.5).to(dt)
    wo = (torch.randn(hidden, hq * d, generator=g, device="cuda") * (hq * d) ** -0.5).to(dt)
    bq = torch.randn(hq * d, generator=g, device="cuda").to(dt) * 0.1 if bias else None
    bkv = torch.randn(2 * hkv * d, generator=g, device="cuda").to(dt) * 0.1 if bias else None
    bo = torch.randn(hidden, generator=g, device="cuda").to(dt) * 0.1 if bias else None
    wkv = torch.cat([wk, wv], dim=0).contiguous()  # one GEMM for k and v
    # the cached context: random K/V rows (already rotated) in the pools
    k_pool = torch.zeros(nblk, 1, hkv, bs, d, dtype=dt, device="cuda")
    v_pool = torch.zeros_like(k_pool)
    kc = torch.randn(nblk, 1, hkv, bs, d, generator=g, device="cuda").to(dt)
    vc = torch.randn(nblk, 1, hkv, bs, d, generator=g, device="cuda").to(dt)
    k_pool.copy_(kc)
    v_pool.copy_(vc)
    positions = np.concatenate([ctx_lens[s] + np.arange(new_lens[s]) for s in range(B)])
    seq_of = np.concatenate([np.full(new_lens[s], s) for s in range(B)])
    slots = (tables[seq_of, positions // bs] * bs + positions % bs).astype(np.int32)
    rows = int(total.max()) + 1
    cos_h, sin_h = sp.rope_tables(rows, d, 10000.0)
    cos_d, sin_d = torch.from_numpy(cos_h).cuda(), torch.from_numpy(sin_h).cuda()
    lay = sp.layout(nblk, 1, 0, hkv, bs, d)
    ws = sp.alloc_linear_workspace([(T, hidden, hq * d), (T, hidden, 2 * hkv * d),
                                    (T, hq * d, hidden)])
    # --- the layer through the C ABI ---
    q = torch.empty(T, hq * d, dtype=dt, device="cuda")
    kv = torch.empty(T, 2 * hkv * d, dtype=dt, device="cuda")
    sp.linear(q, x, wq, bq, workspace=ws)
    sp.linear(kv, x, wkv, bkv, workspace=ws)
    q3 = q.view(T, hq, d)
    sp.rope_kv_append(k_pool, v_pool, lay, kv[:, :hkv * d], kv[:, hkv * d:],
                      torch.from_numpy(positions.astype(np.int32)).cuda(),
                      torch.from_numpy(slots).cuda(), cos_d, sin_d, q=q3,
                      token_stride=2 * hkv * d, head_stride=d)
    attn = torch.empty(T, hq, d, dtype=dt, device="cuda")
    tab_d = torch.from_numpy(tables).cuda()
    lens_d = torch.from_numpy(total.astype(np.int32)).cuda()
    if (new_lens == 1).all():
        dws = sp.alloc_decode_workspace(B, hq, int(total.max()), -1, lay)
        sp.paged_decode(attn, q3, k_pool, v_pool, lay, tab_d, lens_d, int(total.max()),
                        d ** -0.5, workspace=dws)
    else:
        cu = torch.from_numpy(np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)).cuda()
        sp.paged_prefill(attn, q3, k_pool, v_pool, lay, tab_d, cu, lens_d, int(new_lens.max()),
                         d ** -0.5)
    out = torch.empty(T, hidden, dtype=dt, device="cuda")
    sp.linear(out, attn.view(T, hq * d), wo, bo, workspace=ws)
    torch.cuda.synchronize()
    # --- float64 chain with the same rounding points ---
    def lin(a, w, b):
        r = _round(a @ w.double().cpu().t(), dtype)
        return _round(r + b.double().cpu(), dtype) if b is not None else r
    x64 = x.double().cpu()
    q_r = lin(x64, wq, bq).view(T, hq, d)
    kv_r = lin(x64, wkv, bkv)
    k_r, v_r = kv_r[:, :hkv * d].reshape(T, hkv, d), kv_r[:, hkv * d:].reshape(T, hkv, d)
    cos_f, sin_f = O.rope_caches(rows, d, 10000.0)
    q_rot = _round(torch.from_numpy(O.rope_apply(q_r.float().cpu().numpy(), positions, cos_f,
                                                 sin_f)).double(), dtype).numpy()
    k_rot = _round(torch.from_numpy(O.rope_apply(k_r.float().cpu().numpy(), positions, cos_f,
                                                 sin_f)).double(), dtype).numpy()
    v_np = v_r.cpu().numpy()
    kc_np, vc_np = kc.double().cpu().numpy(), vc.double().cpu().numpy()
    attn_ref = np.zeros((T, hq, d))
    t0 = 0
    for s in range(B):
        L, n = int(total[s]), int(new_lens[s])
        pos = np.arange(L)
        blk, sl = tables[s, pos // bs], pos % bs
        ks = kc_np[blk, 0, :, sl].copy()  # [L, hkv, d]
        vs = vc_np[blk, 0, :, sl].copy()
        ks[ctx_lens[s]:] = k_rot[t0:t0 + n]
        vs[ctx_lens[s]:] = v_np[t0:t0 + n]
        attn_ref[t0:t0 + n] = O.attention_f64(q_rot[t0:t0 + n].astype(np.float32),
                                              ks.astype(np.float32), vs.astype(np.float32),
                                              scale=d ** -0.5, causal=True,
                                              q_pos0=int(ctx_lens[s]))
        t0 += n
    attn_r = _round(torch.from_numpy(attn_ref), dtype)
    out_ref = lin(attn_r.view(T, hq * d), wo, bo)
    return out.double().cpu(), out_ref, attn.double().cpu(), attn_r


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_layer_decode(dtype):
    """Llama-3-8B layer shape (hidden 4096, Hq 32, Hkv 8, D 128), one new token per sequence."""
    announce(f"attention layer decode {dtype}")
    got, ref, attn, attn_ref = _layer_case(3, new_lens=[1] * 6, ctx_lens=[0, 5, 17, 130, 511, 900],
                                           hidden=4096, hq=32, hkv=8, d=128, bs=16, dtype=dtype,
                                           bias=False)
    assert (attn - attn_ref).abs().max() <= 2e-2
    assert (got - ref).abs().max() <= 2e-2 * max(1.0, float(ref.abs().max()))


def test_layer_chunked_prefill_with_bias():
    """Qwen-style biases on q/k/v (and o), prompt chunks against cached contexts."""
    announce("attention layer chunked prefill bf16 with bias")
    got, ref, attn, attn_ref = _layer_case(4, new_lens=[7, 33, 1, 64], ctx_lens=[0, 40, 300, 16],
                                           hidden=512, hq=8, hkv=2, d=64, bs=16, dtype="bf16",
                                           bias=True)
    assert (attn - attn_ref).abs().max() <= 2e-2
    assert (got - ref).abs().max() <= 2e-2 * max(1.0, float(ref.abs().max()))
