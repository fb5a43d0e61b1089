"""flash_attention at its only caller's shapes and with every FlashAttentionOptions field
(sketchpad-cubecl attention.rs:39-178): the SD-1.x UNet's head dims 40 / 80 / 160 without the
padding its caller applies today (sketchpad-unet/src/cubecl.rs:256-316), the padded 256, cross
attention over the 77 CLIP tokens, a value head dim of its own, out_dtype, and the additive mask
on 16-bit tensors.

Every row is checked against float64 attention computed by torch on the GPU, and sampled rows
against the f64 oracle: f32 at 1e-5 relative per row, 16-bit at 2e-2 absolute."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from tests.helpers import announce, as_f64, assert_attention_close, host_array

pytestmark = pytest.mark.gpu


def _f64_reference(q, k, v, mask=None, causal=False):
    """softmax(q k^T d^-1/2 + mask) v in float64 on the GPU, per (batch, head)."""
    qd, kd, vd = (x.double() for x in (q, k, v))
    sc = torch.matmul(qd, kd.transpose(-1, -2).contiguous()) * q.shape[-1] ** -0.5
    if mask is not None:
        sc = sc + mask.double()
    if causal:
        sq, sk = sc.shape[-2:]
        sc = sc.masked_fill(torch.ones(sq, sk, dtype=torch.bool, device=q.device).triu(1),
                            float("-inf"))
    return torch.matmul(torch.softmax(sc, dim=-1), vd)


def _oracle_rows(q, k, v, rows, dtype, mask=None, causal=False):
    """The f64 oracle (attention_f64) on the given query rows of every (batch, head)."""
    B, H = q.shape[:2]
    qh, kh, vh = host_array(q), host_array(k), host_array(v)
    mh = None if mask is None else mask.expand(B, H, q.shape[2], k.shape[2]).cpu().numpy()
    out = np.zeros((B, H, len(rows), v.shape[-1]))
    for b in range(B):
        for h in range(H):
            m = None
            if mh is not None:
                m = mh[b, h][rows]
            if causal:
                i, j = np.asarray(rows)[:, None], np.arange(k.shape[2])[None, :]
                cm = np.where(j > i, -np.inf, 0.0).astype(np.float32)
                m = cm if m is None else m + cm
            if m is not None:
                # one query at a time: the oracle's mask is [Sq, Sk] for a contiguous block
                for r_i, r in enumerate(rows):
                    out[b, h, r_i] = O.attention_f64(qh[b, h][r:r + 1, None], kh[b, h][:, None],
                                                     vh[b, h][:, None], scale=q.shape[-1] ** -0.5,
                                                     mask=m[r_i:r_i + 1], q_pos0=0,
                                                     dtype=dtype)[0, 0]
            else:
                out[b, h] = O.attention_f64(qh[b, h][rows][:, None], kh[b, h][:, None],
                                            vh[b, h][:, None], scale=q.shape[-1] ** -0.5,
                                            q_pos0=0, dtype=dtype)[:, 0]
    return out


def _check(out, q, k, v, what, *, mask=None, causal=False, rows=(0, 1, 77, 1000)):
    dt_name = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[out.dtype]
    ref = _f64_reference(q, k, v, mask, causal).cpu().numpy()
    got = as_f64(out)
    assert_attention_close(got, ref, dt_name, f"{what} vs float64 torch")
    rows = sorted({r for r in rows if r < q.shape[2]} | {q.shape[2] - 1})
    odt = {torch.float32: O.F32, torch.bfloat16: O.BF16, torch.float16: O.F16}[q.dtype]
    oref = _oracle_rows(q, k, v, rows, odt, mask, causal)
    assert_attention_close(got[:, :, rows], oref, dt_name, f"{what} vs the f64 oracle")


@pytest.mark.parametrize("d", [40, 80, 160, 256])
def test_flash_unet_self_attention_f32(d):
    """SD-1.x self-attention at the largest latent (64x64 = 4096 tokens), 2 x 8 heads, f32 (the
    element type the caller casts to), head dims 40 / 80 / 160 natively and the padded 256."""
    g = torch.Generator(device="cuda").manual_seed(d)
    q, k, v = (torch.randn(2, 8, 4096, d, generator=g, device="cuda") for _ in range(3))
    out = torch.full_like(q, float("nan"))
    announce(f"flash self-attention f32 [2, 8, 4096, {d}]")
    sp.flash_attention(out, q, k, v, d ** -0.5)
    torch.cuda.synchronize()
    _check(out, q, k, v, f"self-attention d={d}")


@pytest.mark.parametrize("d", [40, 80, 160])
def test_flash_unet_cross_attention_f32(d):
    """Cross-attention over the 77 CLIP context tokens without padding them to 128 (the caller
    pads K/V with unmasked zero rows today, which changes the result)."""
    g = torch.Generator(device="cuda").manual_seed(100 + d)
    q = torch.randn(2, 8, 4096, d, generator=g, device="cuda")
    k, v = (torch.randn(2, 8, 77, d, generator=g, device="cuda") for _ in range(2))
    out = torch.full_like(q, float("nan"))
    announce(f"flash cross-attention f32 q [2, 8, 4096, {d}] ctx 77")
    sp.flash_attention(out, q, k, v, d ** -0.5)
    torch.cuda.synchronize()
    _check(out, q, k, v, f"cross-attention d={d}")


@pytest.mark.parametrize("d,dv", [(64, 128), (128, 64), (40, 160), (160, 40), (80, 256)])
def test_flash_value_head_dim(d, dv):
    """v [B, H, Sk, Dv] with Dv != D: out is [B, H, Sq, Dv] (attention.rs:140-143)."""
    g = torch.Generator(device="cuda").manual_seed(d * 7 + dv)
    q = torch.randn(2, 3, 150, d, generator=g, device="cuda")
    k = torch.randn(2, 3, 200, d, generator=g, device="cuda")
    v = torch.randn(2, 3, 200, dv, generator=g, device="cuda")
    out = torch.full((2, 3, 150, dv), float("nan"), device="cuda")
    announce(f"flash f32 d={d} dv={dv}")
    sp.flash_attention_ex(out, q, k, v, d ** -0.5)
    torch.cuda.synchronize()
    _check(out, q, k, v, f"d={d} dv={dv}", rows=(0, 64, 127))


@pytest.mark.parametrize("out_dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_out_dtype(out_dt, causal):
    """FlashAttentionOptions.out_dtype: the f32 result rounded once to the output type, bit for
    bit the rounding of the f32 output (torch's round-to-nearest-even conversion)."""
    g = torch.Generator(device="cuda").manual_seed(5 + causal)
    q, k, v = (torch.randn(1, 4, 300, 80, generator=g, device="cuda") for _ in range(3))
    o32 = torch.empty_like(q)
    o16 = torch.empty(q.shape, dtype=out_dt, device="cuda")
    announce(f"flash f32 -> {out_dt} causal={causal}")
    sp.flash_attention_ex(o32, q, k, v, 80 ** -0.5, causal=causal)
    sp.flash_attention_ex(o16, q, k, v, 80 ** -0.5, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(o16, o32.to(out_dt))
    _check(o32, q, k, v, "f32 out", causal=causal, rows=(0, 150))


def test_flash_bf16_to_f32_out():
    """16-bit inputs with an f32 output: the fp32 result before any 16-bit rounding."""
    g = torch.Generator(device="cuda").manual_seed(9)
    q, k, v = (torch.randn(2, 4, 200, 128, generator=g, device="cuda").bfloat16()
               for _ in range(3))
    o32 = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    o16 = torch.empty_like(q)
    announce("flash bf16 -> f32 out")
    sp.flash_attention_ex(o32, q, k, v, 128 ** -0.5)
    sp.flash_attention_ex(o16, q, k, v, 128 ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(o16, o32.to(torch.bfloat16))
    ref = _f64_reference(q, k, v).cpu().numpy()
    # the bf16 kernel's P is 16-bit: the 2e-2 bar of 16-bit inputs
    assert np.abs(as_f64(o32) - ref).max() <= 2e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("per_head", [False, True])
def test_flash_masked_16bit(dtype, per_head):
    """flash_attention_masked on 16-bit tensors (the mask stays f32): random biases, padded keys
    at -inf, a row half at -1e4, against float64."""
    B, H, sq, sk, d = 2, 3, 90, 150, 64
    g = torch.Generator(device="cuda").manual_seed(71 + per_head)
    q, k, v = (torch.randn(B, H, n, d, generator=g, device="cuda").to(dtype)
               for n in (sq, sk, sk))
    mshape = (B, H, sq, sk) if per_head else (sq, sk)
    mask = 2.0 * torch.randn(*mshape, generator=g, device="cuda")
    mask[..., sk - 7:] = float("-inf")
    mask[..., 5, sk // 2:] = -1e4
    out = torch.full_like(q, float("nan"))
    announce(f"flash_attention_masked {dtype} per_head={per_head}")
    sp.flash_attention_masked(out, q, k, v, mask, d ** -0.5)
    torch.cuda.synchronize()
    _check(out, q, k, v, "masked 16-bit", mask=mask, rows=(0, 5, 89))


def test_flash_ex_rejects_unsupported_dims():
    q = torch.zeros(1, 1, 8, 48, device="cuda")
    with pytest.raises(sp.SketchpadError) as e:
        sp.flash_attention_ex(torch.empty_like(q), q, q, q, 0.1)
    assert e.value.code == sp._lib.SP_EUNSUPPORTED
    qb = torch.zeros(1, 1, 8, 80, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(sp.SketchpadError) as e:
        sp.flash_attention_ex(torch.empty_like(qb), qb, qb, qb, 0.1)
    assert e.value.code == sp._lib.SP_EUNSUPPORTED
