"""The HIP path on the committed golden fixtures (tests/golden/), through the C ABI: the append
bit-exact (pool digests), decode within 1e-5 relative (f32) or 2e-2 absolute (bf16), prefill
within 2e-2 absolute, RoPE-fused append bit-exact, PolarQuant records bit-exact."""
import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from tests.helpers import announce, assert_attention_close

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLDEN / name, allow_pickle=False)


def _dev(a, bf16=False):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if bf16:
        t = t.view(torch.bfloat16)
    return t.cuda()


def _bits(t):
    t = t.contiguous().cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


@pytest.mark.parametrize("name", ["decode_f32.npz", "decode_bf16_window.npz"])
def test_golden_decode(name):
    f = _load(name)
    bf16 = str(f["dtype"]) == "bf16"
    announce(f"golden decode {name}")
    k_pool, v_pool = _dev(f["k_pool"], bf16), _dev(f["v_pool"], bf16)
    q, k_new, v_new = (_dev(f[x], bf16) for x in ("q", "k_new", "v_new"))
    nblk, _, hkv, bs, d = k_pool.shape
    lay = sp.layout(nblk, 1, 0, hkv, bs, d)
    sp.kv_append(k_pool, v_pool, lay, k_new, v_new, _dev(f["slot_mapping"]))
    lens = f["context_lens"]
    window = int(f["window_left"])
    ws = sp.alloc_decode_workspace(len(lens), q.shape[1], int(lens.max()), window, lay)
    out = torch.full_like(q, float("nan"))
    sp.paged_decode(out, q, k_pool, v_pool, lay, _dev(f["block_tables"]), _dev(lens),
                    int(lens.max()), float(f["scale"]), window_left=window, workspace=ws)
    torch.cuda.synchronize()
    assert hashlib.sha256(_bits(k_pool).tobytes()).hexdigest() == str(f["k_pool_after_sha256"])
    assert hashlib.sha256(_bits(v_pool).tobytes()).hexdigest() == str(f["v_pool_after_sha256"])
    got = out.double().cpu().numpy()
    assert_attention_close(got, f["out"], "bf16" if bf16 else "f32", name)


@pytest.mark.parametrize("name", ["prefill_bf16.npz", "prefill_bf16_chunked_window.npz"])
def test_golden_varlen_prefill(name):
    f = _load(name)
    announce(f"golden prefill {name}")
    q, k, v = (_dev(f[x], True) for x in ("q", "k", "v"))
    cu_q, cu_k = f["cu_seqlens_q"], f["cu_seqlens_k"]
    out = torch.full_like(q, float("nan"))
    sp.varlen_prefill(out, q, k, v, _dev(cu_q), _dev(cu_k), int(np.diff(cu_q).max()),
                      float(f["scale"]), causal=sp.SP_CAUSAL_BOTTOM_RIGHT,
                      window_left=int(f["window_left"]))
    torch.cuda.synchronize()
    assert_attention_close(out.double().cpu().numpy(), f["out"].astype(np.float64), "bf16", name)


def test_golden_rope_append():
    f = _load("rope_f32.npz")
    announce("golden rope append")
    x = f["x"]
    t, h, d = x.shape
    rows = int(f["rows"])
    cos, sin = sp.rope_tables(rows, d)
    # the half tables hold each pair's angle once; the reference's caches hold it twice
    assert np.array_equal(cos, f["cos_full"][:, 0::2]) and np.array_equal(sin, f["sin_full"][:, 0::2])
    bs = 16
    lay = sp.layout(1, 1, 0, h, bs, d)
    k_pool = torch.zeros(1, 1, h, bs, d, device="cuda")
    v_pool = torch.zeros_like(k_pool)
    k_new = _dev(x)
    slots = torch.arange(t, dtype=torch.int32, device="cuda")
    sp.rope_kv_append(k_pool, v_pool, lay, k_new, k_new.clone(), _dev(f["positions"]), slots,
                      _dev(cos), _dev(sin))
    torch.cuda.synchronize()
    got = k_pool[0, 0, :, :t].transpose(0, 1).cpu().numpy()  # [T, H, D]
    assert np.array_equal(got.view(np.uint32), f["rotated"].view(np.uint32))
    assert np.array_equal(v_pool[0, 0, :, :t].transpose(0, 1).cpu().numpy(), x)


def test_golden_polar_records():
    f = _load("polar_f32.npz")
    announce("golden polar compress/decompress")
    x = _dev(f["x"])
    rec = torch.zeros(f["records"].shape, dtype=torch.uint8, device="cuda")
    sp.polar_compress(rec, x)
    out = torch.full_like(x, float("nan"))
    sp.polar_decompress(out, rec)
    torch.cuda.synchronize()
    assert np.array_equal(rec.cpu().numpy(), f["records"])
    assert np.array_equal(out.cpu().numpy().view(np.uint32), f["decompressed"].view(np.uint32))


def test_golden_qjl_records():
    f = _load("qjl_f32.npz")
    for d, p in ((32, 8), (64, 16)):
        announce(f"golden qjl d={d} p={p}")
        proj = sp.qjl_projection(p, d)
        assert np.array_equal(proj.cpu().numpy().view(np.uint32), f[f"proj{d}"].view(np.uint32))
        x = _dev(f[f"x{d}"])
        rec = torch.zeros(f[f"records{d}"].shape, dtype=torch.uint8, device="cuda")
        sp.qjl_compress(rec, x, proj)
        out = torch.full_like(x, float("nan"))
        sp.qjl_decompress(out, rec, proj)
        torch.cuda.synchronize()
        assert np.array_equal(rec.cpu().numpy(), f[f"records{d}"])
        assert np.array_equal(out.cpu().numpy().view(np.uint32),
                              f[f"decompressed{d}"].view(np.uint32))


def test_golden_flash_f32():
    """f32 flash attention (plain, causal, additive mask) within 1e-5 per row of the frozen
    float64 outputs."""
    f = _load("flash_f32.npz")
    q, k, v = (torch.from_numpy(f[n]).transpose(0, 1).contiguous()[None].cuda()
               for n in ("q", "k", "v"))
    d = q.shape[-1]
    for name, causal, mask in (("out_full", False, None), ("out_causal", True, None),
                               ("out_masked", False, f["mask"])):
        announce(f"golden flash f32 {name}")
        out = torch.full_like(q, float("nan"))
        if mask is None:
            sp.flash_attention(out, q, k, v, d ** -0.5, causal=causal)
        else:
            sp.flash_attention_masked(out, q, k, v, torch.from_numpy(mask).cuda(), d ** -0.5)
        torch.cuda.synchronize()
        got = out[0].transpose(0, 1).double().cpu().numpy()
        assert_attention_close(got, f[name], "f32", name)
