"""The C-ABI library: it loads, exports every entry point include/*.h declares, and rejects
invalid arguments on the host with a status code and message (no GPU needed: validation runs
before anything is enqueued)."""
import ctypes
import re
from pathlib import Path

import pytest

from sketchpad_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def _declared_functions():
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(sp_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = _declared_functions()
    for n in ("sp_version", "sp_last_error", "sp_kv_append", "sp_kv_gather",
              "sp_paged_decode", "sp_paged_decode_workspace_size"):
        assert n in names


def test_library_exports_every_declared_symbol(sp_lib):
    missing = [n for n in _declared_functions() if not hasattr(sp_lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    assert set(_declared_functions()) <= set(_lib._SIGNATURES), \
        set(_declared_functions()) - set(_lib._SIGNATURES)


def test_version(sp_lib):
    assert sp_lib.sp_version() == 1


def _lay(**kw):
    d = dict(num_blocks=8, num_layers=1, layer=0, num_kv_heads=2, block_size=16, head_dim=64)
    d.update(kw)
    return _lib.CacheLayout(**d)


def _expect(code, rc, needle):
    lib = _lib.load()
    assert rc == code, (rc, lib.sp_last_error())
    assert needle in lib.sp_last_error().decode()


def test_append_validation(sp_lib):
    f = sp_lib.sp_kv_append
    fake = ctypes.c_void_p(0x1000)
    _expect(_lib.SP_EINVAL, f(fake, fake, None, fake, fake, 128, 64, fake, 1, 0, None), "layout")
    _expect(_lib.SP_EOOB, f(fake, fake, ctypes.byref(_lay(layer=1)), fake, fake, 128, 64, fake, 1,
                            0, None), "layer 1")
    _expect(_lib.SP_EINVAL, f(fake, fake, ctypes.byref(_lay(block_size=0)), fake, fake, 128, 64,
                              fake, 1, 0, None), "positive")
    _expect(_lib.SP_EINVAL, f(fake, fake, ctypes.byref(_lay()), fake, fake, 128, 64, fake, 1, 9,
                              None), "dtype")
    _expect(_lib.SP_EINVAL, f(None, fake, ctypes.byref(_lay()), fake, fake, 128, 64, fake, 1, 0,
                              None), "NULL")
    assert f(None, None, ctypes.byref(_lay()), None, None, 0, 0, None, 0, 0, None) == 0


def test_gather_validation(sp_lib):
    f = sp_lib.sp_kv_gather
    fake = ctypes.c_void_p(0x1000)
    _expect(_lib.SP_EOOB, f(fake, fake, fake, fake, ctypes.byref(_lay()), fake, 1, 17, 0, None),
            "needs 2 blocks")
    assert f(None, None, None, None, ctypes.byref(_lay()), None, 0, 0, 0, None) == 0


def test_decode_validation(sp_lib):
    f = sp_lib.sp_paged_decode
    fake = ctypes.c_void_p(0x1000)

    def call(lay, hq=4, max_ctx=32, mbs=2, window=-1, ws=None, ws_bytes=0, dtype=1, scale=0.125):
        return f(fake, fake, fake, fake, ctypes.byref(lay), fake, mbs, fake, max_ctx, 3, hq, scale,
                 window, dtype, ws, ws_bytes, None)

    _expect(_lib.SP_EINVAL, call(_lay(), hq=3), "multiple")
    _expect(_lib.SP_EUNSUPPORTED, call(_lay(), hq=34), "GQA group 17")
    _expect(_lib.SP_EUNSUPPORTED, call(_lay(head_dim=96)), "head_dim 96")
    _expect(_lib.SP_EOOB, call(_lay(), max_ctx=33), "exceeds the block tables")
    _expect(_lib.SP_EINVAL, call(_lay(), window=-2), "window_left")
    _expect(_lib.SP_EINVAL, call(_lay(), scale=float("inf")), "scale")
    # dense pools take any block size (the GPU tests run 1-8, 12, 16, 24, 32, 48); the PolarQuant
    # pools' multiple-of-16 rule is checked in test_polar_pool_bytes_and_validation
    # a batch needing split-K partials refuses a missing workspace
    lay = _lay(num_blocks=4096)
    need = sp_lib.sp_paged_decode_workspace_size(3, 4, 4096, -1, ctypes.byref(lay))
    assert need > 0
    _expect(_lib.SP_ENOSPACE, call(lay, max_ctx=4096, mbs=256), "workspace")
    # (the size is the larger of the dense and the PolarQuant plans' partials, so the dense
    # plan's own boundary is not visible here: a workspace far below it)
    _expect(_lib.SP_ENOSPACE, call(lay, max_ctx=4096, mbs=256, ws=fake, ws_bytes=need // 8),
            "workspace")


def test_append_decode_validation(sp_lib):
    f = sp_lib.sp_paged_append_decode
    fake = ctypes.c_void_p(0x1000)

    def call(lay, kn=fake, vn=fake, ts=256, hs=64, hq=4, max_ctx=32, mbs=2, seqs=3, dtype=1,
             out=fake):
        return f(out, fake, fake, fake, ctypes.byref(lay), kn, vn, ts, hs, fake, mbs, fake,
                 max_ctx, seqs, hq, 0.125, -1, dtype, None, 0, None)

    # the decode's own checks come first
    _expect(_lib.SP_EINVAL, call(_lay(), hq=3), "multiple")
    _expect(_lib.SP_EOOB, call(_lay(), max_ctx=33), "exceeds the block tables")
    # then the new rows'
    _expect(_lib.SP_EINVAL, call(_lay(), kn=None), "NULL")
    _expect(_lib.SP_EINVAL, call(_lay(), vn=None), "NULL")
    _expect(_lib.SP_EINVAL, call(_lay(), ts=-1), "negative stride")
    _expect(_lib.SP_EINVAL, call(_lay(), hs=4), "16-byte aligned")         # 8 bytes (bf16)
    _expect(_lib.SP_EINVAL, call(_lay(), kn=ctypes.c_void_p(0x1008)), "16-byte aligned")
    _expect(_lib.SP_EINVAL, call(_lay(), out=ctypes.c_void_p(0x1008)), "16-byte aligned")
    assert call(_lay(), seqs=0) == 0  # an empty batch enqueues nothing


def test_rope_validation(sp_lib):
    f = sp_lib.sp_rope_kv_append
    fake = ctypes.c_void_p(0x1000)

    def call(lay, q=None, hq=0, tokens=1, rows=8, dtype=1, cos=fake):
        return f(fake, fake, ctypes.byref(lay), fake, fake, 128, 64, q, 256, 64, hq, fake, fake,
                 tokens, cos, fake, rows, dtype, None)

    _expect(_lib.SP_EINVAL, call(_lay(head_dim=63)), "odd")
    _expect(_lib.SP_EINVAL, call(_lay(), tokens=-1), "num_tokens")
    _expect(_lib.SP_EINVAL, call(_lay(), cos=None), "NULL")
    _expect(_lib.SP_EINVAL, call(_lay(), q=fake, hq=0), "num_q_heads")
    _expect(_lib.SP_EINVAL, call(_lay(), dtype=7), "dtype")
    assert call(_lay(), tokens=0) == 0
    t = sp_lib.sp_rope_tables
    _expect(_lib.SP_EINVAL, t(fake, fake, 4, 7, ctypes.c_float(10000.0)), "even")
    _expect(_lib.SP_EINVAL, t(fake, fake, 4, 8, ctypes.c_float(-1.0)), "base")
    assert t(None, None, 0, 8, ctypes.c_float(10000.0)) == 0


def test_polar_pool_bytes_and_validation(sp_lib):
    lay = _lay(num_blocks=10, num_layers=3, num_kv_heads=4, block_size=16, head_dim=128)
    # regions of BS * (D/2 + 2) bytes per (block, layer, KV head)
    assert sp_lib.sp_polar_pool_bytes(ctypes.byref(lay)) == 10 * 3 * 4 * 16 * 66
    assert sp_lib.sp_polar_pool_bytes(ctypes.byref(_lay(head_dim=63))) == 0
    assert sp_lib.sp_polar_pool_bytes(ctypes.byref(_lay(block_size=6))) == 0
    fake = ctypes.c_void_p(0x1000)
    app = sp_lib.sp_polar_kv_append
    _expect(_lib.SP_EUNSUPPORTED, app(fake, fake, ctypes.byref(_lay(head_dim=63)), fake, fake,
                                      128, 64, fake, 1, 1, None), "even head_dim")
    _expect(_lib.SP_EUNSUPPORTED, app(fake, fake, ctypes.byref(_lay(block_size=6)), fake, fake,
                                      128, 64, fake, 1, 1, None), "multiple of 4")
    _expect(_lib.SP_EINVAL, app(ctypes.c_void_p(0x1008), fake, ctypes.byref(_lay()), fake, fake,
                                128, 64, fake, 1, 1, None), "16-byte aligned")
    _expect(_lib.SP_EINVAL, app(fake, fake, ctypes.byref(_lay()), fake, fake, 128, 64, None, 1,
                                1, None), "NULL")
    assert app(None, None, ctypes.byref(_lay()), None, None, 0, 0, None, 0, 1, None) == 0
    gat = sp_lib.sp_polar_kv_gather
    _expect(_lib.SP_EOOB, gat(fake, fake, fake, fake, ctypes.byref(_lay()), fake, 1, 17, 1, None),
            "needs 2 blocks")
    exp = sp_lib.sp_polar_kv_export
    _expect(_lib.SP_EOOB, exp(fake, fake, fake, fake, ctypes.byref(_lay()), fake, 1, 17, None),
            "needs 2 blocks")
    comp = sp_lib.sp_polar_compress
    _expect(_lib.SP_EINVAL, comp(fake, fake, 4, 0, 0, None), "head_dim 0")
    _expect(_lib.SP_EINVAL, comp(fake, ctypes.c_void_p(0x1001), 4, 8, 0, None), "aligned")
    assert comp(None, None, 0, 8, 0, None) == 0
    dec = sp_lib.sp_polar_paged_decode

    def call(lay, dtype=1, hq=4, max_ctx=32, mbs=2):
        return dec(fake, fake, fake, fake, ctypes.byref(lay), fake, mbs, fake, max_ctx, 3, hq,
                   0.125, -1, dtype, None, 0, None)

    _expect(_lib.SP_EUNSUPPORTED, call(_lay(), dtype=0), "bf16, f16")
    _expect(_lib.SP_EUNSUPPORTED, call(_lay(head_dim=96)), "head_dim 96")
    _expect(_lib.SP_EUNSUPPORTED, call(_lay(block_size=8), mbs=4), "block_size 8")
    _expect(_lib.SP_EUNSUPPORTED, call(_lay(block_size=24), mbs=4), "block_size 24")
    _expect(_lib.SP_EINVAL, call(_lay(), hq=3), "multiple")


def test_workspace_size_monotone(sp_lib):
    lay = _lay(num_blocks=100000, num_kv_heads=8, head_dim=128)
    sizes = [sp_lib.sp_paged_decode_workspace_size(64, 32, L, -1, ctypes.byref(lay))
             for L in (16, 512, 4096, 32768)]
    assert sizes == sorted(sizes)
    # a window bounds the split count whatever the context length
    w1 = sp_lib.sp_paged_decode_workspace_size(16, 32, 32768, 4096, ctypes.byref(lay))
    w2 = sp_lib.sp_paged_decode_workspace_size(16, 32, 8192, 4096, ctypes.byref(lay))
    assert w1 == w2 > 0


def test_flash_attention_masked_validation(sp_lib):
    """A NULL or misaligned mask, a negative stride and head dims without a kernel are
    rejected before any launch (the mask itself is f32 for every tensor dtype)."""
    def call(dtype, mask=1 << 20, sb=0, d=64):
        return sp_lib.sp_flash_attention_masked(16, 16, 16, 16, mask, sb, 0, 8, 1, 2, 8, 8, d,
                                                0.125, 0, dtype, None)
    assert call(_lib.SP_F32, mask=None) == _lib.SP_EINVAL
    assert call(_lib.SP_BF16, mask=None) == _lib.SP_EINVAL
    assert call(_lib.SP_F32, mask=(1 << 20) + 2) == _lib.SP_EINVAL
    assert call(_lib.SP_F32, sb=-1) == _lib.SP_EINVAL
    assert call(_lib.SP_BF16, d=80) == _lib.SP_EUNSUPPORTED  # 16-bit kernels: 64 / 128
    assert call(_lib.SP_F32, d=48) == _lib.SP_EUNSUPPORTED


def test_flash_attention_ex_validation(sp_lib):
    """sp_flash_attention_ex: value head dims and output dtypes checked before any launch."""
    def call(d=80, dv=80, dtype=_lib.SP_F32, out_dtype=_lib.SP_F32):
        return sp_lib.sp_flash_attention_ex(16, 16, 16, 16, None, 0, 0, 0, 1, 2, 8, 8, d, dv,
                                            0.125, 0, dtype, out_dtype, None)
    assert call(dv=82) == _lib.SP_EUNSUPPORTED        # not a multiple of 4
    assert call(dv=260) == _lib.SP_EUNSUPPORTED       # past 256
    assert call(dv=0) == _lib.SP_EINVAL
    assert call(out_dtype=7) == _lib.SP_EINVAL
    assert call(d=128, dv=64, dtype=_lib.SP_BF16) == _lib.SP_EUNSUPPORTED  # 16-bit: Dv == D
    for d in (40, 64, 80, 128, 160, 256):             # f32 head dims with kernels: no error
        assert sp_lib.sp_flash_attention_ex(0, 0, 0, 0, None, 0, 0, 0, 0, 2, 8, 8, d, d, 0.1, 0,
                                            _lib.SP_F32, _lib.SP_F32, None) == _lib.SP_OK


def test_paged_prefill_workspace_size(sp_lib):
    """Key splits are planned only while the split grid stays within one round of resident
    workgroups (512), with at least 16 key tiles per split and at most 8 splits, as fp32
    (m, l, acc) records: one 512-query chunk of 28 heads (112 workgroups) on a 32k context gets 4,
    two 128-query chunks (56 workgroups) on contexts of up to 428 blocks of 16 get 107 / 16 = 6;
    C4's shape (4 x 512 queries, 448 workgroups), a C3-sized batch and short contexts get none."""
    lay = _lib.layout(10_000, 1, 0, 4, 16, 128)
    rec = 128 + 4
    assert sp_lib.sp_paged_prefill_workspace_size(1, 512, 28, ctypes.byref(lay), 2016) == \
        1 * 512 * 28 * 4 * rec * 4
    assert sp_lib.sp_paged_prefill_workspace_size(2, 128, 28, ctypes.byref(lay), 428) == \
        2 * 128 * 28 * 6 * rec * 4
    assert sp_lib.sp_paged_prefill_workspace_size(4, 512, 28, ctypes.byref(lay), 428) == 0
    lay32 = _lib.layout(10_000, 1, 0, 8, 16, 128)
    assert sp_lib.sp_paged_prefill_workspace_size(8, 1672, 32, ctypes.byref(lay32), 105) == 0
    assert sp_lib.sp_paged_prefill_workspace_size(4, 512, 28, ctypes.byref(lay), 10) == 0
    assert sp_lib.sp_paged_prefill_workspace_size(0, 512, 28, ctypes.byref(lay), 428) == 0
    assert sp_lib.sp_paged_prefill_workspace_size(4, 512, 28, None, 428) == 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.load()


def test_ragged_paged_attention_validation(sp_lib):
    """sp_ragged_paged_attention: the group split and pointers are checked before any launch;
    the workspace holds the decode's partials (rounded up to 256 bytes) followed by the
    prefill's."""
    lay = _lib.layout(10_000, 1, 0, 4, 16, 128)

    def call(num_seqs=4, num_prefill=2, cu=1 << 20, tok=100):
        return sp_lib.sp_ragged_paged_attention(16, 16, 16, 16, ctypes.byref(lay), 16, 8, cu, 16,
                                                num_seqs, num_prefill, tok, 64, 100, 28, 0.1, -1,
                                                _lib.SP_BF16, None, 0, None)
    assert call(num_prefill=5) == _lib.SP_EINVAL
    assert call(num_prefill=-1) == _lib.SP_EINVAL
    assert call(tok=-1) == _lib.SP_EINVAL
    assert call(cu=None) == _lib.SP_EINVAL
    assert call(num_seqs=0, num_prefill=0) == _lib.SP_OK
    # both halves: the decode half's workspace is checked before anything is enqueued
    assert call() == _lib.SP_ENOSPACE
    assert "required" in sp_lib.sp_last_error().decode()
    # C4's shape: the chunks do not split, so the decode partials are all
    dec = sp_lib.sp_paged_decode_workspace_size(128, 28, 4096, -1, ctypes.byref(lay))
    assert dec > 0
    dec_al = (dec + 255) // 256 * 256
    assert sp_lib.sp_paged_prefill_workspace_size(4, 512, 28, ctypes.byref(lay), 547) == 0
    assert sp_lib.sp_ragged_attention_workspace_size(132, 4, 512, 4096, 28, -1,
                                                     ctypes.byref(lay), 547) == dec_al
    # one chunk on a 32k context splits: both regions
    pre = sp_lib.sp_paged_prefill_workspace_size(1, 512, 28, ctypes.byref(lay), 2016)
    assert pre > 0
    assert sp_lib.sp_ragged_attention_workspace_size(129, 1, 512, 4096, 28, -1,
                                                     ctypes.byref(lay), 2016) == dec_al + pre
    assert sp_lib.sp_ragged_attention_workspace_size(128, 0, 0, 4096, 28, -1, ctypes.byref(lay),
                                                     547) == dec_al
    assert sp_lib.sp_ragged_attention_workspace_size(1, 1, 512, 0, 28, -1, ctypes.byref(lay),
                                                     2016) == pre


def test_softcap_validation(sp_lib):
    """The *_softcap entry points: 0 is the namesake, > 0 runs at head_dims 256 and 512 on bf16 /
    f16 only, a negative or non-finite cap is rejected; all before anything is enqueued."""
    fake = ctypes.c_void_p(0x1000)
    d = sp_lib.sp_paged_decode_softcap

    def dec(lay, cap, dtype=1):
        return d(fake, fake, fake, fake, ctypes.byref(lay), fake, 2, fake, 32, 3, 4, 0.125, cap, -1,
                 dtype, None, 0, None)

    cap_dims = "head_dims 256 and 512"
    _expect(_lib.SP_EUNSUPPORTED, dec(_lay(head_dim=128), 50.0), cap_dims)
    _expect(_lib.SP_EUNSUPPORTED, dec(_lay(head_dim=256), 50.0, dtype=0), "head_dim 256")
    _expect(_lib.SP_EUNSUPPORTED, dec(_lay(head_dim=512), 50.0, dtype=0), "head_dim 512")
    _expect(_lib.SP_EINVAL, dec(_lay(head_dim=256), -1.0), "logit_softcap")
    _expect(_lib.SP_EINVAL, dec(_lay(head_dim=256), float("nan")), "logit_softcap")
    a = sp_lib.sp_paged_append_decode_softcap
    _expect(_lib.SP_EUNSUPPORTED,
            a(fake, fake, fake, fake, ctypes.byref(_lay()), fake, fake, 128, 64, fake, 2, fake, 32,
              3, 4, 0.125, 50.0, -1, 1, None, 0, None), cap_dims)
    v = sp_lib.sp_varlen_prefill_softcap
    _expect(_lib.SP_EUNSUPPORTED,
            v(fake, fake, fake, fake, fake, fake, 2, 16, 4, 2, 128, 0.125, 50.0, 1, -1, 1, None),
            cap_dims)
    _expect(_lib.SP_EINVAL,
            v(fake, fake, fake, fake, fake, fake, 2, 16, 4, 2, 256, 0.125, float("inf"), 1, -1, 1,
              None), "logit_softcap")
    p = sp_lib.sp_paged_prefill_softcap
    _expect(_lib.SP_EUNSUPPORTED,
            p(fake, fake, fake, fake, ctypes.byref(_lay()), fake, 2, fake, fake, 2, 16, 4, 0.125,
              50.0, -1, 1, None, 0, None), cap_dims)
    r = sp_lib.sp_ragged_paged_attention_softcap
    _expect(_lib.SP_EUNSUPPORTED,
            r(fake, fake, fake, fake, ctypes.byref(_lay()), fake, 2, fake, fake, 3, 1, 16, 16, 32,
              4, 0.125, 50.0, -1, 1, None, 0, None), cap_dims)
