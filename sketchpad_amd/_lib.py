"""ctypes binding of the C ABI in include/sketchpad_attn.h.

The shared library is built in-tree by ``python -m sketchpad_amd.build`` (or
``__graft_entry__.build()``). Loading fails loudly when it is missing: there is no CPU or
PyTorch fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libsketchpad_attn.so"
HEADER = Path(__file__).resolve().parent.parent / "include" / "sketchpad_attn.h"

SP_OK, SP_EINVAL, SP_EUNSUPPORTED, SP_EHIP, SP_EOOB, SP_ENOSPACE = range(6)
SP_F32, SP_BF16, SP_F16 = 0, 1, 2
SP_CAUSAL_NONE, SP_CAUSAL_BOTTOM_RIGHT, SP_CAUSAL_TOP_LEFT = 0, 1, 2

STATUS_NAMES = {
    SP_OK: "SP_OK",
    SP_EINVAL: "SP_EINVAL",
    SP_EUNSUPPORTED: "SP_EUNSUPPORTED",
    SP_EHIP: "SP_EHIP",
    SP_EOOB: "SP_EOOB",
    SP_ENOSPACE: "SP_ENOSPACE",
}


class SketchpadError(RuntimeError):
    """A nonzero sp_status, with the library's message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


class CacheLayout(ctypes.Structure):
    """sp_cache_layout: one layer's view of a [num_blocks, num_layers, Hkv, BS, D] pool."""

    _fields_ = [
        ("num_blocks", c_int32),
        ("num_layers", c_int32),
        ("layer", c_int32),
        ("num_kv_heads", c_int32),
        ("block_size", c_int32),
        ("head_dim", c_int32),
    ]

    def __repr__(self) -> str:
        return ("CacheLayout(num_blocks={0.num_blocks}, num_layers={0.num_layers}, "
                "layer={0.layer}, num_kv_heads={0.num_kv_heads}, block_size={0.block_size}, "
                "head_dim={0.head_dim})").format(self)


_SIGNATURES = {
    "sp_version": (c_int32, []),
    "sp_last_error": (ctypes.c_char_p, []),
    "sp_kv_append": (c_int32, [c_void_p, c_void_p, POINTER(CacheLayout), c_void_p, c_void_p,
                               c_int64, c_int64, c_void_p, c_int32, c_int32, c_void_p]),
    "sp_kv_gather": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, POINTER(CacheLayout),
                               c_void_p, c_int32, c_int32, c_int32, c_void_p]),
    "sp_rope_tables": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_float]),
    "sp_rope_kv_append": (c_int32, [c_void_p, c_void_p, POINTER(CacheLayout), c_void_p, c_void_p,
                                    c_int64, c_int64, c_void_p, c_int64, c_int64, c_int32,
                                    c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int32,
                                    c_int32, c_void_p]),
    "sp_paged_decode_workspace_size": (c_size_t, [c_int32, c_int32, c_int32, c_int32,
                                                  POINTER(CacheLayout)]),
    "sp_paged_decode": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, POINTER(CacheLayout),
                                  c_void_p, c_int32, c_void_p, c_int32, c_int32, c_int32,
                                  c_float, c_int32, c_int32, c_void_p, c_size_t, c_void_p]),
    "sp_paged_append_decode": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p,
                                         POINTER(CacheLayout), c_void_p, c_void_p, c_int64,
                                         c_int64, c_void_p, c_int32, c_void_p, c_int32, c_int32,
                                         c_int32, c_float, c_int32, c_int32, c_void_p, c_size_t,
                                         c_void_p]),
    "sp_paged_decode_noalloc": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p,
                                          POINTER(CacheLayout), c_void_p, c_int32, c_void_p,
                                          c_int32, c_int32, c_int32, c_float, c_int32, c_int32,
                                          c_void_p]),
    "sp_ragged_attention_workspace_size": (c_size_t, [c_int32, c_int32, c_int32, c_int32,
                                                      c_int32, c_int32, POINTER(CacheLayout),
                                                      c_int32]),
    "sp_ragged_paged_attention": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p,
                                            POINTER(CacheLayout), c_void_p, c_int32, c_void_p,
                                            c_void_p, c_int32, c_int32, c_int32, c_int32,
                                            c_int32, c_int32, c_float, c_int32, c_int32,
                                            c_void_p, c_size_t, c_void_p]),
    "sp_varlen_prefill": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                    c_int32, c_int32, c_int32, c_int32, c_int32, c_float,
                                    c_int32, c_int32, c_int32, c_void_p]),
    "sp_paged_prefill_workspace_size": (c_size_t, [c_int32, c_int32, c_int32,
                                                   POINTER(CacheLayout), c_int32]),
    "sp_paged_prefill": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, POINTER(CacheLayout),
                                   c_void_p, c_int32, c_void_p, c_void_p, c_int32, c_int32,
                                   c_int32, c_float, c_int32, c_int32, c_void_p, c_size_t,
                                   c_void_p]),
    # the *_softcap entry points: the namesake's arguments with logit_softcap after scale
    "sp_paged_decode_softcap": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p,
                                          POINTER(CacheLayout), c_void_p, c_int32, c_void_p,
                                          c_int32, c_int32, c_int32, c_float, c_float, c_int32,
                                          c_int32, c_void_p, c_size_t, c_void_p]),
    "sp_paged_append_decode_softcap": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                 POINTER(CacheLayout), c_void_p, c_void_p,
                                                 c_int64, c_int64, c_void_p, c_int32, c_void_p,
                                                 c_int32, c_int32, c_int32, c_float, c_float,
                                                 c_int32, c_int32, c_void_p, c_size_t,
                                                 c_void_p]),
    "sp_varlen_prefill_softcap": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                            c_void_p, c_int32, c_int32, c_int32, c_int32,
                                            c_int32, c_float, c_float, c_int32, c_int32, c_int32,
                                            c_void_p]),
    "sp_paged_prefill_softcap": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p,
                                           POINTER(CacheLayout), c_void_p, c_int32, c_void_p,
                                           c_void_p, c_int32, c_int32, c_int32, c_float, c_float,
                                           c_int32, c_int32, c_void_p, c_size_t, c_void_p]),
    "sp_ragged_paged_attention_softcap": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                    POINTER(CacheLayout), c_void_p, c_int32,
                                                    c_void_p, c_void_p, c_int32, c_int32,
                                                    c_int32, c_int32, c_int32, c_int32, c_float,
                                                    c_float, c_int32, c_int32, c_void_p,
                                                    c_size_t, c_void_p]),
    "sp_flash_attention": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
                                     c_int32, c_int32, c_int32, c_float, c_int32, c_int32,
                                     c_void_p]),
    "sp_flash_attention_ex": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_int64, c_int64, c_int64, c_int32, c_int32, c_int32,
                                        c_int32, c_int32, c_int32, c_float, c_int32, c_int32,
                                        c_int32, c_void_p]),
    "sp_qjl_record_bytes": (c_int64, [c_int32]),
    "sp_qjl_projection": (c_int32, [c_void_p, c_int32, c_int32]),
    "sp_qjl_compress": (c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_int32,
                                  c_int32, c_void_p]),
    "sp_qjl_decompress": (c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_int32,
                                    c_int32, c_void_p]),
    "sp_flash_attention_masked": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                            c_int64, c_int64, c_int64, c_int32, c_int32, c_int32,
                                            c_int32, c_int32, c_float, c_int32, c_int32,
                                            c_void_p]),
    "sp_polar_record_bytes": (c_int64, [c_int32]),
    "sp_polar_pool_bytes": (c_size_t, [POINTER(CacheLayout)]),
    "sp_polar_compress": (c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_int32, c_void_p]),
    "sp_polar_decompress": (c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_int32, c_void_p]),
    "sp_polar_kv_append": (c_int32, [c_void_p, c_void_p, POINTER(CacheLayout), c_void_p,
                                     c_void_p, c_int64, c_int64, c_void_p, c_int32, c_int32,
                                     c_void_p]),
    "sp_polar_kv_gather": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p,
                                     POINTER(CacheLayout), c_void_p, c_int32, c_int32, c_int32,
                                     c_void_p]),
    "sp_polar_kv_export": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p,
                                     POINTER(CacheLayout), c_void_p, c_int32, c_int32, c_void_p]),
    "sp_polar_paged_decode": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p,
                                        POINTER(CacheLayout), c_void_p, c_int32, c_void_p,
                                        c_int32, c_int32, c_int32, c_float, c_int32, c_int32,
                                        c_void_p, c_size_t, c_void_p]),
    "sp_linear_workspace_size": (c_size_t, [c_int64, c_int64, c_int64]),
    "sp_linear": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64,
                            c_int32, c_void_p, c_size_t, c_void_p]),
    "sp_linear_weight_nk": (c_int32, [c_void_p, c_void_p, c_int64, c_int64, c_int32, c_void_p]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libsketchpad_attn.so (once) and bind every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m sketchpad_amd.build` "
            "(there is no fallback path)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(code: int) -> None:
    if code != SP_OK:
        raise SketchpadError(code, load().sp_last_error().decode())


def layout(num_blocks: int, num_layers: int, layer: int, num_kv_heads: int, block_size: int,
           head_dim: int) -> CacheLayout:
    return CacheLayout(num_blocks, num_layers, layer, num_kv_heads, block_size, head_dim)


# ---------------------------------------------------------------------------------------------
# torch-tensor helpers: torch only supplies device memory and the stream.
# ---------------------------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def sp_dtype(t) -> int:
    torch = _torch()
    m = {torch.float32: SP_F32, torch.bfloat16: SP_BF16, torch.float16: SP_F16}
    if t.dtype not in m:
        raise SketchpadError(SP_EUNSUPPORTED, f"dtype {t.dtype} has no kernel")
    return m[t.dtype]


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int | None:
    if stream is not None:
        return stream
    torch = _torch()
    return torch.cuda.current_stream().cuda_stream


def kv_append(k_pool, v_pool, lay: CacheLayout, k_new, v_new, slot_mapping, *,
              token_stride: int | None = None, head_stride: int | None = None,
              stream=None) -> None:
    """sp_kv_append. k_new/v_new default to token-major [T, Hkv, D] contiguous tensors."""
    if token_stride is None:
        token_stride = k_new.stride(0)
    if head_stride is None:
        head_stride = k_new.stride(1)
    assert slot_mapping.dtype == _torch().int32
    check(load().sp_kv_append(_ptr(k_pool), _ptr(v_pool), ctypes.byref(lay), _ptr(k_new),
                              _ptr(v_new), token_stride, head_stride, _ptr(slot_mapping),
                              slot_mapping.numel(), sp_dtype(k_pool), _stream(stream)))


def rope_tables(rows: int, head_dim: int, base: float = 10000.0):
    """sp_rope_tables: host fp32 (cos, sin) numpy arrays of shape [rows, head_dim // 2]."""
    import numpy as np
    cos = np.zeros((max(rows, 0), head_dim // 2), dtype=np.float32)
    sin = np.zeros_like(cos)
    check(load().sp_rope_tables(cos.ctypes.data, sin.ctypes.data, rows, head_dim, base))
    return cos, sin


def rope_kv_append(k_pool, v_pool, lay: CacheLayout, k_new, v_new, positions, slot_mapping,
                   cos_table, sin_table, *, q=None, token_stride: int | None = None,
                   head_stride: int | None = None, stream=None) -> None:
    """sp_rope_kv_append: rotate K (and Q in place, when given) by the tables' angles at each
    token's position and append K/V through the slot mapping. k_new/v_new default to
    token-major [T, Hkv, D]; q is [T, Hq, D]; cos/sin tables are device fp32 [rows, D/2]."""
    torch = _torch()
    if token_stride is None:
        token_stride = k_new.stride(0)
    if head_stride is None:
        head_stride = k_new.stride(1)
    assert slot_mapping.dtype == torch.int32 and positions.dtype == torch.int32
    assert cos_table.dtype == torch.float32 and sin_table.dtype == torch.float32
    qp, qts, qhs, hq = None, 0, 0, 0
    if q is not None:
        qp, qts, qhs, hq = _ptr(q), q.stride(0), q.stride(1), q.shape[1]
    check(load().sp_rope_kv_append(_ptr(k_pool), _ptr(v_pool), ctypes.byref(lay), _ptr(k_new),
                                   _ptr(v_new), token_stride, head_stride, qp, qts, qhs, hq,
                                   _ptr(positions), _ptr(slot_mapping), slot_mapping.numel(),
                                   _ptr(cos_table), _ptr(sin_table), cos_table.shape[0],
                                   sp_dtype(k_pool), _stream(stream)))


def kv_gather(k_out, v_out, k_pool, v_pool, lay: CacheLayout, block_table, seq_len: int, *,
              stream=None) -> None:
    """sp_kv_gather into [Hkv, seq_len, D] tensors."""
    check(load().sp_kv_gather(_ptr(k_out), _ptr(v_out), _ptr(k_pool), _ptr(v_pool),
                              ctypes.byref(lay), _ptr(block_table), block_table.numel(), seq_len,
                              sp_dtype(k_pool), _stream(stream)))


def paged_decode_workspace_size(num_seqs: int, num_q_heads: int, max_context_len: int,
                                window_left: int, lay: CacheLayout) -> int:
    return int(load().sp_paged_decode_workspace_size(num_seqs, num_q_heads, max_context_len,
                                                     window_left, ctypes.byref(lay)))


def paged_append_decode(out, q, k_pool, v_pool, lay: CacheLayout, k_new, v_new, block_tables,
                        context_lens, max_context_len: int, scale: float, *, window_left: int = -1,
                        workspace=None, softcap: float = 0.0, stream=None) -> None:
    """sp_paged_append_decode (sp_paged_append_decode_softcap when softcap != 0). k_new/v_new
    are [num_seqs, Hkv, D] (any strides the C call takes); the rest as paged_decode."""
    num_seqs, hq = q.shape[0], q.shape[1]
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    head = (_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), ctypes.byref(lay), _ptr(k_new),
            _ptr(v_new), k_new.stride(0), k_new.stride(1), _ptr(block_tables),
            block_tables.shape[1], _ptr(context_lens), max_context_len, num_seqs, hq, scale)
    tail = (window_left, sp_dtype(q), _ptr(workspace), ws_bytes, _stream(stream))
    if softcap:
        check(load().sp_paged_append_decode_softcap(*head, softcap, *tail))
    else:
        check(load().sp_paged_append_decode(*head, *tail))


def paged_decode(out, q, k_pool, v_pool, lay: CacheLayout, block_tables, context_lens,
                 max_context_len: int, scale: float, *, window_left: int = -1, workspace=None,
                 softcap: float = 0.0, stream=None) -> None:
    """sp_paged_decode (sp_paged_decode_softcap when softcap != 0). q/out are
    [num_seqs, Hq, D]; block_tables [num_seqs, max_blocks]."""
    num_seqs, hq = q.shape[0], q.shape[1]
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    head = (_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), ctypes.byref(lay),
            _ptr(block_tables), block_tables.shape[1], _ptr(context_lens), max_context_len,
            num_seqs, hq, scale)
    tail = (window_left, sp_dtype(q), _ptr(workspace), ws_bytes, _stream(stream))
    if softcap:
        check(load().sp_paged_decode_softcap(*head, softcap, *tail))
    else:
        check(load().sp_paged_decode(*head, *tail))


def paged_decode_noalloc(out, q, k_pool, v_pool, lay: CacheLayout, block_tables, context_lens,
                         max_context_len: int, scale: float, *, window_left: int = -1,
                         stream=None) -> None:
    """sp_paged_decode_noalloc: sp_paged_decode with the split partials in the library's own
    per-GPU scratch (no workspace argument, no allocation)."""
    num_seqs, hq = q.shape[0], q.shape[1]
    check(load().sp_paged_decode_noalloc(_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool),
                                         ctypes.byref(lay), _ptr(block_tables),
                                         block_tables.shape[1], _ptr(context_lens),
                                         max_context_len, num_seqs, hq, scale, window_left,
                                         sp_dtype(q), _stream(stream)))


def ragged_paged_attention(out, q, k_pool, v_pool, lay: CacheLayout, block_tables, cu_seqlens_q,
                           context_lens, *, num_prefill_seqs: int, num_prefill_tokens: int,
                           prefill_max_seqlen_q: int, decode_max_context_len: int, scale: float,
                           window_left: int = -1, workspace=None, softcap: float = 0.0,
                           stream=None) -> None:
    """sp_ragged_paged_attention (sp_ragged_paged_attention_softcap when softcap != 0): one mixed
    batch, chunks [0, num_prefill_seqs) first, then one token per decode sequence; q/out
    [total_q, Hq, D]."""
    hq = q.shape[1]
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    head = (_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), ctypes.byref(lay), _ptr(block_tables),
            block_tables.shape[1], _ptr(cu_seqlens_q), _ptr(context_lens), context_lens.numel(),
            num_prefill_seqs, num_prefill_tokens, prefill_max_seqlen_q, decode_max_context_len,
            hq, scale)
    tail = (window_left, sp_dtype(q), _ptr(workspace), ws_bytes, _stream(stream))
    if softcap:
        check(load().sp_ragged_paged_attention_softcap(*head, softcap, *tail))
    else:
        check(load().sp_ragged_paged_attention(*head, *tail))


def alloc_ragged_workspace(num_seqs: int, num_prefill_seqs: int, prefill_max_seqlen_q: int,
                           decode_max_context_len: int, num_q_heads: int, lay: CacheLayout,
                           max_blocks_per_seq: int, window_left: int = -1, device="cuda"):
    """A workspace of sp_ragged_attention_workspace_size() bytes (None when none is needed)."""
    torch = _torch()
    n = int(load().sp_ragged_attention_workspace_size(num_seqs, num_prefill_seqs,
                                                      prefill_max_seqlen_q,
                                                      decode_max_context_len, num_q_heads,
                                                      window_left, ctypes.byref(lay),
                                                      max_blocks_per_seq))
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


def alloc_decode_workspace(num_seqs: int, num_q_heads: int, max_context_len: int,
                           window_left: int, lay: CacheLayout, device="cuda"):
    """Allocate a decode workspace of sp_paged_decode_workspace_size() bytes."""
    torch = _torch()
    n = paged_decode_workspace_size(num_seqs, num_q_heads, max_context_len, window_left, lay)
    return torch.empty(max(n, 256), dtype=torch.uint8, device=device)


def varlen_prefill(out, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int, scale: float, *,
                   causal: int = SP_CAUSAL_BOTTOM_RIGHT, window_left: int = -1,
                   softcap: float = 0.0, stream=None) -> None:
    """sp_varlen_prefill (sp_varlen_prefill_softcap when softcap != 0). q/out [total_q, Hq, D],
    k/v [total_k, Hkv, D] contiguous."""
    head = (_ptr(out), _ptr(q), _ptr(k), _ptr(v), _ptr(cu_seqlens_q), _ptr(cu_seqlens_k),
            cu_seqlens_q.numel() - 1, max_seqlen_q, q.shape[1], k.shape[1], q.shape[2], scale)
    tail = (causal, window_left, sp_dtype(q), _stream(stream))
    if softcap:
        check(load().sp_varlen_prefill_softcap(*head, softcap, *tail))
    else:
        check(load().sp_varlen_prefill(*head, *tail))


def paged_prefill_workspace_size(num_seqs: int, max_seqlen_q: int, num_q_heads: int,
                                 lay: CacheLayout, max_blocks_per_seq: int) -> int:
    return int(load().sp_paged_prefill_workspace_size(num_seqs, max_seqlen_q, num_q_heads,
                                                      ctypes.byref(lay), max_blocks_per_seq))


def alloc_paged_prefill_workspace(num_seqs: int, max_seqlen_q: int, num_q_heads: int,
                                  lay: CacheLayout, max_blocks_per_seq: int, device="cuda"):
    """A workspace of sp_paged_prefill_workspace_size() bytes (None when no split is planned)."""
    n = paged_prefill_workspace_size(num_seqs, max_seqlen_q, num_q_heads, lay, max_blocks_per_seq)
    return _torch().empty(n, dtype=_torch().uint8, device=device) if n > 0 else None


def paged_prefill(out, q, k_pool, v_pool, lay: CacheLayout, block_tables, cu_seqlens_q,
                  context_lens, max_seqlen_q: int, scale: float, *, window_left: int = -1,
                  workspace=None, softcap: float = 0.0, stream=None) -> None:
    """sp_paged_prefill (sp_paged_prefill_softcap when softcap != 0). q/out [total_q, Hq, D];
    the new tokens are already in the pools. workspace: optional device tensor for the
    split-key partials (None: no split)."""
    ws_ptr = _ptr(workspace) if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    head = (_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), ctypes.byref(lay),
            _ptr(block_tables), block_tables.shape[1], _ptr(cu_seqlens_q), _ptr(context_lens),
            cu_seqlens_q.numel() - 1, max_seqlen_q, q.shape[1], scale)
    tail = (window_left, sp_dtype(q), ws_ptr, ws_bytes, _stream(stream))
    if softcap:
        check(load().sp_paged_prefill_softcap(*head, softcap, *tail))
    else:
        check(load().sp_paged_prefill(*head, *tail))


def flash_attention_masked(out, q, k, v, mask, scale: float, *, causal: bool = False,
                           stream=None) -> None:
    """sp_flash_attention_masked on f32 [B, H, S, D] tensors; mask: an f32 tensor that expands
    to [B, H, Sq, Sk] (its strides are passed, so broadcast views work; last stride 1)."""
    b, h, sq, d = q.shape
    sk = k.shape[2]
    m = mask.expand(b, h, sq, sk)
    if sk > 1 and m.stride(3) != 1:
        raise ValueError("mask: the key dimension must be contiguous")
    check(load().sp_flash_attention_masked(_ptr(out), _ptr(q), _ptr(k), _ptr(v), _ptr(m),
                                           m.stride(0), m.stride(1), m.stride(2), b, h, sq, sk,
                                           d, scale, int(bool(causal)), sp_dtype(q),
                                           _stream(stream)))


def flash_attention(out, q, k, v, scale: float, *, causal: bool = False, stream=None) -> None:
    """sp_flash_attention on [B, H, S, D] tensors."""
    b, h, sq, d = q.shape
    check(load().sp_flash_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), b, h, sq, k.shape[2],
                                    d, scale, int(bool(causal)), sp_dtype(q), _stream(stream)))


def flash_attention_ex(out, q, k, v, scale: float, *, mask=None, causal: bool = False,
                       stream=None) -> None:
    """sp_flash_attention_ex: q, k [B, H, S, D], v [B, H, Sk, Dv], out [B, H, Sq, Dv] of any
    supported dtype (FlashAttentionOptions.out_dtype), optional f32 additive mask that expands to
    [B, H, Sq, Sk] (last stride 1)."""
    b, h, sq, d = q.shape
    sk, dv = v.shape[2], v.shape[3]
    mp, ms = None, (0, 0, 0)
    if mask is not None:
        m = mask.expand(b, h, sq, sk)
        if sk > 1 and m.stride(3) != 1:
            raise ValueError("mask: the key dimension must be contiguous")
        mp, ms = _ptr(m), (m.stride(0), m.stride(1), m.stride(2))
    check(load().sp_flash_attention_ex(_ptr(out), _ptr(q), _ptr(k), _ptr(v), mp, *ms, b, h, sq,
                                       sk, d, dv, scale, int(bool(causal)), sp_dtype(q),
                                       sp_dtype(out), _stream(stream)))


# ---------------------------------------------------------------------------------------------
# PolarQuant compressed paged cache (KvQuantMethod::PolarQuant, kv_cache.rs:437-532)
# ---------------------------------------------------------------------------------------------

def polar_record_bytes(head_dim: int) -> int:
    """sp_polar_record_bytes: 2 + ceil(head_dim / 2)."""
    return int(load().sp_polar_record_bytes(head_dim))


def polar_pool_bytes(lay: CacheLayout) -> int:
    """sp_polar_pool_bytes: bytes of one paged PolarQuant pool (K or V) for this layout."""
    n = int(load().sp_polar_pool_bytes(ctypes.byref(lay)))
    if n == 0:
        raise SketchpadError(SP_EUNSUPPORTED, load().sp_last_error().decode())
    return n


def alloc_polar_pools(lay: CacheLayout, device="cuda"):
    """Zeroed uint8 K and V PolarQuant pools for this layout."""
    torch = _torch()
    n = polar_pool_bytes(lay)
    return (torch.zeros(n, dtype=torch.uint8, device=device),
            torch.zeros(n, dtype=torch.uint8, device=device))


def polar_compress(records, x, *, stream=None) -> None:
    """sp_polar_compress: x [..., D] contiguous -> records [..., record_bytes] uint8."""
    d = x.shape[-1]
    check(load().sp_polar_compress(_ptr(records), _ptr(x), x.numel() // d, d, sp_dtype(x),
                                   _stream(stream)))


def polar_decompress(out, records, *, stream=None) -> None:
    """sp_polar_decompress: records [..., record_bytes] -> out [..., D] (its dtype)."""
    d = out.shape[-1]
    check(load().sp_polar_decompress(_ptr(out), _ptr(records), out.numel() // d, d,
                                     sp_dtype(out), _stream(stream)))


def polar_kv_append(k_pool, v_pool, lay: CacheLayout, k_new, v_new, slot_mapping, *,
                    token_stride: int | None = None, head_stride: int | None = None,
                    stream=None) -> None:
    """sp_polar_kv_append. k_new/v_new default to token-major [T, Hkv, D] contiguous tensors."""
    ts = token_stride if token_stride is not None else lay.num_kv_heads * lay.head_dim
    hs = head_stride if head_stride is not None else lay.head_dim
    check(load().sp_polar_kv_append(_ptr(k_pool), _ptr(v_pool), ctypes.byref(lay),
                                    _ptr(k_new), _ptr(v_new), ts, hs, _ptr(slot_mapping),
                                    slot_mapping.numel(), sp_dtype(k_new), _stream(stream)))


def polar_kv_gather(k_out, v_out, k_pool, v_pool, lay: CacheLayout, block_table, seq_len: int, *,
                    stream=None) -> None:
    """sp_polar_kv_gather: decompressed [Hkv, seq_len, D] in k_out's dtype."""
    check(load().sp_polar_kv_gather(_ptr(k_out), _ptr(v_out), _ptr(k_pool), _ptr(v_pool),
                                    ctypes.byref(lay), _ptr(block_table), block_table.numel(),
                                    seq_len, sp_dtype(k_out), _stream(stream)))


def polar_kv_export(k_rec, v_rec, k_pool, v_pool, lay: CacheLayout, block_table, seq_len: int, *,
                    stream=None) -> None:
    """sp_polar_kv_export: records [Hkv, seq_len, record_bytes] uint8."""
    check(load().sp_polar_kv_export(_ptr(k_rec), _ptr(v_rec), _ptr(k_pool), _ptr(v_pool),
                                    ctypes.byref(lay), _ptr(block_table), block_table.numel(),
                                    seq_len, _stream(stream)))


def polar_paged_decode(out, q, k_pool, v_pool, lay: CacheLayout, block_tables, context_lens,
                       max_context_len: int, scale: float, *, window_left: int = -1,
                       workspace=None, stream=None) -> None:
    """sp_polar_paged_decode (workspace as for paged_decode)."""
    num_seqs, hq = q.shape[0], q.shape[1]
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(load().sp_polar_paged_decode(_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool),
                                       ctypes.byref(lay), _ptr(block_tables),
                                       block_tables.shape[1], _ptr(context_lens),
                                       max_context_len, num_seqs, hq, scale, window_left,
                                       sp_dtype(q), _ptr(workspace), ws_bytes, _stream(stream)))


# ---------------------------------------------------------------------------------------------
# Projections (burn's nn::Linear in MultiHeadAttention, transformer.rs:196-208, :249-253)
# ---------------------------------------------------------------------------------------------

def linear_workspace_size(m: int, k: int, n: int) -> int:
    """Bytes of split-K partials sp_linear uses for this shape (0: it does not split)."""
    return int(load().sp_linear_workspace_size(m, k, n))


def alloc_linear_workspace(shapes, device="cuda"):
    """A device workspace large enough for every (M, K, N) in shapes (at least 16 bytes)."""
    torch = _torch()
    need = max([16] + [linear_workspace_size(*s) for s in shapes])
    return torch.empty(need, dtype=torch.uint8, device=device)


def linear(y, x, w, bias=None, *, workspace=None, stream=None) -> None:
    """sp_linear: y[M, N] = x[M, K] @ w[N, K]^T (+ bias[N]); w is [out, in] (PyTorch layout);
    contiguous row-major tensors."""
    k = x.shape[-1]
    m = x.numel() // k
    n = w.shape[0]
    if w.numel() != n * k or y.numel() != m * n:
        raise ValueError(f"linear: x {tuple(x.shape)}, w {tuple(w.shape)}, y {tuple(y.shape)}")
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(load().sp_linear(_ptr(y), _ptr(x), _ptr(w), _ptr(bias), m, k, n, sp_dtype(x),
                           _ptr(workspace), ws_bytes, _stream(stream)))


def linear_weight_nk(w_kn, *, stream=None):
    """sp_linear_weight_nk: burn's [in, out] weight -> a new [out, in] tensor."""
    torch = _torch()
    k, n = w_kn.shape
    dst = torch.empty(n, k, dtype=w_kn.dtype, device=w_kn.device)
    check(load().sp_linear_weight_nk(_ptr(dst), _ptr(w_kn), k, n, sp_dtype(w_kn),
                                     _stream(stream)))
    return dst


# ---------------------------------------------------------------------------------------------
# QJL codec (KvQuantMethod::QJL, kv_cache.rs:300-324, :534-617)
# ---------------------------------------------------------------------------------------------
def qjl_record_bytes(proj_dim: int) -> int:
    return int(load().sp_qjl_record_bytes(proj_dim))


def qjl_projection(proj_dim: int, head_dim: int, device="cuda"):
    """The reference's fixed QJL projection R [proj_dim, head_dim] (sp_qjl_projection on the
    host), as a float32 tensor on `device`."""
    torch = _torch()
    host = torch.empty(proj_dim, head_dim, dtype=torch.float32)
    check(load().sp_qjl_projection(ctypes.c_void_p(host.data_ptr()), proj_dim, head_dim))
    return host.to(device)


def qjl_compress(records, x, proj, stream=None) -> None:
    """sp_qjl_compress: x [..., head_dim] -> uint8 records [..., qjl_record_bytes(P)]."""
    d = x.shape[-1]
    check(load().sp_qjl_compress(_ptr(records), _ptr(x), x.numel() // d, d, _ptr(proj),
                                 proj.shape[0], sp_dtype(x), _stream(stream)))


def qjl_decompress(out, records, proj, stream=None) -> None:
    """sp_qjl_decompress: uint8 records -> out [..., head_dim] (out's dtype)."""
    d = out.shape[-1]
    check(load().sp_qjl_decompress(_ptr(out), _ptr(records), out.numel() // d, d, _ptr(proj),
                                   proj.shape[0], sp_dtype(out), _stream(stream)))
