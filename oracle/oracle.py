"""ctypes front end of the C oracle (oracle/sp_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() (as the checker) and
bench.py's cpu_baseline leg. The product never imports it. Each function names the reference
item it restates; sp_oracle.h lists the check that pins it.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

import numpy as np

# SP_ORACLE_LIB: another build of the same source (oracle/sanitize.sh loads its instrumented one)
LIB_PATH = Path(os.environ.get("SP_ORACLE_LIB") or
                Path(__file__).resolve().parent / "build" / "libsp_oracle.so")

F32, BF16, F16 = 0, 1, 2


class Layout(ctypes.Structure):
    _fields_ = [("num_blocks", c_int32), ("num_layers", c_int32), ("layer", c_int32),
                ("num_kv_heads", c_int32), ("block_size", c_int32), ("head_dim", c_int32)]


_SIG = {
    "spo_get_block": (c_int64, [c_void_p, c_int64, c_int64, c_int]),
    "spo_get_slot": (c_int64, [c_int64, c_int]),
    "spo_needs_new_block": (c_int, [c_int64, c_int]),
    "spo_blocks_needed": (c_int64, [c_int64, c_int]),
    "spo_blocks_from_memory_budget": (c_int64, [c_int64, c_int64, c_int64, c_int64, c_int64]),
    "spo_slot_mapping": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int, c_void_p]),
    "spo_store_kv": (c_int, [c_void_p, c_void_p, POINTER(Layout), c_void_p, c_int64, c_void_p,
                             c_void_p, c_int64, c_int64, c_int]),
    "spo_gather_kv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, POINTER(Layout), c_void_p,
                              c_int64, c_int64, c_int]),
    "spo_rope_caches": (None, [c_void_p, c_void_p, c_int64, c_int64, c_float]),
    "spo_rope_apply": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p,
                               c_void_p, c_void_p, c_int64]),
    "spo_f32_to_f16_bits": (ctypes.c_uint16, [c_float]),
    "spo_f16_bits_to_f32": (c_float, [ctypes.c_uint16]),
    "spo_polar_record_bytes": (c_int64, [c_int64]),
    "spo_polar_compress": (None, [c_void_p, c_void_p, c_int64, c_int64]),
    "spo_polar_decompress": (None, [c_void_p, c_void_p, c_int64, c_int64]),
    "spo_polar_compression_ratio": (c_double, [c_int64]),
    "spo_qjl_lcg_normal": (None, [c_void_p, c_int64, c_float]),
    "spo_qjl_projection": (None, [c_void_p, c_int64, c_int64]),
    "spo_qjl_record_bytes": (c_int64, [c_int64]),
    "spo_qjl_compress": (None, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64]),
    "spo_qjl_decompress": (None, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64]),
    "spo_qjl_compression_ratio": (c_double, [c_int64, c_int64]),
    "spo_causal_mask": (None, [c_int64, c_void_p]),
    "spo_prefill_causal_mask": (None, [c_int64, c_int64, c_void_p]),
    "spo_sliding_window_mask": (None, [c_int64, c_int64, c_void_p]),
    "spo_sliding_window_prefill_mask": (None, [c_int64, c_int64, c_int64, c_void_p]),
    "spo_attention_f64_v": (None, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64,
                                   c_void_p, c_int64, c_int64, c_int32, c_int64, c_int64, c_int32,
                                   c_int32, c_int32, c_double, c_void_p, c_int32, c_int64,
                                   c_int64, c_int32, c_void_p]),
    "spo_attention_f64_cap": (None, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64,
                                     c_void_p, c_int64, c_int64, c_int32, c_int64, c_int64,
                                     c_int32, c_int32, c_int32, c_double, c_double, c_void_p,
                                     c_int32, c_int64, c_int64, c_int32, c_void_p]),
    "spo_attention_f64": (None, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                 c_int64, c_int64, c_int64, c_int, c_int, c_int, c_double,
                                 c_void_p, c_int, c_int64, c_int64, c_int, c_void_p]),
    "spo_attention_f32_refops": (None, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                        c_int64, c_int64, c_int64, c_int, c_int, c_int, c_float,
                                        c_void_p, c_int, c_int64, c_int64, c_int, c_void_p]),
    "spo_cpu_decode_baseline": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, POINTER(Layout), c_void_p, c_int64, c_void_p,
                                       c_int64, c_int, c_float, c_int64, c_int]),
    "spo_cpu_prefill_baseline": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_int64, c_int, c_int, c_int, c_float, c_int]),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run oracle/build.sh")
        l = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIG.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(c_void_p)


def _c(a, dtype=None):
    return np.ascontiguousarray(a if dtype is None else np.asarray(a, dtype=dtype))


def _dtype_code(a: np.ndarray, dtype: int | None) -> int:
    if dtype is not None:
        return dtype
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.uint16:
        return BF16
    raise TypeError(f"oracle: unsupported array dtype {a.dtype}")


def make_layout(num_blocks, num_layers, layer, num_kv_heads, block_size, head_dim) -> Layout:
    return Layout(num_blocks, num_layers, layer, num_kv_heads, block_size, head_dim)


# --- BlockTable arithmetic (paged_attention.rs:124-137) ---------------------------------------

def get_block(table, pos: int, block_size: int):
    t = _c(table, np.int32)
    r = lib().spo_get_block(_p(t), len(t), pos, block_size)
    return None if r < 0 else int(r)


def get_slot(pos: int, block_size: int) -> int:
    return int(lib().spo_get_slot(pos, block_size))


def needs_new_block(seq_len: int, block_size: int) -> bool:
    return bool(lib().spo_needs_new_block(seq_len, block_size))


def blocks_needed(new_len: int, block_size: int) -> int:
    return int(lib().spo_blocks_needed(new_len, block_size))


def blocks_from_memory_budget(memory_bytes, num_kv_heads, head_dim, num_layers, block_size):
    return int(lib().spo_blocks_from_memory_budget(memory_bytes, num_kv_heads, head_dim,
                                                   num_layers, block_size))


def slot_mapping(table, start_pos: int, count: int, block_size: int) -> np.ndarray | None:
    t = _c(table, np.int32)
    out = np.empty(count, dtype=np.int32)
    rc = lib().spo_slot_mapping(_p(t), len(t), start_pos, count, block_size, _p(out))
    return None if rc else out


# --- store_kv / gather_kv (paged_attention.rs:230-378) ----------------------------------------

def store_kv(k_pool: np.ndarray, v_pool: np.ndarray, lay: Layout, table, k: np.ndarray,
             v: np.ndarray, start_pos: int) -> int:
    """In place on the pools. k, v are [Hkv, S, D] (the reference's head-major layout)."""
    assert k_pool.flags.c_contiguous and v_pool.flags.c_contiguous
    t = _c(table, np.int32)
    k, v = _c(k), _c(v)
    return int(lib().spo_store_kv(_p(k_pool), _p(v_pool), ctypes.byref(lay), _p(t), len(t), _p(k),
                                  _p(v), k.shape[1], start_pos, k.itemsize))


def gather_kv(k_pool: np.ndarray, v_pool: np.ndarray, lay: Layout, table, seq_len: int):
    t = _c(table, np.int32)
    shape = (lay.num_kv_heads, seq_len, lay.head_dim)
    ko = np.zeros(shape, dtype=k_pool.dtype)
    vo = np.zeros(shape, dtype=v_pool.dtype)
    rc = lib().spo_gather_kv(_p(ko), _p(vo), _p(_c(k_pool)), _p(_c(v_pool)), ctypes.byref(lay),
                             _p(t), len(t), seq_len, k_pool.itemsize)
    if rc:
        raise IndexError("gather_kv: table does not cover seq_len")
    return ko, vo


# --- masks -------------------------------------------------------------------------------------

def causal_mask(n: int) -> np.ndarray:
    out = np.empty((n, n), dtype=np.float32)
    lib().spo_causal_mask(n, _p(out))
    return out


def prefill_causal_mask(new_len: int, total_len: int) -> np.ndarray:
    out = np.empty((new_len, total_len), dtype=np.float32)
    lib().spo_prefill_causal_mask(new_len, total_len, _p(out))
    return out


def sliding_window_mask(n: int, window: int) -> np.ndarray:
    out = np.empty((n, n), dtype=np.float32)
    lib().spo_sliding_window_mask(n, window, _p(out))
    return out


def sliding_window_prefill_mask(new_len: int, total_len: int, window: int) -> np.ndarray:
    out = np.empty((new_len, total_len), dtype=np.float32)
    lib().spo_sliding_window_prefill_mask(new_len, total_len, window, _p(out))
    return out


# --- attention --------------------------------------------------------------------------------

def attention_f64(q, k, v, *, scale: float, mask=None, causal: bool = False, q_pos0: int = 0,
                  window_left: int = -1, dtype: int | None = None,
                  softcap: float = 0.0) -> np.ndarray:
    """q [Sq, Hq, D], k [Lk, Hkv, D], v [Lk, Hkv, Dv] (float32, or uint16 bf16 bits) ->
    float64 [Sq, Hq, Dv]. mask: additive [Sq, Lk] (replaces the causal / window predicate).
    softcap > 0: Gemma-4's logit soft cap on the scaled logits, before the mask."""
    q, k, v = _c(q), _c(k), _c(v)
    dt = _dtype_code(q, dtype)
    sq, hq, d = q.shape
    lk, hkv, _ = k.shape
    dv = v.shape[2]
    if softcap:
        out = np.empty((sq, hq, dv), dtype=np.float64)
        m = None if mask is None else _c(mask, np.float32)
        lib().spo_attention_f64_cap(_p(q), hq * d, d, _p(k), hkv * d, d, _p(v), hkv * dv, dv, dv,
                                    sq, lk, hq, hkv, d, scale, softcap, _p(m), int(causal),
                                    q_pos0, window_left, dt, _p(out))
        return out
    if dv == d:
        out = np.empty((sq, hq, d), dtype=np.float64)
        m = None if mask is None else _c(mask, np.float32)
        lib().spo_attention_f64(_p(q), hq * d, d, _p(k), _p(v), hkv * d, d, sq, lk, hq, hkv, d,
                                scale, _p(m), int(causal), q_pos0, window_left, dt, _p(out))
        return out
    out = np.empty((sq, hq, dv), dtype=np.float64)
    m = None if mask is None else _c(mask, np.float32)
    lib().spo_attention_f64_v(_p(q), hq * d, d, _p(k), hkv * d, d, _p(v), hkv * dv, dv, dv, sq,
                              lk, hq, hkv, d, scale, _p(m), int(causal), q_pos0, window_left, dt,
                              _p(out))
    return out


def attention_f32_refops(q, k, v, *, scale: float, mask=None, causal: bool = False,
                         q_pos0: int = 0, window_left: int = -1,
                         dtype: int | None = None) -> np.ndarray:
    """The reference's f32 op order (transformer.rs:234-243) -> float32 [Sq, Hq, D]."""
    q, k, v = _c(q), _c(k), _c(v)
    dt = _dtype_code(q, dtype)
    sq, hq, d = q.shape
    lk, hkv, _ = k.shape
    out = np.empty((sq, hq, d), dtype=np.float32)
    m = None if mask is None else _c(mask, np.float32)
    lib().spo_attention_f32_refops(_p(q), hq * d, d, _p(k), _p(v), hkv * d, d, sq, lk, hq, hkv,
                                   d, scale, _p(m), int(causal), q_pos0, window_left, dt, _p(out))
    return out


def paged_decode_f64(q, k_pool, v_pool, lay: Layout, block_tables, context_lens, *, scale: float,
                     window_left: int = -1, dtype: int | None = None,
                     softcap: float = 0.0) -> np.ndarray:
    """Reference decode for a batch: per sequence gather_kv (paged_attention.rs:313-378), then
    softmax((q k^T) scale) v over all gathered keys (decode has no mask, llama.rs:255-260),
    optionally restricted to the last window_left+1 keys. -> float64 [B, Hq, D]."""
    q = _c(q)
    b, hq, d = q.shape
    out = np.zeros((b, hq, d), dtype=np.float64)
    for s in range(b):
        L = int(context_lens[s])
        if L == 0:
            continue
        kg, vg = gather_kv(k_pool, v_pool, lay, block_tables[s], L)  # [Hkv, L, D]
        kt = np.ascontiguousarray(kg.transpose(1, 0, 2))               # [L, Hkv, D]
        vt = np.ascontiguousarray(vg.transpose(1, 0, 2))
        out[s] = attention_f64(q[s:s + 1], kt, vt, scale=scale, causal=True, q_pos0=L - 1,
                               window_left=window_left, dtype=dtype, softcap=softcap)[0]
    return out


def cpu_decode_baseline(out, q, k_new, v_new, k_pool, v_pool, lay: Layout, block_tables,
                        context_lens, *, scale: float, window_left: int = -1, threads: int = 0):
    """Timed CPU port of the reference's decode op sequence (all float32 arrays, in place)."""
    bt = _c(block_tables, np.int32)
    cl = _c(context_lens, np.int32)
    lib().spo_cpu_decode_baseline(_p(out), _p(q), _p(k_new), _p(v_new), _p(k_pool), _p(v_pool),
                                  ctypes.byref(lay), _p(bt), bt.shape[1], _p(cl), len(cl),
                                  q.shape[1], scale, window_left, threads)


def cpu_prefill_baseline(out, q, k, v, cu_seqlens, *, hq: int, hkv: int, d: int, scale: float,
                         threads: int = 0):
    cu = _c(cu_seqlens, np.int32)
    lib().spo_cpu_prefill_baseline(_p(out), _p(q), _p(k), _p(v), _p(cu), len(cu) - 1, hq, hkv, d,
                                   scale, threads)


def rope_caches(rows: int, head_dim: int, base: float = 10000.0):
    """RotaryEmbedding::with_base (rope.rs:60-102): full f32 caches [rows, head_dim] with each
    pair's cos / sin repeated (repeat_interleave)."""
    cos = np.zeros((rows, head_dim), dtype=np.float32)
    sin = np.zeros_like(cos)
    lib().spo_rope_caches(_p(cos), _p(sin), rows, head_dim, base)
    return cos, sin


def rope_apply(x: np.ndarray, positions, cos_full: np.ndarray, sin_full: np.ndarray) -> np.ndarray:
    """apply_rotary (rope.rs:136-170) on a float32 [T, H, D] copy of x: token t rotated by the
    caches' row positions[t]. Returns the rotated copy."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    t, h, d = y.shape
    pos = _c(positions, np.int32)
    rc = lib().spo_rope_apply(_p(y), t, h, d, h * d, d, _p(pos), _p(np.ascontiguousarray(cos_full)),
                              _p(np.ascontiguousarray(sin_full)), cos_full.shape[0])
    if rc != 0:
        raise ValueError("position outside the rotary caches")
    return y


# --- PolarQuant codec (kv_cache.rs:437-532) ---------------------------------------------------

def f32_to_f16_bits(x: float) -> int:
    """f16::from_f32(x).to_bits() (IEEE round to nearest even)."""
    return int(lib().spo_f32_to_f16_bits(float(x)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().spo_f16_bits_to_f32(int(h) & 0xFFFF))


def polar_record_bytes(head_dim: int) -> int:
    """Bytes of one PolarQuant record: 2 (f16 magnitude) + ceil(head_dim / 2) (kv_cache.rs:441-443)."""
    return int(lib().spo_polar_record_bytes(head_dim))


def polar_compress(x: np.ndarray) -> np.ndarray:
    """polar_quant_compress (kv_cache.rs:437-483) of the float32 rows of x [..., head_dim]:
    uint8 records [..., record_bytes]."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    d = a.shape[-1]
    n = a.size // d if d else 0
    out = np.zeros(a.shape[:-1] + (polar_record_bytes(d),), dtype=np.uint8)
    lib().spo_polar_compress(_p(out), _p(a), n, d)
    return out


def polar_decompress(records: np.ndarray, head_dim: int) -> np.ndarray:
    """polar_quant_decompress (kv_cache.rs:486-532): uint8 records [..., record_bytes] -> float32
    rows [..., head_dim]."""
    r = np.ascontiguousarray(records, dtype=np.uint8)
    assert r.shape[-1] == polar_record_bytes(head_dim)
    n = r.size // r.shape[-1]
    out = np.zeros(r.shape[:-1] + (head_dim,), dtype=np.float32)
    lib().spo_polar_decompress(_p(out), _p(r), n, head_dim)
    return out


def polar_compression_ratio(head_dim: int) -> float:
    """KvQuantMethod::PolarQuant.compression_ratio (kv_cache.rs:315-318)."""
    return float(lib().spo_polar_compression_ratio(head_dim))


def qjl_lcg_normal(count: int, scale: float) -> np.ndarray:
    """lcg_normal_f32 (kv_cache.rs:373-396): the reference's seed-42 LCG + Box-Muller, float32."""
    out = np.zeros(count, dtype=np.float32)
    lib().spo_qjl_lcg_normal(_p(out), count, scale)
    return out


def qjl_projection(proj_dim: int, head_dim: int) -> np.ndarray:
    """The QJL projection R [proj_dim, head_dim] of CompressedKvCache::new (kv_cache.rs:417-424)."""
    out = np.zeros((proj_dim, head_dim), dtype=np.float32)
    lib().spo_qjl_projection(_p(out), proj_dim, head_dim)
    return out


def qjl_record_bytes(proj_dim: int) -> int:
    return int(lib().spo_qjl_record_bytes(proj_dim))


def qjl_compress(x: np.ndarray, proj: np.ndarray) -> np.ndarray:
    """qjl_compress (kv_cache.rs:534-569) of the float32 rows of x [..., head_dim]."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    r = np.ascontiguousarray(proj, dtype=np.float32)
    p, d = r.shape
    n = a.size // d if d else 0
    out = np.zeros(a.shape[:-1] + (qjl_record_bytes(p),), dtype=np.uint8)
    lib().spo_qjl_compress(_p(out), _p(a), n, d, _p(r), p)
    return out


def qjl_decompress(records: np.ndarray, proj: np.ndarray) -> np.ndarray:
    """qjl_decompress (kv_cache.rs:571-617): uint8 records -> float32 rows [..., head_dim]."""
    r = np.ascontiguousarray(proj, dtype=np.float32)
    p, d = r.shape
    b = np.ascontiguousarray(records, dtype=np.uint8)
    assert b.shape[-1] == qjl_record_bytes(p)
    n = b.size // b.shape[-1]
    out = np.zeros(b.shape[:-1] + (d,), dtype=np.float32)
    lib().spo_qjl_decompress(_p(out), _p(b), n, d, _p(r), p)
    return out


def qjl_compression_ratio(proj_dim: int, head_dim: int) -> float:
    """KvQuantMethod::QJL.compression_ratio (kv_cache.rs:319-321)."""
    return float(lib().spo_qjl_compression_ratio(proj_dim, head_dim))
