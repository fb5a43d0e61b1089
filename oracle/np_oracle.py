"""Independent numpy (float64) restatement of the path, used to cross-check the C oracle.

TEST INFRASTRUCTURE ONLY. Written from the reference's semantics, not from sp_oracle.c:
dense masks are built by predicate arrays and attention is an einsum over the whole sequence.
  BlockTable.get_block/get_slot      paged_attention.rs:124-132
  store_kv / gather_kv               paged_attention.rs:230-378
  causal / window / prefill masks    transformer.rs:415-451, llama.rs:374-388, gemma4.rs:1086-1108
  attention + repeat_kv              transformer.rs:227-271
"""
from __future__ import annotations

import numpy as np


def bf16_bits_to_f64(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def to_f64(a: np.ndarray) -> np.ndarray:
    if a.dtype == np.uint16:
        return bf16_bits_to_f64(a)
    return a.astype(np.float64)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def causal_mask(n: int) -> np.ndarray:
    i, j = np.indices((n, n))
    return np.where(j > i, -np.inf, 0.0).astype(np.float32)


def prefill_causal_mask(new_len: int, total_len: int) -> np.ndarray:
    i, j = np.indices((new_len, total_len))
    return np.where(j > (total_len - new_len) + i, -np.inf, 0.0).astype(np.float32)


def sliding_window_mask(n: int, window: int) -> np.ndarray:
    i, j = np.indices((n, n))
    return np.where((j > i) | (i > j + window), -np.inf, 0.0).astype(np.float32)


def sliding_window_prefill_mask(new_len: int, total_len: int, window: int) -> np.ndarray:
    i, j = np.indices((new_len, total_len))
    p = (total_len - new_len) + i
    bad = (j > p) | ((p >= window) & (j < p - window + 1))
    return np.where(bad, -np.inf, 0.0).astype(np.float32)


def attention(q, k, v, scale: float, mask=None, softcap: float = 0.0) -> np.ndarray:
    """q [Sq, Hq, D], k/v [Lk, Hkv, D] -> [Sq, Hq, D] float64; rows with no visible key are 0.
    softcap > 0: softcap * tanh(logits / softcap) before the mask (gemma4.rs:366-377)."""
    q, k, v = to_f64(q), to_f64(k), to_f64(v)
    hq, hkv = q.shape[1], k.shape[1]
    rep = hq // hkv
    kr = np.repeat(k, rep, axis=1)  # repeat_kv: head h -> kv head h // rep
    vr = np.repeat(v, rep, axis=1)
    s = np.einsum("ihd,jhd->hij", q, kr) * scale
    if softcap > 0:
        s = softcap * np.tanh(s / softcap)
    if mask is not None:
        s = s + mask[None].astype(np.float64)
    m = s.max(axis=2, keepdims=True)
    ok = np.isfinite(m)
    e = np.where(ok, np.exp(s - np.where(ok, m, 0.0)), 0.0)
    den = e.sum(axis=2, keepdims=True)
    p = np.where(den > 0, e / np.where(den > 0, den, 1.0), 0.0)
    return np.einsum("hij,jhd->ihd", p, vr)


def pool_index(layout, blk: int, layer: int, head: int, slot: int) -> tuple:
    return (blk, layer, head, slot)


def store_kv(k_pool, v_pool, layer: int, table, k, v, start_pos: int, block_size: int) -> None:
    """pools are [num_blocks, num_layers, Hkv, BS, D] arrays; k, v are [Hkv, S, D]."""
    for i in range(k.shape[1]):
        pos = start_pos + i
        bn = pos // block_size
        if bn >= len(table):
            raise IndexError("Block not allocated")
        k_pool[table[bn], layer, :, pos % block_size, :] = k[:, i, :]
        v_pool[table[bn], layer, :, pos % block_size, :] = v[:, i, :]


def gather_kv(k_pool, v_pool, layer: int, table, seq_len: int, block_size: int):
    hkv, d = k_pool.shape[2], k_pool.shape[4]
    if seq_len == 0:
        return (np.zeros((hkv, 0, d), k_pool.dtype), np.zeros((hkv, 0, d), v_pool.dtype))
    pos = np.arange(seq_len)
    blk = np.asarray(table)[pos // block_size]
    slot = pos % block_size
    k = k_pool[blk, layer, :, slot, :].transpose(1, 0, 2)  # [Hkv, L, D]
    v = v_pool[blk, layer, :, slot, :].transpose(1, 0, 2)
    return np.ascontiguousarray(k), np.ascontiguousarray(v)
