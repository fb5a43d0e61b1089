"""Seeded synthetic workloads for the five benchmark configurations (C1-C5).

Metadata (context lengths, block tables, sequence offsets) comes from numpy's PCG64 with seed
0x5EED0000 + config index, so it is identical on every machine. Tensor contents are N(0, 1)
drawn by torch on the target device from the same seed, and handed to the oracle by copying
them back to the host.

    C1  f32 paged decode, 4 seqs, L = 17/64/129/250, 8 q / 8 kv heads, D 64, BS 16, 64 blocks
    C2  Llama-3-8B bf16 paged decode, B 64, L ~ U[512, 4096], 32/8 heads, D 128, BS 16
    C3  ragged causal prefill bf16, 8 seqs L ~ U[256, 2048], 32/8 heads, D 128
    C4  Qwen2.5-7B mixed: 4 chunks x 512 on context U[1024, 8192] + 128 decode U[256, 4096], 28/4
    C5  Mistral-7B windowed decode bf16, B 16, L ~ U[8192, 32768], 32/8 heads, W 4096
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SEED_BASE = 0x5EED0000


def seed_for(config_index: int) -> int:
    return SEED_BASE + config_index


@dataclass
class DecodeWorkload:
    """One decode step over a ragged batch: append one token per sequence, then attend."""

    name: str
    seed: int
    num_seqs: int
    hq: int
    hkv: int
    head_dim: int
    block_size: int
    dtype: str                    # "f32" | "bf16"
    context_lens: np.ndarray      # int32 [B], includes the token appended this step
    block_tables: np.ndarray      # int32 [B, max_blocks]
    num_blocks: int               # pool size
    window_left: int = -1         # -1: no window; Mistral window W -> W
    num_layers: int = 1
    layer: int = 0
    extra: dict = field(default_factory=dict)

    @property
    def max_context_len(self) -> int:
        return int(self.context_lens.max()) if self.num_seqs else 0

    @property
    def max_blocks(self) -> int:
        return int(self.block_tables.shape[1])

    @property
    def elem_bytes(self) -> int:
        return 4 if self.dtype == "f32" else 2

    def slot_mapping(self) -> np.ndarray:
        """Slot of the appended token of each sequence (position L-1): block * BS + slot."""
        pos = self.context_lens.astype(np.int64) - 1
        blk = self.block_tables[np.arange(self.num_seqs), pos // self.block_size]
        return (blk.astype(np.int64) * self.block_size + pos % self.block_size).astype(np.int32)

    def attended_keys(self) -> np.ndarray:
        lens = self.context_lens.astype(np.int64)
        if self.window_left < 0:
            return lens
        return np.minimum(lens, self.window_left + 1)

    def decode_bytes(self) -> int:
        """Algorithmic HBM bytes of the attention launch: each attended K/V row once, q, out,
        the block-table entries walked and the context lengths."""
        e = self.elem_bytes
        kv = int(self.attended_keys().sum()) * 2 * self.hkv * self.head_dim * e
        qo = self.num_seqs * self.hq * self.head_dim * 2 * e
        tables = int(((self.attended_keys() + self.block_size - 1) // self.block_size).sum()) * 4
        return kv + qo + tables + self.num_seqs * 4

    def append_bytes(self) -> int:
        """Algorithmic bytes of the append: read + write of one K and one V row per sequence
        and KV head, plus the slot mapping."""
        e = self.elem_bytes
        return self.num_seqs * self.hkv * self.head_dim * e * 2 * 2 + self.num_seqs * 4

    def polar_record_bytes(self) -> int:
        """PolarQuant record of one vector: binary16 norm + head_dim/2 code bytes."""
        return 2 + self.head_dim // 2

    def polar_decode_bytes(self) -> int:
        """decode_bytes with every attended K/V row read as a PolarQuant record."""
        kv = int(self.attended_keys().sum()) * 2 * self.hkv * self.polar_record_bytes()
        return self.decode_bytes() - int(self.attended_keys().sum()) * 2 * self.hkv * \
            self.head_dim * self.elem_bytes + kv

    def polar_append_bytes(self) -> int:
        """Encode on append: read one K and one V row per sequence and KV head, write their
        records, plus the slot mapping."""
        return self.num_seqs * self.hkv * 2 * (self.head_dim * self.elem_bytes +
                                               self.polar_record_bytes()) + self.num_seqs * 4

    def layout(self):
        from ._lib import layout
        return layout(self.num_blocks, self.num_layers, self.layer, self.hkv, self.block_size,
                      self.head_dim)


def _tables_from_pool(rng: np.random.Generator, lens: np.ndarray, block_size: int,
                      num_blocks: int) -> np.ndarray:
    """Block tables as consecutive slices of one seeded permutation of the pool's block ids."""
    need = (lens + block_size - 1) // block_size
    assert need.sum() <= num_blocks
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = np.full((len(lens), max(int(need.max()), 1)), -1, dtype=np.int32)
    off = 0
    for s, n in enumerate(need):
        tables[s, :n] = perm[off:off + n]
        off += n
    return tables


def decode_c1() -> DecodeWorkload:
    seed = seed_for(1)
    rng = np.random.default_rng(seed)
    lens = np.array([17, 64, 129, 250], dtype=np.int32)
    tables = _tables_from_pool(rng, lens, 16, 64)
    return DecodeWorkload("C1-f32-decode", seed, 4, 8, 8, 64, 16, "f32", lens, tables, 64)


def decode_c2() -> DecodeWorkload:
    seed = seed_for(2)
    rng = np.random.default_rng(seed)
    lens = rng.integers(512, 4096, size=64, endpoint=True).astype(np.int32)
    nblk = int(((lens + 15) // 16).sum())
    tables = _tables_from_pool(rng, lens, 16, nblk)
    return DecodeWorkload("C2-llama3-8b-decode", seed, 64, 32, 8, 128, 16, "bf16", lens, tables,
                          nblk)


def decode_c4() -> DecodeWorkload:
    """The decode half of the C4 mixed batch (Qwen2.5-7B heads: 28 q / 4 kv, GQA 7)."""
    seed = seed_for(4)
    rng = np.random.default_rng(seed)
    lens = rng.integers(256, 4096, size=128, endpoint=True).astype(np.int32)
    nblk = int(((lens + 15) // 16).sum())
    tables = _tables_from_pool(rng, lens, 16, nblk)
    return DecodeWorkload("C4-qwen25-7b-decode", seed, 128, 28, 4, 128, 16, "bf16", lens, tables,
                          nblk)


def decode_c5() -> DecodeWorkload:
    seed = seed_for(5)
    rng = np.random.default_rng(seed)
    lens = rng.integers(8192, 32768, size=16, endpoint=True).astype(np.int32)
    nblk = int(((lens + 15) // 16).sum())
    tables = _tables_from_pool(rng, lens, 16, nblk)
    return DecodeWorkload("C5-mistral-7b-window-decode", seed, 16, 32, 8, 128, 16, "bf16", lens,
                          tables, nblk, window_left=4096)


def decode_gemma4_d256() -> DecodeWorkload:
    """Gemma-4's sliding-window layers (head_dim_swa 256, 16 query / 8 KV heads, a window of
    1024 keys: window_left 1023; gemma4.rs:94-102, :1086-1108) at C2's batch: 64 sequences with
    contexts U[512, 4096], bf16, block size 16. Not one of the five benchmark configurations."""
    seed = seed_for(6)
    rng = np.random.default_rng(seed)
    lens = rng.integers(512, 4096, size=64, endpoint=True).astype(np.int32)
    nblk = int(((lens + 15) // 16).sum())
    tables = _tables_from_pool(rng, lens, 16, nblk)
    return DecodeWorkload("gemma4-d256-window-decode", seed, 64, 16, 8, 256, 16, "bf16", lens,
                          tables, nblk, window_left=1023)


def decode_gemma4_d512() -> DecodeWorkload:
    """Gemma-4's global-attention layers (head_dim 512, 16 query / 8 KV heads, no window;
    gemma4.rs:82-107) at C2's batch: 64 sequences with contexts U[512, 4096], bf16, block size
    16. Not one of the five benchmark configurations."""
    seed = seed_for(8)
    rng = np.random.default_rng(seed)
    lens = rng.integers(512, 4096, size=64, endpoint=True).astype(np.int32)
    nblk = int(((lens + 15) // 16).sum())
    tables = _tables_from_pool(rng, lens, 16, nblk)
    return DecodeWorkload("gemma4-d512-global-decode", seed, 64, 16, 8, 512, 16, "bf16", lens,
                          tables, nblk)


DECODE_CONFIGS = {"C1": decode_c1, "C2": decode_c2, "C4": decode_c4, "C5": decode_c5}


def random_decode(seed: int, num_seqs: int, hq: int, hkv: int, head_dim: int, block_size: int,
                  dtype: str, min_len: int, max_len: int, window_left: int = -1,
                  spare_blocks: int = 3, num_layers: int = 1, layer: int = 0) -> DecodeWorkload:
    """A small seeded decode batch for parity tests (lengths may be 0 when min_len is 0)."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(min_len, max_len, size=num_seqs, endpoint=True).astype(np.int32)
    nblk = int(((lens + block_size - 1) // block_size).sum()) + spare_blocks
    tables = _tables_from_pool(rng, lens, block_size, nblk)
    return DecodeWorkload(f"random-decode-{seed}", seed, num_seqs, hq, hkv, head_dim, block_size,
                          dtype, lens, tables, nblk, window_left=window_left,
                          num_layers=num_layers, layer=layer)


# ---------------------------------------------------------------------------------------------
# device tensors for a decode workload
# ---------------------------------------------------------------------------------------------

def torch_dtype(name: str):
    import torch
    return {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[name]


def make_decode_tensors(w: DecodeWorkload, device="cuda") -> dict:
    """Pools filled with N(0,1) (every slot, so stale data sits past each context end), the
    step's q / k_new / v_new, and the int32 metadata, all on `device`."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    dt = torch_dtype(w.dtype)
    pool_shape = (w.num_blocks, w.num_layers, w.hkv, w.block_size, w.head_dim)

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32).to(dt)

    t = {
        "k_pool": randn(*pool_shape),
        "v_pool": randn(*pool_shape),
        "q": randn(w.num_seqs, w.hq, w.head_dim),
        "k_new": randn(w.num_seqs, w.hkv, w.head_dim),
        "v_new": randn(w.num_seqs, w.hkv, w.head_dim),
        "block_tables": torch.from_numpy(w.block_tables).to(device),
        "context_lens": torch.from_numpy(w.context_lens).to(device),
        "slot_mapping": torch.from_numpy(w.slot_mapping()).to(device),
    }
    t["out"] = torch.empty_like(t["q"])
    return t


# ---------------------------------------------------------------------------------------------
# prefill workloads
# ---------------------------------------------------------------------------------------------

@dataclass
class PrefillWorkload:
    """Causal self-attention prefill of a ragged batch packed into one token stream. The step
    also appends every token's K/V into a paged pool (block size 16) through a slot mapping."""

    name: str
    seed: int
    lens: np.ndarray          # int32 [num_seqs] tokens per sequence
    hq: int
    hkv: int
    head_dim: int
    dtype: str
    block_size: int = 16
    window_left: int = -1     # -1: causal only; W keys [p - W + 1, p] (gemma-4) -> W - 1

    @property
    def num_seqs(self) -> int:
        return len(self.lens)

    @property
    def cu_seqlens(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.lens)]).astype(np.int32)

    @property
    def total_tokens(self) -> int:
        return int(self.lens.sum())

    @property
    def max_seqlen(self) -> int:
        return int(self.lens.max())

    def flops(self) -> int:
        """4 * Hq * D per visible (query, key) pair; causal: L(L+1)/2 pairs per sequence, and
        query i sees min(i + 1, window_left + 1) keys under a window."""
        L = self.lens.astype(np.int64)
        if self.window_left < 0:
            pairs = (L * (L + 1) // 2).sum()
        else:
            w = self.window_left + 1
            full = np.minimum(L, w)  # queries 0 .. full-1 see i + 1 keys, the rest w keys
            pairs = (full * (full + 1) // 2 + (L - full) * w).sum()
        return int(4 * self.hq * self.head_dim * pairs)

    def pool_tables(self):
        rng = np.random.default_rng(self.seed + 1)
        nblk = int(((self.lens + self.block_size - 1) // self.block_size).sum())
        return _tables_from_pool(rng, self.lens, self.block_size, nblk), nblk

    def slot_mapping(self) -> np.ndarray:
        tables, _ = self.pool_tables()
        out = []
        for s, L in enumerate(self.lens):
            pos = np.arange(L)
            out.append(tables[s, pos // self.block_size] * self.block_size + pos % self.block_size)
        return np.concatenate(out).astype(np.int32)


def prefill_c3() -> PrefillWorkload:
    seed = seed_for(3)
    rng = np.random.default_rng(seed)
    lens = rng.integers(256, 2048, size=8, endpoint=True).astype(np.int32)
    return PrefillWorkload("C3-llama3-8b-ragged-prefill", seed, lens, 32, 8, 128, "bf16")


def prefill_gemma4_d256() -> PrefillWorkload:
    """Gemma-4 sliding-layer prefill: C3's lengths drawn again (8 sequences U[256, 2048]) at
    head_dim 256, 16 query / 8 KV heads, causal within a 1024-key window, bf16."""
    seed = seed_for(7)
    rng = np.random.default_rng(seed)
    lens = rng.integers(256, 2048, size=8, endpoint=True).astype(np.int32)
    return PrefillWorkload("gemma4-d256-window-prefill", seed, lens, 16, 8, 256, "bf16",
                           window_left=1023)


def prefill_gemma4_d512() -> PrefillWorkload:
    """Gemma-4 global-layer prefill: C3's lengths drawn again (8 sequences U[256, 2048]) at
    head_dim 512, 16 query / 8 KV heads, causal, bf16."""
    seed = seed_for(9)
    rng = np.random.default_rng(seed)
    lens = rng.integers(256, 2048, size=8, endpoint=True).astype(np.int32)
    return PrefillWorkload("gemma4-d512-global-prefill", seed, lens, 16, 8, 512, "bf16")


def make_prefill_tensors(w: PrefillWorkload, device="cuda", with_pool: bool = True) -> dict:
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    dt = torch_dtype(w.dtype)

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32).to(dt)

    T = w.total_tokens
    t = {
        "q": randn(T, w.hq, w.head_dim),
        "k": randn(T, w.hkv, w.head_dim),
        "v": randn(T, w.hkv, w.head_dim),
        "cu_seqlens": torch.from_numpy(w.cu_seqlens).to(device),
    }
    t["out"] = torch.empty_like(t["q"])
    if with_pool:
        tables, nblk = w.pool_tables()
        t["k_pool"] = torch.zeros(nblk, 1, w.hkv, w.block_size, w.head_dim, dtype=dt, device=device)
        t["v_pool"] = torch.zeros_like(t["k_pool"])
        t["block_tables"] = torch.from_numpy(tables).to(device)
        t["slot_mapping"] = torch.from_numpy(w.slot_mapping()).to(device)
        t["num_blocks"] = nblk
    return t


@dataclass
class ChunkedPrefillWorkload:
    """New-token chunks attending to a paged context that already holds them (bottom-right
    causal), i.e. forward_cached with seq_len > 1 and prefill_causal_mask."""

    name: str
    seed: int
    chunk_lens: np.ndarray     # int32 [S] new tokens per sequence
    ctx_before: np.ndarray     # int32 [S] cached tokens before the chunk
    hq: int
    hkv: int
    head_dim: int
    dtype: str
    block_size: int = 16
    window_left: int = -1

    @property
    def num_seqs(self) -> int:
        return len(self.chunk_lens)

    @property
    def context_lens(self) -> np.ndarray:
        return (self.ctx_before + self.chunk_lens).astype(np.int32)

    @property
    def cu_seqlens_q(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.chunk_lens)]).astype(np.int32)

    @property
    def max_seqlen_q(self) -> int:
        return int(self.chunk_lens.max())

    def flops(self) -> int:
        c = self.chunk_lens.astype(np.int64)
        b = self.ctx_before.astype(np.int64)
        pairs = (c * b + c * (c + 1) // 2).sum()
        return int(4 * self.hq * self.head_dim * pairs)

    def tables(self):
        rng = np.random.default_rng(self.seed + 1)
        lens = self.context_lens
        nblk = int(((lens + self.block_size - 1) // self.block_size).sum())
        return _tables_from_pool(rng, lens, self.block_size, nblk), nblk

    def slot_mapping(self) -> np.ndarray:
        tables, _ = self.tables()
        out = []
        for s in range(self.num_seqs):
            pos = np.arange(self.ctx_before[s], self.context_lens[s])
            out.append(tables[s, pos // self.block_size] * self.block_size + pos % self.block_size)
        return np.concatenate(out).astype(np.int32)


def chunked_prefill_c4() -> ChunkedPrefillWorkload:
    """The prefill half of C4: 4 chunks of 512 new tokens on contexts U[1024, 8192]."""
    seed = seed_for(4) + 100
    rng = np.random.default_rng(seed)
    ctx = rng.integers(1024, 8192, size=4, endpoint=True).astype(np.int32)
    chunks = np.full(4, 512, dtype=np.int32)
    return ChunkedPrefillWorkload("C4-qwen25-7b-chunked-prefill", seed, chunks, ctx, 28, 4, 128,
                                  "bf16")


def make_chunked_tensors(w: ChunkedPrefillWorkload, device="cuda") -> dict:
    """Pools with random cached context, the chunk's q/k/v, metadata."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    dt = torch_dtype(w.dtype)
    tables, nblk = w.tables()

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32).to(dt)

    T = int(w.chunk_lens.sum())
    t = {
        "k_pool": randn(nblk, 1, w.hkv, w.block_size, w.head_dim),
        "v_pool": randn(nblk, 1, w.hkv, w.block_size, w.head_dim),
        "q": randn(T, w.hq, w.head_dim),
        "k_new": randn(T, w.hkv, w.head_dim),
        "v_new": randn(T, w.hkv, w.head_dim),
        "block_tables": torch.from_numpy(tables).to(device),
        "context_lens": torch.from_numpy(w.context_lens).to(device),
        "cu_seqlens_q": torch.from_numpy(w.cu_seqlens_q).to(device),
        "slot_mapping": torch.from_numpy(w.slot_mapping()).to(device),
        "num_blocks": nblk,
    }
    t["out"] = torch.empty_like(t["q"])
    return t


# ---------------------------------------------------------------------------------------------
# mixed chunked-prefill + decode batch (C4)
# ---------------------------------------------------------------------------------------------

@dataclass
class MixedWorkload:
    """One scheduler iteration as a single ragged batch over one paged pool: prompt chunks first
    (each attending to its cached context plus itself, bottom-right causal), then one new token
    per decoding sequence (no mask) — the order build_ragged_batch produces."""

    name: str
    seed: int
    chunk_lens: np.ndarray     # int32 [P] new tokens per chunk
    ctx_before: np.ndarray     # int32 [P] cached tokens before each chunk
    decode_lens: np.ndarray    # int32 [Bd] context of each decode sequence, its new token included
    hq: int
    hkv: int
    head_dim: int
    dtype: str
    block_size: int = 16

    @property
    def num_prefill_seqs(self) -> int:
        return len(self.chunk_lens)

    @property
    def num_decode_seqs(self) -> int:
        return len(self.decode_lens)

    @property
    def num_seqs(self) -> int:
        return self.num_prefill_seqs + self.num_decode_seqs

    @property
    def new_tokens(self) -> np.ndarray:
        return np.concatenate([self.chunk_lens, np.ones(self.num_decode_seqs, np.int32)]
                              ).astype(np.int32)

    @property
    def context_lens(self) -> np.ndarray:
        return np.concatenate([self.ctx_before + self.chunk_lens, self.decode_lens]
                              ).astype(np.int32)

    @property
    def num_prefill_tokens(self) -> int:
        return int(self.chunk_lens.sum())

    @property
    def cu_seqlens_q(self) -> np.ndarray:
        """Token offsets of the chunks (the decode tokens follow them, one each)."""
        return np.concatenate([[0], np.cumsum(self.chunk_lens)]).astype(np.int32)

    def prefill_flops(self) -> int:
        c = self.chunk_lens.astype(np.int64)
        b = self.ctx_before.astype(np.int64)
        return int(4 * self.hq * self.head_dim * (c * b + c * (c + 1) // 2).sum())

    def decode_bytes(self) -> int:
        e = 4 if self.dtype == "f32" else 2
        L = self.decode_lens.astype(np.int64)
        return int((L * 2 * self.hkv * self.head_dim * e).sum()
                   + self.num_decode_seqs * self.hq * self.head_dim * e * 2
                   + ((L + self.block_size - 1) // self.block_size * 4).sum()
                   + self.num_decode_seqs * 4)

    def tables(self):
        rng = np.random.default_rng(self.seed + 1)
        lens = self.context_lens
        nblk = int(((lens + self.block_size - 1) // self.block_size).sum())
        return _tables_from_pool(rng, lens, self.block_size, nblk), nblk

    def positions(self) -> np.ndarray:
        lens, new = self.context_lens, self.new_tokens
        return np.concatenate([np.arange(L - n, L) for L, n in zip(lens, new)]).astype(np.int32)

    def slot_mapping(self) -> np.ndarray:
        tables, _ = self.tables()
        out = []
        for s, (L, n) in enumerate(zip(self.context_lens, self.new_tokens)):
            pos = np.arange(L - n, L)
            out.append(tables[s, pos // self.block_size] * self.block_size + pos % self.block_size)
        return np.concatenate(out).astype(np.int32)


def mixed_c4() -> MixedWorkload:
    """C4: Qwen2.5-7B heads (28 q / 4 kv, D 128, bf16, BS 16); 4 chunks of
    512 new tokens on contexts U[1024, 8192] plus 128 decode sequences with contexts
    U[256, 4096], one seeded shuffle of one pool."""
    pre, dec = chunked_prefill_c4(), decode_c4()
    return MixedWorkload("C4-qwen25-7b-mixed", seed_for(4) + 200, pre.chunk_lens, pre.ctx_before,
                         dec.context_lens, 28, 4, 128, "bf16")


def make_mixed_tensors(w: MixedWorkload, device="cuda") -> dict:
    """One pool with random cached context, the batch's q / k_new / v_new (chunk tokens first)
    and the int32 metadata."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    dt = torch_dtype(w.dtype)
    tables, nblk = w.tables()

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32).to(dt)

    T = int(w.new_tokens.sum())
    t = {
        "k_pool": randn(nblk, 1, w.hkv, w.block_size, w.head_dim),
        "v_pool": randn(nblk, 1, w.hkv, w.block_size, w.head_dim),
        "q": randn(T, w.hq, w.head_dim),
        "k_new": randn(T, w.hkv, w.head_dim),
        "v_new": randn(T, w.hkv, w.head_dim),
        "block_tables": torch.from_numpy(tables).to(device),
        "context_lens": torch.from_numpy(w.context_lens).to(device),
        "cu_seqlens_q": torch.from_numpy(w.cu_seqlens_q).to(device),
        "slot_mapping": torch.from_numpy(w.slot_mapping()).to(device),
        "num_blocks": nblk,
    }
    t["out"] = torch.empty_like(t["q"])
    return t
