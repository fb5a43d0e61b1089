"""GPU parity of sp_rope_kv_append (RoPE fused into the paged-cache append) against the oracle:
RotaryEmbedding::forward restated in oracle/sp_oracle.c (rope.rs:60-170) followed by the slot-mapped
store (paged_attention.rs:230-310). Bit-exact: f32 rows equal the oracle's fp32 op sequence; bf16 /
f16 rows equal that fp32 result rounded once (round to nearest even); V rows and untouched slots
are copies / zeros; skipped tokens leave pools and Q untouched."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import announce

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _run(seed, *, tokens, hq, hkv, d, bs, num_blocks, dtype, rows=4096, base=10000.0,
         num_layers=1, layer=0, head_major=False, with_q=True, positions=None, skip_slot=(),
         skip_pos=()):
    announce(f"rope seed={seed} T={tokens} hq={hq} hkv={hkv} d={d} bs={bs} {dtype} "
             f"layers={num_layers}/{layer} head_major={head_major}")
    rng = np.random.default_rng(seed)
    dt = DT[dtype]
    if positions is None:
        positions = rng.integers(0, rows, tokens)
    positions = np.asarray(positions, dtype=np.int32).copy()
    slots = rng.choice(num_blocks * bs, tokens, replace=False).astype(np.int32)
    for t in skip_slot:
        slots[t] = -1
    for t in skip_pos:
        positions[t] = rows  # outside the tables
    g = torch.Generator(device="cuda").manual_seed(seed)
    k32 = torch.randn(tokens, hkv, d, generator=g, device="cuda")
    v32 = torch.randn(tokens, hkv, d, generator=g, device="cuda")
    q32 = torch.randn(tokens, hq, d, generator=g, device="cuda")
    k_new, v_new, q = k32.to(dt), v32.to(dt), q32.to(dt)
    q_in = q.clone()
    pool_shape = (num_blocks, num_layers, hkv, bs, d)
    k_pool = torch.zeros(pool_shape, dtype=dt, device="cuda")
    v_pool = torch.zeros_like(k_pool)
    cos, sin = sp.rope_tables(rows, d, base)
    cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    lay = sp.layout(num_blocks, num_layers, layer, hkv, bs, d)
    pos_d = torch.from_numpy(positions).cuda()
    slot_d = torch.from_numpy(slots).cuda()
    if head_major:  # the reference's [Hkv, T, D] layout (paged_attention.rs:234)
        k_src = k_new.transpose(0, 1).contiguous()
        v_src = v_new.transpose(0, 1).contiguous()
        sp.rope_kv_append(k_pool, v_pool, lay, k_src, v_src, pos_d, slot_d, cos_d, sin_d,
                          q=q if with_q else None, token_stride=d, head_stride=tokens * d)
    else:
        sp.rope_kv_append(k_pool, v_pool, lay, k_new, v_new, pos_d, slot_d, cos_d, sin_d,
                          q=q if with_q else None)
    torch.cuda.synchronize()

    # oracle: rotate in fp32 with the reference's caches, round once to the storage type
    cos_full, sin_full = O.rope_caches(rows, d, base)
    ok = (slots >= 0) & (positions < rows)
    safe_pos = np.where(positions < rows, positions, 0)
    k_rot = O.rope_apply(k_new.float().cpu().numpy(), safe_pos, cos_full, sin_full)
    q_rot = O.rope_apply(q_in.float().cpu().numpy(), safe_pos, cos_full, sin_full)
    k_exp = torch.from_numpy(k_rot).to(dt)
    q_exp = torch.from_numpy(q_rot).to(dt)
    kp_exp = torch.zeros(pool_shape, dtype=dt)
    vp_exp = torch.zeros(pool_shape, dtype=dt)
    v_host = v_new.cpu()
    for t in range(tokens):
        if not ok[t]:
            continue
        blk, off = divmod(int(slots[t]), bs)
        kp_exp[blk, layer, :, off] = k_exp[t]
        vp_exp[blk, layer, :, off] = v_host[t]
    bits = (lambda x: x.view(torch.int32)) if dtype == "f32" else (lambda x: x.view(torch.int16))
    assert torch.equal(bits(k_pool.cpu()), bits(kp_exp)), "rotated K rows differ"
    assert torch.equal(bits(v_pool.cpu()), bits(vp_exp)), "V rows differ"
    if with_q:
        q_want = torch.where(torch.from_numpy(positions < rows)[:, None, None], q_exp, q_in.cpu())
        assert torch.equal(bits(q.cpu()), bits(q_want)), "rotated Q rows differ"
    else:
        assert torch.equal(q, q_in)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("d", [64, 128])
def test_rope_append_dtypes(dtype, d):
    _run(100 + d, tokens=37, hq=8, hkv=2, d=d, bs=16, num_blocks=32, dtype=dtype)


def test_rope_append_c2_decode_step():
    """One decode step of C2 (64 sequences, Llama-3-8B heads): positions = context_len - 1."""
    w = W.decode_c2()
    pos = (w.context_lens - 1).astype(np.int32)
    _run(2, tokens=w.num_seqs, hq=w.hq, hkv=w.hkv, d=w.head_dim, bs=16, num_blocks=w.num_blocks,
         dtype="bf16", rows=8192, positions=pos, base=500000.0)


def test_rope_append_c3_prefill_stream():
    """The C3 packed stream (9,476 tokens): positions 0..L-1 within each sequence."""
    w = W.prefill_c3()
    pos = np.concatenate([np.arange(L) for L in w.lens]).astype(np.int32)
    _run(3, tokens=w.total_tokens, hq=w.hq, hkv=w.hkv, d=w.head_dim, bs=16,
         num_blocks=(w.total_tokens + 15) // 16 + 8, dtype="bf16", rows=2048, positions=pos)


def test_rope_append_head_major_and_layers():
    """The reference's head-major [Hkv, T, D] input into layer 2 of a 3-layer pool, no Q."""
    _run(5, tokens=50, hq=4, hkv=4, d=128, bs=32, num_blocks=16, dtype="bf16", num_layers=3,
         layer=2, head_major=True, with_q=False)


def test_rope_append_skips_invalid_tokens():
    """A negative slot skips the token's K/V write (its Q is still rotated); a position outside
    the tables skips the whole token."""
    _run(9, tokens=20, hq=8, hkv=2, d=64, bs=16, num_blocks=8, dtype="f32", rows=64,
         skip_slot=(0, 7), skip_pos=(3, 19))
