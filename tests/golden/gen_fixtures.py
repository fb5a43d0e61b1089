"""Writes the committed golden fixtures of the attention path (tests/golden/*.npz, kats.json).

    python tests/golden/gen_fixtures.py          # rewrite every fixture
    python tests/golden/gen_fixtures.py --check  # recompute and compare, write nothing

Inputs come from numpy's PCG64 (machine independent); expected outputs come from the CPU oracle
(oracle/), whose functions are pinned separately (tests/test_oracle*.py), and each attention
output is also checked here against torch's float64 scaled_dot_product_attention before it is
written. kats.json holds the reference's own unit-test known answers as data, each with the
reference file:line it comes from. The fixtures are small on purpose (a few hundred KB in all).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402

SEED = 0x601D0000


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (inputs here are finite)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def torch_attention_f64(q, k, v, scale, *, q_pos0, causal, window_left=-1):
    """Independent check: torch float64 SDPA with an explicit boolean mask, GQA by repeat."""
    import torch
    sq, hq, d = q.shape
    lk, hkv, _ = k.shape
    rep = hq // hkv
    qt = torch.from_numpy(np.asarray(q, np.float64)).permute(1, 0, 2)
    kt = torch.from_numpy(np.asarray(k, np.float64)).permute(1, 0, 2).repeat_interleave(rep, 0)
    vt = torch.from_numpy(np.asarray(v, np.float64)).permute(1, 0, 2).repeat_interleave(rep, 0)
    pos = torch.arange(sq)[:, None] + q_pos0
    key = torch.arange(lk)[None, :]
    vis = torch.ones(sq, lk, dtype=torch.bool)
    if causal:
        vis &= key <= pos
    if window_left >= 0:
        vis &= key >= pos - window_left
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=vis, scale=scale)
    out = torch.where(vis.any(-1)[None, :, None], out, torch.zeros_like(out))
    return out.permute(1, 0, 2).numpy()


# ---------------------------------------------------------------------------------------------

def decode_case(rng, lens, hq, hkv, d, bs, dtype, window_left=-1, spare=1):
    """One decode step: append one token per sequence at position L-1, then attend."""
    lens = np.asarray(lens, np.int32)
    need = (lens + bs - 1) // bs
    nblk = int(need.sum()) + spare
    perm = rng.permutation(nblk).astype(np.int32)
    tables = np.full((len(lens), max(int(need.max()), 1)), -1, np.int32)
    off = 0
    for s, n in enumerate(need):
        tables[s, :n] = perm[off:off + n]
        off += n
    pool_shape = (nblk, 1, hkv, bs, d)
    k_pool = rng.standard_normal(pool_shape, dtype=np.float32)
    v_pool = rng.standard_normal(pool_shape, dtype=np.float32)
    q = rng.standard_normal((len(lens), hq, d), dtype=np.float32)
    k_new = rng.standard_normal((len(lens), hkv, d), dtype=np.float32)
    v_new = rng.standard_normal((len(lens), hkv, d), dtype=np.float32)
    if dtype == "bf16":
        k_pool, v_pool, q, k_new, v_new = (bf16_to_f32(bf16_bits(a)) for a in
                                           (k_pool, v_pool, q, k_new, v_new))
    lay = O.make_layout(nblk, 1, 0, hkv, bs, d)
    slots = np.empty(len(lens), np.int32)
    kp, vp = k_pool.copy(), v_pool.copy()
    for s, L in enumerate(lens):
        slots[s] = O.slot_mapping(tables[s], int(L) - 1, 1, bs)[0]
        rc = O.store_kv(kp, vp, lay, tables[s], k_new[s][:, None, :], v_new[s][:, None, :],
                        int(L) - 1)
        assert rc == 0
    scale = d ** -0.5
    out = O.paged_decode_f64(q, kp, vp, lay, tables, lens, scale=scale, window_left=window_left)
    for s, L in enumerate(lens):  # independent check of every row
        kg, vg = O.gather_kv(kp, vp, lay, tables[s], int(L))
        ref = torch_attention_f64(q[s:s + 1], kg.transpose(1, 0, 2), vg.transpose(1, 0, 2), scale,
                                  q_pos0=int(L) - 1, causal=True, window_left=window_left)
        assert np.abs(ref[0] - out[s]).max() < 1e-12
    store = (lambda a: bf16_bits(a)) if dtype == "bf16" else (lambda a: a)
    return dict(
        dtype=np.array(dtype), num_q_heads=np.int32(hq), block_size=np.int32(bs),
        window_left=np.int32(window_left), scale=np.float64(scale),
        context_lens=lens, block_tables=tables, slot_mapping=slots,
        k_pool=store(k_pool), v_pool=store(v_pool), q=store(q), k_new=store(k_new),
        v_new=store(v_new), out=out,
        k_pool_after_sha256=np.array(sha256(store(kp))),
        v_pool_after_sha256=np.array(sha256(store(vp))),
    )


def prefill_case(rng, lens_q, lens_k, hq, hkv, d, causal, window_left=-1):
    """Packed varlen prefill, bf16 inputs, bottom-right causal alignment."""
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lens_k)]).astype(np.int32)
    q = bf16_bits(rng.standard_normal((int(cu_q[-1]), hq, d), dtype=np.float32))
    k = bf16_bits(rng.standard_normal((int(cu_k[-1]), hkv, d), dtype=np.float32))
    v = bf16_bits(rng.standard_normal((int(cu_k[-1]), hkv, d), dtype=np.float32))
    scale = d ** -0.5
    out = np.zeros(q.shape, np.float64)
    for s in range(len(lens_q)):
        qa, qb, ka, kb = cu_q[s], cu_q[s + 1], cu_k[s], cu_k[s + 1]
        if qb == qa:
            continue
        pos0 = int((kb - ka) - (qb - qa))
        out[qa:qb] = O.attention_f64(q[qa:qb], k[ka:kb], v[ka:kb], scale=scale, causal=causal,
                                     q_pos0=pos0, window_left=window_left, dtype=O.BF16)
        ref = torch_attention_f64(bf16_to_f32(q[qa:qb]), bf16_to_f32(k[ka:kb]),
                                  bf16_to_f32(v[ka:kb]), scale, q_pos0=pos0, causal=causal,
                                  window_left=window_left)
        assert np.abs(ref - out[qa:qb]).max() < 1e-12
    return dict(num_q_heads=np.int32(hq), causal=np.int32(causal),
                window_left=np.int32(window_left), scale=np.float64(scale),
                cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, q=q, k=k, v=v,
                out=out.astype(np.float32))  # float32 is far inside the bf16 tolerance


def rope_case(rng):
    t, h, d, rows = 6, 2, 64, 64
    x = rng.standard_normal((t, h, d), dtype=np.float32)
    pos = np.array([0, 1, 7, 31, 32, 63], np.int32)
    cos, sin = O.rope_caches(rows, d)
    return dict(x=x, positions=pos, rows=np.int32(rows), cos_full=cos, sin_full=sin,
                rotated=O.rope_apply(x, pos, cos, sin))


def polar_case(rng):
    d = 64
    rows = [rng.standard_normal(d, dtype=np.float32) * s for s in (1.0, 1e-3, 300.0)]
    one_hot = np.zeros(d, np.float32)
    one_hot[5] = -2.5
    halfway = np.tile(np.array([5, 11, -5, 5], np.float32), d // 4)
    rows += [np.zeros(d, np.float32), one_hot, halfway]
    x = np.stack(rows)
    rec = O.polar_compress(x)
    return dict(x=x, records=rec, decompressed=O.polar_decompress(rec, d))


def qjl_case(rng):
    """QJL at the reference test's shape (head_dim 32, proj_dim 8) and at 64 / 16: the fixed
    projection, the records and the decompressed rows (random, zero and one-hot vectors)."""
    out = {}
    for d, p in ((32, 8), (64, 16)):
        rows = [rng.standard_normal(d, dtype=np.float32) * s for s in (1.0, 1e-2, 50.0)]
        one_hot = np.zeros(d, np.float32)
        one_hot[3] = 1.0
        x = np.stack(rows + [np.zeros(d, np.float32), one_hot])
        proj = O.qjl_projection(p, d)
        rec = O.qjl_compress(x, proj)
        out.update({f"x{d}": x, f"proj{d}": proj, f"records{d}": rec,
                    f"decompressed{d}": O.qjl_decompress(rec, proj)})
    return out


def flash_f32_case(rng):
    """Dense f32 flash attention [1, 2, 40, 64] (the reference flash_attention's element type):
    non-causal, top-left causal, and with an additive [40, 40] mask; outputs from the f64 oracle,
    each checked against torch float64 SDPA."""
    h, s, d = 2, 40, 64
    q, k, v = (rng.standard_normal((s, h, d), dtype=np.float32) for _ in range(3))
    mask = (2.0 * rng.standard_normal((s, s))).astype(np.float32)
    mask[:, 33:] = -np.inf
    scale = d ** -0.5
    res = {}
    for name, causal, m in (("out_full", False, None), ("out_causal", True, None),
                            ("out_masked", False, mask)):
        o = O.attention_f64(q, k, v, scale=scale, causal=causal, q_pos0=0, mask=m, dtype=O.F32)
        if m is None:
            ref = torch_attention_f64(q, k, v, scale, q_pos0=0, causal=causal)
            assert np.abs(ref - o).max() < 1e-12
        else:
            import torch
            qt, kt, vt = (torch.from_numpy(a).double().transpose(0, 1) for a in (q, k, v))
            sc = qt @ kt.transpose(1, 2) * scale + torch.from_numpy(m).double()
            ref = (torch.softmax(sc, -1) @ vt).transpose(0, 1).numpy()
            assert np.abs(ref - o).max() < 1e-12
        res[name] = o
    return dict(q=q, k=k, v=v, mask=mask, scale=np.float64(scale), **res)


def kats() -> dict:
    """The reference's unit-test known answers, as data."""
    return {
        "block_table": {
            "source": "crates/sketchpad-core/src/paged_attention.rs:568-598",
            "block_size": 4,
            "table": [0, 5],
            "get_block": {"0": 0, "3": 0, "4": 5, "5": 5},
            "get_slot": {"0": 0, "3": 3, "4": 0, "5": 1},
            "needs_new_block": {"0": False, "4": True, "6": False},
        },
        "allocation": {
            "source": "crates/sketchpad-core/src/paged_attention.rs:601-620",
            "num_blocks": 10, "free_after_two_allocs": 8, "free_after_one_free": 9,
        },
        "scheduler": {
            "source": "crates/sketchpad-core/src/paged_attention.rs:623-645",
            "block_size": 4, "num_blocks": 10, "allocs": [3, 5],
            "free_after_allocs": 7, "free_after_freeing_first": 8,
        },
        "memory_budget": {
            "source": "crates/sketchpad-core/src/paged_attention.rs:648-661",
            "bytes": 1 << 30, "num_kv_heads": 8, "head_dim": 128, "num_layers": 32,
            "block_size": 16, "num_blocks": 256,
        },
        "gather_empty": {
            "source": "crates/sketchpad-core/src/paged_attention.rs:664-674",
            "num_kv_heads": 8, "head_dim": 64, "dims": [8, 0, 64],
        },
        "causal_mask": {
            "source": "crates/sketchpad-core/src/transformer.rs:524-536",
            "n": 4, "entries": {"0": 0.0, "1": "-inf", "2": "-inf", "4": 0.0, "5": 0.0},
        },
        "sliding_window_mask": {
            "source": "crates/sketchpad-core/src/transformer.rs:539-561",
            "n": 5, "window": 2,
            "entries": {"0": 0.0, "1": "-inf", "15": "-inf", "16": 0.0, "17": 0.0, "18": 0.0,
                        "20": "-inf", "21": "-inf", "22": 0.0, "23": 0.0, "24": 0.0},
        },
        "rope": {
            "source": "crates/sketchpad-core/src/rope.rs:180-230",
            "zeros_stay_zeros": {"head_dim": 32, "max_seq_len": 256, "offset": 100, "seq": 8},
            "ones_change": {"head_dim": 4, "max_seq_len": 16, "seq": 4, "min_change": 1e-6},
        },
    }


FIXTURES = {
    "decode_f32.npz": lambda rng: decode_case(rng, [1, 17, 40], 8, 2, 64, 16, "f32"),
    "decode_bf16_window.npz": lambda rng: decode_case(rng, [33, 70], 8, 2, 128, 16, "bf16",
                                                      window_left=40),
    "prefill_bf16.npz": lambda rng: prefill_case(rng, [5, 37, 0, 50], [5, 37, 0, 50], 4, 2, 64,
                                                 True),
    "prefill_bf16_chunked_window.npz": lambda rng: prefill_case(rng, [9, 20], [41, 20], 4, 2, 64,
                                                                True, window_left=16),
    "rope_f32.npz": rope_case,
    "polar_f32.npz": polar_case,
    "qjl_f32.npz": qjl_case,
    "flash_f32.npz": flash_f32_case,
}


# seed offsets: a fixture's position here (new fixtures go at the end, so existing ones keep theirs)
SEED_ORDER = ["decode_bf16_window.npz", "decode_f32.npz", "polar_f32.npz", "prefill_bf16.npz",
              "prefill_bf16_chunked_window.npz", "rope_f32.npz", "qjl_f32.npz", "flash_f32.npz"]


def build(name: str) -> dict:
    rng = np.random.default_rng(SEED + SEED_ORDER.index(name))
    return FIXTURES[name](rng)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true")
    args = ap.parse_args()
    bad = []
    for name in sorted(FIXTURES):
        data = build(name)
        path = HERE / name
        if args.check:
            old = np.load(path, allow_pickle=False)
            for key, val in data.items():
                if not np.array_equal(old[key], val):
                    bad.append(f"{name}:{key}")
        else:
            np.savez_compressed(path, **data)
    kat_path = HERE / "kats.json"
    if args.check:
        if json.loads(kat_path.read_text()) != kats():
            bad.append("kats.json")
    else:
        kat_path.write_text(json.dumps(kats(), indent=1) + "\n")
    if bad:
        raise SystemExit("fixtures differ: " + ", ".join(bad))
    print("ok" if args.check else f"wrote {len(FIXTURES) + 1} fixtures to {HERE}")


if __name__ == "__main__":
    main()
