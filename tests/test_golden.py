"""The committed golden fixtures (tests/golden/) against the CPU oracle and the reference's own
known answers (kats.json, each entry citing its reference test). No GPU.

The fixtures freeze the oracle's results on small seeded inputs; this file checks that the
oracle still reproduces them bit for bit, that the frozen attention outputs agree with an
independent float64 computation (torch SDPA), and that the oracle meets every known answer the
reference's unit tests hold for this path."""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from tests.golden import gen_fixtures as G

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLDEN / name, allow_pickle=False)


@pytest.mark.parametrize("name", sorted(G.FIXTURES))
def test_fixture_reproduced_by_oracle(name):
    """Regenerating from the seed gives the committed arrays exactly."""
    old = _load(name)
    new = G.build(name)
    assert sorted(old.files) == sorted(new)
    for key, val in new.items():
        assert np.array_equal(old[key], val), f"{name}:{key}"


def test_kats_file_matches_generator():
    assert json.loads((GOLDEN / "kats.json").read_text()) == G.kats()


@pytest.mark.parametrize("name", ["decode_f32.npz", "decode_bf16_window.npz"])
def test_decode_fixture_independent(name):
    """Expected decode rows = float64 SDPA over the fixture's pool after the append, gathered
    with plain numpy indexing (no oracle call)."""
    f = _load(name)
    bf16 = str(f["dtype"]) == "bf16"
    val = (lambda a: G.bf16_to_f32(a)) if bf16 else (lambda a: a)
    kp, vp = val(f["k_pool"]).copy(), val(f["v_pool"]).copy()
    bs = int(f["block_size"])
    for s, slot in enumerate(f["slot_mapping"]):
        blk, off = divmod(int(slot), bs)
        kp[blk, 0, :, off] = val(f["k_new"])[s]
        vp[blk, 0, :, off] = val(f["v_new"])[s]
    store = G.bf16_bits if bf16 else (lambda a: a)
    assert G.sha256(store(kp)) == str(f["k_pool_after_sha256"])
    assert G.sha256(store(vp)) == str(f["v_pool_after_sha256"])
    q = val(f["q"])
    for s, L in enumerate(f["context_lens"]):
        L = int(L)
        pos = np.arange(L)
        rows = f["block_tables"][s][pos // bs], pos % bs
        k = kp[rows[0], 0, :, rows[1]]          # [L, Hkv, D]
        v = vp[rows[0], 0, :, rows[1]]
        ref = G.torch_attention_f64(q[s:s + 1], k, v, float(f["scale"]), q_pos0=L - 1,
                                    causal=True, window_left=int(f["window_left"]))
        assert np.abs(ref[0] - f["out"][s]).max() < 1e-12


@pytest.mark.parametrize("name", ["prefill_bf16.npz", "prefill_bf16_chunked_window.npz"])
def test_prefill_fixture_independent(name):
    f = _load(name)
    cu_q, cu_k = f["cu_seqlens_q"], f["cu_seqlens_k"]
    q, k, v = (G.bf16_to_f32(f[x]) for x in ("q", "k", "v"))
    for s in range(len(cu_q) - 1):
        qa, qb, ka, kb = cu_q[s], cu_q[s + 1], cu_k[s], cu_k[s + 1]
        if qb == qa:
            continue
        ref = G.torch_attention_f64(q[qa:qb], k[ka:kb], v[ka:kb], float(f["scale"]),
                                    q_pos0=int((kb - ka) - (qb - qa)), causal=bool(f["causal"]),
                                    window_left=int(f["window_left"]))
        assert np.abs(ref - f["out"][qa:qb]).max() < 1e-6


def test_rope_fixture_independent():
    """Rotated pairs = complex multiplication by e^{i p theta_j} in float64, within f32
    rounding; the caches hold each pair's value twice."""
    f = _load("rope_f32.npz")
    d = f["x"].shape[-1]
    theta = 10000.0 ** (-np.arange(0, d, 2, dtype=np.float64) / d)
    ang = f["positions"][:, None].astype(np.float64) * theta[None, :]       # [T, D/2]
    z = f["x"][..., 0::2].astype(np.float64) + 1j * f["x"][..., 1::2]
    r = z * np.exp(1j * ang)[:, None, :]
    assert np.abs(f["rotated"][..., 0::2] - r.real).max() < 1e-5
    assert np.abs(f["rotated"][..., 1::2] - r.imag).max() < 1e-5
    assert np.array_equal(f["cos_full"][:, 0::2], f["cos_full"][:, 1::2])
    assert np.array_equal(f["rotated"][0], f["x"][0])  # position 0 is the identity


def test_polar_fixture_independent():
    """Each record: binary16 norm (numpy's float16 rounding) then codes that decode within
    |x|/14 of x plus the norm's rounding; the zero row is all zeros."""
    f = _load("polar_f32.npz")
    x, rec, dec = f["x"], f["records"], f["decompressed"]
    d = x.shape[-1]
    for i in range(len(x)):
        n = np.sqrt(np.sum(x[i].astype(np.float64) ** 2))
        norm16 = rec[i, :2].view(np.float16)[0]
        assert norm16 == np.float16(np.float32(n)) or abs(float(norm16) - n) <= abs(n) * 2 ** -10
        bound = n / 14 + abs(float(norm16) - n) / 7 * 8 + 1e-6
        assert np.abs(dec[i] - x[i]).max() <= bound
    assert not rec[3].any() and not dec[3].any()
    assert rec.shape[-1] == 2 + d // 2


# ---------------------------------------------------------------------------------------------
# the reference's known answers (kats.json) against the oracle
# ---------------------------------------------------------------------------------------------

KATS = json.loads((GOLDEN / "kats.json").read_text())


def _f(x):
    return -np.inf if x == "-inf" else float(x)


def test_qjl_fixture_independent():
    """QJL records: magnitude bytes are binary16 of the float64 norm (within its rounding), the
    one-hot row's sign bits are the signs of its projection column, the zero row is all zeros,
    and the frozen projection has the N(0, 1/P) scale."""
    f = _load("qjl_f32.npz")
    for d, p in ((32, 8), (64, 16)):
        x, proj, rec = f[f"x{d}"], f[f"proj{d}"], f[f"records{d}"]
        assert rec.shape == (len(x), 2 + (p + 7) // 8)
        assert abs(proj.std() - p ** -0.5) < 0.25 * p ** -0.5
        for i, row in enumerate(x):
            m = O.f16_bits_to_f32(int(rec[i, 0]) | (int(rec[i, 1]) << 8))
            n = np.linalg.norm(row.astype(np.float64))
            assert abs(m - n) <= max(n * 2 ** -10, 6e-8)
        assert not rec[3].any()
        bits = np.array([(rec[4, 2 + k // 8] >> (k % 8)) & 1 for k in range(p)])
        assert np.array_equal(bits, (proj[:, 3] >= 0).astype(int))


def test_flash_f32_fixture_independent():
    """The frozen f32 flash outputs against a float64 softmax computed here with numpy."""
    f = _load("flash_f32.npz")
    q, k, v, mask = (f[n].astype(np.float64) for n in ("q", "k", "v", "mask"))
    s_, h, d = q.shape
    for name, causal, m in (("out_full", False, None), ("out_causal", True, None),
                            ("out_masked", False, mask)):
        sc = np.einsum("ihd,jhd->hij", q, k) * d ** -0.5
        if causal:
            sc = sc + np.where(np.arange(s_)[None, :] > np.arange(s_)[:, None], -np.inf, 0.0)
        if m is not None:
            sc = sc + m
        w = np.exp(sc - sc.max(-1, keepdims=True))
        ref = np.einsum("hij,jhd->ihd", w / w.sum(-1, keepdims=True), v)
        assert np.abs(ref - f[name]).max() < 1e-12


def test_kat_block_table():
    k = KATS["block_table"]
    for pos, blk in k["get_block"].items():
        assert O.get_block(k["table"], int(pos), k["block_size"]) == blk
    for pos, slot in k["get_slot"].items():
        assert O.get_slot(int(pos), k["block_size"]) == slot
    for n, need in k["needs_new_block"].items():
        assert O.needs_new_block(int(n), k["block_size"]) == need


def test_kat_scheduler_and_budget():
    k = KATS["scheduler"]
    used = sum(O.blocks_needed(n, k["block_size"]) for n in k["allocs"])
    assert k["num_blocks"] - used == k["free_after_allocs"]
    assert k["free_after_allocs"] + O.blocks_needed(k["allocs"][0], k["block_size"]) == \
        k["free_after_freeing_first"]
    b = KATS["memory_budget"]
    assert O.blocks_from_memory_budget(b["bytes"], b["num_kv_heads"], b["head_dim"],
                                       b["num_layers"], b["block_size"]) == b["num_blocks"]


def test_kat_gather_empty():
    k = KATS["gather_empty"]
    lay = O.make_layout(4, 1, 0, k["num_kv_heads"], 4, k["head_dim"])
    pool = np.zeros((4, 1, k["num_kv_heads"], 4, k["head_dim"]), np.float32)
    ko, vo = O.gather_kv(pool, pool.copy(), lay, [], 0)
    assert list(ko.shape) == k["dims"] and list(vo.shape) == k["dims"]


def test_kat_masks():
    k = KATS["causal_mask"]
    m = O.causal_mask(k["n"]).ravel()
    for i, val in k["entries"].items():
        assert m[int(i)] == _f(val)
    k = KATS["sliding_window_mask"]
    m = O.sliding_window_mask(k["n"], k["window"]).ravel()
    for i, val in k["entries"].items():
        assert m[int(i)] == _f(val)


def test_kat_rope():
    k = KATS["rope"]["zeros_stay_zeros"]
    cos, sin = O.rope_caches(k["max_seq_len"], k["head_dim"])
    x = np.zeros((k["seq"], 4, k["head_dim"]), np.float32)
    pos = np.arange(k["seq"], dtype=np.int32) + k["offset"]
    assert not O.rope_apply(x, pos, cos, sin).any()
    k = KATS["rope"]["ones_change"]
    cos, sin = O.rope_caches(k["max_seq_len"], k["head_dim"])
    x = np.ones((k["seq"], 1, k["head_dim"]), np.float32)
    y = O.rope_apply(x, np.arange(k["seq"], dtype=np.int32), cos, sin)
    assert (np.abs(y - x) > k["min_change"]).any()
