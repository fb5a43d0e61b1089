"""A mixed ragged batch (prompt chunks + one-token decode sequences over one paged pool) through
sp_ragged_paged_attention, the entry point BatchedPagedAttention calls for every layer of a
scheduler iteration: at the full C4 size (Qwen2.5-7B heads) and on a small
batch with a window. Every decode row is checked against the oracle's paged decode (gather_kv
then softmax(q k^T d^-1/2) v with no mask, llama.rs:255-260), every chunk row against f64
attention over the gathered context with prefill_causal_mask (llama.rs:374-388), and both halves
bit for bit against the separate sp_paged_prefill / sp_paged_decode calls on the same data."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from sketchpad_amd import workloads as W
from tests.helpers import announce, as_f64, assert_attention_close, host_array, oracle_dtype

pytestmark = pytest.mark.gpu


def _run(w: W.MixedWorkload, window_left: int = -1, repeats: int = 1, softcap: float = 0.0,
         qscale: float = 1.0):
    t = W.make_mixed_tensors(w)
    if qscale != 1.0:
        t["q"].mul_(qscale)
    lay = sp.layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
    P, T0 = w.num_prefill_seqs, w.num_prefill_tokens
    pmax = int(w.chunk_lens.max()) if P else 0
    dmax = int(w.decode_lens.max()) if w.num_decode_seqs else 0
    mb = t["block_tables"].shape[1]
    ws = sp.alloc_ragged_workspace(w.num_seqs, P, pmax, dmax, w.hq, lay, mb, window_left)
    announce(f"ragged {w.name}: {P} chunks {list(w.chunk_lens)} on {list(w.ctx_before)}, "
             f"{w.num_decode_seqs} decode seqs, window {window_left}, softcap {softcap}")
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])
    scale = w.head_dim ** -0.5
    first = None
    for r in range(repeats):
        t["out"].fill_(float("nan"))
        sp.ragged_paged_attention(t["out"], t["q"], t["k_pool"], t["v_pool"], lay,
                                  t["block_tables"], t["cu_seqlens_q"], t["context_lens"],
                                  num_prefill_seqs=P, num_prefill_tokens=T0,
                                  prefill_max_seqlen_q=pmax, decode_max_context_len=dmax,
                                  scale=scale, window_left=window_left, workspace=ws,
                                  softcap=softcap)
        if r == 0:
            first = t["out"].clone()
        else:
            assert torch.equal(t["out"], first), f"call {r} differs from the first"
    # the same halves through their own entry points, each with the workspace it asks for
    if P:
        pre = torch.full_like(t["q"][:T0], float("nan"))
        pws = sp.alloc_paged_prefill_workspace(P, pmax, w.hq, lay, mb)
        sp.paged_prefill(pre, t["q"][:T0], t["k_pool"], t["v_pool"], lay, t["block_tables"][:P],
                         t["cu_seqlens_q"], t["context_lens"][:P], pmax, scale,
                         window_left=window_left, workspace=pws, softcap=softcap)
    if w.num_decode_seqs:
        dec = torch.full_like(t["q"][T0:], float("nan"))
        dws = sp.alloc_decode_workspace(w.num_decode_seqs, w.hq, dmax, window_left, lay)
        sp.paged_decode(dec, t["q"][T0:], t["k_pool"], t["v_pool"], lay, t["block_tables"][P:],
                        t["context_lens"][P:], dmax, scale, window_left=window_left,
                        workspace=dws, softcap=softcap)
    torch.cuda.synchronize()
    if P:
        assert torch.equal(t["out"][:T0], pre), "chunk rows differ from sp_paged_prefill"
    if w.num_decode_seqs:
        assert torch.equal(t["out"][T0:], dec), "decode rows differ from sp_paged_decode"

    olay = O.make_layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
    kp, vp, q = host_array(t["k_pool"]), host_array(t["v_pool"]), host_array(t["q"])
    tables = t["block_tables"].cpu().numpy()
    lens = w.context_lens
    got = as_f64(t["out"])
    odt = oracle_dtype(t["q"])
    # decode rows: every sequence, every head
    if w.num_decode_seqs:
        ref = O.paged_decode_f64(q[T0:], kp, vp, olay, tables[P:], lens[P:], scale=scale,
                                 window_left=window_left, dtype=odt, softcap=softcap)
        assert_attention_close(got[T0:], ref, w.dtype, f"{w.name} decode rows")
    # chunk rows: every row of every chunk (queries at positions L - lq .. L - 1)
    cu = w.cu_seqlens_q
    for s in range(P):
        L, lq = int(lens[s]), int(w.chunk_lens[s])
        kg, vg = O.gather_kv(kp, vp, olay, tables[s], L)
        kt = np.ascontiguousarray(kg.transpose(1, 0, 2))
        vt = np.ascontiguousarray(vg.transpose(1, 0, 2))
        r = O.attention_f64(q[cu[s]:cu[s] + lq], kt, vt, scale=scale, causal=True,
                            q_pos0=L - lq, window_left=window_left, dtype=odt, softcap=softcap)
        assert_attention_close(got[cu[s]:cu[s] + lq], r, w.dtype, f"{w.name} chunk {s}")


def test_ragged_c4_mixed_full_size():
    """C4: 4 chunks x 512 new tokens on contexts U[1024, 8192] + 128 decode sequences with
    contexts U[256, 4096], one pool; every decode row and every chunk row."""
    _run(W.mixed_c4())


@pytest.mark.parametrize("window", [-1, 100])
def test_ragged_small_mixed(window):
    w = W.MixedWorkload("mixed-small", 77, np.array([33, 2, 130], np.int32),
                        np.array([0, 500, 40], np.int32),
                        np.array([1, 17, 300, 64, 129], np.int32), 8, 2, 128, "bf16")
    _run(w, window_left=window)


def test_ragged_split_prefill_with_decode():
    """A short chunk on a long context splits its key walk (partials in the back of the
    workspace) while the decode half's partials take the front: both halves through one call,
    three calls in a row giving the same bits."""
    w = W.MixedWorkload("mixed-split", 80, np.array([64, 100], np.int32),
                        np.array([4000, 2500], np.int32),
                        np.array([3000, 17, 1500, 640, 2049, 1], np.int32), 8, 2, 128, "bf16")
    t_lay = sp.layout(4096, 1, 0, w.hkv, w.block_size, w.head_dim)
    mb = int(-(-int(w.context_lens.max()) // w.block_size))
    assert sp.paged_prefill_workspace_size(2, 100, w.hq, t_lay, mb) > 0, "the plan must split"
    _run(w, repeats=3)


@pytest.mark.parametrize("seed", range(8))
def test_ragged_random_batches(seed):
    """Seeded random mixed batches: 0-4 chunks of 1-300 new tokens on 0-3000 cached tokens,
    0-12 one-token sequences of 1-2500 tokens, GQA groups 1-8, head_dim 64 / 128, block size
    16 / 32, with and without a window; every row against the oracle and each half bit for bit
    against its own entry point."""
    rng = np.random.default_rng(1000 + seed)
    n_chunks = int(rng.integers(0, 5))
    n_dec = int(rng.integers(0 if n_chunks else 1, 13))
    hkv = int(rng.choice([1, 2, 4]))
    group = int(rng.choice([1, 2, 4, 7, 8]))
    d = int(rng.choice([64, 128]))
    bs = int(rng.choice([16, 32]))
    chunks = rng.integers(1, 301, n_chunks).astype(np.int32)
    ctx = rng.integers(0, 3001, n_chunks).astype(np.int32)
    dec = rng.integers(1, 2501, n_dec).astype(np.int32)
    window = int(rng.choice([-1, int(rng.integers(0, 600))]))
    w = W.MixedWorkload(f"mixed-random-{seed}", 2000 + seed, chunks, ctx, dec, hkv * group, hkv,
                        d, "bf16", block_size=bs)
    _run(w, window_left=window)


def test_ragged_decode_only_and_prefill_only():
    """The two degenerate batches: no chunks (decode alone) and no decode sequences."""
    only_dec = W.MixedWorkload("mixed-decode-only", 78, np.zeros(0, np.int32),
                               np.zeros(0, np.int32), np.array([5, 40, 200], np.int32),
                               8, 2, 64, "bf16")
    _run(only_dec)
    only_pre = W.MixedWorkload("mixed-prefill-only", 79, np.array([7, 64], np.int32),
                               np.array([10, 0], np.int32), np.zeros(0, np.int32),
                               8, 2, 64, "bf16")
    _run(only_pre)


@pytest.mark.parametrize("d,softcap", [(128, 0.0), (256, 50.0), (512, 50.0)])
def test_ragged_mixed_graph_capture(d, softcap):
    """The mixed step's fork / join (decode on the library's side stream) captured into a HIP
    graph through torch: four replays, each after eager work that overwrites the output, each
    bit-identical to the eager call. Also at head dims 256 and 512 with Gemma-4's logit soft cap
    (sp_ragged_paged_attention_softcap)."""
    w = W.MixedWorkload("mixed-graph", 81, np.array([64, 100], np.int32),
                        np.array([4000, 300], np.int32),
                        np.array([3000, 17, 1500, 640], np.int32), 8, 2, d, "bf16")
    t = W.make_mixed_tensors(w)
    if softcap:
        t["q"].mul_(8.0)  # logits that reach the cap
    lay = sp.layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
    P, T0 = w.num_prefill_seqs, w.num_prefill_tokens
    pmax, dmax = int(w.chunk_lens.max()), int(w.decode_lens.max())
    mb = t["block_tables"].shape[1]
    ws = sp.alloc_ragged_workspace(w.num_seqs, P, pmax, dmax, w.hq, lay, mb)
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])

    def call(stream):
        sp.ragged_paged_attention(t["out"], t["q"], t["k_pool"], t["v_pool"], lay,
                                  t["block_tables"], t["cu_seqlens_q"], t["context_lens"],
                                  num_prefill_seqs=P, num_prefill_tokens=T0,
                                  prefill_max_seqlen_q=pmax, decode_max_context_len=dmax,
                                  scale=w.head_dim ** -0.5, workspace=ws, softcap=softcap,
                                  stream=stream)

    announce(f"ragged mixed step under graph capture, D={d}, softcap={softcap}")
    call(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = t["out"].clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call(s.cuda_stream)
    torch.cuda.current_stream().wait_stream(s)
    for r in range(4):
        t["out"].fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(t["out"], eager), f"replay {r} differs from the eager call"


def test_ragged_mixed_from_two_host_threads():
    """Two host threads issue mixed steps on their own streams, with their own buffers, at the
    same time (each caller stream has its own side stream and events): every output is
    bit-identical to the same call made alone."""
    import threading
    w = W.MixedWorkload("mixed-threads", 82, np.array([64, 100], np.int32),
                        np.array([2000, 300], np.int32),
                        np.array([3000, 17, 1500, 640], np.int32), 8, 2, 128, "bf16")
    runs = []
    for _ in range(2):
        t = W.make_mixed_tensors(w)
        lay = sp.layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
        P, T0 = w.num_prefill_seqs, w.num_prefill_tokens
        pmax, dmax = int(w.chunk_lens.max()), int(w.decode_lens.max())
        ws = sp.alloc_ragged_workspace(w.num_seqs, P, pmax, dmax, w.hq, lay,
                                       t["block_tables"].shape[1])
        sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])
        runs.append((t, lay, ws, torch.cuda.Stream()))
    torch.cuda.synchronize()

    def call(r):
        t, lay, ws, st = r
        sp.ragged_paged_attention(t["out"], t["q"], t["k_pool"], t["v_pool"], lay,
                                  t["block_tables"], t["cu_seqlens_q"], t["context_lens"],
                                  num_prefill_seqs=w.num_prefill_seqs,
                                  num_prefill_tokens=w.num_prefill_tokens,
                                  prefill_max_seqlen_q=int(w.chunk_lens.max()),
                                  decode_max_context_len=int(w.decode_lens.max()),
                                  scale=w.head_dim ** -0.5, workspace=ws, stream=st.cuda_stream)

    announce("ragged mixed steps from two host threads")
    call(runs[0])
    torch.cuda.synchronize()
    alone = runs[0][0]["out"].clone()
    errors = []

    def worker(r, n):
        try:
            for _ in range(n):
                call(r)
        except Exception as e:  # surfaced below
            errors.append(e)

    for _ in range(3):
        for r in runs:
            r[0]["out"].fill_(float("nan"))
        torch.cuda.synchronize()
        th = [threading.Thread(target=worker, args=(r, 20)) for r in runs]
        for x in th:
            x.start()
        for x in th:
            x.join()
        torch.cuda.synchronize()
        assert not errors, errors
        for r in runs:
            assert torch.equal(r[0]["out"], alone), "a concurrent call differs from the call alone"



_INDEPENDENCE_CHILD = r'''
import sys, time
sys.path.insert(0, sys.argv[1])
import numpy as np, torch
import sketchpad_amd as sp
from sketchpad_amd import workloads as W
w = W.MixedWorkload("mixed-streams", 83, np.array([64, 100], np.int32),
                    np.array([2000, 300], np.int32),
                    np.array([3000, 17, 1500, 640], np.int32), 8, 2, 128, "bf16")
runs = []
for _ in range(2):
    t = W.make_mixed_tensors(w)
    lay = sp.layout(t["num_blocks"], 1, 0, w.hkv, w.block_size, w.head_dim)
    ws = sp.alloc_ragged_workspace(w.num_seqs, w.num_prefill_seqs, int(w.chunk_lens.max()),
                                   int(w.decode_lens.max()), w.hq, lay, t["block_tables"].shape[1])
    sp.kv_append(t["k_pool"], t["v_pool"], lay, t["k_new"], t["v_new"], t["slot_mapping"])
    runs.append((t, lay, ws, torch.cuda.Stream()))
def call(r):
    t, lay, ws, st = r
    sp.ragged_paged_attention(t["out"], t["q"], t["k_pool"], t["v_pool"], lay, t["block_tables"],
                              t["cu_seqlens_q"], t["context_lens"],
                              num_prefill_seqs=w.num_prefill_seqs,
                              num_prefill_tokens=w.num_prefill_tokens,
                              prefill_max_seqlen_q=int(w.chunk_lens.max()),
                              decode_max_context_len=int(w.decode_lens.max()),
                              scale=w.head_dim ** -0.5, workspace=ws, stream=st.cuda_stream)
for r in runs:  # first calls make each caller stream's side stream
    call(r)
torch.cuda.synchronize()
alone = runs[1][0]["out"].clone()
sa, sb = runs[0][3], runs[1][3]
# calibrate a spin kernel of about 200 ms on stream A
e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
with torch.cuda.stream(sa):
    e0.record(); torch.cuda._sleep(1 << 22); e1.record()
torch.cuda.synchronize()
cycles = int((1 << 22) * 200.0 / max(e0.elapsed_time(e1), 1e-3))
with torch.cuda.stream(sa):
    e0.record(); torch.cuda._sleep(cycles); e1.record()
call(runs[0])  # A's mixed step waits behind the spin kernel on its stream
b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
runs[1][0]["out"].fill_(float("nan"))
with torch.cuda.stream(sb):
    b0.record()
call(runs[1])  # B's, enqueued after A's, on its own caller stream
with torch.cuda.stream(sb):
    b1.record()
torch.cuda.synchronize()
same = bool(torch.equal(runs[1][0]["out"], alone))
print(f"RESULT spin_ms={e0.elapsed_time(e1):.3f} b_ms={b0.elapsed_time(b1):.3f} same={same}",
      flush=True)
'''


def test_ragged_mixed_steps_on_two_streams_do_not_wait_for_each_other():
    """Each caller stream forks to a side stream of its own: stream A holds a ~200 ms spin kernel
    ahead of its mixed step, and stream B's mixed step, enqueued after A's, completes in its own
    time. (With one side stream shared by both callers, B's decode half would queue behind A's,
    which waits for the spin kernel.) Run in a child process with eight hardware queues, so that
    the four streams involved do not share one."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parent.parent)
    announce("ragged mixed steps on two caller streams: independence (child process)")
    env = dict(os.environ, GPU_MAX_HW_QUEUES="8")
    proc = subprocess.run([sys.executable, "-c", _INDEPENDENCE_CHILD, root], env=env,
                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=240)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout
    line = [x for x in proc.stdout.splitlines() if x.startswith("RESULT")][-1]
    vals = dict(kv.split("=") for kv in line.split()[1:])
    spin, b = float(vals["spin_ms"]), float(vals["b_ms"])
    assert vals["same"] == "True", "stream B's output differs from the call alone"
    assert spin > 50.0, f"the spin kernel took only {spin} ms"
    assert b < spin / 4, f"stream B's mixed step took {b} ms behind A's {spin} ms spin kernel"
