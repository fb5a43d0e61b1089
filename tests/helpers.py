"""Shared helpers for the GPU parity tests: host copies in the oracle's formats, tolerances."""
from __future__ import annotations

import sys

import numpy as np

# Output tolerances of the path: f32 within 1e-5 relative, measured per output row
# (one sequence x head vector) against the row's largest magnitude; 16-bit types within 2e-2
# absolute (fp32 softmax / accumulation, one final rounding to the storage type).
F32_REL_TOL = 1e-5
LOWP_ABS_TOL = 2e-2


def announce(msg: str) -> None:
    """Name the case before a GPU step so a fault can be attributed."""
    print(f"[gpu-case] {msg}", file=sys.stdout, flush=True)


def host_array(t) -> np.ndarray:
    """torch tensor -> numpy in the oracle's element formats (f32 stays f32, 16-bit -> bits)."""
    import torch
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.float32:
        return t.numpy()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def oracle_dtype(t) -> int:
    import torch
    from oracle import oracle as O
    return {torch.float32: O.F32, torch.bfloat16: O.BF16, torch.float16: O.F16}[t.dtype]


def as_f64(t) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_attention_close(got: np.ndarray, ref: np.ndarray, dtype_name: str, what: str = ""):
    """got/ref: [..., D] float64. f32: per-row relative; 16-bit: absolute."""
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref)
    if dtype_name == "f32":
        row_scale = np.maximum(np.abs(ref).max(axis=-1, keepdims=True), 1e-30)
        rel = (err / row_scale).max()
        assert rel <= F32_REL_TOL, f"{what}: f32 relative error {rel:.3e} > {F32_REL_TOL}"
    else:
        worst = err.max()
        assert worst <= LOWP_ABS_TOL, f"{what}: abs error {worst:.3e} > {LOWP_ABS_TOL}"
