"""GPU parity of the QJL codec (KvQuantMethod::QJL, kv_cache.rs:534-617) against the oracle:
records and decompressed values bit for bit (f32, bf16, f16 inputs; f32 output, 16-bit outputs
as the f32 value rounded once), over head_dim / proj_dim shapes including odd ones and the
reference's default proj_dim = head_dim / 4, with zero, one-hot and sign-tie rows."""
import numpy as np
import pytest
import torch

import sketchpad_amd as sp
from oracle import oracle as O
from tests.helpers import announce

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _case(n, d, p, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, d, generator=g).to(DT[dtype])
    x[0] = 0.0                      # zero vector: magnitude 0, no sign bits
    x[1] = 0.0
    x[1, d // 2] = 1.0              # one-hot
    x[2] = x[3]                     # duplicate rows give duplicate records
    return x


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("d,p", [(32, 8), (64, 16), (128, 32), (128, 128), (37, 100), (16, 65)])
def test_qjl_compress_decompress_bit_exact(dtype, d, p):
    announce(f"qjl d={d} p={p} {dtype}")
    n = 300
    x = _case(n, d, p, dtype, seed=d * 7 + p)
    proj = sp.qjl_projection(p, d)
    assert np.array_equal(proj.cpu().numpy().view(np.uint32),
                          O.qjl_projection(p, d).view(np.uint32))
    xd = x.cuda()
    rec = torch.empty(n, sp.qjl_record_bytes(p), dtype=torch.uint8, device="cuda")
    sp.qjl_compress(rec, xd, proj)
    out32 = torch.empty(n, d, dtype=torch.float32, device="cuda")
    sp.qjl_decompress(out32, rec, proj)
    out16 = torch.empty(n, d, dtype=torch.bfloat16, device="cuda")
    sp.qjl_decompress(out16, rec, proj)
    torch.cuda.synchronize()
    R = O.qjl_projection(p, d)
    ref_rec = O.qjl_compress(x.float().numpy(), R)
    assert np.array_equal(rec.cpu().numpy(), ref_rec)
    ref_out = O.qjl_decompress(ref_rec, R)
    assert np.array_equal(out32.cpu().numpy().view(np.uint32), ref_out.view(np.uint32))
    assert torch.equal(out16.cpu(), torch.from_numpy(ref_out).to(torch.bfloat16))


def test_qjl_empty_and_validation():
    proj = sp.qjl_projection(8, 32)
    rec = torch.empty(0, 3, dtype=torch.uint8, device="cuda")
    sp.qjl_compress(rec, torch.empty(0, 32, device="cuda"), proj)  # no vectors: no work
    with pytest.raises(sp.SketchpadError):
        sp.qjl_compress(rec, torch.empty(4, 32, device="cuda"), proj[:0])
