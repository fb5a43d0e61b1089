"""Register, LDS and scratch budgets of every kernel in the built library, read from the gfx950
code objects' metadata (CPU only: the library is inspected, not loaded).

The kernels' occupancy is a design decision (three 32-key-tile prefill workgroups per CU, two for
the 64-key-tile and head-dim-256 prefills, four decode waves per SIMD at head dims 128 and 512,
...). The compiler holds the register count to a kernel's __launch_bounds__, but nothing holds
its static LDS to the same occupancy, and a private segment (scratch) appears silently when a
change spills. These tests pin all three on the library as built."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest
import yaml

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "sketchpad_amd" / "lib" / "libsketchpad_attn.so"
LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

LDS_PER_CU = 160 * 1024
VGPRS_PER_SIMD_LANE = 512   # unified architectural + accumulation file, wave64
VGPR_GRANULE = 8
MAX_WAVES_PER_SIMD = 8
SIMDS_PER_CU = 4


def _tools():
    tools = {"objcopy": shutil.which("objcopy"), "bundler": LLVM / "clang-offload-bundler",
             "readelf": LLVM / "llvm-readelf", "cxxfilt": shutil.which("c++filt")}
    missing = [k for k, v in tools.items() if v is None or not Path(v).exists()]
    if missing:
        pytest.skip(f"code-object tools missing: {missing}")
    if not LIB.exists():
        pytest.fail(f"{LIB} is missing: build it with `python -m sketchpad_amd.build`")
    return tools


def load_kernels(d: Path) -> dict:
    """name (demangled) -> metadata dict, over every code object bundled into the library;
    intermediate files go to the directory d."""
    t = _tools()
    fatbin = d / "fatbin.bin"
    # input and output both named: objcopy given one file rewrites it, here a library that
    # this test process (or another test in it) may have mapped
    subprocess.run([t["objcopy"], "-O", "binary", "--only-section=.hip_fatbin", str(LIB),
                    str(fatbin)], check=True)
    data = fatbin.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(BUNDLE_MAGIC), data)] + [len(data)]
    assert len(starts) > 1, "no offload bundle in .hip_fatbin"
    out = {}
    for i in range(len(starts) - 1):
        part, co = d / f"b{i}.bin", d / f"b{i}.o"
        part.write_bytes(data[starts[i]:starts[i + 1]])
        subprocess.run([str(t["bundler"]), "--unbundle", "--type=o", f"--targets={TARGET}",
                        f"--input={part}", f"--output={co}"], check=True)
        notes = subprocess.run([str(t["readelf"]), "--notes", str(co)], check=True,
                               capture_output=True, text=True).stdout
        doc = notes.split("---", 1)[1].split("\n...", 1)[0]
        for k in yaml.safe_load(doc)["amdhsa.kernels"]:
            name = subprocess.run([t["cxxfilt"]], input=k[".name"], capture_output=True,
                                  text=True, check=True).stdout.strip()
            out[name] = k
    return out


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    return load_kernels(tmp_path_factory.mktemp("co"))


def _waves_per_simd(k) -> int:
    regs = k[".vgpr_count"]
    if k.get(".agpr_count", 0):
        regs = -(-regs // 4) * 4 + k[".agpr_count"]
    regs = -(-regs // VGPR_GRANULE) * VGPR_GRANULE
    return min(MAX_WAVES_PER_SIMD, VGPRS_PER_SIMD_LANE // regs)


def _workgroups_per_cu(k) -> int:
    """Resident workgroups per CU that the registers allow (each wave sits on one SIMD)."""
    waves_per_wg = -(-k[".max_flat_workgroup_size"] // 64)
    return _waves_per_simd(k) * SIMDS_PER_CU // waves_per_wg


def _select(kernels, pattern):
    found = {n: k for n, k in kernels.items() if re.search(pattern, n)}
    assert found, f"no kernel matches {pattern!r}"
    return found


def test_every_path_has_its_kernels(kernels):
    for family in ["kv_append_kernel", "kv_gather_kernel", "paged_decode_kernel",
                   "decode_combine_kernel", "prefill_kernel<", "prefill_k32_kernel",
                   "prefill_wide_kernel", "prefill_d512_kernel", "prefill_combine_kernel",
                   "prefill_f32_kernel", "rope_kv_append_kernel", "polar_append_kernel",
                   "polar_decode_kernel", "linear_kernel", "linear_big_kernel"]:
        _select(kernels, re.escape(family))


def test_no_scratch_except_the_paged_head_dim_256_prefill(kernels):
    """No kernel spills VGPRs to scratch, except the paged head-dim-256 prefill (at most 16 bytes:
    one store before the key loop, one load after it)."""
    for name, k in kernels.items():
        private = k[".private_segment_fixed_size"]
        if re.search(r"prefill_wide_kernel<[^,]+, 256, true", name):
            assert private <= 16 and k[".vgpr_spill_count"] <= 4, (name, private)
        else:
            assert private == 0 and k[".vgpr_spill_count"] == 0, (name, private)
        assert not k.get(".uses_dynamic_stack", False), name


def test_lds_never_lowers_register_occupancy(kernels):
    """The workgroups per CU that the registers allow also fit the 160 KiB of LDS."""
    for name, k in kernels.items():
        wgs = max(1, _workgroups_per_cu(k))
        lds = k[".group_segment_fixed_size"]
        assert lds * wgs <= LDS_PER_CU, (name, lds, wgs)


@pytest.mark.parametrize("pattern,wgs_per_cu,waves_per_simd", [
    (r"prefill_k32_kernel", 3, 3),                 # 32-key tiles, three workgroups per CU
    (r"prefill_kernel<sp::(bf|f)16_t, 128", 2, 2),  # 64-key tiles, two per CU
    (r"prefill_wide_kernel<", 2, 2),              # head dim 256
    (r"prefill_d512_kernel<", 1, 2),              # head dim 512: eight waves, one per CU
    (r"paged_decode_kernel<sp::(bf|f)16_t, 128, false", 4, 4),
    (r"paged_decode_kernel<sp::(bf|f)16_t, 256", 2, 2),
    (r"paged_decode_kernel<sp::(bf|f)16_t, 512, false", 4, 4),
    (r"paged_decode_kernel<sp::(bf|f)16_t, 512, true", 3, 3),
    (r"polar_decode_kernel<", 4, 4),
])
def test_documented_occupancy(kernels, pattern, wgs_per_cu, waves_per_simd):
    for name, k in _select(kernels, pattern).items():
        assert _waves_per_simd(k) >= waves_per_simd, (name, k[".vgpr_count"])
        assert _workgroups_per_cu(k) >= wgs_per_cu, name
        assert k[".group_segment_fixed_size"] * wgs_per_cu <= LDS_PER_CU, name
