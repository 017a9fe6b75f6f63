"""Register and scratch budgets of the projection kernels, from the device
assembly of csrc/kernels/proj.hip built with the Makefile's flags (CPU
only: hipcc compiles for gfx950 without a GPU).  The budgets are what the
measured forms rely on -- the number of waves a SIMD holds (512 registers
per lane: 168 or fewer for three, 256 or fewer for two) and no spills in the
GEMV -- so a change that silently moves a kernel across one of them fails
here rather than in a benchmark."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "qwen3.8_27b_in_rust_amd", "csrc")
HIPCC = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")

# held to three waves per SIMD by their launch attributes
THREE_WAVES = {"q6k", "iq4xs", "iq2xs", "iq2s", "iq3xxs"}


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "proj.s"
    flags = ["--offload-arch=gfx950", "--cuda-device-only", "-S", "-O3", "-std=c++17", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form",
             "-I" + os.path.join(CSRC, "kernels"), "-I" + CSRC]
    subprocess.run([HIPCC, *flags, "-o", str(out), os.path.join(CSRC, "kernels", "proj.hip")], check=True,
                   capture_output=True)
    text = out.read_text()
    res = {}
    for m in re.finditer(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", text, re.S):
        body = m.group(2)
        vgpr = int(re.search(r"\.amdhsa_next_free_vgpr (\d+)", body).group(1))
        scratch = int(re.search(r"\.amdhsa_private_segment_fixed_size (\d+)", body).group(1))
        res[m.group(1)] = (vgpr, scratch)
    assert res, "no kernels found in the assembly"
    return res


def test_gemv_kernels_do_not_spill(kernels):
    gemv = {k: v for k, v in kernels.items() if k.startswith("q38_gemv_q8k_")}
    assert len(gemv) == 14
    for name, (vgpr, scratch) in gemv.items():
        assert scratch == 0, (name, vgpr, scratch)
        assert vgpr <= 256, (name, vgpr)


def test_gemm_tiles_keep_two_or_three_waves(kernels):
    gemm = {k: v for k, v in kernels.items() if k.startswith("q38_gemm_q8k_")}
    assert len(gemm) == 14
    for name, (vgpr, scratch) in gemm.items():
        fmt = name[len("q38_gemm_q8k_"):]
        limit = 168 if fmt in THREE_WAVES else 256
        assert vgpr <= limit, (name, vgpr, limit)
        assert scratch <= 24, (name, scratch)


def test_split_block_gemm_fits_its_workgroups(kernels):
    """8-wave workgroups (512 threads) launch only at 256 registers or fewer,
    16-wave ones (1024 threads) at 128 or fewer; the 4-wave ones are held to
    256 so that two share a SIMD."""
    ks = {k: v for k, v in kernels.items() if k.startswith("q38_gemm_ks_q8k_")}
    ks16 = {k: v for k, v in kernels.items() if k.startswith("q38_gemm_ks16_q8k_")}
    ks4 = {k: v for k, v in kernels.items() if k.startswith("q38_gemm_ks4_q8k_")}
    assert len(ks) == 13 and len(ks16) == 13 and len(ks4) == 13
    for name, (vgpr, scratch) in {**ks, **ks4}.items():
        assert vgpr <= 256 and scratch == 0, (name, vgpr, scratch)
    for name, (vgpr, scratch) in ks16.items():
        assert vgpr <= 128 and scratch <= 48, (name, vgpr, scratch)


def test_f32_path_kernels_do_not_spill(kernels):
    """The f32-input path: the GEMV and the bf16 matrix-unit form (two
    workgroups per CU: at most 256 registers), no spills."""
    f32 = {k: v for k, v in kernels.items()
           if k.startswith(("q38_gemv_f32_", "q38_gemm_f32_", "q38_gemm_f32s_", "q38_gemm_f32w_"))}
    assert len(f32) == 18
    for name, (vgpr, scratch) in f32.items():
        assert scratch == 0 and vgpr <= 256, (name, vgpr, scratch)
