"""The prefill job planner (host logic of q38_attn_prefill) checked on the
CPU: tests/host/prefill_plan_check.cpp includes the library's source and
walks prompts of 1..4096 tokens after prefixes of 0..16,773,120 (coverage of
every job's key blocks, piece starts every row sees whole, dense unique
partial slots, table bounds)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


@pytest.mark.skipif(shutil.which("g++") is None or not os.path.isdir(os.path.join(ROCM, "include", "hip")),
                    reason="needs g++ and the HIP headers")
def test_prefill_planner(tmp_path):
    exe = tmp_path / "prefill_plan_check"
    csrc = os.path.join(HERE, "..", "qwen3.8_27b_in_rust_amd", "csrc")
    build = subprocess.run(["g++", "-O1", "-std=c++17", f"-I{ROCM}/include", f"-I{csrc}", "-o", str(exe),
                            os.path.join(HERE, "host", "prefill_plan_check.cpp"),
                            os.path.join(csrc, "host", "q38_gguf.cpp"),
                            f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-ldl"],
                           capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-2000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout[-2000:]
    assert "cases ok" in run.stdout
