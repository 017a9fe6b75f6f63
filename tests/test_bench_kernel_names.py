"""Every kernel name bench.py hands to q38_kernel_timer_start is one the
library's lookup accepts (CPU only: the lookup's names are read from its
source), so that no measurement fails on an unknown name at run time."""
import os
import re

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "qwen3.8_27b_in_rust_amd", "csrc", "host", "q38_attn.cpp")


def _timer_names():
    src = open(HOST).read()
    body = src[src.index("int q38_kernel_timer_start("):]
    body = body[:body.index("\n}\n")]
    names = set(re.findall(r'name == "(q38_[a-z0-9_]+)"', body))
    table = src[src.index("constexpr GemvType kGemv[] = {"):]
    table = table[:table.index("};")]
    names |= set(re.findall(r'"(q38_[a-z0-9_]+)"', table))
    return names


def _accepts(names, name):
    return name in names


def test_bench_timer_names_are_known():
    names = _timer_names()
    used = {bench.DECODE_KERNEL, "q38_attn_decode_merge", "q38_gdn_step_rows", "q38_noop", "q38_gdn_decode",
            "q38_attn_prefill_mfma", "q38_prefill_merge", "q38_kv_split_mfma", "q38_attn_decode_split_many",
            "q38_gdn_pre", "q38_gdn_post", "q38_copy_f32"}
    for ty in bench.GEMV_KERNELS:
        used.update(bench._q8k_kernels(ty))
    for ty in bench.F32_PATH_TYPES:
        used.update(bench._f32_path_kernels(ty))
    unknown = sorted(n for n in used if not _accepts(names, n))
    assert not unknown, unknown


def test_bench_literal_kernel_names_are_known():
    """Every literal "q38_..." kernel name passed to kernel_timer_start in
    bench.py."""
    names = _timer_names()
    src = open(os.path.join(ROOT, "bench.py")).read()
    lits = set(re.findall(r'kernel_timer_start\("(q38_[a-z0-9_]+)"', src))
    for tup in re.findall(r'for name in \(([^)]*)\)', src):
        lits |= set(re.findall(r'"(q38_[a-z0-9_]+)"', tup))
    assert lits, "no literal names found"
    assert not sorted(n for n in lits if not _accepts(names, n))
