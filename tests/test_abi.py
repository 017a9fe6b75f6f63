"""The C ABI library: it loads, exports every function include/q38_attn.h
declares, and fails cleanly (-1 with a message) on bad input before touching a
device.  CPU only: no kernel is launched."""
import ctypes
import os

import numpy as np
import pytest


def test_library_exports_every_declared_function(pkg):
    lib = pkg.lib()
    names = pkg.header_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_function(pkg):
    assert sorted(pkg._SIGNATURES) == pkg.header_functions()


def test_code_objects_are_built_for_gfx950(pkg):
    for name in ("attn_decode", "attn_prefill", "gdn", "gdn_chunk", "proj", "synth"):
        path = os.path.join(pkg.LIB_DIR, name + ".hsaco")
        assert os.path.exists(path), path
        with open(path, "rb") as f:
            blob = f.read()
        # an ELF code object or a clang offload bundle holding one
        assert blob[:4] == b"\x7fELF" or blob.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
        assert b"gfx950" in blob


def test_null_and_bad_arguments_fail_cleanly(pkg):
    lib = pkg.lib()
    assert lib.q38_ctx_create(None, 0, None) == -1
    assert b"NULL" in lib.q38_last_error()
    assert lib.q38_sync(None) == -1
    assert lib.q38_kv_create(None, 17, 1, 1, 1, None) == -1
    assert lib.q38_attn_decode(None, 3, 1, None, None, None, None, None, None, None) == -1
    assert lib.q38_gdn_step(None, 1, None, 0, None, None, None, None, None, None) == -1
    assert lib.q38_seq_create(None, None) == -1
    # zero-length work is a successful no-op even without a context
    assert lib.q38_gdn_step(None, 0, None, 0, None, None, None, None, None, None) == -1  # ctx checked first


def test_no_device_is_reported(pkg):
    if pkg.device_count() > 0:
        pytest.skip("a device is present")
    with pytest.raises(pkg.Q38Error, match="no HIP device"):
        pkg.Context(0)


def test_kargs_layout_matches_device_expectations():
    """The argument blocks travel by value; their sizes must stay below the
    4 KiB kernarg limit.  Checked by compiling a sizeof probe with the host
    compiler."""
    import subprocess
    import tempfile
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    hdr = os.path.join(root, "qwen3.8_27b_in_rust_amd", "csrc", "q38_kargs.h")
    src = f'#include "{hdr}"\n#include <stdio.h>\nint main(){{printf("%zu %zu %zu\\n", sizeof(q38_decode_args), sizeof(q38_gdn_pre_args), sizeof(q38_gdn_args));return 0;}}\n'
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "p.c")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-o", os.path.join(d, "p"), c], check=True)
        out = subprocess.run([os.path.join(d, "p")], capture_output=True, text=True, check=True).stdout
    sizes = [int(x) for x in out.split()]
    assert all(s < 4096 for s in sizes), sizes


def test_noalloc_scratch_size_matches_header(pkg):
    import re
    text = open(os.path.join(pkg.INCLUDE_DIR, "q38_attn.h")).read()
    m = re.search(r"#define Q38_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == pkg.NOALLOC_SCRATCH_BYTES
