"""The GGUF reader (q38_gguf_open and the table accessors) against files
written from the published layout (tests/gguf_files.py): the accepted file's
alignment, data offset and tensor table, and every rejection the reference's
Gguf::open makes (src/gguf/mod.rs:347-532), each with its message.  Host-only:
no device is touched."""
import struct

import pytest

import gguf_files as gf


def _write(tmp_path, blob, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(blob)
    return str(p)


def _model_tensors():
    return [("blk.0.attn_q_norm.weight", 0, [256], gf.tensor_bytes(0, [256], 1)),
            ("blk.0.attn_qkv.weight", 12, [512, 3], gf.tensor_bytes(12, [512, 3], 2)),
            ("blk.0.ffn_down.weight", 14, [256, 2], gf.tensor_bytes(14, [256, 2], 3)),
            ("token_embd.weight", 8, [64, 5], gf.tensor_bytes(8, [64, 5], 4))]


META = [("general.architecture", gf.STRING, "qwen38"),
        ("qwen38.block_count", gf.U32, 64),
        ("tokenizer.ggml.tokens", gf.ARRAY, ["a", "bb", "ccc"], gf.STRING),
        ("tokenizer.ggml.token_type", gf.ARRAY, [1, 2, 3], gf.I32),
        ("qwen38.rope.freq_base", gf.F32, 1e7),
        ("general.flag", gf.BOOL, True)]


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_accepted_file_table(pkg, tmp_path, alignment):
    blob, offsets, data_offset = gf.build(_model_tensors(), META, alignment=alignment)
    with pkg.Gguf(_write(tmp_path, blob)) as g:
        info = g.info()
        assert info == {"version": 3, "alignment": alignment or 32, "data_offset": data_offset,
                        "n_tensors": 4, "n_metadata": len(META) + (alignment is not None)}
        assert info["data_offset"] % (alignment or 32) == 0
        for i, (name, ty, shape, data) in enumerate(_model_tensors()):
            t = g.tensor(i)
            assert t == {"name": name, "type": ty, "shape": shape, "offset": offsets[name][0],
                         "nbytes": len(data)}
            assert g.find_tensor(name) == i
            assert blob[data_offset + t["offset"]: data_offset + t["offset"] + t["nbytes"]] == data
        assert g.meta_u32("qwen38.block_count") == 64
        with pytest.raises(pkg.Q38Error, match="not a Uint32"):
            g.meta_u32("general.architecture")
        with pytest.raises(pkg.Q38Error, match="not found"):
            g.meta_u32("qwen38.context_length")
        with pytest.raises(pkg.Q38Error, match="not found"):
            g.find_tensor("output.weight")
        with pytest.raises(pkg.Q38Error, match="outside"):
            g.tensor(4)


def test_version_2_and_first_duplicate_wins(pkg, tmp_path):
    ts = _model_tensors()[:1] + [("blk.0.attn_q_norm.weight", 0, [256], gf.tensor_bytes(0, [256], 9))]
    blob, offsets, _ = gf.build(ts, version=2)
    with pkg.Gguf(_write(tmp_path, blob)) as g:
        assert g.info()["version"] == 2
        assert g.find_tensor("blk.0.attn_q_norm.weight") == 0


def test_alignment_of_another_type_is_ignored(pkg, tmp_path):
    """general.alignment counts only as a Uint32 (mod.rs:491-500)."""
    blob, _, data_offset = gf.build(_model_tensors(), [("general.alignment", gf.U64, 64)])
    with pkg.Gguf(_write(tmp_path, blob)) as g:
        assert g.info()["alignment"] == 32 and g.info()["data_offset"] == data_offset


def _header(n_tensors=1, n_meta=0, version=3, magic=b"GGUF"):
    return magic + struct.pack("<IQQ", version, n_tensors, n_meta)


def _tensor_info(name="t", dims=(256,), ty=0, offset=0):
    return gf.gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", ty, offset)


def _pad(blob, extra=0):
    n = (len(blob) + 31) // 32 * 32
    return blob + b"\0" * (n - len(blob) + extra)


REJECTIONS = [
    ("tiny", b"GGUF" + b"\0" * 19, "file smaller than 24 bytes"),
    ("magic", _pad(_header(magic=b"GGML") + _tensor_info(), 1024), "unsupported or corrupt GGUF header"),
    ("version 1", _pad(_header(version=1) + _tensor_info(), 1024), "unsupported or corrupt GGUF header"),
    ("version 4", _pad(_header(version=4) + _tensor_info(), 1024), "unsupported or corrupt GGUF header"),
    ("no tensors", _pad(_header(n_tensors=0) + b"\0" * 8), "unsupported or corrupt GGUF header"),
    ("key", _header(n_meta=1) + struct.pack("<Q", 1 << 40), "metadata key"),
    ("meta type", _header(n_meta=1) + gf.gstr("k") + struct.pack("<I", 13) + b"\0" * 16, "unknown meta type"),
    ("nested", _header(n_meta=1) + gf.gstr("k") + struct.pack("<II", gf.ARRAY, gf.ARRAY) + b"\0" * 16,
     "nested arrays not allowed"),
    ("array type", _header(n_meta=1) + gf.gstr("k") + struct.pack("<II", gf.ARRAY, 99) + b"\0" * 16,
     "unknown array type"),
    ("array value", _header(n_meta=1) + gf.gstr("k") + struct.pack("<IIQ", gf.ARRAY, gf.U32, 1 << 40),
     "array value"),
    ("meta string", _header(n_meta=1) + gf.gstr("k") + struct.pack("<IQ", gf.STRING, 1 << 40), "meta string"),
    ("scalar", _header(n_meta=1) + gf.gstr("k") + struct.pack("<I", gf.U64) + b"\0" * 2, "scalar value"),
    ("n_dims 0", _pad(_header() + _tensor_info(dims=()), 1024), "tensor n_dims"),
    ("n_dims 9", _pad(_header() + _tensor_info(dims=(1,) * 9), 1024), "tensor n_dims"),
    ("zero extent", _pad(_header() + _tensor_info(dims=(256, 0)), 1024), "tensor shape overflow"),
    ("extent overflow", _pad(_header() + _tensor_info(dims=(1 << 40, 1 << 40)), 1024), "tensor shape overflow"),
    ("tensor type", _pad(_header() + _tensor_info(ty=4), 1024), "unknown tensor type"),
    ("block", _pad(_header() + _tensor_info(dims=(100,), ty=12), 1024), "tensor bytes overflow"),
    ("outside", _pad(_header() + _tensor_info(dims=(256,), ty=0), 1000), "tensor outside GGUF file"),
    ("offset", _pad(_header() + _tensor_info(offset=(1 << 64) - 8), 1024), "tensor offset overflow"),
]


@pytest.mark.parametrize("case,blob,message", REJECTIONS, ids=[r[0] for r in REJECTIONS])
def test_rejections(pkg, tmp_path, case, blob, message):
    with pytest.raises(pkg.Q38Error, match="invalid GGUF: " + message):
        pkg.Gguf(_write(tmp_path, blob))


@pytest.mark.parametrize("alignment", [0, 48])
def test_rejects_bad_alignment(pkg, tmp_path, alignment):
    blob, _, _ = gf.build(_model_tensors(), alignment=32)
    # rewrite the general.alignment value in place
    key = gf.gstr("general.alignment") + struct.pack("<I", gf.U32)
    i = blob.index(key) + len(key)
    blob = blob[:i] + struct.pack("<I", alignment) + blob[i + 4:]
    with pytest.raises(pkg.Q38Error, match="invalid GGUF: invalid GGUF alignment"):
        pkg.Gguf(_write(tmp_path, blob))


def test_data_offset_past_end(pkg, tmp_path):
    """A table that ends short of the alignment boundary at the end of file."""
    blob = _header() + _tensor_info(dims=(1,), ty=0)  # 57 bytes; the data would start at 64
    assert len(blob) % 32 != 0
    with pytest.raises(pkg.Q38Error, match="invalid GGUF: tensor data begins past end of file"):
        pkg.Gguf(_write(tmp_path, blob))


def test_missing_file(pkg, tmp_path):
    with pytest.raises(pkg.Q38Error, match="I/O error"):
        pkg.Gguf(str(tmp_path / "absent.gguf"))


def test_mutated_files_are_accepted_or_rejected_cleanly(pkg, tmp_path):
    """2,000 seeded corruptions of valid files (byte flips, truncations,
    insertions, 0xFF runs): every open either succeeds, with a table whose
    accessors answer, or fails with an "invalid GGUF" / I/O message -- never
    a crash.  (The same mutations, 200,000 of them, ran clean under the host
    address and undefined-behaviour sanitizers.)"""
    import numpy as np

    seeds = [gf.build(_model_tensors(), META, alignment=al, version=v)[0] for al, v in ((None, 3), (64, 3), (32, 2))]
    rng = np.random.default_rng(0x51334F00)
    path = tmp_path / "fuzz.gguf"
    accepted = 0
    for it in range(2000):
        b = bytearray(seeds[it % len(seeds)])
        for _ in range(int(rng.integers(1, 9))):
            if not b:
                break
            at = int(rng.integers(0, len(b)))
            kind = int(rng.integers(0, 4))
            if kind == 0:
                b[at] = int(rng.integers(0, 256))
            elif kind == 1:
                del b[at:]
            elif kind == 2:
                b[at:at + 8] = b"\xff" * len(b[at:at + 8])
            else:
                b.insert(at, int(rng.integers(0, 256)))
        path.write_bytes(bytes(b))
        try:
            g = pkg.Gguf(str(path))
        except pkg.Q38Error as e:
            assert "invalid GGUF" in str(e) or "I/O error" in str(e), str(e)
            continue
        with g:
            accepted += 1
            info = g.info()
            for i in range(info["n_tensors"]):
                t = g.tensor(i)
                try:
                    assert g.find_tensor(t["name"]) <= i
                except pkg.Q38Error as e:  # a name cut at an embedded NUL byte
                    assert "not found" in str(e), str(e)
    assert 0 < accepted < 2000
