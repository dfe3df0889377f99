"""GGUF v3 reader (sgq_gguf_*) on files written by tests/_gguf.py.

Template: crates/sg-gguf/src/parse.rs (tests of the tensor table, metadata
kinds, alignment and every malformed-input error).  Runs without a GPU: the
reader is host code."""
import struct

import numpy as np
import pytest

from _gguf import write_gguf

pytestmark = []


def _sample(tmp_path, **kw):
    rng = np.random.default_rng(1)
    q4 = rng.integers(0, 256, 18 * 6, dtype=np.uint8).tobytes()
    f32 = np.arange(64, dtype=np.float32).tobytes()
    meta = [("general.architecture", "str", "gemma4"), ("general.alignment", "u32", 64),
            ("gemma4.block_count", "u32", 62), ("gemma4.rope.freq_base", "f32", 1e6),
            ("gemma4.attention.sliding_window", "u64", 1024), ("x.neg", "i32", -7),
            ("x.flag", "bool", 1), ("x.list", "arr:i16", [1, -2, 3]), ("x.f64", "f64", 0.25)]
    tensors = [("blk.0.attn_q.weight", [64, 3], "Q4_0", q4),
               ("output_norm.weight", [64], "F32", f32)]
    p = tmp_path / "m.gguf"
    write_gguf(p, meta, tensors, alignment=64, **kw)
    return p, q4, f32


def test_gguf_reads_table_metadata_and_data(tmp_path):
    import sgq

    p, q4, f32 = _sample(tmp_path)
    g = sgq.Gguf(str(p))
    ts = g.tensors()
    assert [t.name for t in ts] == ["blk.0.attn_q.weight", "output_norm.weight"]
    q, n = ts
    assert (q.type, q.dims, q.nbytes) == (2, (64, 3), 108)
    assert (n.type, n.dims, n.nbytes) == (0, (64,), 256)
    assert q.offset % 64 == 0 and n.offset % 64 == 0
    assert g.data(q) == q4 and g.data(g.find("output_norm.weight")) == f32
    assert g.meta_string("general.architecture") == "gemma4"
    assert g.meta_int("gemma4.block_count") == 62
    assert g.meta_int("gemma4.attention.sliding_window") == 1024
    assert g.meta_int("x.neg") == -7 and g.meta_int("x.flag") == 1
    assert g.meta_float("gemma4.rope.freq_base") == 1e6 and g.meta_float("x.f64") == 0.25
    with pytest.raises(sgq.ValidationError):
        g.find("nope")
    with pytest.raises(sgq.ValidationError):
        g.meta_int("general.architecture")  # a string
    g.close()


@pytest.mark.parametrize("kw,msg", [
    (dict(magic=b"GGUX"), b"bad magic"),
    (dict(version=2), b"unsupported version"),
    (dict(truncate=40), b"truncated"),
    (dict(offsets=[0, 100]), b"not aligned"),
    (dict(offsets=[0, 1 << 20]), b"outside the data section"),
])
def test_gguf_rejects_malformed_files(tmp_path, kw, msg):
    import sgq

    p, _, _ = _sample(tmp_path, **kw)
    with pytest.raises(sgq.ValidationError):
        sgq.Gguf(str(p))
    assert msg in sgq.lib().sgq_last_error(), sgq.lib().sgq_last_error()


def test_gguf_rejects_bad_tensor_blocks_and_duplicates(tmp_path):
    import sgq

    p = tmp_path / "b.gguf"
    write_gguf(p, [], [("w", [33, 2], "Q4_0", b"\0" * 72)])  # 66 elements: not whole blocks
    with pytest.raises(sgq.ValidationError):
        sgq.Gguf(str(p))
    write_gguf(p, [], [("w", [32], "F32", b"\0" * 128), ("w", [32], "F32", b"\0" * 128)])
    with pytest.raises(sgq.ValidationError):
        sgq.Gguf(str(p))
    write_gguf(p, [("k", "u32", 1), ("k", "u32", 2)], [])
    with pytest.raises(sgq.ValidationError):
        sgq.Gguf(str(p))
    with pytest.raises(sgq.ValidationError):
        sgq.Gguf(str(tmp_path / "missing.gguf"))


def _nested(depth):
    """An array of arrays `depth` levels deep with one u8 at the bottom."""
    body = struct.pack("<IQ", 0, 1) + b"\x05"
    for _ in range(depth - 1):
        body = struct.pack("<IQ", 9, 1) + body
    return (9, body)


@pytest.mark.parametrize("meta,dims,msg", [
    ([("b", "raw", (7, b"\x02"))], [32], b"bool value"),
    ([("b", "arr:bool", [1, 0, 3])], [32], b"bool value"),
    ([("u", "raw", (13, b""))], [32], b"unknown value type"),
    ([("n", "raw", _nested(9))], [32], b"nested too deep"),
    ([("general.alignment", "u32", 24)], [32], b"alignment"),
    ([("general.alignment", "u32", 0)], [32], b"alignment"),
    ([("general.alignment", "str", "32")], [32], b"alignment"),
    ([], [2, 2, 2, 2, 2], b"dims"),
])
def test_gguf_rejects_bad_values(tmp_path, meta, dims, msg):
    """parse.rs error kinds: InvalidBool, UnknownValueType, ArrayTooDeep,
    BadAlignment, TooManyDims."""
    import sgq

    p = tmp_path / "v.gguf"
    write_gguf(p, meta, [("w", dims, "F32", b"\0" * 128)])
    with pytest.raises(sgq.ValidationError):
        sgq.Gguf(str(p))
    assert msg in sgq.lib().sgq_last_error(), sgq.lib().sgq_last_error()


def test_gguf_accepts_nesting_at_the_limit(tmp_path):
    import sgq

    p = tmp_path / "n.gguf"
    write_gguf(p, [("n", "raw", _nested(8)), ("k", "u16", 9)], [("w", [32], "F32", b"\0" * 128)])
    g = sgq.Gguf(str(p))
    assert g.meta_int("k") == 9 and g.find("w").dims == (32,)
    g.close()
