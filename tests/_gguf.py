"""A minimal GGUF v3 writer for tests (the public layout: header, metadata
key/values, tensor infos, aligned data section).  Test infrastructure only:
it builds files for the library's reader to parse."""
import struct

TYPES = {"u8": (0, "<B"), "i8": (1, "<b"), "u16": (2, "<H"), "i16": (3, "<h"), "u32": (4, "<I"),
         "i32": (5, "<i"), "f32": (6, "<f"), "bool": (7, "<B"), "u64": (10, "<Q"),
         "i64": (11, "<q"), "f64": (12, "<d")}
GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q8_0": 8, "Q6_K": 14}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind, v) -> bytes:
    if kind == "str":
        return struct.pack("<I", 8) + _str(v)
    if kind == "raw":  # (type code, payload bytes) written as given
        return struct.pack("<I", v[0]) + v[1]
    if kind.startswith("arr:"):
        et = kind[4:]
        code, fmt = TYPES[et]
        return struct.pack("<IIQ", 9, code, len(v)) + b"".join(struct.pack(fmt, x) for x in v)
    code, fmt = TYPES[kind]
    return struct.pack("<I", code) + struct.pack(fmt, v)


def write_gguf(path, metadata, tensors, alignment=32, version=3, magic=b"GGUF",
               offsets=None, truncate=None):
    """metadata: [(key, kind, value)]; tensors: [(name, dims (ggml order),
    type name, data bytes)].  `offsets`/`truncate` let tests corrupt files."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(metadata))
    for k, kind, v in metadata:
        head += _str(k) + _value(kind, v)
    data = b""
    offs = []
    for i, (name, dims, ty, blob) in enumerate(tensors):
        pad = (-len(data)) % alignment
        data += b"\0" * pad
        offs.append(len(data) if offsets is None else offsets[i])
        data += blob
    for i, (name, dims, ty, blob) in enumerate(tensors):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", GGML[ty], offs[i])
    head += b"\0" * ((-len(head)) % alignment)
    out = head + data
    if truncate is not None:
        out = out[:truncate]
    with open(path, "wb") as f:
        f.write(out)
