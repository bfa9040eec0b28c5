"""A GGUF writer for the tests, written from the published format (magic "GGUF", u32 version, u64 tensor count, u64
key-value count; key = u64-length string, u32 value type, value; tensor info = name, u32 n_dims, u64 dims innermost
first, u32 ggml type, u64 offset into the data section; data section at the header's end rounded up to
general.alignment, default 32). Independent of the library's reader it checks."""
import struct

KIND = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7, "str": 8, "arr": 9, "u64": 10, "i64": 11, "f64": 12}
FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind: int, v) -> bytes:
    if kind == 8:
        return _str(v)
    if kind == 9:
        ek, items = v
        return struct.pack("<IQ", ek, len(items)) + b"".join(_value(ek, x) for x in items)
    return struct.pack(FMT[kind], v)


def write(path, kvs, tensors, version=3, alignment=None, offset_fn=None):
    """kvs: [(key, kind_name, value)] (arrays: ("arr", (elem_kind_int, [values]))); tensors: [(name, dims, ggml_type,
    bytes)]; data blobs are placed at aligned offsets (offset_fn(i, natural) may override an offset)."""
    al = alignment or 32
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for key, kind, v in kvs:
        k = KIND[kind]
        head += _str(key) + struct.pack("<I", k) + _value(k, v)
    offsets, at = [], 0
    for i, (_, _, _, blob) in enumerate(tensors):
        off = at if offset_fn is None else offset_fn(i, at)
        offsets.append(off)
        at = (max(at, off + len(blob)) + al - 1) // al * al
    for (name, dims, ty, _), off in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, off)
    data_start = (len(head) + al - 1) // al * al
    body = bytearray(at)
    for (_, _, _, blob), off in zip(tensors, offsets):
        body[off : off + len(blob)] = blob
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_start - len(head)) + bytes(body))
    return data_start, offsets
