"""A minimal GGUF writer for the tests, following the layout that
third_party/ggml/include/gguf.h documents: "GGUF", u32 version, u64 tensor
count, u64 key/value count, the typed key/values, the tensor infos (name,
dims, ne, ggml type, offset within the data section), then the data section
at the next multiple of the alignment, each tensor's data aligned in it."""
import struct

T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_FMT = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f", T_BOOL: "<?",
        T_U64: "<Q", T_I64: "<q", T_F64: "<d"}
GGML_F32, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 8, 12, 14


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _val(t, v):
    if t == T_STR:
        return _str(v)
    if t == T_ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def write_gguf(path, kvs, tensors, alignment=None, version=3):
    """kvs: [(key, gguf type, value)], an array value being (element type,
    items); tensors: [(name, ggml type, ne, data bytes)].  Returns the
    absolute file offset of every tensor's data."""
    kvs = list(kvs) + ([("general.alignment", T_U32, alignment)] if alignment is not None else [])
    align = alignment or 32
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += _str(k) + struct.pack("<I", t) + _val(t, v)
    rel, pos = [], 0
    for _, _, _, data in tensors:
        pos = (pos + align - 1) // align * align
        rel.append(pos)
        pos += len(data)
    for (name, gt, ne, _), off in zip(tensors, rel):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", gt, off)
    data_off = (len(head) + align - 1) // align * align
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_off - len(head)))
        cur = 0
        for (_, _, _, data), off in zip(tensors, rel):
            f.write(b"\0" * (off - cur))
            f.write(data)
            cur = off + len(data)
    return {t[0]: data_off + off for t, off in zip(tensors, rel)}
