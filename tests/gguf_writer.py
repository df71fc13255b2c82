"""Minimal GGUF writer for the tests (written from the file format, not from
any reader): key/values of every value type, tensors placed at aligned
offsets of the data section, versions 1-3 (version < 2: absolute tensor
offsets, as the engine's own self-test writes them)."""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_PACK = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
         I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value_bytes(t, v):
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value_bytes(et, x) for x in items)
    return struct.pack(_PACK[t], v)


def _align(n, a):
    return (n + a - 1) // a * a


def gguf_bytes(kv, tensors, version=3, alignment=32, counts_override=None):
    """kv: [(key, type, value)]; tensors: [(name, type id, dims (ne0 first), data bytes)].
    Returns the file bytes. `alignment` places the data section and each
    tensor; it should equal general.alignment when kv holds that key."""
    n_t, n_kv = (len(tensors), len(kv)) if counts_override is None else counts_override
    head = b"GGUF" + struct.pack("<IQQ", version, n_t, n_kv)
    for key, t, v in kv:
        head += _str(key) + struct.pack("<I", t) + value_bytes(t, v)
    rel, off = [], 0
    for _, _, _, data in tensors:
        off = _align(off, alignment)
        rel.append(off)
        off += len(data)
    info_len = sum(8 + len(name.encode()) + 4 + 8 * len(dims) + 4 + 8 for name, _, dims, _ in tensors)
    data_start = _align(len(head) + info_len, alignment)
    infos = b""
    for (name, ty, dims, _), r in zip(tensors, rel):
        o = r if version >= 2 else data_start + r
        infos += _str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) + struct.pack(
            "<IQ", ty, o)
    out = bytearray(head + infos)
    out += b"\0" * (data_start - len(out))
    for (_, _, _, data), r in zip(tensors, rel):
        out += b"\0" * (data_start + r - len(out))
        out += data
    return bytes(out)


def write_gguf(path, kv, tensors, version=3, alignment=32):
    with open(path, "wb") as f:
        f.write(gguf_bytes(kv, tensors, version, alignment))
