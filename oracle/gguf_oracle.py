"""CPU restatement of the engine's GGUF reader - test infrastructure only.

Follows src/gguf/gguf_reader.cpp of the reference (GgufReader::open,
:100-287, and read_tensor_raw, :288-305) including which metadata it keeps:
strings (all), integers of types U32/I32/BOOL/U64/I64 (kv_int_), F32 (kv_float_),
numeric arrays of at most 4096 elements of types U8/I8/U16/I16/U32/I32/BOOL
outside "tokenizer." (kv_arr_, as uint32 values), and the tokenizer arrays
(tokens, merges, scores, token_type). U16/I16/F64 scalars are skipped. The
data section starts at the end of the tensor infos rounded up to
general.alignment (power of two, default 32) for version >= 2, and at 0 (the
offsets are absolute) otherwise. Row sizes follow quant/quant.cpp:839-910.

Pinned by tests/test_gguf.py: the reference self-test's own file construction
(tests/selftest.cpp:333-440, version 1 with absolute offsets) read back to the
bytes it wrote, writer round trips of every value type, and hand-computed
offsets.
"""
import struct

KV_ARR_MAX = 4096  # gguf_reader.cpp:92

# (block size, block bytes) per tensor type id (quant/quant.h:24-265, 439-476)
TYPE_TRAITS = {
    0: (1, 4), 1: (1, 2), 30: (1, 2), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8),
    2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36), 20: (32, 18), 39: (32, 17),
    40: (64, 36), 41: (128, 18), 42: (64, 18),
    10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
    16: (256, 66), 17: (256, 74), 18: (256, 98), 19: (256, 50), 21: (256, 110), 22: (256, 82), 23: (256, 136),
    29: (256, 56), 34: (256, 54), 35: (256, 66),
}


def row_size(t, ne0):
    """desireeia_row_size (quant/quant.cpp:905-910)."""
    if t not in TYPE_TRAITS:
        return 0
    blck, nbytes = TYPE_TRAITS[t]
    return (ne0 // blck + (1 if ne0 % blck else 0)) * nbytes


_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


class _Rd:
    def __init__(self, b):
        self.b, self.p = b, 0

    def get(self, fmt):
        n = struct.calcsize(fmt)
        if self.p + n > len(self.b):
            raise EOFError
        v = struct.unpack_from(fmt, self.b, self.p)[0]
        self.p += n
        return v

    def string(self):
        n = self.get("<Q")
        if self.p + n > len(self.b):
            raise EOFError
        s = self.b[self.p:self.p + n]
        self.p += n
        return s.decode("utf-8", "surrogateescape")

    def skip(self, t):
        # skip_gguf_value (gguf_reader.cpp:46-67)
        if t in _SCALAR:
            self.get(_SCALAR[t])
        elif t == 8:
            self.string()
        elif t == 9:
            elem = self.get("<I")
            n = self.get("<Q")
            for _ in range(n):
                self.skip(elem)
        else:
            raise ValueError("unknown value type")


def read(data):
    """Parses GGUF bytes as GgufReader::open does. Returns None where it
    returns false."""
    r = _Rd(data)
    try:
        if r.get("<I") != 0x46554747:
            return None
        version = r.get("<I")
        n_tensors = r.get("<Q")
        n_kv = r.get("<Q")
        kv_string, kv_int, kv_float, kv_arr, vocab = {}, {}, {}, {}, {}
        for _ in range(n_kv):
            key = r.string()
            t = r.get("<I")
            if t == 8:
                kv_string[key] = r.string()
            elif t == 9:
                elem = r.get("<I")
                n = r.get("<Q")
                if key == "tokenizer.ggml.tokens" and elem == 8:
                    vocab["tokens"] = [r.string() for _ in range(n)]
                elif key == "tokenizer.ggml.merges" and elem == 8:
                    vocab["merges"] = [r.string() for _ in range(n)]
                elif key == "tokenizer.ggml.scores" and elem == 6:
                    vocab["scores"] = [r.get("<f") for _ in range(n)]
                elif key == "tokenizer.ggml.token_type" and elem in (4, 5):
                    vocab["token_type"] = [r.get("<i") for _ in range(n)]
                elif 0 < n <= KV_ARR_MAX and not key.startswith("tokenizer.") and elem in (7, 0, 1, 2, 3, 4, 5):
                    vals = []
                    for _ in range(n):
                        v = r.get(_SCALAR[elem])
                        vals.append(v & 0xFFFFFFFF)  # signed kinds sign-extended, then uint32
                    kv_arr[key] = vals
                else:
                    for _ in range(n):
                        r.skip(elem)
            elif t in (10, 11, 4, 5, 7):
                # U64 as is; I64 as its uint64 bits; U32 and I32 both read as
                # uint32 (gguf_reader.cpp:224-250); BOOL as its byte
                v = r.get(_SCALAR[t])
                if t == 11:
                    v &= (1 << 64) - 1
                elif t == 5:
                    v &= 0xFFFFFFFF
                kv_int[key] = v
            elif t == 6:
                kv_float[key] = r.get("<f")
            else:
                r.skip(t)
        tensors = []
        for _ in range(n_tensors):
            name = r.string()
            nd = r.get("<I")
            dims = [r.get("<Q") for _ in range(nd)]
            t = r.get("<I")
            off = r.get("<Q")
            tensors.append((name, t, dims, off))
    except (EOFError, ValueError):
        return None
    alignment = 32
    a = kv_int.get("general.alignment")
    if a is not None and a > 0 and (a & (a - 1)) == 0:
        alignment = a
    pos = r.p
    data_start = (pos + alignment - 1) // alignment * alignment if version >= 2 else 0
    return {"version": version, "kv_string": kv_string, "kv_int": kv_int, "kv_float": kv_float, "kv_arr": kv_arr,
            "vocab": vocab, "tensors": tensors, "alignment": alignment, "data_start": data_start}


def read_tensor_raw(data, info, name):
    """read_tensor_raw: (bytes, type, ne0, rows) or None."""
    for tname, t, dims, off in info["tensors"]:
        if tname != name:
            continue
        if not dims:
            return None
        rb = row_size(t, dims[0])
        if rb == 0:
            return None
        rows = 1
        for d in dims[1:]:
            rows *= d
        start = info["data_start"] + off
        if start + rb * rows > len(data):
            return None
        return data[start:start + rb * rows], t, dims[0], rows
    return None
