"""GGUF byte builders for the loader tests (test infrastructure).

reference_dialect(): the layout the reference's parser reads and its own fixture
builder writes (src/model/inference/gguf.rs:2687-2752): one-byte value / array-element
/ tensor types, absolute tensor offsets (each data block placed at the next multiple
of 32, as that builder does).
standard(): GGUF v3 as specified: uint32 type fields, offsets relative to the data
section, which starts at the end of the tensor infos rounded up to the alignment.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v, one_byte: bool) -> bytes:
    tid = (lambda t: struct.pack("<B", t)) if one_byte else (lambda t: struct.pack("<I", t))
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        return tid(etype) + struct.pack("<Q", len(items)) + b"".join(_value(etype, x, one_byte) for x in items)
    return struct.pack(_FMT[vtype], v)


def build(metadata, tensors, dialect: str, version: int = 3, alignment: int = 32, data_shift: int = 0) -> bytes:
    """metadata: [(key, vtype, value)]; tensors: [(name, dims (GGUF order), type id,
    data bytes)].  data_shift (reference dialect): each data block starts that many bytes
    past its 32-byte boundary (the reference applies no alignment of its own)."""
    one = dialect == "reference"
    tid = (lambda t: struct.pack("<B", t)) if one else (lambda t: struct.pack("<I", t))
    buf = bytearray(struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(metadata)))
    for key, vtype, value in metadata:
        buf += _str(key) + tid(vtype) + _value(vtype, value, one)
    if one:
        # absolute offsets: compute the end of the infos first, then place each block
        info_len = sum(len(_str(n)) + 4 + 8 * len(d) + 1 + 8 for n, d, _, _ in tensors)
        pos = len(buf) + info_len
        offsets = []
        for _, _, _, data in tensors:
            pos = (pos + 31) // 32 * 32 + data_shift
            offsets.append(pos)
            pos += len(data)
        for (name, dims, t, _), off in zip(tensors, offsets):
            buf += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            buf += tid(t) + struct.pack("<Q", off)
        for (_, _, _, data), off in zip(tensors, offsets):
            buf += bytes(off - len(buf)) + bytes(data)
        return bytes(buf)
    rel, pos = [], 0
    for _, _, _, data in tensors:
        pos = (pos + alignment - 1) // alignment * alignment
        rel.append(pos)
        pos += len(data)
    for (name, dims, t, _), off in zip(tensors, rel):
        buf += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        buf += tid(t) + struct.pack("<Q", off)
    start = (len(buf) + alignment - 1) // alignment * alignment
    buf += bytes(start - len(buf))
    for (_, _, _, data), off in zip(tensors, rel):
        buf += bytes(start + off - len(buf)) + bytes(data)
    return bytes(buf)


def build_minimal_gguf() -> bytes:
    """gguf.rs:2687-2752: v3, metadata general.architecture = "llama",
    llama.embedding_length = 4096 (u32), llama.block_count = 32 (u32); one F32 tensor
    "model.token_embd.weight" [4096] of 0.5 at the next 32-aligned absolute offset."""
    return build([("general.architecture", STRING, "llama"), ("llama.embedding_length", U32, 4096),
                  ("llama.block_count", U32, 32)],
                 [("model.token_embd.weight", [4096], 0, np.full(4096, 0.5, dtype=np.float32).tobytes())],
                 "reference")


def mutations(seed: int, count: int):
    """Fixed-seed mutants of a multi-tensor file in both dialects: (dialect name, bytes)
    with byte overwrites, 64-bit counts / lengths / offsets set to extreme values, and
    truncation."""
    import random
    rng = random.Random(seed)
    q = np.random.default_rng(1).integers(0, 256, 2 * 18 * 4, dtype=np.uint8)
    meta = [("general.architecture", STRING, "llama"), ("a", ARRAY, (U32, [1, 2])), ("f", F32, 1.5)]
    tens = [("w", [64, 4], 2, q.tobytes()), ("x", [8], 0, bytes(32))]
    bases = {"reference": build(meta, tens, "reference"), "standard": build(meta, tens, "standard")}
    for _ in range(count):
        dialect = rng.choice(sorted(bases))
        b = bytearray(bases[dialect])
        for _ in range(rng.randint(1, 6)):
            pos = rng.randrange(len(b))
            r = rng.random()
            if r < 0.5:
                b[pos] = rng.randrange(256)
            elif r < 0.85 and pos + 8 <= len(b):
                b[pos:pos + 8] = struct.pack("<Q", rng.choice([0, 1, 2**31, 2**32 - 1, 2**63, 2**64 - 1,
                                                                rng.randrange(2**64)]))
            else:
                del b[pos:]
                break
        yield dialect, bytes(b)
