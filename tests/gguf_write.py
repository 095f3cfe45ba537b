"""Test helper: writes GGUF files (the published format, version 3) for the reader's tests.  The reference's tests
write theirs with gguf-py's GGUFWriter (T/test_gguf_reader.py:7-17), which is not installed here."""
import struct

import numpy as np

GGML_IDS = {"F32": 0, "F16": 1, "Q2_K": 10, "Q3_K": 11, "IQ3_S": 21, "IQ2_S": 22, "IQ4_XS": 23, "BF16": 30}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(v):
    """(type id, bytes) of a metadata value: int -> u32, float -> f32, str -> string, list of ints -> u32 array."""
    if isinstance(v, bool):
        return 7, struct.pack("<?", v)
    if isinstance(v, int):
        return 4, struct.pack("<I", v)
    if isinstance(v, float):
        return 6, struct.pack("<f", v)
    if isinstance(v, str):
        return 8, _str(v)
    if isinstance(v, list):
        return 9, struct.pack("<IQ", 4, len(v)) + b"".join(struct.pack("<I", x) for x in v)
    raise TypeError(type(v))


def write_gguf(path, kv, tensors, alignment=32):
    """kv: {key: value}; tensors: [(name, dims [ne0, ne1, ...], ggml type name, raw bytes)]."""
    if alignment != 32:
        kv = dict(kv, **{"general.alignment": alignment})
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for k, v in kv.items():
        t, b = _value(v)
        head += _str(k) + struct.pack("<I", t) + b
    offs, off = [], 0
    for name, dims, ty, raw in tensors:
        offs.append(off)
        off += (len(raw) + alignment - 1) // alignment * alignment
    for (name, dims, ty, raw), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", GGML_IDS[ty], o)
    head += b"\0" * ((-len(head)) % alignment)
    with open(path, "wb") as f:
        f.write(head)
        for (name, dims, ty, raw), o in zip(tensors, offs):
            raw = bytes(raw)
            f.write(raw + b"\0" * ((-len(raw)) % alignment))


F16_AT = {"Q2_K": (80, 82), "Q3_K": (108,)}       # where the block's f16 scales sit (IQ formats: byte 0)


def expert_tensor(rng, qtype, E, out, inn, block_bytes, scale=0.02):
    """Random expert blocks [E, out, inn/256, block_bytes] with finite f16 scales, and the tensor's GGUF dims."""
    raw = rng.integers(0, 256, (E, out, inn // 256, block_bytes), dtype=np.uint8)
    for o in F16_AT.get(qtype, (0,)):
        d = rng.uniform(0.5 * scale, scale, (E, out, inn // 256)).astype(np.float16)
        raw[..., o:o + 2] = np.frombuffer(d.tobytes(), np.uint8).reshape(E, out, inn // 256, 2)
    return raw, [inn, out, E]
