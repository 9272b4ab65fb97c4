"""A minimal GGUF (version 3) writer for the tests, written from the container layout (magic, version,
counts, metadata entries, tensor table, data section aligned to 32 bytes): it makes the adapter files the
loader reads, with chosen raw tensor bytes."""
import struct

import numpy as np

TYPES = {"u32": (4, "<I"), "i32": (5, "<i"), "f32": (6, "<f"), "str": (8, None), "u64": (10, "<Q")}


def _str(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def write(path, meta, tensors, align=32):
    """meta: [(key, kind, value)] with kind in TYPES; tensors: [(name, ne, ggml_type, raw bytes)]."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta)))
    for key, kind, value in meta:
        vt, fmt = TYPES[kind]
        out += _str(key) + struct.pack("<I", vt) + (_str(value) if kind == "str" else struct.pack(fmt, value))
    off, blobs = 0, []
    for name, ne, gt, raw in tensors:
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", gt, off)
        blobs.append((off, raw))
        off = (off + len(raw) + align - 1) // align * align
    out += b"\0" * ((-len(out)) % align)
    start = len(out)
    out += b"\0" * off
    for o, raw in blobs:
        out[start + o:start + o + len(raw)] = raw
    with open(path, "wb") as f:
        f.write(bytes(out))


def q8_0(rows, width, rng):
    """Random Q8_0 bytes [rows, width / 32 * 34]: scales |d| in [2^-12, 2^-4] (fp16), codes in [-128, 127]."""
    d = (rng.uniform(2.0 ** -12, 2.0 ** -4, (rows, width // 32, 1)) * rng.choice([-1, 1], (rows, width // 32, 1)))
    q = rng.integers(-128, 128, (rows, width // 32, 32), dtype=np.int64).astype(np.int8)
    blk = np.concatenate([d.astype(np.float16).view(np.uint8), q.view(np.uint8)], axis=2)
    return np.ascontiguousarray(blk.reshape(rows, width // 32 * 34))
