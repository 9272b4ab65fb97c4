"""A GGUF (version 2 / 3) container reader for the llama.cpp adapter files of the reference's 27B kit
(code/qwen38-27b-kit/identity_projector.py:15-80): the metadata key-value pairs and the tensor table,
with each tensor's bytes as a read-only memory map (nothing in the file is executed).

Layout, little-endian: magic "GGUF", version u32, tensor count u64, metadata count u64; each metadata
entry a string key (u64 length + UTF-8), a u32 value type and the value (scalars; strings; arrays as an
element type u32, a count u64 and the elements); each tensor a string name, n_dims u32, the dims ne[]
as u64 (ne[0] varies fastest), a ggml type u32 and a u64 offset into the data section, which starts at
the next multiple of general.alignment (default 32) after the table. A tensor with ne = [n_in, n_out]
holds n_out rows of n_in values: the [out, in] layout of a linear layer's weight.
"""
import struct
from dataclasses import dataclass

import numpy as np

MAGIC = b"GGUF"
_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
STRING, ARRAY = 8, 9
# ggml type -> (values per block, bytes per block) for the types a map file uses
BLOCKS = {0: (1, 4), 1: (1, 2), 8: (32, 34), 30: (1, 2)}
TYPE_NAMES = {0: "F32", 1: "F16", 8: "Q8_0", 30: "BF16"}
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30


class GGUFError(ValueError):
    """A file that is not a readable GGUF container."""


@dataclass
class Tensor:
    name: str
    ne: tuple           # ggml dims, ne[0] fastest
    ggml_type: int
    data: np.ndarray    # uint8 [rows, row_bytes] memory map (rows = prod(ne[1:]))

    @property
    def shape(self):
        """The numpy / PyTorch shape (ne reversed)."""
        return tuple(reversed(self.ne))


class _Cursor:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, fmt):
        n = struct.calcsize(fmt)
        if self.pos + n > len(self.buf):
            raise GGUFError("truncated file")
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += n
        return v

    def string(self):
        n = self.take("<Q")
        if self.pos + n > len(self.buf):
            raise GGUFError("truncated string")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8")
        self.pos += n
        return s

    def value(self, vt):
        if vt in _SCALARS:
            return self.take(_SCALARS[vt])
        if vt == STRING:
            return self.string()
        if vt == ARRAY:
            et, n = self.take("<I"), self.take("<Q")
            return [self.value(et) for _ in range(n)]
        raise GGUFError(f"metadata value type {vt}")


def read(path):
    """(metadata {key: value}, {name: Tensor}) of a GGUF file."""
    buf = np.memmap(path, dtype=np.uint8, mode="r")
    if len(buf) < 24 or bytes(buf[:4]) != MAGIC:
        raise GGUFError(f"{path}: not a GGUF file")
    c = _Cursor(buf)
    c.pos = 4
    version = c.take("<I")
    if version not in (2, 3):
        raise GGUFError(f"{path}: GGUF version {version} (2 or 3)")
    n_tensors, n_kv = c.take("<Q"), c.take("<Q")
    meta = {}
    for _ in range(n_kv):
        key = c.string()
        meta[key] = c.value(c.take("<I"))
    infos = []
    for _ in range(n_tensors):
        name = c.string()
        nd = c.take("<I")
        ne = tuple(c.take("<Q") for _ in range(nd))
        infos.append((name, ne, c.take("<I"), c.take("<Q")))
    align = int(meta.get("general.alignment", 32))
    start = (c.pos + align - 1) // align * align
    tensors = {}
    for name, ne, gt, off in infos:
        if gt not in BLOCKS:
            raise GGUFError(f"{name}: ggml type {gt} (map files use F32, F16, Q8_0, BF16)")
        per, nb = BLOCKS[gt]
        if not ne or ne[0] % per:
            raise GGUFError(f"{name}: dims {ne} for ggml type {TYPE_NAMES[gt]}")
        rows = int(np.prod(ne[1:])) if len(ne) > 1 else 1
        row_bytes = ne[0] // per * nb
        a = start + off
        if off % align or a + rows * row_bytes > len(buf):
            raise GGUFError(f"{name}: data at {a} ({rows} x {row_bytes} bytes) outside the file or misaligned")
        tensors[name] = Tensor(name, ne, gt, buf[a:a + rows * row_bytes].reshape(rows, row_bytes))
    return meta, tensors
