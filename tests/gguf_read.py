"""A minimal GGUF (v3) reader for tests: the tensor table and raw tensor bytes.

Follows the file layout the reference reads (nm/src/gguf.cpp): magic, version,
tensor and key/value counts, the key/value pairs, the tensor infos (name, dims,
ggml type, offset), then the data section at `general.alignment` (default 32).
"""
import struct

import numpy as np

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
TYPE_BYTES = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


class _Cursor:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def string(self):
        n = self.take("<Q")
        s = bytes(self.buf[self.pos:self.pos + n]).decode()
        self.pos += n
        return s

    def value(self, vtype):
        if vtype == 8:
            return self.string()
        if vtype == 9:
            et, n = self.take("<I"), self.take("<Q")
            return [self.value(et) for _ in range(n)]
        return self.take(_SCALAR[vtype])


def read(image):
    """-> (metadata dict, {name: (ggml type, dims, uint8 view of the bytes)})"""
    buf = memoryview(np.ascontiguousarray(image, np.uint8))
    c = _Cursor(buf)
    assert bytes(buf[:4]) == b"GGUF", "not a GGUF image"
    c.pos = 4
    c.take("<I")
    n_tensors, n_kv = c.take("<Q"), c.take("<Q")
    meta = {}
    for _ in range(n_kv):
        key = c.string()
        meta[key] = c.value(c.take("<I"))
    infos = []
    for _ in range(n_tensors):
        name = c.string()
        dims = [c.take("<Q") for _ in range(c.take("<I"))]
        infos.append((name, dims, c.take("<I"), c.take("<Q")))
    align = int(meta.get("general.alignment", 32))
    data0 = (c.pos + align - 1) // align * align
    arr = np.frombuffer(buf, np.uint8)
    tensors = {}
    for name, dims, ttype, off in infos:
        n = int(np.prod(dims))
        block, nbytes = TYPE_BYTES[ttype]
        size = n // block * nbytes
        tensors[name] = (ttype, dims, arr[data0 + off:data0 + off + size])
    return meta, tensors
