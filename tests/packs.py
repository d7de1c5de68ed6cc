"""Writes weight files in the reference's pack format (test infrastructure).

A restatement of FileSink (src/pack.rs:482-600): "TELMOPAK", the u32 version and 4 zero bytes;
each entry's data padded to a multiple of 64 bytes (a matrix's values, then its scales); the
JSON index (entries in write order, members name, kind fields, offset, bytes); the index's
offset and length as little-endian u64s and "TELMOIDX".
"""
import json
import struct

import numpy as np

PRECISION_NAMES = ["f32", "f16", "bf16", "int8", "q8_0"]


class PackWriter:
    def __init__(self, model, metadata=()):
        self.buf = bytearray(b"TELMOPAK" + struct.pack("<I", 1) + bytes(4))
        self.model = model
        self.metadata = list(metadata)
        self.index = []

    def _put(self, data: bytes) -> int:
        self.buf += bytes((-len(self.buf)) % 64)
        at = len(self.buf)
        self.buf += data
        return at

    def matrix(self, name, values, scales, precision, n, k):
        at = self._put(np.ascontiguousarray(values).tobytes())
        rec = {"name": name, "type": "matrix", "precision": PRECISION_NAMES[precision], "n": n, "k": k}
        if scales is not None and len(scales):
            sb = np.ascontiguousarray(scales, np.float32).tobytes()
            rec["scales_offset"] = self._put(sb)
            rec["scales_bytes"] = len(sb)
        rec["offset"] = at
        rec["bytes"] = len(values)
        self.index.append(rec)

    def f32(self, name, shape, data):
        b = np.ascontiguousarray(data, np.float32).tobytes()
        at = self._put(b)
        self.index.append({"name": name, "type": "f32", "shape": list(shape), "offset": at, "bytes": len(b)})

    def bytes_entry(self, name, data: bytes):
        at = self._put(data)
        self.index.append({"name": name, "type": "bytes", "offset": at, "bytes": len(data)})

    def finish(self, index_text=None) -> bytes:
        root = {"model": self.model, "metadata": dict(self.metadata), "entries": self.index}
        text = (index_text if index_text is not None else json.dumps(root, separators=(",", ":"))).encode()
        at = len(self.buf)
        return bytes(self.buf + text + struct.pack("<QQ", at, len(text)) + b"TELMOIDX")


def sample_weights():
    """The rows of the reference's sample pack: w[i] = (i % 17) * 0.1 - 0.8 over 40 x 64, in f32."""
    i = np.arange(40 * 64)
    return (np.float32(1) * (i % 17).astype(np.float32) * np.float32(0.1) - np.float32(0.8)).astype(np.float32)


def sample_pack(encode) -> bytes:
    """The reference's sample (src/pack.rs:614-628): int8, Q8_0 and f16 matrices of the same rows,
    an f32 tensor and a bytes entry; model "test", metadata source = "x"."""
    w = sample_weights().reshape(40, 64)
    sink = PackWriter("test", [("source", "x")])
    for name, prec in (("w8", 3), ("wq", 4), ("wh", 1)):
        values, scales = encode(w, 40, 64, prec)
        sink.matrix(name, values, scales, prec, 40, 64)
    sink.f32("bias", [2, 3], np.array([1, 2, 3, 4, 5, 6], np.float32))
    sink.bytes_entry("config.json", b'{"a":1}')
    return sink.finish()
