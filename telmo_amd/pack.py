"""Python mirror of the reference's weight files (``Pack``, src/pack.rs) over the C ABI.

``Pack.open`` maps a pack file and checks its index as ``Pack::parse`` does
(src/pack.rs:98-259), raising ``TelmoError`` with the reference's message when it is not
usable. ``matrix`` follows ``Pack::matrix`` (src/pack.rs:279-305) and uploads the weights to
the device once; ``vector`` and ``bytes`` read f32 tensors and raw entries (src/pack.rs:307-328).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Tuple

import numpy as np

from . import _lib
from .kernels import Kernels, PackedWeights, Precision, TelmoError, _check

MATRIX, F32, BYTES = 0, 1, 2


class _Entry(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_uint32), ("precision", ctypes.c_uint32),
                ("n", ctypes.c_size_t), ("k", ctypes.c_size_t), ("rank", ctypes.c_size_t),
                ("shape", ctypes.c_size_t * 8), ("data", ctypes.c_void_p), ("bytes", ctypes.c_size_t),
                ("scales", ctypes.c_void_p), ("n_scales", ctypes.c_size_t)]


@dataclass
class Entry:
    """One entry: a matrix (precision, n, k), an f32 tensor (shape) or raw bytes."""
    name: str
    kind: int
    precision: Optional[Precision]
    n: int
    k: int
    shape: Tuple[int, ...]
    bytes: int
    n_scales: int

    def size(self) -> int:
        """Bytes of data, scales included (Entry::size)."""
        return self.bytes + 4 * self.n_scales


def _pack_check(code: int) -> None:
    if code != 0:
        raise TelmoError(code, _lib.lib().tg_pack_last_error().decode() or "pack error")


class Pack:
    def __init__(self, handle):
        self._h = handle

    @staticmethod
    def open(path: str) -> "Pack":
        h = ctypes.c_void_p()
        _pack_check(_lib.lib().tg_pack_open(str(path).encode(), ctypes.byref(h)))
        return Pack(h)

    @staticmethod
    def from_bytes(data: bytes) -> "Pack":
        h = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(bytes(data), len(data)) if data else None
        _pack_check(_lib.lib().tg_pack_from_bytes(buf, len(data), ctypes.byref(h)))
        return Pack(h)

    def close(self) -> None:
        if self._h:
            _lib.lib().tg_pack_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def model(self) -> str:
        return _lib.lib().tg_pack_model(self._h).decode()

    def metadata(self) -> List[Tuple[str, str]]:
        L = _lib.lib()
        out = []
        for i in range(L.tg_pack_meta_count(self._h)):
            key, value = ctypes.c_char_p(), ctypes.c_char_p()
            _pack_check(L.tg_pack_meta_at(self._h, i, ctypes.byref(key), ctypes.byref(value)))
            out.append((key.value.decode(), value.value.decode()))
        return out

    def meta(self, key: str) -> Optional[str]:
        v = _lib.lib().tg_pack_meta(self._h, key.encode())
        return None if v is None else v.decode()

    def is_mapped(self) -> bool:
        return bool(_lib.lib().tg_pack_is_mapped(self._h))

    @staticmethod
    def _to_entry(e: _Entry) -> Entry:
        return Entry(e.name.decode(), e.type, Precision(e.precision) if e.type == MATRIX else None, e.n, e.k,
                     tuple(e.shape[i] for i in range(e.rank)), e.bytes, e.n_scales)

    def entries(self) -> List[Entry]:
        L = _lib.lib()
        out = []
        for i in range(L.tg_pack_entry_count(self._h)):
            e = _Entry()
            _pack_check(L.tg_pack_entry_at(self._h, i, ctypes.byref(e)))
            out.append(self._to_entry(e))
        return out

    def _find(self, name: str) -> _Entry:
        e = _Entry()
        _pack_check(_lib.lib().tg_pack_find(self._h, name.encode(), ctypes.byref(e)))
        return e

    def matrix(self, kernels: Kernels, name: str, n: int, k: int) -> PackedWeights:
        """The named weight matrix of n outputs and k inputs, uploaded to the kernels' device."""
        out = ctypes.c_void_p()
        rc = _lib.lib().tg_pack_upload_matrix(kernels._ctx, self._h, name.encode(), n, k, ctypes.byref(out))
        _check(rc, kernels._ctx)
        return PackedWeights(kernels, out, n, k, Precision(self._find(name).precision))

    def matrix_parts(self, name: str):
        """The named matrix's panel values and scales as host arrays (copies)."""
        e = self._find(name)
        if e.type != MATRIX:
            raise TelmoError(-7, f"The pack file isn't usable. Entry {name} isn't a matrix.")
        values = np.ctypeslib.as_array((ctypes.c_uint8 * e.bytes).from_address(e.data)).copy()
        scales = (np.ctypeslib.as_array((ctypes.c_float * e.n_scales).from_address(e.scales)).copy()
                  if e.n_scales else None)
        return values, scales

    def vector(self, name: str, shape) -> np.ndarray:
        """An f32 tensor of the given shape (a copy)."""
        e = self._find(name)
        shape = tuple(int(d) for d in shape)
        if e.type != F32:
            raise TelmoError(-7, f"The pack file isn't usable. Entry {name} isn't an f32 tensor.")
        have = tuple(e.shape[i] for i in range(e.rank))
        if have != shape:
            raise TelmoError(-2, f"The pack file isn't usable. Entry {name} has shape {list(have)}, and the "
                                 f"model needs {list(shape)}.")
        count = e.bytes // 4
        data = np.ctypeslib.as_array((ctypes.c_float * count).from_address(e.data)) if count else np.zeros(0)
        return np.array(data, np.float32).reshape(shape)

    def bytes(self, name: str) -> bytes:
        e = self._find(name)
        if e.type != BYTES:
            raise TelmoError(-7, f"The pack file isn't usable. Entry {name} isn't a bytes entry.")
        return ctypes.string_at(e.data, e.bytes)

    def precision(self) -> Optional[Precision]:
        """The precision of the weight matrices, if they share one."""
        found = None
        for e in self.entries():
            if e.kind == MATRIX:
                if found is None:
                    found = e.precision
                elif found != e.precision:
                    return None
        return found

    def data_bytes(self) -> int:
        return sum(e.size() for e in self.entries())
