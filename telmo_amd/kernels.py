"""Python mirror of telmo's matrix-product operator surface over the HIP library's C ABI.

Names, argument meanings and refusals follow the reference:

* ``Precision`` - src/quant.rs:20-83 (``name``, ``from_name``, ``value_bytes``, ``panel_bytes``,
  ``scale_count``, ``fits``)
* ``Act``, ``Epilogue`` - src/kernels/mod.rs:366-398 (``Epilogue.PLAIN``, ``Epilogue.bias``)
* ``PackedWeights`` - src/kernels/mod.rs:173-304 (``from_rows``, ``encode``, ``from_parts``,
  ``n``/``k``/``precision``, ``bytes``, ``to_rows``)
* ``Kernels.linear`` / ``Kernels.matmul`` - src/kernels/mod.rs:657-701

Where the reference panics on a violated precondition, these raise ``TelmoError`` with the
library's status code. Host arrays are numpy float32; the ``*_device`` methods take torch tensors
already on the GPU and queue the work on the context's stream. The library must be built
(``telmo_amd.build``): nothing here falls back to the CPU.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass
from typing import NamedTuple, Optional

import numpy as np

from . import _lib


# The library's status for a precision, mode or size it does not run (TG_ERR_UNSUPPORTED).
TG_ERR_UNSUPPORTED = -5


class TelmoError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{message} (status {code})")
        self.code = code


class Precision(enum.IntEnum):
    F32 = 0
    F16 = 1
    BF16 = 2
    INT8 = 3
    Q8_0 = 4

    def name_(self) -> str:
        return ["f32", "f16", "bf16", "int8", "q8_0"][self]

    @staticmethod
    def from_name(name: str) -> Optional["Precision"]:
        for p in Precision:
            if p.name_() == name:
                return p
        return None

    def value_bytes(self) -> int:
        return {0: 4, 1: 2, 2: 2, 3: 1, 4: 1}[int(self)]

    def panel_bytes(self, n: int, k: int) -> int:
        return _lib.lib().tg_panel_bytes(int(self), n, k)

    def scale_count(self, n: int, k: int) -> int:
        return _lib.lib().tg_scale_count(int(self), n, k)

    def fits(self, k: int) -> bool:
        return bool(_lib.lib().tg_fits(int(self), k))


class Act(enum.IntEnum):
    NONE = 0
    RELU = 1
    SILU = 2


@dataclass
class Epilogue:
    """c = (accumulate ? c : 0) + scale * act(sum + bias)."""

    bias: Optional[object] = None
    act: Act = Act.NONE
    scale: float = 1.0
    accumulate: bool = False

    @staticmethod
    def with_bias(bias) -> "Epilogue":
        return Epilogue(bias=bias)


Epilogue.PLAIN = Epilogue()


def _f32(x) -> np.ndarray:
    arr = np.asarray(x)
    if arr.dtype != np.float32 or not arr.flags.c_contiguous:
        raise TypeError("host buffers must be C-contiguous float32 arrays")
    return arr


def _dev(t, dtype: str, name: str) -> ctypes.c_void_p:
    """The device address of GPU tensor t, after checking that t is a GPU tensor of the element type
    the library reads there: the lengths passed beside it count elements of that type."""
    if str(t.dtype) != "torch." + dtype or not t.is_cuda:
        raise TypeError(f"{name} must be a {dtype} GPU tensor, not {t.dtype} on {t.device}")
    return ctypes.c_void_p(t.data_ptr())


def _avail(t) -> int:
    """Elements of t's storage from t's first element to the storage's end: all the library can
    reach from t's address without leaving the allocation."""
    return t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()


def _len(t, given: Optional[int], name: str) -> int:
    """The length in elements passed to the library beside tensor t: `given` when set, else t's
    element count, which needs t contiguous (an expanded or overlapping view counts elements its
    storage does not hold). Either way the length must stay inside t's storage."""
    if given is None:
        if not t.is_contiguous():
            raise ValueError(f"{name} is not contiguous: pass the length the call may read or write")
        given = t.numel()
    if given < 0 or given > _avail(t):
        raise ValueError(f"{name}: a length of {given} elements runs past the tensor's storage "
                         f"({_avail(t)} elements from its start)")
    return given


def _check(code: int, ctx) -> None:
    if code != 0:
        msg = _lib.lib().tg_last_error(ctx).decode() if ctx else "error"
        raise TelmoError(code, msg or "telmo_hip call failed")


class PackedWeights:
    """A weight matrix of n outputs and k inputs, uploaded once to the context's device."""

    def __init__(self, kernels: "Kernels", handle, n: int, k: int, precision: Precision):
        self._kernels = kernels
        self._handle = handle
        self._n, self._k, self._precision = n, k, Precision(precision)

    @staticmethod
    def from_parts(kernels: "Kernels", n: int, k: int, precision: Precision, values, scales=None):
        """Weights already in the panel layout, as a pack stores them (host numpy arrays)."""
        values = np.ascontiguousarray(values, np.uint8)
        sc = None if scales is None else _f32(np.ascontiguousarray(scales, np.float32))
        out = ctypes.c_void_p()
        L = _lib.lib()
        rc = L.tg_weights_upload(kernels._ctx, values.ctypes.data_as(ctypes.c_void_p), values.size,
                                 None if sc is None else sc.ctypes.data_as(ctypes.c_void_p),
                                 0 if sc is None else sc.size, int(precision), n, k, ctypes.byref(out))
        _check(rc, kernels._ctx)
        return PackedWeights(kernels, out, n, k, precision)

    @staticmethod
    def from_device(kernels: "Kernels", n: int, k: int, precision: Precision, values, scales=None):
        """from_parts on GPU tensors (uint8 values, float32 scales) already in the panel layout."""
        out = ctypes.c_void_p()
        rc = _lib.lib().tg_weights_upload_device(kernels._ctx, _dev(values, "uint8", "values"),
                                                 _len(values, None, "values"),
                                                 None if scales is None else _dev(scales, "float32", "scales"),
                                                 0 if scales is None else _len(scales, None, "scales"),
                                                 int(precision), n, k,
                                                 ctypes.byref(out))
        _check(rc, kernels._ctx)
        return PackedWeights(kernels, out, n, k, precision)

    @staticmethod
    def encode(kernels: "Kernels", rows, n: int, k: int, precision: Precision):
        """Packs row-major [n, k] f32 rows in `precision`, quantising or rounding as needed."""
        values, scales = encode(rows, n, k, precision)
        return PackedWeights.from_parts(kernels, n, k, precision, values, scales if scales.size else None)

    @staticmethod
    def from_rows(kernels: "Kernels", rows, n: int, k: int):
        return PackedWeights.encode(kernels, rows, n, k, Precision.F32)

    def n(self) -> int:
        return self._n

    def k(self) -> int:
        return self._k

    def precision(self) -> Precision:
        return self._precision

    def bytes(self) -> int:
        return _lib.lib().tg_weights_bytes(self._handle)

    def close(self) -> None:
        if self._handle:
            _lib.lib().tg_weights_free(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def encode(rows, n: int, k: int, precision: Precision):
    """quant::encode of row-major f32 rows: (values u8, scales f32) in the panel layout."""
    rows = _f32(np.ascontiguousarray(rows, np.float32).reshape(-1))
    p = Precision(precision)
    values = np.zeros(p.panel_bytes(n, k), np.uint8)
    scales = np.zeros(p.scale_count(n, k), np.float32)
    rc = _lib.lib().tg_encode(rows.ctypes.data_as(ctypes.c_void_p), n, k, int(p),
                              values.ctypes.data_as(ctypes.c_void_p), values.size,
                              scales.ctypes.data_as(ctypes.c_void_p), scales.size)
    _check(rc, None)
    return values, scales


def random(length: int, seed: int) -> np.ndarray:
    """The reference's test generator random(len, seed) (src/kernels/mod.rs:795-805): float32 values
    in [-1, 1) from xorshift64, the same sequence for the same seed."""
    out = np.empty(length, np.float32)
    _lib.lib().tg_random(out.ctypes.data_as(ctypes.c_void_p), length, seed & (2**64 - 1))
    return out


def decode(values, scales, n: int, k: int, precision: Precision) -> np.ndarray:
    """quant::decode: the row-major [n, k] values a stored matrix stands for."""
    values = np.ascontiguousarray(values, np.uint8)
    scales = np.ascontiguousarray(scales if scales is not None else np.zeros(0), np.float32)
    out = np.zeros(n * k, np.float32)
    rc = _lib.lib().tg_decode(values.ctypes.data_as(ctypes.c_void_p), values.size,
                              scales.ctypes.data_as(ctypes.c_void_p), scales.size, int(precision), n, k,
                              out.ctypes.data_as(ctypes.c_void_p))
    _check(rc, None)
    return out.reshape(n, k)


class _Epi(ctypes.Structure):
    _fields_ = [("bias", ctypes.c_void_p), ("bias_len", ctypes.c_size_t), ("act", ctypes.c_uint32),
                ("scale", ctypes.c_float), ("accumulate", ctypes.c_int32)]


class Kernels:
    """The GPU matrix-product entry points of one device and stream (one C-ABI context)."""

    FAST = 0
    EXACT = 1

    def __init__(self, device: int = 0, stream: Optional[int] = None, mode: int = FAST):
        L = _lib.lib()
        ctx = ctypes.c_void_p()
        rc = L.tg_ctx_create(device, ctypes.c_void_p(stream) if stream else None, ctypes.byref(ctx))
        if rc != 0:
            raise TelmoError(rc, f"no gfx950 context on device {device}")
        self._ctx = ctx
        self.set_mode(mode)

    def set_mode(self, mode: int) -> None:
        _check(_lib.lib().tg_ctx_set_mode(self._ctx, mode), self._ctx)

    def mode(self) -> int:
        return _lib.lib().tg_ctx_mode(self._ctx)

    def set_guard(self, on: bool) -> None:
        """The fast path's accuracy guard (on by default): rows whose two digits drop more than 2^-12
        of them take the reference's fused sums (tg_ctx_set_guard)."""
        _check(_lib.lib().tg_ctx_set_guard(self._ctx, int(bool(on))), self._ctx)

    def guard(self) -> bool:
        return bool(_lib.lib().tg_ctx_guard(self._ctx))

    def close(self) -> None:
        if self._ctx:
            _lib.lib().tg_ctx_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- host buffers ---------------------------------------------------------------------
    def _epi_host(self, epi: Optional[Epilogue], keep):
        if epi is None:
            return None
        e = _Epi()
        if epi.bias is not None:
            b = _f32(epi.bias)
            keep.append(b)
            e.bias, e.bias_len = b.ctypes.data, b.size
        e.act, e.scale, e.accumulate = int(epi.act), float(epi.scale), int(bool(epi.accumulate))
        return ctypes.byref(e)

    def matmul(self, a, lda: int, m: int, w: PackedWeights, c, ldc: int, epi: Epilogue = Epilogue.PLAIN):
        """c[m, n] = epilogue(a[m, k] * w^T) with a rows lda apart and c rows ldc apart, in place."""
        a, c = _f32(a), _f32(c)
        keep = []
        rc = _lib.lib().tg_matmul(self._ctx, a.ctypes.data_as(ctypes.c_void_p), a.size, lda, m, w._handle,
                                  c.ctypes.data_as(ctypes.c_void_p), c.size, ldc, self._epi_host(epi, keep))
        _check(rc, self._ctx)

    def linear(self, a, m: int, w: PackedWeights, c, epi: Epilogue = Epilogue.PLAIN):
        """c = epilogue(a * w^T) for contiguous a [m, k] and c [m, n], in place."""
        self.matmul(a, w.k(), m, w, c, w.n(), epi)

    # -- device buffers (torch tensors) -----------------------------------------------------
    def _epi_dev(self, epi: Optional[Epilogue]):
        if epi is None:
            return None
        e = _Epi()
        if epi.bias is not None:
            e.bias, e.bias_len = _dev(epi.bias, "float32", "bias").value, _len(epi.bias, None, "bias")
        e.act, e.scale, e.accumulate = int(epi.act), float(epi.scale), int(bool(epi.accumulate))
        return ctypes.byref(e)

    def matmul_device(self, a, lda: int, m: int, w: PackedWeights, c, ldc: int, epi: Epilogue = Epilogue.PLAIN,
                      a_len: Optional[int] = None, c_len: Optional[int] = None):
        """Queues the product on GPU tensors (float32). a_len / c_len default to the tensors' sizes."""
        rc = _lib.lib().tg_matmul_device(self._ctx, _dev(a, "float32", "a"), _len(a, a_len, "a"), lda, m, w._handle,
                                         _dev(c, "float32", "c"), _len(c, c_len, "c"), ldc, self._epi_dev(epi))
        _check(rc, self._ctx)

    def matmul_device_noalloc(self, a, lda: int, m: int, w: PackedWeights, c, ldc: int,
                              epi: Epilogue = Epilogue.PLAIN, a_len: Optional[int] = None,
                              c_len: Optional[int] = None):
        """matmul_device with no allocation: the quantised rows go to the library's per-GPU scratch
        (16 MiB). Calls that overlap on one GPU race."""
        rc = _lib.lib().tg_matmul_device_noalloc(self._ctx, _dev(a, "float32", "a"), _len(a, a_len, "a"), lda, m,
                                                 w._handle, _dev(c, "float32", "c"), _len(c, c_len, "c"), ldc,
                                                 self._epi_dev(epi))
        _check(rc, self._ctx)

    def linear_device(self, a, m: int, w: PackedWeights, c, epi: Epilogue = Epilogue.PLAIN):
        self.matmul_device(a, w.k(), m, w, c, w.n(), epi)

    def linear_glu_device(self, a, m: int, w: PackedWeights, out, ldo: Optional[int] = None,
                          epi: Epilogue = Epilogue.PLAIN, a_len: Optional[int] = None,
                          out_len: Optional[int] = None):
        """out = glu(epi(a . w)) on GPU tensors: linear_device into [m, n] then glu_device, fused into
        one GEMM for int8 weights in fast mode (n a multiple of 64). out is [m, ldo], ldo >= n / 2
        (default n / 2); epi must not accumulate."""
        ldo = w.n() // 2 if ldo is None else ldo
        rc = _lib.lib().tg_linear_glu_device(self._ctx, _dev(a, "float32", "a"), _len(a, a_len, "a"), m, w._handle,
                                             _dev(out, "float32", "out"), _len(out, out_len, "out"), ldo,
                                             self._epi_dev(epi))
        _check(rc, self._ctx)

    def matmul_rowmajor_device(self, a, lda: int, m: int, b, k: int, n: int, ldb: int, c, ldc: int,
                               epi: Epilogue = Epilogue.PLAIN, a_len: Optional[int] = None,
                               b_len: Optional[int] = None, c_len: Optional[int] = None):
        """matmul with BView::row_major(b, k, n, ldb) as the right-hand side: f32 GPU tensors, the
        reference's fused sums. b must hold whole 16-column panels, as the reference's view checks."""
        rc = _lib.lib().tg_matmul_rowmajor_device(
            self._ctx, _dev(a, "float32", "a"), _len(a, a_len, "a"), lda, m,
            _dev(b, "float32", "b"), _len(b, b_len, "b"), k, n, ldb,
            _dev(c, "float32", "c"), _len(c, c_len, "c"), ldc, self._epi_dev(epi))
        _check(rc, self._ctx)

    def quant_bytes(self, m: int, k: int) -> int:
        return _lib.lib().tg_quant_bytes(m, k)

    def quantize_rows_device(self, a, lda: int, m: int, k: int, qa, exps, a_len: Optional[int] = None):
        """Splits rows of a GPU tensor into the two-digit form (qa: uint8 tensor, exps: int32)."""
        if _len(exps, None, "exps") < m:
            raise ValueError("exps must hold m exponents")
        rc = _lib.lib().tg_quantize_rows_device(self._ctx, _dev(a, "float32", "a"), _len(a, a_len, "a"), lda, m, k,
                                                _dev(qa, "uint8", "qa"), _len(qa, None, "qa"),
                                                _dev(exps, "int32", "exps"))
        _check(rc, self._ctx)

    def matmul_quantized_device(self, qa, exps, m: int, w: PackedWeights, c, ldc: int,
                                epi: Epilogue = Epilogue.PLAIN):
        """The MFMA GEMM alone over rows quantised by quantize_rows_device."""
        if _len(exps, None, "exps") < m:
            raise ValueError("exps must hold m exponents")
        rc = _lib.lib().tg_matmul_quantized_device(self._ctx, _dev(qa, "uint8", "qa"), _len(qa, None, "qa"),
                                                   _dev(exps, "int32", "exps"), m, w._handle,
                                                   _dev(c, "float32", "c"), _len(c, None, "c"), ldc,
                                                   self._epi_dev(epi))
        _check(rc, self._ctx)

    def matmul_quantized_glu_device(self, qa, exps, m: int, w: PackedWeights, out, ldo: Optional[int] = None,
                                    epi: Epilogue = Epilogue.PLAIN, out_len: Optional[int] = None):
        """linear_glu_device on quantised rows: out = glu(epi(qa . w)) with the GLU in the GEMM's epilogue."""
        ldo = w.n() // 2 if ldo is None else ldo
        if _len(exps, None, "exps") < m:
            raise ValueError("exps must hold m exponents")
        rc = _lib.lib().tg_matmul_quantized_glu_device(self._ctx, _dev(qa, "uint8", "qa"), _len(qa, None, "qa"),
                                                       _dev(exps, "int32", "exps"), m, w._handle,
                                                       _dev(out, "float32", "out"), _len(out, out_len, "out"), ldo,
                                                       self._epi_dev(epi))
        _check(rc, self._ctx)

    def matmul_quantized_to_quant_device(self, qa, exps, m: int, w: PackedWeights, qa_out, exps_out,
                                         epi: Epilogue = Epilogue.PLAIN):
        """The MFMA GEMM over quantised rows with its outputs epi(qa . w) quantised into qa_out and exps_out
        (the f32 rows never reach memory); epi must not accumulate."""
        for t, name, need in ((exps, "exps", m), (exps_out, "exps_out", m)):
            if _len(t, None, name) < need:
                raise ValueError(f"{name} must hold m exponents")
        rc = _lib.lib().tg_matmul_quantized_to_quant_device(
            self._ctx, _dev(qa, "uint8", "qa"), _len(qa, None, "qa"), _dev(exps, "int32", "exps"), m, w._handle,
            self._epi_dev(epi), _dev(qa_out, "uint8", "qa_out"), _len(qa_out, None, "qa_out"),
            _dev(exps_out, "int32", "exps_out"), _len(exps_out, None, "exps_out"))
        _check(rc, self._ctx)

    def glu_device(self, x, ldx: int, m: int, half: int, out, ldo: int, x_len: Optional[int] = None,
                   out_len: Optional[int] = None):
        rc = _lib.lib().tg_glu_device(self._ctx, _dev(x, "float32", "x"), _len(x, x_len, "x"), ldx, m, half,
                                      _dev(out, "float32", "out"), _len(out, out_len, "out"), ldo)
        _check(rc, self._ctx)

    def softmax_device(self, x, ldx: int, m: int, n: int, x_len: Optional[int] = None):
        """Kernels::softmax (src/kernels/avx512.rs:382-407) of m rows of n values of GPU tensor x, in
        place."""
        rc = _lib.lib().tg_softmax_device(self._ctx, _dev(x, "float32", "x"), _len(x, x_len, "x"), ldx, m, n)
        _check(rc, self._ctx)

    def average_pairs_device(self, x, ldx: int, frames: int, n: int, out, ldo: int, batch: int = 1,
                             x_len: Optional[int] = None, out_len: Optional[int] = None):
        """Granite's strided-block pooling (src/granite.rs:918-931): row r of each of batch sequences
        of frames rows becomes (x[2 r] + x[2 r + 1]) / 2 in out (frames // 2 rows per sequence)."""
        rc = _lib.lib().tg_average_pairs_device(self._ctx, _dev(x, "float32", "x"), _len(x, x_len, "x"), ldx,
                                                frames, batch, n, _dev(out, "float32", "out"),
                                                _len(out, out_len, "out"), ldo)
        _check(rc, self._ctx)

    def layer_norm_device(self, x, ldx: int, m: int, n: int, gamma, beta, eps: float, out, ldo: int,
                          x_len: Optional[int] = None, out_len: Optional[int] = None):
        """LayerNorm of m rows of GPU tensor x (n values each) into out (may be x)."""
        rc = _lib.lib().tg_layer_norm_device(self._ctx, _dev(x, "float32", "x"), _len(x, x_len, "x"), ldx, m, n,
                                             _dev(gamma, "float32", "gamma"), _len(gamma, None, "gamma"),
                                             _dev(beta, "float32", "beta"), _len(beta, None, "beta"),
                                             float(eps), _dev(out, "float32", "out"), _len(out, out_len, "out"), ldo)
        _check(rc, self._ctx)

    def layer_norm_quant_device(self, x, ldx: int, m: int, n: int, gamma, beta, eps: float, qa, exps, out=None,
                                ldo: Optional[int] = None, x_len: Optional[int] = None, out_len: Optional[int] = None):
        """LayerNorm of m rows of GPU tensor x, quantised into qa (uint8, quant_bytes(m, n)) and exps (int32,
        m) for matmul_quantized_device; out (optional, may be x) also gets the f32 LayerNorm."""
        ldo = n if ldo is None else ldo
        rc = _lib.lib().tg_layer_norm_quant_device(
            self._ctx, _dev(x, "float32", "x"), _len(x, x_len, "x"), ldx, m, n, _dev(gamma, "float32", "gamma"),
            _len(gamma, None, "gamma"), _dev(beta, "float32", "beta"), _len(beta, None, "beta"), float(eps),
            None if out is None else _dev(out, "float32", "out"), 0 if out is None else _len(out, out_len, "out"),
            ldo, _dev(qa, "uint8", "qa"), _len(qa, None, "qa"), _dev(exps, "int32", "exps"), _len(exps, None, "exps"))
        _check(rc, self._ctx)

    def layer_norm_pair_quant_device(self, x, ldx: int, m: int, n: int, gamma, beta, eps: float, gamma2, beta2,
                                     eps2: float, qa, exps, x_len: Optional[int] = None):
        """A layer boundary: x = LayerNorm(x; gamma, beta) in place, then LayerNorm(x; gamma2, beta2) of
        the result quantised into qa and exps, the bits of layer_norm_device then layer_norm_quant_device."""
        rc = _lib.lib().tg_layer_norm_pair_quant_device(
            self._ctx, _dev(x, "float32", "x"), _len(x, x_len, "x"), ldx, m, n, _dev(gamma, "float32", "gamma"),
            _len(gamma, None, "gamma"), _dev(beta, "float32", "beta"), _len(beta, None, "beta"), float(eps),
            _dev(gamma2, "float32", "gamma2"), _len(gamma2, None, "gamma2"), _dev(beta2, "float32", "beta2"),
            _len(beta2, None, "beta2"), float(eps2), _dev(qa, "uint8", "qa"), _len(qa, None, "qa"),
            _dev(exps, "int32", "exps"), _len(exps, None, "exps"))
        _check(rc, self._ctx)

    def dwconv1d_device(self, x, ldx: int, frames: int, channels: int, w, kernel: int, bias, out, ldo: int,
                        rows: int = None, t0: int = 0, stride: int = 1, act: "Act" = None, batch: int = 1,
                        x_len: Optional[int] = None, out_len: Optional[int] = None):
        """Depthwise convolution of GPU tensor x (frames x channels) into out: row r is
        dwconv1d_frame at frame t0 + r * stride (rows defaults to frames), then SiLU when act is
        Act.SILU, as the conv module applies it. batch equal-length sequences of frames rows
        (rows output rows each) laid one after another are convolved each on its own."""
        rows = frames if rows is None else rows
        a = int(Act.NONE if act is None else act)
        xp = _dev(x, "float32", "x") if x is not None else None
        xl = _len(x, x_len, "x") if x is not None else 0
        rc = _lib.lib().tg_dwconv1d_device(self._ctx, xp, xl, ldx, frames, batch, channels,
                                           _dev(w, "float32", "w"), _len(w, None, "w"), kernel,
                                           _dev(bias, "float32", "bias"), _len(bias, None, "bias"),
                                           t0, stride, rows, a, _dev(out, "float32", "out"),
                                           _len(out, out_len, "out"), ldo)
        _check(rc, self._ctx)

    def dwconv1d_quant_device(self, x, ldx: int, frames: int, channels: int, w, kernel: int, bias, qa, exps,
                              act: "Act" = None, batch: int = 1, out=None, ldo: int = 0,
                              x_len: Optional[int] = None, out_len: Optional[int] = None) -> bool:
        """dwconv1d_device of whole sequences (rows = frames, t0 = 0, stride 1) writing its output
        rows quantised into qa / exps, as quantize_rows_device would write them (k = channels);
        out (optional) also receives the f32 rows. Returns False, with nothing queued, when the
        fused kernel does not take the shape (channels beyond 2048 or kernel beyond 32): the caller
        then makes the two calls."""
        a = int(Act.NONE if act is None else act)
        rc = _lib.lib().tg_dwconv1d_quant_device(
            self._ctx, _dev(x, "float32", "x"), _len(x, x_len, "x"), ldx, frames, batch, channels,
            _dev(w, "float32", "w"), _len(w, None, "w"), kernel, _dev(bias, "float32", "bias"),
            _len(bias, None, "bias"), a, _dev(out, "float32", "out") if out is not None else None,
            _len(out, out_len, "out") if out is not None else 0, ldo, _dev(qa, "uint8", "qa"),
            _len(qa, None, "qa"), _dev(exps, "int32", "exps"), _len(exps, None, "exps"))
        if rc == TG_ERR_UNSUPPORTED:
            return False
        _check(rc, self._ctx)
        return True

    def synchronize(self) -> None:
        _check(_lib.lib().tg_synchronize(self._ctx), self._ctx)


class Token(NamedTuple):
    """An emitted token (src/parakeet.rs Token): id, frame (relative to enc_proj's first row) and
    duration."""
    id: int
    frame: int
    duration: int


class TdtDecoder:
    """Parakeet's prediction network and joint on the GPU (src/parakeet.rs:1412-1577): int8 or Q8_0
    PackedWeights for the joint ((vocab + durations) x h), the LSTM layers (4h x 2h, gates i, f, g,
    o of [x; h_l]) and the projection (h x h); biases and the embedding (vocab x h) as float32 GPU
    tensors. The blank is the last token. The weights and tensors are held, not copied."""

    def __init__(self, kernels: "Kernels", hidden: int, vocab: int, durations, max_symbols: int,
                 joint: PackedWeights, joint_bias, embedding, lstm, lstm_bias, proj: PackedWeights, proj_bias):
        self._kernels = kernels
        self._keep = (joint, joint_bias, embedding, list(lstm), list(lstm_bias), proj, proj_bias)
        self.hidden, self.vocab, self.max_symbols = hidden, vocab, max_symbols
        self.layers = len(lstm)
        self.durations = [int(d) for d in durations]
        self._durs = (ctypes.c_int32 * len(self.durations))(*self.durations)
        desc = _lib.TdtDesc()
        desc.hidden, desc.vocab, desc.max_symbols, desc.layers = hidden, vocab, max_symbols, len(lstm)
        desc.durations = ctypes.cast(self._durs, ctypes.POINTER(ctypes.c_int32))
        desc.n_durations = len(self.durations)
        desc.joint, desc.joint_bias = joint._handle, _dev(joint_bias, "float32", "joint_bias").value
        desc.joint_bias_len = _len(joint_bias, None, "joint_bias")
        desc.embedding = _dev(embedding, "float32", "embedding").value
        desc.embedding_len = _len(embedding, None, "embedding")
        if len(lstm) > 4 or len(lstm) != len(lstm_bias):
            raise ValueError("1 to 4 LSTM layers, each with its bias")
        for i, (w, b) in enumerate(zip(lstm, lstm_bias)):
            desc.lstm[i] = w._handle
            desc.lstm_bias[i] = _dev(b, "float32", "lstm_bias").value
            desc.lstm_bias_len[i] = _len(b, None, "lstm_bias")
        desc.proj, desc.proj_bias = proj._handle, _dev(proj_bias, "float32", "proj_bias").value
        desc.proj_bias_len = _len(proj_bias, None, "proj_bias")
        handle = ctypes.c_void_p()
        _check(_lib.lib().tg_tdt_create(kernels._ctx, ctypes.addressof(desc), ctypes.byref(handle)), kernels._ctx)
        self._handle = handle

    def max_rows(self) -> int:
        return int(_lib.lib().tg_tdt_max_rows(self._handle))

    def predict_rows(self, tokens, states, preds) -> None:
        """predict_rows: each token runs through the LSTM layers with its row of states (GPU tensor,
        rows x layers x [h, c]), updated in place; preds (rows x h) gets the projection."""
        toks = (ctypes.c_int32 * max(len(tokens), 1))(*[int(t) for t in tokens])
        _check(_lib.lib().tg_tdt_predict_device(self._kernels._ctx, self._handle, ctypes.addressof(toks), len(tokens),
                                                _dev(states, "float32", "states"), _len(states, None, "states"),
                                                _dev(preds, "float32", "preds"), _len(preds, None, "preds")),
               self._kernels._ctx)

    @property
    def resident(self) -> bool:
        """Whether decode runs resident: one launch for the steps, the matrices held in LDS."""
        return bool(_lib.lib().tg_tdt_is_resident(self._handle))

    def set_resident(self, on: bool) -> None:
        """Resident decode (raises where the network cannot run it) or one graph of step kernels."""
        _check(_lib.lib().tg_tdt_set_resident(self._kernels._ctx, self._handle, 1 if on else 0), self._kernels._ctx)

    @property
    def last_resident(self) -> Optional[int]:
        """How the last decode ran: 1 resident, 0 on the step kernels, 2 several streams in one
        resident launch; None before the first. A decode falls back to the step kernels while
        another one holds the device resident."""
        v = int(_lib.lib().tg_tdt_last_resident(self._handle))
        return None if v < 0 else v

    @property
    def last_steps(self) -> int:
        """Steps of the last resident decode (one step scores one window of frames per stream)."""
        return int(_lib.lib().tg_tdt_last_steps(self._handle))

    def set_resident_limits(self, steps_per_launch: int = 0, wait_us: int = 0) -> None:
        """The resident decode's steps per launch (0: 16384) and longest wait between workgroups in
        microseconds (0: one second); a wait past it fails the decode and leaves state and pred as
        they were passed."""
        _check(_lib.lib().tg_tdt_set_resident_limits(self._kernels._ctx, self._handle, steps_per_launch, wait_us),
               self._kernels._ctx)

    def decode(self, enc_proj, state, pred, frame: int = 0, on_frame: int = 0, cap: Optional[int] = None):
        """The greedy decode over the rows of enc_proj (GPU tensor, frames x >= h) from frame with
        on_frame tokens on it; state (layers x [h, c]) and pred (h) are updated in place. Returns
        (tokens, frame, on_frame)."""
        if enc_proj.dim() != 2 or enc_proj.stride(1) != 1:
            raise ValueError("enc_proj must be a 2-D tensor whose rows are contiguous")
        frames = enc_proj.shape[0]
        if cap is None:
            cap = max(frames - frame, 0) * max(self.max_symbols, 1)
        out = (_lib.Token * max(cap, 1))()
        f, o, n = ctypes.c_size_t(frame), ctypes.c_size_t(on_frame), ctypes.c_size_t(0)
        enc_len = (frames - 1) * enc_proj.stride(0) + enc_proj.shape[1] if frames else 0
        rc = _lib.lib().tg_tdt_decode_device(self._kernels._ctx, self._handle, _dev(enc_proj, "float32", "enc_proj"),
                                             _len(enc_proj, enc_len, "enc_proj"), enc_proj.stride(0), frames,
                                             _dev(state, "float32", "state"), _len(state, None, "state"),
                                             _dev(pred, "float32", "pred"), _len(pred, None, "pred"),
                                             ctypes.byref(f), ctypes.byref(o), ctypes.addressof(out), cap,
                                             ctypes.byref(n))
        _check(rc, self._kernels._ctx)
        return [Token(t.id, t.frame, t.duration) for t in out[:n.value]], f.value, o.value

    def decode_streams(self, encs, states, preds, frames=None, caps=None):
        """Several independent greedy decodes (tg_tdt_decode_streams_device): encs, states and preds
        are per-stream GPU tensors as decode takes them, each stream from frame 0 (or frames[i]).
        Returns [(tokens, frame, on_frame)] per stream, what decode returns for each."""
        m = len(encs)
        arr = (_lib.TdtStream * max(m, 1))()
        outs = []
        for i, (e, st, pr) in enumerate(zip(encs, states, preds)):
            if e.dim() != 2 or e.stride(1) != 1:
                raise ValueError("enc_proj must be a 2-D tensor whose rows are contiguous")
            nf = e.shape[0]
            f0 = 0 if frames is None else frames[i]
            cap = max(nf - f0, 0) * max(self.max_symbols, 1) if caps is None else caps[i]
            out = (_lib.Token * max(cap, 1))()
            outs.append(out)
            enc_len = (nf - 1) * e.stride(0) + e.shape[1] if nf else 0
            s = arr[i]
            s.enc_proj, s.enc_len, s.lde, s.frames = _dev(e, "float32", "enc_proj").value, _len(e, enc_len, "enc_proj"), \
                e.stride(0), nf
            s.state, s.state_len = _dev(st, "float32", "state").value, _len(st, None, "state")
            s.pred, s.pred_len = _dev(pr, "float32", "pred").value, _len(pr, None, "pred")
            s.frame, s.on_frame, s.tokens, s.cap = f0, 0, ctypes.addressof(out), cap
        rc = _lib.lib().tg_tdt_decode_streams_device(self._kernels._ctx, self._handle, ctypes.addressof(arr), m)
        _check(rc, self._kernels._ctx)
        return [([Token(t.id, t.frame, t.duration) for t in outs[i][:arr[i].count]], arr[i].frame, arr[i].on_frame)
                for i in range(m)]

    def close(self) -> None:
        if self._handle:
            _lib.lib().tg_tdt_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
