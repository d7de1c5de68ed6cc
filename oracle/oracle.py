"""ctypes view of the oracle library (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this module,
and only to check results against. The product (``telmo_amd``) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
CPUBASE = os.path.join(HERE, "libcpubase.so")

F32, F16, BF16, INT8, Q8_0 = range(5)
NONE, RELU, SILU = range(3)
EXP_NONFINITE = -(2**31)

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_sz = ctypes.c_size_t


def build():
    """Compile the oracle libraries in place (gcc/g++ only)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        L.or_random.argtypes = [_f32p, _sz, ctypes.c_uint64]
        L.or_value_bytes.argtypes = [ctypes.c_int]
        L.or_value_bytes.restype = _sz
        L.or_panel_bytes.argtypes = [ctypes.c_int, _sz, _sz]
        L.or_panel_bytes.restype = _sz
        L.or_scale_count.argtypes = [ctypes.c_int, _sz, _sz]
        L.or_scale_count.restype = _sz
        L.or_fits.argtypes = [ctypes.c_int, _sz]
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f32_to_bf16.argtypes = [ctypes.c_float]
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_bf16_to_f32.restype = ctypes.c_float
        L.or_quantize_q8_0_block.argtypes = [_f32p, _sz, _i8p]
        L.or_quantize_q8_0_block.restype = ctypes.c_float
        L.or_quantize_row_int8.argtypes = [_f32p, _sz, _i8p]
        L.or_quantize_row_int8.restype = ctypes.c_float
        L.or_encode_f32.argtypes = [_f32p, _sz, _sz, ctypes.c_int, _u8p, _f32p]
        L.or_encode_q8.argtypes = [_f32p, _i8p, _sz, _sz, ctypes.c_int, _u8p, _f32p]
        L.or_decode.argtypes = [_u8p, _f32p, _sz, _sz, ctypes.c_int, _f32p]
        L.or_widen.argtypes = [ctypes.c_int, _sz, _u8p, _f32p, _f32p]
        L.or_tile.argtypes = [ctypes.c_int, _sz, _f32p, _sz, _sz, _f32p, _sz, _f32p, ctypes.c_int]
        L.or_exp_simd.argtypes = [ctypes.c_float]
        L.or_exp_simd.restype = ctypes.c_float
        L.or_silu_simd.argtypes = [ctypes.c_float]
        L.or_silu_simd.restype = ctypes.c_float
        L.or_glu.argtypes = [_f32p, _f32p, _f32p, _sz]
        L.or_layer_norm.argtypes = [_f32p, _sz, _f32p, _f32p, _f32p, ctypes.c_float]
        L.or_softmax.argtypes = [_f32p, _sz]
        _vp = ctypes.c_void_p
        L.or_tdt_predict.argtypes = [ctypes.c_int, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _vp]
        L.or_tdt_decode.argtypes = [ctypes.c_int, _sz, _sz, _sz, _vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                    _vp, _vp, _vp, _vp, _sz, _sz, _vp, _vp, ctypes.POINTER(_sz),
                                    ctypes.POINTER(_sz), _vp, _sz]
        L.or_tdt_decode.restype = _sz
        L.or_dwconv1d_frame.argtypes = [_f32p, _sz, _sz, _sz, _f32p, _sz, _f32p, _f32p]
        L.or_dwconv1d.argtypes = [_f32p, _sz, _sz, _sz, _f32p, _sz, _f32p, _sz, _sz, _sz, ctypes.c_int,
                                  _f32p, _sz]
        L.or_store.argtypes = [ctypes.c_int, _f32p, _f32p, _sz, ctypes.c_void_p, ctypes.c_int, ctypes.c_float,
                               ctypes.c_int]
        mm = [_f32p, _sz, _sz, _sz, _u8p, ctypes.c_void_p, ctypes.c_int, _sz, _sz, _f32p, _sz, _sz,
              ctypes.c_void_p, _sz, ctypes.c_int, ctypes.c_float, ctypes.c_int]
        L.or_matmul.argtypes = [ctypes.c_int] + mm
        L.or_matmul_fast.argtypes = [_f32p, _sz, _sz, _sz, _u8p, _f32p, _sz, _sz, _f32p, _sz, _sz,
                                     ctypes.c_void_p, _sz, ctypes.c_int, ctypes.c_float, ctypes.c_int]
        L.or_matmul_fast_q8.argtypes = L.or_matmul_fast.argtypes
        L.or_row_exponent.argtypes = [_f32p, _sz]
        L.or_guard_flag.argtypes = [_f32p, _sz]
        L.or_guard_flag.restype = ctypes.c_int
        L.or_row_exponent.restype = ctypes.c_int32
        L.or_quantize_rows.argtypes = [_f32p, _sz, _sz, _sz, _i8p, _i8p, _i32p]
        L.or_int_products.argtypes = [_i8p, _i8p, _sz, _sz, _i8p, _sz, _i32p, _i32p]
        L.or_dequant.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_float]
        L.or_dequant.restype = ctypes.c_float
        _lib = L
    return _lib


def _ptr(x):
    return None if x is None else x.ctypes.data_as(ctypes.c_void_p)


def random(length, seed):
    """The reference's xorshift test generator: `length` values in [-1, 1)."""
    out = np.empty(length, np.float32)
    lib().or_random(out, length, seed)
    return out


def value_bytes(p):
    return lib().or_value_bytes(p)


def panel_bytes(p, n, k):
    return lib().or_panel_bytes(p, n, k)


def scale_count(p, n, k):
    return lib().or_scale_count(p, n, k)


def fits(p, k):
    return bool(lib().or_fits(p, k))


def f32_to_f16(x):
    return lib().or_f32_to_f16(float(x))


def f16_to_f32(h):
    return np.float32(lib().or_f16_to_f32(int(h)))


def f32_to_bf16(x):
    return lib().or_f32_to_bf16(float(x))


def bf16_to_f32(h):
    return np.float32(lib().or_bf16_to_f32(int(h)))


def quantize_q8_0_block(x):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(len(x), np.int8)
    d = lib().or_quantize_q8_0_block(x, len(x), q)
    return np.float32(d), q


def quantize_row_int8(x):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(len(x), np.int8)
    d = lib().or_quantize_row_int8(x, len(x), q)
    return np.float32(d), q


def encode(w, n, k, p):
    """Row-major [n, k] f32 rows into the panel layout: (values u8, scales f32)."""
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    values = np.zeros(panel_bytes(p, n, k), np.uint8)
    scales = np.zeros(max(scale_count(p, n, k), 1), np.float32)
    rc = lib().or_encode_f32(w if w.size else np.zeros(1, np.float32), n, k, p, values if values.size else
                             np.zeros(1, np.uint8), scales)
    if rc != 0:
        raise ValueError(f"encode failed ({rc})")
    return values, scales[: scale_count(p, n, k)]


def encode_q8(d, q, n, k, p):
    """Q8_0 blocks (d: n*k/32 scales, q: n*k values) into the panel layout of precision p."""
    d = np.ascontiguousarray(d, np.float32)
    q = np.ascontiguousarray(q, np.int8)
    values = np.zeros(max(panel_bytes(p, n, k), 1), np.uint8)
    scales = np.zeros(max(scale_count(p, n, k), 1), np.float32)
    rc = lib().or_encode_q8(d, q, n, k, p, values, scales)
    if rc != 0:
        raise ValueError(f"encode failed ({rc})")
    return values[: panel_bytes(p, n, k)], scales[: scale_count(p, n, k)]


def decode(values, scales, n, k, p):
    out = np.zeros(max(n * k, 1), np.float32)
    values = np.ascontiguousarray(values, np.uint8)
    scales = np.ascontiguousarray(scales if scales is not None and len(scales) else np.zeros(1), np.float32)
    lib().or_decode(values if values.size else np.zeros(1, np.uint8), scales, n, k, p, out)
    return out[: n * k].reshape(n, k)


def widen(p, k, src, scales):
    out = np.zeros(max(k * 16, 1), np.float32)
    scales = np.ascontiguousarray(scales if scales is not None and len(scales) else np.zeros(1), np.float32)
    lib().or_widen(p, k, np.ascontiguousarray(src, np.uint8), scales, out)
    return out[: k * 16].reshape(k, 16)


def tile(fused, k, a, lda, rows, b, k_stride, out, load):
    lib().or_tile(int(fused), k, a, lda, rows, b, k_stride, out, int(load))


def exp_simd(x):
    return np.float32(lib().or_exp_simd(float(x)))


def silu_simd(x):
    return np.float32(lib().or_silu_simd(float(x)))


def glu(a, b):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    out = np.zeros_like(a)
    lib().or_glu(a, b, out, a.size)
    return out


def layer_norm(x, gamma, beta, eps):
    """One row, the reference's AVX-512 order."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    lib().or_layer_norm(x, x.size, out, np.ascontiguousarray(gamma, np.float32),
                        np.ascontiguousarray(beta, np.float32), float(eps))
    return out


def softmax(x):
    """One row (or each row of a 2-D array), the reference's AVX-512 softmax; returns a copy."""
    x = np.array(x, dtype=np.float32, copy=True)
    rows = x.reshape(-1, x.shape[-1]) if x.ndim > 1 else x.reshape(1, -1)
    for r in range(rows.shape[0]):
        row = np.ascontiguousarray(rows[r])
        lib().or_softmax(row, row.size)
        rows[r] = row
    return rows.reshape(x.shape)


def dwconv1d_frame(x, t, w, bias):
    """One output frame of the depthwise convolution over x [frames, channels], w [kernel, channels]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    frames, channels = x.shape
    out = np.empty(channels, np.float32)
    lib().or_dwconv1d_frame(x.reshape(-1) if x.size else np.zeros(1, np.float32), channels, frames, t,
                            w.reshape(-1) if w.size else np.zeros(1, np.float32), w.shape[0],
                            np.ascontiguousarray(bias, np.float32), out)
    return out


def dwconv1d(x, w, bias, rows=None, t0=0, stride=1, silu=False):
    """Output rows r = 0 .. rows - 1 of dwconv1d_frame at t0 + r * stride, then SiLU when silu."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    frames, channels = x.shape
    rows = frames if rows is None else rows
    out = np.empty((rows, channels), np.float32)
    if rows:
        lib().or_dwconv1d(x.reshape(-1) if x.size else np.zeros(1, np.float32), channels, frames, channels,
                          w.reshape(-1) if w.size else np.zeros(1, np.float32), w.shape[0],
                          np.ascontiguousarray(bias, np.float32), t0, stride, rows, int(silu), out.reshape(-1),
                          channels)
    return out


def _addr(x):
    return x.ctypes.data_as(ctypes.c_void_p)


def _tdt_common(net):
    """Pointer arrays of a TDT network (a dict of contiguous numpy arrays; see tests/helpers.py)."""
    L = len(net["lstm"])
    keep = [net["emb"], net["proj"][0], net["proj"][1], net["proj_b"]]
    lv = (ctypes.c_void_p * L)(*[w[0].ctypes.data for w in net["lstm"]])
    ls = (ctypes.c_void_p * L)(*[w[1].ctypes.data for w in net["lstm"]])
    lb = (ctypes.c_void_p * L)(*[b.ctypes.data for b in net["lstm_b"]])
    return keep, lv, ls, lb


def tdt_predict(net, tokens, states, preds):
    """predict_rows in place: states [rows, layers * 2h] and preds [rows, h] (float32, C order)."""
    keep, lv, ls, lb = _tdt_common(net)
    toks = np.ascontiguousarray(tokens, np.int32)
    lib().or_tdt_predict(net["p"], net["h"], len(net["lstm"]), _addr(net["emb"]), lv, ls, lb, _addr(net["proj"][0]),
                         _addr(net["proj"][1]), _addr(net["proj_b"]), _addr(toks), toks.size, _addr(states),
                         _addr(preds))


def tdt_decode(net, enc, state, pred, frame=0, on_frame=0):
    """decode_inner over the rows of enc [frames, h]: returns ([(id, frame, duration)], frame,
    on_frame); state [layers * 2h] and pred [h] are updated in place."""
    keep, lv, ls, lb = _tdt_common(net)
    enc = np.ascontiguousarray(enc, np.float32)
    frames = enc.shape[0]
    durs = np.ascontiguousarray(net["durations"], np.int32)
    cap = max(frames - frame, 0) * max(net["max_symbols"], 1) + 1
    toks = np.zeros(3 * cap, np.int32)
    f, o = ctypes.c_size_t(frame), ctypes.c_size_t(on_frame)
    n = lib().or_tdt_decode(net["p"], net["h"], len(net["lstm"]), net["vocab"], _addr(durs), durs.size,
                            net["max_symbols"], _addr(net["joint"][0]), _addr(net["joint"][1]),
                            _addr(net["joint_b"]), _addr(net["emb"]), lv, ls, lb, _addr(net["proj"][0]),
                            _addr(net["proj"][1]), _addr(net["proj_b"]), _addr(enc), enc.shape[1], frames,
                            _addr(state), _addr(pred), ctypes.byref(f), ctypes.byref(o), _addr(toks), cap)
    return [tuple(int(v) for v in toks[3 * i:3 * i + 3]) for i in range(n)], f.value, o.value


_CB = None


def cpubase():
    """The CPU baseline library (the C++ port of telmo's SIMD + pool path)."""
    global _CB
    if _CB is None:
        L = ctypes.CDLL(CPUBASE)
        L.cb_isa.restype = ctypes.c_int
        L.cb_pool_new.restype = ctypes.c_void_p
        L.cb_pool_new.argtypes = [ctypes.c_size_t]
        L.cb_pool_free.argtypes = [ctypes.c_void_p]
        sz, vp = ctypes.c_size_t, ctypes.c_void_p
        L.cb_tdt_decode.restype = ctypes.c_long
        L.cb_tdt_decode.argtypes = [vp, ctypes.c_int, ctypes.c_int, sz, sz, sz, vp, sz, sz, vp, vp, vp, vp, vp, vp,
                                    vp, vp, vp, vp, vp, sz, sz, vp, vp, vp, vp, vp, sz]
        _CB = L
    return _CB


def cpu_tdt_decode(net, enc, state, pred, pool, frame=0, on_frame=0, isa=0):
    """decode_inner on the CPU baseline's pool `pool` (from cpubase().cb_pool_new): the same
    arguments and results as tdt_decode, every product by the SIMD port."""
    keep, lv, ls, lb = _tdt_common(net)
    enc = np.ascontiguousarray(enc, np.float32)
    frames = enc.shape[0]
    durs = np.ascontiguousarray(net["durations"], np.int32)
    cap = max(frames - frame, 0) * max(net["max_symbols"], 1) + 1
    toks = np.zeros(3 * cap, np.int32)
    f, o = ctypes.c_size_t(frame), ctypes.c_size_t(on_frame)
    n = cpubase().cb_tdt_decode(pool, isa, net["p"], net["h"], len(net["lstm"]), net["vocab"], _addr(durs), durs.size,
                                net["max_symbols"], _addr(net["joint"][0]), _addr(net["joint"][1]),
                                _addr(net["joint_b"]), _addr(net["emb"]), lv, ls, lb, _addr(net["proj"][0]),
                                _addr(net["proj"][1]), _addr(net["proj_b"]), _addr(enc), enc.shape[1], frames,
                                _addr(state), _addr(pred), ctypes.byref(f), ctypes.byref(o), _addr(toks), cap)
    if n < 0:
        raise RuntimeError(f"cb_tdt_decode failed ({n})")
    return [tuple(int(v) for v in toks[3 * i:3 * i + 3]) for i in range(n)], f.value, o.value


def store(fused, acc, c, cols, bias, act, scale, accumulate):
    lib().or_store(int(fused), acc, c, cols, _ptr(bias), act, scale, int(accumulate))


def matmul(fused, a, lda, m, values, scales, p, n, k, c, ldc, bias=None, act=NONE, scale=1.0,
           accumulate=False):
    """Kernels::matmul over packed weights, in place on `c`. Returns the status (0 or negative)."""
    scales = None if scales is None or len(scales) == 0 else np.ascontiguousarray(scales, np.float32)
    return lib().or_matmul(int(fused), a, a.size, lda, m, values, _ptr(scales), p, n, k, c, c.size, ldc,
                           _ptr(bias), 0 if bias is None else bias.size, act, scale, int(accumulate))


def guard_flags(a, lda, m, k):
    """The accuracy guard's flag of each of m rows of a (rows lda apart)."""
    a = np.ascontiguousarray(a, np.float32)
    return np.array([lib().or_guard_flag(np.ascontiguousarray(a[r * lda:r * lda + k]) if k else
                                         np.zeros(1, np.float32), k) for r in range(m)], np.int32)


def _guarded(fast, a, lda, m, values, scales, p, n, k, c, ldc, bias, act, scale, accumulate, guard):
    """A fast-path oracle with the accuracy guard: flagged rows take the fused reference (or_matmul)
    on their own, accumulating onto the row as it was before the call."""
    if not guard or m == 0 or n == 0:
        return fast()
    flags = guard_flags(a, lda, m, k)
    old = {r: c[r * ldc:r * ldc + n].copy() for r in np.flatnonzero(flags)}
    rc = fast()
    if rc:
        return rc
    for r, row_c in old.items():
        ar = np.ascontiguousarray(a[r * lda:r * lda + k]) if k else np.zeros(1, np.float32)
        rc = matmul(True, ar, k, 1, values, scales, p, n, k, row_c, n, bias, act, scale, accumulate)
        if rc:
            return rc
        c[r * ldc:r * ldc + n] = row_c
    return 0


def matmul_fast(a, lda, m, values, scales, n, k, c, ldc, bias=None, act=NONE, scale=1.0, accumulate=False,
                guard=False):
    """The integer oracle of the fast int8 path, in place on `c`; guard: the product entry points'
    accuracy guard (rows it flags take the fused reference)."""
    fast = lambda: lib().or_matmul_fast(a, a.size, lda, m, values, scales, n, k, c, c.size, ldc,  # noqa: E731
                                        _ptr(bias), 0 if bias is None else bias.size, act, scale, int(accumulate))
    return _guarded(fast, a, lda, m, values, scales, INT8, n, k, c, ldc, bias, act, scale, accumulate, guard)


def matmul_fast_q8(a, lda, m, values, scales, n, k, c, ldc, bias=None, act=NONE, scale=1.0, accumulate=False,
                   guard=False):
    """The integer oracle of the fast Q8_0 path (block sums scaled in block order), in place on `c`;
    guard as matmul_fast."""
    fast = lambda: lib().or_matmul_fast_q8(a, a.size, lda, m, values, scales, n, k, c, c.size, ldc,  # noqa: E731
                                           _ptr(bias), 0 if bias is None else bias.size, act, scale,
                                           int(accumulate))
    return _guarded(fast, a, lda, m, values, scales, Q8_0, n, k, c, ldc, bias, act, scale, accumulate, guard)


def row_exponent(row):
    row = np.ascontiguousarray(row, np.float32)
    return lib().or_row_exponent(row if row.size else np.zeros(1, np.float32), row.size)


def quantize_rows(a, lda, m, k):
    hi = np.zeros(max(m * k, 1), np.int8)
    lo = np.zeros(max(m * k, 1), np.int8)
    ex = np.zeros(max(m, 1), np.int32)
    lib().or_quantize_rows(a, lda, m, k, hi, lo, ex)
    return hi[: m * k].reshape(m, k), lo[: m * k].reshape(m, k), ex[:m]


def int_products(hi, lo, q):
    """acc_hi, acc_lo [m, n] of digit planes [m, k] against int8 q [n, k]."""
    m, k = hi.shape
    n = q.shape[0]
    acc_hi = np.zeros(max(m * n, 1), np.int32)
    acc_lo = np.zeros(max(m * n, 1), np.int32)
    lib().or_int_products(np.ascontiguousarray(hi), np.ascontiguousarray(lo), m, k, np.ascontiguousarray(q), n,
                          acc_hi, acc_lo)
    return acc_hi[: m * n].reshape(m, n), acc_lo[: m * n].reshape(m, n)


def dequant(acc_hi, acc_lo, e, scale):
    return np.float32(lib().or_dequant(int(acc_hi), int(acc_lo), int(e), float(scale)))
