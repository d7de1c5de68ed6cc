"""Loads libtelmo_hip.so (built in place by telmo_amd.build) and declares its C ABI."""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libtelmo_hip.so")

_sz = ctypes.c_size_t
_p = ctypes.c_void_p
_u32 = ctypes.c_uint32



class TdtDesc(ctypes.Structure):
    """tg_tdt_desc."""
    _fields_ = [("hidden", _sz), ("vocab", _sz), ("durations", ctypes.POINTER(ctypes.c_int32)),
                ("n_durations", _sz), ("max_symbols", _sz), ("layers", _sz), ("joint", _p), ("joint_bias", _p),
                ("embedding", _p), ("lstm", _p * 4), ("lstm_bias", _p * 4), ("proj", _p), ("proj_bias", _p),
                ("joint_bias_len", _sz), ("embedding_len", _sz), ("lstm_bias_len", _sz * 4), ("proj_bias_len", _sz)]


class Token(ctypes.Structure):
    """tg_token."""
    _fields_ = [("id", ctypes.c_uint32), ("frame", ctypes.c_uint32), ("duration", ctypes.c_uint32)]


class TdtStream(ctypes.Structure):
    """tg_tdt_stream."""
    _fields_ = [("enc_proj", _p), ("enc_len", _sz), ("lde", _sz), ("frames", _sz), ("state", _p), ("state_len", _sz),
                ("pred", _p), ("pred_len", _sz), ("frame", _sz), ("on_frame", _sz), ("tokens", _p), ("cap", _sz),
                ("count", _sz)]


_szp = ctypes.POINTER(_sz)

# name: (restype, argtypes), in the order of include/telmo_hip.h
SIGNATURES = {
    "tg_ctx_create": (ctypes.c_int, [ctypes.c_int, _p, ctypes.POINTER(_p)]),
    "tg_ctx_destroy": (None, [_p]),
    "tg_ctx_set_mode": (ctypes.c_int, [_p, _u32]),
    "tg_ctx_mode": (_u32, [_p]),
    "tg_ctx_set_guard": (ctypes.c_int, [_p, ctypes.c_int]),
    "tg_ctx_guard": (ctypes.c_int, [_p]),
    "tg_last_error": (ctypes.c_char_p, [_p]),
    "tg_synchronize": (ctypes.c_int, [_p]),
    "tg_weights_upload": (ctypes.c_int, [_p, _p, _sz, _p, _sz, _u32, _sz, _sz, ctypes.POINTER(_p)]),
    "tg_weights_upload_device": (ctypes.c_int, [_p, _p, _sz, _p, _sz, _u32, _sz, _sz, ctypes.POINTER(_p)]),
    "tg_weights_free": (None, [_p]),
    "tg_weights_bytes": (_sz, [_p]),
    "tg_weights_n": (_sz, [_p]),
    "tg_weights_k": (_sz, [_p]),
    "tg_weights_precision": (_u32, [_p]),
    "tg_matmul": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _p, _p, _sz, _sz, _p]),
    "tg_linear": (ctypes.c_int, [_p, _p, _sz, _sz, _p, _p, _sz, _p]),
    "tg_matmul_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _p, _p, _sz, _sz, _p]),
    "tg_linear_device": (ctypes.c_int, [_p, _p, _sz, _sz, _p, _p, _sz, _p]),
    "tg_matmul_device_noalloc": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _p, _p, _sz, _sz, _p]),
    "tg_matmul_rowmajor_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _p, _sz, _sz, _sz, _sz, _p, _sz, _sz, _p]),
    "tg_quant_bytes": (_sz, [_sz, _sz]),
    "tg_quantize_rows_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _sz, _p, _sz, _p]),
    "tg_matmul_quantized_device": (ctypes.c_int, [_p, _p, _sz, _p, _sz, _p, _p, _sz, _sz, _p]),
    "tg_matmul_quantized_glu_device": (ctypes.c_int, [_p, _p, _sz, _p, _sz, _p, _p, _sz, _sz, _p]),
    "tg_matmul_quantized_to_quant_device": (ctypes.c_int, [_p, _p, _sz, _p, _sz, _p, _p, _p, _sz, _p, _sz]),
    "tg_glu_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _sz, _p, _sz, _sz]),
    "tg_softmax_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _sz]),
    "tg_average_pairs_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _sz, _sz, _p, _sz, _sz]),
    "tg_linear_glu_device": (ctypes.c_int, [_p, _p, _sz, _sz, _p, _p, _sz, _sz, _p]),
    "tg_layer_norm_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _sz, _p, _sz, _p, _sz, ctypes.c_float, _p, _sz,
                                             _sz]),
    "tg_layer_norm_quant_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _sz, _p, _sz, _p, _sz, ctypes.c_float, _p,
                                                   _sz, _sz, _p, _sz, _p, _sz]),
    "tg_layer_norm_pair_quant_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _sz, _p, _sz, _p, _sz, ctypes.c_float,
                                                        _p, _sz, _p, _sz, ctypes.c_float, _p, _sz, _p, _sz]),
    "tg_dwconv1d_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _sz, _sz, _p, _sz, _sz, _p, _sz, _sz, _sz, _sz,
                                           _u32, _p, _sz, _sz]),
    "tg_dwconv1d_quant_device": (ctypes.c_int, [_p, _p, _sz, _sz, _sz, _sz, _sz, _p, _sz, _sz, _p, _sz, _u32, _p,
                                                 _sz, _sz, _p, _sz, _p, _sz]),
    "tg_tdt_create": (ctypes.c_int, [_p, _p, ctypes.POINTER(_p)]),
    "tg_tdt_destroy": (None, [_p]),
    "tg_tdt_max_rows": (_sz, [_p]),
    "tg_tdt_predict_device": (ctypes.c_int, [_p, _p, _p, _sz, _p, _sz, _p, _sz]),
    "tg_tdt_decode_device": (ctypes.c_int, [_p, _p, _p, _sz, _sz, _sz, _p, _sz, _p, _sz, _szp, _szp, _p, _sz,
                                             _szp]),
    "tg_tdt_set_resident": (ctypes.c_int, [_p, _p, ctypes.c_int]),
    "tg_tdt_is_resident": (ctypes.c_int, [_p]),
    "tg_tdt_last_resident": (ctypes.c_int, [_p]),
    "tg_tdt_last_steps": (_sz, [_p]),
    "tg_tdt_decode_streams_device": (ctypes.c_int, [_p, _p, _p, _sz]),
    "tg_tdt_set_resident_limits": (ctypes.c_int, [_p, _p, _u32, ctypes.c_uint64]),
    "tg_pack_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_p)]),
    "tg_pack_from_bytes": (ctypes.c_int, [_p, _sz, ctypes.POINTER(_p)]),
    "tg_pack_close": (None, [_p]),
    "tg_pack_last_error": (ctypes.c_char_p, []),
    "tg_pack_is_mapped": (ctypes.c_int, [_p]),
    "tg_pack_model": (ctypes.c_char_p, [_p]),
    "tg_pack_meta": (ctypes.c_char_p, [_p, ctypes.c_char_p]),
    "tg_pack_meta_count": (_sz, [_p]),
    "tg_pack_meta_at": (ctypes.c_int, [_p, _sz, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p)]),
    "tg_pack_entry_count": (_sz, [_p]),
    "tg_pack_entry_at": (ctypes.c_int, [_p, _sz, _p]),
    "tg_pack_find": (ctypes.c_int, [_p, ctypes.c_char_p, _p]),
    "tg_pack_upload_matrix": (ctypes.c_int, [_p, _p, ctypes.c_char_p, _sz, _sz, ctypes.POINTER(_p)]),
    "tg_panel_bytes": (_sz, [_u32, _sz, _sz]),
    "tg_scale_count": (_sz, [_u32, _sz, _sz]),
    "tg_fits": (ctypes.c_int, [_u32, _sz]),
    "tg_encode": (ctypes.c_int, [_p, _sz, _sz, _u32, _p, _sz, _p, _sz]),
    "tg_random": (None, [_p, _sz, ctypes.c_uint64]),
    "tg_decode": (ctypes.c_int, [_p, _sz, _p, _sz, _u32, _sz, _sz, _p]),
}

_lib = None


def _share_the_process_hip_runtime():
    """PyTorch-ROCm ships its own libamdhip64 / libhsa-runtime64 (same sonames, loaded by path).
    Two HIP runtimes in one process cannot both open the GPU, so when torch is installed it is
    loaded first: this library's dependencies then resolve to the runtime already in the
    process. Without torch the system ROCm runtime is used."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def lib():
    """The loaded library. Raises if it has not been built: there is no fallback."""
    global _lib
    if _lib is None:
        _share_the_process_hip_runtime()
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m telmo_amd.build` "
                               "(or __graft_entry__.build()); telmo_amd has no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib
