"""The C ABI without a GPU: the library loads, exports every entry point include/telmo_hip.h
declares, its host layout utilities match the oracle bit for bit, and its refusals follow the
reference's preconditions."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "telmo_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tg_[a-z0-9_]+)\s*\(", text)))


def test_the_library_exports_every_declared_entry_point():
    from telmo_amd import _lib

    names = declared_functions()
    assert len(names) >= 20
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in names:
        assert hasattr(raw, name), name
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_sizes_match_the_reference_layout(orc):
    from telmo_amd import Precision

    for p in Precision:
        for n, k in [(1, 1), (16, 32), (37, 64), (8198, 640), (4096, 1024)]:
            assert p.panel_bytes(n, k) == orc.panel_bytes(int(p), n, k)
            assert p.scale_count(n, k) == orc.scale_count(int(p), n, k)
        assert p.fits(64) and p.fits(33) == (p != Precision.Q8_0)
    assert Precision.from_name("q8_0") == Precision.Q8_0 and Precision.from_name("int4") is None


def test_host_encode_and_decode_match_the_oracle(orc):
    from telmo_amd import Precision, decode, encode

    for n, k in [(37, 64), (5, 7), (20, 96), (1, 1)]:
        i = np.arange(n * k)
        w = (orc.random(n * k, 5) * (1 + i // max(k, 1)).astype(np.float32)).astype(np.float32)
        w[::17] = 0.0
        for p in Precision:
            if not p.fits(k):
                continue
            v1, s1 = encode(w, n, k, p)
            v2, s2 = orc.encode(w, n, k, int(p))
            assert np.array_equal(v1, v2), (p, n, k)
            assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32)), (p, n, k)
            d1 = decode(v1, s1, n, k, p)
            d2 = orc.decode(v2, s2, n, k, int(p))
            assert np.array_equal(d1.view(np.uint32), d2.view(np.uint32)), (p, n, k)


def test_special_values_encode_like_the_oracle(orc):
    from telmo_amd import Precision, encode

    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65520.0, 65519.0, 2.0**-24, 2.0**-25,
                         1.5 * 2.0**-25, 3.4e38, 1e-40, -7.5, 1.0 + 2.0**-11] + [0.0] * 2, np.float32)
    for p in (Precision.F16, Precision.BF16):
        v1, _ = encode(specials, 1, specials.size, p)
        v2, _ = orc.encode(specials, 1, specials.size, int(p))
        assert np.array_equal(v1, v2), p


def test_encode_refuses_what_the_reference_refuses():
    from telmo_amd import Precision, TelmoError, encode

    with pytest.raises(TelmoError):
        encode(np.zeros(3 * 65, np.float32), 3, 65, Precision.Q8_0)


def test_entry_points_refuse_null_contexts_without_a_gpu():
    from telmo_amd import _lib

    L = _lib.lib()
    assert L.tg_ctx_set_mode(None, 0) == -1
    assert L.tg_synchronize(None) == -1
    assert L.tg_linear(None, None, 0, 0, None, None, 0, None) == -1
    assert L.tg_matmul_device(None, None, 0, 0, 0, None, None, 0, 0, None) == -1
    assert L.tg_last_error(None) == b"null context"
    out = ctypes.c_void_p()
    assert L.tg_ctx_create(0, None, None) == -1
    assert L.tg_weights_bytes(None) == 0
    L.tg_weights_free(None)
    L.tg_ctx_destroy(None)
    del out


def test_no_gpu_means_a_clean_error_not_a_fallback():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from telmo_amd import Kernels, TelmoError

    with pytest.raises(TelmoError):
        Kernels()


def test_gpu_tensors_are_checked_for_their_element_type_before_the_library_sees_them():
    """The lengths passed with a device pointer count elements of the type the library reads, so a
    half-precision or host tensor must never reach it: the wrapper refuses it first."""
    import torch

    from telmo_amd.kernels import _dev

    with pytest.raises(TypeError, match="a must be a float32 GPU tensor"):
        _dev(torch.zeros(4, dtype=torch.float32), "float32", "a")  # on the host
    with pytest.raises(TypeError, match="qa must be a uint8 GPU tensor"):
        _dev(torch.zeros(4, dtype=torch.int8), "uint8", "qa")


def test_half_and_bfloat16_encodings_match_the_oracle_over_many_bit_patterns(orc):
    """layout.cpp rounds on the value (frexp, ldexp, nearbyint); the oracle follows the reference's
    bit operations (src/quant.rs:91-156). They must agree on every f32 whose bits are drawn here:
    all 65536 halves widened to f32 and nudged by one f32 ulp either way (the rounding ties and their
    neighbours), every exponent with random significands, and the NaN payloads."""
    from telmo_amd import Precision, encode

    h = np.arange(65536, dtype=np.uint32)
    widened = np.array([orc.f16_to_f32(int(x)) for x in h], np.float32).view(np.uint32)
    rng = np.random.default_rng(6)
    bits = np.concatenate([widened, widened + 1, widened - 1,
                           rng.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32),
                           (0x33000000 + np.arange(-4096, 4096)).astype(np.uint32),  # around 2^-25
                           (0x477FF000 + np.arange(-4096, 4096)).astype(np.uint32),  # around 65520
                           (0x7F800001 + rng.integers(0, 2**23 - 1, 2000)).astype(np.uint32)])
    vals = bits.view(np.float32)
    for p in (Precision.F16, Precision.BF16):
        v1, _ = encode(vals, 1, vals.size, p)
        v2, _ = orc.encode(vals, 1, vals.size, int(p))
        assert np.array_equal(v1, v2), p


def test_random_is_the_references_generator(orc):
    """tg_random reproduces telmo's test generator (src/kernels/mod.rs:795-805), checked against a
    plain-Python xorshift written from that source, and against the oracle's."""
    from telmo_amd import random

    def xorshift(length, seed):
        mask = (1 << 64) - 1
        s = (seed * 0x9E3779B97F4A7C15 & mask) | 1
        out = []
        for _ in range(length):
            s ^= (s << 13) & mask
            s ^= s >> 7
            s ^= (s << 17) & mask
            out.append(np.float32(np.float32(s >> 40) / np.float32(1 << 24)) * np.float32(2.0) - np.float32(1.0))
        return np.array(out, np.float32)

    for seed in (0, 1, 7, 2**63 + 5):
        want = xorshift(700, seed)
        assert np.array_equal(random(700, seed).view(np.uint32), want.view(np.uint32)), seed
        assert np.array_equal(orc.random(700, seed % 2**64).view(np.uint32), want.view(np.uint32)), seed
    # seed 0: the state starts at 1, and the first step is 1 ^ 1 << 13 = 0x2001, then ...
    first = random(1, 0)[0]
    s = 1
    s ^= s << 13
    s ^= s >> 7
    s ^= (s << 17) & ((1 << 64) - 1)
    assert first == np.float32((s >> 40) / 2**24 * 2 - 1)


def test_device_lengths_stay_inside_the_tensor_storage():
    """The wrappers pass a length beside every device pointer; it defaults to the element count only
    for a contiguous tensor and never runs past the tensor's storage (an expanded or overlapping view
    counts more elements than its storage holds)."""
    import torch

    from telmo_amd.kernels import _len

    t = torch.zeros(100)
    assert _len(t, None, "t") == 100
    assert _len(t[10:], None, "t") == 90
    assert _len(t[10:], 90, "t") == 90
    with pytest.raises(ValueError, match="runs past"):
        _len(t[10:], 91, "t")
    with pytest.raises(ValueError, match="not contiguous"):
        _len(torch.zeros(1).expand(50), None, "t")
    with pytest.raises(ValueError, match="runs past"):
        _len(torch.zeros(1).expand(50), 50, "t")
    strided = torch.zeros(8, 12)[:, 4:]
    with pytest.raises(ValueError, match="not contiguous"):
        _len(strided, None, "v")
    assert _len(strided, 7 * 12 + 8, "v") == 92
