"""Pins the oracle's restatement of src/quant.rs against the reference's own known answers
(src/quant.rs:305-455) and against numpy's IEEE conversions."""
import numpy as np
import pytest

F32, F16, BF16, INT8, Q8_0 = range(5)
ALL = [F32, F16, BF16, INT8, Q8_0]


def bits(x):
    return int(np.float32(x).view(np.uint32))


def test_every_half_round_trips_through_f32(orc):
    # src/quant.rs:309-319, plus numpy's exact half -> single conversion as a library check.
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    lib_vals = halves.view(np.float16).astype(np.float32)
    for h in range(65536):
        f = orc.f16_to_f32(h)
        if np.isnan(f):
            back = orc.f32_to_f16(f)
            assert back & 0x7C00 == 0x7C00 and back & 0x3FF != 0
            # A signalling NaN becomes quiet with the same payload.
            assert bits(f) & 0x400000
            assert (bits(f) >> 13) & 0x1FF == h & 0x1FF
            continue
        assert bits(f) == bits(lib_vals[h]), hex(h)
        assert orc.f32_to_f16(f) == h, hex(h)


def test_halves_round_to_nearest_even(orc):
    # src/quant.rs:321-335
    assert orc.f32_to_f16(1.0 + 2.0**-11) == 0x3C00
    assert orc.f32_to_f16(1.0 + 3.0 * 2.0**-11) == 0x3C02
    assert orc.f32_to_f16(65520.0) == 0x7C00
    assert orc.f32_to_f16(65519.0) == 0x7BFF
    assert orc.f32_to_f16(2.0**-24) == 1
    assert orc.f32_to_f16(2.0**-25) == 0
    assert orc.f32_to_f16(1.5 * 2.0**-25) == 1
    assert orc.f32_to_f16(-0.0) == 0x8000


def test_halves_match_an_ieee_conversion(orc):
    # src/quant.rs:337-361 compares with F16C; numpy's float16 cast is the same IEEE RNE rule.
    s = 0x9E3779B97F4A7C15
    mask = (1 << 64) - 1
    xs = []
    for _ in range(200_000):
        s ^= (s << 13) & mask
        s ^= s >> 7
        s ^= (s << 17) & mask
        xs.append(s & 0xFFFFFFFF)
    xs = np.array(xs, np.uint32).view(np.float32)
    xs = xs[~np.isnan(xs)]
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    for x, w in zip(xs[:50_000], want[:50_000]):
        assert orc.f32_to_f16(x) == w, repr(x)


def test_bf16_rounds_to_nearest_even(orc):
    # src/quant.rs:363-373
    assert orc.f32_to_bf16(1.0) == 0x3F80
    assert orc.f32_to_bf16(np.uint32(0x3F808000).view(np.float32)) == 0x3F80
    assert orc.f32_to_bf16(np.uint32(0x3F818000).view(np.float32)) == 0x3F82
    assert orc.f32_to_bf16(np.uint32(0x3F808001).view(np.float32)) == 0x3F81
    assert np.isnan(orc.bf16_to_f32(orc.f32_to_bf16(np.nan)))
    for h in [0, 0x8000, 0x3F80, 0x7F7F, 0xFF80]:
        assert orc.f32_to_bf16(orc.bf16_to_f32(h)) == h


def test_q8_0_blocks_follow_the_reference_quantizer(orc):
    # src/quant.rs:375-388
    x = (np.arange(32, dtype=np.float32) - np.float32(15.5)) * np.float32(0.37)
    d, q = orc.quantize_q8_0_block(x)
    assert q[0] == -127
    assert q.max() == 127
    assert np.all(np.abs(q.astype(np.float32) * d - x) <= 0.5 * d * 1.01)
    d0, q0 = orc.quantize_q8_0_block(np.zeros(32, np.float32))
    assert d0 == 0.0 and np.all(q0 == 0)
    # The stored scale is the f16 rounding of amax / 127.
    amax = np.float32(np.abs(x).max())
    assert d == np.float32(np.float16(amax / np.float32(127.0)))


def test_int8_rows_round_half_away_and_clamp(orc):
    # src/quant.rs:189-198: d = amax / 127 (unrounded), q = clamp(round(v / d)), round half away.
    x = np.array([1.27, -1.27, 0.005, -0.005, 0.015, 0.0], np.float32)
    d, q = orc.quantize_row_int8(x)
    assert d == np.float32(np.float32(1.27) / np.float32(127.0))
    id_ = np.float32(1.0) / d
    want = [int(np.sign(v) * np.floor(abs(np.float32(v) * id_) + 0.5)) for v in x]
    assert list(q) == want
    assert q.max() == 127 and q.min() == -127


def _round_trip_tolerance(p, v, amax):
    if p == F32:
        return 0.0
    if p == F16:
        return abs(v) * 2.0**-11
    if p == BF16:
        return abs(v) * 2.0**-8
    if p == INT8:
        return amax / 127.0 * 0.51
    return amax / 127.0 * 0.6


def test_every_precision_round_trips_within_its_resolution(orc):
    # src/quant.rs:390-417
    n, k = 37, 64
    i = np.arange(n * k)
    w = ((i * 7919 % 1000).astype(np.float32) / np.float32(500.0) - np.float32(1.0)) * (
        np.float32(1.0) + (i // k).astype(np.float32))
    w = w.astype(np.float32)
    for p in ALL:
        values, scales = orc.encode(w, n, k, p)
        assert len(values) == orc.panel_bytes(p, n, k)
        assert len(scales) == orc.scale_count(p, n, k)
        back = orc.decode(values, scales, n, k, p)
        for o in range(n):
            row = w[o * k:(o + 1) * k]
            amax = float(np.abs(row).max())
            for b, v in zip(back[o], row):
                assert abs(float(b) - float(v)) <= _round_trip_tolerance(p, float(v), amax), (p, o)


def test_q8_0_blocks_are_laid_out_unchanged(orc):
    # src/quant.rs:419-454
    n, k = 20, 64
    q = (np.arange(n * k) % 255).astype(np.uint8).view(np.int8)
    d = np.array([orc.f16_to_f32(orc.f32_to_f16(np.float32(0.01) * np.float32(i + 1)))
                  for i in range(n * k // 32)], np.float32)
    values, scales = orc.encode_q8(d, q, n, k, Q8_0)
    back = orc.decode(values, scales, n, k, Q8_0)
    want = q.reshape(n, k).astype(np.float32) * np.repeat(d.reshape(n, 2), 32, axis=1)
    assert np.array_equal(back.view(np.uint32), want.astype(np.float32).view(np.uint32))
    f32v, _ = orc.encode_q8(d, q, n, k, F32)
    assert np.array_equal(orc.decode(f32v, None, n, k, F32), back)


def test_the_panel_layout_matches_its_definition(orc):
    # src/quant.rs:1-13: panels of 16 outputs, k runs of 16 values, zero padding past n.
    n, k = 37, 24
    w = orc.random(n * k, 9).reshape(n, k)
    values, _ = orc.encode(w, n, k, F32)
    panels = -(-n // 16)
    pad = np.zeros((panels * 16, k), np.float32)
    pad[:n] = w
    want = pad.reshape(panels, 16, k).transpose(0, 2, 1).reshape(-1)
    assert np.array_equal(values.view(np.float32), want)
    values8, scales8 = orc.encode(w, n, k, INT8)
    q = values8.view(np.int8).reshape(panels, k, 16).transpose(0, 2, 1).reshape(panels * 16, k)
    assert np.all(q[n:] == 0) and np.all(scales8[n:] == 0)
    d = np.abs(w).max(axis=1) / np.float32(127.0)
    assert np.array_equal(scales8[:n], d.astype(np.float32))


def test_sizes_follow_the_precision(orc):
    # src/quant.rs:56-83
    assert [orc.value_bytes(p) for p in ALL] == [4, 2, 2, 1, 1]
    assert orc.panel_bytes(INT8, 4096, 1024) == 4_194_304
    assert orc.scale_count(INT8, 4096, 1024) == 4096
    assert orc.panel_bytes(INT8, 8198, 640) == 5_253_120
    assert orc.scale_count(INT8, 8198, 640) == 8208
    assert orc.scale_count(Q8_0, 20, 64) == 2 * 2 * 16
    assert orc.fits(Q8_0, 64) and not orc.fits(Q8_0, 65) and orc.fits(INT8, 65)
    with pytest.raises(ValueError):
        orc.encode(np.zeros(65 * 3, np.float32), 3, 65, Q8_0)
