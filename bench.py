"""Benchmark of the MI355X int8-weight matrix product on telmo's encoder shapes.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

A step is one pass of the hot path over one Conformer layer's projection set at T = 750 frames
(60 s of audio at 80 ms per frame), d = 1024, ff = 4096, all weights int8 with per-output
scales, activations f32 ~N(0, 1):

    FF1 up 1024->4096 (SiLU), FF1 down 4096->1024 (x0.5, accumulate), QKV 1024->3072,
    attention out 1024->1024 (input: the V third of QKV, accumulate), conv pw1 1024->2048,
    GLU -> 1024, pw2 1024->1024 (accumulate), FF2 up and down as FF1.

Each step first restores the layer input (a 3 MB device copy), so every step does the same work
on the same data. The step runs as one captured HIP graph; the eager (stream) figure is reported
beside it. value = 2 * sum(M N K) over the 8 GEMMs / step time, in TOPS.

The JSON line also carries:
  roofline      the GEMM kernels alone: each of the layer's 8 shapes on pre-quantised rows, timed
                with HIP events on the library's stream; achieved = algorithmic ops / kernel time,
                against the dense int8 MFMA peak. traffic comes from the rocprofv3 PMC summary in
                profiles/ when one is there.
  cpu_baseline  the C++ port of telmo's AVX-512 8x16 tile + thread pool (oracle/cpu_baseline.cpp,
                bit-identical to the fused oracle) on the host's cores, on the same bytes.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

T_FRAMES = 750
D, FF, CONV = 1024, 4096, 2048
DW_KERNEL = 9  # the conv module's depthwise kernel (parakeet's conv_kernel_size)
PEAK_INT8 = 5.0e15  # dense int8 MFMA ops/s (MI355X)
PEAK_HBM = 8.0e12   # bytes/s
METRIC = "int8 GEMM TOPS & %MFMA peak; decode GEMV GB/s & %HBM; encoder audio-s/s"

# (name, k, n, act, scale, accumulate, input)
LAYER = [
    ("ff1_up", D, FF, "silu", 1.0, False, "x"),
    ("ff1_down", FF, D, "none", 0.5, True, "h"),
    ("qkv", D, 3 * D, "none", 1.0, False, "x"),
    ("att_out", D, D, "none", 1.0, True, "v"),
    ("pw1", D, CONV, "none", 1.0, False, "x"),
    ("pw2", D, D, "none", 1.0, True, "u"),
    ("ff2_up", D, FF, "silu", 1.0, False, "x"),
    ("ff2_down", FF, D, "none", 0.5, True, "h"),
]


# ---------------------------------------------------------------- synthetic inputs
# Every input is drawn from telmo's test generator (src/kernels/mod.rs:795-805, exported as
# telmo_amd.random): u in [-1, 1) and u01 = (u + 1) / 2. N(0, 1) activations by Box-Muller over
# pairs of u01 (cos and sin of one pair give two values), int8 weights floor(u01 * 255) - 127 in
# [-127, 127], scales 0.001 + 0.009 u01. Each tensor has a seed of its own.


def synth_u01(length, seed):
    import telmo_amd

    return (telmo_amd.random(length, seed).astype(np.float64) + 1.0) * 0.5


def synth_normal(shape, seed):
    count = int(np.prod(shape))
    u = synth_u01(2 * ((count + 1) // 2), seed).reshape(-1, 2)
    r = np.sqrt(-2.0 * np.log1p(-u[:, 0]))
    z = np.stack([r * np.cos(2.0 * np.pi * u[:, 1]), r * np.sin(2.0 * np.pi * u[:, 1])], axis=1).reshape(-1)
    return z[:count].astype(np.float32).reshape(shape)


def synth_int8(n, k, seed):
    return (np.floor(synth_u01(n * k, seed) * 255.0) - 127.0).astype(np.int8).reshape(n, k)


def synth_scales(n, seed):
    return (0.001 + 0.009 * synth_u01(n, seed)).astype(np.float32)


def panel_layout(q, s):
    """int8 rows q [n, k] and scales s [n] in the panel layout (src/quant.rs:200-269)."""
    n, k = q.shape
    panels = -(-n // 16)
    pad = np.zeros((panels * 16, k), np.int8)
    pad[:n] = q
    values = pad.reshape(panels, 16, k).transpose(0, 2, 1).reshape(-1).view(np.uint8).copy()
    scales = np.zeros(panels * 16, np.float32)
    scales[:n] = s
    return values, scales


def ops_of(m):
    return sum(2 * m * k * n for _, k, n, *_ in LAYER)


def bytes_of(m):
    """Algorithmic HBM bytes of the 8 GEMMs: A f32, int8 weights, f32 scales, C f32 (+ C read when
    accumulating), each tensor once (panels padded to 16 outputs)."""
    total = 0
    for _, k, n, _, _, acc, _ in LAYER:
        npad = -(-n // 16) * 16
        total += 4 * m * k + npad * k + 4 * npad + 4 * m * n * (2 if acc else 1)
    return total


def run_layer(kern, W, bufs, T, dw=None):
    """The layer's products in order: FFN (SiLU, half-step residual), QKV, attention output (the V
    third of QKV standing in for attention), the conv module's pointwise pair around the GLU (pw1
    and the GLU as one fused GEMM; given dw = (weights [DW_KERNEL, D], bias [D], utterances), the
    depthwise convolution + SiLU between GLU and pw2, each of the utterances' T / dw[2] frames on
    its own), and the second FFN. bufs holds x [T, D], h [T, FF], qkv [T, 3D], u and d [T, D]."""
    from telmo_amd import Act, Epilogue

    x, h, qkv, u = (bufs[key] for key in ("x", "h", "qkv", "u"))
    silu = Epilogue(act=Act.SILU)
    half_acc = Epilogue(scale=0.5, accumulate=True)
    acc = Epilogue(accumulate=True)
    kern.linear_device(x, T, W["ff1_up"], h, silu)
    kern.linear_device(h, T, W["ff1_down"], x, half_acc)
    kern.linear_device(x, T, W["qkv"], qkv)
    kern.matmul_device(qkv[:, 2 * D:], 3 * D, T, W["att_out"], x, D, acc, a_len=qkv.numel() - 2 * D)
    kern.linear_glu_device(x, T, W["pw1"], u)  # pw1 with the GLU in its epilogue
    if dw is not None:
        seqs = dw[2]  # equal-length utterances stacked along the rows, each convolved on its own
        kern.dwconv1d_device(u, D, T // seqs, D, dw[0], DW_KERNEL, dw[1], bufs["d"], D, act=Act.SILU, batch=seqs)
        u = bufs["d"]
    kern.linear_device(u, T, W["pw2"], x, acc)
    kern.linear_device(x, T, W["ff2_up"], h, silu)
    kern.linear_device(h, T, W["ff2_down"], x, half_acc)


def layer_buffers(T, dev="cuda"):
    import torch

    return {"x": torch.empty((T, D), dtype=torch.float32, device=dev),
            "h": torch.empty((T, FF), dtype=torch.float32, device=dev),
            "qkv": torch.empty((T, 3 * D), dtype=torch.float32, device=dev),
            "u": torch.empty((T, D), dtype=torch.float32, device=dev),
            "d": torch.empty((T, D), dtype=torch.float32, device=dev)}


def make_weights(rng):
    out = []
    for name, k, n, *_ in LAYER:
        q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
        s = (0.001 + 0.009 * rng.random(n)).astype(np.float32)
        panels = -(-n // 16)
        pad = np.zeros((panels * 16, k), np.int8)
        pad[:n] = q
        values = pad.reshape(panels, 16, k).transpose(0, 2, 1).reshape(-1).view(np.uint8).copy()
        scales = np.zeros(panels * 16, np.float32)
        scales[:n] = s
        out.append((name, k, n, values, scales))
    return out


def gpu_leg(args, weights, x0_host):
    import torch

    import telmo_amd
    from telmo_amd import Act, Epilogue

    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    W = {name: telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, v, s)
         for name, k, n, v, s in weights}
    T = T_FRAMES
    dev = "cuda"
    x0 = torch.from_numpy(x0_host).to(dev)
    bufs = layer_buffers(T, dev)
    x, h, qkv, u = bufs["x"], bufs["h"], bufs["qkv"], bufs["u"]
    v = qkv[:, 2 * D:]

    def step():
        x.copy_(x0)
        run_layer(kern, W, bufs, T)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    if not torch.isfinite(x).all():
        raise RuntimeError("the layer output is not finite")

    def timed(fn, reps):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps  # ms

    eager_ms = timed(step, args.steps)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    for _ in range(args.warmup):
        graph.replay()
    graph_ms = timed(graph.replay, args.steps)
    # The graph's output equals the eager step's.
    graph.replay()
    torch.cuda.synchronize()
    out_graph = x.clone()
    step()
    torch.cuda.synchronize()
    if not torch.equal(out_graph, x):
        raise RuntimeError("graph replay differs from the eager step")

    # Roofline leg: the GEMM kernel alone, per shape, on pre-quantised rows.
    per_shape = []
    inputs = {"x": x, "h": h, "v": v, "u": u}
    for name, k, n, act, scale, accumulate, src in LAYER:
        a = inputs[src]
        lda = 3 * D if src == "v" else k
        qa = torch.empty(kern.quant_bytes(T, k), dtype=torch.uint8, device=dev)
        ex = torch.empty(T, dtype=torch.int32, device=dev)
        kern.quantize_rows_device(a, lda, T, k, qa, ex, a_len=(T - 1) * lda + k)
        c = torch.zeros((T, n), dtype=torch.float32, device=dev)
        epi = Epilogue(act=Act.SILU if act == "silu" else Act.NONE, scale=scale, accumulate=accumulate)
        launch = lambda: kern.matmul_quantized_device(qa, ex, T, W[name], c, n, epi)  # noqa: E731
        for _ in range(5):
            launch()
        ms = timed(launch, args.kernel_reps)
        per_shape.append({"gemm": name, "m": T, "k": k, "n": n, "us": round(ms * 1e3, 3),
                          "tops": round(2 * T * k * n / (ms * 1e-3) / 1e12, 1)})
    for w in W.values():
        w.close()
    kern.close()
    return eager_ms, graph_ms, per_shape


ENC_LAYERS = 24
# (workload, rows, audio seconds, utterances): 32 utterances of 30 s at 80 ms per frame; one 600 s
# utterance.
ENC_CASES = [("batch of 32 x 30 s utterances", 32 * 375, 960.0, 32), ("one 600 s utterance", 7500, 600.0, 1)]


def encoder_leg(args):
    """The encoder stack: 24 Conformer layers of the layer step's shapes, each with its own random
    int8 weights and scales (580 MB in all, generated on the GPU), the conv module's depthwise
    convolution (kernel 9, per utterance) + SiLU between GLU and pw2, and LayerNorm (gamma 1,
    beta 0) after every layer to keep the activations N(0, 1). Audio-seconds per second = the audio
    the rows stand for / the time of one pass over all 24 layers. The depthwise convolution is
    also timed alone (HIP events, 20 launches) against HBM: its algorithmic bytes are the input and
    output rows plus its weights."""
    import torch

    import telmo_amd

    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    layers, wbytes = [], 0
    for _ in range(ENC_LAYERS):
        W = {}
        for name, k, n, *_ in LAYER:
            q = torch.randint(-127, 128, (n * k,), generator=gen, device="cuda", dtype=torch.int16)
            q = q.to(torch.int8).view(torch.uint8)
            sc = 0.001 + 0.009 * torch.rand(n, generator=gen, device="cuda")
            W[name] = telmo_amd.PackedWeights.from_device(kern, n, k, telmo_amd.Precision.INT8, q, sc)
            wbytes += W[name].bytes()
            del q, sc
        dw = (0.3 * torch.randn((DW_KERNEL, D), generator=gen, device="cuda"),
              0.1 * torch.randn(D, generator=gen, device="cuda"))
        layers.append((W, dw))
    gamma = torch.ones(D, device="cuda")
    beta = torch.zeros(D, device="cuda")
    out = []
    for label, M, audio_s, seqs in ENC_CASES:
        x0 = torch.randn((M, D), generator=gen, device="cuda")
        bufs = layer_buffers(M)
        x = bufs["x"]

        def run():
            x.copy_(x0)
            for W, dw in layers:
                run_layer(kern, W, bufs, M, dw + (seqs,))
                kern.layer_norm_device(x, D, M, D, gamma, beta, 1e-5, x, D)

        run()
        torch.cuda.synchronize()
        if not torch.isfinite(x).all():
            raise RuntimeError("the encoder output is not finite")
        reps = 3
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            run()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        dw_w, dw_b = layers[0][1]
        e0.record(stream)
        for _ in range(20):
            kern.dwconv1d_device(bufs["u"], D, M // seqs, D, dw_w, DW_KERNEL, dw_b, bufs["d"], D,
                                 act=telmo_amd.Act.SILU, batch=seqs)
        e1.record(stream)
        torch.cuda.synchronize()
        dw_s = e0.elapsed_time(e1) / 20 * 1e-3
        dw_bytes = 4 * (2 * M * D + DW_KERNEL * D + D)
        ops = ENC_LAYERS * ops_of(M)
        out.append({"workload": f"{ENC_LAYERS}-layer encoder, {label}", "m": M, "audio_s": audio_s,
                    "ms_per_pass": round(ms, 3), "audio_s_per_s": round(audio_s / (ms * 1e-3), 1),
                    "tops": round(ops / (ms * 1e-3) / 1e12, 1), "weights_mb": round(wbytes / 1e6, 1),
                    "dwconv_us": round(dw_s * 1e6, 2),
                    "dwconv_hbm_frac": round(dw_bytes / dw_s / PEAK_HBM, 3)})
        del bufs, x0
    for W, _ in layers:
        for w in W.values():
            w.close()
    kern.close()
    return out


def q8_leg(args):
    """The same Conformer layer step (T=750) and the decode GEMVs (m = 1, weights rotated past the
    Infinity Cache) with Q8_0 weights: one f16-exact scale per 32 inputs of each output."""
    import torch

    import telmo_amd

    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(13)

    def q8_weights(n, k):
        q = torch.randint(-127, 128, (-(-n // 16) * 16 * k,), generator=gen, device="cuda", dtype=torch.int16)
        q = q.to(torch.int8).view(torch.uint8)
        d = (0.001 + 0.009 * torch.rand(-(-n // 16) * 16 * (k // 32), generator=gen, device="cuda")).half().float()
        return telmo_amd.PackedWeights.from_device(kern, n, k, telmo_amd.Precision.Q8_0, q, d)

    def timed(fn, reps):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(reps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3

    W = {name: q8_weights(n, k) for name, k, n, *_ in LAYER}
    T = T_FRAMES
    x0 = torch.randn((T, D), generator=gen, device="cuda")
    bufs = layer_buffers(T)

    def step(_):
        bufs["x"].copy_(x0)
        run_layer(kern, W, bufs, T)

    for i in range(10):
        step(i)
    t = timed(step, 50)
    out = {"layer_step": {"workload": "conformer layer projection set at T=750 (8 GEMMs + GLU), Q8_0 weights",
                          "ms_per_step": round(t * 1e3, 4), "tops": round(ops_of(T) / t / 1e12, 1)},
           "rotating": []}
    for w in W.values():
        w.close()
    for name, k, n in (("joint", 640, 8198), ("gates", 640, 2560)):
        one = q8_weights(n, k)
        copies = [one] + [q8_weights(n, k) for _ in range(int(600e6 // one.bytes()))]
        a = torch.randn(1, k, device="cuda")
        c = torch.empty(1, n, device="cuda")
        call = lambda i: kern.linear_device(a, 1, copies[i % len(copies)], c)  # noqa: E731
        for i in range(len(copies)):
            call(i)
        t = timed(call, 4 * len(copies))
        out["rotating"].append({"gemv": name, "m": 1, "k": k, "n": n, "weight_mb": round(one.bytes() / 1e6, 3),
                                "us": round(t * 1e6, 2), "gb_s": round(one.bytes() / t / 1e9, 1),
                                "hbm_frac": round(one.bytes() / t / PEAK_HBM, 3)})
        for w in copies:
            w.close()
    kern.close()
    return out


def _pack(rng, n, k):
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    s = (0.001 + 0.009 * rng.random(n)).astype(np.float32)
    panels = -(-n // 16)
    pad = np.zeros((panels * 16, k), np.int8)
    pad[:n] = q
    values = pad.reshape(panels, 16, k).transpose(0, 2, 1).reshape(-1).view(np.uint8).copy()
    scales = np.zeros(panels * 16, np.float32)
    scales[:n] = s
    return values, scales


def gemv_leg(args):
    """The TDT decode-step GEMVs (m = 1, 4, 8 streams) on the HBM roofline.

    (i) each shape with its weights evicted: calls rotate over copies totalling more than 512 MB
        (twice the 256 MB Infinity Cache), so every call streams its weights from HBM;
    (ii) the same kernel on one large matrix (64 - 256 MB) for its asymptotic HBM rate;
    (iii) the token loop: 2000 dependent steps of gates 640 -> 2560 then joint 640 -> 8198 (+ bias),
        each step's input taken from the previous step's gate output, weights reused (cache-resident).
    GB/s counts the weight bytes of the panel layout plus scales once per call.
    """
    import torch

    import telmo_amd
    from telmo_amd import Epilogue

    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    rng = np.random.default_rng(5)
    out = {"rotating": [], "sweep": [], "token_loop": []}

    def timed(fn, reps):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(reps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3  # s

    shapes = [("joint", 640, 8198, True), ("gates", 640, 2560, False), ("lstm_layer", 1280, 2560, False)]
    for name, k, n, with_bias in shapes:
        values, scales = _pack(rng, n, k)
        one = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
        wbytes = one.bytes()
        copies = [one] + [telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
                          for _ in range(int(600e6 // wbytes))]
        bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda() if with_bias else None
        for m in (1, 4, 8):
            a = torch.randn(m, k, device="cuda")
            c = torch.empty(m, n, device="cuda")
            epi = Epilogue(bias=bias)
            call = lambda i: kern.linear_device(a, m, copies[i % len(copies)], c, epi)  # noqa: E731
            for i in range(len(copies)):
                call(i)
            t = timed(call, 4 * len(copies))
            out["rotating"].append({"gemv": name, "m": m, "k": k, "n": n, "weight_mb": round(wbytes / 1e6, 3),
                                    "us": round(t * 1e6, 2), "gb_s": round(wbytes / t / 1e9, 1),
                                    "hbm_frac": round(wbytes / t / PEAK_HBM, 3)})
        for w in copies:
            w.close()
    for mb in (64, 256):
        k = 640
        n = int(mb * 1e6 // k) // 16 * 16
        values, scales = _pack(rng, n, k)
        w = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
        del values
        for m in (1, 4, 8):
            a = torch.randn(m, k, device="cuda")
            c = torch.empty(m, n, device="cuda")
            call = lambda i: kern.linear_device(a, m, w, c)  # noqa: E731
            call(0)
            t = timed(call, 20)
            out["sweep"].append({"m": m, "k": k, "n": n, "weight_mb": round(w.bytes() / 1e6, 1), "us": round(t * 1e6, 1),
                                 "gb_s": round(w.bytes() / t / 1e9, 1), "hbm_frac": round(w.bytes() / t / PEAK_HBM, 3)})
        w.close()
    # Token loop.
    vg, sg = _pack(rng, 2560, 640)
    vj, sj = _pack(rng, 8198, 640)
    wg = telmo_amd.PackedWeights.from_parts(kern, 2560, 640, telmo_amd.Precision.INT8, vg, sg)
    wj = telmo_amd.PackedWeights.from_parts(kern, 8198, 640, telmo_amd.Precision.INT8, vj, sj)
    bg = torch.from_numpy(rng.standard_normal(2560).astype(np.float32)).cuda()
    bj = torch.from_numpy(rng.standard_normal(8198).astype(np.float32)).cuda()
    steps = 2000
    for m in (1, 4, 8):
        gates = torch.randn(m, 2560, device="cuda")
        logits = torch.empty(m, 8198, device="cuda")
        g_epi = Epilogue(bias=bg, scale=1.0 / 16)
        j_epi = Epilogue(bias=bj)
        h = gates[:, 640:1280]
        z = gates[:, :640]
        alen = (m - 1) * 2560 + 640

        def step():
            kern.matmul_device(h, 2560, m, wg, gates, 2560, g_epi, a_len=alen)
            kern.matmul_device(z, 2560, m, wj, logits, 8198, j_epi, a_len=alen)

        for _ in range(10):
            step()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(100):
                step()
        graph.replay()
        t = timed(lambda i: graph.replay(), steps // 100) / 100  # s per step
        if not torch.isfinite(logits).all():
            raise RuntimeError("the token loop diverged")
        step_bytes = wg.bytes() + wj.bytes()
        out["token_loop"].append({"m": m, "steps": steps, "us_per_step": round(t * 1e6, 2),
                                  "tokens_per_s": round(m / t, 1), "effective_gb_s": round(step_bytes / t / 1e9, 1),
                                  "note": "weights reused every step (cache-resident), effective rate"})
    wg.close()
    wj.close()
    kern.close()
    return out


def host_leg(weights, x0):
    """The single GEMM 750 x 1024 -> 4096 through the host-pointer entry point (tg_linear): the
    PCIe-inclusive rate a caller handing host slices sees (a copied in, c copied back)."""
    import telmo_amd

    kern = telmo_amd.Kernels(0)
    name, k, n, values, scales = weights[0]
    w = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
    a = np.ascontiguousarray(x0[:, :k])
    c = np.zeros(T_FRAMES * n, np.float32)
    kern.linear(a.reshape(-1), T_FRAMES, w, c)
    reps = 20
    t0 = time.perf_counter()
    for _ in range(reps):
        kern.linear(a.reshape(-1), T_FRAMES, w, c)
    dt = (time.perf_counter() - t0) / reps
    w.close()
    kern.close()
    ops = 2.0 * T_FRAMES * k * n
    moved = 4 * T_FRAMES * (k + n)
    return {"workload": f"one GEMM {T_FRAMES} x {k} -> {n} ({name}) via tg_linear on host buffers",
            "us": round(dt * 1e6, 1), "tops": round(ops / dt / 1e12, 2), "host_bytes_moved": moved,
            "note": "includes the copy of a to the device and of c back; not the headline value"}


def cpu_leg(weights, x0_host, budget_s):
    """telmo's SIMD + pool path (C++ port) on every host core, same bytes, 8 GEMMs per layer."""
    from oracle import oracle as orc

    L = ctypes.CDLL(orc.CPUBASE)
    L.cb_isa.restype = ctypes.c_int
    L.cb_pool_new.restype = ctypes.c_void_p
    L.cb_pool_new.argtypes = [ctypes.c_size_t]
    L.cb_pool_free.argtypes = [ctypes.c_void_p]
    L.cb_matmul.argtypes = ([ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                             ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t,
                             ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_void_p,
                             ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_int])
    isa = L.cb_isa()
    if isa == 0:
        return None
    cores = len(os.sched_getaffinity(0))
    pool = L.cb_pool_new(cores)
    T = T_FRAMES
    x = x0_host.copy()
    h = np.zeros((T, FF), np.float32)
    qkv = np.zeros((T, 3 * D), np.float32)
    u = np.random.default_rng(1).standard_normal((T, D)).astype(np.float32)
    bufs = {"x": x, "h": h, "u": u}
    p = lambda arr: arr.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    W = {name: (k, n, v, s) for name, k, n, v, s in weights}

    def gemm(name, act, scale, accumulate, src, out, ldc):
        k, n, v, s = W[name]
        if src == "v":  # the V third of QKV: rows 3D apart, starting at column 2D
            a_ptr, lda = ctypes.c_void_p(qkv.ctypes.data + 4 * 2 * D), 3 * D
        else:
            a_ptr, lda = p(bufs[src]), k
        rc = L.cb_matmul(pool, isa, a_ptr, (T - 1) * lda + k, lda, T, p(v), p(s), 3, n, k, p(out), out.size, ldc,
                         None, 0, 2 if act == "silu" else 0, scale, int(accumulate))
        assert rc == 0, rc

    outs = {"ff1_up": h, "ff1_down": x, "qkv": qkv, "att_out": x, "pw1": np.zeros((T, CONV), np.float32),
            "pw2": x, "ff2_up": h, "ff2_down": x}

    def layer():
        for name, k, n, act, scale, accumulate, src in LAYER:
            gemm(name, act, scale, accumulate, src, outs[name], n)

    # Bit-identity with the fused oracle before timing (FF1 up on the layer input).
    k, n, v, s = W["ff1_up"]
    got, want = np.zeros((T, n), np.float32), np.zeros((T, n), np.float32)
    assert L.cb_matmul(pool, isa, p(x0_host), x0_host.size, k, T, p(v), p(s), 3, n, k, p(got), got.size, n, None, 0,
                       2, 1.0, 0) == 0
    orc.matmul(True, x0_host.reshape(-1), k, T, v, s, 3, n, k, want.reshape(-1), n, None, 2, 1.0, False)
    if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
        raise RuntimeError("the CPU baseline differs from the fused oracle")

    t0 = time.perf_counter()
    x[:] = x0_host
    layer()
    one = time.perf_counter() - t0
    reps = max(1, int(budget_s / 5 / one))
    best = float("inf")
    for _ in range(5):
        t0 = time.perf_counter()
        for _ in range(reps):
            x[:] = x0_host
            layer()
        best = min(best, (time.perf_counter() - t0) / reps)
    L.cb_pool_free(pool)
    return {"value": round(ops_of(T) / best / 1e12, 4), "unit": "TOPS", "cores": cores,
            "kind": "port", "isa": "avx512" if isa == 2 else "avx2",
            "sample": f"the same 8-GEMM layer at T={T}, best of 5 rounds of {reps} layers "
                      f"({reps * 5 * best:.1f} s in all), {cores} threads",
            "ms_per_step": round(best * 1e3, 3),
            "encoder_audio_s_per_s": round(T * 0.08 / (ENC_LAYERS * best), 1),
            "encoder_note": f"{ENC_LAYERS} layers of this step per {T} frames (80 ms each): the CPU path's "
                            "encoder audio-seconds per second, GEMMs only, scaled from the sample"}



# The TDT decoder of Parakeet: h = 640, vocab 8193 (blank last) + 5 durations, 2 LSTM layers.
TDT_H, TDT_VOCAB, TDT_DURS, TDT_MAX_SYMBOLS = 640, 8193, [0, 1, 2, 3, 4], 10
TDT_BLANK_BIAS = 28.0  # on random weights: blank runs between tokens


def _panels(q, s):
    n, k = q.shape
    panels = -(-n // 16)
    pad = np.zeros((panels * 16, k), np.int8)
    pad[:n] = q
    values = pad.reshape(panels, 16, k).transpose(0, 2, 1).reshape(-1).view(np.uint8).copy()
    scales = np.zeros(panels * 16, np.float32)
    scales[:n] = s
    return values, scales


def tdt_network(seed=21):
    """Random int8 network of Parakeet's decoder shapes in the panel layout (numpy)."""
    rng = np.random.default_rng(seed)
    h, vocab = TDT_H, TDT_VOCAB

    def mat(n, k, lo, hi):
        q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
        return _panels(q, (lo + (hi - lo) * rng.random(n)).astype(np.float32))

    outputs = vocab + len(TDT_DURS)
    joint_b = (0.5 * rng.standard_normal(outputs)).astype(np.float32)
    joint_b[vocab - 1] += TDT_BLANK_BIAS
    return {"p": 3, "h": h, "vocab": vocab, "durations": TDT_DURS, "max_symbols": TDT_MAX_SYMBOLS,
            "joint": mat(outputs, h, 0.001, 0.01), "joint_b": joint_b,
            "emb": (0.5 * rng.standard_normal((vocab, h))).astype(np.float32),
            "lstm": [mat(4 * h, 2 * h, 0.0004, 0.0008) for _ in range(2)],
            "lstm_b": [(0.1 * rng.standard_normal(4 * h)).astype(np.float32) for _ in range(2)],
            "proj": mat(h, h, 0.001, 0.003), "proj_b": (0.1 * rng.standard_normal(h)).astype(np.float32)}


def tdt_leg(args, net, enc_host):
    """The greedy TDT decode of 60 s of audio (750 encoder frames) on the device, from the start
    state (the blank through the prediction network), through tg_tdt_decode_device: one call, every
    step on the GPU, the host waking once per batch of steps. Reported per decode (median of 5)."""
    import torch

    import telmo_amd

    kern = telmo_amd.Kernels(0)
    h, vocab = net["h"], net["vocab"]
    P = telmo_amd.Precision.INT8
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    joint = telmo_amd.PackedWeights.from_parts(kern, vocab + len(TDT_DURS), h, P, *net["joint"])
    lstm = [telmo_amd.PackedWeights.from_parts(kern, 4 * h, 2 * h, P, *w) for w in net["lstm"]]
    proj = telmo_amd.PackedWeights.from_parts(kern, h, h, P, *net["proj"])
    dec = telmo_amd.TdtDecoder(kern, h, vocab, TDT_DURS, TDT_MAX_SYMBOLS, joint, dev(net["joint_b"]),
                               dev(net["emb"]), lstm, [dev(b) for b in net["lstm_b"]], proj, dev(net["proj_b"]))
    enc = dev(enc_host)
    state0 = torch.zeros(2 * 2 * h, device="cuda")
    pred0 = torch.zeros(h, device="cuda")
    dec.predict_rows([vocab - 1], state0.view(1, -1), pred0.view(1, -1))
    kern.synchronize()
    times, toks = [], None
    for _ in range(6):
        state, pred = state0.clone(), pred0.clone()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks, frame, _ = dec.decode(enc, state, pred)
        times.append(time.perf_counter() - t0)
    ms = float(np.median(times[1:])) * 1e3
    frames = enc_host.shape[0]
    weight_bytes = joint.bytes() + sum(w.bytes() for w in lstm) + proj.bytes()
    out = {"workload": f"greedy TDT decode, {frames} frames (60 s audio), h={h}, vocab {vocab} + "
                       f"{len(TDT_DURS)} durations, 2 LSTM layers, int8",
           "frames": frames, "tokens": len(toks), "tokens_per_frame": round(len(toks) / frames, 3),
           "ms_per_decode": round(ms, 3), "us_per_token": round(ms * 1e3 / max(len(toks), 1), 2),
           "audio_s_per_s": round(60.0 / (ms * 1e-3), 1), "decoder_weight_mb": round(weight_bytes / 1e6, 2),
           "timing": "wall clock around tg_tdt_decode_device (blocks until the decode ends), median of 5"}
    dec.close()
    kern.close()
    return out, toks


def cpu_tdt(net, enc_host, frames):
    """telmo's decode_inner on the CPU: the C++ port (every product by the SIMD port on a pool of
    all host cores, libm gate math) over the whole decode, best of 3; and, as the parity check, the
    oracle's decode (scalar C, the fast path's integer products) over the first `frames` frames."""
    from oracle import oracle as orc

    L = orc.cpubase()
    if L.cb_isa() == 0:
        return None, None, None
    cores = len(os.sched_getaffinity(0))
    pool = L.cb_pool_new(cores)
    start = np.zeros(2 * 2 * TDT_H, np.float32), np.zeros(TDT_H, np.float32)
    orc.tdt_predict(net, [TDT_VOCAB - 1], start[0].reshape(1, -1), start[1].reshape(1, -1))
    best, toks = float("inf"), None
    for _ in range(3):
        state, pred = start[0].copy(), start[1].copy()
        t0 = time.perf_counter()
        toks, _, _ = orc.cpu_tdt_decode(net, enc_host, state, pred, pool)
        best = min(best, time.perf_counter() - t0)
    L.cb_pool_free(pool)
    state, pred = start[0].copy(), start[1].copy()
    t0 = time.perf_counter()
    oracle_toks, _, _ = orc.tdt_decode(net, enc_host[:frames], state, pred)
    dt = time.perf_counter() - t0
    out = {"value": round(best * 1e3, 3), "unit": "ms per decode", "cores": cores, "kind": "port",
           "ms_per_token": round(best * 1e3 / max(len(toks), 1), 4), "tokens": len(toks),
           "sample": f"the whole decode ({enc_host.shape[0]} frames) by the C++ port of decode_inner and "
                     f"predict_rows, products on the SIMD pool port, best of 3",
           "oracle_scalar": {"ms_per_token": round(dt * 1e3 / max(len(oracle_toks), 1), 3), "cores": 1,
                             "sample": f"the oracle's decode over the first {frames} frames: "
                                       f"{len(oracle_toks)} tokens in {dt:.2f} s"}}
    return out, toks, oracle_toks


def shape_leg(m, k, n, reps):
    """One product shape alone, the program rocprofv3 runs for per-shape kernel statistics and
    counters: rows quantised once, then `reps` launches of the MFMA GEMM alone
    (tg_matmul_quantized_device) on the context's stream between HIP events on that stream. int8
    weights and scales and N(0, 1) rows from telmo's test generator (seeds 1, 2 and 3)."""
    import torch

    import telmo_amd

    values, scales = panel_layout(synth_int8(n, k, 1), synth_scales(n, 2))
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    w = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
    a = torch.from_numpy(synth_normal((m, k), 3)).cuda()
    qa = torch.empty(kern.quant_bytes(m, k), dtype=torch.uint8, device="cuda")
    exps = torch.empty(m, dtype=torch.int32, device="cuda")
    c = torch.empty((m, n), device="cuda")
    kern.quantize_rows_device(a, k, m, k, qa, exps)
    for _ in range(3):
        kern.matmul_quantized_device(qa, exps, m, w, c, n)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        kern.matmul_quantized_device(qa, exps, m, w, c, n)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / reps * 1e3
    w.close()
    kern.close()
    return {"shape": [m, k, n], "reps": reps, "us_per_launch": round(us, 3),
            "tops": round(2 * m * n * k / us / 1e6, 1)}


def load_traffic():
    path = os.path.join(ROOT, "profiles", "gemm_layer_T750_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes_per_launch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--kernel-reps", type=int, default=500)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemv", action="store_true")
    ap.add_argument("--no-encoder", action="store_true")
    ap.add_argument("--no-q8", action="store_true")
    ap.add_argument("--no-tdt", action="store_true")
    ap.add_argument("--shape", type=int, nargs=3, metavar=("M", "K", "N"),
                    help="time one product shape alone (the program for per-shape rocprofv3 runs) and exit")
    ap.add_argument("--reps", type=int, default=20, help="launches timed with --shape")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        sys.exit("bench.py measures one GPU and has no multi-GPU path: run it with --gpus 1")
    if args.shape:
        print(json.dumps(shape_leg(*args.shape, args.reps)), flush=True)
        return

    rng = np.random.default_rng(0)
    weights = make_weights(rng)
    x0 = rng.standard_normal((T_FRAMES, D)).astype(np.float32)

    eager_ms, graph_ms, per_shape = gpu_leg(args, weights, x0)
    ops = ops_of(T_FRAMES)
    gemm_us = sum(s["us"] for s in per_shape)
    achieved = ops / (gemm_us * 1e-6)
    traffic = load_traffic()
    roofline = {"bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": PEAK_INT8 / 1e12,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_INT8, 4), "traffic": traffic,
                "kernel": "gemm_lds_kernel<4,4,3> (n >= 2048), gemm_i8_kq_kernel<5> (k = 4096, n = 1024) and "
                          "gemm_i8_kernel<2,2,6> (k = 1024, n = 1024)", "avg_launch_us": round(gemm_us / len(per_shape), 3),
                "ops_per_launch_avg": ops / len(per_shape),
                "mfma_int8_ops_per_launch_avg": 2 * ops / len(per_shape),
                "mfma_busy_frac": round(2 * achieved / PEAK_INT8, 4),
                "note": "two int8 digits per activation: the MFMA executes 2x the algorithmic ops",
                "per_shape": per_shape}
    gemv = None if args.no_gemv else gemv_leg(args)
    host = host_leg(weights, x0)
    encoder = None if args.no_encoder else encoder_leg(args)
    q8 = None if args.no_q8 else q8_leg(args)
    tdt = None
    if not args.no_tdt:
        net = tdt_network()
        enc = np.random.default_rng(22).standard_normal((T_FRAMES, TDT_H)).astype(np.float32)
        tdt, gpu_toks = tdt_leg(args, net, enc)
    cpu = None if args.no_cpu else cpu_leg(weights, x0, args.cpu_seconds)
    if cpu is not None and tdt is not None:
        cpu["tdt_decode"], port_toks, oracle_toks = cpu_tdt(net, enc, 150)
        if port_toks is not None:
            gpu = [tuple(t) for t in gpu_toks]
            # the port's tokens (fused f32 sums, as telmo's decode) are the GPU decode's, and the
            # oracle's over the first frames are its first tokens
            tdt["cpu_port_tokens_match"] = gpu == port_toks
            tdt["oracle_sample_tokens_match"] = gpu[:len(oracle_toks)] == oracle_toks
    # The step runs either as a captured HIP graph or launched eagerly on one stream; both run the
    # same kernels on the same resident inputs, and the faster of the two is the step time.
    step_ms = min(graph_ms, eager_ms)
    value = ops / (step_ms * 1e-3) / 1e12
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "conformer layer projection set: 8 int8 GEMMs + GLU at T=750 frames "
                               "(60 s audio), d=1024, ff=4096, conv 2048",
                   "frames": T_FRAMES, "ops_per_step": ops, "hbm_bytes_per_step": bytes_of(T_FRAMES),
                   "ms_per_step_eager": round(eager_ms, 5), "ms_per_step_graph": round(graph_ms, 5),
                   "timing": "HIP events around the timed steps; the faster of eager launches and HIP graph replay",
                   "audio_s_per_s_one_layer": round(60.0 / (step_ms * 1e-3), 1)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "gemv": gemv,
        "pcie_inclusive": host,
        "encoder": encoder,
        "q8_0": q8,
        "tdt": tdt,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
