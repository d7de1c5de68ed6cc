"""Benchmark of the MI355X int8-weight matrix product on telmo's encoder and decoder shapes.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-gemv] [--no-encoder] ...
    python bench.py --shape M K N [--reps R]      (one product shape alone, for rocprofv3)

A step is one Conformer layer of Parakeet's encoder (src/parakeet.rs:1011-1172) on the device at
T = 750 frames (60 s of audio at 80 ms per frame), d = 1024, ff = 4096, conv 2048 -> GLU -> 1024, all
eight products int8 with per-output scales (the layer's projection set):

    FF1 in 1024->4096 (SiLU), FF1 out 4096->1024 (x0.5, accumulate), QKV 1024->3072, attention
    out 1024->1024 (the V third of QKV standing in for the attention core, accumulate), pw1
    1024->2048 + GLU, the depthwise convolution (9 taps) + SiLU, pw2 1024->1024 (accumulate), FF2
    in and out as FF1,

run as telmo_amd.conformer.ConformerLayer runs it: the five LayerNorms write quantised rows, FF in
writes quantised hidden rows, pw1 carries the GLU in its epilogue. The LayerNorms, GLU and
convolution are extra work beside the projection set, inside the timed step. Each step is one layer
of a stack, applied in place to the previous step's outputs: it starts from the quantised rows of
its first LayerNorm, which the previous step left, and ends with the layer boundary (its last
LayerNorm and the next layer's first in one launch). The step is timed launched eagerly on one
stream and replayed as a captured HIP graph; the faster is the step time. value = 2 sum(M N K) over
the eight products / step time, in TOPS. Inputs come from telmo's test generator (seeded xorshift,
src/kernels/mod.rs:795-805): synthetic data of the workloads' distributions, random weights.

The JSON line also carries:
  roofline      the eight products' GEMM kernels, each launched alone on the step's quantised rows
                and timed with HIP events on the library's stream: achieved = algorithmic ops per
                launch / average launch time, against the dense int8 MFMA peak (and the dense f16
                peak, the two-digit path's ceiling: it executes two int8 MFMAs per product).
                traffic is the HBM bytes per launch from the rocprofv3 PMC summary committed in
                profiles/ (FETCH_SIZE and WRITE_SIZE scaled by a copy kernel's reading).
  encoder       24 layers at M = 12000 (32 utterances of 30 s) and M = 7500 (one 600 s utterance):
                audio-seconds per second.
  granite       Granite's 16-block encoder (blocks 0 and 1 strided, the self-conditioning) on 60 s.
  timed_s_total the seconds inside every timed region of the run (HIP events).
  gemv, tdt     the decoder's GEMVs on the HBM roofline and the greedy TDT decode.
  vendor        the same product shapes on hipBLASLt (int8 over both digit planes: the same MFMA work)
                and torch's bf16 / f16 GEMMs, for scale.
  cpu_baseline  the C++ port of telmo's SIMD tile + thread pool (oracle/cpu_baseline.cpp,
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
PEAK_F16 = 2.5e15   # dense f16 / bf16 MFMA flop/s (MI355X)
PEAK_HBM = 8.0e12   # bytes/s
METRIC = "int8 GEMM TOPS & %MFMA peak; decode GEMV GB/s & %HBM; encoder audio-s/s"

# The layer's products (the reference's Layer fields, src/parakeet.rs:1011-1172):
# (name, k, n, act, scale, accumulate)
PRODUCTS = [
    ("ff1_in", D, FF, "silu", 1.0, False),
    ("ff1_out", FF, D, "none", 0.5, True),
    ("qkv", D, 3 * D, "none", 1.0, False),
    ("out", D, D, "none", 1.0, True),
    ("pw1", D, CONV, "none", 1.0, False),
    ("pw2", D, D, "none", 1.0, True),
    ("ff2_in", D, FF, "silu", 1.0, False),
    ("ff2_out", FF, D, "none", 0.5, True),
]
NORMS = ("norm_ff1", "norm_att", "norm_conv", "norm_ff2", "norm_out")

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
    """floor(u01 * 255) - 127, worked in integers: u01 = j / 2^24 for the generator's 24-bit j."""
    import telmo_amd

    j = ((telmo_amd.random(n * k, seed) + np.float32(1.0)) * np.float32(8388608.0)).astype(np.int64)
    return (((j * 255) >> 24) - 127).astype(np.int8).reshape(n, k)


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
    return sum(2 * m * k * n for _, k, n, *_ in PRODUCTS)


def bytes_of(m):
    """Algorithmic HBM bytes of the eight products at the f32 surface: A f32, int8 weights, f32
    scales, C f32 (+ C read when accumulating), each tensor once (panels padded to 16 outputs)."""
    total = 0
    for _, k, n, _, _, acc in PRODUCTS:
        npad = -(-n // 16) * 16
        total += 4 * m * k + npad * k + 4 * npad + 4 * m * n * (2 if acc else 1)
    return total


def layer_params(seed, precision=3):
    """One layer's parameters from telmo's generator, on the host: {name: (values, scales, n, k)} in
    the panel layout (int8 with per-output scales U(0.001, 0.01), or Q8_0 (precision 4) with f16-exact
    block scales of the same range), LayerNorms near (1, 0), depthwise taps [9, d] and bias [d]."""
    mats = {}
    for i, (name, k, n, *_) in enumerate(PRODUCTS):
        q = synth_int8(n, k, seed + 10 * i)
        if precision == 4:
            panels, blocks = -(-n // 16), k // 32
            d = synth_scales(panels * 16 * blocks, seed + 10 * i + 1).astype(np.float16).astype(np.float32)
            values, _ = panel_layout(q, np.ones(n, np.float32))
            mats[name] = (values, d, n, k)
        else:
            values, scales = panel_layout(q, synth_scales(n, seed + 10 * i + 1))
            mats[name] = (values, scales, n, k)
    norms = {}
    for i, name in enumerate(NORMS):
        g = (1.0 + 0.1 * synth_normal((D,), seed + 200 + 2 * i)).astype(np.float32)
        b = (0.1 * synth_normal((D,), seed + 201 + 2 * i)).astype(np.float32)
        norms[name] = (g, b)
    dw_w = (0.3 * synth_normal((DW_KERNEL, D), seed + 300)).astype(np.float32)
    dw_b = (0.1 * synth_normal((D,), seed + 301)).astype(np.float32)
    return mats, norms, dw_w, dw_b


# Granite Speech 5's encoder shapes (src/granite.rs:1153-1170): d_model 1024, feed-forward 4096,
# 2048 convolution channels (expansion 2), kernel 7, vocabulary 16384; blocks 0 and 1 are strided.
G_D, G_FF, G_CC, G_KERNEL, G_VOCAB = 1024, 4096, 2048, 7, 16384
G_PRODUCTS = [("ff1_up", G_D, G_FF), ("ff1_down", G_FF, G_D), ("qkv", G_D, 3 * G_D), ("out", G_D, G_D),
              ("pw1", G_D, 2 * G_CC), ("pw2", G_CC, G_D), ("ff2_up", G_D, G_FF), ("ff2_down", G_FF, G_D)]
G_NORMS = ("ff1_norm", "norm_att", "norm_conv", "ff2_norm", "norm_out")


def granite_block_params(seed, strided):
    """One Granite block's parameters from telmo's generator, on the host: int8 matrices {name:
    (values, scales, n, k)} with scales U(0.001, 0.01), biases N(0, 0.1^2) (qkv has none), LayerNorms
    near (1, 0), depthwise taps [7, 2048] and bias [2048], and the stride flag."""
    mats, biases, norms = {}, {}, {}
    for i, (name, k, n) in enumerate(G_PRODUCTS):
        mats[name] = panel_layout(synth_int8(n, k, seed + 10 * i), synth_scales(n, seed + 10 * i + 1)) + (n, k)
        if name != "qkv":
            biases[name] = (0.1 * synth_normal((n,), seed + 10 * i + 2)).astype(np.float32)
    for i, name in enumerate(G_NORMS):
        norms[name] = ((1.0 + 0.1 * synth_normal((G_D,), seed + 200 + 2 * i)).astype(np.float32),
                       (0.1 * synth_normal((G_D,), seed + 201 + 2 * i)).astype(np.float32))
    dw_w = (0.3 * synth_normal((G_KERNEL, G_CC), seed + 300)).astype(np.float32)
    dw_b = (0.1 * synth_normal((G_CC,), seed + 301)).astype(np.float32)
    return mats, biases, norms, dw_w, dw_b, strided


def granite_head_params(seed):
    """The CTC head (vocab x d) and out_mid (d x vocab) with their biases, int8 as above."""
    head = panel_layout(synth_int8(G_VOCAB, G_D, seed), synth_scales(G_VOCAB, seed + 1)) + (G_VOCAB, G_D)
    mid = panel_layout(synth_int8(G_D, G_VOCAB, seed + 2), synth_scales(G_D, seed + 3)) + (G_D, G_VOCAB)
    head_b = (0.1 * synth_normal((G_VOCAB,), seed + 4)).astype(np.float32)
    mid_b = (0.1 * synth_normal((G_D,), seed + 5)).astype(np.float32)
    return head, head_b, mid, mid_b


def upload_granite_block(kern, params):
    import torch

    import telmo_amd
    from telmo_amd.granite import BlockWeights

    mats, biases, norms, dw_w, dw_b, strided = params
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    W = {name: telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, v, s)
         for name, (v, s, n, k) in mats.items()}
    return BlockWeights(W, {name: dev(b) for name, b in biases.items()},
                        {name: (dev(g), dev(b)) for name, (g, b) in norms.items()}, dev(dw_w), dev(dw_b), strided)


def upload_layer(kern, params, precision=3):
    import torch

    import telmo_amd
    from telmo_amd.conformer import LayerWeights

    mats, norms, dw_w, dw_b = params
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    W = {name: telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision(precision), v, s)
         for name, (v, s, n, k) in mats.items()}
    return LayerWeights(W, {name: (dev(g), dev(b)) for name, (g, b) in norms.items()}, dev(dw_w), dev(dw_b))


def close_layer(w):
    for m in w.mats.values():
        m.close()


# Seconds inside every timed region of the run (HIP events), reported as timed_s_total.
TIMED_S = [0.0]


def timed_on(stream, fn, reps):
    """Mean ms per call of fn over reps calls, HIP events on `stream` around them."""
    import torch

    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    TIMED_S[0] += e0.elapsed_time(e1) * 1e-3
    return e0.elapsed_time(e1) / reps


def graph_timed(stream, fn, reps, replays=10):
    """Mean ms per call of fn on the GPU: reps calls captured as one HIP graph, replayed `replays`
    times between HIP events on `stream` (a small kernel's eager launch through Python costs more
    host time than its GPU time, so eager back-to-back calls would time the host)."""
    import torch

    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(reps):
            fn(i)
    graph.replay()
    ms = timed_on(stream, lambda i: graph.replay(), replays) / reps
    del graph
    return ms


def step_times(stream, step, steps, warmup, check, reset):
    """(eager ms, graph ms) of `step`, the graph's output checked equal to an eager step's by check().
    A step works in place on its input rows, so each timed step takes the previous one's outputs as
    its inputs (as the next layer of a stack would); reset() puts the first inputs back, outside the
    timed region, before the comparison of the graph with the eager step."""
    import torch

    for _ in range(warmup):
        step(0)
    eager_ms = timed_on(stream, step, steps)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step(0)
    for _ in range(warmup):
        graph.replay()
    graph_ms = timed_on(stream, lambda i: graph.replay(), steps)
    reset()
    graph.replay()
    torch.cuda.synchronize()
    after_graph = check()
    reset()
    step(0)
    torch.cuda.synchronize()
    if not torch.equal(after_graph, check()):
        raise RuntimeError("graph replay differs from the eager step")
    del graph
    return eager_ms, graph_ms


def gpu_leg(args, params, x0_host):
    """The layer step at T = 750 (eager and graph), then each product's kernel and each row kernel
    of the step launched alone on the step's own buffers."""
    import torch

    import telmo_amd
    from telmo_amd import Act, Epilogue
    from telmo_amd.conformer import ConformerLayer

    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    w = upload_layer(kern, params)
    T = T_FRAMES
    layer = ConformerLayer(kern, D, FF, DW_KERNEL, T)
    x0 = torch.from_numpy(x0_host).cuda()
    x = x0.clone()

    # One layer of a stack: it starts from the quantised rows of its first LayerNorm (norm_ff1), which
    # the previous layer's boundary left, and ends with the boundary (its norm_out in place and the
    # next layer's norm_ff1 in one launch); the same layer stands for the next one.
    def step(_):
        layer.forward(x, T, w, prepared=True, next_norm=w.norms["norm_ff1"])

    def reset():
        x.copy_(x0)
        layer.prepare(x, T, w)

    reset()
    eager_ms, graph_ms = step_times(stream, step, args.steps, args.warmup, lambda: x.clone(), reset)
    if not torch.isfinite(x).all():
        raise RuntimeError("the layer output is not finite")

    # Each product's kernel alone, on quantised rows of the step's kind.
    m = w.mats
    qb = lambda k: torch.empty(kern.quant_bytes(T, k), dtype=torch.uint8, device="cuda")  # noqa: E731
    ex = lambda: torch.empty(T, dtype=torch.int32, device="cuda")  # noqa: E731
    g, b = w.norms["norm_ff1"]
    qa_d, ex_d = qb(D), ex()
    kern.layer_norm_quant_device(x0, D, T, D, g, b, 1e-5, qa_d, ex_d)
    qa_h, ex_h = qb(FF), ex()
    kern.matmul_quantized_to_quant_device(qa_d, ex_d, T, m["ff1_in"], qa_h, ex_h, Epilogue(act=Act.SILU))
    qa_o, ex_o = qb(FF), ex()
    c = torch.zeros((T, D), device="cuda")
    qkv = torch.zeros((T, 3 * D), device="cuda")
    glu = torch.zeros((T, D), device="cuda")
    silu, half_acc, acc = Epilogue(act=Act.SILU), Epilogue(scale=0.5, accumulate=True), Epilogue(accumulate=True)
    hid = torch.zeros((T, FF), device="cuda")
    # FF in as the step runs it: the quantised-output product (the product, then the quantiser of its rows).
    launches = {
        "ff1_in": lambda i: kern.matmul_quantized_to_quant_device(qa_d, ex_d, T, m["ff1_in"], qa_o, ex_o, silu),
        "ff1_out": lambda i: kern.matmul_quantized_device(qa_h, ex_h, T, m["ff1_out"], c, D, half_acc),
        "qkv": lambda i: kern.matmul_quantized_device(qa_d, ex_d, T, m["qkv"], qkv, 3 * D),
        "out": lambda i: kern.matmul_quantized_device(qa_d, ex_d, T, m["out"], c, D, acc),
        "pw1": lambda i: kern.matmul_quantized_glu_device(qa_d, ex_d, T, m["pw1"], glu, D),
        "pw2": lambda i: kern.matmul_quantized_device(qa_d, ex_d, T, m["pw2"], c, D, acc),
        "ff2_in": lambda i: kern.matmul_quantized_to_quant_device(qa_d, ex_d, T, m["ff2_in"], qa_o, ex_o, silu),
        "ff2_out": lambda i: kern.matmul_quantized_device(qa_h, ex_h, T, m["ff2_out"], c, D, half_acc),
    }
    per_shape = []
    for name, k, n, *_ in PRODUCTS:
        for i in range(5):
            launches[name](i)
        ms = graph_timed(stream, launches[name], args.kernel_reps)
        per_shape.append({"product": name, "m": T, "k": k, "n": n, "us": round(ms * 1e3, 3),
                          "tops": round(2 * T * k * n / (ms * 1e-3) / 1e12, 1)})
    dw_out = torch.empty((T, D), device="cuda")
    rows = {
        "layer_norm_quant": lambda i: kern.layer_norm_quant_device(x0, D, T, D, g, b, 1e-5, qa_d, ex_d),
        "quantize_rows (attention output)": lambda i: kern.quantize_rows_device(qkv[:, 2 * D:], 3 * D, T, D, qa_d,
                                                                                ex_d, a_len=qkv.numel() - 2 * D),
        "quantize_rows (hidden)": lambda i: kern.quantize_rows_device(hid, FF, T, FF, qa_o, ex_o),
        "ff_in with quantised output": lambda i: kern.matmul_quantized_to_quant_device(qa_d, ex_d, T, m["ff1_in"],
                                                                                       qa_o, ex_o, silu),
        "dwconv1d + SiLU": lambda i: kern.dwconv1d_device(glu, D, T, D, w.dw_w, DW_KERNEL, w.dw_b, dw_out, D,
                                                          act=Act.SILU),
        "dwconv1d + SiLU, quantised output": lambda i: kern.dwconv1d_quant_device(glu, D, T, D, w.dw_w, DW_KERNEL,
                                                                                  w.dw_b, qa_d, ex_d, act=Act.SILU),
        "quantize_rows (conv output)": lambda i: kern.quantize_rows_device(dw_out, D, T, D, qa_d, ex_d),
        "layer_norm (in place)": lambda i: kern.layer_norm_device(dw_out, D, T, D, g, b, 1e-5, dw_out, D),
    }
    row_us = {}
    for name, fn in rows.items():
        for i in range(5):
            fn(i)
        row_us[name] = round(graph_timed(stream, fn, args.kernel_reps) * 1e3, 3)
    kern.synchronize()
    close_layer(w)
    kern.close()
    return eager_ms, graph_ms, per_shape, row_us


ENC_LAYERS = 24
# (workload, rows, audio seconds, utterances): 32 utterances of 30 s at 80 ms per frame; one 600 s
# utterance.
ENC_CASES = [("batch of 32 x 30 s utterances", 32 * 375, 960.0, 32), ("one 600 s utterance", 7500, 600.0, 1)]


def encoder_leg(args):
    """The encoder stack: 24 device Conformer layers, each with its own weights from telmo's generator
    (580 MB of int8 weights in all), N(0, 1) input rows. One pass runs the 24 layers in order (each
    ending in its LayerNorm); timed eagerly and as a replayed HIP graph, the faster counts.
    Audio-seconds per second = the audio the rows stand for / the time of one pass."""
    import torch

    import telmo_amd
    from telmo_amd.conformer import ConformerLayer

    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    host = [layer_params(5000 + 97 * i) for i in range(ENC_LAYERS)]
    layers = [upload_layer(kern, p) for p in host]
    wbytes = sum(m.bytes() for w in layers for m in w.mats.values())
    stack = ConformerLayer(kern, D, FF, DW_KERNEL, max(rows for _, rows, _, _ in ENC_CASES))
    out = []
    for label, M, audio_s, utt in ENC_CASES:
        x0 = torch.from_numpy(synth_normal((M, D), 60 + M)).cuda()
        x = x0.clone()

        def run(_):
            stack.run_stack(x, M, layers, utterances=utt)

        eager_ms, graph_ms = step_times(stream, run, 3, 1, lambda: x.clone(), lambda: x.copy_(x0))
        if not torch.isfinite(x).all():
            raise RuntimeError("the encoder output is not finite")
        ms = min(eager_ms, graph_ms)
        ops = ENC_LAYERS * ops_of(M)
        out.append({"workload": f"{ENC_LAYERS}-layer encoder, {label}", "m": M, "audio_s": audio_s,
                    "ms_per_pass": round(ms, 3), "ms_per_pass_eager": round(eager_ms, 3),
                    "ms_per_pass_graph": round(graph_ms, 3), "audio_s_per_s": round(audio_s / (ms * 1e-3), 1),
                    "tops": round(ops / (ms * 1e-3) / 1e12, 1), "frac_int8_peak": round(ops / (ms * 1e-3) / PEAK_INT8, 4),
                    "weights_mb": round(wbytes / 1e6, 1)})
        del x0, x
    for w in layers:
        close_layer(w)
    kern.close()
    return out, host


# Granite Speech 5's encoder (src/granite.rs:606-650): 16 blocks, 0 and 1 strided, the
# self-conditioning after block 7 (layers / 2 - 1). 60 s of audio: 3000 rows into block 0, 750 out.
G_BLOCKS, G_STRIDED, G_SELFCOND, G_ROWS = 16, (0, 1), 7, 3000


def granite_ops(rows):
    """2 m n k of one pass's products: the blocks at their row counts and the self-conditioning."""
    ops, t = 0, rows
    for i in range(G_BLOCKS):
        n = t // 2 if i in G_STRIDED else t
        for name, k, nout in G_PRODUCTS:
            m = n if name in ("pw2", "ff2_up", "ff2_down") else t
            ops += 2 * m * k * nout
        if i == G_SELFCOND:
            ops += 2 * 2 * n * G_D * G_VOCAB
        t = n
    return ops


def granite_leg(args):
    """Granite's encoder on the device (telmo_amd.granite): 16 blocks with their own int8 weights from
    telmo's generator (blocks 0 and 1 strided), the self-conditioning after block 7, over 3000 rows
    (60 s of audio) of N(0, 1) input; the attention core is the V third of qkv as in the Parakeet
    leg. One pass timed eagerly (the strided blocks allocate their outputs), median of 5."""
    import torch

    import telmo_amd
    from telmo_amd.granite import GraniteBlock, self_conditioning

    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    blocks = [upload_granite_block(kern, granite_block_params(9000 + 53 * i, i in G_STRIDED))
              for i in range(G_BLOCKS)]
    head, head_b, mid, mid_b = granite_head_params(9900)
    H = telmo_amd.PackedWeights.from_parts(kern, head[2], head[3], telmo_amd.Precision.INT8, head[0], head[1])
    M = telmo_amd.PackedWeights.from_parts(kern, mid[2], mid[3], telmo_amd.Precision.INT8, mid[0], mid[1])
    hb, mb = torch.from_numpy(head_b).cuda(), torch.from_numpy(mid_b).cuda()
    blk = GraniteBlock(kern, G_D, G_FF, G_CC, G_KERNEL, G_ROWS)
    x0 = torch.from_numpy(synth_normal((G_ROWS, G_D), 9950)).cuda()
    bufs = [torch.empty((G_ROWS // 2, G_D), device="cuda"), torch.empty((G_ROWS // 4, G_D), device="cuda")]
    logits = torch.empty(G_ROWS // 4 * G_VOCAB, device="cuda")
    x = torch.empty_like(x0)

    def run(_):
        x.copy_(x0)
        cur, t = x, G_ROWS
        blk.prepare(cur, t, blocks[0])
        ready = True
        for i, w in enumerate(blocks):
            # each block boundary's two LayerNorms in one launch, except where the self-conditioning
            # rewrites the rows between them
            pair = i + 1 < len(blocks) and i != G_SELFCOND
            cur, t = blk.forward(cur, t, w, out=bufs[i] if i in G_STRIDED else None, prepared=ready,
                                 next_norm=blocks[i + 1].norms["ff1_norm"] if pair else None)
            ready = pair
            if i == G_SELFCOND:
                self_conditioning(kern, cur, t, H, hb, M, mb, logits)
        return cur

    for i in range(2):
        run(i)
    times = [timed_on(stream, run, 1) for _ in range(5)]
    ms = float(np.median(times))
    y = run(0)
    kern.synchronize()
    if not torch.isfinite(y).all():
        raise RuntimeError("the Granite encoder output is not finite")
    ops = granite_ops(G_ROWS)
    wbytes = sum(m.bytes() for w in blocks for m in w.mats.values()) + H.bytes() + M.bytes()
    out = {"workload": f"Granite encoder, {G_BLOCKS} blocks (0, 1 strided) and the self-conditioning, "
                       f"{G_ROWS} input rows (60 s audio), d {G_D}, ff {G_FF}, conv {G_CC}, vocab {G_VOCAB}, int8",
           "ms_per_pass": round(ms, 3), "audio_s_per_s": round(60.0 / (ms * 1e-3), 1),
           "tops": round(ops / (ms * 1e-3) / 1e12, 1), "frac_int8_peak": round(ops / (ms * 1e-3) / PEAK_INT8, 4),
           "ops_per_pass": ops, "weights_mb": round(wbytes / 1e6, 1),
           "timing": "HIP events around one eager pass, median of 5"}
    for w in blocks:
        close_layer(w)
    H.close()
    M.close()
    kern.close()
    return out


def q8_leg(args):
    """The same layer step (T = 750) with Q8_0 weights (one f16-exact scale per 32 inputs of each
    output), and the decode joint GEMV (m = 1) with its weights rotated past the Infinity Cache."""
    import torch

    import telmo_amd
    from telmo_amd.conformer import ConformerLayer

    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    w = upload_layer(kern, layer_params(8000, precision=4), precision=4)
    T = T_FRAMES
    layer = ConformerLayer(kern, D, FF, DW_KERNEL, T)
    x0 = torch.from_numpy(synth_normal((T, D), 8100)).cuda()
    x = x0.clone()

    def step(_):  # in place on the previous step's outputs, as the int8 step is timed
        layer.forward(x, T, w, prepared=True, next_norm=w.norms["norm_ff1"])

    def reset():
        x.copy_(x0)
        layer.prepare(x, T, w)

    reset()
    eager_ms, graph_ms = step_times(stream, step, 200, 10, lambda: x.clone(), reset)
    t = min(eager_ms, graph_ms) * 1e-3
    out = {"layer_step": {"workload": "the device Conformer layer at T=750, Q8_0 weights",
                          "ms_per_step": round(t * 1e3, 4), "ms_per_step_eager": round(eager_ms, 4),
                          "ms_per_step_graph": round(graph_ms, 4), "tops": round(ops_of(T) / t / 1e12, 1),
                          "timing": "as the int8 step: the faster of eager launches and HIP graph replay"},
           "rotating": []}
    close_layer(w)
    for name, k, n in (("joint", 640, 8198), ("gates", 640, 2560)):
        panels = -(-n // 16)
        q = synth_int8(n, k, 8200)
        values, _ = panel_layout(q, np.ones(n, np.float32))
        d = synth_scales(panels * 16 * (k // 32), 8201).astype(np.float16).astype(np.float32)
        one = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.Q8_0, values, d)
        copies = [one] + [telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.Q8_0, values, d)
                          for _ in range(int(600e6 // one.bytes()))]
        a = torch.from_numpy(synth_normal((1, k), 8202)).cuda()
        c = torch.empty(1, n, device="cuda")
        call = lambda i: kern.linear_device(a, 1, copies[i % len(copies)], c)  # noqa: E731
        for i in range(len(copies)):
            call(i)
        t = timed_on(stream, call, 4 * len(copies)) * 1e-3
        out["rotating"].append({"gemv": name, "m": 1, "k": k, "n": n, "weight_mb": round(one.bytes() / 1e6, 3),
                                "us": round(t * 1e6, 2), "gb_s": round(one.bytes() / t / 1e9, 1),
                                "hbm_frac": round(one.bytes() / t / PEAK_HBM, 3)})
        for cw in copies:
            cw.close()
    kern.close()
    return out


def gemv_kernel(m):
    """The GEMV body the library runs for m aligned rows of int8 products."""
    return "gemv_dot4" if m == 1 else "gemv_mfma"


def gemv_leg(args):
    """The TDT decode-step GEMVs (m = 1, 4, 8 streams) on the HBM roofline, for the library's choice on
    16-byte aligned rows ("gemv": the dot4 body with no MFMA for one row, the MFMA body for batches of
    streams) and for the row-at-a-time dot4 kernel the library takes for rows that are not 16-byte
    aligned ("dot4_rows": the same call on rows starting one float in).

    (i) each shape with its weights evicted: one pass over copies totalling more than 600 MB (twice
        the 256 MB Infinity Cache and more) is captured as a HIP graph and replayed, so every call
        streams its weights from HBM and the time is the GPU's, not the host's launch loop;
    (ii) the same kernels on one large matrix (64 - 256 MB) for their asymptotic HBM rate;
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
    out = {"rotating": [], "sweep": [], "token_loop": []}

    def rows(m, k, seed, aligned):
        """m rows of k inputs, 16-byte aligned or starting one float in."""
        buf = torch.from_numpy(synth_normal((m * k + 4,), seed)).cuda()
        return buf[:m * k].view(m, k) if aligned else buf[1:1 + m * k].view(m, k)

    def graph_of(calls):
        """The calls captured as one HIP graph (after one eager pass)."""
        for fn in calls:
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for fn in calls:
                fn()
        return g

    shapes = [("joint", 640, 8198, True), ("gates", 640, 2560, False), ("lstm_layer", 1280, 2560, False)]
    for si, (name, k, n, with_bias) in enumerate(shapes):
        values, scales = panel_layout(synth_int8(n, k, 7000 + si), synth_scales(n, 7100 + si))
        one = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
        wbytes = one.bytes()
        copies = [one] + [telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
                          for _ in range(int(600e6 // wbytes))]
        bias = torch.from_numpy(synth_normal((n,), 7200 + si)).cuda() if with_bias else None
        epi = Epilogue(bias=bias)
        for m in (1, 4, 8):
            for kernel, aligned in ((gemv_kernel(m), True), ("dot4_rows", False)):
                a = rows(m, k, 7300 + m, aligned)
                c = torch.empty(m, n, device="cuda")
                alen = (m - 1) * k + k
                g = graph_of([lambda w=w: kern.matmul_device(a, k, m, w, c, n, epi, a_len=alen) for w in copies])
                t = timed_on(stream, lambda i: g.replay(), 4) * 1e-3 / len(copies)
                out["rotating"].append({"gemv": name, "kernel": kernel, "m": m, "k": k, "n": n,
                                        "weight_mb": round(wbytes / 1e6, 3), "us": round(t * 1e6, 2),
                                        "gb_s": round(wbytes / t / 1e9, 1), "hbm_frac": round(wbytes / t / PEAK_HBM, 3)})
                del g
        for w in copies:
            w.close()
    for mb in (64, 256):
        k = 640
        n = int(mb * 1e6 // k) // 16 * 16
        values, scales = panel_layout(synth_int8(n, k, 7400 + mb), synth_scales(n, 7500 + mb))
        w = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
        del values
        for m in (1, 4, 8):
            for kernel, aligned in ((gemv_kernel(m), True), ("dot4_rows", False)):
                a = rows(m, k, 7600 + m, aligned)
                c = torch.empty(m, n, device="cuda")
                call = lambda i: kern.matmul_device(a, k, m, w, c, n, a_len=m * k)  # noqa: E731
                call(0)
                t = timed_on(stream, call, 20) * 1e-3
                out["sweep"].append({"kernel": kernel, "m": m, "k": k, "n": n, "weight_mb": round(w.bytes() / 1e6, 1),
                                     "us": round(t * 1e6, 1), "gb_s": round(w.bytes() / t / 1e9, 1),
                                     "hbm_frac": round(w.bytes() / t / PEAK_HBM, 3)})
        w.close()
    # Token loop.
    vg, sg = panel_layout(synth_int8(2560, 640, 7700), synth_scales(2560, 7701))
    vj, sj = panel_layout(synth_int8(8198, 640, 7702), synth_scales(8198, 7703))
    wg = telmo_amd.PackedWeights.from_parts(kern, 2560, 640, telmo_amd.Precision.INT8, vg, sg)
    wj = telmo_amd.PackedWeights.from_parts(kern, 8198, 640, telmo_amd.Precision.INT8, vj, sj)
    bg = torch.from_numpy(synth_normal((2560,), 7704)).cuda()
    bj = torch.from_numpy(synth_normal((8198,), 7705)).cuda()
    steps = 2000
    for m in (1, 4, 8):
        gates = torch.from_numpy(synth_normal((m, 2560), 7706 + m)).cuda()
        logits = torch.empty(m, 8198, device="cuda")
        g_epi = Epilogue(bias=bg, scale=1.0 / 16)
        j_epi = Epilogue(bias=bj)
        h = gates[:, 640:1280]
        z = gates[:, :640]
        alen = (m - 1) * 2560 + 640

        def step():
            kern.matmul_device(h, 2560, m, wg, gates, 2560, g_epi, a_len=alen)
            kern.matmul_device(z, 2560, m, wj, logits, 8198, j_epi, a_len=alen)

        graph = graph_of([step] * 100)
        graph.replay()
        t = timed_on(stream, lambda i: graph.replay(), steps // 100) * 1e-3 / 100  # s per step
        if not torch.isfinite(logits).all():
            raise RuntimeError("the token loop diverged")
        step_bytes = wg.bytes() + wj.bytes()
        out["token_loop"].append({"m": m, "steps": steps, "us_per_step": round(t * 1e6, 2),
                                  "tokens_per_s": round(m / t, 1), "effective_gb_s": round(step_bytes / t / 1e9, 1),
                                  "note": "weights reused every step (cache-resident), effective rate"})
        del graph
    wg.close()
    wj.close()
    kern.close()
    return out


def host_leg(params, x0):
    """The single GEMM 750 x 1024 -> 4096 (FF1 in, no activation) through the host-pointer entry point
    (tg_linear): the PCIe-inclusive rate a caller handing host slices sees (a copied in, c back)."""
    import telmo_amd

    kern = telmo_amd.Kernels(0)
    values, scales, n, k = params[0]["ff1_in"]
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
    return {"workload": f"one GEMM {T_FRAMES} x {k} -> {n} via tg_linear on host buffers",
            "us": round(dt * 1e6, 1), "tops": round(ops / dt / 1e12, 2), "host_bytes_moved": moved,
            "note": "includes the copy of a to the device and of c back; not the headline value"}


def host_cpu():
    """The host's CPU model and the vector extensions the port can use, from /proc/cpuinfo."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    isa = [x for x in ("avx2", "fma", "avx512f", "avx512bw", "avx512vnni", "avx512_bf16") if x in flags]
    return {"model": model, "logical_cpus_usable": len(os.sched_getaffinity(0)), "isa_flags": isa}


def cpu_leg(params, x0_host, budget_s, enc_params=None):
    """telmo's SIMD + pool path (the C++ port) on the same bytes: the eight products of the layer on
    every host core and on one thread (best of 5 rounds each), the decode joint GEMV (m = 1) on all
    cores with its weights rotated over copies larger than the host's caches, and (enc_params: the 24
    layers' parameters of the GPU encoder leg) one pass of the 24 layers' products over 750 rows,
    best of 3."""
    from oracle import oracle as orc

    L = orc.cpubase()
    L.cb_matmul.argtypes = ([ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                             ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t,
                             ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_void_p,
                             ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_int])
    isa = L.cb_isa()
    if isa == 0:
        return None
    cores = len(os.sched_getaffinity(0))
    T = T_FRAMES
    mats = params[0]
    x = x0_host.copy()
    h = np.zeros((T, FF), np.float32)
    qkv = np.zeros((T, 3 * D), np.float32)
    u = synth_normal((T, D), 9100)
    outs = {"ff1_in": h, "ff1_out": x, "qkv": qkv, "out": x, "pw1": np.zeros((T, CONV), np.float32), "pw2": x,
            "ff2_in": h, "ff2_out": x}
    srcs = {"ff1_in": x, "ff1_out": h, "qkv": x, "pw1": x, "pw2": u, "ff2_in": x, "ff2_out": h}
    p = lambda arr: arr.ctypes.data_as(ctypes.c_void_p)  # noqa: E731

    def gemm(pool, name, act, scale, accumulate, mats_of=None):
        values, scales, n, k = (mats_of or mats)[name]
        if name == "out":  # the V third of QKV: rows 3D apart, starting at column 2D
            a_ptr, lda = ctypes.c_void_p(qkv.ctypes.data + 4 * 2 * D), 3 * D
        else:
            a_ptr, lda = p(srcs[name]), k
        out = outs[name]
        rc = L.cb_matmul(pool, isa, a_ptr, (T - 1) * lda + k, lda, T, p(values), p(scales), 3, n, k, p(out),
                         out.size, n, None, 0, 2 if act == "silu" else 0, scale, int(accumulate))
        assert rc == 0, rc

    def layer(pool, mats_of=None):
        for name, k, n, act, scale, accumulate in PRODUCTS:
            gemm(pool, name, act, scale, accumulate, mats_of)

    # Bit-identity with the fused oracle before timing (FF1 in on the layer input).
    pool = L.cb_pool_new(cores)
    values, scales, n, k = mats["ff1_in"]
    got, want = np.zeros((T, n), np.float32), np.zeros((T, n), np.float32)
    assert L.cb_matmul(pool, isa, p(x0_host), x0_host.size, k, T, p(values), p(scales), 3, n, k, p(got), got.size, n,
                       None, 0, 2, 1.0, 0) == 0
    orc.matmul(True, x0_host.reshape(-1), k, T, values, scales, 3, n, k, want.reshape(-1), n, None, 2, 1.0, False)
    if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
        raise RuntimeError("the CPU baseline differs from the fused oracle")

    def best_of(pool, seconds):
        t0 = time.perf_counter()
        x[:] = x0_host
        layer(pool)
        one = time.perf_counter() - t0
        reps = max(1, int(seconds / 5 / one))
        best = float("inf")
        for _ in range(5):
            t0 = time.perf_counter()
            for _ in range(reps):
                x[:] = x0_host
                layer(pool)
            best = min(best, (time.perf_counter() - t0) / reps)
        return best, reps

    best, reps = best_of(pool, budget_s * 0.5)
    pool1 = L.cb_pool_new(1)
    best1, reps1 = best_of(pool1, budget_s * 0.3)
    L.cb_pool_free(pool1)
    # The joint GEMV (m = 1, 640 -> 8198) over copies larger than the caches, as benches/weights.rs does.
    k, n = 640, 8198
    jv, js = panel_layout(synth_int8(n, k, 9200), synth_scales(n, 9201))
    copies = [jv.copy() for _ in range(max(2, int(256e6 // jv.nbytes)))]
    a = synth_normal((1, k), 9202).reshape(-1)
    c = np.zeros(n, np.float32)
    jbytes = jv.nbytes + js.nbytes
    for cv in copies:
        L.cb_matmul(pool, isa, p(a), k, k, 1, p(cv), p(js), 3, n, k, p(c), n, n, None, 0, 0, 1.0, 0)
    gemv_best = float("inf")
    for _ in range(3):
        t0 = time.perf_counter()
        for cv in copies:
            L.cb_matmul(pool, isa, p(a), k, k, 1, p(cv), p(js), 3, n, k, p(c), n, n, None, 0, 0, 1.0, 0)
        gemv_best = min(gemv_best, (time.perf_counter() - t0) / len(copies))
    enc = None
    if enc_params:
        enc = float("inf")
        for _ in range(3):
            t0 = time.perf_counter()
            x[:] = x0_host
            for lp in enc_params:
                layer(pool, lp[0])
            enc = min(enc, time.perf_counter() - t0)
    L.cb_pool_free(pool)
    return {"value": round(ops_of(T) / best / 1e12, 4), "unit": "TOPS", "cores": cores,
            "kind": "port", "isa": "avx512" if isa == 2 else "avx2", "host": host_cpu(),
            "sample": f"the layer's eight products at T={T} (GEMMs only: LayerNorms, GLU and convolution not "
                      f"ported), best of 5 rounds of {reps} layers on {cores} threads "
                      f"({reps * 5 * best:.1f} s), the same bytes as the GPU step",
            "ms_per_step": round(best * 1e3, 3),
            "one_thread": {"value": round(ops_of(T) / best1 / 1e12, 4), "unit": "TOPS", "cores": 1,
                           "ms_per_step": round(best1 * 1e3, 3),
                           "sample": f"best of 5 rounds of {reps1} layers on one thread"},
            "gemv_rotating": {"gemv": "joint 640 -> 8198, m = 1", "copies": len(copies),
                              "copy_mb": round(jbytes / 1e6, 2), "us": round(gemv_best * 1e6, 1),
                              "gb_s": round(jbytes / gemv_best / 1e9, 2), "cores": cores},
            "encoder_audio_s_per_s": None if enc is None else round(T * 0.08 / enc, 1),
            "encoder_ms_per_pass": None if enc is None else round(enc * 1e3, 1),
            "encoder_note": f"one pass of {ENC_LAYERS} layers' products (each layer its own weights, those of the "
                            f"GPU encoder leg) over {T} frames (80 ms each, 60 s of audio) on {cores} threads, best "
                            "of 3, measured: the CPU path's encoder audio-seconds per second, GEMMs only (the "
                            "LayerNorms, GLU and convolution are not ported)"}


# The TDT decoder of Parakeet: h = 640, vocab 8193 (blank last) + 5 durations, 2 LSTM layers.
TDT_H, TDT_VOCAB, TDT_DURS, TDT_MAX_SYMBOLS = 640, 8193, [0, 1, 2, 3, 4], 10
TDT_BLANK_BIAS = 28.0  # on random weights: blank runs between tokens


def tdt_network(seed=21, precision=3):
    """A random network of Parakeet's decoder shapes in the panel layout (numpy), from telmo's
    generator: int8 weights with per-output scales in [lo, hi) (precision 3), or the same int8 values
    with f16-exact scales in [lo, hi) per 32 inputs of each output (Q8_0, precision 4); N(0, 1)
    biases and embedding."""
    h, vocab = TDT_H, TDT_VOCAB
    seeds = iter(range(seed * 100, seed * 100 + 100))

    def mat(n, k, lo, hi):
        q = synth_int8(n, k, next(seeds))
        if precision == 4:
            values, _ = panel_layout(q, np.ones(n, np.float32))
            d = lo + (hi - lo) * synth_u01(-(-n // 16) * 16 * (k // 32), next(seeds))
            return values, d.astype(np.float16).astype(np.float32)
        return panel_layout(q, (lo + (hi - lo) * synth_u01(n, next(seeds))).astype(np.float32))

    outputs = vocab + len(TDT_DURS)
    joint_b = (0.5 * synth_normal((outputs,), next(seeds))).astype(np.float32)
    joint_b[vocab - 1] += TDT_BLANK_BIAS
    return {"p": precision, "h": h, "vocab": vocab, "durations": TDT_DURS, "max_symbols": TDT_MAX_SYMBOLS,
            "joint": mat(outputs, h, 0.001, 0.01), "joint_b": joint_b,
            "emb": (0.5 * synth_normal((vocab, h), next(seeds))).astype(np.float32),
            "lstm": [mat(4 * h, 2 * h, 0.0004, 0.0008) for _ in range(2)],
            "lstm_b": [(0.1 * synth_normal((4 * h,), next(seeds))).astype(np.float32) for _ in range(2)],
            "proj": mat(h, h, 0.001, 0.003), "proj_b": (0.1 * synth_normal((h,), next(seeds))).astype(np.float32)}


def tdt_leg(args, net, enc_host):
    """The greedy TDT decode of 60 s of audio (750 encoder frames) on the device, from the start
    state (the blank through the prediction network), through tg_tdt_decode_device: one call, every
    step on the GPU, the host waking once per batch of steps. Reported per decode (median of 5)."""
    import torch

    import telmo_amd

    kern = telmo_amd.Kernels(0)
    h, vocab = net["h"], net["vocab"]
    P = telmo_amd.Precision(net["p"])
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

    def timed():
        times, toks, state = [], None, None
        for _ in range(6):
            state, pred = state0.clone(), pred0.clone()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            toks, frame, _ = dec.decode(enc, state, pred)
            times.append(time.perf_counter() - t0)
        return float(np.median(times[1:])) * 1e3, toks, state.cpu().numpy()

    resident = dec.resident
    ms, toks, state_r = timed()
    steps_one = dec.last_steps if resident else None
    steps_ms = None
    if resident:  # the same decode as a graph of step kernels, for comparison
        dec.set_resident(False)
        steps_ms, steps_toks, state_s = timed()
        if steps_toks != toks or np.max(np.abs(state_s - state_r)) > 1e-4:
            raise RuntimeError("the resident and step-kernel decodes differ")
        dec.set_resident(True)
    frames = enc_host.shape[0]
    weight_bytes = joint.bytes() + sum(w.bytes() for w in lstm) + proj.bytes()
    # Several streams of 60 s each in one resident launch (M concurrent decode streams), each
    # with encoder rows of its own; the first stream's are the single decode's.
    multi = []
    if resident and net["p"] == 3:
        for m in (4, 8):
            encs = [enc] + [dev(synth_normal(enc_host.shape, 2300 + q)) for q in range(1, m)]
            times, got = [], None
            for _ in range(4):
                sts = [state0.clone() for _ in range(m)]
                prs = [pred0.clone() for _ in range(m)]
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                got = dec.decode_streams(encs, sts, prs)
                times.append(time.perf_counter() - t0)
            if got[0][0] != toks:
                raise RuntimeError("the multi-stream decode's first stream differs from the single decode")
            mms = float(np.median(times[1:])) * 1e3
            ntok = sum(len(g[0]) for g in got)
            steps = dec.last_steps
            multi.append({"streams": m, "ms_per_decode": round(mms, 3), "steps": steps,
                          "us_per_step": round(mms * 1e3 / max(steps, 1), 2), "tokens": ntok,
                          "tokens_per_s": round(ntok / (mms * 1e-3), 1),
                          "audio_s_per_s": round(60.0 * m / (mms * 1e-3), 1)})
    out = {"workload": f"greedy TDT decode, {frames} frames (60 s audio), h={h}, vocab {vocab} + "
                       f"{len(TDT_DURS)} durations, 2 LSTM layers, {'Q8_0' if net['p'] == 4 else 'int8'}",
           "frames": frames, "tokens": len(toks), "tokens_per_frame": round(len(toks) / frames, 3),
           "ms_per_decode": round(ms, 3), "us_per_token": round(ms * 1e3 / max(len(toks), 1), 2),
           "audio_s_per_s": round(60.0 / (ms * 1e-3), 1), "decoder_weight_mb": round(weight_bytes / 1e6, 2),
           "resident": resident,
           "steps": steps_one, "us_per_step": None if not steps_one else round(ms * 1e3 / steps_one, 2),
           "multi_stream": multi,
           "step_kernels_ms_per_decode": None if steps_ms is None else round(steps_ms, 3),
           "step_kernels_us_per_token": None if steps_ms is None else round(steps_ms * 1e3 / max(len(toks), 1), 2),
           "timing": "wall clock around tg_tdt_decode_device (blocks until the decode ends), median of 5; "
                     "resident: one launch with the matrices in LDS; step kernels: four kernels per step as a graph"}
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


VENDOR_SHAPES = [(750, 1024, 4096), (750, 4096, 1024), (750, 1024, 1024), (12000, 1024, 4096), (12000, 4096, 1024),
                 (12000, 1024, 1024)]


def vendor_leg(reps=20):
    """The same products on the vendor library, for scale. For each shape: this library's product on
    quantised rows (tg_matmul_quantized_device, f32 out), hipBLASLt's int8 GEMM through
    torch._int_mm on both digit planes stacked (2m x k int8 times k x n int8, int32 out: the same
    MFMA work as the two-digit product, without its dequantisation), on one digit plane (m rows:
    a plain int8 GEMM, which misses the 1e-3 gate) and torch's bf16 and f16 GEMMs (m x k times
    k x n). All timed with HIP events over `reps` launches after 3 untimed ones."""
    import torch

    import telmo_amd

    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)

    def us_of(fn):
        for _ in range(3):
            fn(0)
        return timed_on(stream, fn, reps) * 1e3

    out = []
    for m, k, n in VENDOR_SHAPES:
        values, scales = panel_layout(synth_int8(n, k, 1), synth_scales(n, 2))
        w = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
        a = torch.from_numpy(synth_normal((m, k), 3)).cuda()
        qa = torch.empty(kern.quant_bytes(m, k), dtype=torch.uint8, device="cuda")
        exps = torch.empty(m, dtype=torch.int32, device="cuda")
        c = torch.empty((m, n), device="cuda")
        kern.quantize_rows_device(a, k, m, k, qa, exps)
        ours = us_of(lambda i: kern.matmul_quantized_device(qa, exps, m, w, c, n))
        w.close()
        del qa, exps, c
        a8 = torch.randint(-127, 128, (2 * m, k), dtype=torch.int8, device="cuda")
        b8 = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda").t()
        two = us_of(lambda i: torch._int_mm(a8, b8))
        one = us_of(lambda i: torch._int_mm(a8[:m], b8))
        del a8, b8
        row = {"shape": [m, k, n], "ours_us": round(ours, 2), "hipblaslt_int8_two_planes_us": round(two, 2),
               "hipblaslt_int8_one_plane_us": round(one, 2)}
        for name, dt in (("torch_bf16_us", torch.bfloat16), ("torch_f16_us", torch.float16)):
            x = a.to(dt)
            y = torch.randn(k, n, dtype=dt, device="cuda")
            row[name] = round(us_of(lambda i: x @ y), 2)
            del x, y
        row["ours_vs_hipblaslt_two_planes"] = round(two / ours, 3)
        out.append(row)
        del a
    kern.close()
    torch.cuda.synchronize()
    return {"note": "vendor GEMMs on the same shapes: hipBLASLt int8 over both digit planes is the two-digit "
                    "product's MFMA work (int32 out, no epilogue); bf16 misses the 1e-3 gate, f16 passes it "
                    "without exact integer sums",
            "shapes": out}


def gemv_shape_leg(m, k, n, reps):
    """One decode GEMV shape alone (tg_matmul_device on m rows of k inputs, the GEMV path), the
    program rocprofv3 runs for the GEMV's kernel statistics and HBM byte counters: `reps` eager
    launches rotating over copies of the weights totalling more than 600 MB (twice the 256 MB
    Infinity Cache and more), so every launch streams its weights from HBM."""
    import torch

    import telmo_amd

    values, scales = panel_layout(synth_int8(n, k, 7000), synth_scales(n, 7100))
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    one = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
    copies = [one] + [telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
                      for _ in range(int(600e6 // one.bytes()))]
    a = torch.from_numpy(synth_normal((m, k), 7300 + m)).cuda()
    c = torch.empty((m, n), device="cuda")
    for w in copies[:3]:
        kern.matmul_device(a, k, m, w, c, n)
    ms = timed_on(stream, lambda i: kern.matmul_device(a, k, m, copies[i % len(copies)], c, n), reps)
    wbytes = one.bytes()
    for w in copies:
        w.close()
    kern.close()
    return {"gemv_shape": [m, k, n], "reps": reps, "copies": len(copies), "weight_bytes": wbytes,
            "us_per_launch": round(ms * 1e3, 3), "gb_s": round(wbytes / (ms * 1e-3) / 1e9, 1),
            "note": "eager launches (the launch gaps included); rotating copies, weights from HBM"}


def load_traffic():
    path = os.path.join(ROOT, "profiles", "layer_T750_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--kernel-reps", type=int, default=100,
                    help="launches per captured graph in the per-kernel legs (the graph is replayed 10 times)")
    ap.add_argument("--cpu-seconds", type=float, default=16.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemv", action="store_true")
    ap.add_argument("--no-encoder", action="store_true")
    ap.add_argument("--no-q8", action="store_true")
    ap.add_argument("--no-tdt", action="store_true")
    ap.add_argument("--no-vendor", action="store_true")
    ap.add_argument("--no-granite", action="store_true")
    ap.add_argument("--shape", type=int, nargs=3, metavar=("M", "K", "N"),
                    help="time one product shape alone (the program for per-shape rocprofv3 runs) and exit")
    ap.add_argument("--gemv", type=int, nargs=3, metavar=("M", "K", "N"),
                    help="time one decode GEMV shape over rotating weight copies (for rocprofv3 runs) and exit")
    ap.add_argument("--reps", type=int, default=20, help="launches timed with --shape or --gemv")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        sys.exit("bench.py measures one GPU and has no multi-GPU path: run it with --gpus 1")
    if args.shape:
        print(json.dumps(shape_leg(*args.shape, args.reps)), flush=True)
        return
    if args.gemv:
        print(json.dumps(gemv_shape_leg(*args.gemv, args.reps)), flush=True)
        return

    params = layer_params(100)
    x0 = synth_normal((T_FRAMES, D), 0)
    eager_ms, graph_ms, per_shape, row_us = gpu_leg(args, params, x0)
    ops = ops_of(T_FRAMES)
    gemm_us = sum(s["us"] for s in per_shape)
    achieved = ops / (gemm_us * 1e-6)
    dominant = max(per_shape, key=lambda s: s["us"])
    traffic = load_traffic()
    roofline = {"bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": PEAK_INT8 / 1e12, "unit": "TOPS",
                "frac": round(achieved / PEAK_INT8, 4),
                "frac_vs_dense_f16_peak": round(achieved / PEAK_F16, 4),
                "mfma_exec_frac_derived": round(2 * achieved / PEAK_INT8, 4),
                "traffic": traffic.get("traffic_bytes_per_launch") if traffic else None,
                "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of these launches, committed in "
                                  "profiles/layer_T750_traffic.json (not measured in this run)" if traffic else None,
                "kernel": "the eight products of the layer step as it runs them, each launched alone (FF in: the "
                          "quantised-output product and its row quantiser), GPU time per launch from a replayed graph "
                          "of back-to-back launches",
                "dominant": dominant["product"],
                "avg_launch_us": round(gemm_us / len(per_shape), 3), "ops_per_launch_avg": ops / len(per_shape),
                "note": "two int8 digits per activation: the MFMAs execute 2x the algorithmic ops, so the "
                        "two-digit path's ceiling is the dense f16 rate; mfma_exec_frac_derived = 2 achieved / "
                        "int8 peak, computed, not a counter",
                "per_shape": per_shape, "row_kernels_us": row_us}
    gemv = None if args.no_gemv else gemv_leg(args)
    host = host_leg(params, x0)
    encoder, enc_params = (None, None) if args.no_encoder else encoder_leg(args)
    granite = None if args.no_granite else granite_leg(args)
    q8 = None if args.no_q8 else q8_leg(args)
    tdt = None
    if not args.no_tdt:
        net = tdt_network()
        enc = synth_normal((T_FRAMES, TDT_H), 22)
        tdt, gpu_toks = tdt_leg(args, net, enc)
        if q8 is not None:
            q8["tdt"], _ = tdt_leg(args, tdt_network(precision=4), enc)
    vendor = None if args.no_vendor else vendor_leg()
    cpu = None if args.no_cpu else cpu_leg(params, x0, args.cpu_seconds, enc_params)
    if cpu is not None and tdt is not None:
        cpu["tdt_decode"], port_toks, oracle_toks = cpu_tdt(net, enc, 150)
        if port_toks is not None:
            gpu = [tuple(t) for t in gpu_toks]
            # the port's tokens (fused f32 sums, as telmo's decode) are the GPU decode's, and the
            # oracle's over the first frames are its first tokens
            tdt["cpu_port_tokens_match"] = gpu == port_toks
            tdt["oracle_sample_tokens_match"] = gpu[:len(oracle_toks)] == oracle_toks
    step_ms = min(graph_ms, eager_ms)
    value = ops / (step_ms * 1e-3) / 1e12
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic (telmo's seeded test generator)",
        "config": {"workload": "one Conformer layer on the device at T=750 frames (60 s audio), d=1024, ff=4096, "
                               "conv 2048: the eight int8 products of the layer projection set in Parakeet::layer's "
                               "order, with its LayerNorms, GLU and depthwise convolution",
                   "frames": T_FRAMES, "ops_per_step": ops, "hbm_bytes_per_step_f32_surface": bytes_of(T_FRAMES),
                   "ms_per_step_eager": round(eager_ms, 5), "ms_per_step_graph": round(graph_ms, 5),
                   "timing": "HIP events around the timed steps; the faster of eager launches and HIP graph replay",
                   "audio_s_per_s_one_layer": round(60.0 / (step_ms * 1e-3), 1)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "gemv": gemv,
        "pcie_inclusive": host,
        "encoder": encoder,
        "granite": granite,
        "q8_0": q8,
        "tdt": tdt,
        "vendor": vendor,
        "timed_s_total": round(TIMED_S[0], 3),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
