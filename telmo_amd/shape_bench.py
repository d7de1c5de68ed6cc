"""Times one int8-weight product shape on the GPU: python -m telmo_amd.shape_bench M K N [REPS].

The activations are quantised once; the timed region holds REPS launches of the MFMA GEMM alone
(tg_matmul_quantized_device) on the context's stream, bracketed by HIP events on that stream.
Weights are int8 uniform in [-127, 127] with per-row scales in [0.001, 0.01) (seed 0), activations
N(0, 1). Prints the mean time per launch and the algorithmic rate, 2 M N K / time. Used as the
program under rocprofv3 for per-shape kernel statistics and counters."""
import sys

import numpy as np


def main(argv):
    if len(argv) not in (3, 4):
        print(__doc__.splitlines()[0])
        return 2
    import torch

    import telmo_amd

    m, k, n = (int(x) for x in argv[:3])
    reps = int(argv[3]) if len(argv) == 4 else 20
    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    s = (0.001 + 0.009 * rng.random(n)).astype(np.float32)
    panels = -(-n // 16)
    pad = np.zeros((panels * 16, k), np.int8)
    pad[:n] = q
    values = pad.reshape(panels, 16, k).transpose(0, 2, 1).reshape(-1).view(np.uint8).copy()
    scales = np.zeros(panels * 16, np.float32)
    scales[:n] = s
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    w = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    a = torch.randn((m, k), generator=gen, device="cuda")
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
    print(f"M={m} K={k} N={n}: {us:.2f} us per launch, {2 * m * n * k / us / 1e6:.1f} TOPS", flush=True)
    w.close()
    kern.close()
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
