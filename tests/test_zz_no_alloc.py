"""tg_matmul_device_noalloc, the entry point that allocates nothing, against tg_matmul_device through
the C ABI on an MI355X: the same bits for the same inputs, on consecutive calls that share the
per-GPU scratch (the second with a smaller input), and a clear refusal past the scratch's size."""
import numpy as np
import pytest

import bench
from helpers import rel_norm_err

pytestmark = pytest.mark.gpu


def say(*args):
    print("[case]", *args, flush=True)


def weights(tk, n, k, seed):
    import telmo_amd

    values, scales = bench.panel_layout(bench.synth_int8(n, k, seed), bench.synth_scales(n, seed + 1))
    return values, scales, telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)


# (m, k, n, lda, act, accumulate): a large product first, then smaller ones reusing the scratch;
# a strided input; a GEMV-sized one (no scratch); the exact mode's.
CASES = [(750, 4096, 1024, 4096, 2, False), (300, 1000, 500, 1000, 0, True), (37, 1024, 3072, 3072, 1, False),
         (8, 640, 2560, 640, 0, False)]


def test_no_alloc_matches_matmul_device_on_consecutive_calls(tk, orc):
    import torch

    import telmo_amd

    for i, (m, k, n, lda, act, acc) in enumerate(CASES):
        values, scales, w = weights(tk, n, k, 500 + i)
        a = torch.from_numpy(bench.synth_normal((m, lda), 510 + i)).cuda()
        c0 = torch.from_numpy(bench.synth_normal((m, n), 520 + i)).cuda()
        epi = telmo_amd.Epilogue(act=telmo_amd.Act(act), scale=0.5, accumulate=acc)
        alen = (m - 1) * lda + k
        say("no-alloc", m, k, n, lda)
        want = c0.clone()
        tk.matmul_device(a, lda, m, w, want, n, epi, a_len=alen)
        got = c0.clone()
        tk.matmul_device_noalloc(a, lda, m, w, got, n, epi, a_len=alen)
        tk.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (m, k, n)
        ref = c0.cpu().numpy().reshape(-1).copy()
        orc.matmul_fast(a.cpu().numpy().reshape(-1)[:alen], lda, m, values, scales, n, k, ref, n, None, act, 0.5, acc)
        assert np.array_equal(got.cpu().numpy().reshape(-1).view(np.uint32), ref.view(np.uint32))
        w.close()


def test_no_alloc_in_exact_mode_and_past_the_scratch(tk, orc):
    import torch

    import telmo_amd

    m, k, n = 40, 300, 70
    values, scales, w = weights(tk, n, k, 600)
    a = torch.from_numpy(bench.synth_normal((m, k), 601)).cuda()
    tk.set_mode(tk.EXACT)
    try:
        got = torch.zeros((m, n), device="cuda")
        tk.matmul_device_noalloc(a, k, m, w, got, n)
        tk.synchronize()
    finally:
        tk.set_mode(tk.FAST)
    want = np.zeros(m * n, np.float32)
    orc.matmul(True, a.cpu().numpy().reshape(-1), k, m, values, scales, 3, n, k, want, n)
    assert np.array_equal(got.cpu().numpy().reshape(-1).view(np.uint32), want.view(np.uint32))
    w.close()
    # 2100 rows of 4096 inputs need 33 x 64 x 2 KB = 16.5 MiB of quantised rows: refused, c untouched
    m, k, n = 2100, 4096, 64
    values, scales, w = weights(tk, n, k, 610)
    a = torch.zeros((m, k), device="cuda")
    c = torch.full((m, n), 5.0, device="cuda")
    with pytest.raises(telmo_amd.TelmoError, match="no-allocation scratch"):
        tk.matmul_device_noalloc(a, k, m, w, c, n)
    tk.synchronize()
    assert bool((c == 5.0).all())
    w.close()
