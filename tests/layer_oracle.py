"""Parakeet::layer (src/parakeet.rs:1011-1172) composed from the oracle's functions, what the tests
check the device layer (telmo_amd.conformer) against: LayerNorm rows (or_layer_norm), products (the integer oracle
or_matmul_fast of the fast path, or the fused f32 reference or_matmul), the GLU, the depthwise
convolution + SiLU per utterance, in the reference's order, with the V third of qkv standing in for
the attention core as the device layer's default does. Products the device makes through
tg_matmul_device (the attention output's, which quantises f32 rows itself) take the integer oracle
with the entry point's accuracy guard; the staged products of quantised rows take it without."""
import numpy as np

NONE, SILU = 0, 2
INT8, Q8_0 = 3, 4


def oracle_layer(orc, x, mats, norms, dw_w, dw_b, utterances=1, fast=True, precision=INT8):
    """The layer on numpy rows x [t, d] (returned, x untouched): fast = True composes the integer
    oracle (the device layer's bits), False the reference's fused f32 products. precision Q8_0 (4):
    the matrices are Q8_0 (the Q8_0 integer oracle)."""
    x = x.copy()
    t, d = x.shape
    q8 = precision == Q8_0

    def linear(a, lda, name, c, act=NONE, scale=1.0, accumulate=False, guard=False):
        values, scales, n, k = mats[name]
        flat = np.ascontiguousarray(a).reshape(-1)
        out = c.reshape(-1)
        if fast:
            rc = (orc.matmul_fast_q8 if q8 else orc.matmul_fast)(flat, lda, t, values, scales, n, k, out, n, None,
                                                                 act, scale, accumulate, guard=guard)
        else:
            rc = orc.matmul(True, flat, lda, t, values, scales, precision, n, k, out, n, None, act, scale,
                            accumulate)
        assert rc == 0
        return out.reshape(t, n)

    def ln(rows, norm):
        g, b = norms[norm]
        return np.stack([orc.layer_norm(rows[r], g, b, 1e-5) for r in range(t)])

    def feed_forward(norm, w_in, w_out):
        h = ln(x, norm)
        hid = linear(h, d, w_in, np.zeros((t, mats[w_in][2]), np.float32), SILU)
        linear(hid, hid.shape[1], w_out, x, NONE, 0.5, True)

    feed_forward("norm_ff1", "ff1_in", "ff1_out")
    h = ln(x, "norm_att")
    qkv = linear(h, d, "qkv", np.zeros((t, 3 * d), np.float32))
    linear(qkv.reshape(-1)[2 * d:], 3 * d, "out", x, NONE, 1.0, True, guard=True)  # tg_matmul_device
    h = ln(x, "norm_conv")
    g = linear(h, d, "pw1", np.zeros((t, 2 * d), np.float32))
    u = np.stack([orc.glu(g[r, :d], g[r, d:]) for r in range(t)])
    frames = t // utterances
    conv = np.concatenate([orc.dwconv1d(u[s * frames:(s + 1) * frames], dw_w, dw_b, silu=True)
                           for s in range(utterances)])
    linear(conv, d, "pw2", x, NONE, 1.0, True)
    feed_forward("norm_ff2", "ff2_in", "ff2_out")
    return ln(x, "norm_out")


def oracle_granite_block(orc, x, mats, biases, norms, dw_w, dw_b, strided, utterances=1, fast=True):
    """Granite::block_span (src/granite.rs:800-952) over whole utterances on numpy rows x [t, d],
    composed from the oracle's functions; returns the output rows (t // utterances // 2 per utterance
    for a strided block, else t). fast as in oracle_layer."""
    x = x.copy()
    t, d = x.shape

    def linear(a, rows, name, c, act=NONE, scale=1.0, accumulate=False, lda=None, guard=False):
        values, scales, n, k = mats[name]
        flat = np.ascontiguousarray(a).reshape(-1)
        out = c.reshape(-1)
        bias = biases.get(name)
        lda = k if lda is None else lda
        if fast:
            rc = orc.matmul_fast(flat, lda, rows, values, scales, n, k, out, n, bias, act, scale, accumulate,
                                 guard=guard)
        else:
            rc = orc.matmul(True, flat, lda, rows, values, scales, INT8, n, k, out, n, bias, act, scale,
                            accumulate)
        assert rc == 0
        return out.reshape(rows, n)

    def ln(rows, norm):
        g, b = norms[norm]
        return np.stack([orc.layer_norm(r, g, b, 1e-5) for r in rows])

    def feed_forward(y, which):
        rows = y.shape[0]
        h = ln(y, which + "_norm")
        hid = linear(h, rows, which + "_up", np.zeros((rows, mats[which + "_up"][2]), np.float32), SILU)
        linear(hid, rows, which + "_down", y, NONE, 0.5, True)

    feed_forward(x, "ff1")
    h = ln(x, "norm_att")
    qkv = linear(h, t, "qkv", np.zeros((t, 3 * d), np.float32))
    linear(qkv.reshape(-1)[2 * d:], t, "out", x, NONE, 1.0, True, lda=3 * d, guard=True)  # tg_matmul_device
    h = ln(x, "norm_conv")
    cc = mats["pw2"][3]
    g = linear(h, t, "pw1", np.zeros((t, 2 * cc), np.float32))
    u = np.stack([orc.glu(g[r, :cc], g[r, cc:]) for r in range(t)])
    frames = t // utterances
    if strided:
        rows = frames // 2
        conv = np.concatenate([orc.dwconv1d(u[s * frames:(s + 1) * frames], dw_w, dw_b, rows=rows, stride=2,
                                            silu=True) for s in range(utterances)])
        out = np.concatenate([(x[s * frames:s * frames + 2 * rows:2] + x[s * frames + 1:s * frames + 2 * rows:2])
                              / np.float32(2.0) for s in range(utterances)]).astype(np.float32)
    else:
        conv = np.concatenate([orc.dwconv1d(u[s * frames:(s + 1) * frames], dw_w, dw_b, silu=True)
                               for s in range(utterances)])
        out = x
    n = out.shape[0]
    linear(conv, n, "pw2", out, NONE, 1.0, True)
    feed_forward(out, "ff2")
    return ln(out, "norm_out")


def oracle_self_conditioning(orc, x, head, head_b, mid, mid_b, fast=True):
    """x + mid(softmax(head(x) + head.b)) + mid.b (src/granite.rs:1040-1069, 639-647) on numpy rows,
    the injection added by the product's accumulating epilogue as the device does (the same bits as
    the reference's separate add)."""
    x = x.copy()
    t, d = x.shape

    def linear(a, name_mat, bias, c, accumulate):
        values, scales, n, k = name_mat
        flat = np.ascontiguousarray(a).reshape(-1)
        out = c.reshape(-1)
        if fast:  # both products go through tg_matmul_device, whose guard applies
            rc = orc.matmul_fast(flat, k, t, values, scales, n, k, out, n, bias, NONE, 1.0, accumulate, guard=True)
        else:
            rc = orc.matmul(True, flat, k, t, values, scales, INT8, n, k, out, n, bias, NONE, 1.0, accumulate)
        assert rc == 0
        return out.reshape(t, n)

    logits = linear(x, head, head_b, np.zeros((t, head[2]), np.float32), False)
    post = orc.softmax(logits)
    linear(post, mid, mid_b, x, True)
    return x
