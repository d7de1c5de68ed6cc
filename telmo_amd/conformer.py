"""One Conformer layer of Parakeet's encoder on the device, in the reference's order.

``ConformerLayer.forward`` runs ``Parakeet::layer`` (src/parakeet.rs:1011-1172) on rows resident in
GPU memory, with every int8 product on the library's fast path and the rows between products kept
quantised wherever the product is their only reader:

    FF1   LayerNorm(norm_ff1)       -> quantised rows          tg_layer_norm_quant_device
          ff1_in + SiLU             -> quantised hidden rows   tg_matmul_quantized_device + the row
                                                               quantiser, or (quantised_hidden)
                                                               tg_matmul_quantized_to_quant_device
          ff1_out, x += 0.5 * .                                tg_matmul_quantized_device
    att   LayerNorm(norm_att)       -> quantised rows
          qkv                       -> f32 q, k, v (the attention core reads them)
          [pos_proj of the positions, when given]
          attention(q, k, v) -> att  (the caller's; outside this path: the V third stands in)
          out, x += .                                          tg_matmul_device (quantises att)
    conv  LayerNorm(norm_conv)      -> quantised rows
          pw1 + GLU                 -> f32                     tg_matmul_quantized_glu_device
          depthwise conv + SiLU     -> quantised rows (each       tg_dwconv1d_quant_device
                                       utterance on its own)
          pw2, x += .                                          tg_matmul_quantized_device
    FF2   as FF1 with norm_ff2, ff2_in, ff2_out
    out   LayerNorm(norm_out), in place                        tg_layer_norm_device

In a stack (``run_stack``) a layer boundary is one call: the layer's norm_out in place and the next
layer's norm_ff1 quantised, tg_layer_norm_pair_quant_device (one launch below 2048 rows of up to
1024 values), and the next layer starts from those quantised rows (``prepared``).

Each step writes exactly the bits the unfused calls write (LayerNorm then quantise, product then
quantise), so the layer is the reference's sequence evaluated with the fast path's products: the
integer oracle composed in the same order reproduces it bit for bit. Q8_0 matrices take the same
entry points; for them the quantised-output product and the quantised GLU run the product into a
context buffer and then the quantiser or the GLU kernel (the same bits as the two calls).
Batches of equal-length utterances are stacked along the rows; only the depthwise convolution sees
the boundaries. The matrices must be int8 or Q8_0, the staged entry points' precisions; a layer
holding another precision raises ValueError before any launch."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, Optional

from .kernels import Act, Epilogue, Kernels, PackedWeights, Precision

# The layer's products (src/parakeet.rs:1011-1172): name -> (inputs, outputs) in units of d_model
# (ff_mult for the feed-forward hidden width); pos is the attention's position projection.
PRODUCTS = ("ff1_in", "ff1_out", "qkv", "pos", "out", "pw1", "pw2", "ff2_in", "ff2_out")
NORMS = ("norm_ff1", "norm_att", "norm_conv", "norm_ff2", "norm_out")


@dataclass
class LayerWeights:
    """A layer's matrices (int8 PackedWeights: ff1_in d -> ff, ff1_out ff -> d, qkv d -> 3d, out d -> d,
    pw1 d -> 2d, pw2 d -> d, ff2_in, ff2_out, optionally pos d -> d), its five LayerNorms as
    (gamma, beta) float32 GPU tensors of d values, and the depthwise convolution's taps
    [conv_kernel, d] and bias [d]."""
    mats: Dict[str, PackedWeights]
    norms: Dict[str, tuple]
    dw_w: object
    dw_b: object


class ConformerLayer:
    """Parakeet::layer on the device for up to `rows` frames of width d (ff hidden), on one context."""

    def __init__(self, kern: Kernels, d: int, ff: int, conv_kernel: int, rows: int, eps: float = 1e-5,
                 quantised_hidden: bool = True):
        import torch

        self.kern, self.d, self.ff, self.conv_kernel, self.rows, self.eps = kern, d, ff, conv_kernel, rows, eps
        # FF in writes its hidden rows quantised (tg_matmul_quantized_to_quant_device) when set (as
        # fast at 750 rows, 7% faster from 3000), else in f32 followed by the row quantiser: the same
        # bits either way.
        self.quantised_hidden = quantised_hidden
        dev = "cuda"
        u8 = lambda n: torch.empty(n, dtype=torch.uint8, device=dev)  # noqa: E731
        i32 = lambda n: torch.empty(n, dtype=torch.int32, device=dev)  # noqa: E731
        f32 = lambda *shape: torch.empty(shape, dtype=torch.float32, device=dev)  # noqa: E731
        self.qa_d, self.ex_d = u8(kern.quant_bytes(rows, d)), i32(rows)
        self.qa_ff, self.ex_ff = u8(kern.quant_bytes(rows, ff)), i32(rows)
        self.qkv = f32(rows, 3 * d)
        self.glu = f32(rows, d)
        self.conv = f32(rows, d)
        self._f32 = {}  # f32 rows of the unfused feed-forward, made on first use

    def _rows(self, name: str, width: int):
        import torch

        if name not in self._f32:
            self._f32[name] = torch.empty((self.rows, width), dtype=torch.float32, device="cuda")
        return self._f32[name]

    def prepare(self, x, t: int, w: LayerWeights) -> None:
        """The quantised rows of the layer's first LayerNorm (norm_ff1) of x, for forward(prepared=True)."""
        g, b = w.norms["norm_ff1"]
        self.kern.layer_norm_quant_device(x, self.d, t, self.d, g, b, self.eps, self.qa_d, self.ex_d)

    def run_stack(self, x, t: int, layers, utterances: int = 1, attention: Optional[Callable] = None) -> None:
        """The layers in turn on x (the reference's encode loop, src/parakeet.rs:893-894), each boundary
        between two layers as one call: norm_out of one and norm_ff1 of the next."""
        for i, w in enumerate(layers):
            nxt = layers[i + 1].norms["norm_ff1"] if i + 1 < len(layers) else None
            self.forward(x, t, w, utterances=utterances, attention=attention, prepared=i > 0, next_norm=nxt)

    def forward(self, x, t: int, w: LayerWeights, utterances: int = 1,
                attention: Optional[Callable] = None, pos=None, p_out=None, prepared: bool = False,
                next_norm: Optional[tuple] = None) -> None:
        """x: [t, d] float32 GPU tensor (the layer's input rows, updated in place); t frames in all,
        `utterances` equal-length utterances stacked along the rows. attention(qkv, p) -> att returns
        the heads' outputs [t, d] (rows at any stride, as a tensor view) from the f32 q, k, v rows and
        the projected positions; None uses the V third of qkv as the stand-in. pos ([2 t - 1, d] per
        utterance) and p_out receive the position projection when both are given.

        prepared: the quantised rows of norm_ff1(x) are already in the layer's buffers (prepare(), or
        the previous layer's boundary), so the first LayerNorm is not run again. next_norm: the next
        layer's norm_ff1 (gamma, beta); the last LayerNorm then also leaves that LayerNorm's quantised
        rows of the output for the next forward(prepared=True) on this object."""
        k, d, ff, eps = self.kern, self.d, self.ff, self.eps
        if t > self.rows or t % utterances:
            raise ValueError("t must fit the layer's rows and split into equal utterances")
        m = w.mats
        silu = Epilogue(act=Act.SILU)
        half_acc = Epilogue(scale=0.5, accumulate=True)
        acc = Epilogue(accumulate=True)

        for name, mat in m.items():
            if mat.precision() not in (Precision.INT8, Precision.Q8_0):
                raise ValueError(f"the device layer takes int8 or Q8_0 matrices ({name} is {mat.precision().name})")

        def feed_forward(norm, w_in, w_out, ready=False):
            g, b = w.norms[norm]
            if not ready:
                k.layer_norm_quant_device(x, d, t, d, g, b, eps, self.qa_d, self.ex_d)
            if self.quantised_hidden:
                k.matmul_quantized_to_quant_device(self.qa_d, self.ex_d, t, m[w_in], self.qa_ff, self.ex_ff, silu)
            else:  # the same bits through f32 rows and the row quantiser
                hid = self._rows("hid", ff)[:t]
                k.matmul_quantized_device(self.qa_d, self.ex_d, t, m[w_in], hid, ff, silu)
                k.quantize_rows_device(hid, ff, t, ff, self.qa_ff, self.ex_ff)
            k.matmul_quantized_device(self.qa_ff, self.ex_ff, t, m[w_out], x, d, half_acc)

        feed_forward("norm_ff1", "ff1_in", "ff1_out", ready=prepared)
        # self-attention: q, k, v in f32 for the attention core
        g, b = w.norms["norm_att"]
        k.layer_norm_quant_device(x, d, t, d, g, b, eps, self.qa_d, self.ex_d)
        qkv = self.qkv[:t]
        k.matmul_quantized_device(self.qa_d, self.ex_d, t, m["qkv"], qkv, 3 * d)
        if pos is not None and p_out is not None and "pos" in m:
            k.linear_device(pos, pos.shape[0], m["pos"], p_out)
        if attention is None:
            att, lda = qkv[:, 2 * d:], 3 * d
        else:
            att = attention(qkv, p_out)
            lda = att.stride(0)
        k.matmul_device(att, lda, t, m["out"], x, d, acc, a_len=(t - 1) * lda + d)
        # convolution module
        g, b = w.norms["norm_conv"]
        k.layer_norm_quant_device(x, d, t, d, g, b, eps, self.qa_d, self.ex_d)
        k.matmul_quantized_glu_device(self.qa_d, self.ex_d, t, m["pw1"], self.glu[:t], d)
        # the convolution writes its rows quantised for pw2 when the fused kernel takes the shape
        if k.dwconv1d_quant_device(
                self.glu, d, t // utterances, d, w.dw_w, self.conv_kernel, w.dw_b, self.qa_d, self.ex_d,
                act=Act.SILU, batch=utterances, x_len=t * d):
            k.matmul_quantized_device(self.qa_d, self.ex_d, t, m["pw2"], x, d, acc)
        else:
            k.dwconv1d_device(self.glu, d, t // utterances, d, w.dw_w, self.conv_kernel, w.dw_b, self.conv, d,
                              act=Act.SILU, batch=utterances, x_len=t * d, out_len=t * d)
            k.linear_device(self.conv[:t], t, m["pw2"], x, acc)
        feed_forward("norm_ff2", "ff2_in", "ff2_out")
        g, b = w.norms["norm_out"]
        if next_norm is None:
            k.layer_norm_device(x, d, t, d, g, b, eps, x, d)
        else:
            g2, b2 = next_norm
            k.layer_norm_pair_quant_device(x, d, t, d, g, b, eps, g2, b2, eps, self.qa_d, self.ex_d)
