"""Granite Speech's encoder block and self-conditioning on the device, in the reference's order.

``GraniteBlock.forward`` runs ``Granite::block_span`` (src/granite.rs:800-952) over whole utterances,
as ``Granite::encode`` calls it (src/granite.rs:628-650: start 0, out_start 0, no left context), on
rows resident in GPU memory, every int8 product on the library's fast path:

    FF1   LayerNorm(ff1.norm)      -> quantised rows          tg_layer_norm_quant_device
          ff1.up + bias, SiLU      -> quantised hidden rows   tg_matmul_quantized_to_quant_device
          ff1.down + bias, x += 0.5 * .                       tg_matmul_quantized_device
    att   LayerNorm(norm_att)      -> quantised rows
          qkv (no bias)            -> f32 q, k, v (the attention core reads them)
          attention(q, k, v) -> att  (the caller's; outside this path: the V third stands in)
          out + bias, x += .                                  tg_matmul_device (quantises att)
    conv  LayerNorm(norm_conv)     -> quantised rows of the t input frames
          pw1 + bias, GLU          -> f32 [t, conv_channels]  tg_matmul_quantized_glu_device
          depthwise conv + SiLU    -> quantised rows          stride 1: tg_dwconv1d_quant_device;
                                                              stride 2 (frames 0, 2, 4, ...):
                                                              tg_dwconv1d_device, then
                                                              tg_quantize_rows_device
          pool                     out = x (stride 1), or (x[2r] + x[2r + 1]) / 2
                                                              tg_average_pairs_device
          pw2 + bias, out += .                                tg_matmul_quantized_device
    FF2   as FF1, on the n output rows
    out   LayerNorm(norm_out), in place

A strided block (Granite's subsample_layers, blocks 0 and 1) leaves t // 2 rows per utterance, a last
odd frame dropped. ``self_conditioning`` is ``Granite::self_conditioning`` (src/granite.rs:1040-1069)
with its injection added to the rows (src/granite.rs:639-647): x += mid(softmax(head(x) + head.b)) +
mid.b. The reference computes the injection into a buffer and then adds it; the product's
accumulating epilogue adds the same value (scale 1 is exact), so the bits are the same.

Each step writes what its unfused calls write (LayerNorm then quantise, product then quantise), so the
block is the reference's sequence evaluated with the fast path's products: the integer oracle composed
in the same order reproduces it bit for bit. Batches of equal-length utterances are stacked along the
rows; only the depthwise convolution and the pooling see the boundaries. The matrices must be int8
or Q8_0; a block holding another precision raises ValueError before any launch."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, Optional

from .kernels import Act, Epilogue, Kernels, PackedWeights, Precision

# The block's products (src/granite.rs:191-212, 455-487): name -> (outputs, inputs) in terms of
# d_model d, the feed-forward width ff and the convolution channels cc. Every one but qkv has a bias.
PRODUCTS = {"ff1_up": ("ff", "d"), "ff1_down": ("d", "ff"), "qkv": ("3d", "d"), "out": ("d", "d"),
            "pw1": ("2cc", "d"), "pw2": ("d", "cc"), "ff2_up": ("ff", "d"), "ff2_down": ("d", "ff")}
NORMS = ("ff1_norm", "norm_att", "norm_conv", "ff2_norm", "norm_out")


@dataclass
class BlockWeights:
    """A block's matrices (PackedWeights named as PRODUCTS), their biases (float32 GPU tensors, by
    the same names; qkv has none), its five LayerNorms as (gamma, beta) GPU tensors of d values, the
    depthwise taps [conv_kernel, cc] and bias [cc], and whether the block is strided."""
    mats: Dict[str, PackedWeights]
    biases: Dict[str, object]
    norms: Dict[str, tuple]
    dw_w: object
    dw_b: object
    strided: bool


class GraniteBlock:
    """Granite::block_span on the device for up to `rows` input frames of width d, on one context."""

    def __init__(self, kern: Kernels, d: int, ff: int, conv_channels: int, conv_kernel: int, rows: int,
                 eps: float = 1e-5):
        import torch

        self.kern, self.d, self.ff, self.cc, self.conv_kernel, self.rows, self.eps = \
            kern, d, ff, conv_channels, conv_kernel, rows, eps
        dev = "cuda"
        u8 = lambda n: torch.empty(n, dtype=torch.uint8, device=dev)  # noqa: E731
        i32 = lambda n: torch.empty(n, dtype=torch.int32, device=dev)  # noqa: E731
        f32 = lambda *shape: torch.empty(shape, dtype=torch.float32, device=dev)  # noqa: E731
        self.qa_d, self.ex_d = u8(kern.quant_bytes(rows, d)), i32(rows)
        self.qa_ff, self.ex_ff = u8(kern.quant_bytes(rows, ff)), i32(rows)
        self.qa_cc, self.ex_cc = u8(kern.quant_bytes(rows, conv_channels)), i32(rows)
        self.qkv = f32(rows, 3 * d)
        self.glu = f32(rows, conv_channels)
        self.conv = f32(rows, conv_channels)

    def prepare(self, x, t: int, w: BlockWeights) -> None:
        """The digits of ff1's LayerNorm of x's t rows in the block's buffers: what forward(...,
        prepared=True) expects, as the previous block's forward(..., next_norm=...) leaves them."""
        g, b = w.norms["ff1_norm"]
        self.kern.layer_norm_quant_device(x, self.d, t, self.d, g, b, self.eps, self.qa_d, self.ex_d)

    def _feed_forward(self, x, t: int, w: BlockWeights, which: str, ready: bool = False) -> None:
        """x += 0.5 * (down(silu(up(norm(x)) + up.b)) + down.b) (src/granite.rs:752-793). ready: the
        digits of norm(x) are already in the block's buffers."""
        k, d = self.kern, self.d
        g, b = w.norms[which + "_norm"]
        up, down = w.mats[which + "_up"], w.mats[which + "_down"]
        if not ready:
            k.layer_norm_quant_device(x, d, t, d, g, b, self.eps, self.qa_d, self.ex_d)
        silu = Epilogue(bias=w.biases[which + "_up"], act=Act.SILU)
        half_acc = Epilogue(bias=w.biases[which + "_down"], scale=0.5, accumulate=True)
        k.matmul_quantized_to_quant_device(self.qa_d, self.ex_d, t, up, self.qa_ff, self.ex_ff, silu)
        k.matmul_quantized_device(self.qa_ff, self.ex_ff, t, down, x, d, half_acc)

    def forward(self, x, t: int, w: BlockWeights, utterances: int = 1, attention: Optional[Callable] = None,
                out=None, prepared: bool = False, next_norm=None):
        """x: [t, d] float32 GPU tensor, the block's input rows (rewritten: afterwards it holds the
        post-attention states, as the reference leaves it); t frames in all, `utterances` equal-length
        utterances stacked along the rows. attention(qkv) -> att returns the heads' outputs [t, d]
        (rows at any stride, as a tensor view) from the f32 q, k, v rows; None uses the V third of qkv.
        Returns (y, n): the block's output rows and their count, n = t (y is x) or, for a strided
        block, utterances * (t / utterances // 2) rows written to `out` ([n, d] float32 GPU tensor,
        allocated when None). prepared: the digits of ff1's LayerNorm of x are already in the block's
        buffers (prepare, or the previous block's next_norm). next_norm = (gamma, beta): the next
        block's ff1 LayerNorm, whose digits of the output rows are left in the buffers for it, the
        block boundary in one launch (tg_layer_norm_pair_quant_device): the same bits as
        prepare on the output."""
        import torch

        k, d, cc, eps = self.kern, self.d, self.cc, self.eps
        if t > self.rows or t % utterances:
            raise ValueError("t must fit the block's rows and split into equal utterances")
        frames = t // utterances
        m = w.mats
        for name, mat in m.items():
            if mat.precision() not in (Precision.INT8, Precision.Q8_0):
                raise ValueError(f"the device block takes int8 or Q8_0 matrices ({name} is {mat.precision().name})")
        self._feed_forward(x, t, w, "ff1", ready=prepared)
        g, b = w.norms["norm_att"]
        k.layer_norm_quant_device(x, d, t, d, g, b, eps, self.qa_d, self.ex_d)
        qkv = self.qkv[:t]
        k.matmul_quantized_device(self.qa_d, self.ex_d, t, m["qkv"], qkv, 3 * d)
        if attention is None:
            att, lda = qkv[:, 2 * d:], 3 * d
        else:
            att = attention(qkv)
            lda = att.stride(0)
        k.matmul_device(att, lda, t, m["out"], x, d, Epilogue(bias=w.biases["out"], accumulate=True),
                        a_len=(t - 1) * lda + d)
        # convolution module over the post-attention states of all t frames
        g, b = w.norms["norm_conv"]
        k.layer_norm_quant_device(x, d, t, d, g, b, eps, self.qa_d, self.ex_d)
        k.matmul_quantized_glu_device(self.qa_d, self.ex_d, t, m["pw1"], self.glu[:t], cc,
                                      epi=Epilogue(bias=w.biases["pw1"]))
        if w.strided:
            rows = frames // 2
            n = rows * utterances
            k.dwconv1d_device(self.glu, cc, frames, cc, w.dw_w, self.conv_kernel, w.dw_b, self.conv, cc,
                              rows=rows, t0=0, stride=2, act=Act.SILU, batch=utterances, x_len=t * cc,
                              out_len=max(n, 1) * cc)
            if out is None:
                out = torch.empty((max(n, 1), d), dtype=torch.float32, device="cuda")
            k.average_pairs_device(x, d, frames, d, out, d, batch=utterances, x_len=t * d)
            y = out
            if n == 0:
                return y, 0
            k.quantize_rows_device(self.conv, cc, n, cc, self.qa_cc, self.ex_cc, a_len=n * cc)
        else:
            n, y = t, x
            if not k.dwconv1d_quant_device(self.glu, cc, frames, cc, w.dw_w, self.conv_kernel, w.dw_b,
                                           self.qa_cc, self.ex_cc, act=Act.SILU, batch=utterances,
                                           x_len=t * cc):
                k.dwconv1d_device(self.glu, cc, frames, cc, w.dw_w, self.conv_kernel, w.dw_b, self.conv, cc,
                                  act=Act.SILU, batch=utterances, x_len=t * cc, out_len=t * cc)
                k.quantize_rows_device(self.conv, cc, t, cc, self.qa_cc, self.ex_cc, a_len=t * cc)
        k.matmul_quantized_device(self.qa_cc, self.ex_cc, n, m["pw2"], y, d,
                                  Epilogue(bias=w.biases["pw2"], accumulate=True))
        self._feed_forward(y, n, w, "ff2")
        g, b = w.norms["norm_out"]
        if next_norm is None:
            k.layer_norm_device(y, d, n, d, g, b, eps, y, d)
        else:
            k.layer_norm_pair_quant_device(y, d, n, d, g, b, eps, next_norm[0], next_norm[1], eps, self.qa_d,
                                           self.ex_d, x_len=n * d)
        return y, n


def self_conditioning(kern: Kernels, x, t: int, head: PackedWeights, head_b, mid: PackedWeights, mid_b,
                      logits) -> None:
    """x[:t] += mid(softmax(head(x) + head.b)) + mid.b on the device (src/granite.rs:1040-1069 and the
    injection of src/granite.rs:639-647). logits: a float32 GPU tensor of at least t * vocab values,
    the CTC logits' rows (left holding the posteriors)."""
    vocab = head.n()
    kern.linear_device(x, t, head, logits, Epilogue(bias=head_b))
    kern.softmax_device(logits, vocab, t, vocab, x_len=t * vocab)
    kern.matmul_device(logits, vocab, t, mid, x, mid.n(), Epilogue(bias=mid_b, accumulate=True),
                       a_len=t * vocab)
