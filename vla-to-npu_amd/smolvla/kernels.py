"""Per-kernel harness surface: the reference's AIE kernel names and argument
order, outputs written in place into caller-allocated tensors.

Each function replaces the ``ExternalModule(top=<name>)`` + ``df.build`` module
the reference's harness tests call (e.g. vla/tests/test_rms_norm_960_bf16.py:31-58)
and runs the corresponding gfx950 kernel through ``libsvla.so``.  Shapes are
whatever the caller passes (the reference's fixed tile shapes are the
common case).  Arguments are GPU tensors.
"""

from __future__ import annotations

import torch

from . import ops

BF16 = torch.bfloat16
F32 = torch.float32


def _into(dst, src):
    if dst.data_ptr() != src.data_ptr():
        dst.copy_(src)
    return dst


# ---- normalisation --------------------------------------------------------
def rms_norm_960_bf16(A, B, C):
    """cc/bf16/rms_norm_960_bf16.cc:60 (eps 1e-6, :16)."""
    ops.rmsnorm(A, B, 1e-6, out=C)


def rms_norm_bf16(A, B, C):
    """cc/bf16_old/rms_norm_bf16.cc:60 (eps 1e-5, :14)."""
    ops.rmsnorm(A, B, 1e-5, out=C)


def layer_norm_bf16(A, B, C, bias=None, eps=1e-5):
    """cc/bf16_old/layer_norm_bf16.cc:67 (gamma only; the reference adds the
    bias with a second kernel, vla/vision_block_bf16.py:120-127 -- here it is
    the optional ``bias``)."""
    ops.layernorm(A, B, bias, eps, out=C)


# ---- activations ----------------------------------------------------------
def silu_160_bf16(A, C):
    """cc/bf16/silu_160_bf16.cc:124."""
    ops.silu(A, out=C)


def silu_256_bf16(A, C):
    """cc/bf16/silu_256_bf16.cc:114."""
    ops.silu(A, out=C)


def silu_128_bf16(A, C):
    """cc/bf16/silu_128_bf16.cc:107 (the reference pads 128 -> 256 columns)."""
    ops.silu(A, out=C)


def silu_bf16(A, C):
    """cc/bf16_old/silu_bf16.cc:192."""
    ops.silu(A, out=C)


def gelu_bf16(A, C, kind="tanh"):
    """cc/bf16_old/gelu_bf16.cc:83 (tanh-GELU)."""
    ops.gelu(A, kind=kind, out=C)


# ---- softmax ----------------------------------------------------------------
def masked_softmax_128_bf16(scores, row_start, weights):
    """cc/bf16/masked_softmax_128_bf16.cc:251; ``row_start`` an int or a
    1-element int32 tensor (host or device), as the reference passes
    ``np.array([row_start], dtype=np.int32)``."""
    rs = int(row_start.reshape(-1)[0].item()) if torch.is_tensor(row_start) else int(
        row_start[0] if hasattr(row_start, "__len__") else row_start)
    ops.masked_softmax(scores, rs, out=weights)


def softmax_bf16(scores, weights):
    """softmax_bf16_{4_768,4_1024,8_512,16_256,32_128,64_64}
    (cc/bf16_old/v2_softmax_bf16.cc:552-663)."""
    ops.softmax(scores, out=weights)


def softmax_bf16_seq1024(scores, weights):
    """cc/bf16_old/v1_softmax_bf16.cc:159: [4, 512] storage = 2 rows of 1024."""
    rows = scores.numel() // 1024
    ops.softmax(scores.reshape(rows, 1024), out=weights.view(rows, 1024))


def softmax_float32_seq1024(scores, weights):
    """cc/float/v1_softmax_float.cc:117 (fp32 in / fp32 out, rows of 1024)."""
    rows = scores.numel() // 1024
    ops.softmax(scores.reshape(rows, 1024), out=weights.view(rows, 1024))


# ---- products ---------------------------------------------------------------
def transpose_matmul_with_scale_bf16(A, B, C, scale=0.125):
    """C = scale * A . B^T (cc/bf16_old/transpose_matmul_with_scale_bf16.cc:52).
    ``B`` is already in the packed [N, K] form the GEMM consumes."""
    ops.linear(A, B, alpha=scale, out=C)


def gemm(A, B, C):
    """Tiled GEMM C = A . B with B ``[K, N]`` (the Allo GEMM module contract,
    cc/gemm.py:44-77; gemm/v1_test_tiled_gemm.py)."""
    ops.linear(A, ops.pack_weight(B), out=C)


# ---- RoPE -------------------------------------------------------------------
def rope_fused_float32(x, sin_cos, out):
    """cc/float/rope_fused.cc:17: one head tile; ``sin_cos[r] = [sin | cos]``."""
    half = x.shape[1] // 2
    s = sin_cos[:, :half].contiguous()
    c = sin_cos[:, half:].contiguous()
    ops.rope(x, 1, c, s, pos_offset=0, out=out)


# ---- fp32 and "new" bf16 variants -----------------------------------------
def _same(A, C):
    if C.dtype != A.dtype or C.shape != A.shape:
        raise ValueError("output must match the input's shape and dtype")


def add(x, y, out):
    """cc/bf16_old/add_32_32_bf16.cc (add/test_add.py: out = x + y, bf16)."""
    ops.add(x, y, out=out)


def silu_float32(A, C):
    """cc/float/silu.cc (silu/test_silu.py: nn.SiLU in fp32)."""
    _same(A, C)
    ops.unary(A, "silu", out=C)


silu_128_float32 = silu_float32  # cc/float/silu_128.cc (vla/tests/test_silu_128.py)
silu_160_float32 = silu_float32  # cc/float/silu_160.cc (vla/tests/test_silu_160.py)


def silu_bf16_small(A, C):
    """cc/bf16_new/silu_bf16.cc small-tile entry (silu/test_silu_bf16_new.py:159-225)."""
    _same(A, C)
    ops.unary(A, "silu", out=C)


def gelu(A, C):
    """``gelu`` of cc/float/gelu.cc (fp32) and cc/bf16_new/gelu_bf16.cc (bf16):
    nn.GELU() -- the exact erf form -- as gelu/test_gelu.py and
    gelu/test_gelu_bf16_new.py compare against."""
    _same(A, C)
    ops.unary(A, "gelu_erf", out=C)


gelu_small = gelu  # cc/bf16_new/gelu_bf16.cc small-tile entry (gelu/test_gelu_bf16_new.py:210)


def sin_float32(A, C):
    """cc/float/sine.cc:64 (sine/test_sine.py)."""
    _same(A, C)
    ops.unary(A, "sin", out=C)


def cos_float32(A, C):
    """cc/float/cosine.cc:66 (cosine/test_cosine.py)."""
    _same(A, C)
    ops.unary(A, "cos", out=C)


sin_bfloat16 = sin_float32  # cc/bf16_new/sine_bf16.cc (sine/test_sine_bf16_new.py); dtype follows A
cos_bfloat16 = cos_float32  # cc/bf16_new/cosine_bf16.cc (cosine/test_cosine_bf16.py)


def rms_norm(A, B, C, eps=1e-6):
    """``rms_norm`` of cc/float/rms_norm.cc and cc/bf16_new/rms_norm_bf16.cc:
    the harness module y = x / (||x|| / sqrt(N) + eps) * w
    (rms_norm/test_rms.py:25-33); bf16 rounds after every op like the torch
    bf16 reference of rms_norm/test_rms_norm_bf16_new.py."""
    ops.row_norm(A, B, eps, "rms_add", round_ops=A.dtype == BF16, out=C)


rms_norm_small = rms_norm  # cc/bf16_new/rms_norm_bf16.cc small-tile entry


def rms_norm_960(A, B, C, eps=1e-6):
    """cc/float/rms_norm_960.cc (vla/tests/test_rms_norm_960.py): fp32, the
    harness module y = x / (||x|| / sqrt(N) + eps) * w it is checked against
    (:18-26)."""
    ops.row_norm(A, B, eps, "rms_add", out=C)


def layer_norm(A, B, C, bias=None, eps=1e-5):
    """``layer_norm`` of cc/float/layer_norm.cc (gamma; the fp32 test adds the
    beta separately, layer_norm/test_layer.py:56-80 -- here the optional
    ``bias``) and cc/bf16_new/layer_norm_bf16.cc (gamma only, torch bf16 op
    chain of layer_norm/test_layer_bf16_new.py:25-34)."""
    ops.row_norm(A, B, eps, "layer", b=bias, round_ops=A.dtype == BF16, out=C)


layer_norm_small = layer_norm  # cc/bf16_new/layer_norm_bf16.cc small-tile entry


def masked_softmax_float32(scores, tile_row_start, weights, heads=1):
    """cc/float/masked_softmax.cc:72-127: rows of ``heads`` consecutive
    segments of keys (masked_softmax/test_masked_softmax.py: [64, 3 * 64]),
    key c of row r masked when c > row_start + r."""
    rs = int(tile_row_start.reshape(-1)[0].item()) if torch.is_tensor(tile_row_start) else int(
        tile_row_start[0] if hasattr(tile_row_start, "__len__") else tile_row_start)
    rows = scores.shape[0] * heads
    cols = scores.numel() // rows
    ops.softmax_rows(scores.reshape(rows, cols), rs, heads, out=weights.view(rows, cols))


def masked_softmax_128_float32(scores, row_start, weights):
    """cc/float/masked_softmax_128.cc (vla/tests/test_masked_softmax_128.py)."""
    masked_softmax_float32(scores, row_start, weights, heads=1)


def conv(images, kernel, out, bias=None):
    """cc/float/conv.cc:12-55: fp32 patch convolution (kernel = stride = patch),
    out [patches, E] (conv/test_conv.py)."""
    ops.conv_patch_f32(images.reshape(-1, *images.shape[-3:]) if images.dim() == 4
                       else images.unsqueeze(0), kernel, bias, out=out)
