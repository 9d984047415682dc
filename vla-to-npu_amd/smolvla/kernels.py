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
