"""GPU transformer layers built from the C-ABI kernels.

Weights are prepared once into the packed layouts the kernels consume
(``prep_*``), then each layer is a short, fixed sequence of launches on the
current stream, writing into caller-provided buffers so a whole chunk can be
captured in one HIP graph.  Activations are row-major ``[B*S, H]`` bf16.

Per decoder layer (vla/text_encoder_bf16.py:480-595 -> 7 launches):
  RMSNorm -> [QKV GEMM -> RoPE] -> fused GQA attention -> [O GEMM + residual]
  -> RMSNorm -> [gate|up GEMM -> SiLU*up] -> [down GEMM + residual]
(brackets = one kernel).  Each RMSNorm rounds once, bf16((x * (1/rms)) *
gain), as torch's bf16 RMSNorm does.  It runs as its own bandwidth kernel
into a buffer.  The GEMMs can also take it in their A path (``norm=``: each
workgroup forms its rows' 1/rms first, then rounds every operand element the
same way, bit-identical operands), but that extra pass over a tile's A rows
costs more than the standalone kernel on every engine shape measured on
MI355X (batch-32 chunk 41.3 ms with standalone norms, 42.4 ms fused; batch-1
chunk 8.13 vs 8.15 ms), so FUSED_NORM_MAX_ROWS keeps it off.  RoPE'd Q and K
also carry their bf16 remainders into the attention, which then scores the
fp32 values as the reference module does.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import ops
from .config import DecoderConfig, VitConfig, resolve_eps

BF16 = torch.bfloat16


# ------------------------------------------------------------ weight prep ---
def is_bf16_bits(a):
    """A numpy array holding bfloat16 values as 2-byte words: the reference's
    ``ml_dtypes.bfloat16`` arrays (``NP_DTYPE``, vla/text_encoder_bf16.py:55),
    or raw ``uint16`` bit patterns of a caller without ml_dtypes."""
    return a.dtype.itemsize == 2 and (a.dtype.name == "bfloat16" or a.dtype == np.uint16)


def host_tensor(a):
    """A torch tensor as is; a numpy array (how the reference builds ``params``
    and its inputs, vla/text_encoder_bf16.py:599-609) as a CPU torch tensor:
    floating arrays keep their values, bfloat16 words (:func:`is_bf16_bits`)
    are reinterpreted bit for bit, integer ids stay integers."""
    if torch.is_tensor(a):
        return a
    a = np.asarray(a)
    if is_bf16_bits(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(BF16)
    if a.dtype.kind not in "fiub":
        raise TypeError(f"unsupported array dtype {a.dtype}")
    return torch.from_numpy(np.ascontiguousarray(a))


def _dev(t, device):
    """A weight (torch tensor or numpy array) as a contiguous bf16 tensor on
    ``device``."""
    return host_tensor(t).to(device=device, dtype=BF16).contiguous()


def _pack_cols(ws, device):
    """Pack ``[K, N_i]`` reference weights side by side into one ``[sum N_i, K]``."""
    K = ws[0].shape[0]
    out = torch.empty(sum(w.shape[1] for w in ws), K, dtype=BF16, device=device)
    r = 0
    for w in ws:
        ops.pack_weight(_dev(w, device), out=out[r:r + w.shape[1]])
        r += w.shape[1]
    return out


def prep_decoder(p, device):
    """SmolLM2 decoder / expert self layer: fused QKV [q|k|v, H], O, gate|up, down."""
    return dict(
        wqkv=_pack_cols([p["Wq"], p["Wk"], p["Wv"]], device),
        wo=ops.pack_weight(_dev(p["Wo"], device)),
        wgu=ops.pack_gate_up(_dev(p["W_gate"], device), _dev(p["W_up"], device)),
        wd=ops.pack_weight(_dev(p["W_down"], device)),
        n1=_dev(p["W_norm_1"], device), n2=_dev(p["W_norm_2"], device),
    )


def prep_cross(p, device):
    """Expert cross layer: Q, the cross K/V projections, O, gate|up, down.
    ``wkvc`` packs both cross projections block-diagonally ([K | V] of the
    prefix cache -> [K' | V'] in one GEMM; the zero blocks add exact zeros, so
    the products equal the two separate GEMMs')."""
    wk, wv = _dev(p["Wk_cross"], device), _dev(p["Wv_cross"], device)
    kin, kout = wk.shape
    vin, vout = wv.shape
    wbd = torch.zeros(kin + vin, kout + vout, dtype=wk.dtype, device=wk.device)
    wbd[:kin, :kout] = wk
    wbd[kin:, kout:] = wv
    return dict(
        wq=ops.pack_weight(_dev(p["Wq"], device)),
        wkc=ops.pack_weight(wk),
        wvc=ops.pack_weight(wv),
        wkvc=ops.pack_weight(wbd.contiguous()),
        wo=ops.pack_weight(_dev(p["Wo"], device)),
        wgu=ops.pack_gate_up(_dev(p["W_gate"], device), _dev(p["W_up"], device)),
        wd=ops.pack_weight(_dev(p["W_down"], device)),
        n1=_dev(p["W_norm_1"], device), n2=_dev(p["W_norm_2"], device),
    )


def prep_vit(p, device, rows=None):
    """Packed ViT block weights.  ``rows`` (the engine's row count, images x
    tokens): also slab-blocked copies of the weights that
    :func:`vit_blocked_plan` puts on the 256x256 GEMM at that row count."""
    H = p["Wq"].shape[0]
    bqkv = None
    if p.get("bq") is not None:
        bqkv = torch.empty(3 * H, dtype=BF16, device=device)
        for i, k in enumerate(("bq", "bk", "bv")):
            bqkv[i * H:(i + 1) * H].copy_(_dev(p[k], device))
    opt = lambda k: _dev(p[k], device) if p.get(k) is not None else None  # noqa: E731
    P = dict(
        wqkv=_pack_cols([p["Wq"], p["Wk"], p["Wv"]], device), bqkv=bqkv,
        wo=ops.pack_weight(_dev(p["Wo"], device)), bo=opt("bo"),
        wup=ops.pack_weight(_dev(p["W_up"], device)), bup=opt("b_up"),
        wd=ops.pack_weight(_dev(p["W_down"], device)), bd=opt("b_down"),
        g1=_dev(p["W_norm_1"], device), b1=opt("b_norm_1"),
        g2=_dev(p["W_norm_2"], device), b2=opt("b_norm_2"),
    )
    if rows:
        plan = vit_blocked_plan(H, P["wup"].shape[0], rows)
        for k, w in VIT_PROJ.items():
            if plan[k]:
                P[w + "_blk"] = ops.slab_block(P[w])
    return P


VIT_PROJ = {"qkv": "wqkv", "o": "wo", "up": "wup", "down": "wd"}

# The 256x256 GEMM on slab-blocked operands beats the automatic tile choice on
# row-major operands once a projection has at least this many 256x256 output
# tiles (MI355X, the SigLIP shapes at 1-10 images of 3 cameras: QKV wins from
# 216 tiles and loses at 108, O and down win from 144 and lose at 108, the
# up-projection wins from 144).
WIDE_MIN_TILES = 144


def vit_blocked_plan(hidden: int, inter: int, rows: int) -> dict:
    """Which ViT projections run on the 256x256 GEMM with slab-blocked
    weights at ``rows`` rows: those whose shape the kernel takes and that
    have at least ``WIDE_MIN_TILES`` output tiles.  QKV and the
    up-projection then read a slab-blocked LayerNorm output; the
    down-projection reads the up-projection's output slab-blocked, so it goes
    blocked only together with the up-projection; O reads the attention
    output row-major.  A projection the plan moves gives the same bits on
    either path (measured at 3 and 12 images: the automatic tiles it replaces
    accumulate K in the same order); only the 96x96 tile the batch-1
    down-projection keeps sums in another order, which the plan never
    replaces."""
    shapes = {"qkv": (3 * hidden, hidden), "o": (hidden, hidden),
              "up": (inter, hidden), "down": (hidden, inter)}
    plan = {name: (rows % 256 == 0 and n % 256 == 0 and k % 128 == 0 and k >= 256 and
                   (rows // 256) * (n // 256) >= WIDE_MIN_TILES)
            for name, (n, k) in shapes.items()}
    plan["down"] = plan["down"] and plan["up"]
    return plan


@dataclass
class Rope:
    cos: torch.Tensor
    sin: torch.Tensor
    seq_len: int

    @classmethod
    def make(cls, seq_len, head_dim, theta, device):
        c, s = ops.rope_table(seq_len, head_dim, theta, device=device)
        return cls(c, s, seq_len)


class Buffers:
    """Lazily allocated, reusable activation buffers keyed by name."""

    def __init__(self, device):
        self.device = device
        self._b = {}

    def get(self, name, rows, cols, dtype=BF16):
        t = self._b.get(name)
        if t is None or t.shape[0] < rows or t.shape[1] != cols or t.dtype != dtype:
            t = torch.empty(rows, cols, dtype=dtype, device=self.device)
            self._b[name] = t
        return t[:rows]


# ----------------------------------------------------------------- layers ---
# fuse the RMSNorm into the consuming GEMM up to this many rows (the same
# rounding either way; 0: never, the faster choice measured, see above)
FUSED_NORM_MAX_ROWS = 0


def _normed(x, w, eps, M, bufs, name):
    """(A operand, norm argument) for a GEMM that consumes RMSNorm(x): fused
    into the GEMM up to FUSED_NORM_MAX_ROWS rows, else a standalone RMSNorm
    into a buffer."""
    if M <= FUSED_NORM_MAX_ROWS:
        return x, (w, eps)
    return ops.rmsnorm(x, w, eps, out=bufs.get(name, M, x.shape[1])), None


def decoder_layer(x, P, cfg: DecoderConfig, B, L, rope: Rope, mask="causal", prefix_len=0,
                  bufs: Optional[Buffers] = None, qkv_out=None, mid_out=None):
    """One SmolLM2-style block on ``x [B*L, H]`` **in place**; returns the
    fused projection buffer ``[B*L, q|k|v]`` whose K (post-RoPE) and V column
    slices are this layer's KV cache (vla/text_encoder_bf16.py:480-595).
    ``mid_out`` (optional) receives the mid-block residual (after attention)."""
    bufs = bufs or Buffers(x.device)
    M = B * L
    qd, kvd = cfg.q_dim, cfg.kv_dim
    eps = resolve_eps(cfg.rms_eps)
    qkv = qkv_out if qkv_out is not None else bufs.get("qkv", M, qd + 2 * kvd)
    # remainders of the fp32 post-RoPE Q and K, which the reference module
    # scores in fp32 (vla/text_encoder_bf16.py:92-104, 117-122); the cache
    # keeps the bf16 values (:595)
    lo = bufs.get("qkv_lo", M, qkv.stride(0))[:, :qd + 2 * kvd]
    a, nrm = _normed(x, P["n1"], eps, M, bufs, "xn")
    ops.linear_rope(a, P["wqkv"], qd + kvd, L, rope.cos, rope.sin, out=qkv, norm=nrm, out_lo=lo)
    q3, l3 = qkv.view(B, L, -1), lo.view(B, L, -1)
    attn = bufs.get("attn", M, qd)
    ops.attention(q3[:, :, :qd], q3[:, :, qd:qd + kvd], q3[:, :, qd + kvd:],
                  attn.view(B, L, qd), cfg.n_q_heads, cfg.n_kv_heads, mask, prefix_len,
                  q_lo=l3[:, :, :qd], k_lo=l3[:, :, qd:qd + kvd])
    ops.linear(attn, P["wo"], res=x, out=x)
    if mid_out is not None:
        mid_out.copy_(x)
    _mlp(x, P, cfg, M, eps, bufs)
    return qkv


def _mlp(x, P, cfg, M, eps, bufs):
    a, nrm = _normed(x, P["n2"], eps, M, bufs, "xn")
    act = ops.linear_silu_mul(a, P["wgu"], out=bufs.get("mlp", M, cfg.inter), norm=nrm)
    ops.linear(act, P["wd"], res=x, out=x)


def _adjacent(a, b):
    """``b`` starts right after ``a``'s columns in the same rows (two column
    slices of one row-major buffer)."""
    return (a.dim() == 2 and b.dim() == 2 and a.shape[0] == b.shape[0] and a.stride(1) == 1
            and b.stride(1) == 1 and a.stride(0) == b.stride(0)
            and b.data_ptr() == a.data_ptr() + a.shape[1] * a.element_size())


def cross_kv(k_src, v_src, P, out_k=None, out_v=None):
    """Cross-attention K/V projections of the prefix cache
    (vla/action_expert_bf16.py:757-758).  When K and V are adjacent column
    slices of one buffer (the prefix KV cache rows [.. | K | V]), so are the
    outputs, and the rows are few enough for the launch to dominate (up to
    2048; measured on MI355X: 241 rows 7.6 -> 4.3 us for both, 7712 rows
    15.1 -> 16.7 us, the zero blocks doubling the MFMA work), both projections
    run as one GEMM on the block-diagonal weight."""
    if ("wkvc" in P and out_k is not None and out_v is not None and k_src.shape[0] <= 2048
            and _adjacent(k_src, v_src) and _adjacent(out_k, out_v)):
        M, ld = k_src.shape[0], k_src.stride(0)
        a = torch.as_strided(k_src, (M, k_src.shape[1] + v_src.shape[1]), (ld, 1))
        c = torch.as_strided(out_k, (M, out_k.shape[1] + out_v.shape[1]), (out_k.stride(0), 1))
        ops.linear(a, P["wkvc"], out=c)
        return out_k, out_v
    k = ops.linear(k_src, P["wkc"], out=out_k)
    v = ops.linear(v_src, P["wvc"], out=out_v)
    return k, v


def cross_layer(x, ck, cv, P, cfg: DecoderConfig, B, L, Lc, rope: Rope,
                bufs: Optional[Buffers] = None):
    """Expert cross-attention block on ``x [B*L, H]`` in place, attending to
    the already projected ``ck``/``cv [B*Lc, kv]`` (vla/action_expert_bf16.py:731-803;
    RoPE on Q only, no mask)."""
    bufs = bufs or Buffers(x.device)
    M = B * L
    qd = cfg.q_dim
    eps = resolve_eps(cfg.rms_eps)
    a, nrm = _normed(x, P["n1"], eps, M, bufs, "xn")
    q_lo = bufs.get("q_lo", M, qd)
    q = ops.linear_rope(a, P["wq"], qd, L, rope.cos, rope.sin, out=bufs.get("q", M, qd),
                        norm=nrm, out_lo=q_lo)
    attn = bufs.get("attn", M, qd)
    ops.attention(q.view(B, L, qd), ck.view(B, Lc, -1), cv.view(B, Lc, -1), attn.view(B, L, qd),
                  cfg.n_q_heads, cfg.n_kv_heads, "none", 0, q_lo=q_lo.view(B, L, qd))
    ops.linear(attn, P["wo"], res=x, out=x)
    _mlp(x, P, cfg, M, eps, bufs)


def vit_layer(x, P, cfg: VitConfig, n_img, T, bufs: Optional[Buffers] = None, plan=None):
    """SigLIP-style block on ``x [n_img*T, H]`` in place
    (vla/vision_block_bf16.py:308-420).  Each projection that ``plan``
    (default: :func:`vit_blocked_plan` at these rows) marks and whose
    slab-blocked weight ``P`` holds runs on the 256x256 GEMM, and the
    LayerNorm output (or MLP activation) it reads is written slab-blocked, so
    its K loop streams both operands as contiguous kilobytes; the others run
    on the automatic tile choice.  The residual stream stays row-major."""
    from .ops import LAYOUT_A_BLOCKED as AB, LAYOUT_W_BLOCKED as WB, LAYOUT_C_BLOCKED as CB
    bufs = bufs or Buffers(x.device)
    M, H, I = n_img * T, cfg.hidden, cfg.inter
    plan = plan or vit_blocked_plan(H, I, M)
    blk = {k: bool(plan[k]) and w + "_blk" in P for k, w in VIT_PROJ.items()}
    blk["down"] = blk["down"] and blk["up"]

    def norm(g, b, blocked):
        out = bufs.get("vh", M, H)
        if blocked:
            return ops.layernorm(x, g, b, cfg.ln_eps, out=out.view(H // 32, M, 32), blocked=True)
        return ops.layernorm(x, g, b, cfg.ln_eps, out=out)

    h = norm(P["g1"], P["b1"], blk["qkv"])
    qkv = bufs.get("vqkv", M, 3 * H)
    if blk["qkv"]:
        ops.linear_wide(h, P["wqkv_blk"], M, 3 * H, H, bias=P["bqkv"], out=qkv, layout=AB | WB)
    else:
        ops.linear(h, P["wqkv"], bias=P["bqkv"], out=qkv)
    q3 = qkv.view(n_img, T, 3 * H)
    attn = bufs.get("vattn", M, H)
    ops.attention(q3[:, :, :H], q3[:, :, H:2 * H], q3[:, :, 2 * H:], attn.view(n_img, T, H),
                  cfg.n_heads, cfg.n_heads, "none", 0, scale=1.0 / math.sqrt(cfg.head_dim))
    if blk["o"]:
        ops.linear_wide(attn, P["wo_blk"], M, H, H, bias=P["bo"], res=x, out=x, layout=WB)
    else:
        ops.linear(attn, P["wo"], bias=P["bo"], res=x, out=x)
    h = norm(P["g2"], P["b2"], blk["up"])
    gelu = "gelu_" + cfg.gelu
    act = bufs.get("vmlp", M, I)
    if blk["down"]:                       # up is blocked too: hand the activation over blocked
        act = act.view(I // 32, M, 32)
        ops.linear_wide(h, P["wup_blk"], M, I, H, bias=P["bup"], act=gelu, out=act,
                        layout=AB | WB | CB)
        ops.linear_wide(act, P["wd_blk"], M, H, I, bias=P["bd"], res=x, out=x, layout=AB | WB)
        return
    if blk["up"]:
        ops.linear_wide(h, P["wup_blk"], M, I, H, bias=P["bup"], act=gelu, out=act,
                        layout=AB | WB)
    else:
        ops.linear(h, P["wup"], bias=P["bup"], act=gelu, out=act)
    ops.linear(act, P["wd"], bias=P["bd"], res=x, out=x)
