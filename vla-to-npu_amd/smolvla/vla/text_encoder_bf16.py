"""SmolVLA text-encoder (prefix) layer, bf16, on gfx950.

Drop-in for ``text_encoder_forward(x, params) -> (output, key, value)``
(reference vla/text_encoder_bf16.py:480-595).  ``x`` is ``[SEQ, EMBD]`` (or
``[B, SEQ, EMBD]``); ``params`` has the reference keys ``Wq Wk Wv Wo W_gate W_up
W_down W_norm_1 W_norm_2`` with ``[in, out]`` weights.

Defaults follow the target configuration (RoPE theta 1e5, RMSNorm eps 1e-5,
causal mask); the reference's own constants (theta 1e4, torch's default eps)
are one ``cfg`` away.  ``kv_export`` picks which K/V are returned: ``"cache"``
(post-RoPE K and V of this layer's QKV projection, the reference NPU path's
return value, :499-500/595) or ``"torch_ref"`` (the torch module's
``k_proj(ln_1(mid-block residual))`` recomputation, :132-135).
"""

from __future__ import annotations

import torch

from .. import layers, ops
from ..config import DecoderConfig, resolve_eps
from ._common import as_batched, prepared, to_device

SEQ = 128
EMBD = 960
Q_H = 15
KV_H = 5
HEAD_DIM = 64
FFN_HID = 2560
DEFAULT_CFG = DecoderConfig(hidden=EMBD, n_q_heads=Q_H, n_kv_heads=KV_H, head_dim=HEAD_DIM,
                            inter=FFN_HID)


def text_encoder_forward(x_np, params, cfg: DecoderConfig = DEFAULT_CFG, mask="causal",
                         prefix_len=0, kv_export="cache"):
    x, back = to_device(x_np)
    x3, squeeze = as_batched(x)
    B, L, H = x3.shape
    P = prepared(params, layers.prep_decoder)
    qd, kvd = cfg.q_dim, cfg.kv_dim
    out = x3.reshape(B * L, H).clone()
    rope = layers.Rope.make(L, cfg.head_dim, cfg.rope_theta, out.device)
    bufs = layers.Buffers(out.device)
    mid = torch.empty_like(out) if kv_export == "torch_ref" else None
    qkv = layers.decoder_layer(out, P, cfg, B, L, rope, mask, prefix_len, bufs, mid_out=mid)
    if kv_export == "cache":
        key, value = qkv[:, qd:qd + kvd].clone(), qkv[:, qd + kvd:].clone()
    elif kv_export == "torch_ref":
        hn = ops.rmsnorm(mid, P["n1"], resolve_eps(cfg.rms_eps))
        key = ops.linear(hn, P["wqkv"][qd:qd + kvd])
        value = ops.linear(hn, P["wqkv"][qd + kvd:])
    else:
        raise ValueError(kv_export)
    shape = (L, -1) if squeeze else (B, L, -1)
    return (back(out.view(*shape)), back(key.reshape(*shape)), back(value.reshape(*shape)))
