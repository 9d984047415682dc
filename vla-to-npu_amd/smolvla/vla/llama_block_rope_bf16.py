"""Llama-style decoder block with RoPE, bf16, on gfx950 (the reference's
768-wide prototype block).

Drop-ins for ``llama_block_rope(x, params) -> (out, key, value)`` and
``llama_block_rope_cross(key, value, x, params) -> out``
(reference vla/llama_block_rope_bf16.py:519-614 and :617-708).  The cross
variant projects Q from ``x``, applies RoPE to Q and to the given ``key``,
and attends causally to ``key``/``value``.  Defaults are the reference block's
dimensions (SEQ 64, EMBD 768, 15/5 heads, FFN 3072) with the target numerics
(theta 1e5, eps 1e-5).
"""

from __future__ import annotations

import torch

from .. import layers, ops
from ..config import DecoderConfig, resolve_eps
from ._common import as_batched, prepared, to_device
from .text_encoder_bf16 import text_encoder_forward

SEQ = 64
EMBD = 768
Q_H = 15
KV_H = 5
HEAD_DIM = 64
FFN_HID = 3072
DEFAULT_CFG = DecoderConfig(hidden=EMBD, inter=FFN_HID)


def llama_block_rope(x_np, params, cfg: DecoderConfig = DEFAULT_CFG):
    return text_encoder_forward(x_np, params, cfg, mask="causal", kv_export="cache")


def _prep_q_only(p, device):
    d = lambda t: layers._dev(t, device)  # noqa: E731
    return dict(
        wq=ops.pack_weight(d(p["Wq"])), wo=ops.pack_weight(d(p["Wo"])),
        wgu=ops.pack_gate_up(d(p["W_gate"]), d(p["W_up"])), wd=ops.pack_weight(d(p["W_down"])),
        n1=d(p["W_norm_1"]), n2=d(p["W_norm_2"]),
    )


def llama_block_rope_cross(key, value, x_np, params, cfg: DecoderConfig = DEFAULT_CFG):
    x, back = to_device(x_np)
    k, _ = to_device(key)
    v, _ = to_device(value)
    x3, squeeze = as_batched(x)
    k3, _ = as_batched(k)
    v3, _ = as_batched(v)
    B, L, H = x3.shape
    Lk = k3.shape[1]
    P = prepared(params, _prep_q_only)
    qd, kvd = cfg.q_dim, cfg.kv_dim
    eps = resolve_eps(cfg.rms_eps)
    dev = x.device
    out = x3.reshape(B * L, H).clone()
    rope_q = layers.Rope.make(L, cfg.head_dim, cfg.rope_theta, dev)
    rope_k = layers.Rope.make(Lk, cfg.head_dim, cfg.rope_theta, dev)
    h = ops.rmsnorm(out, P["n1"], eps)
    q = ops.linear_rope(h, P["wq"], qd, L, rope_q.cos, rope_q.sin)
    kr = torch.empty(B, Lk, kvd, dtype=torch.bfloat16, device=dev)
    for b in range(B):
        ops.rope(k3[b].contiguous(), cfg.n_kv_heads, rope_k.cos, rope_k.sin, out=kr[b])
    attn = torch.empty(B, L, qd, dtype=torch.bfloat16, device=dev)
    ops.attention(q.view(B, L, qd), kr, v3.contiguous(), attn, cfg.n_q_heads, cfg.n_kv_heads,
                  "causal")
    ops.linear(attn.view(B * L, qd), P["wo"], res=out, out=out)
    h = ops.rmsnorm(out, P["n2"], eps)
    act = ops.linear_silu_mul(h, P["wgu"])
    ops.linear(act, P["wd"], res=out, out=out)
    return back(out.view(L, H) if squeeze else out.view(B, L, H))
