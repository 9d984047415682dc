"""SmolVLA action-expert layers, bf16, on gfx950.

Drop-ins for ``action_expert_self_forward(x, params)`` and
``action_expert_cross_forward(x, text_k, text_v, params)``
(reference vla/action_expert_bf16.py:662-728 and :731-803).  Self layers:
causal GQA self-attention with RoPE on Q and K.  Cross layers: Q from the action
tokens (RoPE on Q only), K/V = ``Wk_cross``/``Wv_cross`` projections of the
text encoder's K/V, no mask.  Defaults are the target expert width (hidden
720, FFN 2048, theta 1e5, eps 1e-5); the reference module's 768-wide toy is
``DecoderConfig(hidden=768, inter=2048, rope_theta=1e4)``.
"""

from __future__ import annotations

from .. import layers
from ..config import DecoderConfig
from ._common import as_batched, prepared, to_device

SEQ = 50
TEXT_SEQ = 241
EMBD = 720
Q_H = 15
KV_H = 5
HEAD_DIM = 64
KV_DIM = KV_H * HEAD_DIM
FFN_HID = 2048
DEFAULT_CFG = DecoderConfig(hidden=EMBD, inter=FFN_HID)


def action_expert_self_forward(x_np, params, cfg: DecoderConfig = DEFAULT_CFG):
    x, back = to_device(x_np)
    x3, squeeze = as_batched(x)
    B, L, H = x3.shape
    P = prepared(params, layers.prep_decoder)
    out = x3.reshape(B * L, H).clone()
    rope = layers.Rope.make(L, cfg.head_dim, cfg.rope_theta, out.device)
    layers.decoder_layer(out, P, cfg, B, L, rope, "causal", 0)
    return back(out.view(L, H) if squeeze else out.view(B, L, H))


def action_expert_cross_forward(x_np, text_k_np, text_v_np, params,
                                cfg: DecoderConfig = DEFAULT_CFG):
    x, back = to_device(x_np)
    tk, _ = to_device(text_k_np)
    tv, _ = to_device(text_v_np)
    x3, squeeze = as_batched(x)
    tk3, _ = as_batched(tk)
    tv3, _ = as_batched(tv)
    B, L, H = x3.shape
    Lc = tk3.shape[1]
    P = prepared(params, layers.prep_cross)
    ck, cv = layers.cross_kv(tk3.reshape(B * Lc, -1), tv3.reshape(B * Lc, -1), P)
    out = x3.reshape(B * L, H).clone()
    rope = layers.Rope.make(L, cfg.head_dim, cfg.rope_theta, out.device)
    layers.cross_layer(out, ck, cv, P, cfg, B, L, Lc, rope)
    return back(out.view(L, H) if squeeze else out.view(B, L, H))
