"""SigLIP-style ViT block, bf16, on gfx950.

Drop-in for ``vision_block(x, params) -> out`` (reference
vla/vision_block_bf16.py:308-420): pre-LayerNorm (with the ``b_norm_*``
shifts), multi-head attention (12 heads x 64, no mask), GELU MLP, residuals.
Optional SigLIP biases ``bq bk bv bo b_up b_down`` are honoured when present.
Defaults: LN eps 1e-6 and tanh-GELU (target configuration); the reference
module's choices are ``VitConfig(ln_eps=1e-5, gelu="erf")``.
"""

from __future__ import annotations

from .. import layers
from ..config import VitConfig
from ._common import as_batched, prepared, to_device

SEQ = 1024
EMBD = 768
N_HEAD = 12
HEAD_DIM = 64
FFN_HID = 3072
DEFAULT_CFG = VitConfig()


def vision_block(x_np, params, cfg: VitConfig = DEFAULT_CFG):
    x, back = to_device(x_np)
    x3, squeeze = as_batched(x)
    B, T, H = x3.shape
    P = prepared(params, layers.prep_vit)
    out = x3.reshape(B * T, H).clone()
    layers.vit_layer(out, P, cfg, B, T)
    return back(out.view(T, H) if squeeze else out.view(B, T, H))


def vision_encoder(num_layers, x, params, cfg: VitConfig = DEFAULT_CFG):
    """``vision_encoder`` (vla/vla.py:185-188): the same block applied
    ``num_layers`` times, or a list of per-layer params."""
    plist = params if isinstance(params, (list, tuple)) else [params] * num_layers
    for p in plist[:num_layers]:
        x = vision_block(x, p, cfg)
    return x
