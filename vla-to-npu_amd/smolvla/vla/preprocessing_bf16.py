"""SigLIP patch embedding, bf16, on gfx950.

Drop-in for ``preprocessing_block(img, params) -> [1024, 768]`` (reference
vla/preprocessing_bf16.py:105-109, which loops 14,592 single-channel 16x16
conv dispatches): one im2col GEMM over ``params["kernel"] [768, 3, 16, 16]``,
with the optional conv ``bias`` and learned position embedding ``pos_emb``
(vla/vit_emb.py:43-47) fused into the epilogue.  ``img`` is ``[3, H, W]`` or
``[n, 3, H, W]``.
"""

from __future__ import annotations

from .. import ops
from ..layers import _dev
from ._common import to_device

CHANNELS = 3
PIX_LEN = 512
KERNEL_DIM = 16
SEQ = 1024
EMBD_DIM = 768


def preprocessing_block(x_np, params):
    img, back = to_device(x_np)
    squeeze = img.dim() == 3
    img4 = img.unsqueeze(0) if squeeze else img
    kern = _dev(params["kernel"], img.device)
    E, C, P, _ = kern.shape
    w = kern.reshape(E, C * P * P).contiguous()
    bias = params.get("bias")
    pos = params.get("pos_emb")
    bias = _dev(bias, img.device) if bias is not None else None
    pos = _dev(pos, img.device) if pos is not None else None
    out = ops.patch_embed(img4.contiguous(), w, bias, pos, P)
    n = img4.shape[0]
    return back(out if squeeze else out.view(n, -1, E))
