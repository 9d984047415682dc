"""Pixel-shuffle connector, bf16, on gfx950.

Drop-in for ``connector_block(x, params) -> out`` (reference
vla/connector_bf16.py:136-139; formula ``con_ref`` vla/vla.py:434-437):
pixel-shuffle ``[1024, 768] -> [64, 12288]`` (scale 4) then ``@ W [12288, 960]``.
The shuffle is folded into the GEMM's A-operand addressing.  ``x`` may be
``[N, E]`` or ``[n_img, N, E]``.
"""

from __future__ import annotations

from .. import layers, ops
from ._common import prepared, to_device

SEQ = 1024
EMBD = 768
SCALE_FACTOR = 4
NEW_SEQ = 64
NEW_EMBD = 12288
TEXT = 960


def _prep_connector(p, device):
    return ops.pack_weight(layers._dev(p["W"], device))


def connector_block(x_np, params, scale=SCALE_FACTOR):
    x, back = to_device(x_np)
    squeeze = x.dim() == 2
    x3 = x.unsqueeze(0) if squeeze else x
    w = prepared(params, _prep_connector)
    out = ops.connector(x3.contiguous(), w, scale)
    n = x3.shape[0]
    return back(out if squeeze else out.view(n, -1, out.shape[1]))
