"""SmolVLA pipeline functions with the reference's names
(vla/vla.py:169-222, 228-389), running on gfx950.

* ``create_text_emb(ids, table)``       -- Embedding(ids) * sqrt(H)   (vla.py:169-174)
* ``create_state_emb(state, weights)``  -- state @ W_state             (vla.py:177-182)
* ``vision_encoder(n, x, params)``      -- stacked ViT blocks          (vla.py:185-188)
* ``joint_transformer(...)``            -- VLM layer i feeds expert layer i,
                                           self when i % 2 == 0        (vla.py:194-212)
* ``postprocessing(out, out_params)``   -- RMSNorm then W_action_out   (vla.py:218-222)
* ``smolvla_chunk(...)``                -- the whole target pipeline, via
                                           :class:`smolvla.pipeline.SmolVLAEngine`
"""

from __future__ import annotations

import math

import torch

from .. import ops
from ..config import DecoderConfig, resolve_eps
from ..layers import _dev, host_tensor
from ..pipeline import SmolVLAEngine
from ._common import to_device
from .action_expert_bf16 import action_expert_cross_forward, action_expert_self_forward
from .text_encoder_bf16 import text_encoder_forward
from .vision_block_bf16 import vision_encoder  # noqa: F401

SEQ_T = 48
SKIP = 2
MAX_STATE_DIM = 32


def create_text_emb(lang_tokens, table):
    ids = host_tensor(lang_tokens).to("cuda").reshape(-1)
    t = _dev(table, "cuda")
    out = torch.empty(ids.numel(), t.shape[1], dtype=torch.bfloat16, device="cuda")
    return ops.embed(ids, t, math.sqrt(t.shape[1]), out)


def create_state_emb(state_input, weights):
    s, back = to_device(state_input)
    s2 = s.reshape(-1, s.shape[-1]).contiguous()
    w = ops.pack_weight(_dev(weights, "cuda"))
    return back(ops.linear(s2, w))


def joint_transformer(num_layers, vlm_input, action, vlm_params, exp_self_params,
                      exp_cross_params, vlm_cfg: DecoderConfig = None,
                      exp_cfg: DecoderConfig = None):
    """Per-layer params may be single dicts (shared, as in the reference) or lists."""
    from .action_expert_bf16 import DEFAULT_CFG as EXP
    from .text_encoder_bf16 import DEFAULT_CFG as VLM
    vlm_cfg = vlm_cfg or VLM
    exp_cfg = exp_cfg or EXP
    pick = lambda p, i: p[i] if isinstance(p, (list, tuple)) else p  # noqa: E731
    for i in range(num_layers):
        vlm_input, text_k, text_v = text_encoder_forward(vlm_input, pick(vlm_params, i), vlm_cfg)
        if i % SKIP == 0:
            action = action_expert_self_forward(action, pick(exp_self_params, i), exp_cfg)
        else:
            action = action_expert_cross_forward(action, text_k, text_v,
                                                 pick(exp_cross_params, i), exp_cfg)
    return action


def postprocessing(out, out_params, eps=1e-5):
    x, back = to_device(out)
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    w = _dev(out_params["W_exp_norm"], "cuda")
    h = ops.rmsnorm(x2, w, resolve_eps(eps))
    wo = ops.pack_weight(_dev(out_params["W_action_out"], "cuda"))
    return back(ops.linear(h, wo))


def smolvla_chunk(images, lang_ids, state, noise, params, cfg, use_graph=True):
    """Full SmolVLA inference (3 cameras, 241-token prefix, 10 Euler steps)."""
    eng = SmolVLAEngine(cfg, params, batch=images.shape[0], use_graph=use_graph)
    dev = eng.device
    return eng.run(images.to(dev), lang_ids.to(dev), state.to(dev), noise.to(dev))
