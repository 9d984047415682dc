"""Seeded random-init parameters with the reference's ``params`` naming.

Linear weights are ``[in, out]`` bf16 drawn from N(0, 0.02) (the reference
builds ``params`` by transposing ``nn.Linear.weight``,
vla/text_encoder_bf16.py:601-611; key names ``Wq Wk Wv Wo W_gate W_up W_down
W_norm_1 W_norm_2`` there, ``Wk_cross Wv_cross`` at
vla/action_expert_bf16.py:880-890, ``b_norm_*`` / ``W_up`` / ``W_down`` at
vla/vision_block_bf16.py:438-449, ``W`` for the connector at
vla/connector_bf16.py:151 and ``kernel`` for the patch embedding at
vla/vla.py:246-248).

Norm gains default to 1 and LayerNorm shifts to 0 (torch's default init, as
the reference's modules use); ``norm_init="random"`` draws them around 1 / 0
so that tests exercise the gain and shift paths.
"""

from __future__ import annotations

import torch

from .config import DecoderConfig, SmolVLAConfig, VitConfig

BF16 = torch.bfloat16


class _Gen:
    def __init__(self, seed: int, device="cpu", std: float = 0.02, norm_init: str = "ones"):
        self.g = torch.Generator(device=device)
        self.g.manual_seed(seed)
        self.device = device
        self.std = std
        self.norm_init = norm_init

    def randn(self, *shape, std=None):
        s = self.std if std is None else std
        t = torch.randn(*shape, generator=self.g, device=self.device, dtype=torch.float32)
        return (t * s).to(BF16)

    def lin(self, n_in, n_out):
        return self.randn(n_in, n_out)

    def gain(self, n):
        if self.norm_init == "random":
            return (1.0 + self.randn(n, std=0.1).float()).to(BF16)
        return torch.ones(n, dtype=BF16, device=self.device)

    def shift(self, n):
        if self.norm_init == "random":
            return self.randn(n, std=0.1)
        return torch.zeros(n, dtype=BF16, device=self.device)


def decoder_layer_params(gen: _Gen, cfg: DecoderConfig):
    H, I = cfg.hidden, cfg.inter
    return dict(
        Wq=gen.lin(H, cfg.q_dim), Wk=gen.lin(H, cfg.kv_dim), Wv=gen.lin(H, cfg.kv_dim),
        Wo=gen.lin(cfg.q_dim, H),
        W_gate=gen.lin(H, I), W_up=gen.lin(H, I), W_down=gen.lin(I, H),
        W_norm_1=gen.gain(H), W_norm_2=gen.gain(H),
    )


def expert_cross_layer_params(gen: _Gen, cfg: DecoderConfig, kv_in: int):
    H, I = cfg.hidden, cfg.inter
    return dict(
        Wq=gen.lin(H, cfg.q_dim),
        Wk_cross=gen.lin(kv_in, cfg.kv_dim), Wv_cross=gen.lin(kv_in, cfg.kv_dim),
        Wo=gen.lin(cfg.q_dim, H),
        W_gate=gen.lin(H, I), W_up=gen.lin(H, I), W_down=gen.lin(I, H),
        W_norm_1=gen.gain(H), W_norm_2=gen.gain(H),
    )


def vit_layer_params(gen: _Gen, cfg: VitConfig, biases: bool = True):
    H, I = cfg.hidden, cfg.inter
    p = dict(
        Wq=gen.lin(H, H), Wk=gen.lin(H, H), Wv=gen.lin(H, H), Wo=gen.lin(H, H),
        W_up=gen.lin(H, I), W_down=gen.lin(I, H),
        W_norm_1=gen.gain(H), b_norm_1=gen.shift(H),
        W_norm_2=gen.gain(H), b_norm_2=gen.shift(H),
    )
    if biases:
        p.update(bq=gen.randn(H), bk=gen.randn(H), bv=gen.randn(H), bo=gen.randn(H),
                 b_up=gen.randn(I), b_down=gen.randn(H))
    return p


def smolvla_params(cfg: SmolVLAConfig, seed: int = 0, device="cpu", norm_init="ones"):
    """All parameters of the pipeline as nested dicts/lists of bf16 tensors."""
    gen = _Gen(seed, device=device, norm_init=norm_init)
    v, d, e = cfg.vit, cfg.decoder, cfg.expert
    P = {}
    P["patch"] = dict(
        kernel=gen.randn(v.hidden, v.channels, v.patch, v.patch),
        bias=gen.randn(v.hidden),
        pos_emb=gen.randn(v.tokens, v.hidden),
    )
    P["vit"] = [vit_layer_params(gen, v) for _ in range(v.layers)]
    P["connector"] = dict(W=gen.lin(v.hidden * cfg.pixel_shuffle ** 2, d.hidden))
    P["embed"] = gen.randn(cfg.vocab, d.hidden)
    P["state"] = dict(W=gen.lin(cfg.state_dim, d.hidden))
    P["prefix"] = [decoder_layer_params(gen, d) for _ in range(cfg.prefix_layers)]
    P["expert"] = [
        expert_cross_layer_params(gen, e, d.kv_dim) if cfg.is_cross(i)
        else decoder_layer_params(gen, e)
        for i in range(cfg.expert_layers)
    ]
    H = e.hidden
    P["expert_io"] = dict(
        W_action_in=gen.lin(cfg.action_dim, H), b_action_in=gen.randn(H),
        W_time_in=gen.lin(2 * H, H), b_time_in=gen.randn(H),
        W_time_out=gen.lin(H, H), b_time_out=gen.randn(H),
        W_exp_norm=gen.gain(H),
        W_action_out=gen.lin(H, cfg.action_dim),
    )
    return P


def smolvla_inputs(cfg: SmolVLAConfig, batch: int, seed: int = 1, device="cpu"):
    """Synthetic inputs: pixels U(-1,1), language ids U{0..vocab-1}, state
    N(0,1), noise N(0,1) (fp32)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    v = cfg.vit
    images = (torch.rand(batch, cfg.n_cameras, v.channels, v.image, v.image, generator=g,
                         device=device) * 2 - 1).to(BF16)
    ids = torch.randint(0, cfg.vocab, (batch, cfg.lang_tokens), generator=g, device=device)
    state = torch.randn(batch, cfg.state_dim, generator=g, device=device)
    noise = torch.randn(batch, cfg.chunk, cfg.action_dim, generator=g, device=device)
    return images, ids, state, noise


def tree_map(fn, tree):
    if isinstance(tree, dict):
        return {k: tree_map(fn, v) for k, v in tree.items()}
    if isinstance(tree, (list, tuple)):
        return type(tree)(tree_map(fn, v) for v in tree)
    if isinstance(tree, torch.Tensor):
        return fn(tree)
    return tree
