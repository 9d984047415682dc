"""Frozen configuration objects for the SmolVLA hot path.

One dataclass per sub-model.  The defaults are the target configuration
(SmolVLA dimensions); every numerical choice on which the reference is
inconsistent is an explicit field:

* ``rope_theta``: the reference hard-codes 10 000
  (vla/text_encoder_bf16.py:79); the target uses 100 000.
* ``rms_eps``: the reference's ``nn.RMSNorm(EMBD)`` has ``eps=None``
  (vla/text_encoder_bf16.py:74) which torch resolves to FLT_EPSILON for bf16
  input; the target uses 1e-5.  ``None`` is accepted and means FLT_EPSILON.
* ``ln_eps`` / ``gelu``: the reference's ViT module uses ``nn.LayerNorm``
  (1e-5) and exact-erf ``nn.GELU`` (vla/vision_block_bf16.py:61-65); the target
  uses 1e-6 and tanh-GELU (the reference's AIE kernel form,
  cc/bf16_old/gelu_bf16.cc:94-97).
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field

FLT_EPSILON = 1.1920928955078125e-07


def resolve_eps(eps):
    """``None`` -> FLT_EPSILON (torch's default for ``nn.RMSNorm(eps=None)``)."""
    return FLT_EPSILON if eps is None else float(eps)


@dataclass(frozen=True)
class DecoderConfig:
    """SmolLM2-style decoder block (vla/text_encoder_bf16.py:39-56)."""
    hidden: int = 960
    n_q_heads: int = 15
    n_kv_heads: int = 5
    head_dim: int = 64
    inter: int = 2560
    rope_theta: float = 100000.0
    rms_eps: float = 1e-5

    @property
    def q_dim(self):
        return self.n_q_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim


@dataclass(frozen=True)
class VitConfig:
    """SigLIP-style ViT (vla/vision_block_bf16.py:39-45; vla/vit_emb.py:18-24)."""
    hidden: int = 768
    n_heads: int = 12
    head_dim: int = 64
    inter: int = 3072
    ln_eps: float = 1e-6
    gelu: str = "tanh"
    layers: int = 12
    image: int = 512
    patch: int = 16
    channels: int = 3

    @property
    def grid(self):
        return self.image // self.patch

    @property
    def tokens(self):
        return self.grid * self.grid


def expert_default():
    return DecoderConfig(hidden=720, inter=2048)


@dataclass(frozen=True)
class SmolVLAConfig:
    """The whole pipeline."""
    vit: VitConfig = field(default_factory=VitConfig)
    decoder: DecoderConfig = field(default_factory=DecoderConfig)
    expert: DecoderConfig = field(default_factory=expert_default)
    n_cameras: int = 3
    pixel_shuffle: int = 4
    lang_tokens: int = 48
    vocab: int = 49152
    state_dim: int = 32
    action_dim: int = 32
    chunk: int = 50
    prefix_layers: int = 16
    expert_layers: int = 16
    num_steps: int = 10
    prefix_mask: str = "prefix_lm"
    cross_every: int = 2

    def is_cross(self, layer: int) -> bool:
        """Expert layer ``i`` cross-attends when ``i % 2 == 1``
        (vla/vla.py:204-211, ``SKIP = 2``)."""
        return layer % self.cross_every == 1

    @property
    def image_tokens(self):
        return self.vit.tokens // (self.pixel_shuffle ** 2)

    @property
    def prefix_len(self):
        return self.n_cameras * self.image_tokens + self.lang_tokens + 1

    @property
    def prefix_bidir_len(self):
        """Image + language tokens attend bidirectionally; the state token
        starts a causal block."""
        return self.n_cameras * self.image_tokens + self.lang_tokens

    def replace(self, **kw):
        return dataclasses.replace(self, **kw)


def small_config() -> SmolVLAConfig:
    """A reduced configuration (same structure, small sizes) for fast tests."""
    return SmolVLAConfig(
        vit=VitConfig(hidden=128, n_heads=2, inter=256, layers=2, image=64, patch=16),
        decoder=DecoderConfig(hidden=192, inter=256, n_q_heads=3, n_kv_heads=1),
        expert=DecoderConfig(hidden=144, inter=192, n_q_heads=3, n_kv_heads=1),
        n_cameras=2, pixel_shuffle=2, lang_tokens=8, vocab=1000, chunk=10,
        prefix_layers=4, expert_layers=4, num_steps=3,
    )
