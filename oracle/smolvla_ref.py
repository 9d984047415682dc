"""PyTorch-CPU restatement of the reference's SmolVLA modules (the parity oracle).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Conventions (same as the reference):

* tensors are ``torch.bfloat16`` unless a function says otherwise;
* linear weights are stored ``[in, out]`` (the reference transposes
  ``nn.Linear.weight`` with ``.T`` when it builds ``params``,
  vla/text_encoder_bf16.py:601-611), so ``linear(x, W) == x @ W``;
* rounding points follow the reference's torch modules: projections round to
  bf16, RoPE returns fp32 (vla/text_encoder_bf16.py:92-104, where ``x`` is
  re-bound to fp32 before ``out.to(x.dtype)``), scores and softmax are fp32,
  probabilities are rounded to bf16 before the P.V product
  (vla/text_encoder_bf16.py:121-126).

Configuration objects are duck-typed: any object with the attribute names
used below works (the product's frozen dataclasses, or ``types.SimpleNamespace``
in tests), so the oracle does not import the product package.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16
F32 = torch.float32

# Dtype the attention probabilities are rounded to before the P.V product
# (bf16 in the reference, vla/text_encoder_bf16.py:124).  Pinning tests set it
# to fp32 to compare the block structure against fp32 implementations.
P_DTYPE = torch.bfloat16

__all__ = [
    "rms_norm", "layer_norm", "linear", "silu", "gelu", "rope_tables", "apply_rope",
    "make_mask", "gqa_attention", "decoder_block", "expert_self_block",
    "expert_cross_block", "vit_block", "patch_embed", "pixel_shuffle",
    "connector", "lang_embed", "state_embed", "time_embedding", "expert_input",
    "expert_output", "vision_encoder", "prefix_forward", "cross_kv", "expert_velocity",
    "smolvla_chunk", "masked_softmax_rows", "softmax_rows",
]


# --------------------------------------------------------------------------
# elementwise / normalisation
# --------------------------------------------------------------------------
def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: Optional[float]) -> torch.Tensor:
    """``nn.RMSNorm(H)(x)`` with weight ``w`` (vla/text_encoder_bf16.py:74,78).

    ``eps=None`` reproduces the reference's default-constructed ``nn.RMSNorm``
    (torch 2.10 then uses ``finfo(fp32).eps`` for bf16 input).
    """
    return F.rms_norm(x, (x.shape[-1],), w, eps)


def layer_norm(x, g, b, eps: float) -> torch.Tensor:
    """``nn.LayerNorm`` with affine ``g``/``b`` (vla/vision_block_bf16.py:61,65)."""
    return F.layer_norm(x, (x.shape[-1],), g, b, eps)


def linear(x: torch.Tensor, w_in_out: torch.Tensor, bias: Optional[torch.Tensor] = None):
    """``nn.Linear`` with the reference's ``[in, out]`` weight (x @ W + b)."""
    return F.linear(x, w_in_out.t(), bias)


def silu(x):
    """``nn.SiLU`` (vla/text_encoder_bf16.py:76)."""
    return F.silu(x)


def gelu(x, kind: str = "tanh"):
    """GELU; the reference module uses exact erf ``nn.GELU()``
    (vla/vision_block_bf16.py:64) while its AIE kernel and the target
    configuration use the tanh form (cc/bf16_old/gelu_bf16.cc:94-97)."""
    return F.gelu(x, approximate="tanh" if kind == "tanh" else "none")


# --------------------------------------------------------------------------
# RoPE
# --------------------------------------------------------------------------
def rope_tables(length: int, head_dim: int, theta: float):
    """cos/sin tables ``[L, D/2]`` fp32, angle = pos / theta^(2k/D).

    Follows ``apply_rope`` (vla/text_encoder_bf16.py:80-84, 92-97): the
    timescale is ``theta ** ((2/D) * k)`` and radians are ``pos / timescale``.
    """
    half = head_dim // 2
    freq_exponents = (2.0 / head_dim) * torch.arange(half, dtype=F32)
    timescale = theta ** freq_exponents
    pos = torch.arange(length, dtype=F32)
    radians = pos[:, None] / timescale[None, :]
    return torch.cos(radians), torch.sin(radians)


def apply_rope(x: torch.Tensor, theta: float) -> torch.Tensor:
    """Rotate-half RoPE on ``x [B, L, H, D]``; returns **fp32**
    (vla/text_encoder_bf16.py:92-104, positions 0..L-1 per call)."""
    B, L, H, D = x.shape
    half = D // 2
    c, s = rope_tables(L, D, theta)
    c = c[None, :, None, :]
    s = s[None, :, None, :]
    xf = x.to(F32)
    x1, x2 = xf[..., :half], xf[..., half:]
    out = torch.empty_like(xf)
    out[..., :half] = x1 * c - x2 * s
    out[..., half:] = x2 * c + x1 * s
    return out


# --------------------------------------------------------------------------
# attention
# --------------------------------------------------------------------------
def make_mask(kind: str, lq: int, lk: int, prefix_len: int = 0) -> Optional[torch.Tensor]:
    """Boolean mask, ``True`` = masked out.

    * ``causal``: key j > query i masked (vla/text_encoder_bf16.py:123);
    * ``none``: cross-attention / ViT (vla/action_expert_bf16.py:196);
    * ``prefix_lm``: keys ``< prefix_len`` are visible to every query, later
      keys causally (image+language tokens attend bidirectionally, the state
      token attends to everything before it).
    """
    if kind == "none":
        return None
    i = torch.arange(lq)[:, None]
    j = torch.arange(lk)[None, :]
    if kind == "causal":
        return j > i
    if kind == "prefix_lm":
        return (j > i) & (j >= prefix_len)
    raise ValueError(f"unknown mask kind {kind!r}")


def gqa_attention(q, k, v, mask: Optional[torch.Tensor]) -> torch.Tensor:
    """Grouped-query attention exactly as the reference's torch module.

    ``q [B, L, Hq, D]`` (fp32 after RoPE), ``k [B, Lk, Hkv, D]`` (fp32 or bf16),
    ``v [B, Lk, Hkv, D]`` bf16.  Query head h reads KV head ``h*Hkv // Hq``
    (vla/text_encoder_bf16.py:117-126).  Returns ``ctx [B, L, Hq*D]`` bf16.
    """
    B, L, Hq, D = q.shape
    Hkv = k.shape[2]
    kv_map = torch.div(torch.arange(Hq) * Hkv, Hq, rounding_mode="floor")
    k_sel = k.index_select(2, kv_map)
    v_sel = v.index_select(2, kv_map)
    q_h = q.transpose(1, 2).float()
    k_h = k_sel.transpose(1, 2).float()
    scores = torch.matmul(q_h, k_h.transpose(-2, -1)) / (D ** 0.5)
    if mask is not None:
        scores.masked_fill_(mask, float("-inf"))
    attn = torch.softmax(scores, dim=-1).to(P_DTYPE)
    v_h = v_sel.transpose(1, 2)
    ctx = torch.matmul(attn.float(), v_h.float()).to(v.dtype)
    return ctx.transpose(1, 2).contiguous().view(B, L, Hq * D)


def masked_softmax_rows(scores: torch.Tensor, row_start: int) -> torch.Tensor:
    """Per-kernel harness semantics of ``masked_softmax_128_bf16``: causal
    mask at global row ``row_start + r``, fp32 softmax, bf16 out
    (vla/tests/test_masked_softmax_128_bf16.py:47-55)."""
    R, C = scores.shape
    rows = torch.arange(R)[:, None] + row_start
    cols = torch.arange(C)[None, :]
    s = scores.float().masked_fill(cols > rows, float("-inf"))
    return F.softmax(s, dim=-1).to(BF16)


def softmax_rows(scores: torch.Tensor) -> torch.Tensor:
    """Unmasked row softmax in fp32, bf16 out
    (softmax_bf16/test_softmax_bf16_seq1024.py:87-95)."""
    return F.softmax(scores.float(), dim=-1).to(BF16)


# --------------------------------------------------------------------------
# transformer blocks
# --------------------------------------------------------------------------
def _mlp_silu(x, p):
    """``down(silu(gate(x)) * up(x))`` (vla/text_encoder_bf16.py:130-131)."""
    return linear(silu(linear(x, p["W_gate"])) * linear(x, p["W_up"]), p["W_down"])


def decoder_block(x, p, cfg, mask_kind="causal", prefix_len=0, kv_export="cache"):
    """SmolLM2-style decoder block, ``TextEncoderBlock.forward``
    (vla/text_encoder_bf16.py:106-135).

    ``x [B, L, H]`` bf16.  Returns ``(out, key, value)`` with key/value
    ``[B, L, Hkv*D]`` bf16.

    ``kv_export`` chooses between the reference's two conflicting definitions
    of the K/V handed to the action expert:
    * ``"cache"`` (default): post-RoPE K and V from this layer's own QKV step,
      as the reference's NPU path returns them (vla/text_encoder_bf16.py:499-500,
      595) -- this is what the KV cache holds;
    * ``"torch_ref"``: the torch module's recomputation
      ``k_proj(ln_1(mid-block residual))`` without RoPE (:132-135).
    """
    B, L, _ = x.shape
    Hq, Hkv, D = cfg.n_q_heads, cfg.n_kv_heads, cfg.head_dim
    residual = x
    h = rms_norm(x, p["W_norm_1"], cfg.rms_eps)
    q = linear(h, p["Wq"]).view(B, L, Hq, D)
    k = linear(h, p["Wk"]).view(B, L, Hkv, D)
    v = linear(h, p["Wv"]).view(B, L, Hkv, D)
    q = apply_rope(q, cfg.rope_theta)
    k = apply_rope(k, cfg.rope_theta)
    ctx = gqa_attention(q, k, v, make_mask(mask_kind, L, L, prefix_len))
    x = linear(ctx, p["Wo"]) + residual
    residual = x
    x = _mlp_silu(rms_norm(x, p["W_norm_2"], cfg.rms_eps), p) + residual
    if kv_export == "cache":
        k_out = k.to(v.dtype).reshape(B, L, Hkv * D)
        v_out = v.reshape(B, L, Hkv * D)
    elif kv_export == "torch_ref":
        hn = rms_norm(residual, p["W_norm_1"], cfg.rms_eps)
        k_out = linear(hn, p["Wk"])
        v_out = linear(hn, p["Wv"])
    else:
        raise ValueError(kv_export)
    return x, k_out, v_out


def expert_self_block(x, p, cfg):
    """``ActionExpertSelfBlock.forward`` (vla/action_expert_bf16.py:102-128):
    causal GQA self-attention over the action tokens, RoPE on Q and K."""
    out, _, _ = decoder_block(x, p, cfg, mask_kind="causal")
    return out


def expert_cross_block(x, text_k, text_v, p, cfg):
    """``ActionExpertCrossBlock.forward`` (vla/action_expert_bf16.py:163-207).

    Q from the action tokens (RoPE on Q only), K/V = ``Linear(Hkv*D -> Hkv*D)``
    of the prefix K/V (``Wk_cross``/``Wv_cross``), no mask.
    ``text_k``/``text_v`` are ``[B, Lc, Hkv*D]`` bf16.
    """
    B, L, _ = x.shape
    Lc = text_k.shape[1]
    Hq, Hkv, D = cfg.n_q_heads, cfg.n_kv_heads, cfg.head_dim
    residual = x
    xn = rms_norm(x, p["W_norm_1"], cfg.rms_eps)
    q = linear(xn, p["Wq"]).view(B, L, Hq, D)
    k = linear(text_k, p["Wk_cross"]).view(B, Lc, Hkv, D)
    v = linear(text_v, p["Wv_cross"]).view(B, Lc, Hkv, D)
    q = apply_rope(q, cfg.rope_theta)
    ctx = gqa_attention(q, k, v, None)
    x = linear(ctx, p["Wo"]) + residual
    residual = x
    return _mlp_silu(rms_norm(x, p["W_norm_2"], cfg.rms_eps), p) + residual


def vit_block(x, p, cfg):
    """``MiniVit.forward`` (vla/vision_block_bf16.py:67-79): pre-LN, MHA
    (``nn.MultiheadAttention``, which for ``need_weights=False`` calls
    scaled-dot-product attention), GELU MLP, residuals.

    Biases ``bq/bk/bv/bo/b_up/b_down`` are optional (the reference zeroes the
    attention biases and has none on the MLP; SigLIP has all of them).
    """
    B, L, H = x.shape
    nh, D = cfg.n_heads, cfg.head_dim
    residual = x
    h = layer_norm(x, p["W_norm_1"], p["b_norm_1"], cfg.ln_eps)
    w_in = torch.cat([p["Wq"], p["Wk"], p["Wv"]], dim=1)
    b_in = None
    if p.get("bq") is not None:
        b_in = torch.cat([p["bq"], p["bk"], p["bv"]])
    qkv = linear(h, w_in, b_in)
    q, k, v = qkv.split(H, dim=-1)
    q = q.view(B, L, nh, D).transpose(1, 2)
    k = k.view(B, L, nh, D).transpose(1, 2)
    v = v.view(B, L, nh, D).transpose(1, 2)
    a = F.scaled_dot_product_attention(q, k, v)
    a = a.transpose(1, 2).reshape(B, L, H)
    x = linear(a, p["Wo"], p.get("bo")) + residual
    residual = x
    h = layer_norm(x, p["W_norm_2"], p["b_norm_2"], cfg.ln_eps)
    h = gelu(linear(h, p["W_up"], p.get("b_up")), cfg.gelu)
    return residual + linear(h, p["W_down"], p.get("b_down"))


# --------------------------------------------------------------------------
# embeddings / connector
# --------------------------------------------------------------------------
def patch_embed(img, kernel, bias, pos_emb):
    """SigLIP patch embedding: ``Conv2d(3->E, k=s=P)`` then flatten over the
    patch grid row-major and add the learned position embedding
    (vla/vla.py:396-408; vla/vit_emb.py:43-47).  ``img [B,3,H,W]`` bf16."""
    P = kernel.shape[-1]
    y = F.conv2d(img, kernel, bias, stride=P)
    y = y.flatten(2).transpose(1, 2)
    return y + pos_emb[None]


def pixel_shuffle(x, scale: int):
    """Pixel-shuffle of ``x [B, N, E]`` (N a square) to ``[B, N/s^2, E*s^2]``,
    the reshape/transpose chain of ``con_ref`` (vla/vla.py:435)."""
    B, N, E = x.shape
    g = int(round(math.sqrt(N)))
    x = x.reshape(B, g, g, E)
    x = x.reshape(B, g, g // scale, E * scale).transpose(1, 2)
    x = x.reshape(B, g // scale, g // scale, E * scale * scale).transpose(1, 2)
    return x.reshape(B, N // (scale * scale), E * scale * scale)


def connector(x, w, scale: int):
    """``con_ref``: pixel-shuffle then ``@ W`` (vla/vla.py:434-437)."""
    return linear(pixel_shuffle(x, scale), w)


def lang_embed(ids, table):
    """``Embedding(ids) * sqrt(H)`` (vla/vla.py:169-174)."""
    return (table[ids].float() * math.sqrt(table.shape[1])).to(table.dtype)


def state_embed(state, w):
    """State projection ``state @ W_state`` (vla/vla.py:177-182, 357)."""
    return linear(state, w)


def time_embedding(t: torch.Tensor, dim: int, min_period=4e-3, max_period=4.0):
    """Sinusoidal time embedding ``[sin(2pi t/p), cos(2pi t/p)]`` over
    geometrically spaced periods (absent from the reference; the target
    configuration's flow-matching time input).  fp32 ``[T, dim]``."""
    fraction = torch.linspace(0.0, 1.0, dim // 2, dtype=torch.float64)
    period = min_period * (max_period / min_period) ** fraction
    scaling = (1.0 / period) * 2 * math.pi
    sin_input = scaling[None, :] * t.to(torch.float64)[:, None]
    return torch.cat([torch.sin(sin_input), torch.cos(sin_input)], dim=1).to(F32)


# --------------------------------------------------------------------------
# pipeline pieces
# --------------------------------------------------------------------------
def vision_encoder(images, params, cfg):
    """``[B, C, 3, H, W]`` -> per-camera ViT output ``[B, C, N, E]``."""
    B, C = images.shape[:2]
    x = patch_embed(images.reshape(B * C, *images.shape[2:]), params["patch"]["kernel"],
                    params["patch"]["bias"], params["patch"]["pos_emb"])
    for lp in params["vit"]:
        x = vit_block(x, lp, cfg.vit)
    return x.reshape(B, C, x.shape[1], x.shape[2])


def build_prefix(vis, lang_ids, state, params, cfg):
    """Concatenate ``[cam0 | cam1 | cam2 | language | state]`` tokens
    (vla/vla.py:326; 3 cameras and no padding in the target config)."""
    B, C, N, E = vis.shape
    con = connector(vis.reshape(B * C, N, E), params["connector"]["W"], cfg.pixel_shuffle)
    con = con.reshape(B, C * con.shape[1], con.shape[2])
    lang = lang_embed(lang_ids, params["embed"])
    wdt = params["state"]["W"].dtype
    st = state_embed(state.to(wdt)[:, None, :], params["state"]["W"])
    return torch.cat([con, lang, st], dim=1)


def prefix_forward(prefix, params, cfg, kv_export="cache"):
    """16 decoder layers with the prefix-LM mask; returns the final hidden
    state and the per-layer K/V cache ``[(k, v)]``."""
    x = prefix
    kv = []
    for lp in params["prefix"]:
        x, k, v = decoder_block(x, lp, cfg.decoder, cfg.prefix_mask, cfg.prefix_bidir_len,
                                kv_export)
        kv.append((k, v))
    return x, kv


def cross_kv(kv, params, cfg):
    """Cross-layer K/V projections of the cache (hoisted out of the Euler
    loop; the reference applies them inside every cross layer,
    vla/action_expert_bf16.py:182-183)."""
    out = {}
    for i, lp in enumerate(params["expert"]):
        if cfg.is_cross(i):
            k, v = kv[i]
            out[i] = (linear(k, lp["Wk_cross"]), linear(v, lp["Wv_cross"]))
    return out


def expert_input(x_t, t, params, cfg):
    """Action/time embedding of the noisy chunk: ``action_in`` (Linear 32->H),
    concat with the sinusoidal time embedding, ``time_in`` (2H->H), SiLU,
    ``time_out`` (H->H).  ``x_t [B, 50, 32]`` fp32, ``t`` python float."""
    io = params["expert_io"]
    B, L, _ = x_t.shape
    H = cfg.expert.hidden
    wdt = io["W_action_in"].dtype                       # bf16 (fp32 in pinning tests)
    a = linear(x_t.to(wdt), io["W_action_in"], io["b_action_in"])
    te = time_embedding(torch.tensor([t]), H).to(wdt)
    te = te[:, None, :].expand(B, L, H)
    h = linear(torch.cat([a, te], dim=2), io["W_time_in"], io["b_time_in"])
    return linear(silu(h), io["W_time_out"], io["b_time_out"])


def expert_output(h, params, cfg):
    """Final expert RMSNorm then action projection (vla/vla.py:218-222, 506-516)."""
    io = params["expert_io"]
    return linear(rms_norm(h, io["W_exp_norm"], cfg.expert.rms_eps), io["W_action_out"])


def expert_velocity(x_t, t, ckv, params, cfg, cross_src=None):
    """One evaluation of the expert: ``v = f(x_t, t; prefix KV)``.

    Layer i is self-attention when ``i % 2 == 0`` and cross-attention on layer
    i's prefix K/V otherwise (vla/vla.py:194-212).  ``ckv`` holds the already
    projected cross K/V (``cross_kv``)."""
    h = expert_input(x_t, t, params, cfg)
    for i, lp in enumerate(params["expert"]):
        if cfg.is_cross(i):
            h = _cross_with_projected(h, ckv[i][0], ckv[i][1], lp, cfg.expert)
        else:
            h = expert_self_block(h, lp, cfg.expert)
    return expert_output(h, params, cfg)


def _cross_with_projected(x, k, v, p, cfg):
    """``expert_cross_block`` with K/V already projected by Wk/Wv_cross."""
    B, L, _ = x.shape
    Lc = k.shape[1]
    Hq, Hkv, D = cfg.n_q_heads, cfg.n_kv_heads, cfg.head_dim
    residual = x
    xn = rms_norm(x, p["W_norm_1"], cfg.rms_eps)
    q = apply_rope(linear(xn, p["Wq"]).view(B, L, Hq, D), cfg.rope_theta)
    ctx = gqa_attention(q, k.view(B, Lc, Hkv, D), v.view(B, Lc, Hkv, D), None)
    x = linear(ctx, p["Wo"]) + residual
    residual = x
    return _mlp_silu(rms_norm(x, p["W_norm_2"], cfg.rms_eps), p) + residual


def smolvla_chunk(images, lang_ids, state, noise, params, cfg, capture=None):
    """Full SmolVLA inference producing one action chunk per sample.

    vision -> connector -> prefix (KV cache) -> ``cfg.num_steps`` Euler steps
    ``x <- x + dt * v(x, t)``, ``t`` from 1.0 with ``dt = -1/num_steps``.
    ``noise [B, 50, 32]`` fp32; returns fp32 ``[B, 50, 32]``.  ``capture`` (a
    dict) receives the intermediate stages.
    """
    vis = vision_encoder(images, params, cfg)
    prefix = build_prefix(vis, lang_ids, state, params, cfg)
    _, kv = prefix_forward(prefix, params, cfg)
    ckv = cross_kv(kv, params, cfg)
    x_t = noise.to(F32).clone()
    dt = -1.0 / cfg.num_steps
    t = 1.0
    vels = []
    for _ in range(cfg.num_steps):
        v = expert_velocity(x_t, t, ckv, params, cfg)
        vels.append(v)
        x_t = x_t + dt * v.float()
        t = t + dt
    if capture is not None:
        capture.update(vision=vis, prefix=prefix, kv=kv, cross_kv=ckv, velocities=vels)
    return x_t
