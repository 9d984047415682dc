"""Pipeline parameters on disk: safetensors files from local paths only
(nothing is fetched by name).

Two layouts are understood:

* this package's own: the nested ``params`` tree (``smolvla.params``) flattened
  with ``"."`` (``"prefix.3.W_gate"``, ``"expert_io.W_action_in"``), weights
  ``[in, out]`` exactly as the reference builds its ``params`` dicts
  (vla/text_encoder_bf16.py:601-611, vla/action_expert_bf16.py:880-890,
  vla/vision_block_bf16.py:438-449, vla/connector_bf16.py:151, vla/vla.py:240-301).
  ``save_params`` / ``load_params`` round-trip it bit for bit.
* a Hugging Face / LeRobot-style SmolVLA state dict: ``nn.Linear`` weights
  ``[out, in]`` under module names such as
  ``model.vlm_with_expert.vlm.model.text_model.layers.3.mlp.gate_proj.weight``
  (the table in ``hf_name_map``).  ``from_hf_state_dict`` transposes and
  renames; tensors the pipeline does not use (e.g. a final vision LayerNorm,
  the text model's final norm, projection biases the reference modules do not
  have) are returned as ``ignored`` instead of being silently dropped.  The
  module names follow the public SmolVLA policy layout; no such checkpoint is
  available offline, so the mapping is exercised on synthetic state dicts
  written with these names, and a different naming can be passed in as a
  table.
"""

from __future__ import annotations

import pathlib
from typing import Dict, List, Optional, Tuple

import torch

from .config import SmolVLAConfig

BF16 = torch.bfloat16


# ------------------------------------------------------------ own layout ---
def flatten(params, prefix="") -> Dict[str, torch.Tensor]:
    out = {}
    if isinstance(params, dict):
        for k, v in params.items():
            if k.startswith("__"):  # device-side caches (packed weights)
                continue
            out.update(flatten(v, f"{prefix}{k}."))
    elif isinstance(params, (list, tuple)):
        for i, v in enumerate(params):
            out.update(flatten(v, f"{prefix}{i}."))
    else:
        out[prefix[:-1]] = params
    return out


def unflatten(flat: Dict[str, torch.Tensor]):
    root: dict = {}
    for key, t in flat.items():
        parts = key.split(".")
        node = root
        for a, b in zip(parts[:-1], parts[1:]):
            node = node.setdefault(a, {})
        node[parts[-1]] = t

    def lists(n):
        if not isinstance(n, dict):
            return n
        if n and all(k.isdigit() for k in n):
            return [lists(n[str(i)]) for i in range(len(n))]
        return {k: lists(v) for k, v in n.items()}
    return lists(root)


def expected_shapes(cfg: SmolVLAConfig) -> Dict[str, Tuple[int, ...]]:
    """Key -> shape of every parameter the pipeline consumes for ``cfg``."""
    v, d, e = cfg.vit, cfg.decoder, cfg.expert
    s: Dict[str, Tuple[int, ...]] = {
        "patch.kernel": (v.hidden, v.channels, v.patch, v.patch),
        "patch.bias": (v.hidden,), "patch.pos_emb": (v.tokens, v.hidden),
        "connector.W": (v.hidden * cfg.pixel_shuffle ** 2, d.hidden),
        "embed": (cfg.vocab, d.hidden), "state.W": (cfg.state_dim, d.hidden),
    }
    H = v.hidden
    for i in range(v.layers):
        p = f"vit.{i}."
        for n in ("Wq", "Wk", "Wv", "Wo"):
            s[p + n] = (H, H)
        s[p + "W_up"], s[p + "W_down"] = (H, v.inter), (v.inter, H)
        for n in ("bq", "bk", "bv", "bo", "b_down", "W_norm_1", "b_norm_1", "W_norm_2",
                  "b_norm_2"):
            s[p + n] = (H,)
        s[p + "b_up"] = (v.inter,)

    def dec(p, c, cross_in=None):
        Hd, I = c.hidden, c.inter
        s[p + "Wq"], s[p + "Wo"] = (Hd, c.q_dim), (c.q_dim, Hd)
        if cross_in is None:
            s[p + "Wk"], s[p + "Wv"] = (Hd, c.kv_dim), (Hd, c.kv_dim)
        else:
            s[p + "Wk_cross"], s[p + "Wv_cross"] = (cross_in, c.kv_dim), (cross_in, c.kv_dim)
        s[p + "W_gate"], s[p + "W_up"], s[p + "W_down"] = (Hd, I), (Hd, I), (I, Hd)
        s[p + "W_norm_1"], s[p + "W_norm_2"] = (Hd,), (Hd,)
    for i in range(cfg.prefix_layers):
        dec(f"prefix.{i}.", d)
    for i in range(cfg.expert_layers):
        dec(f"expert.{i}.", e, d.kv_dim if cfg.is_cross(i) else None)
    He = e.hidden
    s.update({
        "expert_io.W_action_in": (cfg.action_dim, He), "expert_io.b_action_in": (He,),
        "expert_io.W_time_in": (2 * He, He), "expert_io.b_time_in": (He,),
        "expert_io.W_time_out": (He, He), "expert_io.b_time_out": (He,),
        "expert_io.W_exp_norm": (He,), "expert_io.W_action_out": (He, cfg.action_dim),
    })
    return s


def check_params(params, cfg: SmolVLAConfig, allow_missing_vit_bias: bool = True):
    """Raise ValueError listing every missing, unexpected or mis-shaped tensor."""
    flat = flatten(params)
    want = expected_shapes(cfg)
    optional = {k for k in want if allow_missing_vit_bias and k.startswith("vit.")
                and k.rsplit(".", 1)[1] in ("bq", "bk", "bv", "bo", "b_up", "b_down")}
    problems = [f"missing {k}" for k in want if k not in flat and k not in optional]
    problems += [f"unexpected {k}" for k in flat if k not in want]
    problems += [f"{k}: shape {tuple(flat[k].shape)} != {want[k]}" for k in flat
                 if k in want and tuple(flat[k].shape) != want[k]]
    if problems:
        raise ValueError("parameter set does not match the configuration:\n  "
                         + "\n  ".join(problems[:40]))


def save_params(params, path) -> None:
    from safetensors.torch import save_file
    flat = {k: t.detach().to("cpu").contiguous() for k, t in flatten(params).items()}
    save_file(flat, str(path))


def load_params(path, cfg: Optional[SmolVLAConfig] = None, device="cpu"):
    """Load a parameter file written by ``save_params`` (local path)."""
    from safetensors.torch import load_file
    path = pathlib.Path(path)
    if not path.is_file():
        raise FileNotFoundError(f"no parameter file at {path} (local paths only)")
    params = unflatten(load_file(str(path), device=str(device)))
    if cfg is not None:
        check_params(params, cfg)
    return params


# ------------------------------------------------ HF / LeRobot-style names ---
VLM = "model.vlm_with_expert.vlm.model."
EXPERT = "model.vlm_with_expert.lm_expert."


def hf_name_map(cfg: SmolVLAConfig) -> Dict[str, Tuple[str, bool]]:
    """HF-style name -> (own key, transpose).  ``nn.Linear`` weights are
    ``[out, in]`` there and ``[in, out]`` here; conv kernels, embeddings, norms
    and biases keep their layout."""
    m: Dict[str, Tuple[str, bool]] = {
        VLM + "vision_model.embeddings.patch_embedding.weight": ("patch.kernel", False),
        VLM + "vision_model.embeddings.patch_embedding.bias": ("patch.bias", False),
        VLM + "vision_model.embeddings.position_embedding.weight": ("patch.pos_emb", False),
        VLM + "connector.modality_projection.proj.weight": ("connector.W", True),
        VLM + "text_model.embed_tokens.weight": ("embed", False),
        "model.state_proj.weight": ("state.W", True),
        "model.action_in_proj.weight": ("expert_io.W_action_in", True),
        "model.action_in_proj.bias": ("expert_io.b_action_in", False),
        "model.action_time_mlp_in.weight": ("expert_io.W_time_in", True),
        "model.action_time_mlp_in.bias": ("expert_io.b_time_in", False),
        "model.action_time_mlp_out.weight": ("expert_io.W_time_out", True),
        "model.action_time_mlp_out.bias": ("expert_io.b_time_out", False),
        EXPERT + "norm.weight": ("expert_io.W_exp_norm", False),
        "model.action_out_proj.weight": ("expert_io.W_action_out", True),
    }
    for i in range(cfg.vit.layers):
        h, o = f"{VLM}vision_model.encoder.layers.{i}.", f"vit.{i}."
        for proj, w, b in (("q_proj", "Wq", "bq"), ("k_proj", "Wk", "bk"),
                           ("v_proj", "Wv", "bv"), ("out_proj", "Wo", "bo")):
            m[h + f"self_attn.{proj}.weight"] = (o + w, True)
            m[h + f"self_attn.{proj}.bias"] = (o + b, False)
        m[h + "mlp.fc1.weight"], m[h + "mlp.fc1.bias"] = (o + "W_up", True), (o + "b_up", False)
        m[h + "mlp.fc2.weight"], m[h + "mlp.fc2.bias"] = (o + "W_down", True), (o + "b_down", False)
        for n in ("1", "2"):
            m[h + f"layer_norm{n}.weight"] = (o + f"W_norm_{n}", False)
            m[h + f"layer_norm{n}.bias"] = (o + f"b_norm_{n}", False)

    def dec(h, o, cross):
        m[h + "self_attn.q_proj.weight"] = (o + "Wq", True)
        m[h + "self_attn.k_proj.weight"] = (o + ("Wk_cross" if cross else "Wk"), True)
        m[h + "self_attn.v_proj.weight"] = (o + ("Wv_cross" if cross else "Wv"), True)
        m[h + "self_attn.o_proj.weight"] = (o + "Wo", True)
        for proj, w in (("gate_proj", "W_gate"), ("up_proj", "W_up"), ("down_proj", "W_down")):
            m[h + f"mlp.{proj}.weight"] = (o + w, True)
        m[h + "input_layernorm.weight"] = (o + "W_norm_1", False)
        m[h + "post_attention_layernorm.weight"] = (o + "W_norm_2", False)
    for i in range(cfg.prefix_layers):
        dec(f"{VLM}text_model.layers.{i}.", f"prefix.{i}.", False)
    for i in range(cfg.expert_layers):
        dec(f"{EXPERT}layers.{i}.", f"expert.{i}.", cfg.is_cross(i))
    return m


def from_hf_state_dict(sd: Dict[str, torch.Tensor], cfg: SmolVLAConfig,
                       name_map: Optional[Dict[str, Tuple[str, bool]]] = None,
                       dtype=BF16) -> Tuple[dict, List[str]]:
    """Map an HF-style state dict to the pipeline's params; returns
    ``(params, ignored_keys)``.  Raises ValueError if a tensor the pipeline
    needs is missing or mis-shaped."""
    name_map = hf_name_map(cfg) if name_map is None else name_map
    flat, ignored = {}, []
    for name, t in sd.items():
        if name not in name_map:
            ignored.append(name)
            continue
        key, transpose = name_map[name]
        t = t.t() if transpose else t
        flat[key] = t.to(dtype).contiguous()
    params = unflatten(flat)
    check_params(params, cfg)
    return params, sorted(ignored)


def to_hf_state_dict(params, cfg: SmolVLAConfig,
                     name_map: Optional[Dict[str, Tuple[str, bool]]] = None):
    """Inverse of ``from_hf_state_dict`` (export, and the mapping's own test)."""
    name_map = hf_name_map(cfg) if name_map is None else name_map
    flat = flatten(params)
    out = {}
    for name, (key, transpose) in name_map.items():
        if key in flat:
            t = flat[key]
            out[name] = (t.t() if transpose else t).contiguous()
    return out


def load_hf_safetensors(paths, cfg: SmolVLAConfig, **kw):
    """``from_hf_state_dict`` over one or more local ``.safetensors`` files."""
    from safetensors.torch import load_file
    if isinstance(paths, (str, pathlib.Path)):
        paths = [paths]
    sd = {}
    for p in paths:
        p = pathlib.Path(p)
        if not p.is_file():
            raise FileNotFoundError(f"no checkpoint shard at {p} (local paths only)")
        sd.update(load_file(str(p)))
    return from_hf_state_dict(sd, cfg, **kw)
