"""Observation pre-processing in front of the pipeline.

* camera frames: uint8 RGB ``[h, w, 3]`` -> bf16 ``[3, 512, 512]`` in [-1, 1]
  on the GPU (``ops.image_to_bf16``: aspect-preserving bilinear resize, black
  padding);
* robot state: zero-padded to the model's 32 dims, as the reference's demo
  caller does (simulation/demo_cpu.py:274-277);
* language: token ids padded / truncated to the 48 prompt positions the prefix
  holds; ids come from any tokenizer with an ``encode`` method (the
  ``tokenizers`` library's ``Tokenizer`` loaded from a local file -- nothing
  is fetched), then embedded by the pipeline (create_text_emb, vla/vla.py:169-174).
"""

from __future__ import annotations

import numpy as np
import torch

from . import ops


def images(frames, out_size=512, device="cuda"):
    """``frames``: uint8 array/tensor ``[cams, h, w, 3]`` or ``[B, cams, h, w, 3]``
    -> bf16 ``[B, cams, 3, S, S]`` on the GPU."""
    t = torch.as_tensor(frames)
    if t.dim() == 4:
        t = t.unsqueeze(0)
    if t.dim() != 5:
        raise ValueError("frames must be [cams, h, w, 3] or [B, cams, h, w, 3]")
    B, C = t.shape[:2]
    out = ops.image_to_bf16(t.reshape(B * C, *t.shape[2:]).to(device), out_size)
    return out.view(B, C, 3, out_size, out_size)


def pad_state(state, dim=32):
    """Zero-pad (or reject) a robot state to ``dim`` values, fp32 ``[B, dim]``."""
    s = torch.as_tensor(np.asarray(state, dtype=np.float32))
    if s.dim() == 1:
        s = s.unsqueeze(0)
    if s.shape[-1] > dim:
        raise ValueError(f"state has {s.shape[-1]} values, the model takes at most {dim}")
    out = torch.zeros(s.shape[0], dim, dtype=torch.float32)
    out[:, :s.shape[-1]] = s
    return out


def token_ids(texts, tokenizer, length=48, pad_id=0):
    """Encode ``texts`` (str or list of str) with ``tokenizer.encode`` and
    pad / truncate every row to ``length`` ids: int64 ``[B, length]``."""
    if isinstance(texts, str):
        texts = [texts]
    rows = []
    for t in texts:
        enc = tokenizer.encode(t)
        ids = list(getattr(enc, "ids", enc))[:length]
        rows.append(ids + [pad_id] * (length - len(ids)))
    return torch.tensor(rows, dtype=torch.int64)
