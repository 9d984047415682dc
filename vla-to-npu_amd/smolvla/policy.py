"""Closed-loop caller: one action per control step, one pipeline pass per chunk.

Mirrors the reference demo loop (simulation/demo_cpu.py:452-469): keep the
current chunk's actions in a buffer; when it is empty, run the whole pipeline
once on the latest observation (camera frames, robot state, prompt) and refill
it with the new ``[chunk, action_dim]`` actions (optionally only their first
``action_dims`` components, as the demo keeps the first 2 for PushT).  The
pipeline here is the batch-1 ``SmolVLAEngine`` (HIP graph), so one refill is one
graph replay; observations are pre-processed on the GPU (``smolvla.preprocess``).
"""

from __future__ import annotations

from collections import deque
from typing import Optional

import numpy as np
import torch

from . import preprocess
from .config import SmolVLAConfig
from .pipeline import SmolVLAEngine


class ChunkPolicy:
    def __init__(self, cfg: SmolVLAConfig, params, action_dims: Optional[int] = None,
                 device="cuda", seed: int = 0, use_graph: bool = True):
        self.cfg = cfg
        self.device = torch.device(device)
        self.engine = SmolVLAEngine(cfg, params, batch=1, device=device, use_graph=use_graph)
        self.action_dims = cfg.action_dim if action_dims is None else action_dims
        self.gen = torch.Generator(device=self.device)
        self.gen.manual_seed(seed)
        self.buffer: deque = deque()
        self.chunks = 0
        self.last_chunk: Optional[np.ndarray] = None

    def reset(self):
        self.buffer.clear()

    def infer_chunk(self, frames, state, lang_ids):
        """One pipeline pass: frames uint8 ``[cams, h, w, 3]`` (or already
        pre-processed bf16 ``[cams, 3, S, S]``), state (any length <= 32),
        lang_ids int ``[48]`` -> fp32 actions ``[chunk, action_dim]``."""
        cfg = self.cfg
        with torch.cuda.device(self.device):
            t = torch.as_tensor(frames)
            if t.dtype == torch.uint8:
                images = preprocess.images(t, cfg.vit.image, device=self.device)
            else:
                images = t.to(device=self.device, dtype=torch.bfloat16).reshape(
                    1, cfg.n_cameras, cfg.vit.channels, cfg.vit.image, cfg.vit.image)
            st = preprocess.pad_state(state, cfg.state_dim).to(self.device)
            ids = torch.as_tensor(lang_ids, dtype=torch.int64).reshape(1, cfg.lang_tokens)
            noise = torch.randn(1, cfg.chunk, cfg.action_dim, generator=self.gen,
                                device=self.device)
            actions = self.engine.run(images, ids.to(self.device), st, noise)
        self.chunks += 1
        return actions[0].cpu().numpy()

    def act(self, frames, state, lang_ids) -> np.ndarray:
        """The next action; runs the pipeline when the chunk buffer is empty."""
        if not self.buffer:
            chunk = self.infer_chunk(frames, state, lang_ids)
            self.last_chunk = chunk
            self.buffer.extend(chunk[:, :self.action_dims])
        return self.buffer.popleft()
