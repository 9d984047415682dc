"""Shared plumbing for the reference-signature layer functions."""

from __future__ import annotations

import torch

BF16 = torch.bfloat16
_PREP_KEY = "__svla_prepared__"


def to_device(x):
    """Accept a CPU/GPU tensor or a numpy array; return (bf16 GPU tensor,
    function mapping a GPU result back to the caller's device)."""
    if not torch.is_tensor(x):
        x = torch.as_tensor(x)
    if x.is_cuda:
        return x.to(BF16), (lambda t: t)
    dev = torch.device("cuda")
    return x.to(device=dev, dtype=BF16), (lambda t: t.cpu())


def as_batched(x):
    """[S, H] -> [1, S, H]; returns (tensor3d, squeeze_back flag)."""
    if x.dim() == 2:
        return x.unsqueeze(0), True
    return x, False


def prepared(params, prep_fn):
    """Pack reference-layout weights once per params dict (cached in it)."""
    cache = params.get(_PREP_KEY)
    if cache is None or cache[0] is not prep_fn:
        cache = (prep_fn, prep_fn(params, torch.device("cuda")))
        params[_PREP_KEY] = cache
    return cache[1]
