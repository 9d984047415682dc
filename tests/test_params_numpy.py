"""The reference builds ``params`` as numpy arrays (``p[name].T.astype(NP_DTYPE)``
with ``NP_DTYPE = ml_dtypes.bfloat16``, vla/text_encoder_bf16.py:55, 599-609)
and passes them, with numpy inputs, straight to the layer functions.  CPU
checks of that boundary: array conversion and the packed-weight cache kept
outside the caller's dict (no GPU needed: the cache is exercised with a
CPU-only preparation function)."""

import numpy as np
import pytest
import torch

from smolvla.layers import host_tensor, is_bf16_bits
from smolvla.vla import _common


def test_bf16_words_are_read_bit_for_bit():
    vals = torch.tensor([1.0, -2.5, 3.140625, 1e-3, -0.0], dtype=torch.bfloat16)
    words = vals.view(torch.int16).numpy().view(np.uint16)
    assert is_bf16_bits(words)
    got = host_tensor(words)
    assert got.dtype == torch.bfloat16 and torch.equal(got.view(torch.int16), vals.view(torch.int16))


def test_transposed_fp32_arrays_keep_values():
    w = np.random.default_rng(0).standard_normal((6, 4)).astype(np.float32)
    wt = w.T                                  # the reference's [in, out] view of nn.Linear.weight
    assert not wt.flags["C_CONTIGUOUS"]
    got = host_tensor(wt)
    assert got.dtype == torch.float32 and torch.equal(got, torch.from_numpy(w.T.copy()))
    assert host_tensor(np.arange(5)).dtype == torch.int64     # token ids stay integers
    with pytest.raises(TypeError):
        host_tensor(np.array(["a"]))


class _CountingPrep:
    def __init__(self):
        self.calls = 0

    def __call__(self, p, device):
        self.calls += 1
        return {k: host_tensor(v).float().sum().item() for k, v in p.items()}


def test_prepared_cache_stays_outside_the_dict_and_follows_updates():
    prep = _CountingPrep()
    params = {"Wq": np.ones((4, 3), np.float32), "Wo": torch.ones(3, 4)}
    keys = set(params)
    a = _common.prepared(params, prep)
    b = _common.prepared(params, prep)
    assert prep.calls == 1 and a is b
    assert set(params) == keys                              # nothing added to the caller's dict
    params["Wq"][0, 0] = 5.0                                # numpy in-place update
    c = _common.prepared(params, prep)
    assert prep.calls == 2 and c["Wq"] == 16.0
    params["Wo"].mul_(2.0)                                  # torch in-place update
    d = _common.prepared(params, prep)
    assert prep.calls == 3 and d["Wo"] == 24.0
    params["Wo"] = torch.ones(3, 4)                         # replaced object
    _common.prepared(params, prep)
    assert prep.calls == 4
    _common.prepared(dict(params), prep)                    # another dict: its own entry
    assert prep.calls == 5
    assert _common.prepared(params, prep)["Wo"] == 12.0 and prep.calls == 5
