"""Parameter files on the GPU path: seeded parameters written to a local
safetensors file (the build's own layout, and HF-style names with nn.Linear
[out, in] weights), loaded back with ``weights.load_params`` /
``weights.load_hf_safetensors`` and run through the engine.  The chunk must
be bit-identical to the engine on the original parameters and within the
action tolerance of the oracle on them (parameter naming and transposition
of vla/text_encoder_bf16.py:601-611)."""

import pytest
import torch
from safetensors.torch import save_file

import oracle.smolvla_ref as ref
from smolvla import weights
from smolvla.config import small_config
from smolvla.params import smolvla_inputs, smolvla_params

pytestmark = pytest.mark.gpu
ACTION_ATOL = 5e-2


@pytest.fixture(scope="module")
def case():
    from smolvla.pipeline import SmolVLAEngine
    cfg = small_config()
    P = smolvla_params(cfg, seed=21, norm_init="random")
    inputs = smolvla_inputs(cfg, batch=2, seed=22)
    base = SmolVLAEngine(cfg, P, batch=2).run(*[t.cuda() for t in inputs]).cpu()
    want = ref.smolvla_chunk(*inputs, P, cfg)
    return cfg, P, inputs, base, want


def _run(cfg, params, inputs):
    from smolvla.pipeline import SmolVLAEngine
    return SmolVLAEngine(cfg, params, batch=2).run(*[t.cuda() for t in inputs]).cpu()


def test_engine_on_own_layout_file(case, tmp_path):
    cfg, P, inputs, base, want = case
    path = tmp_path / "smolvla.safetensors"
    weights.save_params(P, path)
    got = _run(cfg, weights.load_params(path, cfg), inputs)
    assert torch.equal(got, base)
    assert (got - want).abs().max().item() <= ACTION_ATOL


def test_engine_on_hf_named_file(case, tmp_path):
    cfg, P, inputs, base, want = case
    sd = weights.to_hf_state_dict(P, cfg)
    linear = [k for k in sd if k.endswith("proj.weight")]
    assert linear, "HF-style names expected"
    path = tmp_path / "model.safetensors"
    save_file(sd, str(path))
    loaded, ignored = weights.load_hf_safetensors(path, cfg)
    assert ignored == []
    got = _run(cfg, loaded, inputs)
    assert torch.equal(got, base)
    assert (got - want).abs().max().item() <= ACTION_ATOL
