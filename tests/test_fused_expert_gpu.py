"""The fused action expert (one persistent launch for the whole 10-step
flow-matching loop, ``svla_expert_*``) against the oracle and against the
layer-by-layer engine on the same seeded weights and inputs.

Tolerances: final fp32 actions max |d| <= 5e-2 absolute (as every chunk
test); fused vs layer-by-layer engine <= 2e-2 (same kernels' arithmetic
except the attention softmax, normalised before its bf16 rounding here as in
the reference torch module, and K split differently over waves).  Graph
replays are bit-identical, and so are the whole-chip and one-XCD teams (each
unit's arithmetic does not depend on which CU runs it)."""

import pytest
import torch

import oracle.smolvla_ref as ref
from smolvla.config import SmolVLAConfig, small_config
from smolvla.params import smolvla_inputs, smolvla_params

pytestmark = pytest.mark.gpu
ACTION_ATOL = 5e-2
ENGINE_ATOL = 2e-2


def _engine(cfg, P, batch, **kw):
    from smolvla.pipeline import SmolVLAEngine
    return SmolVLAEngine(cfg, P, batch=batch, **kw)


@pytest.mark.parametrize("batch", [1, 2])
def test_small_config_fused_expert(batch):
    cfg = small_config()
    P = smolvla_params(cfg, seed=31, norm_init="random")
    inputs = smolvla_inputs(cfg, batch=batch, seed=32)
    dev = [t.cuda() for t in inputs]
    eng = _engine(cfg, P, batch, fused_expert=True)
    print(f"small config batch {batch}: fused expert", flush=True)
    got = eng.run(*dev).cpu()
    assert eng.fx.status() == 0
    want = ref.smolvla_chunk(*inputs, P, cfg)
    layered = _engine(cfg, P, batch, fused_expert=False).run(*dev).cpu()
    e_ref = (got - want).abs().max().item()
    e_eng = (got - layered).abs().max().item()
    print(f"small batch {batch}: fused vs oracle {e_ref:.3e}, vs layered engine {e_eng:.3e}")
    assert torch.isfinite(got).all()
    assert e_ref <= ACTION_ATOL and e_eng <= ENGINE_ATOL


@pytest.fixture(scope="module")
def full1():
    cfg = SmolVLAConfig()
    P = smolvla_params(cfg, seed=0, norm_init="random")
    inputs = smolvla_inputs(cfg, batch=1, seed=1)
    with torch.inference_mode():
        want = ref.smolvla_chunk(*inputs, P, cfg)
    return cfg, P, inputs, want


def test_full_config_fused_expert_batch1(full1):
    cfg, P, inputs, want = full1
    dev = [t.cuda() for t in inputs]
    eng = _engine(cfg, P, 1)
    assert eng.fx is not None                      # the batch-1 default
    print("full config batch 1: fused expert", flush=True)
    got = eng.run(*dev).cpu()
    assert eng.fx.status() == 0
    layered = _engine(cfg, P, 1, fused_expert=False).run(*dev).cpu()
    e_ref = (got - want).abs().max().item()
    e_eng = (got - layered).abs().max().item()
    print(f"full batch 1: fused vs oracle {e_ref:.3e}, vs layered engine {e_eng:.3e}")
    assert torch.isfinite(got).all()
    assert e_ref <= ACTION_ATOL and e_eng <= ENGINE_ATOL
    # graph replays with eager work between them: bit-identical
    first = got.clone()
    for i in range(3):
        torch.randn(1000, device="cuda").sum().item()
        again = eng.run(*dev).cpu()
        assert torch.equal(again, first), f"replay {i} differs"
    assert eng.fx.status() == 0


def test_fused_expert_one_xcd_team_matches(full1):
    cfg, P, inputs, _ = full1
    dev = [t.cuda() for t in inputs]
    a = _engine(cfg, P, 1, expert_team_xcd=-1).run(*dev).cpu()
    eng = _engine(cfg, P, 1, expert_team_xcd=0)
    print("full config batch 1: fused expert on one XCD", flush=True)
    b = eng.run(*dev).cpu()
    assert eng.fx.status() == 0
    assert torch.equal(a, b)
