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
LAYER_RTOL = 1e-2      # north star: max relative error per layer output
CHAIN_RTOL = 3e-2      # 16 stacked layers from the oracle's own step input (as for the stacks)


def _rel(got, want):
    """max |got - want| / max |want| in fp32."""
    got, want = got.float(), want.float()
    return ((got - want).abs().max() / want.abs().max()).item()


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


def test_full_config_fused_expert_per_layer(full1):
    """Every layer of the fused expert (the batch-1 default path) against the
    oracle's layer on the same input: the fused launch's per-layer outputs
    are read back from its workspace (``svla_expert_trace_offset``), as the
    reference checks each expert layer on its own
    (vla/action_expert_bf16.py:848-906).  Steps 0 and 9; plus the step-0
    expert input against the oracle's action/time embedding, and the 16
    layers chained from the oracle's own step-0 input.  The layer-by-layer
    kernels (the batch-32 path) run on the same inputs to the same bound."""
    cfg, P, inputs, _ = full1
    dev = [t.cuda() for t in inputs]
    eng = _engine(cfg, P, 1)
    print("full config batch 1: fused expert, per layer", flush=True)
    eng.run(*dev)
    e, L, Lc = cfg.expert, cfg.chunk, cfg.prefix_len
    ckv = {i: (ck.cpu().reshape(1, Lc, -1), cv.cpu().reshape(1, Lc, -1))
           for i, (ck, cv) in eng.cross.items()}
    from smolvla import layers
    worst = worst_l = 0.0
    with torch.inference_mode():
        for step in (0, cfg.num_steps - 1):
            for li in range(cfg.expert_layers):
                x = eng.fx.trace(step, li).cpu().view(1, L, e.hidden)
                got = eng.fx.trace(step, li + 1).cpu().view(1, L, e.hidden)
                lp = P["expert"][li]
                if cfg.is_cross(li):
                    want = ref._cross_with_projected(x, *ckv[li], lp, e)
                else:
                    want = ref.expert_self_block(x, lp, e)
                err = _rel(got, want)
                worst = max(worst, err)
                assert err <= LAYER_RTOL, f"step {step} layer {li}: {err:.3e}"
                # the layer-by-layer kernels (the batch-32 path) on the same
                # real expert activations
                xl = x.reshape(L, e.hidden).cuda().clone()
                if cfg.is_cross(li):
                    ck, cv = eng.cross[li]
                    layers.cross_layer(xl, ck, cv, eng.expert[li], e, 1, L, Lc, eng.rope_expert)
                else:
                    layers.decoder_layer(xl, eng.expert[li], e, 1, L, eng.rope_expert, "causal")
                err_l = _rel(xl.cpu().view(1, L, e.hidden), want)
                worst_l = max(worst_l, err_l)
                assert err_l <= LAYER_RTOL, f"layered, step {step} layer {li}: {err_l:.3e}"
        # step 0's expert input: action_in / time MLP of the noise at t = 1
        h0 = ref.expert_input(inputs[3].float(), 1.0, P, cfg)
        e_in = _rel(eng.fx.trace(0, 0).cpu().view(1, L, e.hidden), h0)
        assert e_in <= LAYER_RTOL, e_in
        # the oracle's own chain from its step-0 input
        h = h0
        for li in range(cfg.expert_layers):
            lp = P["expert"][li]
            h = (ref._cross_with_projected(h, *ckv[li], lp, e) if cfg.is_cross(li)
                 else ref.expert_self_block(h, lp, e))
            e_ch = _rel(eng.fx.trace(0, li + 1).cpu().view(1, L, e.hidden), h)
            assert e_ch <= CHAIN_RTOL, f"chain layer {li}: {e_ch:.3e}"
    print(f"fused expert per layer: worst {worst:.3e} (layer-by-layer kernels {worst_l:.3e}), "
          f"input {e_in:.3e}, chain end {e_ch:.3e}")


def test_run_raises_on_expert_status():
    """A non-zero status word makes the engine raise (the word planted from
    the host into the workspace after a good run; no kernel is made to fail)."""
    cfg = small_config()
    P = smolvla_params(cfg, seed=31, norm_init="random")
    dev = [t.cuda() for t in smolvla_inputs(cfg, batch=1, seed=32)]
    eng = _engine(cfg, P, 1, fused_expert=True)
    eng.run(*dev)
    eng.check()
    fx = eng.fx
    off = fx.plan.status - fx.workspace.data_ptr()
    fx.workspace[off:off + 4].copy_(torch.tensor([1, 0, 0, 0], dtype=torch.uint8))
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="status 1"):
        eng.check()
    real = fx.status
    fx.status = lambda: 2                      # a run() whose expert reports a team failure
    try:
        with pytest.raises(RuntimeError, match="status 2"):
            eng.run(*dev)
    finally:
        fx.status = real
    eng.run(*dev)                              # the next good run clears the word
    assert fx.status() == 0


def test_expert_gives_up_loudly_with_a_tiny_spin_limit():
    """The failure path itself, forced from the host: with a spin limit of
    one poll, some phase wait gives up; every workgroup still leaves (the
    launch returns), the status word reads 1 and the actions are NaN.  A
    later run with the normal limit is correct again."""
    cfg = small_config()
    P = smolvla_params(cfg, seed=31, norm_init="random")
    dev = [t.cuda() for t in smolvla_inputs(cfg, batch=1, seed=32)]
    eng = _engine(cfg, P, 1, fused_expert=True, use_graph=False)
    good = eng.run(*dev).cpu()
    fx = eng.fx
    limit = fx.plan.spin_limit
    assert limit > 1000
    fx.plan.spin_limit = 1
    print("fused expert with spin limit 1 (forced give-up)", flush=True)
    try:
        eng.load_inputs(*dev)
        eng.step()
        torch.cuda.synchronize()
        bad = eng.x_t.cpu()
        assert fx.status() == 1
        assert torch.isnan(bad).all()
        with pytest.raises(RuntimeError, match="status 1"):
            eng.check()
    finally:
        fx.plan.spin_limit = limit
    again = eng.run(*dev).cpu()
    assert torch.equal(again, good)


def test_phase_stamps(full1):
    """plan.stamps: one start and one arrival clock stamp per phase from the
    team's first workgroup, increasing through the launch (a phase starts
    after the previous one's stamps), one per named phase; the run's actions
    are bit-identical to a run without stamps."""
    cfg, P, inputs, _ = full1
    dev = [t.cuda() for t in inputs]
    eng = _engine(cfg, P, 1, use_graph=False)
    print("full config batch 1: fused expert with phase stamps", flush=True)
    want = eng.run(*dev).cpu()
    eng.x_t.copy_(eng.in_noise.view(-1, cfg.action_dim))
    st = eng.fx.phase_stamps()
    assert eng.fx.status() == 0
    got = eng.x_t.view(1, cfg.chunk, cfg.action_dim).cpu()
    assert torch.equal(got, want)
    kinds = eng.fx.phase_kinds()
    assert st.shape == (len(kinds), 2) == (eng.fx.plan.n_phases, 2)
    flat = st.reshape(-1)
    assert (flat > 0).all() and (flat[1:] >= flat[:-1]).all()
    assert kinds[0] == "V^T transposes" and kinds[-1] == "action out + Euler"
    span_ms = (st[-1, 1] - st[0, 0]).item() * 10 / 1e6
    assert 0.5 < span_ms < 100, span_ms
