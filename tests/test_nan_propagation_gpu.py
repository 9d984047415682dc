"""Failure propagation, forced from the host (no kernel is made to fault).

The reference patches its NPU SiLU on the CPU where the Taylor-series kernel
overflows (|x| > 2.5) and where NaN / Inf appear (vla/text_encoder_bf16.py:
545-579, vla/action_expert_bf16.py:604-626).  Here: the SiLU paths stay
finite and exact for any gate magnitude (nothing to patch), and a NaN planted
in one input reaches exactly the outputs that depend on it -- the same rows
of a norm or a GEMM, the same column for a weight, the queries that see a
key, and, end to end, only the sample it was planted in (the other sample's
actions are bit-identical to a clean run)."""

import pytest
import torch

import oracle.smolvla_ref as ref
from smolvla.config import small_config
from smolvla.params import smolvla_inputs, smolvla_params

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16
NAN = float("nan")


@pytest.fixture(scope="module")
def ops():
    from smolvla import _lib
    from smolvla import ops as _ops
    _lib.load()
    return _ops


def randn(seed, *shape, std=1.0):
    return (torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * std).to(BF16)


def test_silu_paths_finite_for_large_gates(ops):
    """The gate range where the reference's SiLU kernel overflows: the
    harness SiLU and the fused gate|up SiLU*up epilogue stay finite and follow
    torch (fp32 SiLU, bf16 out) within one bf16 ulp."""
    x = torch.linspace(-3000.0, 3000.0, 8192).to(BF16)
    got = ops.silu(x.cuda()).cpu()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got.float(), ref.silu(x.float()).to(BF16).float(), atol=1e-2,
                               rtol=2 ** -7)
    a = randn(1, 50, 720, std=40.0)                  # gate values of a few hundred
    wg, wu = randn(2, 720, 2048, std=0.5), randn(3, 720, 2048, std=0.02)
    out = ops.linear_silu_mul(a.cuda(), ops.pack_gate_up(wg.cuda(), wu.cuda())).cpu()
    gate = ref.linear(a, wg)
    assert gate.float().abs().max() > 100
    want = ref.silu(gate) * ref.linear(a, wu)
    assert torch.isfinite(out).all()
    assert ((out.float() - want.float()).abs().max() / want.float().abs().max()).item() <= 1e-2


@pytest.mark.parametrize("rows,cols", [(50, 720), (241, 960), (1600, 720)])
def test_nan_row_rmsnorm(ops, rows, cols):
    x = randn(4, rows, cols)
    w = (1 + 0.1 * torch.randn(cols, generator=torch.Generator().manual_seed(5))).to(BF16)
    clean = ops.rmsnorm(x.cuda(), w.cuda(), 1e-5).cpu()
    x[3, 17] = NAN
    got = ops.rmsnorm(x.cuda(), w.cuda(), 1e-5).cpu()
    assert torch.isnan(got[3]).all()
    keep = torch.ones(rows, dtype=torch.bool)
    keep[3] = False
    assert torch.equal(got[keep], clean[keep])


@pytest.mark.parametrize("m,n,k", [(50, 720, 960), (241, 960, 2560), (1600, 720, 2048),
                                   (3072, 768, 768), (7712, 960, 960)])
def test_nan_gemm_reaches_its_row_and_column(ops, m, n, k):
    """A NaN in A[5, k0] reaches output row 5 only; one in W[:, n0] (input
    feature k1 of output column n0) reaches column n0 only; with the residual
    epilogue as the engine runs it.  Row counts cover the engine's tile
    families (skinny / 32-row / pipeline / line-DMA)."""
    a, w, r = randn(6, m, k), randn(7, k, n, std=0.02), randn(8, m, n)
    wp = ops.pack_weight(w.cuda())
    clean = ops.linear(a.cuda(), wp, res=r.cuda()).cpu()
    a_bad = a.clone()
    a_bad[5, k // 3] = NAN
    got = ops.linear(a_bad.cuda(), wp, res=r.cuda()).cpu()
    rows = torch.ones(m, dtype=torch.bool)
    rows[5] = False
    assert torch.isnan(got[5]).all() and torch.equal(got[rows], clean[rows])
    w_bad = w.clone()
    w_bad[k // 2, 13] = NAN
    got = ops.linear(a.cuda(), ops.pack_weight(w_bad.cuda()), res=r.cuda()).cpu()
    cols = torch.ones(n, dtype=torch.bool)
    cols[13] = False
    assert torch.isnan(got[:, 13]).all() and torch.equal(got[:, cols], clean[:, cols])


@pytest.mark.parametrize("lo", [False, True])
@pytest.mark.parametrize("B,S,mask", [(2, 50, "causal"), (2, 241, "prefix_lm")])
def test_nan_attention_key_and_query(ops, B, S, mask, lo):
    """A NaN in key j of (sample 1, KV head 2) reaches exactly the queries
    that see key j in the three query heads of that group (causal: i >= j;
    prefix-LM: every query for a prefix key); a NaN query reaches only its own
    output row of its head.  Plain and fp32-remainder forms."""
    hq, hkv = 15, 5
    prefix = 240 if mask == "prefix_lm" else 0
    q, k, v = randn(9, B, S, hq * 64), randn(10, B, S, hkv * 64), randn(11, B, S, hkv * 64)
    kw = {}
    if lo:
        kw = dict(q_lo=(randn(12, B, S, hq * 64) * 2 ** -9).cuda(),
                  k_lo=(randn(13, B, S, hkv * 64) * 2 ** -9).cuda())

    def run(qq, kk):
        out = torch.empty(B, S, hq * 64, dtype=BF16, device="cuda")
        ops.attention(qq.cuda(), kk.cuda(), v.cuda(), out, hq, hkv, mask, prefix, **kw)
        return out.cpu().view(B, S, hq, 64)

    clean = run(q, k)
    j = 20
    k_bad = k.clone()
    k_bad[1, j, 2 * 64 + 5] = NAN
    got = run(q, k_bad)
    sees = torch.zeros(B, S, hq, dtype=torch.bool)
    qi = torch.arange(S)
    vis = (qi >= j) | (j < prefix) if mask == "prefix_lm" else qi >= j
    for h in (6, 7, 8):
        sees[1, :, h] = vis
    assert torch.isnan(got[sees]).all()
    assert torch.equal(got[~sees], clean[~sees])
    q_bad = q.clone()
    q_bad[0, 7, 4 * 64 + 3] = NAN
    got = run(q_bad, k)
    only = torch.zeros(B, S, hq, dtype=torch.bool)
    only[0, 7, 4] = True
    assert torch.isnan(got[only]).all() and torch.equal(got[~only], clean[~only])


@pytest.mark.parametrize("fused", [True, False])
def test_nan_pixel_stays_in_its_sample(fused):
    """End to end at batch 2 (small config): a NaN pixel in sample 0's second
    camera makes sample 0's actions NaN and leaves sample 1's bit-identical
    to a clean run -- no kernel (norm, GEMM, attention, connector gather,
    fused or layer-by-layer expert) lets one sample's values into another."""
    from smolvla.pipeline import SmolVLAEngine
    cfg = small_config()
    P = smolvla_params(cfg, seed=51, norm_init="random")
    images, ids, state, noise = smolvla_inputs(cfg, batch=2, seed=52)
    eng = SmolVLAEngine(cfg, P, batch=2, fused_expert=fused)
    clean = eng.run(images.cuda(), ids.cuda(), state.cuda(), noise.cuda()).cpu()
    bad = images.clone()
    bad[0, 1, 2, 10, 33] = NAN
    eng.load_inputs(bad.cuda(), ids.cuda(), state.cuda(), noise.cuda())
    eng.step()
    torch.cuda.synchronize()
    got = eng.x_t.view(2, cfg.chunk, cfg.action_dim).cpu()
    assert torch.isnan(got[0]).all()
    assert torch.equal(got[1], clean[1])
