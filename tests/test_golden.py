"""Golden fixtures (``tests/golden/``) against the CPU oracle.

The fixtures were written by ``tests/golden/make_golden.py`` from the oracle
after ``tests/test_oracle_pin.py`` pinned it.  Here the oracle recomputes
every fixture from its stored inputs (weights regenerated from the stated
seeds) and must reproduce the stored outputs: a change to the oracle, to the
seeded generators or to torch's CPU numerics shows up as a mismatch.
Tolerance: bf16 tensors within one bf16 ulp of the stored value per element
(relative 2^-7, CPU GEMM blocking may differ between hosts), fp32 actions
within 1e-3 absolute.
"""

import json
import pathlib
import sys

import numpy as np
import pytest
import torch

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_golden  # noqa: E402

BF16 = torch.bfloat16


def _close(got, want):
    if want.dtype == BF16:
        torch.testing.assert_close(got.float(), want.float(), rtol=2 ** -7, atol=1e-6)
    elif want.dtype.is_floating_point:
        torch.testing.assert_close(got, want, rtol=0, atol=1e-3)
    else:
        assert torch.equal(got, want)


def test_manifest_matches_files():
    man = json.loads((GOLDEN / "manifest.json").read_text())
    assert set(man["fixtures"]) == set(make_golden.FIXTURES)
    for name, meta in man["fixtures"].items():
        with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
            assert set(z.files) == set(meta["arrays"])
            for k, (shape, dtype) in meta["arrays"].items():
                assert list(z[k].shape) == shape and str(z[k].dtype) == dtype, (name, k)


@pytest.mark.parametrize("name", sorted(make_golden.FIXTURES))
def test_oracle_reproduces_golden(name):
    stored = make_golden.load(name)
    with torch.inference_mode():
        fresh, _ = make_golden.FIXTURES[name]()
    assert set(fresh) == set(stored)
    for k in stored:
        assert fresh[k].shape == stored[k].shape, (name, k)
        _close(fresh[k], stored[k])


def test_golden_invariants():
    """Properties the stored outputs must have whatever produced them."""
    h = make_golden.load("harness")
    p = h["ms_p"].float()
    rows = torch.arange(8)[:, None] + 37
    assert (p[torch.arange(128)[None, :] > rows] == 0).all()       # masked exactly 0
    assert torch.allclose(p.sum(-1), torch.ones(8), atol=2e-2)     # rows sum to 1 (bf16)
    assert torch.allclose(h["sm_p"].float().sum(-1), torch.ones(4), atol=2e-2)
    # RoPE preserves the norm of every (d, d+32) pair and is the identity at pos 0
    x, y = h["rp_x"], h["rp_y"]
    nx = x[:, :32] ** 2 + x[:, 32:] ** 2
    ny = y[:, :32] ** 2 + y[:, 32:] ** 2
    torch.testing.assert_close(ny, nx, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(y[0], x[0])
    # RMSNorm with gain w: y / w has unit RMS per row
    r = (h["rn_y"].float() / h["rn_w"].float()).pow(2).mean(-1).sqrt()
    torch.testing.assert_close(r, torch.ones(16), rtol=2e-2, atol=0)
    # the chunk: finite actions, one per (sample, step, action dim)
    c = make_golden.load("small_chunk")
    assert c["actions"].shape == (2, 10, 32) and torch.isfinite(c["actions"]).all()
