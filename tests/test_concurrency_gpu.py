"""Two engines on two streams of one device at the same time.

What stays shared per device by design is excluded: the skinny GEMMs'
split-K workspace (split turned off here) and the persistent fused expert,
which needs every CU of the device (layered expert here).  Everything else --
the pipelined GEMMs, attention, norms -- must then be stream-safe: each
engine's chunk, replayed concurrently with the other's, equals its chunk run
alone, bit for bit.  (A race in the pipelined kernels' LDS refills, now
fixed, made concurrent runs corrupt prefix rows.)
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_two_engines_on_two_streams_match_serial():
    from smolvla import _lib
    from smolvla.config import SmolVLAConfig
    from smolvla.params import smolvla_inputs, smolvla_params
    from smolvla.pipeline import SmolVLAEngine

    lib = _lib.load()
    cfg = SmolVLAConfig()
    P = smolvla_params(cfg, seed=0)
    assert lib.svla_gemm_set_split(1) == 0
    try:
        engines = []
        for seed in (2, 3):
            e = SmolVLAEngine(cfg, P, batch=1, fused_expert=False)
            e.load_inputs(*smolvla_inputs(cfg, 1, seed=seed, device="cuda"))
            e.capture()
            engines.append(e)
        refs = []
        for e in engines:  # alone
            e.step()
            torch.cuda.synchronize()
            refs.append(e.x_t.clone())
        cur = torch.cuda.current_stream()
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        for rnd in range(8):
            for s in streams:
                s.wait_stream(cur)
            for e, s in zip(engines, streams):
                with torch.cuda.stream(s):
                    e.step()
            for s in streams:
                cur.wait_stream(s)
            torch.cuda.synchronize()
            for i, (e, ref) in enumerate(zip(engines, refs)):
                assert torch.equal(e.x_t, ref), f"engine {i} differs in concurrent round {rnd}"
    finally:
        lib.svla_gemm_set_split(-1)
