"""The allocation-free GEMM entry point ``svla_linear_scratch_bf16`` (split-K
partials in a static device array) against ``svla_linear_bf16`` (allocated
workspace), called through the C-ABI: bit-identical outputs on two calls in a
row, the second with a smaller problem (whatever the first left in the
scratch must not matter), a problem that does not split, and a split that
needs more scratch than the array holds (SVLA_ENOSPC, nothing launched).

The automatic tile choice no longer splits K for dense problems (their
32-row tiles fill the chip without it), so the split cases force the skinny
tiles that do (svla_gemm_set_tile, both entry points alike)."""

import ctypes

import pytest
import torch

from smolvla import _lib

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _gemm(entry, a, w, out, res=None, norm=None):
    M, K = a.shape
    N = w.shape[0]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return getattr(_lib.load(), entry)(
        _ptr(a), a.stride(0), _ptr(w), w.stride(0), None, None, _ptr(res),
        res.stride(0) if res is not None else 0, _ptr(out), out.stride(0), M, N, K,
        ctypes.c_float(1.0), 0, 0, _ptr(norm), ctypes.c_float(1e-5), stream)


def _case(M, N, K, seed, with_res=True, with_norm=True):
    g = torch.Generator(device="cuda").manual_seed(seed)
    a = torch.randn(M, K, device="cuda", generator=g).to(BF16)
    w = (0.02 * torch.randn(N, K, device="cuda", generator=g)).to(BF16)
    res = torch.randn(M, N, device="cuda", generator=g).to(BF16) if with_res else None
    norm = (1 + 0.1 * torch.randn(K, device="cuda", generator=g)).to(BF16) if with_norm else None
    return a, w, res, norm


class _forced_tile:
    """svla_gemm_set_tile(tile) for the duration of a with-block."""

    def __init__(self, tile):
        self.tile = tile

    def __enter__(self):
        assert _lib.load().svla_gemm_set_tile(self.tile) == 0

    def __exit__(self, *exc):
        _lib.load().svla_gemm_set_tile(-1)


def _both(M, N, K, seed, **kw):
    a, w, res, norm = _case(M, N, K, seed, **kw)
    out_ref = torch.full((M, N), float("nan"), device="cuda", dtype=BF16)
    out_scr = torch.full((M, N), float("nan"), device="cuda", dtype=BF16)
    print(f"no-alloc GEMM {M}x{N}x{K}", flush=True)
    assert _gemm("svla_linear_bf16", a, w, out_ref, res, norm) == 0
    assert _gemm("svla_linear_scratch_bf16", a, w, out_scr, res, norm) == 0
    torch.cuda.synchronize()
    return out_ref, out_scr


def test_scratch_entry_point_matches_linear_twice_then_smaller():
    # on the 32-column skinny tile 50x720x2048 splits K over 4 workgroups per
    # tile, 20x320x1536 over 3
    for (M, N, K), seed in (((50, 720, 2048), 1), ((20, 320, 1536), 2)):
        with _forced_tile(5):
            ref, got = _both(M, N, K, seed)
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref), (M, N, K)


def test_scratch_entry_point_unsplit_and_plain():
    for (M, N, K), seed in (((300, 512, 768), 3), ((64, 256, 512), 4)):
        ref, got = _both(M, N, K, seed, with_res=False, with_norm=False)
        assert torch.equal(got, ref), (M, N, K)


def test_scratch_too_small_is_enospc():
    # 256x2048x2048 on the 64-column skinny tile: 128 tiles of 64x64 split
    # twice need 1.06M partial floats
    a, w, res, norm = _case(256, 2048, 2048, 5, with_res=False, with_norm=False)
    out = torch.zeros(256, 2048, device="cuda", dtype=BF16)
    with _forced_tile(4):
        assert _gemm("svla_linear_scratch_bf16", a, w, out) == -28
        torch.cuda.synchronize()
        assert (out == 0).all()                   # nothing was launched
        ref = torch.zeros_like(out)
        assert _gemm("svla_linear_bf16", a, w, ref) == 0   # the allocated workspace holds it
