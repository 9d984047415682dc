"""CPU-side checks of the drop-in boundary: ``libsvla.so`` loads, exports every
entry point declared in ``include/svla.h``, and the ctypes table covers them
all (no compute calls: there is no GPU here)."""

import ctypes
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "svla.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(?:int|long)\s+(svla_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "svla_linear_bf16" in syms and "svla_attention_bf16" in syms
    assert len(syms) >= 20


def test_library_exports_every_declared_symbol():
    from smolvla import _lib
    if not _lib.LIB_PATH.exists():
        pytest.fail("libsvla.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"declared but not exported: {missing}"


def test_ctypes_table_matches_header():
    from smolvla import _lib
    assert sorted(_lib.SIGNATURES) == declared_symbols()
    lib = _lib.load()
    assert lib.svla_version() == 200


def test_ops_refuse_cpu_tensors():
    import torch
    from smolvla import ops
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensors"):
        ops.rmsnorm(x, torch.ones(64, dtype=torch.bfloat16), 1e-5)


@pytest.mark.parametrize("m,n,k,tile", [
    (50, 720, 960, 17),      # layered batch-1 expert O: 32x32 small tile
    (50, 720, 2048, 17),     # layered batch-1 expert down (no K split)
    (241, 960, 960, 17),     # batch-1 prefix O
    (241, 960, 2560, 17),    # batch-1 prefix down
    (241, 320, 320, 17),     # batch-1 cross K/V projection
    (256, 4096, 720, 4),     # past 512 small tiles: 64-column skinny tile
    (3072, 768, 3072, 19),   # batch-1 ViT down: 96x96 small tile (256 tiles)
    (3072, 768, 768, 16),    # batch-1 ViT O: 64x64 line-DMA pipeline
    (3072, 3072, 768, 14),   # batch-1 ViT up: 128x64 line-DMA pipeline
    (1600, 720, 960, 9),     # batch-32 expert O: 64x64 pipeline (short K)
    (1600, 720, 2048, 10),   # batch-32 expert down: 128x64 pipeline (long K)
    (7712, 960, 2560, 13),   # batch-32 prefix down: 128x128 line-DMA pipeline
    (7712, 320, 320, 16),    # batch-32 cross K/V projection: 64x64 line-DMA
    (98304, 3072, 768, 8),   # batch-32 ViT up: persistent 256x256 tile
])
def test_gemm_tile_choice(m, n, k, tile):
    """The automatic GEMM tile choice (a host-only query, no GPU call) for
    the shapes the engine runs; numbering as svla_gemm_set_tile."""
    from smolvla import _lib
    lib = _lib.load()
    assert lib.svla_gemm_tile_choice(m, n, k, 0) == tile


@pytest.mark.parametrize("tile,norm,rope", [
    (8, True, False),    # 256x256 pipeline: no fused-norm kernel
    (10, False, True),   # 128x64 pipeline: no paired RoPE epilogue
    (5, False, True),    # 32-column skinny tile: no paired RoPE epilogue
    (17, False, True),   # 32x32 small tile: no paired RoPE epilogue
])
def test_strict_forced_tile_without_kernel_is_einval(tile, norm, rope):
    """A strictly forced tile / epilogue pair that has no kernel returns
    SVLA_EINVAL before any launch (so this runs without a GPU: the pointers
    are never dereferenced)."""
    import ctypes as C
    from smolvla import _lib
    lib = _lib.load()
    fake = C.c_void_p(1 << 20)           # 16-byte aligned, never touched
    assert lib.svla_gemm_set_tile(tile | 0x100) == 0
    try:
        if rope:
            rc = lib.svla_linear_rope_bf16(fake, 64, fake, 64, fake, 128, 64, 128, 64, 64, 64,
                                           fake, fake, None, C.c_float(1e-5), None)
        else:
            rc = lib.svla_linear_bf16(fake, 768, fake, 768, None, None, None, 0, fake, 768, 1024,
                                      768, 768, C.c_float(1.0), 0, 0,
                                      fake if norm else None, C.c_float(1e-5), None)
    finally:
        lib.svla_gemm_set_tile(-1)
    assert rc == -22
    assert lib.svla_gemm_set_tile(20 | 0x100) == -22


def _fake_expert_desc(cfg):
    """An expert descriptor with placeholder (never dereferenced) addresses:
    the plan and the trace offsets are computed on the host alone."""
    from smolvla import _lib
    e = cfg.expert
    layers = (_lib.ExpertLayer * cfg.expert_layers)()
    for i in range(cfg.expert_layers):
        L = layers[i]
        L.cross = int(cfg.is_cross(i))
        L.w_qkv = L.w_o = L.w_gu = L.w_down = L.norm1 = L.norm2 = 0x10000
        if L.cross:
            L.cross_k = L.cross_v = 0x10000
    d = _lib.ExpertDesc()
    d.batch, d.chunk, d.hidden = 1, cfg.chunk, e.hidden
    d.n_q_heads, d.n_kv_heads, d.head_dim, d.inter = e.n_q_heads, e.n_kv_heads, 64, e.inter
    d.action_dim, d.n_layers, d.prefix_len = cfg.action_dim, cfg.expert_layers, cfg.prefix_len
    d.num_steps, d.ld_cross, d.rms_eps, d.dt = cfg.num_steps, 2 * e.kv_dim, 1e-5, -0.1
    for f in ("w_action_in", "b_action_in", "w_time_in_a", "time_bias", "w_time_out",
              "b_time_out", "norm_out", "w_action_out", "rope_cos", "rope_sin", "x_in", "x_out"):
        setattr(d, f, 0x10000)
    d.layers = layers
    return d, layers


def test_expert_trace_offsets_host_only():
    """svla_expert_trace_offset: one distinct, 256-byte aligned buffer per
    layer boundary of every Euler step, inside the workspace, in step order;
    -1 past the ends."""
    from smolvla import _lib
    from smolvla.config import SmolVLAConfig
    cfg = SmolVLAConfig()
    d, _keep = _fake_expert_desc(cfg)
    lib = _lib.load()
    size = lib.svla_expert_workspace_size(ctypes.byref(d))
    assert size > 0
    buf = ((cfg.expert.hidden + 31) // 32) * 4096
    offs = [lib.svla_expert_trace_offset(ctypes.byref(d), s, l)
            for s in range(cfg.num_steps) for l in range(cfg.expert_layers + 1)]
    assert all(o >= 0 and o % 256 == 0 and o + buf <= size for o in offs)
    assert offs == sorted(offs) and len(set(offs)) == len(offs)
    assert all(b - a >= buf for a, b in zip(offs, offs[1:]))
    for s, l in ((-1, 0), (cfg.num_steps, 0), (0, -1), (0, cfg.expert_layers + 1)):
        assert lib.svla_expert_trace_offset(ctypes.byref(d), s, l) == -1
    d.head_dim = 32                                      # unsupported: invalid descriptor
    assert lib.svla_expert_trace_offset(ctypes.byref(d), 0, 0) == -1
