"""Kernel-level parity: each HIP kernel (through the C-ABI) vs the CPU oracle
(``oracle/smolvla_ref.py``) or the torch fp32 formula it mirrors, on seeded
inputs.  Tolerances (written per test):

* bf16 GEMM / fused-epilogue outputs: max |got - want| / max |want| <= 1e-2
  (the per-layer-output bound) and elementwise allclose at the reference
  harness tolerance (atol 1e-1, rtol 1e-2, gemm/v1_test_tiled_gemm.py:150-151);
* norms / elementwise: <= 1 bf16 ulp relative (2^-7) plus atol 1e-2;
* attention: max relative error <= 1e-2.
"""

import math

import pytest
import torch

import oracle.smolvla_ref as ref

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
F32 = torch.float32


@pytest.fixture(scope="module")
def ops():
    from smolvla import ops as _ops
    from smolvla import _lib
    _lib.load()
    return _ops


def rel_err(got, want):
    got, want = got.float().cpu(), want.float().cpu()
    return ((got - want).abs().max() / want.abs().max().clamp_min(1e-6)).item()


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(g, *shape, std=1.0):
    return (torch.randn(*shape, generator=g) * std).to(BF16)


def assert_close_bf16(got, want, rel=1e-2, atol=1e-1, rtol=1e-2):
    got_c, want_c = got.float().cpu(), want.float().cpu()
    assert torch.isfinite(got_c).all()
    e = rel_err(got_c, want_c)
    assert e <= rel, f"max relative error {e:.3e} > {rel}"
    torch.testing.assert_close(got_c, want_c, atol=atol, rtol=rtol)


# ------------------------------------------------------------------ norms ---
@pytest.mark.parametrize("rows,cols,eps", [(4, 960, 1e-6), (241, 960, 1e-5), (50, 720, 1e-5),
                                           (3, 2048, None), (1, 64, 1e-5)])
def test_rmsnorm(ops, rows, cols, eps):
    g = gen(1)
    x = randn(g, rows, cols)
    w = (1 + 0.1 * torch.randn(cols, generator=g)).to(BF16)
    got = ops.rmsnorm(x.cuda(), w.cuda(), eps)
    want = ref.rms_norm(x, w, eps)
    torch.testing.assert_close(got.cpu().float(), want.float(), atol=1e-2, rtol=2 ** -7)


def test_rmsnorm_strided_rows(ops):
    g = gen(2)
    big = randn(g, 10, 1024)
    x = big[:, :960]                               # leading dim 1024
    w = randn(g, 960)
    out = torch.zeros(10, 1024, dtype=BF16, device="cuda")
    ops.rmsnorm(big.cuda()[:, :960], w.cuda(), 1e-5, out=out[:, :960])
    torch.testing.assert_close(out[:, :960].cpu().float(), ref.rms_norm(x, w, 1e-5).float(),
                               atol=1e-2, rtol=2 ** -7)
    assert (out[:, 960:] == 0).all()


@pytest.mark.parametrize("rows,cols", [(1024, 768), (4, 768), (7, 128), (9, 768), (5, 1536)])
def test_layernorm(ops, rows, cols):
    g = gen(3)
    x = (torch.randn(rows, cols, generator=g) * 2 + 0.5).to(BF16)
    gm = (1 + 0.1 * torch.randn(cols, generator=g)).to(BF16)
    bt = randn(g, cols, std=0.1)
    got = ops.layernorm(x.cuda(), gm.cuda(), bt.cuda(), 1e-6)
    want = ref.layer_norm(x, gm, bt, 1e-6)
    torch.testing.assert_close(got.cpu().float(), want.float(), atol=1e-2, rtol=2 ** -7)
    # the slab-blocked output holds the same values, bit for bit
    blk = ops.layernorm(x.cuda(), gm.cuda(), bt.cuda(), 1e-6, blocked=True)
    assert blk.shape == (cols // 32, rows, 32)
    assert torch.equal(ops.unblock(blk), got)


def test_layernorm_blocked_rejects_bad_cols(ops):
    from smolvla._lib import SvlaError
    x = torch.zeros(4, 80, dtype=BF16, device="cuda")
    with pytest.raises(SvlaError):
        ops.layernorm(x, x[0], x[0], 1e-6, blocked=True)    # cols % 32 != 0


# ------------------------------------------------------------------- GEMM ---
GEMM_SHAPES = [
    # small-M (64x64 / 64x128 tiles, 16x16x32 MFMA, split-K)
    (1, 32, 32), (50, 960, 720), (50, 720, 960), (50, 32, 720), (128, 960, 960),
    (241, 1600, 960), (241, 960, 2560), (192, 960, 12288), (1024, 2304, 768),
    (1024, 768, 3072), (3, 720, 1440), (77, 100, 24),
    # 128x128 and 256x256 tiles (32x32x16 MFMA)
    (4096, 1024, 256), (7712, 960, 960), (8192, 2304, 768), (9000, 772, 200),
]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_linear(ops, M, N, K):
    g = gen(M * 7 + N + K)
    a = randn(g, M, K)
    w = randn(g, K, N, std=0.02)
    wp = ops.pack_weight(w.cuda())
    torch.testing.assert_close(wp.cpu(), w.t().contiguous())
    got = ops.linear(a.cuda(), wp)
    want = ref.linear(a, w)
    assert_close_bf16(got, want)


def test_linear_bias_act_residual(ops):
    g = gen(11)
    M, N, K = 130, 3072, 768
    a, w, b = randn(g, M, K), randn(g, K, N, std=0.02), randn(g, N, std=0.02)
    wp = ops.pack_weight(w.cuda())
    got = ops.linear(a.cuda(), wp, bias=b.cuda(), act="gelu_tanh")
    want = ref.gelu(ref.linear(a, w, b), "tanh")
    assert_close_bf16(got, want)
    res = randn(g, M, N)
    got = ops.linear(a.cuda(), wp, bias=b.cuda(), res=res.cuda())
    want = ref.linear(a, w, b) + res
    assert_close_bf16(got, want)
    got = ops.linear(a.cuda(), wp, act="silu")
    assert_close_bf16(got, ref.silu(ref.linear(a, w)))
    bf = torch.randn(N, generator=g) * 0.1
    got = ops.linear(a.cuda(), wp, bias_f32=bf.cuda(), out_f32=True)
    want = a.float() @ w.float() + bf
    assert rel_err(got, want) < 1e-3


@pytest.mark.parametrize("M,N,K", [(300, 264, 128), (1000, 704, 384), (513, 1032, 768),
                                   (256, 256, 3072), (300, 260, 128), (520, 512, 256)])
def test_wide_tile_forced(ops, force_tile, M, N, K):
    """The 256x256 wide kernel (K % 128 == 0, N % 8 == 0) on ragged M / N
    tails, through the plain epilogues it serves: bias + GELU, bias +
    residual (also in place), alpha, fp32 bias, fp32 out (which, like
    N % 8 != 0, takes the 128x128 pipeline instead)."""
    g = gen(M + N + K)
    force_tile(8)
    a, w, b = randn(g, M, K), randn(g, K, N, std=0.05), randn(g, N, std=0.05)
    wp = ops.pack_weight(w.cuda())
    assert_close_bf16(ops.linear(a.cuda(), wp, bias=b.cuda(), act="gelu_tanh"),
                      ref.gelu(ref.linear(a, w, b), "tanh"))
    res = randn(g, M, N)
    assert_close_bf16(ops.linear(a.cuda(), wp, bias=b.cuda(), res=res.cuda()),
                      ref.linear(a, w, b) + res)
    assert_close_bf16(ops.linear(a.cuda(), wp, alpha=0.125), (ref.linear(a, w).float() * 0.125))
    inplace = res.cuda()
    ops.linear(a.cuda(), wp, res=inplace, out=inplace)
    assert_close_bf16(inplace, ref.linear(a, w) + res)
    bf = torch.randn(N, generator=g) * 0.1
    assert_close_bf16(ops.linear(a.cuda(), wp, bias_f32=bf.cuda()),
                      (a.float() @ w.float() + bf).to(BF16))
    got = ops.linear(a.cuda(), wp, bias_f32=bf.cuda(), out_f32=True)
    assert rel_err(got, a.float() @ w.float() + bf) < 1e-3


@pytest.mark.parametrize("K", [256, 640, 768])
def test_wide_tile_several_tiles_per_workgroup(ops, force_tile, K):
    """More tiles than workgroups (25 x 11 = 275 > 256): the K tiles of a
    workgroup's consecutive tiles stream through one 5-stage LDS ring, so each
    tile starts at a different ring position (K / 32 = 8, 20, 24 K tiles), and
    the epilogue stages through the ring.  Checked against the 128x128
    pipeline kernel (itself checked against the oracle), with bias + GELU and
    bias + residual."""
    g = gen(K + 7)
    M, N = 6400, 2816
    a, b = randn(g, M, K).cuda(), randn(g, N, std=0.05).cuda()
    wp = ops.pack_weight(randn(g, K, N, std=0.05).cuda())
    res = randn(g, M, N).cuda()
    force_tile(8)
    got = ops.linear(a, wp, bias=b, act="gelu_tanh")
    got_res = ops.linear(a, wp, bias=b, res=res)
    force_tile(7)
    assert_close_bf16(got, ops.linear(a, wp, bias=b, act="gelu_tanh"))
    assert_close_bf16(got_res, ops.linear(a, wp, bias=b, res=res))


@pytest.mark.parametrize("M,N", [(24800, 3072), (30700, 768)])
def test_wide_tile_column_resident_order(ops, force_tile, M, N):
    """Grids where each XCD keeps a fixed set of column blocks (their weight
    panels fit its L2) and walks its own row blocks: 97 x 12 tiles, 6 column
    blocks per XCD and a short last row range per column group; 120 x 3
    tiles, all 3 column blocks on every XCD; ragged last row blocks.  Checked
    against the 128x128 pipeline kernel, bias + GELU and bias + residual."""
    g = gen(M + N)
    K = 768
    a, b = randn(g, M, K).cuda(), randn(g, N, std=0.05).cuda()
    wp = ops.pack_weight(randn(g, K, N, std=0.05).cuda())
    res = randn(g, M, N).cuda()
    force_tile(8)
    got = ops.linear(a, wp, bias=b, act="gelu_tanh")
    got_res = ops.linear(a, wp, bias=b, res=res)
    force_tile(7)
    assert_close_bf16(got, ops.linear(a, wp, bias=b, act="gelu_tanh"))
    assert_close_bf16(got_res, ops.linear(a, wp, bias=b, res=res))


def test_slab_block_roundtrip(ops):
    g = gen(40)
    x = randn(g, 300, 96).cuda()
    xb = ops.slab_block(x)
    assert xb.shape == (3, 300, 32)
    assert torch.equal(ops.unblock(xb), x)
    assert torch.equal(xb[1, 7], x[7, 32:64])


@pytest.mark.parametrize("layout", range(8))
def test_linear_wide_layouts(ops, force_tile, layout):
    """svla_linear_wide_bf16 with every combination of slab-blocked A, W and C
    gives bit-for-bit the row-major result of the same (forced) kernel: bias +
    GELU, and bias + residual when C is row-major."""
    g = gen(41 + layout)
    M, N, K = 512, 768, 384
    a, w, b = randn(g, M, K).cuda(), randn(g, K, N, std=0.05).cuda(), randn(g, N, std=0.05).cuda()
    wp = ops.pack_weight(w)
    force_tile(8)
    want = ops.linear(a, wp, bias=b, act="gelu_tanh")
    res = randn(g, M, N).cuda()
    want_res = ops.linear(a, wp, bias=b, res=res)
    force_tile(-1)
    A = ops.slab_block(a) if layout & ops.LAYOUT_A_BLOCKED else a
    W = ops.slab_block(wp) if layout & ops.LAYOUT_W_BLOCKED else wp
    got = ops.linear_wide(A, W, M, N, K, bias=b, act="gelu_tanh", layout=layout)
    if layout & ops.LAYOUT_C_BLOCKED:
        got = ops.unblock(got)
    assert torch.equal(got, want)
    if not layout & ops.LAYOUT_C_BLOCKED:
        got = ops.linear_wide(A, W, M, N, K, bias=b, res=res, layout=layout)
        assert torch.equal(got, want_res)
    assert_close_bf16(want, ref.gelu(ref.linear(a.cpu(), w.cpu(), b.cpu()), "tanh"))


@pytest.mark.parametrize("act,alpha", [("gelu_erf", 1.0), ("silu", 1.0), ("silu", 0.5),
                                       ("gelu_tanh", 0.25), (None, 0.5)])
def test_linear_wide_epilogues(ops, force_tile, act, alpha):
    """Every activation of the wide kernel's epilogue, with and without a
    scale, is bit-for-bit the (forced) 128x128 kernel's result; the wide
    kernel rounds the scaled, biased value to bf16 two values per conversion
    before the activation, the 128x128 kernel one at a time."""
    g = gen(77)
    M, N, K = 768, 512, 640
    a, w, b = randn(g, M, K).cuda(), randn(g, K, N, std=0.05).cuda(), randn(g, N, std=0.05).cuda()
    wp = ops.pack_weight(w)
    force_tile(8)
    want = ops.linear(a, wp, bias=b, act=act, alpha=alpha)
    force_tile(-1)
    got = ops.linear_wide(ops.slab_block(a), ops.slab_block(wp), M, N, K, bias=b, act=act,
                          alpha=alpha, layout=ops.LAYOUT_A_BLOCKED | ops.LAYOUT_W_BLOCKED)
    assert torch.equal(got, want)
    # fp32 affine part rounded once to bf16, then the activation in fp32
    lin = (ref.linear(a.cpu().float(), w.cpu().float()) * alpha + b.cpu().float()).bfloat16()
    lin = lin.float()
    exp = {None: lambda x: x, "silu": ref.silu, "gelu_erf": lambda x: ref.gelu(x, "none"),
           "gelu_tanh": lambda x: ref.gelu(x, "tanh")}[act](lin)
    assert_close_bf16(got, exp)


def test_linear_wide_rejects_bad_shapes(ops):
    a = torch.zeros(300, 384, dtype=BF16, device="cuda")
    w = torch.zeros(768, 384, dtype=BF16, device="cuda")
    from smolvla._lib import SvlaError
    with pytest.raises(SvlaError):
        ops.linear_wide(a, w, 300, 768, 384)        # M % 256 != 0
    with pytest.raises(SvlaError):
        ops.linear_wide(a[:256], w[:700], 256, 700, 384)  # N % 256 != 0


def test_wide_tile_auto_vit_up(ops):
    # a ViT MLP up-projection large enough for the automatic wide-tile choice
    g = gen(17)
    M, N, K = 16384, 3072, 768
    a, w, b = randn(g, M, K), randn(g, K, N, std=0.02), randn(g, N, std=0.02)
    got = ops.linear(a.cuda(), ops.pack_weight(w.cuda()), bias=b.cuda(), act="gelu_tanh")
    assert_close_bf16(got, ref.gelu(ref.linear(a, w, b), "tanh"))


def test_linear_gelu_big_tile(ops):
    # the ViT MLP up-projection shape class on the 256x256 tile
    g = gen(13)
    M, N, K = 8192, 3072, 768
    a, w, b = randn(g, M, K), randn(g, K, N, std=0.02), randn(g, N, std=0.02)
    got = ops.linear(a.cuda(), ops.pack_weight(w.cuda()), bias=b.cuda(), act="gelu_tanh")
    assert_close_bf16(got, ref.gelu(ref.linear(a, w, b), "tanh"))


@pytest.mark.parametrize("M,K", [(50, 720), (241, 960), (7712, 960), (3, 2048)])
def test_fused_rmsnorm_prologue(ops, M, K):
    """norm=(w, eps): A rows RMS-normalised inside the GEMM ~= rmsnorm then GEMM."""
    g = gen(M + K + 1)
    x = randn(g, M, K, std=2.0)
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(BF16)
    w = randn(g, K, 1600, std=0.02)
    wp = ops.pack_weight(w.cuda())
    h = ref.rms_norm(x, nw, 1e-5)
    got = ops.linear(x.cuda(), wp, norm=(nw.cuda(), 1e-5))
    assert_close_bf16(got, ref.linear(h, w))
    # vs the standalone RMSNorm kernel followed by the GEMM: both round each
    # operand element as bf16((x * (1 / rms)) * gain), so the operands are
    # the same; the automatic tile choice can still differ (the 256-wide
    # kernel takes no norm), and with it the fp32 summation order, so an
    # output can move by an ulp or two (SiLU-mul rounds gate and up): within
    # 2^-6 of the output range (bit-identical per forced tile below)
    def same(a, b):
        assert_close_bf16(a, b, rel=2 ** -6)

    sep = ops.linear(ops.rmsnorm(x.cuda(), nw.cuda(), 1e-5), wp)
    same(got, sep)
    c, s_ = ops.rope_table(50, 64, 1e5)
    if M % 50 == 0:
        got = ops.linear_rope(x.cuda(), wp, 1280, 50, c, s_, norm=(nw.cuda(), 1e-5))
        sep = ops.linear_rope(ops.rmsnorm(x.cuda(), nw.cuda(), 1e-5), wp, 1280, 50, c, s_)
        same(got, sep)
    wg, wu = randn(g, K, 2048, std=0.02), randn(g, K, 2048, std=0.02)
    wgu = ops.pack_gate_up(wg.cuda(), wu.cuda())
    got = ops.linear_silu_mul(x.cuda(), wgu, norm=(nw.cuda(), 1e-5))
    sep = ops.linear_silu_mul(ops.rmsnorm(x.cuda(), nw.cuda(), 1e-5), wgu)
    same(got, sep)


TILES = {0: "256x256/32", 1: "128x128/32", 2: "64x128/16", 3: "64x64/16", 4: "skinny64",
         5: "skinny32", 6: "128x128/16", 7: "pipe128", 8: "wide256", 9: "pipe64",
         10: "pipe128x64", 11: "pipe64x128", 12: "skinny16", 13: "line128", 14: "line128x64",
         15: "line64x128", 16: "line64", 17: "small32", 18: "small32x64",
         19: "small96"}


@pytest.fixture
def force_tile(ops):
    from smolvla import _lib
    lib = _lib.load()
    yield lambda t: lib.svla_gemm_set_tile(t)
    lib.svla_gemm_set_tile(-1)


@pytest.fixture
def force_split(ops):
    from smolvla import _lib
    lib = _lib.load()
    yield lambda s: lib.svla_gemm_set_split(s)
    lib.svla_gemm_set_split(-1)


@pytest.mark.parametrize("tile", sorted(TILES))
def test_every_tile_config_every_epilogue(ops, force_tile, tile):
    """Each GEMM kernel configuration, forced, on ragged shapes (M, N, K
    tails) through every epilogue, the fused RMSNorm and both A gathers."""
    force_tile(tile)
    _every_epilogue(ops, gen(100 + tile), tile)


@pytest.mark.parametrize("tile", sorted(t for t in TILES if t != 8))
def test_fused_norm_bit_identical_to_standalone(ops, force_tile, tile):
    """Each kernel configuration that fuses the RMSNorm (all but the 256-wide
    one) rounds every operand element as the standalone RMSNorm kernel rounds
    its output, bf16((x * (1 / rms)) * gain): with the tile forced,
    norm=(w, eps) on x and the same GEMM on svla_rmsnorm_bf16(x) are
    bit-identical, through the plain, RoPE and SiLU-mul epilogues; ragged M,
    a K tail, and K = 2048 (split over workgroups by the skinny tiles).  The
    16- and 32-column skinny tiles are the exception: without the norm they
    keep 8 k-steps per wave in flight, with it 4 (the gain fragments take
    the registers), so their waves split K differently and the fp32 sums may
    differ in order: there the outputs agree to an ulp or two."""
    force_tile(tile)
    g = gen(300 + tile)

    def same(a, b, what):
        if tile in (5, 12):
            assert_close_bf16(a, b, rel=2 ** -6)
        else:
            assert torch.equal(a, b), what

    for M, K in ((200, 200), (50, 720), (3, 2048)):
        x = randn(g, M, K, std=2.0).cuda()
        nw = (1 + 0.1 * torch.randn(K, generator=g)).to(BF16).cuda()
        nrm = (nw, 1e-5)
        h = ops.rmsnorm(x, nw, 1e-5)
        w = ops.pack_weight(randn(g, K, 192, std=0.05).cuda())
        same(ops.linear(x, w, norm=nrm), ops.linear(h, w), ("plain", M, K))
        if tile == 5:                                  # paired epilogues need 64-wide tiles
            continue
        c, s_ = ops.rope_table(M, 64, 1e4)
        same(ops.linear_rope(x, w, 128, M, c, s_, norm=nrm),
             ops.linear_rope(h, w, 128, M, c, s_), ("rope", M, K))
        wgu = ops.pack_gate_up(randn(g, K, 128, std=0.05).cuda(),
                               randn(g, K, 128, std=0.05).cuda())
        same(ops.linear_silu_mul(x, wgu, norm=nrm), ops.linear_silu_mul(h, wgu),
             ("silu", M, K))


@pytest.mark.parametrize("tile,splits", [(4, 2), (5, 3), (4, 6), (5, 8), (12, 2), (12, 5)])
def test_skinny_split_k_every_epilogue(ops, force_tile, force_split, tile, splits):
    """Skinny kernels with K split over `splits` workgroups (partials summed
    by the last one to arrive), through every epilogue and gather; the K tail
    lands in the last split."""
    force_tile(tile)
    force_split(splits)
    _every_epilogue(ops, gen(200 + 10 * tile + splits), tile)


def test_skinny_split_k_graph_replays(ops, force_tile, force_split):
    """Split-K calls captured in a graph: several replays with eager work in
    between, every replay equal to the eager result (the arrival counters are
    reset by each call), then a smaller problem on the same workspace.  (The
    32-column skinny tile is forced: the automatic choice of these shapes is
    the unsplit 32x32 small tile.)"""
    g = gen(31)
    force_tile(5)
    force_split(4)
    a, w = randn(g, 50, 2048), randn(g, 2048, 720, std=0.02)
    res = randn(g, 50, 720)
    a, wp, res = a.cuda(), ops.pack_weight(w.cuda()), res.cuda()
    want = ref.linear(a.cpu(), w) + res.cpu()
    out = torch.empty(50, 720, dtype=BF16, device="cuda")
    eager = ops.linear(a, wp, res=res)
    assert_close_bf16(eager, want)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.linear(a, wp, res=res, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.linear(a, wp, res=res, out=out)
    for rep in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
        ops.linear(a[:17], wp, out=torch.empty(17, 720, dtype=BF16, device="cuda"))
    small = ops.linear(a[:9, :1536], ops.pack_weight(w[:1536].cuda()))
    assert_close_bf16(small, ref.linear(a[:9, :1536].cpu(), w[:1536]))


@pytest.mark.parametrize("M,K", [(50, 720), (241, 960)])
def test_skinny16_paired_matches_skinny64(ops, force_tile, M, K):
    """The 16-column skinny tile pairs packed columns n and n + 32 through a
    row map of the weight loads; with the fused RMSNorm both tiles split K
    over the waves identically, so RoPE and SiLU outputs are bit-identical to
    the 64-column tile's."""
    g = gen(41)
    x = randn(g, M, K).cuda()
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(BF16).cuda()
    wqkv = ops.pack_weight(randn(g, K, 1600, std=0.02).cuda())
    wgu = ops.pack_gate_up(randn(g, K, 2048, std=0.02).cuda(), randn(g, K, 2048, std=0.02).cuda())
    c, s_ = ops.rope_table(M, 64, 1e5)
    outs = {}
    for tile in (4, 12):
        force_tile(tile)
        outs[tile] = (ops.linear_rope(x, wqkv, 1280, M, c, s_, norm=(nw, 1e-5)),
                      ops.linear_silu_mul(x, wgu, norm=(nw, 1e-5)))
    assert torch.equal(outs[4][0], outs[12][0])
    assert torch.equal(outs[4][1], outs[12][1])


def _every_epilogue(ops, g, tile):
    M, K = 200, 200                                   # K tail (200 = 6*32 + 8)
    x = randn(g, M, K)
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(BF16)
    # plain + bias + GELU, residual, fp32 out
    w, b = randn(g, K, 260, std=0.05), randn(g, 260, std=0.05)
    wp = ops.pack_weight(w.cuda())
    assert_close_bf16(ops.linear(x.cuda(), wp, bias=b.cuda(), act="gelu_tanh"),
                      ref.gelu(ref.linear(x, w, b), "tanh"))
    res = randn(g, M, 260)
    assert_close_bf16(ops.linear(x.cuda(), wp, res=res.cuda()), ref.linear(x, w) + res)
    assert_close_bf16(ops.linear(x.cuda(), wp, norm=(nw.cuda(), 1e-5)),
                      ref.linear(ref.rms_norm(x, nw, 1e-5), w))
    if tile != 5:                                      # paired epilogues need 64-wide tiles
        wq = randn(g, K, 192, std=0.05)
        c, s_ = ops.rope_table(40, 64, 1e4)
        got = ops.linear_rope(x.cuda(), ops.pack_weight(wq.cuda()), 128, 40, c, s_,
                              norm=(nw.cuda(), 1e-5)).cpu()
        h = ref.rms_norm(x, nw, 1e-5)
        qk = ref.apply_rope(ref.linear(h, wq[:, :128]).view(5, 40, 2, 64), 1e4).to(BF16)
        assert_close_bf16(got[:, :128], qk.view(M, 128))
        assert_close_bf16(got[:, 128:], ref.linear(h, wq[:, 128:]))
        wg, wu = randn(g, K, 96, std=0.05), randn(g, K, 96, std=0.05)
        got = ops.linear_silu_mul(x.cuda(), ops.pack_gate_up(wg.cuda(), wu.cuda()))
        assert_close_bf16(got, ref.silu(ref.linear(x, wg)) * ref.linear(x, wu))
    # gathers: im2col patch embedding (2 images of 64x64) and pixel shuffle
    img = (torch.rand(2, 3, 64, 64, generator=g) * 2 - 1).to(BF16)
    kern, kb = randn(g, 96, 3, 16, 16, std=0.05), randn(g, 96, std=0.05)
    pos = randn(g, 16, 96, std=0.05)
    got = ops.patch_embed(img.cuda(), kern.reshape(96, -1).cuda(), kb.cuda(), pos.cuda(), 16)
    assert_close_bf16(got, ref.patch_embed(img, kern, kb, pos).reshape(-1, 96))
    xv = randn(g, 2, 64, 96)
    wc = randn(g, 96 * 4, 64, std=0.05)
    got = ops.connector(xv.cuda(), ops.pack_weight(wc.cuda()), 2)
    assert_close_bf16(got, ref.connector(xv, wc, 2).reshape(-1, 64))


def test_repeated_calls_deterministic(ops):
    """Skinny-M calls of different shapes back to back: each result is
    correct and bit-identical across repetitions (no cross-call state)."""
    g = gen(14)
    cases = []
    for (M, N, K) in ((50, 960, 720), (50, 720, 2048), (241, 320, 320), (50, 960, 720)):
        a, w = randn(g, M, K), randn(g, K, N, std=0.02)
        cases.append((a.cuda(), ops.pack_weight(w.cuda()), ref.linear(a, w)))
    first = [ops.linear(a, wp) for a, wp, _ in cases]
    for rep in range(3):
        for (a, wp, want), f in zip(cases, first):
            got = ops.linear(a, wp)
            assert_close_bf16(got, want)
            assert torch.equal(got, f)


def test_linear_alpha_attn_score_harness(ops):
    # transpose_matmul_with_scale_bf16: C = 0.125 * A . B^T
    # (attn_score/test_attn_score_bf16.py:62-66)
    from smolvla import kernels
    g = gen(12)
    for (M, N) in ((64, 64), (128, 128)):
        A, B = randn(g, M, 64), randn(g, N, 64)
        C = torch.empty(M, N, dtype=BF16, device="cuda")
        kernels.transpose_matmul_with_scale_bf16(A.cuda(), B.cuda(), C)
        want = (A.float() @ B.float().t() * 0.125).to(BF16)
        torch.testing.assert_close(C.cpu().float(), want.float(), atol=1e-1, rtol=1e-2)


@pytest.mark.parametrize("M,L,hid", [(128, 128, 960), (241, 241, 960), (482, 241, 960),
                                     (50, 50, 720), (100, 50, 720), (7712, 241, 960),
                                     (16384, 128, 960)])
def test_linear_rope_qkv(ops, M, L, hid):
    g = gen(M + hid)
    theta = 100000.0
    x = randn(g, M, hid)
    wq, wk, wv = randn(g, hid, 960, std=0.02), randn(g, hid, 320, std=0.02), randn(g, hid, 320,
                                                                                   std=0.02)
    w = torch.cat([wq, wk, wv], dim=1)
    cos_t, sin_t = ops.rope_table(L, 64, theta)
    c_ref, s_ref = ref.rope_tables(L, 64, theta)
    # angles reach ~240 rad: a 1-2 ulp fp32 difference in the angle (powf) is ~4e-6
    torch.testing.assert_close(cos_t.cpu(), c_ref, atol=1e-5, rtol=0)
    torch.testing.assert_close(sin_t.cpu(), s_ref, atol=1e-5, rtol=0)
    got = ops.linear_rope(x.cuda(), ops.pack_weight(w.cuda()), 1280, L, cos_t, sin_t).cpu()
    B = M // L
    q = ref.apply_rope(ref.linear(x, wq).view(B, L, 15, 64), theta).to(BF16).view(M, 960)
    k = ref.apply_rope(ref.linear(x, wk).view(B, L, 5, 64), theta).to(BF16).view(M, 320)
    v = ref.linear(x, wv)
    assert_close_bf16(got[:, :960], q)
    assert_close_bf16(got[:, 960:1280], k)
    assert_close_bf16(got[:, 1280:], v)


@pytest.mark.parametrize("M,L,hid", [(241, 241, 960), (100, 50, 720), (7712, 241, 960)])
def test_linear_rope_remainder(ops, M, L, hid):
    """The RoPE epilogue's optional remainder output: hi is bit-identical to the
    plain call, lo = o - bf16(o) of the fp32 rotation, so hi + lo follows the
    fp32 RoPE of the bf16 projection (the reference's Q and K,
    vla/text_encoder_bf16.py:92-104) to ~2^-16 wherever the projection rounds
    like torch's (rarely 1 bf16 ulp apart: a few elements); V columns of lo
    are left untouched."""
    g = gen(M + 7 * hid)
    theta = 100000.0
    x = randn(g, M, hid)
    w = randn(g, hid, 1600, std=0.02)
    wp = ops.pack_weight(w.cuda())
    cos_t, sin_t = ops.rope_table(L, 64, theta)
    plain = ops.linear_rope(x.cuda(), wp, 1280, L, cos_t, sin_t).cpu()
    lo = torch.full((M, 1600), 7.0, dtype=BF16, device="cuda")
    hi = ops.linear_rope(x.cuda(), wp, 1280, L, cos_t, sin_t, out_lo=lo).cpu()
    lo = lo.cpu()
    assert torch.equal(hi, plain)
    assert (lo[:, 1280:] == 7.0).all()
    B = M // L
    proj = ref.linear(x, w)                                   # bf16, as the kernel rounds it
    q = ref.apply_rope(proj[:, :960].reshape(B, L, 15, 64), theta).reshape(M, 960)
    k = ref.apply_rope(proj[:, 960:1280].reshape(B, L, 5, 64), theta).reshape(M, 320)
    want = torch.cat([q, k], dim=1)                           # fp32
    got = hi[:, :1280].float() + lo[:, :1280].float()
    err = (got - want).abs() / want.abs().clamp_min(1e-3)
    assert (lo[:, :1280].float().abs() <= hi[:, :1280].float().abs() * 2 ** -8 + 1e-30).all()
    assert (err <= 2 ** -15).float().mean().item() >= 0.99, err.median().item()
    assert (got - want).abs().max().item() <= 2e-2


@pytest.mark.parametrize("M,K,inter", [(50, 720, 2048), (241, 960, 2560), (1024, 960, 2560),
                                       (5, 64, 64), (7712, 960, 2560), (3000, 720, 2048)])
def test_linear_silu_mul(ops, M, K, inter):
    g = gen(M + K)
    x = randn(g, M, K)
    wg, wu = randn(g, K, inter, std=0.02), randn(g, K, inter, std=0.02)
    wgu = ops.pack_gate_up(wg.cuda(), wu.cuda())
    got = ops.linear_silu_mul(x.cuda(), wgu)
    want = ref.silu(ref.linear(x, wg)) * ref.linear(x, wu)
    assert_close_bf16(got, want)


def test_patch_embed(ops):
    g = gen(21)
    n, C, H, P, E = 3, 3, 512, 16, 768
    img = (torch.rand(n, C, H, H, generator=g) * 2 - 1).to(BF16)
    kern = randn(g, E, C, P, P, std=0.02)
    bias = randn(g, E, std=0.02)
    pos = randn(g, (H // P) ** 2, E, std=0.02)
    got = ops.patch_embed(img.cuda(), kern.reshape(E, -1).cuda(), bias.cuda(), pos.cuda(), P)
    want = ref.patch_embed(img, kern, bias, pos).reshape(-1, E)
    assert_close_bf16(got, want)


def test_connector(ops):
    g = gen(22)
    x = randn(g, 3, 1024, 768)
    w = randn(g, 12288, 960, std=0.02)
    got = ops.connector(x.cuda(), ops.pack_weight(w.cuda()), 4)
    want = ref.connector(x, w, 4).reshape(-1, 960)
    assert_close_bf16(got, want)


def test_action_out_euler(ops):
    g = gen(23)
    M, N, K = 100, 32, 720
    a, w = randn(g, M, K), randn(g, K, N, std=0.02)
    x = torch.randn(M, N, generator=g)
    xd = x.cuda().clone()
    xb = torch.empty(M, N, dtype=BF16, device="cuda")
    ops.action_out_euler(a.cuda(), ops.pack_weight(w.cuda()), xd, -0.1, x_bf16=xb)
    v = ref.linear(a, w).float()
    want = x + (-0.1) * v
    assert rel_err(xd, want) < 1e-3
    torch.testing.assert_close(xb.cpu(), xd.cpu().to(BF16))
    # with the final expert RMSNorm fused into the A operand
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(BF16)
    xd = x.cuda().clone()
    ops.action_out_euler(a.cuda(), ops.pack_weight(w.cuda()), xd, -0.1,
                         norm=(nw.cuda(), 1e-5))
    v = ref.linear(ref.rms_norm(a, nw, 1e-5), w).float()
    assert rel_err(xd, x + (-0.1) * v) < 1e-3


# -------------------------------------------------------------- attention ---
ATTN_CASES = [
    # B, Sq, Sk, hq, hkv, mask, prefix
    (1, 128, 128, 15, 5, "causal", 0),
    (1, 241, 241, 15, 5, "prefix_lm", 240),
    (2, 241, 241, 15, 5, "prefix_lm", 240),
    (1, 50, 50, 15, 5, "causal", 0),
    (3, 50, 241, 15, 5, "none", 0),
    (1, 1024, 1024, 12, 12, "none", 0),
    (2, 17, 17, 3, 1, "prefix_lm", 16),
    (1, 1, 5, 2, 1, "none", 0),
    (2, 50, 256, 15, 5, "none", 0),     # short queries, full key blocks
    (1, 64, 320, 15, 5, "none", 0),     # largest 2-wave workgroup
    (1, 65, 65, 15, 5, "causal", 0),    # smallest 4-wave launch, mostly padding
    (11, 1000, 1024, 12, 12, "none", 0),  # 64 query rows per wave (528 workgroups), ragged tail
]


@pytest.mark.parametrize("B,Sq,Sk,hq,hkv,mask,prefix", ATTN_CASES)
def test_attention(ops, B, Sq, Sk, hq, hkv, mask, prefix):
    g = gen(B * 1000 + Sq + hq)
    q = randn(g, B, Sq, hq * 64)
    k = randn(g, B, Sk, hkv * 64)
    v = randn(g, B, Sk, hkv * 64)
    out = torch.empty(B, Sq, hq * 64, dtype=BF16, device="cuda")
    ops.attention(q.cuda(), k.cuda(), v.cuda(), out, hq, hkv, mask=mask, prefix_len=prefix)
    m = ref.make_mask(mask, Sq, Sk, prefix)
    want = ref.gqa_attention(q.view(B, Sq, hq, 64).float(), k.view(B, Sk, hkv, 64),
                             v.view(B, Sk, hkv, 64), m)
    assert rel_err(out, want) <= 1e-2
    torch.testing.assert_close(out.cpu().float(), want.float(), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("B,S,Sk,mask,with_k", [(2, 241, 241, "prefix_lm", True),
                                                (3, 50, 50, "causal", True),
                                                (2, 50, 241, "none", False),
                                                (1, 128, 128, "causal", True)])
def test_attention_fp32_qk_remainders(ops, B, S, Sk, mask, with_k):
    """Scores on fp32 Q (and K) carried as bf16 hi + lo (svla_attention_lo_bf16)
    against the oracle's attention on the fp32 values, the reference module's
    own precision (vla/text_encoder_bf16.py:117-122): several times closer
    than the plain bf16 call, and within 1e-2."""
    g = gen(B * 77 + S + Sk)
    qf = torch.randn(B, S, 960, generator=g) * 2.0
    kf = torch.randn(B, Sk, 320, generator=g) * 2.0
    v = randn(g, B, Sk, 320)
    split = lambda t: (t.to(BF16), (t - t.to(BF16).float()).to(BF16))  # noqa: E731
    qh, ql = split(qf)
    kh, kl = split(kf)
    if not with_k:                                # cross layers: K is a plain bf16 projection
        kf, kl = kh.float(), None
    prefix = 240 if mask == "prefix_lm" else 0
    m = ref.make_mask(mask, S, Sk, prefix)
    want = ref.gqa_attention(qf.view(B, S, 15, 64), kf.view(B, Sk, 5, 64), v.view(B, Sk, 5, 64), m)
    out = torch.empty(B, S, 960, dtype=BF16, device="cuda")
    ops.attention(qh.cuda(), kh.cuda(), v.cuda(), out, 15, 5, mask, prefix, q_lo=ql.cuda(),
                  k_lo=kl.cuda() if kl is not None else None)
    plain = torch.empty_like(out)
    ops.attention(qh.cuda(), kh.cuda(), v.cuda(), plain, 15, 5, mask, prefix)
    e_lo, e_plain = rel_err(out, want), rel_err(plain, want)
    print(f"fp32-QK attention: with remainders {e_lo:.3e}, plain bf16 {e_plain:.3e}")
    assert e_lo <= 1e-2 and e_lo <= e_plain


def test_attention_views_into_fused_qkv(ops):
    # Q/K/V as column slices of one [B*S, 1600] projection buffer
    g = gen(31)
    B, S = 2, 241
    qkv = randn(g, B, S, 1600)
    d = qkv.cuda()
    out = torch.empty(B, S, 960, dtype=BF16, device="cuda")
    ops.attention(d[:, :, :960], d[:, :, 960:1280], d[:, :, 1280:], out, 15, 5, "causal")
    want = ref.gqa_attention(qkv[:, :, :960].reshape(B, S, 15, 64).float(),
                             qkv[:, :, 960:1280].reshape(B, S, 5, 64),
                             qkv[:, :, 1280:].reshape(B, S, 5, 64), ref.make_mask("causal", S, S))
    assert rel_err(out, want) <= 1e-2


# ------------------------------------------------------------ elementwise ---
def test_silu_gelu_silu_mul(ops):
    g = gen(41)
    x = randn(g, 4, 2560, std=3.0)
    torch.testing.assert_close(ops.silu(x.cuda()).cpu(), ref.silu(x), atol=1e-2, rtol=2 ** -7)
    torch.testing.assert_close(ops.gelu(x.cuda(), "tanh").cpu(), ref.gelu(x, "tanh"),
                               atol=1e-2, rtol=2 ** -7)
    torch.testing.assert_close(ops.gelu(x.cuda(), "erf").cpu(), ref.gelu(x, "erf"),
                               atol=1e-2, rtol=2 ** -7)
    u = randn(g, 4, 2560)
    torch.testing.assert_close(ops.silu_mul(x.cuda(), u.cuda()).cpu(), ref.silu(x) * u,
                               atol=1e-2, rtol=2 ** -7)
    odd = randn(g, 13)                                   # non-multiple-of-8 tail
    torch.testing.assert_close(ops.silu(odd.cuda()).cpu(), ref.silu(odd), atol=1e-2,
                               rtol=2 ** -7)


def test_softmax_kernels(ops):
    g = gen(42)
    s = randn(g, 8, 128, std=2.0)
    for rs in (0, 96):
        got = ops.masked_softmax(s.cuda(), rs).cpu()
        torch.testing.assert_close(got.float(), ref.masked_softmax_rows(s, rs).float(),
                                   atol=5e-3, rtol=5e-2)
    s32 = torch.randn(24, 1024, generator=g) * 3
    got = ops.softmax(s32.cuda(), out_f32=True).cpu()
    torch.testing.assert_close(got, torch.softmax(s32, -1), atol=1e-6, rtol=1e-4)
    got = ops.softmax(s.cuda()).cpu()
    torch.testing.assert_close(got.float(), ref.softmax_rows(s).float(), atol=5e-3, rtol=2e-2)


def test_rope_standalone(ops):
    g = gen(43)
    L, H = 64, 8
    x = torch.randn(L, H * 64, generator=g)
    c, s = ops.rope_table(L, 64, 10000.0)
    got = ops.rope(x.cuda(), H, c, s).cpu()
    want = ref.apply_rope(x.view(1, L, H, 64), 10000.0).view(L, H * 64)
    torch.testing.assert_close(got, want, rtol=1e-3, atol=1e-4)


def test_embed_and_time_embedding(ops):
    g = gen(44)
    table = randn(g, 1000, 960, std=0.02)
    ids = torch.randint(0, 1000, (2, 48), generator=g)
    out = torch.zeros(2 * 241, 960, dtype=BF16, device="cuda")
    # language rows 192..239 of each 241-row sample
    ops.embed(ids.cuda(), table.cuda(), math.sqrt(960), out[192:], per_sample=48,
              out_bs=241 * 960)
    o = out.view(2, 241, 960).cpu()
    torch.testing.assert_close(o[:, 192:240], ref.lang_embed(ids, table))
    assert (o[:, :192] == 0).all() and (o[:, 240:] == 0).all()
    bad = torch.tensor([5, -1, 1000], dtype=torch.int64)
    ob = ops.embed(bad.cuda(), table.cuda(), 1.0, torch.ones(3, 960, dtype=BF16, device="cuda"))
    assert (ob[1:] == 0).all()
    for t in (1.0, 0.5, 0.1):
        te = ops.time_embedding(t, 720).cpu()
        want = ref.time_embedding(torch.tensor([t]), 720)[0].to(BF16)
        torch.testing.assert_close(te.float(), want.float(), atol=1e-2, rtol=2 ** -7)


def test_bad_shapes_raise(ops):
    from smolvla._lib import SvlaError
    a = torch.zeros(4, 12, dtype=BF16, device="cuda")            # K % 8 != 0
    w = torch.zeros(8, 12, dtype=BF16, device="cuda")
    with pytest.raises(SvlaError):
        ops.linear(a, w)
    q = torch.zeros(1, 4, 96, dtype=BF16, device="cuda")         # head_dim != 64 layout
    with pytest.raises(SvlaError):
        ops.attention(q, q, q, q, 2, 1)


@pytest.mark.parametrize("kind", ["silu_mul", "rope", "attention"])
def test_lds_pipeline_repeat_is_bit_stable(ops, kind):
    """Regression: the LDS-DMA pipelines (64x64 GEMM tile with fused RMSNorm,
    used by the batch-1 prefix's norm + gate|up and norm + QKV + RoPE, and
    the attention kernel) once refilled an LDS stage before every wave had
    finished reading it, so one wave's 16 rows of a tile occasionally read
    the next K tile's data (4 of 12 prefix passes differed).  The same launch,
    repeated with other work between, must give the same bits every time."""
    g = gen(77)
    M, K = 241, 960
    x = torch.randn(M, K, generator=g).to(BF16).cuda()
    gain = (1 + 0.1 * torch.randn(K, generator=g)).to(BF16).cuda()
    if kind == "silu_mul":
        wg = (0.02 * torch.randn(K, 2560, generator=g)).to(BF16).cuda()
        wu = (0.02 * torch.randn(K, 2560, generator=g)).to(BF16).cuda()
        w = ops.pack_gate_up(wg, wu)
        out = torch.empty(M, 2560, dtype=BF16, device="cuda")
        run = lambda: ops.linear_silu_mul(x, w, out=out, norm=(gain, 1e-5))  # noqa: E731
    elif kind == "rope":
        w = ops.pack_weight((0.02 * torch.randn(K, 1600, generator=g)).to(BF16).cuda())
        cos, sin = ops.rope_table(M, 64, 1e5, device="cuda")
        out = torch.empty(M, 1600, dtype=BF16, device="cuda")
        run = lambda: ops.linear_rope(x, w, 1280, M, cos, sin, out=out, norm=(gain, 1e-5))  # noqa: E731
    else:
        qkv = torch.randn(M, 1600, generator=g).to(BF16).cuda().view(1, M, 1600)
        out = torch.empty(1, M, 960, dtype=BF16, device="cuda")
        run = lambda: ops.attention(qkv[:, :, :960], qkv[:, :, 960:1280], qkv[:, :, 1280:],  # noqa: E731
                                    out, 15, 5, "prefix_lm", 240)
    run()
    first = out.clone()
    noise = torch.randn(1 << 22, device="cuda")
    for i in range(40):
        if i % 4 == 0:
            noise.mul_(1.0001).sum().item()          # other work between launches
        run()
        assert torch.equal(out, first), f"{kind}: launch {i} differs"
