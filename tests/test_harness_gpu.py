"""Per-kernel harness parity: one test per reference harness test file.

Each test drives the gfx950 kernel through ``smolvla.kernels`` -- the
reference's kernel name and argument order, output written in place -- on
inputs drawn the way the reference test draws them (shapes, distributions),
and checks it against the same PyTorch reference with the same
``assert_allclose`` tolerance the reference test uses (cited per test).
Where the reference test splits the work into AIE tiles and loops over them,
the kernel here takes the whole tensor in one call unless the harness entry
point itself is tile-shaped (rope_fused_float32).
"""

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

BF16, F32 = torch.bfloat16, torch.float32


@pytest.fixture(scope="module")
def K():
    from smolvla import _lib, kernels
    _lib.load()
    return kernels


def check(got, want, rtol, atol=0.0):
    np.testing.assert_allclose(got.float().cpu().numpy(), want.float().cpu().numpy(),
                               rtol=rtol, atol=atol)


def run(fn, *args, out_like):
    out = torch.zeros_like(out_like, device="cuda")
    fn(*[a.cuda() if torch.is_tensor(a) else a for a in args], out)
    return out


# ------------------------------------------------------------------- add ----
def test_add(K):
    """add/test_add.py:37-43: bf16 32x32 x + y, rtol 1e-1."""
    torch.manual_seed(0)
    x, y = torch.randn(32, 32).to(BF16), torch.randn(32, 32).to(BF16)
    check(run(K.add, x, y, out_like=x), x + y, rtol=1e-1)


# ------------------------------------------------------------ attn score ----
@pytest.mark.parametrize("m,n", [(64, 64), (128, 128)])
def test_attn_score_bf16(K, m, n):
    """attn_score/test_attn_score_bf16.py:62-73, 123-134: C = A . B^T * 0.125
    (bf16), atol 1e-1 rtol 1e-2."""
    torch.manual_seed(0)
    A, B = torch.randn(m, 64).to(BF16), torch.randn(n, 64).to(BF16)
    C = torch.zeros(m, n, dtype=BF16, device="cuda")
    K.transpose_matmul_with_scale_bf16(A.cuda(), B.cuda(), C)
    check(C, (A.float() @ B.float().t() * 0.125).to(BF16), rtol=1e-2, atol=1e-1)


# ------------------------------------------------------------------ conv ----
def test_conv(K):
    """conv/test_conv.py:50-106: fp32 Conv2d(1 -> 1, k = s = 16) of a 64x64
    image, output [16 patches, 1], rtol 1e-1."""
    np.random.seed(0)
    img = np.random.rand(1, 64, 64).astype(np.float32)
    ker = np.random.rand(1, 1, 16, 16).astype(np.float32)
    out = torch.zeros(16, 1, device="cuda")
    K.conv(torch.from_numpy(img).cuda(), torch.from_numpy(ker).cuda(), out)
    conv = nn.Conv2d(1, 1, kernel_size=16, stride=16, padding=0)
    with torch.no_grad():
        conv.weight.copy_(torch.from_numpy(ker))
        conv.bias.zero_()
        want = conv(torch.from_numpy(img).unsqueeze(0)).squeeze(0).flatten(1).t()
    check(out, want, rtol=1e-1)


def test_conv_patch_embed_shape(K):
    """The ViT patch embedding in fp32 (3 -> 768, 512x512, k = s = 16) through
    the same kernel, checked against nn.Conv2d with bias."""
    torch.manual_seed(0)
    img, ker, b = torch.rand(1, 3, 512, 512), torch.randn(768, 3, 16, 16) * 0.02, torch.randn(768)
    out = torch.zeros(1024, 768, device="cuda")
    K.conv(img.cuda(), ker.cuda(), out, bias=b.cuda())
    want = F.conv2d(img, ker, b, stride=16).squeeze(0).flatten(1).t()
    check(out, want, rtol=1e-4, atol=1e-4)


# ----------------------------------------------------------- sine/cosine ----
@pytest.mark.parametrize("fn,ref", [("sin_float32", torch.sin), ("cos_float32", torch.cos)])
def test_sine_cosine_float32(K, fn, ref):
    """sine/test_sine.py:52-89, cosine/test_cosine.py:63-89: fp32 [32, 64]
    uniform in [-20, 20), rtol 1e-2 atol 1e-3."""
    torch.manual_seed(0)
    x = torch.rand(32, 64) * 40.0 - 20.0
    check(run(getattr(K, fn), x, out_like=x), ref(x), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("fn,ref", [("sin_bfloat16", torch.sin), ("cos_bfloat16", torch.cos)])
def test_sine_cosine_bf16(K, fn, ref):
    """sine/test_sine_bf16_new.py:52-89, cosine/test_cosine_bf16.py:64-91:
    bf16 [32, 64], torch.sin / cos on the bf16 tensor, rtol 1e-2 atol 1e-3."""
    torch.manual_seed(0)
    x = torch.rand(32, 64, dtype=BF16) * 40.0 - 20.0
    check(run(getattr(K, fn), x, out_like=x), ref(x), rtol=1e-2, atol=1e-3)


# ------------------------------------------------------------------ gelu ----
@pytest.mark.parametrize("shape", [(4, 768)])
def test_gelu_float32(K, shape):
    """gelu/test_gelu.py:52-110 (single tile and 1x1 tiling): fp32 nn.GELU(),
    rtol 1e-2 atol 1e-3."""
    torch.manual_seed(0)
    x = torch.randn(*shape)
    check(run(K.gelu, x, out_like=x), nn.GELU()(x), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("shape", [(4, 768), (16, 3072)])
def test_gelu_bf16(K, shape):
    """gelu/test_gelu_bf16.py:26-99: bf16 input, reference nn.GELU() on the
    fp32 cast then bf16, atol 1e-1 rtol 1e-2 (the kernel is the tanh form the
    ViT uses, within that tolerance of the erf reference)."""
    np.random.seed(0)
    x = torch.from_numpy(np.random.randn(*shape).astype(np.float32)).to(BF16)
    check(run(K.gelu_bf16, x, out_like=x), nn.GELU()(x.float()).to(BF16), rtol=1e-2, atol=1e-1)


@pytest.mark.parametrize("fn,shape", [("gelu", (4, 768)), ("gelu", (16, 3072)),
                                      ("gelu_small", (16, 768))])
def test_gelu_bf16_new(K, fn, shape):
    """gelu/test_gelu_bf16_new.py:63-290: nn.GELU() on the bf16 tensor, rtol
    1e-2 atol 1e-3 (single tile, 4x4 tiling, small-tile entry)."""
    torch.manual_seed(0)
    x = torch.randn(*shape, dtype=BF16)
    check(run(getattr(K, fn), x, out_like=x), nn.GELU()(x), rtol=1e-2, atol=1e-3)


# ------------------------------------------------------------------ silu ----
@pytest.mark.parametrize("shape", [(4, 768), (16, 3072)])
def test_silu_float32(K, shape):
    """silu/test_silu.py:24-121: fp32 nn.SiLU, rtol 1e-2."""
    torch.manual_seed(0)
    x = torch.randn(*shape)
    check(run(K.silu_float32, x, out_like=x), nn.SiLU()(x), rtol=1e-2)


@pytest.mark.parametrize("shape", [(4, 768), (16, 3072)])
def test_silu_bf16(K, shape):
    """silu/test_silu_bf16.py:24-92: nn.SiLU on the fp32 cast then bf16, atol
    1e-1 rtol 1e-2."""
    np.random.seed(0)
    x = torch.from_numpy(np.random.randn(*shape).astype(np.float32)).to(BF16)
    check(run(K.silu_bf16, x, out_like=x), nn.SiLU()(x.float()).to(BF16), rtol=1e-2, atol=1e-1)


@pytest.mark.parametrize("fn,shape", [("silu_bf16", (4, 768)), ("silu_bf16", (16, 3072)),
                                      ("silu_bf16_small", (16, 768))])
def test_silu_bf16_new(K, fn, shape):
    """silu/test_silu_bf16_new.py:25-225: nn.SiLU on the bf16 tensor, rtol
    1e-2 atol 1e-3."""
    torch.manual_seed(0)
    x = torch.randn(*shape, dtype=BF16)
    check(run(getattr(K, fn), x, out_like=x), nn.SiLU()(x), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("fn,cols", [("silu_128_float32", 128), ("silu_160_float32", 160)])
def test_vla_silu_float32(K, fn, cols):
    """vla/tests/test_silu_128.py:38-48, test_silu_160.py:38-48: fp32 [4, cols],
    rtol 1e-2 atol 1e-3."""
    torch.manual_seed(0)
    x = torch.randn(4, cols)
    check(run(getattr(K, fn), x, out_like=x), nn.SiLU()(x), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("fn,cols", [("silu_128_bf16", 128), ("silu_160_bf16", 160),
                                     ("silu_256_bf16", 256)])
def test_vla_silu_bf16(K, fn, cols):
    """vla/tests/test_silu_{128,160,256}_bf16.py: nn.SiLU on the bf16 tensor,
    rtol 1e-1 atol 5e-2 (the 128-column kernel takes the reference's 256-wide
    zero-padded tile, test_silu_128_bf16.py:50-58)."""
    torch.manual_seed(0)
    x = torch.randn(4, cols, dtype=BF16)
    want = nn.SiLU()(x)
    if cols == 128:
        xp = torch.zeros(4, 256, dtype=BF16)
        xp[:, :128] = x
        got = run(getattr(K, fn), xp, out_like=xp)[:, :128]
    else:
        got = run(getattr(K, fn), x, out_like=x)
    check(got, want, rtol=1e-1, atol=5e-2)


# ----------------------------------------------------------------- norms ----
class RMSNormHarness(nn.Module):
    """The harness tests' module (rms_norm/test_rms.py:25-33)."""

    def __init__(self, eps=1e-6):
        super().__init__()
        self.eps = eps

    def forward(self, x, weight):
        norm = x.norm(2, dim=-1, keepdim=True)
        rms = norm / (x.shape[-1] ** 0.5)
        return x / (rms + self.eps) * weight


def test_rms_norm_float32(K):
    """rms_norm/test_rms.py:36-87: fp32 [4, 768], rtol 1e-2 atol 1e-3."""
    torch.manual_seed(0)
    x, w = torch.randn(4, 768), torch.randn(768)
    out = torch.zeros(4, 768, device="cuda")
    K.rms_norm(x.cuda(), w.cuda(), out)
    check(out, RMSNormHarness()(x, w), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("fn,shape", [("rms_norm", (4, 768)), ("rms_norm", (16, 768)),
                                      ("rms_norm_small", (16, 192))])
def test_rms_norm_bf16_new(K, fn, shape):
    """rms_norm/test_rms_norm_bf16_new.py:36-309: the module on bf16 tensors
    (rounded after every op), rtol 1e-2 atol 1e-3."""
    torch.manual_seed(0)
    x, w = torch.randn(*shape, dtype=BF16), torch.randn(shape[1], dtype=BF16)
    out = torch.zeros(*shape, dtype=BF16, device="cuda")
    getattr(K, fn)(x.cuda(), w.cuda(), out)
    check(out, RMSNormHarness()(x, w), rtol=1e-2, atol=1e-3)


def test_rms_norm_bf16(K):
    """rms_norm/test_rms_norm_bf16.py:51-80: bf16 [64, 768], unit weight,
    reference nn.RMSNorm in fp32 then bf16, atol 1e-1 rtol 1e-2."""
    np.random.seed(0)
    x = torch.from_numpy(np.random.randn(64, 768).astype(np.float32)).to(BF16)
    w = torch.ones(768, dtype=BF16)
    out = torch.zeros(64, 768, dtype=BF16, device="cuda")
    K.rms_norm_bf16(x.cuda(), w.cuda(), out)
    ref = nn.RMSNorm(768, elementwise_affine=True)
    check(out, ref(x.float()).detach().to(BF16), rtol=1e-2, atol=1e-1)


def test_rms_norm_960_float32(K):
    """vla/tests/test_rms_norm_960.py:40-62: fp32 [2, 960], the harness module,
    rtol 1e-3 atol 1e-4."""
    torch.manual_seed(0)
    x, w = torch.randn(2, 960), torch.randn(960)
    out = torch.zeros(2, 960, device="cuda")
    K.rms_norm_960(x.cuda(), w.cuda(), out)
    check(out, RMSNormHarness()(x, w), rtol=1e-3, atol=1e-4)


def test_rms_norm_960_bf16(K):
    """vla/tests/test_rms_norm_960_bf16.py:42-65: bf16 [4, 960], the module in
    fp32 then bf16, rtol 2e-2 atol 1e-1."""
    torch.manual_seed(0)
    x, w = torch.randn(4, 960, dtype=BF16), torch.randn(960, dtype=BF16)
    out = torch.zeros(4, 960, dtype=BF16, device="cuda")
    K.rms_norm_960_bf16(x.cuda(), w.cuda(), out)
    check(out, RMSNormHarness()(x.float(), w.float()).to(BF16), rtol=2e-2, atol=1e-1)


def test_layer_norm_float32(K):
    """layer_norm/test_layer.py:136-183: fp32 [64, 768] uniform in [-1, 1),
    gamma and beta uniform in [0, 1), nn.LayerNorm (eps 1e-5), rtol 1e-2
    atol 1e-3."""
    torch.manual_seed(0)
    x = torch.rand(64, 768) * 2.0 - 1.0
    g, b = torch.rand(768), torch.rand(768)
    out = torch.zeros(64, 768, device="cuda")
    K.layer_norm(x.cuda(), g.cuda(), out, bias=b.cuda())
    ln = nn.LayerNorm(768, elementwise_affine=True)
    with torch.no_grad():
        ln.weight.copy_(g)
        ln.bias.copy_(b)
        want = ln(x)
    check(out, want, rtol=1e-2, atol=1e-3)


def test_layer_norm_bf16(K):
    """layer_norm/test_layer_bf16.py:66-101: bf16 [64, 768], default gamma /
    beta, nn.LayerNorm in fp32 then bf16, atol 1e-1 rtol 1e-2."""
    np.random.seed(0)
    x = torch.from_numpy(np.random.randn(64, 768).astype(np.float32)).to(BF16)
    g, b = torch.ones(768, dtype=BF16), torch.zeros(768, dtype=BF16)
    out = torch.zeros(64, 768, dtype=BF16, device="cuda")
    K.layer_norm_bf16(x.cuda(), g.cuda(), out, bias=b.cuda())
    ln = nn.LayerNorm(768, elementwise_affine=True)
    with torch.no_grad():
        want = ln(x.float()).to(BF16)
    check(out, want, rtol=1e-2, atol=1e-1)


def layernorm_chain(x, weight, eps=1e-5):
    """layer_norm/test_layer_bf16_new.py:25-34 (torch ops on bf16 tensors)."""
    mean = x.mean(dim=-1, keepdim=True)
    var = x.var(dim=-1, unbiased=False, keepdim=True)
    return (x - mean) / torch.sqrt(var + eps) * weight


@pytest.mark.parametrize("fn,shape", [("layer_norm", (4, 768)), ("layer_norm", (16, 768)),
                                      ("layer_norm_small", (16, 192))])
def test_layer_norm_bf16_new(K, fn, shape):
    """layer_norm/test_layer_bf16_new.py:36-306: gamma only, rtol 1e-2 atol
    1e-3."""
    torch.manual_seed(0)
    x, w = torch.randn(*shape, dtype=BF16), torch.randn(shape[1], dtype=BF16)
    out = torch.zeros(*shape, dtype=BF16, device="cuda")
    getattr(K, fn)(x.cuda(), w.cuda(), out)
    check(out, layernorm_chain(x, w), rtol=1e-2, atol=1e-3)


# --------------------------------------------------------------- softmax ----
def test_masked_softmax_float32(K):
    """masked_softmax/test_masked_softmax.py:33-96: fp32 [64, 3 heads x 64],
    causal by global row (tile row starts [0, 32]), rtol 1e-2."""
    torch.manual_seed(0)
    s = torch.randn(64, 3 * 64)
    out = torch.zeros(64, 3 * 64, device="cuda")
    K.masked_softmax_float32(s.cuda(), torch.tensor([0], dtype=torch.int32), out, heads=3)
    t = s.view(64, 3, 64)
    mask = torch.triu(torch.ones(64, 64, dtype=torch.bool), diagonal=1).unsqueeze(1)
    want = F.softmax(t.masked_fill(mask, float("-inf")), dim=-1).view(64, 192)
    check(out, want, rtol=1e-2)


def _causal_ref(s, row_start):
    r = s.clone()
    for i in range(r.shape[0]):
        r[i, row_start + i + 1:] = float("-inf")
    return F.softmax(r, dim=-1)


@pytest.mark.parametrize("row_start", [0, 96])
def test_masked_softmax_128_float32(K, row_start):
    """vla/tests/test_masked_softmax_128.py:43-81: fp32 [8, 128], row_start 0
    and 96, rtol 1e-3 atol 1e-4."""
    torch.manual_seed(row_start)
    s = torch.randn(8, 128)
    out = torch.zeros(8, 128, device="cuda")
    K.masked_softmax_128_float32(s.cuda(), np.array([row_start], dtype=np.int32), out)
    check(out, _causal_ref(s, row_start), rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("row_start", [0, 96])
def test_masked_softmax_128_bf16(K, row_start):
    """vla/tests/test_masked_softmax_128_bf16.py:44-84: bf16 [8, 128], fp32
    reference then bf16, rtol 5e-2 atol 5e-3."""
    torch.manual_seed(row_start)
    s = torch.randn(8, 128, dtype=BF16)
    out = torch.zeros(8, 128, dtype=BF16, device="cuda")
    K.masked_softmax_128_bf16(s.cuda(), np.array([row_start], dtype=np.int32), out)
    check(out, _causal_ref(s.float(), row_start).to(BF16), rtol=5e-2, atol=5e-3)


def test_softmax_bf16_seq1024(K):
    """softmax_bf16/test_softmax_bf16_seq1024.py: [4, 512] storage = 2 rows of
    1024, softmax per 1024-row in fp32, then bf16."""
    torch.manual_seed(0)
    s = torch.randn(4, 512, dtype=BF16)
    out = torch.zeros(4, 512, dtype=BF16, device="cuda")
    K.softmax_bf16_seq1024(s.cuda(), out)
    want = F.softmax(s.float().view(2, 1024), dim=-1).to(BF16).view(4, 512)
    check(out, want, rtol=1e-2, atol=1e-3)


# ------------------------------------------------------------------ GEMM ----
def test_gemm_error(K):
    """gemm/test_gemm_error.py:44-58: 64 x 960 output of a K = 128 bf16 GEMM
    against the fp32 product; the reference's rtol 1e-1 (it also feeds the
    product in two K chunks scaled by 100 -- one fp32-accumulated pass here)."""
    np.random.seed(0)
    x = torch.from_numpy(np.random.randn(64, 128).astype(np.float32)).to(BF16)
    y = torch.from_numpy(np.random.randn(128, 960).astype(np.float32)).to(BF16)
    out = torch.zeros(64, 960, dtype=BF16, device="cuda")
    K.gemm(x.cuda(), y.cuda(), out)
    check(out, (x.float() @ y.float()).to(BF16), rtol=1e-1, atol=1e-2)


def test_connector_precision(K):
    """vla/test_connector_precision.py: the connector product 64 x 960 with
    K = 12288 accumulated in fp32 once (the reference's "float32
    accumulation" variant, its tests 1 and 3), against the fp32 product cast
    to bf16 at the reference's rtol 0.01 (elements above 1e-6; atol 1e-2 for
    the handful near zero)."""
    np.random.seed(0)
    A = torch.from_numpy(np.random.randn(64, 12288).astype(np.float32)).to(BF16)
    B = torch.from_numpy(np.random.randn(12288, 960).astype(np.float32)).to(BF16)
    out = torch.zeros(64, 960, dtype=BF16, device="cuda")
    K.gemm(A.cuda(), B.cuda(), out)
    want = (A.float() @ B.float()).to(BF16)
    check(out, want, rtol=1e-2, atol=1e-2)


def test_pixel_shuffle_layout(K):
    """vla/test_pixel_shuffle.py / the connector's pixel-shuffle reshape chain
    (vla/vla.py:434-437): the gather-addressed A operand against an identity
    weight reproduces the reshaped rows exactly (bit-exact bf16)."""
    from smolvla import ops
    torch.manual_seed(0)
    grid, hid, s = 8, 16, 4
    x = torch.randn(2, grid * grid, hid).to(BF16)
    kdim = hid * s * s
    eye = torch.eye(kdim).to(BF16)
    got = ops.connector(x.cuda(), ops.pack_weight(eye.cuda()), s)
    gs = grid // s
    want = []
    for im in range(2):
        t = x[im].reshape(grid, grid, hid).reshape(grid, gs, s * hid).transpose(0, 1)
        t = t.reshape(gs, gs, s * s * hid).transpose(0, 1).reshape(gs * gs, kdim)
        want.append(t)
    assert torch.equal(got.cpu(), torch.cat(want))


# ------------------------------------------------------------------ RoPE ----
def _precompute_sin_cos(seq_len, d, theta=10_000.0, pos_offset=0):
    """vla/test_rope_fused.py:43-55: packed [sin | cos] per row."""
    half = d // 2
    k = np.arange(half, dtype=np.float32)
    inv_ts = theta ** (-(2.0 / d) * k)
    pos = (pos_offset + np.arange(seq_len)).astype(np.float32)[:, None]
    rad = pos * inv_ts[None, :]
    sc = np.zeros((seq_len, d), dtype=np.float32)
    sc[:, :half] = np.sin(rad)
    sc[:, half:] = np.cos(rad)
    return sc


def test_rope_fused_float32(K):
    """vla/test_rope_fused.py:58-153: 64 rows x 8 heads of 64 in 32-row tiles,
    one rope_fused_float32 call per (tile, head), against apply_rope, rtol
    1e-3 atol 1e-4."""
    torch.manual_seed(0)
    seq, heads, d = 64, 8, 64
    x = torch.randn(1, seq, heads, d)
    q = x.squeeze(0).reshape(seq, heads * d)
    out = torch.zeros(seq, heads * d)
    for t0 in range(0, seq, 32):
        sc = torch.from_numpy(_precompute_sin_cos(32, d, pos_offset=t0)).cuda()
        for h in range(heads):
            tile = q[t0:t0 + 32, h * d:(h + 1) * d].contiguous().cuda()
            o = torch.zeros(32, d, device="cuda")
            K.rope_fused_float32(tile, sc, o)
            out[t0:t0 + 32, h * d:(h + 1) * d] = o.cpu()
    pos = torch.arange(seq, dtype=torch.float32)
    ts = 10_000 ** ((2.0 / d) * torch.arange(d // 2, dtype=torch.float32))
    rad = (pos[:, None] / ts[None, :])[:, None, :]
    x1, x2 = x[0, ..., :d // 2], x[0, ..., d // 2:]
    want = torch.cat([x1 * torch.cos(rad) - x2 * torch.sin(rad),
                      x2 * torch.cos(rad) + x1 * torch.sin(rad)], dim=-1).reshape(seq, heads * d)
    check(out, want, rtol=1e-3, atol=1e-4)


def test_rope_multiple(K):
    """vla/test_rope_multiple.py:262-282: the composed RoPE (radians, pack,
    sin, cos, copy, mul, add, sub, join sub-kernels) on 64 rows x 15 heads,
    here one fused pass over all heads, rtol 1e-3 atol 1e-4."""
    from smolvla import ops
    torch.manual_seed(0)
    seq, heads, d = 64, 15, 64
    q = torch.randn(seq, heads * d)
    cos_t, sin_t = ops.rope_table(seq, d, 10_000.0, device="cuda")
    got = ops.rope(q.cuda(), heads, cos_t, sin_t, pos_offset=0, out_f32=True)
    x4 = q.view(seq, heads, d)
    k = torch.arange(d // 2, dtype=torch.float32)
    inv = (10_000.0 ** (-(2.0 / d) * k)).view(1, 1, -1)
    rad = torch.arange(seq, dtype=torch.float32).view(seq, 1, 1) * inv
    s, c = torch.sin(rad), torch.cos(rad)
    xl, xr = x4[:, :, :d // 2], x4[:, :, d // 2:]
    want = torch.cat([xl * c - xr * s, xr * c + xl * s], dim=-1).reshape(seq, heads * d)
    check(got, want, rtol=1e-3, atol=1e-4)
