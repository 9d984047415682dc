"""Pins the CPU oracle (``oracle/smolvla_ref.py``) against independent checks.

The reference ships no golden vectors (its tests compute expectations live
from seeded torch), so every oracle function is pinned here against something
that does not share its code:

===========================  ===================================================
oracle function              pinned by
===========================  ===================================================
rms_norm                     closed form (fp32, one rounding); unit-RMS invariant
layer_norm                   closed form; zero-mean/unit-var invariant
apply_rope / rope_tables     transformers Llama rotary code (fp32); identity at
                             position 0; norm preservation per pair
gqa_attention / make_mask    float64 brute-force loops; SDPA with enable_gqa;
                             uniform-attention closed form
decoder_block                transformers LlamaDecoderLayer (fp32, local config)
expert_self_block            same (causal decoder layer)
expert_cross_block           float64 brute force; Wq=0 closed form
vit_block                    transformers SiglipEncoderLayer (fp32, local config);
                             torch nn.MultiheadAttention block (reference MiniVit
                             structure, bf16)
patch_embed                  transformers SiglipVisionEmbeddings; brute force
pixel_shuffle / connector    transformers Idefics3Connector; explicit index map
lang_embed / state_embed     nn.Embedding * sqrt(H); matmul
time_embedding               closed form sin/cos; sin^2+cos^2 = 1
masked_softmax_rows          the reference test's own mask loop
smolvla_chunk                Euler loop with a constant velocity (closed form);
                             batch independence
===========================  ===================================================
"""

import math
import types

import pytest
import torch
import torch.nn.functional as F

import oracle.smolvla_ref as ref
from smolvla.config import DecoderConfig, SmolVLAConfig, VitConfig, small_config
from smolvla.params import (decoder_layer_params, expert_cross_layer_params, smolvla_inputs,
                            smolvla_params, vit_layer_params, _Gen, tree_map)

F32 = torch.float32
F64 = torch.float64
BF16 = torch.bfloat16


@pytest.fixture
def fp32_probs(monkeypatch):
    monkeypatch.setattr(ref, "P_DTYPE", torch.float32)


def to32(t):
    return tree_map(lambda x: x.float(), t)


# --------------------------------------------------------------------------
def test_rms_norm_closed_form():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(16, 960, generator=g).to(BF16)
    w = (1 + 0.1 * torch.randn(960, generator=g)).to(BF16)
    for eps in (1e-5, None):
        e = torch.finfo(F32).eps if eps is None else eps
        xf = x.float()
        want = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + e) * w.float()).to(BF16)
        assert torch.equal(ref.rms_norm(x, w, eps), want)
    # unit RMS with unit gain
    y = ref.rms_norm(x.float(), torch.ones(960), 1e-5)
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(16), atol=1e-4)


def test_layer_norm_closed_form():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(8, 768, generator=g) * 3 + 1
    y = ref.layer_norm(x, torch.ones(768), torch.zeros(768), 1e-6)
    assert torch.allclose(y.mean(-1), torch.zeros(8), atol=1e-5)
    assert torch.allclose(y.var(-1, unbiased=False), torch.ones(8), atol=1e-4)
    gam, bet = torch.randn(768, generator=g), torch.randn(768, generator=g)
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    want = (x - mu) / torch.sqrt(var + 1e-6) * gam + bet
    assert torch.allclose(ref.layer_norm(x, gam, bet, 1e-6), want, atol=1e-4)


# --------------------------------------------------------------------------
def test_rope_matches_transformers_llama():
    from transformers.models.llama.configuration_llama import LlamaConfig
    from transformers.models.llama.modeling_llama import (LlamaRotaryEmbedding,
                                                          apply_rotary_pos_emb)
    for theta in (10000.0, 100000.0):
        cfg = LlamaConfig(hidden_size=960, num_attention_heads=15, num_key_value_heads=5,
                          head_dim=64, rope_theta=theta, max_position_embeddings=512)
        rot = LlamaRotaryEmbedding(cfg)
        L = 241
        g = torch.Generator().manual_seed(2)
        x = torch.randn(1, L, 15, 64, generator=g)
        pos = torch.arange(L)[None]
        cos, sin = rot(x, pos)
        want, _ = apply_rotary_pos_emb(x.transpose(1, 2), x.transpose(1, 2), cos, sin)
        got = ref.apply_rope(x, theta)
        # angles up to 240 rad: fp32 pos*inv_freq vs pos/timescale differ by ulps
        assert torch.allclose(got, want.transpose(1, 2), atol=2e-4, rtol=1e-4)


def test_rope_invariants():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 50, 5, 64, generator=g)
    y = ref.apply_rope(x, 100000.0)
    assert torch.equal(y[:, 0], x[:, 0])                     # position 0: identity
    n_in = x[..., :32] ** 2 + x[..., 32:] ** 2
    n_out = y[..., :32] ** 2 + y[..., 32:] ** 2
    assert torch.allclose(n_in, n_out, rtol=1e-5, atol=1e-5)  # rotation per pair
    c, s = ref.rope_tables(3, 64, 100000.0)
    assert abs(c[1, 1].item() - math.cos(1.0 / 100000.0 ** (2 / 64))) < 1e-6
    assert abs(s[2, 31].item() - math.sin(2.0 / 100000.0 ** (62 / 64))) < 1e-7


# --------------------------------------------------------------------------
def _brute_attention(q, k, v, mask):
    """float64 per-head loops from the definition."""
    B, L, Hq, D = q.shape
    Lk, Hkv = k.shape[1], k.shape[2]
    out = torch.zeros(B, L, Hq, D, dtype=F64)
    for b in range(B):
        for h in range(Hq):
            g = h // (Hq // Hkv)
            for i in range(L):
                s = torch.tensor([float(q[b, i, h].double() @ k[b, j, g].double()) / math.sqrt(D)
                                  for j in range(Lk)], dtype=F64)
                if mask is not None:
                    s[mask[i]] = -math.inf
                p = torch.softmax(s, 0)
                out[b, i, h] = p @ v[b, :, g].double()
    return out.reshape(B, L, Hq * D)


@pytest.mark.parametrize("kind", ["causal", "none", "prefix_lm"])
def test_gqa_attention_brute_force(kind, fp32_probs):
    g = torch.Generator().manual_seed(4)
    B, L, Hq, Hkv, D = 2, 9, 6, 2, 16
    q = torch.randn(B, L, Hq, D, generator=g)
    k = torch.randn(B, L, Hkv, D, generator=g)
    v = torch.randn(B, L, Hkv, D, generator=g)
    mask = ref.make_mask(kind, L, L, prefix_len=5)
    got = ref.gqa_attention(q, k, v, mask)
    want = _brute_attention(q, k, v, mask)
    assert torch.allclose(got.double(), want, atol=1e-5)
    sd = F.scaled_dot_product_attention(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
        attn_mask=None if mask is None else ~mask, enable_gqa=True)
    assert torch.allclose(got, sd.transpose(1, 2).reshape(B, L, Hq * D), atol=1e-5)


def test_masks():
    m = ref.make_mask("prefix_lm", 6, 6, prefix_len=4)
    # rows 0..3 see keys 0..3 only; rows 4, 5 see 0..4 / 0..5
    assert m[0].tolist() == [False] * 4 + [True] * 2
    assert m[3].tolist() == [False] * 4 + [True] * 2
    assert m[4].tolist() == [False] * 5 + [True]
    assert not m[5].any()
    c = ref.make_mask("causal", 4, 4)
    assert c.tolist() == [[j > i for j in range(4)] for i in range(4)]


def test_uniform_attention_closed_form():
    # q = 0 -> uniform probabilities -> ctx = mean of visible V rows
    B, L, Hq, Hkv, D = 1, 5, 3, 1, 8
    q = torch.zeros(B, L, Hq, D)
    k = torch.randn(B, L, Hkv, D)
    v = torch.randn(B, L, Hkv, D).to(BF16)
    got = ref.gqa_attention(q, k, v, ref.make_mask("causal", L, L))
    for i in range(L):
        want = v[0, :i + 1, 0].float().mean(0)
        for h in range(Hq):
            assert torch.allclose(got[0, i, h * D:(h + 1) * D].float(), want, atol=2e-2)


# --------------------------------------------------------------------------
def _llama_layer(cfg: DecoderConfig, p, eps):
    from transformers.models.llama.configuration_llama import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer
    lc = LlamaConfig(hidden_size=cfg.hidden, intermediate_size=cfg.inter,
                     num_attention_heads=cfg.n_q_heads, num_key_value_heads=cfg.n_kv_heads,
                     head_dim=cfg.head_dim, rope_theta=cfg.rope_theta, rms_norm_eps=eps,
                     attention_bias=False, mlp_bias=False, hidden_act="silu",
                     max_position_embeddings=1024)
    lc._attn_implementation = "eager"
    layer = LlamaDecoderLayer(lc, 0).eval()
    sd = {
        "self_attn.q_proj.weight": p["Wq"].t(), "self_attn.k_proj.weight": p["Wk"].t(),
        "self_attn.v_proj.weight": p["Wv"].t(), "self_attn.o_proj.weight": p["Wo"].t(),
        "mlp.gate_proj.weight": p["W_gate"].t(), "mlp.up_proj.weight": p["W_up"].t(),
        "mlp.down_proj.weight": p["W_down"].t(),
        "input_layernorm.weight": p["W_norm_1"], "post_attention_layernorm.weight": p["W_norm_2"],
    }
    layer.load_state_dict({k: v.float().contiguous() for k, v in sd.items()})
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    return layer, LlamaRotaryEmbedding(lc)


@pytest.mark.parametrize("mask_kind", ["causal", "prefix_lm"])
def test_decoder_block_matches_transformers_llama(mask_kind, fp32_probs):
    cfg = DecoderConfig()          # 960 / 15q / 5kv / 2560, theta 1e5, eps 1e-5
    gen = _Gen(5, norm_init="random")
    p = to32(decoder_layer_params(gen, cfg))
    L = 64
    x = torch.randn(1, L, cfg.hidden, generator=torch.Generator().manual_seed(6))
    with torch.no_grad():
        got, k, v = ref.decoder_block(x, p, cfg, mask_kind=mask_kind, prefix_len=40)
        layer, rot = _llama_layer(cfg, p, cfg.rms_eps)
        pos = torch.arange(L)[None]
        m = ref.make_mask(mask_kind, L, L, 40)
        add = torch.zeros(1, 1, L, L).masked_fill(m, float("-inf"))
        want = layer(x, attention_mask=add, position_ids=pos, position_embeddings=rot(x, pos))
        want = want[0] if isinstance(want, tuple) else want
    assert torch.allclose(got, want, atol=2e-4, rtol=1e-3), (got - want).abs().max()
    # K/V export (cache mode) = RoPE'd K and V of this layer's own projections
    h = ref.rms_norm(x, p["W_norm_1"], cfg.rms_eps)
    v_want = h @ p["Wv"]
    assert torch.allclose(v, v_want, atol=1e-5)
    k_pre = (h @ p["Wk"]).view(1, L, 5, 64)
    assert torch.allclose(k.view(1, L, 5, 64)[:, 0], k_pre[:, 0], atol=1e-6)
    assert not torch.allclose(k.view(1, L, 5, 64)[:, 5:], k_pre[:, 5:], atol=1e-3)


def test_expert_self_block_is_causal_llama(fp32_probs):
    cfg = DecoderConfig(hidden=720, inter=2048)
    p = to32(decoder_layer_params(_Gen(7, norm_init="random"), cfg))
    x = torch.randn(2, 50, 720, generator=torch.Generator().manual_seed(8))
    with torch.no_grad():
        got = ref.expert_self_block(x, p, cfg)
        layer, rot = _llama_layer(cfg, p, cfg.rms_eps)
        pos = torch.arange(50)[None].expand(2, -1)
        add = torch.zeros(1, 1, 50, 50).masked_fill(ref.make_mask("causal", 50, 50), -math.inf)
        want = layer(x, attention_mask=add, position_ids=pos, position_embeddings=rot(x, pos))
        want = want[0] if isinstance(want, tuple) else want
    assert torch.allclose(got, want, atol=2e-4, rtol=1e-3)


def test_expert_cross_block_brute_force(fp32_probs):
    cfg = DecoderConfig(hidden=144, inter=192, n_q_heads=3, n_kv_heads=1)
    p = to32(expert_cross_layer_params(_Gen(9, norm_init="random"), cfg, 64))
    g = torch.Generator().manual_seed(10)
    x = torch.randn(1, 7, 144, generator=g)
    tk = torch.randn(1, 11, 64, generator=g)
    tv = torch.randn(1, 11, 64, generator=g)
    got = ref.expert_cross_block(x, tk, tv, p, cfg)
    # float64 brute force from the definition
    xd = x.double()
    pd = {k: v.double() for k, v in p.items()}

    def rms(a, w):
        return a / torch.sqrt(a.pow(2).mean(-1, keepdim=True) + cfg.rms_eps) * w
    xn = rms(xd, pd["W_norm_1"])
    q = (xn @ pd["Wq"]).view(1, 7, 3, 64)
    half = 32
    ts = cfg.rope_theta ** ((2.0 / 64) * torch.arange(half, dtype=F64))
    ang = torch.arange(7, dtype=F64)[:, None] / ts[None]
    c, s = torch.cos(ang)[None, :, None], torch.sin(ang)[None, :, None]
    q = torch.cat([q[..., :half] * c - q[..., half:] * s, q[..., half:] * c + q[..., :half] * s], -1)
    k = (tk.double() @ pd["Wk_cross"]).view(1, 11, 1, 64)
    v = (tv.double() @ pd["Wv_cross"]).view(1, 11, 1, 64)
    ctx = _brute_attention(q, k, v, None)
    h = ctx @ pd["Wo"] + xd
    hn = rms(h, pd["W_norm_2"])
    want = (F.silu(hn @ pd["W_gate"]) * (hn @ pd["W_up"])) @ pd["W_down"] + h
    assert torch.allclose(got.double(), want, atol=1e-4)


def test_expert_cross_zero_query_closed_form(fp32_probs):
    # Wq = 0 -> uniform attention over all prefix tokens -> ctx = mean(V)
    cfg = DecoderConfig(hidden=144, inter=192, n_q_heads=3, n_kv_heads=1)
    p = to32(expert_cross_layer_params(_Gen(11), cfg, 64))
    p["Wq"] = torch.zeros_like(p["Wq"])
    p["W_down"] = torch.zeros_like(p["W_down"])
    tk, tv = torch.randn(1, 11, 64), torch.randn(1, 11, 64)
    x = torch.randn(1, 4, 144)
    got = ref.expert_cross_block(x, tk, tv, p, cfg)
    vmean = (tv @ p["Wv_cross"]).mean(1)           # [1, 64]
    ctx = vmean.repeat(1, 3)                       # three query heads share the kv head
    want = x + ctx @ p["Wo"]
    assert torch.allclose(got, want, atol=1e-5)


# --------------------------------------------------------------------------
def _siglip(cfg: VitConfig):
    from transformers.models.siglip.configuration_siglip import SiglipVisionConfig
    sc = SiglipVisionConfig(hidden_size=cfg.hidden, intermediate_size=cfg.inter,
                            num_attention_heads=cfg.n_heads, layer_norm_eps=cfg.ln_eps,
                            hidden_act="gelu_pytorch_tanh", image_size=cfg.image,
                            patch_size=cfg.patch, num_channels=cfg.channels)
    sc._attn_implementation = "eager"
    return sc


def test_vit_block_matches_transformers_siglip():
    from transformers.models.siglip.modeling_siglip import SiglipEncoderLayer
    cfg = VitConfig()
    p = to32(vit_layer_params(_Gen(12, norm_init="random"), cfg))
    layer = SiglipEncoderLayer(_siglip(cfg)).eval()
    sd = {
        "self_attn.q_proj.weight": p["Wq"].t(), "self_attn.q_proj.bias": p["bq"],
        "self_attn.k_proj.weight": p["Wk"].t(), "self_attn.k_proj.bias": p["bk"],
        "self_attn.v_proj.weight": p["Wv"].t(), "self_attn.v_proj.bias": p["bv"],
        "self_attn.out_proj.weight": p["Wo"].t(), "self_attn.out_proj.bias": p["bo"],
        "mlp.fc1.weight": p["W_up"].t(), "mlp.fc1.bias": p["b_up"],
        "mlp.fc2.weight": p["W_down"].t(), "mlp.fc2.bias": p["b_down"],
        "layer_norm1.weight": p["W_norm_1"], "layer_norm1.bias": p["b_norm_1"],
        "layer_norm2.weight": p["W_norm_2"], "layer_norm2.bias": p["b_norm_2"],
    }
    layer.load_state_dict({k: v.contiguous() for k, v in sd.items()})
    x = torch.randn(1, 256, 768, generator=torch.Generator().manual_seed(13))
    with torch.no_grad():
        got = ref.vit_block(x, p, cfg)
        want = layer(x, attention_mask=None)
        want = want[0] if isinstance(want, tuple) else want
    assert torch.allclose(got, want, atol=2e-4, rtol=1e-3)


def test_vit_block_matches_torch_mha_module_bf16():
    """The reference's MiniVit structure built from torch modules
    (nn.MultiheadAttention + LayerNorm + GELU), in bf16."""
    cfg = VitConfig(ln_eps=1e-5, gelu="erf")
    p = vit_layer_params(_Gen(14, norm_init="random"), cfg, biases=False)
    mha = torch.nn.MultiheadAttention(768, 12, batch_first=True)
    with torch.no_grad():
        mha.in_proj_weight.copy_(torch.cat([p["Wq"], p["Wk"], p["Wv"]], 1).t().float())
        mha.in_proj_bias.zero_()
        mha.out_proj.weight.copy_(p["Wo"].t().float())
        mha.out_proj.bias.zero_()
    mha = mha.to(BF16).eval()
    x = torch.randn(1, 128, 768, generator=torch.Generator().manual_seed(15)).to(BF16)
    with torch.no_grad():
        h = F.layer_norm(x, (768,), p["W_norm_1"], p["b_norm_1"], 1e-5)
        a, _ = mha(h, h, h, need_weights=False)
        y = a + x
        h2 = F.layer_norm(y, (768,), p["W_norm_2"], p["b_norm_2"], 1e-5)
        want = y + F.gelu(h2 @ p["W_up"]) @ p["W_down"]
        got = ref.vit_block(x, p, cfg)
    assert torch.allclose(got.float(), want.float(), atol=3e-2, rtol=2e-2)


# --------------------------------------------------------------------------
def test_patch_embed_matches_siglip_embeddings_and_brute_force():
    from transformers.models.siglip.modeling_siglip import SiglipVisionEmbeddings
    cfg = VitConfig(image=64)
    gen = _Gen(16)
    kernel, bias = gen.randn(768, 3, 16, 16).float(), gen.randn(768).float()
    pos = gen.randn(16, 768).float()
    emb = SiglipVisionEmbeddings(_siglip(cfg)).eval()
    emb.load_state_dict({"patch_embedding.weight": kernel, "patch_embedding.bias": bias,
                         "position_embedding.weight": pos}, strict=False)
    img = torch.rand(2, 3, 64, 64) * 2 - 1
    with torch.no_grad():
        got = ref.patch_embed(img, kernel, bias, pos)
        want = emb(img)
    assert torch.allclose(got, want, atol=1e-4)
    # brute force: token r*4+c = dot(patch(r, c), kernel) + bias + pos
    r, c, e = 2, 3, 100
    patch = img[1, :, r * 16:(r + 1) * 16, c * 16:(c + 1) * 16]
    val = (patch * kernel[e]).sum() + bias[e] + pos[r * 4 + c, e]
    assert abs(got[1, r * 4 + c, e].item() - val.item()) < 1e-4


def test_pixel_shuffle_matches_idefics3_and_index_map():
    from transformers.models.idefics3.modeling_idefics3 import Idefics3Connector
    x = torch.randn(2, 1024, 768)
    got = ref.pixel_shuffle(x, 4)
    conn = Idefics3Connector.__new__(Idefics3Connector)
    conn.scale_factor = 4
    want = Idefics3Connector.pixel_shuffle(conn, x, 4)
    assert torch.equal(got, want)
    # explicit index map used by the GPU connector's gathered A operand:
    # out[i][t*3072 + s*768 + c] = x[(4*(i//8)+t)*32 + 4*(i%8)+s][c]
    for i in (0, 9, 63):
        for t in range(4):
            for s in range(4):
                src = (4 * (i // 8) + t) * 32 + 4 * (i % 8) + s
                assert torch.equal(got[1, i, t * 3072 + s * 768:(t * 3072 + s * 768) + 768],
                                   x[1, src])


def test_connector_matches_idefics3():
    from transformers.models.idefics3.configuration_idefics3 import Idefics3Config
    from transformers.models.idefics3.modeling_idefics3 import Idefics3Connector
    cfg = Idefics3Config(scale_factor=4)
    cfg.vision_config.hidden_size = 768
    cfg.text_config.hidden_size = 960
    conn = Idefics3Connector(cfg).eval()
    w = torch.randn(12288, 960) * 0.02
    conn.modality_projection.proj.weight.data.copy_(w.t())
    x = torch.randn(1, 1024, 768)
    with torch.no_grad():
        assert torch.allclose(ref.connector(x, w, 4), conn(x), atol=1e-4)


def test_embeddings():
    table = torch.randn(100, 960).to(BF16)
    ids = torch.tensor([[3, 7, 99]])
    emb = torch.nn.Embedding(100, 960).to(BF16)
    emb.weight.data.copy_(table)
    want = (emb(ids).float() * math.sqrt(960)).to(BF16)
    assert torch.equal(ref.lang_embed(ids, table), want)
    st = torch.randn(2, 1, 32)
    w = torch.randn(32, 960)
    assert torch.allclose(ref.state_embed(st, w), st @ w, atol=1e-5)


def test_time_embedding_closed_form():
    t = torch.tensor([0.0, 0.3, 1.0])
    e = ref.time_embedding(t, 720)
    assert e.shape == (3, 720)
    assert torch.allclose(e[0, :360], torch.zeros(360)) and torch.allclose(e[0, 360:], torch.ones(360))
    assert torch.allclose(e[:, :360] ** 2 + e[:, 360:] ** 2, torch.ones(3, 360), atol=1e-6)
    # first frequency has the minimum period 4e-3, the last the maximum 4.0
    t1 = float(t[1])                                   # fp32 value of 0.3
    assert abs(e[1, 0].item() - math.sin(2 * math.pi * t1 / 4e-3)) < 1e-6
    assert abs(e[1, 359].item() - math.sin(2 * math.pi * t1 / 4.0)) < 1e-6


def test_masked_softmax_rows_matches_reference_test_loop():
    # vla/tests/test_masked_softmax_128_bf16.py:47-55
    g = torch.Generator().manual_seed(42)
    for row_start in (0, 96):
        s = torch.randn(8, 128, generator=g).to(BF16)
        r = s.float().clone()
        for i in range(8):
            for c in range(128):
                if c > row_start + i:
                    r[i, c] = float("-inf")
        want = F.softmax(r, dim=-1).to(BF16)
        got = ref.masked_softmax_rows(s, row_start)
        assert torch.equal(got, want)
        assert torch.allclose(got.float().sum(-1), torch.ones(8), atol=1e-2)
        for i in range(8):
            assert (got[i, row_start + i + 1:] == 0).all()


# --------------------------------------------------------------------------
def test_euler_loop_closed_form(monkeypatch):
    cfg = small_config()
    P = smolvla_params(cfg, seed=0)
    imgs, ids, st, noise = smolvla_inputs(cfg, 1)
    seen = []

    def fake_velocity(x_t, t, ckv, params, c, cross_src=None):
        seen.append(t)
        return torch.full_like(x_t, 0.5).to(BF16)
    monkeypatch.setattr(ref, "expert_velocity", fake_velocity)
    out = ref.smolvla_chunk(imgs, ids, st, noise, P, cfg)
    assert torch.allclose(out, noise - 0.5, atol=1e-6)       # sum of dt = -1
    assert len(seen) == cfg.num_steps
    assert all(abs(a - b) < 1e-9 for a, b in zip(seen, [1 - i / cfg.num_steps
                                                         for i in range(cfg.num_steps)]))


def test_chunk_batch_independence():
    cfg = small_config()
    P = smolvla_params(cfg, seed=0, norm_init="random")
    imgs, ids, st, noise = smolvla_inputs(cfg, 2)
    both = ref.smolvla_chunk(imgs, ids, st, noise, P, cfg)
    one = ref.smolvla_chunk(imgs[1:], ids[1:], st[1:], noise[1:], P, cfg)
    assert torch.allclose(both[1:], one, atol=1e-6)
    assert both.shape == (2, cfg.chunk, cfg.action_dim)
    assert torch.isfinite(both).all()
