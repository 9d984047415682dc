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
is_cross                     layer parity of vla/vla.py:204-211 (SKIP = 2)
expert_input                 float64 closed form; each half of W_time_in zeroed
                             in turn (the output then ignores x, or t)
build_prefix                 a distinct constant per source, checked row by row
                             (the [cameras | language | state] order, vla/vla.py:326)
cross_kv                     float64 projection of the same layer's K/V
_cross_with_projected        equals expert_cross_block (itself brute-forced)
expert_output                float64 RMSNorm then matmul
expert_velocity              zero layer weights (identity blocks) closed form;
                             one live cross layer with Wq = 0 (uniform attention
                             over that layer's projected V)
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


# --------------------------------------------------------------------------
# Wiring of the BASELINE-only pieces (absent from the reference, whose whole
# composition is vla/vla.py:194-222 and :326).  Each pin below is a closed form
# that a plausible wiring mistake (swapped concat or weight half, another token
# order, the wrong cross layer or K/V source, a dropped residual) fails.
def _small_fp32(seed=0):
    cfg = small_config()
    return cfg, to32(smolvla_params(cfg, seed=seed, norm_init="random"))


def _d(t):
    return t.double()


def test_is_cross_layer_parity():
    # vla/vla.py:79, 204-211: layer i self-attends when i % SKIP == 0 (SKIP = 2)
    cfg = SmolVLAConfig()
    assert [cfg.is_cross(i) for i in range(cfg.expert_layers)] == [i % 2 == 1 for i in range(16)]
    cfg_s = small_config()
    P = smolvla_params(cfg_s, seed=0)
    for i, lp in enumerate(P["expert"]):
        assert ("Wk_cross" in lp) == (i % 2 == 1)


def test_expert_input_halves_of_time_in():
    """time_in multiplies concat([action_in(x), temb(t)]): rows [0, H) of
    W_time_in see the action embedding, rows [H, 2H) the time embedding."""
    cfg, P = _small_fp32(1)
    io = P["expert_io"]
    H = cfg.expert.hidden
    g = torch.Generator().manual_seed(3)
    x1 = torch.randn(2, cfg.chunk, cfg.action_dim, generator=g)
    x2 = torch.randn(2, cfg.chunk, cfg.action_dim, generator=g)

    def closed(x, t, w_tin):
        a = _d(x) @ _d(io["W_action_in"]) + _d(io["b_action_in"])
        k = torch.arange(H // 2, dtype=F64)
        period = 4e-3 * (4.0 / 4e-3) ** (k / (H // 2 - 1))
        ang = 2 * math.pi * float(torch.tensor(t, dtype=F32)) / period
        te = torch.cat([torch.sin(ang), torch.cos(ang)])[None, None, :].expand(*a.shape[:2], H)
        h = a @ _d(w_tin[:H]) + te @ _d(w_tin[H:]) + _d(io["b_time_in"])
        h = h * torch.sigmoid(h)
        return h @ _d(io["W_time_out"]) + _d(io["b_time_out"])

    # the full projection against the closed form
    for x, t in ((x1, 1.0), (x2, 0.3)):
        got = ref.expert_input(x, t, P, cfg)
        assert torch.allclose(_d(got), closed(x, t, io["W_time_in"]), atol=1e-4)
    # action half zeroed: the result depends on t only
    Pa = tree_map(lambda t: t.clone(), P)
    Pa["expert_io"]["W_time_in"][:H] = 0
    ya1, ya2 = ref.expert_input(x1, 0.7, Pa, cfg), ref.expert_input(x2, 0.7, Pa, cfg)
    assert torch.equal(ya1, ya2)
    assert not torch.allclose(ya1, ref.expert_input(x1, 0.2, Pa, cfg), atol=1e-3)
    assert torch.allclose(_d(ya1), closed(x1, 0.7, Pa["expert_io"]["W_time_in"]), atol=1e-4)
    # time half zeroed: the result depends on x only
    Pt = tree_map(lambda t: t.clone(), P)
    Pt["expert_io"]["W_time_in"][H:] = 0
    yt1, yt2 = ref.expert_input(x1, 0.7, Pt, cfg), ref.expert_input(x1, 0.2, Pt, cfg)
    assert torch.equal(yt1, yt2)
    assert not torch.allclose(yt1, ref.expert_input(x2, 0.7, Pt, cfg), atol=1e-3)
    assert torch.allclose(_d(yt1), closed(x1, 0.7, Pt["expert_io"]["W_time_in"]), atol=1e-4)


def test_build_prefix_token_order():
    """[camera 0 | camera 1 | ... | language | state] per sample (vla/vla.py:326),
    each source written as a distinct constant so every row names its source."""
    cfg = small_config()
    P = to32(smolvla_params(cfg, seed=0))
    B, C = 2, cfg.n_cameras
    N, E = cfg.vit.tokens, cfg.vit.hidden
    K = E * cfg.pixel_shuffle ** 2
    H = cfg.decoder.hidden
    it = cfg.image_tokens
    vis = torch.empty(B, C, N, E)
    for b in range(B):
        for c in range(C):
            vis[b, c] = 1.0 + c + 10.0 * b          # connector output = mean = this value
    P["connector"]["W"] = torch.full((K, H), 1.0 / K)
    ids = torch.stack([torch.arange(cfg.lang_tokens) + 100 * b for b in range(B)])
    P["embed"] = torch.arange(cfg.vocab, dtype=F32)[:, None].expand(cfg.vocab, H).contiguous()
    state = torch.ones(B, cfg.state_dim)
    P["state"]["W"] = torch.full((cfg.state_dim, H), -7.0 / cfg.state_dim)
    pre = ref.build_prefix(vis, ids, state, P, cfg)
    assert pre.shape == (B, cfg.prefix_len, H)
    sq = math.sqrt(H)
    for b in range(B):
        for c in range(C):
            rows = pre[b, c * it:(c + 1) * it]
            assert torch.allclose(rows, torch.full_like(rows, 1.0 + c + 10.0 * b), atol=1e-4)
        lang = pre[b, C * it:C * it + cfg.lang_tokens, 0]
        want = (torch.arange(cfg.lang_tokens, dtype=F64) + 100 * b) * sq
        assert torch.allclose(_d(lang), want, rtol=1e-6)
        assert torch.allclose(pre[b, -1], torch.full((H,), -7.0), atol=1e-4)
    assert cfg.prefix_len == C * it + cfg.lang_tokens + 1


def test_cross_kv_uses_the_same_layer():
    """cross_kv projects layer i's prefix K/V for every cross layer i, no other
    (vla/vla.py:207-211: text_k/text_v of VLM layer i feed expert layer i)."""
    cfg, P = _small_fp32(2)
    L, d = cfg.prefix_len, cfg.decoder
    g = torch.Generator().manual_seed(4)
    kv = [(torch.randn(1, L, d.kv_dim, generator=g), torch.randn(1, L, d.kv_dim, generator=g))
          for _ in range(cfg.prefix_layers)]
    out = ref.cross_kv(kv, P, cfg)
    assert sorted(out) == [i for i in range(cfg.expert_layers) if i % 2 == 1]
    for i, (k, v) in out.items():
        lp = P["expert"][i]
        assert torch.allclose(_d(k), _d(kv[i][0]) @ _d(lp["Wk_cross"]), atol=1e-5)
        assert torch.allclose(_d(v), _d(kv[i][1]) @ _d(lp["Wv_cross"]), atol=1e-5)


def test_cross_with_projected_equals_cross_block(fp32_probs):
    """The cross layer on K/V projected ahead of time is the reference cross
    block (vla/action_expert_bf16.py:163-207) on the raw prefix K/V."""
    cfg = DecoderConfig(hidden=144, inter=192, n_q_heads=3, n_kv_heads=1)
    p = to32(expert_cross_layer_params(_Gen(13, norm_init="random"), cfg, 64))
    g = torch.Generator().manual_seed(14)
    x = torch.randn(2, 9, 144, generator=g)
    tk, tv = torch.randn(2, 17, 64, generator=g), torch.randn(2, 17, 64, generator=g)
    want = ref.expert_cross_block(x, tk, tv, p, cfg)
    got = ref._cross_with_projected(x, tk @ p["Wk_cross"], tv @ p["Wv_cross"], p, cfg)
    assert torch.allclose(got, want, atol=1e-5)
    # and in bf16, as the chunk runs it
    pb = tree_map(lambda t: t.to(BF16), p)
    xb, tkb, tvb = x.to(BF16), tk.to(BF16), tv.to(BF16)
    want_b = ref.expert_cross_block(xb, tkb, tvb, pb, cfg)
    got_b = ref._cross_with_projected(xb, ref.linear(tkb, pb["Wk_cross"]),
                                      ref.linear(tvb, pb["Wv_cross"]), pb, cfg)
    assert torch.equal(got_b, want_b)


def test_expert_output_closed_form():
    """Final RMSNorm then the action projection (vla/vla.py:218-222, 506-516)."""
    cfg, P = _small_fp32(5)
    io = P["expert_io"]
    h = torch.randn(2, cfg.chunk, cfg.expert.hidden, generator=torch.Generator().manual_seed(6))
    hd = _d(h)
    want = hd / torch.sqrt(hd.pow(2).mean(-1, keepdim=True) + cfg.expert.rms_eps)
    want = (want * _d(io["W_exp_norm"])) @ _d(io["W_action_out"])
    got = ref.expert_output(h, P, cfg)
    assert got.shape == (2, cfg.chunk, cfg.action_dim)
    assert torch.allclose(_d(got), want, atol=1e-4)


def _zero_layers(P):
    for lp in P["expert"]:
        for k in ("Wq", "Wk", "Wv", "Wo", "W_gate", "W_up", "W_down"):
            if k in lp:
                lp[k] = torch.zeros_like(lp[k])


def test_expert_velocity_zero_layers_closed_form(fp32_probs):
    """With every layer's projections zero, each block is the identity (its
    residuals carry x through), so v = expert_output(expert_input(x, t))."""
    cfg, P = _small_fp32(7)
    _zero_layers(P)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, cfg.chunk, cfg.action_dim, generator=g)
    L, kvd = cfg.prefix_len, cfg.expert.kv_dim
    ckv = {i: (torch.randn(1, L, kvd, generator=g), torch.randn(1, L, kvd, generator=g))
           for i in range(cfg.expert_layers) if cfg.is_cross(i)}
    got = ref.expert_velocity(x, 0.4, ckv, P, cfg)
    want = ref.expert_output(ref.expert_input(x, 0.4, P, cfg), P, cfg)
    assert torch.allclose(got, want, atol=1e-5)


def test_expert_velocity_routes_cross_layer_kv(fp32_probs):
    """Only cross layer i is live, with Wq = 0 (uniform attention) and no MLP:
    h = h0 + mean_keys(V_i) . Wo_i, V_i being layer i's projected cross V.  A
    velocity that reads another layer's K/V, treats layer i as a self layer or
    drops the residual fails."""
    cfg, P = _small_fp32(9)
    e = cfg.expert
    _zero_layers(P)
    g = torch.Generator().manual_seed(10)
    L = cfg.prefix_len
    ckv = {i: (torch.randn(1, L, e.kv_dim, generator=g),
               torch.randn(1, L, e.kv_dim, generator=g) + i)
           for i in range(cfg.expert_layers) if cfg.is_cross(i)}
    x = torch.randn(1, cfg.chunk, cfg.action_dim, generator=g)
    h0 = _d(ref.expert_input(x, 0.9, P, cfg))
    for live in ckv:
        Q = tree_map(lambda t: t.clone(), P)
        Q["expert"][live]["Wo"] = torch.randn(e.q_dim, e.hidden, generator=g) * 0.1
        got = ref.expert_velocity(x, 0.9, ckv, Q, cfg)
        vmean = _d(ckv[live][1]).mean(1)                       # [1, kv_dim]
        grp = e.n_q_heads // e.n_kv_heads
        ctx = torch.cat([vmean[:, (h // grp) * e.head_dim:(h // grp + 1) * e.head_dim]
                         for h in range(e.n_q_heads)], dim=1)  # [1, q_dim]
        h = h0 + (ctx @ _d(Q["expert"][live]["Wo"]))[:, None, :]
        want = ref.expert_output(h.float(), Q, cfg)
        assert torch.allclose(got, want, atol=1e-4), live


# --------------------------------------------------------------------------
# stack-level pins: the oracle's vision_encoder and prefix_forward against
# transformers' own stacks (local configs, loaded with the same weights)
def _llama_sd(p, prefix=""):
    sd = {
        "self_attn.q_proj.weight": p["Wq"].t(), "self_attn.k_proj.weight": p["Wk"].t(),
        "self_attn.v_proj.weight": p["Wv"].t(), "self_attn.o_proj.weight": p["Wo"].t(),
        "mlp.gate_proj.weight": p["W_gate"].t(), "mlp.up_proj.weight": p["W_up"].t(),
        "mlp.down_proj.weight": p["W_down"].t(),
        "input_layernorm.weight": p["W_norm_1"], "post_attention_layernorm.weight": p["W_norm_2"],
    }
    return {prefix + k: v.float().contiguous() for k, v in sd.items()}


def test_prefix_forward_matches_transformers_llama_stack(fp32_probs):
    """``prefix_forward`` (16 decoder layers with the prefix-LM mask, per-layer
    K/V cache) against a 2-layer transformers ``LlamaModel`` fed the same
    embeddings with the prefix-LM 4-D mask: every layer's output (forward
    hooks) and every layer's post-RoPE K and V (the model's own cache).  A
    causal mask, or the K/V of the neighbouring layer, fails the comparison."""
    from transformers import LlamaConfig, LlamaModel
    dc = DecoderConfig()
    L, bidir = 41, 40                      # 40 bidirectional tokens, 1 causal state token
    cfg = types.SimpleNamespace(decoder=dc, prefix_mask="prefix_lm", prefix_bidir_len=bidir)
    gen = _Gen(40, norm_init="random")
    layers = [to32(decoder_layer_params(gen, dc)) for _ in range(2)]
    x = torch.randn(1, L, dc.hidden, generator=torch.Generator().manual_seed(41))
    lc = LlamaConfig(hidden_size=dc.hidden, intermediate_size=dc.inter,
                     num_attention_heads=dc.n_q_heads, num_key_value_heads=dc.n_kv_heads,
                     head_dim=dc.head_dim, num_hidden_layers=2, rope_theta=dc.rope_theta,
                     rms_norm_eps=dc.rms_eps, vocab_size=16, max_position_embeddings=512,
                     attention_bias=False, mlp_bias=False, hidden_act="silu")
    lc._attn_implementation = "eager"
    model = LlamaModel(lc).eval()
    sd = {}
    for i, p in enumerate(layers):
        sd.update(_llama_sd(p, f"layers.{i}."))
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all(not k.startswith("layers.") for k in missing)
    outs = []
    hooks = [m.register_forward_hook(lambda mod, a, o: outs.append(o[0] if isinstance(o, tuple) else o))
             for m in model.layers]

    def run_llama(mask_bool):
        outs.clear()
        add = torch.zeros(1, 1, L, L).masked_fill(mask_bool, float("-inf"))
        with torch.no_grad():
            r = model(inputs_embeds=x, attention_mask=add, use_cache=True)
        cache = r.past_key_values
        kv = [(cache.layers[i].keys, cache.layers[i].values) for i in range(2)]
        return list(outs), kv

    with torch.no_grad():
        got_x, got_kv = ref.prefix_forward(x, {"prefix": layers}, cfg)
    hl, kvl = run_llama(ref.make_mask("prefix_lm", L, L, bidir))
    for h in hooks:
        h.remove()
    assert torch.allclose(got_x, hl[1], atol=5e-4, rtol=1e-3), (got_x - hl[1]).abs().max()
    to_bhld = lambda t: t.view(1, L, dc.n_kv_heads, dc.head_dim).transpose(1, 2)  # noqa: E731
    for i in range(2):
        k, v = got_kv[i]
        assert torch.allclose(to_bhld(k), kvl[i][0], atol=2e-4, rtol=1e-3), i
        assert torch.allclose(to_bhld(v), kvl[i][1], atol=2e-4, rtol=1e-3), i
    # sensitivity: the neighbouring layer's K, and a causal mask, do not match
    assert not torch.allclose(to_bhld(got_kv[0][0]), kvl[1][0], atol=1e-2)
    hooks = [m.register_forward_hook(lambda mod, a, o: outs.append(o[0] if isinstance(o, tuple) else o))
             for m in model.layers]
    hc, _ = run_llama(ref.make_mask("causal", L, L))
    for h in hooks:
        h.remove()
    assert not torch.allclose(got_x, hc[1], atol=1e-2)


def test_vision_encoder_matches_siglip_embeddings_and_encoder():
    """``vision_encoder`` (patch embedding + position table, then the ViT
    blocks, no post-LayerNorm) against transformers' ``SiglipVisionEmbeddings``
    followed by a 2-layer ``SiglipEncoder`` on the same weights, for two
    cameras of two samples (the [B, C, N, E] layout)."""
    from transformers.models.siglip.modeling_siglip import SiglipEncoder, SiglipVisionEmbeddings
    vc = VitConfig(image=64, layers=2)
    gen = _Gen(42, norm_init="random")
    vit = [to32(vit_layer_params(gen, vc)) for _ in range(2)]
    kernel, bias = gen.randn(768, 3, 16, 16).float() * 0.05, gen.randn(768).float() * 0.02
    pos = gen.randn(16, 768).float() * 0.02
    params = {"patch": {"kernel": kernel, "bias": bias, "pos_emb": pos}, "vit": vit}
    sc = _siglip(vc)
    sc.num_hidden_layers = 2
    emb = SiglipVisionEmbeddings(sc).eval()
    emb.load_state_dict({"patch_embedding.weight": kernel, "patch_embedding.bias": bias,
                         "position_embedding.weight": pos}, strict=False)
    enc = SiglipEncoder(sc).eval()
    sd = {}
    for i, p in enumerate(vit):
        pre = f"layers.{i}."
        sd.update({
            pre + "self_attn.q_proj.weight": p["Wq"].t(), pre + "self_attn.q_proj.bias": p["bq"],
            pre + "self_attn.k_proj.weight": p["Wk"].t(), pre + "self_attn.k_proj.bias": p["bk"],
            pre + "self_attn.v_proj.weight": p["Wv"].t(), pre + "self_attn.v_proj.bias": p["bv"],
            pre + "self_attn.out_proj.weight": p["Wo"].t(), pre + "self_attn.out_proj.bias": p["bo"],
            pre + "mlp.fc1.weight": p["W_up"].t(), pre + "mlp.fc1.bias": p["b_up"],
            pre + "mlp.fc2.weight": p["W_down"].t(), pre + "mlp.fc2.bias": p["b_down"],
            pre + "layer_norm1.weight": p["W_norm_1"], pre + "layer_norm1.bias": p["b_norm_1"],
            pre + "layer_norm2.weight": p["W_norm_2"], pre + "layer_norm2.bias": p["b_norm_2"],
        })
    enc.load_state_dict({k: v.contiguous() for k, v in sd.items()})
    images = torch.rand(2, 2, 3, 64, 64, generator=torch.Generator().manual_seed(43)) * 2 - 1
    cfg = types.SimpleNamespace(vit=vc)
    with torch.no_grad():
        got = ref.vision_encoder(images, params, cfg)
        want = enc(inputs_embeds=emb(images.reshape(4, 3, 64, 64))).last_hidden_state
    assert got.shape == (2, 2, 16, 768)
    assert torch.allclose(got.reshape(4, 16, 768), want, atol=5e-4, rtol=1e-3), \
        (got.reshape(4, 16, 768) - want).abs().max()
    # camera order: swapping two cameras of one sample moves exactly their tokens
    sw = images[:, [1, 0]]
    with torch.no_grad():
        got_sw = ref.vision_encoder(sw, params, cfg)
    assert torch.allclose(got_sw[:, 0], got[:, 1]) and torch.allclose(got_sw[:, 1], got[:, 0])
