"""The reference's own calling convention, end to end on the GPU: ``params``
built from a module's ``named_parameters()`` as numpy ``[in, out]`` arrays
(vla/text_encoder_bf16.py:599-609; bfloat16 words as ``ml_dtypes`` holds them,
here as uint16 bit patterns since ml_dtypes is not installed, or fp32), numpy
``x`` in, numpy out (the reference test calls ``allo_out.astype(np.float32)``,
:630).  Results against the oracle on the same weights at the per-layer
bound, the caller's dict unchanged, and an in-place weight update honoured.
"""

import numpy as np
import pytest
import torch

import oracle.smolvla_ref as ref
from smolvla.layers import host_tensor

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def rel(got, want):
    got, want = torch.as_tensor(np.asarray(got, dtype=np.float32)), want.float()
    return ((got - want).abs().max() / want.abs().max()).item()


def module_params(seed, hidden, inter, q_dim, kv_dim, cross=False):
    """nn.Linear / nn.RMSNorm default-initialised (seeded), named as the
    reference's blocks name them; returns ``{name: numpy weight}``."""
    torch.manual_seed(seed)
    lin = lambda i, o: torch.nn.Linear(i, o, bias=False)  # noqa: E731
    mods = {"attn.q_proj": lin(hidden, q_dim), "attn.output_proj": lin(q_dim, hidden),
            "gate_proj": lin(hidden, inter), "up_proj": lin(hidden, inter),
            "down_proj": lin(inter, hidden)}
    if cross:
        mods.update({"k_proj": lin(kv_dim, kv_dim), "v_proj": lin(kv_dim, kv_dim)})
    else:
        mods.update({"attn.k_proj": lin(hidden, kv_dim), "attn.v_proj": lin(hidden, kv_dim)})
    p = {f"{n}.weight": m.weight.detach().numpy() for n, m in mods.items()}
    g = torch.Generator().manual_seed(seed + 1)
    for n in ("ln_1.weight", "ln_2.weight"):        # trained-looking gains, not all ones
        p[n] = (1.0 + 0.1 * torch.randn(hidden, generator=g)).numpy()
    return p


def as_np(a, kind):
    """``.astype(NP_DTYPE)``: bf16 words (uint16 bit patterns) or fp32."""
    if kind == "fp32":
        return a.astype(np.float32)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(BF16) \
        .view(torch.int16).numpy().view(np.uint16)


def ref_params(p, kind, cross=False):
    """The reference's params dict (vla/text_encoder_bf16.py:600-610 key map)."""
    out = {"Wq": as_np(p["attn.q_proj.weight"].T, kind),
           "Wo": as_np(p["attn.output_proj.weight"].T, kind),
           "W_gate": as_np(p["gate_proj.weight"].T, kind),
           "W_up": as_np(p["up_proj.weight"].T, kind),
           "W_down": as_np(p["down_proj.weight"].T, kind),
           "W_norm_1": as_np(p["ln_1.weight"], kind), "W_norm_2": as_np(p["ln_2.weight"], kind)}
    if cross:
        out["Wk_cross"] = as_np(p["k_proj.weight"].T, kind)
        out["Wv_cross"] = as_np(p["v_proj.weight"].T, kind)
    else:
        out["Wk"] = as_np(p["attn.k_proj.weight"].T, kind)
        out["Wv"] = as_np(p["attn.v_proj.weight"].T, kind)
    return out


def oracle_view(params):
    return {k: host_tensor(v).to(BF16) for k, v in params.items()}


@pytest.mark.parametrize("kind", ["bf16_words", "fp32"])
def test_text_encoder_forward_numpy_params(kind):
    from smolvla.vla.text_encoder_bf16 import DEFAULT_CFG, EMBD, FFN_HID, SEQ, text_encoder_forward
    cfg = DEFAULT_CFG
    params = ref_params(module_params(200, EMBD, FFN_HID, cfg.q_dim, cfg.kv_dim), kind)
    keys = set(params)
    x_input = torch.randn(1, SEQ, EMBD, generator=torch.Generator().manual_seed(201))[0].numpy()
    print(f"text_encoder_forward, numpy params ({kind})", flush=True)
    out, key, value = text_encoder_forward(x_input, params)
    assert isinstance(out, np.ndarray) and out.shape == (SEQ, EMBD)
    out32 = out.astype(np.float32)                 # the reference test's own use of the result
    w_out, w_k, w_v = ref.decoder_block(torch.from_numpy(x_input).to(BF16)[None],
                                        oracle_view(params), cfg)
    for got, want in ((out32, w_out[0]), (key, w_k[0]), (value, w_v[0])):
        e = rel(got, want)
        print(f"  max rel err {e:.3e}")
        assert e <= 1e-2
    np.testing.assert_allclose(out32, w_out[0].float().numpy(), atol=1e-1, rtol=1e-1)
    assert set(params) == keys                     # the caller's dict is not touched
    # an in-place weight update is honoured (no stale packed copy)
    params["Wo"][...] = 0
    out2, _, _ = text_encoder_forward(x_input, params)
    w2, _, _ = ref.decoder_block(torch.from_numpy(x_input).to(BF16)[None], oracle_view(params), cfg)
    assert rel(out2, w2[0]) <= 1e-2


@pytest.mark.parametrize("kind", ["bf16_words", "fp32"])
def test_action_expert_forward_numpy_params(kind):
    from smolvla.vla.action_expert_bf16 import (DEFAULT_CFG, EMBD, FFN_HID, KV_DIM, SEQ,
                                                TEXT_SEQ, action_expert_cross_forward,
                                                action_expert_self_forward)
    cfg = DEFAULT_CFG
    g = torch.Generator().manual_seed(210)
    x = torch.randn(SEQ, EMBD, generator=g).numpy()
    tk = torch.randn(TEXT_SEQ, KV_DIM, generator=g).numpy()
    tv = torch.randn(TEXT_SEQ, KV_DIM, generator=g).numpy()
    ps = ref_params(module_params(211, EMBD, FFN_HID, cfg.q_dim, cfg.kv_dim), kind)
    pc = ref_params(module_params(212, EMBD, FFN_HID, cfg.q_dim, cfg.kv_dim, cross=True), kind,
                    cross=True)
    print(f"action expert self / cross, numpy params ({kind})", flush=True)
    got_s = action_expert_self_forward(x, ps)
    got_c = action_expert_cross_forward(x, tk, tv, pc)
    xb = torch.from_numpy(x).to(BF16)[None]
    want_s = ref.expert_self_block(xb, oracle_view(ps), cfg)[0]
    want_c = ref.expert_cross_block(xb, torch.from_numpy(tk).to(BF16)[None],
                                    torch.from_numpy(tv).to(BF16)[None], oracle_view(pc), cfg)[0]
    for got, want in ((got_s, want_s), (got_c, want_c)):
        assert isinstance(got, np.ndarray)
        e = rel(got, want)
        print(f"  max rel err {e:.3e}")
        assert e <= 1e-2
