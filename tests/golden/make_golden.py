"""Write the committed golden fixtures from the pinned CPU oracle.

Run in a container with the repository (CPU only):

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path (its tests compute every
expectation live from seeded torch), so these fixtures are generated from the
oracle in ``oracle/smolvla_ref.py`` after it has been pinned by
``tests/test_oracle_pin.py``.  They freeze its outputs so that a later change
to the oracle, to the seeded generators or to the HIP path is caught against
data rather than against another live computation.

Weights are not stored: they are regenerated from the seed by
``smolvla.params`` (listed per fixture in ``manifest.json``).  Inputs and
outputs are stored; bf16 tensors as their raw ``uint16`` bit patterns.

Fixtures
--------
* ``cfg0_decoder_block.npz``  BASELINE config 0: one SmolLM2 decoder block,
  x [128, 960] ~ N(0,1), causal, theta 1e5, eps 1e-5 -> out, K (post-RoPE), V
  (``TextEncoderBlock`` vla/text_encoder_bf16.py:61-135, K/V export of the
  NPU path :595).
* ``expert_cross_block.npz``  one action-expert cross layer, x [50, 720],
  prefix K/V [241, 320] (``ActionExpertCrossBlock``
  vla/action_expert_bf16.py:134-207).
* ``vit_block_small.npz``  one SigLIP block on 64 tokens of width 768
  (``MiniVit`` vla/vision_block_bf16.py:57-79, GELU-tanh, LN eps 1e-6).
* ``small_chunk.npz``  the whole chunk pipeline on ``small_config()`` at
  batch 2: inputs, final actions and the hidden state after the last prefix
  layer.
* ``harness.npz``  per-kernel harness cases: ``rms_norm_960_bf16``
  (cc/bf16/rms_norm_960_bf16.cc, eps 1e-6), ``masked_softmax_128_bf16`` with
  row_start (cc/bf16/masked_softmax_128_bf16.cc:251), ``softmax_bf16_seq1024``
  (cc/bf16_old/v1_softmax_bf16.cc:159) and ``rope_fused_float32``
  (cc/float/rope_fused.cc:17).
"""

from __future__ import annotations

import hashlib
import json
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for _p in (str(ROOT / "vla-to-npu_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import oracle.smolvla_ref as ref  # noqa: E402
from smolvla.config import DecoderConfig, SmolVLAConfig, VitConfig, small_config  # noqa: E402
from smolvla.params import (_Gen, decoder_layer_params, expert_cross_layer_params,  # noqa: E402
                            smolvla_inputs, smolvla_params, vit_layer_params)

BF16 = torch.bfloat16


def enc(t: torch.Tensor) -> np.ndarray:
    """bf16 -> uint16 bit pattern; fp32 / int64 unchanged."""
    t = t.detach().cpu().contiguous()
    if t.dtype == BF16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def dec(a: np.ndarray) -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(BF16)
    return torch.from_numpy(a.copy())


def x_in(seed, *shape, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(BF16)


# ---- the fixtures ---------------------------------------------------------
def cfg0_decoder_block():
    cfg = DecoderConfig()
    p = decoder_layer_params(_Gen(0), cfg)
    x = x_in(1, 128, cfg.hidden)
    out, k, v = ref.decoder_block(x[None], p, cfg, "causal", 0)
    meta = dict(weights="decoder_layer_params(_Gen(0), DecoderConfig())", x="N(0,1) seed 1",
                mask="causal", rope_theta=cfg.rope_theta, rms_eps=cfg.rms_eps)
    return dict(x=x, out=out[0], k=k[0], v=v[0]), meta


def expert_cross_block():
    cfg = DecoderConfig(hidden=720, inter=2048)
    p = expert_cross_layer_params(_Gen(10), cfg, 320)
    x = x_in(11, 50, 720)
    tk, tv = x_in(12, 241, 320), x_in(13, 241, 320)
    out = ref.expert_cross_block(x[None], tk[None], tv[None], p, cfg)
    meta = dict(weights="expert_cross_layer_params(_Gen(10), DecoderConfig(hidden=720, "
                        "inter=2048), 320)", x="N(0,1) seed 11", text_k="N(0,1) seed 12",
                text_v="N(0,1) seed 13")
    return dict(x=x, text_k=tk, text_v=tv, out=out[0]), meta


def vit_block_small():
    cfg = VitConfig()
    p = vit_layer_params(_Gen(20, norm_init="random"), cfg)
    x = x_in(21, 64, cfg.hidden)
    out = ref.vit_block(x[None], p, cfg)
    meta = dict(weights="vit_layer_params(_Gen(20, norm_init='random'), VitConfig())",
                x="N(0,1) seed 21", tokens=64)
    return dict(x=x, out=out[0]), meta


def small_chunk():
    cfg = small_config()
    params = smolvla_params(cfg, seed=0)
    images, ids, state, noise = smolvla_inputs(cfg, 2, seed=1)
    cap = {}
    actions = ref.smolvla_chunk(images, ids, state, noise, params, cfg, capture=cap)
    prefix_out, _ = ref.prefix_forward(cap["prefix"], params, cfg)
    meta = dict(config="small_config()", weights="smolvla_params(small_config(), seed=0)",
                inputs="smolvla_inputs(small_config(), 2, seed=1)",
                prefix_out="hidden state after the last prefix layer")
    return dict(images=images, ids=ids, state=state, noise=noise, actions=actions,
                prefix_out=prefix_out), meta


def harness():
    g = torch.Generator().manual_seed(30)
    rn_x = torch.randn(16, 960, generator=g).to(BF16)
    rn_w = (1 + 0.1 * torch.randn(960, generator=g)).to(BF16)
    rn_y = ref.rms_norm(rn_x, rn_w, 1e-6)
    ms_s = (torch.randn(8, 128, generator=g) * 3).to(BF16)
    ms_p = ref.masked_softmax_rows(ms_s, 37)
    sm_s = (torch.randn(4, 1024, generator=g) * 4).to(BF16)
    sm_p = ref.softmax_rows(sm_s)
    rp_x = torch.randn(64, 64, generator=g)
    cos, sin = ref.rope_tables(64, 64, 1e4)
    rp_y = ref.apply_rope(rp_x.view(1, 64, 1, 64), 1e4).view(64, 64)
    meta = dict(rms_norm_960="eps 1e-6", masked_softmax_128="row_start 37",
                softmax_bf16_seq1024="rows of 1024", rope_fused_float32="theta 1e4, pos 0..63")
    return dict(rn_x=rn_x, rn_w=rn_w, rn_y=rn_y, ms_s=ms_s, ms_p=ms_p, sm_s=sm_s, sm_p=sm_p,
                rp_x=rp_x, rp_cos=cos, rp_sin=sin, rp_y=rp_y), meta


FIXTURES = {
    "cfg0_decoder_block": cfg0_decoder_block,
    "expert_cross_block": expert_cross_block,
    "vit_block_small": vit_block_small,
    "small_chunk": small_chunk,
    "harness": harness,
}


def load(name):
    """Fixture ``name`` as a dict of torch tensors (bf16 restored)."""
    with np.load(HERE / f"{name}.npz", allow_pickle=False) as z:
        return {k: dec(z[k]) for k in z.files}


def main():
    torch.set_num_threads(min(8, torch.get_num_threads()))
    manifest = {"generator": "tests/golden/make_golden.py", "torch": torch.__version__,
                "fixtures": {}}
    with torch.inference_mode():
        for name, fn in FIXTURES.items():
            arrays, meta = fn()
            enc_arrays = {k: enc(v) for k, v in arrays.items()}
            path = HERE / f"{name}.npz"
            np.savez_compressed(path, **enc_arrays)
            digest = hashlib.sha256(path.read_bytes()).hexdigest()[:16]
            meta["arrays"] = {k: [list(a.shape), str(a.dtype)] for k, a in enc_arrays.items()}
            meta["sha256_16"] = digest
            manifest["fixtures"][name] = meta
            print(f"{name}: {path.stat().st_size / 1024:.0f} KiB", flush=True)
    (HERE / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")


if __name__ == "__main__":
    main()
