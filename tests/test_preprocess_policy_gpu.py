"""GPU pre-processing kernel and the closed-loop chunk caller."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.smolvla_ref as ref
from smolvla import ops, preprocess
from smolvla.config import small_config
from smolvla.params import smolvla_params

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _image_ref(frames, S):
    """torch CPU: bilinear (align_corners=False) resize with the aspect ratio
    kept, top-left placement, black padding, x / 255 * 2 - 1, bf16."""
    n, h, w, _ = frames.shape
    scale = min(S / h, S / w)
    rh, rw = max(1, min(S, int(h * scale + 0.5))), max(1, min(S, int(w * scale + 0.5)))
    x = frames.permute(0, 3, 1, 2).float()
    r = F.interpolate(x, size=(rh, rw), mode="bilinear", align_corners=False, antialias=False)
    out = torch.zeros(n, 3, S, S)
    out[:, :, :rh, :rw] = r
    return (out / 255.0 * 2.0 - 1.0).to(BF16)


@pytest.mark.parametrize("h,w,S", [(480, 640, 512), (512, 512, 512), (300, 200, 512),
                                   (96, 700, 224), (1, 1, 16)])
def test_image_to_bf16_matches_torch_bilinear(h, w, S):
    g = torch.Generator().manual_seed(h * 7 + w)
    frames = torch.randint(0, 256, (3, h, w, 3), generator=g, dtype=torch.uint8)
    got = ops.image_to_bf16(frames.cuda(), S).cpu()
    want = _image_ref(frames, S)
    assert got.shape == want.shape
    torch.testing.assert_close(got.float(), want.float(), atol=8e-3, rtol=0)
    # padding is exactly -1 and values stay in [-1, 1]
    assert got.float().min() >= -1 and got.float().max() <= 1


def test_chunk_policy_refills_once_per_chunk_and_matches_the_oracle():
    from smolvla.policy import ChunkPolicy
    cfg = small_config()
    P = smolvla_params(cfg, seed=0)
    pol = ChunkPolicy(cfg, P, action_dims=2, seed=11)
    g = torch.Generator().manual_seed(2)
    frames = torch.randint(0, 256, (cfg.n_cameras, 48, 80, 3), generator=g, dtype=torch.uint8)
    ids = torch.randint(0, cfg.vocab, (cfg.lang_tokens,), generator=g)
    state = np.array([0.3, -0.2, 1.5], dtype=np.float32)
    acts = [pol.act(frames, state, ids) for _ in range(25)]
    assert pol.chunks == 3                       # ceil(25 / chunk 10)
    assert all(a.shape == (2,) for a in acts)
    # the first chunk against the oracle on the same pre-processed inputs / noise
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    noise = torch.randn(1, cfg.chunk, cfg.action_dim, generator=gen, device="cuda").cpu()
    images = preprocess.images(frames, cfg.vit.image).cpu()
    want = ref.smolvla_chunk(images, ids.view(1, -1), preprocess.pad_state(state, cfg.state_dim),
                             noise, P, cfg)[0]
    first = np.stack(acts[:10])
    err = np.abs(first - want[:, :2].numpy()).max()
    print(f"first chunk max abs err vs oracle {err:.3e}")
    assert err <= 5e-2
