"""CPU checks of which ViT projections the engine runs on the 256x256 GEMM
with slab-blocked operands (smolvla.layers.vit_blocked_plan), at the SigLIP
shapes (hidden 768, MLP 3072, 1024 tokens per camera image)."""

import pytest

from smolvla import layers

ALL = {"qkv", "o", "up", "down"}


@pytest.mark.parametrize("images, want", [
    (3, {"up"}),                 # batch 1: 12 row tiles; only the up-projection has 144 tiles
    (6, {"qkv", "up"}),          # batch 2: QKV 216 tiles, O and down 72
    (9, {"qkv", "up"}),          # batch 3: O and down 108
    (12, ALL),                   # batch 4: O and down reach 144
    (96, ALL),                   # batch 32
])
def test_plan_at_camera_batches(images, want):
    plan = layers.vit_blocked_plan(768, 3072, images * 1024)
    assert {k for k, v in plan.items() if v} == want


def test_rows_must_fill_whole_tiles():
    assert not any(layers.vit_blocked_plan(768, 3072, 96 * 1024 + 64).values())


def test_down_goes_blocked_only_with_up():
    # MLP width 384: the up-projection's 384 columns are not whole 256-wide
    # tiles, while the down-projection (768 x 384) alone would qualify.
    plan = layers.vit_blocked_plan(768, 384, 12288)
    assert not plan["up"] and not plan["down"]
    assert plan["qkv"] and plan["o"]
