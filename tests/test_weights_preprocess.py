"""Parameter files (safetensors, own and HF-style layouts) and the host-side
observation pre-processing (state padding, prompt ids).  CPU only."""

import pytest
import torch

from smolvla import preprocess, weights
from smolvla.config import small_config
from smolvla.params import smolvla_params

BF16 = torch.bfloat16


def _equal_trees(a, b):
    fa, fb = weights.flatten(a), weights.flatten(b)
    assert set(fa) == set(fb)
    for k in fa:
        assert fa[k].dtype == fb[k].dtype and torch.equal(fa[k], fb[k]), k


def test_own_layout_round_trip(tmp_path):
    cfg = small_config()
    P = smolvla_params(cfg, seed=3, norm_init="random")
    weights.check_params(P, cfg)
    path = tmp_path / "p.safetensors"
    weights.save_params(P, path)
    _equal_trees(weights.load_params(path, cfg), P)


def test_load_rejects_wrong_config(tmp_path):
    cfg = small_config()
    P = smolvla_params(cfg, seed=3)
    path = tmp_path / "p.safetensors"
    weights.save_params(P, path)
    other = small_config()
    other = type(other)(**{**other.__dict__, "prefix_layers": 5})
    with pytest.raises(ValueError, match="missing prefix.4"):
        weights.load_params(path, other)
    with pytest.raises(FileNotFoundError):
        weights.load_params(tmp_path / "absent.safetensors")


def test_hf_layout_maps_and_transposes(tmp_path):
    cfg = small_config()
    P = smolvla_params(cfg, seed=4, norm_init="random")
    sd = weights.to_hf_state_dict(P, cfg)
    # nn.Linear layout [out, in] on the HF side, e.g. the prefix gate projection
    k = "model.vlm_with_expert.vlm.model.text_model.layers.1.mlp.gate_proj.weight"
    assert torch.equal(sd[k], P["prefix"][1]["W_gate"].t())
    # cross layers' K/V projections come from the cross weights
    kc = "model.vlm_with_expert.lm_expert.layers.1.self_attn.k_proj.weight"
    assert torch.equal(sd[kc], P["expert"][1]["Wk_cross"].t())
    # tensors the pipeline does not use are reported, not dropped silently
    sd["model.vlm_with_expert.vlm.model.vision_model.post_layernorm.weight"] = torch.ones(4)
    from safetensors.torch import save_file
    path = tmp_path / "model.safetensors"
    save_file({n: t.contiguous() for n, t in sd.items()}, str(path))
    got, ignored = weights.load_hf_safetensors(path, cfg)
    _equal_trees(got, P)
    assert ignored == ["model.vlm_with_expert.vlm.model.vision_model.post_layernorm.weight"]
    del sd[k]
    with pytest.raises(ValueError, match="missing prefix.1.W_gate"):
        weights.from_hf_state_dict(sd, cfg)


def test_pad_state():
    s = preprocess.pad_state([0.5, -1.0, 2.0], 32)
    assert s.shape == (1, 32) and s.dtype == torch.float32
    assert s[0, :3].tolist() == [0.5, -1.0, 2.0] and s[0, 3:].abs().sum() == 0
    assert preprocess.pad_state(torch.ones(2, 32)).shape == (2, 32)
    with pytest.raises(ValueError):
        preprocess.pad_state(torch.ones(33))


def test_token_ids_with_a_local_tokenizer():
    from tokenizers import Tokenizer
    from tokenizers.models import WordLevel
    from tokenizers.pre_tokenizers import Whitespace
    vocab = {"[UNK]": 1, "push": 5, "the": 6, "t": 7, "block": 8}
    tok = Tokenizer(WordLevel(vocab, unk_token="[UNK]"))
    tok.pre_tokenizer = Whitespace()
    ids = preprocess.token_ids(["push the t block", "push"], tok, length=6)
    assert ids.dtype == torch.int64 and ids.shape == (2, 6)
    assert ids[0].tolist() == [5, 6, 7, 8, 0, 0] and ids[1].tolist() == [5, 0, 0, 0, 0, 0]
    long_text = " ".join(["block"] * 60)
    assert preprocess.token_ids(long_text, tok).shape == (1, 48)
