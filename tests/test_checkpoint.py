"""Checkpoint directories (linuxformer_amd.checkpoint, lx/lx/merge.py:203-248's layout): a model
saved with transformers' save_pretrained (one file, and sharded with an index) loads back
through the local loader into the same coordinate-form model, every value bit for bit, in the
dtype it was stored in."""

import json

import numpy as np
import pytest
import torch

from linuxformer_amd import checkpoint, synth


def _same(a, b):
    da, db = a.dims, b.dims
    eff = lambda d: d.gated_eps if d.gated_eps is not None else d.rms_eps  # noqa: E731
    assert eff(da) == eff(db)
    assert {k: v for k, v in vars(da).items() if k != "gated_eps"} == \
        {k: v for k, v in vars(db).items() if k != "gated_eps"}
    for la, lb in zip(a.layers, b.layers):
        for name in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj",
                     "gate_proj", "up_proj", "down_proj"):
            ca, cb = getattr(la, name), getattr(lb, name)
            assert ca.shape == cb.shape, name
            assert (np.asarray(ca.rows) == np.asarray(cb.rows)).all(), name
            assert (np.asarray(ca.cols) == np.asarray(cb.cols)).all(), name
            assert (np.asarray(ca.vals, np.float32).view(np.uint32) ==
                    np.asarray(cb.vals, np.float32).view(np.uint32)).all(), name
        for name in ("conv1d", "A_log", "dt_bias", "norm", "input_layernorm",
                     "post_attention_layernorm"):
            x, y = np.asarray(getattr(la, name), np.float32), np.asarray(getattr(lb, name), np.float32)
            assert (x.view(np.uint32) == y.view(np.uint32)).all(), name
    assert (np.asarray(a.embed.vals, np.float32) == np.asarray(b.embed.vals, np.float32)).all()
    assert (np.asarray(a.norm, np.float32) == np.asarray(b.norm, np.float32)).all()


@pytest.mark.parametrize("dtype,shard", [("bf16", None), ("fp32", "20KB")])
def test_saved_directory_loads_back(tmp_path, dtype, shard):
    m = synth.tiny_dense(4, dtype)
    hf = synth.to_hf(m)
    kw = {} if shard is None else {"max_shard_size": shard}
    hf.save_pretrained(tmp_path, **kw)
    (tmp_path / "lx_info.json").write_text(json.dumps({"chip_layers": m.dims.n_layers}))
    if shard is not None:
        assert (tmp_path / "model.safetensors.index.json").exists()
    model, info = checkpoint.load_dir(tmp_path)
    want = torch.bfloat16 if dtype == "bf16" else torch.float32
    assert model.dtype == want and info == {"chip_layers": m.dims.n_layers}
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    _same(checkpoint.load_chip(tmp_path), synth.from_hf(hf))
    if dtype == "fp32":  # (the tiny bf16 model's gated-norm weight 1 + w is not bf16-exact)
        _same(checkpoint.load_chip(tmp_path), m)


def test_missing_tensor_is_refused(tmp_path):
    from safetensors.torch import load_file, save_file

    m = synth.tiny_dense(5, "fp32")
    synth.to_hf(m).save_pretrained(tmp_path)
    sd = load_file(tmp_path / "model.safetensors")
    sd.pop("model.layers.0.mlp.up_proj.weight")
    save_file(sd, str(tmp_path / "model.safetensors"), metadata={"format": "pt"})
    with pytest.raises(ValueError, match="missing"):
        checkpoint.load_dir(tmp_path)
