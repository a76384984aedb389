"""lx.fast's remaining host API (lx/lx/fast.py:33-46 place_lean, :399-430 Fast.to and
Fast.init_cache) on the CPU: the lean placement leaves the chip projections where they were and
moves everything else; init_cache leaves the states a zero token's stock forward leaves (all
zero, conv windows in the model dtype, recurrent states float32), both in a transformers
DynamicCache (the layout the stock layers read) and in this package's StateCache."""

import numpy as np
import pytest
import torch

from linuxformer_amd import fast, synth


def test_place_lean_keeps_the_chip_projections():
    m = synth.tiny_dense(7, "fp32")
    hf = synth.to_hf(m)
    n_chip = m.dims.n_layers
    fast.place_lean(hf, n_chip, "meta")
    kept = moved = 0
    for L, layer in enumerate(hf.model.layers):
        for name, p in layer.named_parameters():
            proj = any(f"{k}.weight" in name for k in fast.PROJ)
            if L < n_chip and proj:
                assert p.device.type == "cpu", name
                kept += 1
            else:
                assert p.device.type == "meta", name
                moved += 1
    assert kept == 8 * n_chip and moved > 0
    assert hf.model.embed_tokens.weight.device.type == "meta"


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_init_cache_dynamic_cache(dtype):
    from transformers import DynamicCache

    m = synth.tiny_dense(7, dtype)
    hf = synth.to_hf(m)
    f = fast.Fast(m)
    cache = DynamicCache(config=hf.config)
    f.init_cache(cache, "cpu")
    d = m.dims
    want = torch.bfloat16 if dtype == "bf16" else torch.float32
    for L in range(d.n_layers):
        conv = cache.layers[L].conv_states[0] if isinstance(cache.layers[L].conv_states, dict) \
            else cache.layers[L].conv_states
        rec = cache.layers[L].recurrent_states[0] if isinstance(cache.layers[L].recurrent_states, dict) \
            else cache.layers[L].recurrent_states
        assert tuple(conv.shape) == (1, d.n_conv, d.conv) and conv.dtype == want
        assert tuple(rec.shape) == (1, d.nv, d.kd, d.vd) and rec.dtype == torch.float32
        assert not conv.any() and not rec.any()


def test_init_cache_state_cache():
    m = synth.tiny_dense(7, "bf16")
    d = m.dims
    rng = np.random.default_rng(0)
    cache = fast.StateCache(rng.standard_normal((d.n_layers, d.n_conv, d.conv)).astype(np.float32),
                            rng.standard_normal((d.n_layers, d.nv, d.kd, d.vd)).astype(np.float32),
                            "bf16", "cpu")
    fast.Fast(m).init_cache(cache, "cpu")
    assert not cache.conv_numpy().any() and not cache.rec_numpy().any()
    assert cache.layers[0].conv_states[0].dtype == torch.bfloat16
