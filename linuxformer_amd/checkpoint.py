"""A merged checkpoint directory (lx/lx/merge.py:203-248's save() layout: safetensors shards with
an optional index, config.json, lx_info.json) loaded from local files, no hub fetch, into the
stock transformers model and then this package's coordinate-form model.

    hf, info = checkpoint.load_dir(path)           # Qwen3_5ForCausalLM, lx_info.json's dict
    model = checkpoint.load_chip(path, n_chip)     # synth.SparseModel of the first n_chip layers

Tensors are loaded as stored (safetensors, which runs nothing from the file), so a bf16
checkpoint stays bf16 and an fp32 one fp32 (merge.load's reason for not using from_pretrained
with a dtype). The reference's circuit-specific layout and allocation (hf.pick_layout, allocate)
are not part of this path; the chip layers' tensors are.
"""

from __future__ import annotations

import json
from pathlib import Path


def load_dir(path, device: str = "cpu"):
    """(model, info) from a checkpoint directory (merge.py:217-248's loading steps)."""
    import torch
    from safetensors.torch import load_file
    from transformers import Qwen3_5ForCausalLM, Qwen3_5TextConfig
    from transformers.models.qwen3_5 import modeling_qwen3_5 as q

    path = Path(path)
    config = Qwen3_5TextConfig.from_pretrained(path)
    with torch.device("meta"):
        model = Qwen3_5ForCausalLM(config)
    idx = path / "model.safetensors.index.json"
    shards = sorted(set(json.loads(idx.read_text())["weight_map"].values())) if idx.exists() \
        else ["model.safetensors"]
    sd = {}
    for f in shards:
        sd.update(load_file(path / f, device=device))
    missing, unexpected = model.load_state_dict(sd, strict=False, assign=True)
    if unexpected or not set(missing) <= {"lm_head.weight"}:
        raise ValueError(f"{path}: tensors missing {sorted(missing)[:5]}, unexpected "
                         f"{sorted(unexpected)[:5]}")
    del sd
    model.tie_weights()
    model.model.rotary_emb = q.Qwen3_5TextRotaryEmbedding(config=config).to(device)
    info_p = path / "lx_info.json"
    info = json.loads(info_p.read_text()) if info_p.exists() else {}
    return model.eval(), info


def load_chip(path, n_chip: int | None = None):
    """The checkpoint's first n_chip layers (default: lx_info.json's chip_layers, else every
    layer), the tied head and the final norm as a synth.SparseModel (coordinate form: the
    packers and the oracle take it)."""
    from . import synth

    model, info = load_dir(path)
    n = n_chip if n_chip is not None else info.get("chip_layers")
    return synth.from_hf(model, n)
