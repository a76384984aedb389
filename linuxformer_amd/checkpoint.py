"""Checkpoint directories from local files (no hub fetch): the layout the reference's merge step
saves (lx/lx/merge.py:203-248) and transformers' save_pretrained writes.

    hf, info = checkpoint.load_dir(path)           # Qwen3_5ForCausalLM, lx_info.json's dict
    model = checkpoint.load_chip(path, n_chip)     # synth.SparseModel of the first n_chip layers

The directory:

    config.json                     a Qwen3_5 text config (hidden size, heads, layers, eps, ...)
    model.safetensors               the tensors, or several shards listed by
    model.safetensors.index.json    {"weight_map": {tensor name: shard file}}
    lx_info.json                    optional: {"chip_layers": n, ...}

Tensor names are transformers' Qwen3_5ForCausalLM state-dict names
(``model.layers.{L}.linear_attn.in_proj_qkv.weight``, ``model.embed_tokens.weight``, ...); a tied
checkpoint stores the head only as the embedding. Tensors keep the dtype they were stored in
(safetensors runs nothing from the file).

``load_dir`` gives the stock model through transformers' own local loader, after checking that
the files hold every tensor the model has. ``load_chip`` reads only the chip layers' tensors, the
embedding and the final norm, shard by shard, straight into coordinate form: the dense model is
never built (the real chip checkpoint is 32 GB dense).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

INDEX = "model.safetensors.index.json"
SINGLE = "model.safetensors"


class Shards:
    """The directory's tensors by name, each read from the shard that holds it."""

    def __init__(self, path):
        self.path = Path(path)
        idx = self.path / INDEX
        if idx.exists():
            self.where = dict(json.loads(idx.read_text())["weight_map"])
        elif (self.path / SINGLE).exists():
            from safetensors import safe_open

            with safe_open(str(self.path / SINGLE), "pt") as f:
                self.where = {k: SINGLE for k in f.keys()}
        else:
            raise ValueError(f"{self.path}: no {SINGLE} and no {INDEX}")
        self._open: dict = {}

    def names(self) -> set:
        return set(self.where)

    def get(self, name: str):
        if name not in self.where:
            raise ValueError(f"{self.path}: tensor {name!r} missing")
        shard = self.where[name]
        if shard not in self._open:
            from safetensors import safe_open

            self._open[shard] = safe_open(str(self.path / shard), "pt")
        return self._open[shard].get_tensor(name)


def _info(path: Path) -> dict:
    p = path / "lx_info.json"
    return json.loads(p.read_text()) if p.exists() else {}


def load_dir(path, device: str = "cpu"):
    """(model, info): the stock transformers model of a checkpoint directory, in the dtype its
    tensors were stored in, and lx_info.json's dict ({} without one). Raises ValueError when the
    files lack a tensor the model has (the head excepted when it is tied)."""
    import torch
    from transformers import Qwen3_5ForCausalLM, Qwen3_5TextConfig

    path = Path(path)
    config = Qwen3_5TextConfig.from_pretrained(path, local_files_only=True)
    with torch.device("meta"):
        expected = set(Qwen3_5ForCausalLM(config).state_dict())
    if config.tie_word_embeddings:
        expected.discard("lm_head.weight")
    stored = Shards(path).names()
    missing = sorted(expected - stored)
    if missing:
        raise ValueError(f"{path}: tensors missing: {missing[:5]}")
    model = Qwen3_5ForCausalLM.from_pretrained(path, config=config, dtype="auto",
                                               local_files_only=True, device_map=device)
    return model.eval(), _info(path)


def load_chip(path, n_chip: int | None = None):
    """The checkpoint's first n_chip layers (default: lx_info.json's chip_layers, else every
    layer), the tied head and the final norm as a synth.SparseModel, read tensor by tensor."""
    import torch

    from . import synth

    path = Path(path)
    cfg = json.loads((path / "config.json").read_text())
    cfg = cfg.get("text_config", cfg)
    sh = Shards(path)
    n = n_chip if n_chip is not None else _info(path).get("chip_layers", cfg["num_hidden_layers"])

    def arr(name):
        return sh.get(name).to(torch.float32).numpy()

    def coo(name):
        w = arr(name)
        r, c = np.nonzero(w)
        return synth.Coo(tuple(w.shape), r.astype(np.int64), c.astype(np.int64), w[r, c])

    emb = "model.embed_tokens.weight" if cfg.get("tie_word_embeddings", True) else "lm_head.weight"
    first = sh.get("model.embed_tokens.weight")
    eps = float(cfg["rms_norm_eps"])
    d = synth.Dims(hidden=cfg["hidden_size"], n_layers=n, nk=cfg["linear_num_key_heads"],
                   kd=cfg["linear_key_head_dim"], nv=cfg["linear_num_value_heads"],
                   vd=cfg["linear_value_head_dim"], conv=cfg["linear_conv_kernel_dim"],
                   inter=cfg["intermediate_size"], vocab=cfg["vocab_size"],
                   dtype="bf16" if first.dtype == torch.bfloat16 else "fp32", rms_eps=eps)
    layers = []
    for L in range(n):
        p = f"model.layers.{L}."
        ga = p + "linear_attn."
        layers.append(synth.Layer(
            in_proj_qkv=coo(ga + "in_proj_qkv.weight"), in_proj_z=coo(ga + "in_proj_z.weight"),
            in_proj_b=coo(ga + "in_proj_b.weight"), in_proj_a=coo(ga + "in_proj_a.weight"),
            out_proj=coo(ga + "out_proj.weight"), conv1d=arr(ga + "conv1d.weight")[:, 0],
            A_log=arr(ga + "A_log"), dt_bias=arr(ga + "dt_bias"), norm=arr(ga + "norm.weight"),
            input_layernorm=arr(p + "input_layernorm.weight"),
            post_attention_layernorm=arr(p + "post_attention_layernorm.weight"),
            gate_proj=coo(p + "mlp.gate_proj.weight"), up_proj=coo(p + "mlp.up_proj.weight"),
            down_proj=coo(p + "mlp.down_proj.weight")))
    return synth.SparseModel(d, layers, coo(emb), arr("model.norm.weight"))
