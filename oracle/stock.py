"""TEST INFRASTRUCTURE ONLY: the stock forward (the reference semantics), run with transformers'
own modules on the CPU. It writes the golden vectors (tests/golden/make_golden.py) and is the CPU
baseline bench.py times; the product never imports it.

lx/lx/hf.py:169-184 defines it: the chip layers as stock Qwen3_5DecoderLayers with no positions
or masks ("chip view"), carrying a DynamicCache; the head is the final norm and the tied
embedding, argmax with first-index ties. transformers' torch fallbacks run (neither fla nor the
hub kernels are installed), i.e. causal_conv1d_update and torch_recurrent_gated_delta_rule
(transformers/models/qwen3_5/modeling_qwen3_5.py:199-216, :330-380) for one-token steps.
"""

from __future__ import annotations

import numpy as np
import torch


def make_cache(m, conv0: np.ndarray, rec0: np.ndarray):
    """A DynamicCache whose layers hold conv windows conv0 (L, C, K) and recurrent states rec0
    (L, NV, KD, VD), marked as having previous state (as lx.fast.Fast.init_cache leaves it)."""
    from transformers import DynamicCache

    cache = DynamicCache(config=m.config)
    dt = m.dtype
    n, C, K = conv0.shape
    for L in range(n):
        cache.update_conv_state(torch.zeros(1, C, 1, dtype=dt), L, conv_kernel_size=K)
        cache.layers[L].conv_states[0].copy_(torch.from_numpy(conv0[L])[None].to(dt))
        cache.update_recurrent_state(torch.zeros(1, *rec0.shape[1:], dtype=torch.float32), L)
        cache.layers[L].recurrent_states[0].copy_(torch.from_numpy(rec0[L])[None])
    return cache


@torch.no_grad()
def chip_forward(m, h: torch.Tensor, cache) -> list:
    """hf.chip_forward (lx/lx/hf.py:169-176) on h (1, T, hidden); returns every layer's output."""
    outs = []
    for layer in m.model.layers[:m.config.num_hidden_layers]:
        h = layer(h, position_embeddings=None, attention_mask=None, position_ids=None,
                  past_key_values=cache)
        h = h[0] if isinstance(h, tuple) else h
        outs.append(h)
    return outs


@torch.no_grad()
def head_argmax(m, h: torch.Tensor) -> torch.Tensor:
    """hf.head_argmax (lx/lx/hf.py:179-184) on rows h (T, hidden)."""
    return torch.nn.functional.linear(m.model.norm(h), m.lm_head.weight).argmax(-1)


@torch.no_grad()
def decode(m, conv0, rec0, forced, n: int):
    """n greedy steps of the stock decode (one token at a time). Returns (preds, per-step
    per-layer residuals (n, L, hidden) float32, final conv (L, C, K) float32, final rec)."""
    cache = make_cache(m, conv0, rec0)
    emb = m.model.embed_tokens.weight
    tok = int(forced[0])
    preds, trace = [], []
    for i in range(n):
        h = emb[tok][None, None]
        outs = chip_forward(m, h, cache)
        trace.append(torch.stack([o[0, 0].float() for o in outs]).numpy())
        p = int(head_argmax(m, outs[-1][0])[0])
        preds.append(p)
        tok = int(forced[i + 1]) if i + 1 < len(forced) else p
    L = m.config.num_hidden_layers
    conv = np.stack([cache.layers[k].conv_states[0][0].float().numpy() for k in range(L)])
    rec = np.stack([cache.layers[k].recurrent_states[0][0].float().numpy() for k in range(L)])
    return np.array(preds, np.int32), np.stack(trace), conv, rec


@torch.no_grad()
def prefill(m, conv0, rec0, tokens):
    """The stock forward over T tokens at once (transformers' T > 1 path: causal_conv1d_fn over
    the cached window and the new inputs, torch_chunk_gated_delta_rule in chunks of 64 from the
    cached state; modeling_qwen3_5.py:249-327, :454-525), then every position's argmax, as
    lx.fast's verified mode compares (lx/lx/fast.py:252-361). Returns (preds (T,), final conv,
    final rec)."""
    cache = make_cache(m, conv0, rec0)
    emb = m.model.embed_tokens.weight
    h = emb[torch.as_tensor(np.asarray(tokens, np.int64))][None]
    outs = chip_forward(m, h, cache)
    preds = head_argmax(m, outs[-1][0]).numpy().astype(np.int32)
    L = m.config.num_hidden_layers
    conv = np.stack([cache.layers[k].conv_states[0][0].float().numpy() for k in range(L)])
    rec = np.stack([cache.layers[k].recurrent_states[0][0].float().numpy() for k in range(L)])
    return preds, conv, rec


def set_embedding(m, coo) -> None:
    """Replace the tied embedding/head rows with a coordinate tensor's values (configs 2 and 3
    share their layers and differ only in the embedding's gate columns)."""
    w = m.model.embed_tokens.weight
    with torch.no_grad():
        w.zero_()
        if coo.nnz:
            w[torch.from_numpy(coo.rows), torch.from_numpy(coo.cols)] = \
                torch.from_numpy(coo.vals).to(w.dtype)
