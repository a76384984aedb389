"""Write the golden vectors: the stock forward's outputs on small seeded inputs.

The stock forward is transformers 5.15.0's Qwen3_5 decoder layers (torch fallbacks; neither
fla nor the hub kernels are installed) in lx/lx/hf.py's chip view, run token by token on the CPU
by oracle/stock.py; the reference pins 5.19.0 (requirements.txt:4), whose qwen3_5 code path for
these ops is the same. Nothing of the reference repository is imported.

    python tests/golden/make_golden.py [names]     # rewrites tests/golden/<name>.npz

Each fixture holds the inputs' seeds and shapes (rebuilt by linuxformer_amd.synth), the greedy
stream, every step's per-layer residual (float32) or a hash of it, and the final states' hashes
plus a sample of their values.
"""

from __future__ import annotations

import hashlib
import os
import sys
from dataclasses import replace

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from linuxformer_amd import synth  # noqa: E402
from oracle import oracle as ox  # noqa: E402
from oracle import stock  # noqa: E402

def c2_cut():
    """Config 2's layer shape (hidden 3572, 16 key x 128 value heads, SwiGLU 1024, bf16, N(0,1)
    state) cut to 3 layers and a 4,096-token vocabulary; every token gates one of the 3 layers."""
    s = synth.config2()
    return replace(s, name="c2s", dims=replace(s.dims, n_layers=3, vocab=4096), p_gate=1.0 / 3)


CASES = {
    # name: (spec builder, steps, keep full traces)
    "c1_256": (lambda: synth.config1(), 256, False),
    "c2s_bf16_64": (c2_cut, 64, False),
    "small_bf16_32": (lambda: synth.small(), 32, True),
    "small_fp32_32": (lambda: synth.small(dtype="fp32", seed=3), 32, True),
    "tiny_fp32_8": (lambda: "tiny_fp32", 8, True),
    "tiny_bf16_8": (lambda: "tiny_bf16", 8, True),
}


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


def sha_state(a: np.ndarray) -> str:
    """sha256 of recurrent-state values with the sign of zero made +0 (x + 0): states are equal
    when every element compares equal, as the reference compares them (x.ne(y),
    lx/tests/check_mega.py:34-36). The stock update S + k (x) delta on every head turns some -0
    entries of a fully decayed head into +0 on later steps, which skipping idle heads (the
    reference's own design, lx/lx/fast.py:8-19) does not."""
    return sha(np.ascontiguousarray(a, np.float32) + np.float32(0.0))


def model_of(name):
    spec = CASES[name][0]()
    if isinstance(spec, str):
        dt = spec.split("_")[1]
        m = synth.tiny_dense(seed=3, dtype=dt)
        d = m.dims
        conv0 = np.zeros((d.n_layers, d.n_conv, 4), np.float32)
        rec0 = np.random.default_rng(5).standard_normal((d.n_layers, d.nv, d.kd, d.vd)).astype(np.float32)
        return m, conv0, rec0, 5
    m = synth.build(spec)
    conv0, rec0 = synth.init_state(m)
    return m, conv0, rec0, synth.start_token(spec)


def chunk_inputs(T: int, seed: int, exact: bool = False):
    """One value head's delta-rule inputs over T positions: query and key l2-normed over 128 live
    dims of 256 (the padded key heads), values, log decays and betas, and an initial state.
    exact: the chip's exact regime (one-hot keys and queries, beta in {0, 1}, no decay, small
    dyadic values), where every product and sum is exact."""
    rng = np.random.default_rng(seed)
    K, V, KL = 256, 128, 128
    if exact:
        q = np.zeros((T, K), np.float32)
        k = np.zeros((T, K), np.float32)
        q[np.arange(T), rng.integers(0, KL, T)] = 1.0
        k[np.arange(T), rng.integers(0, KL, T)] = 1.0
        v = rng.integers(-8, 9, (T, V)).astype(np.float32) / 4
        g = np.zeros(T, np.float32)
        beta = rng.integers(0, 2, T).astype(np.float32)
        S0 = rng.integers(-8, 9, (K, V)).astype(np.float32) / 8
        S0[KL:] = 0.0
        return q, k, v, g, beta, S0

    def unit(x):
        return (x / np.sqrt((x.astype(np.float64) ** 2).sum(-1, keepdims=True))).astype(np.float32)

    q = np.zeros((T, K), np.float32)
    k = np.zeros((T, K), np.float32)
    q[:, :KL] = unit(rng.standard_normal((T, KL)))
    k[:, :KL] = unit(rng.standard_normal((T, KL)))
    v = rng.standard_normal((T, V)).astype(np.float32)
    g = (-0.5 * rng.random(T)).astype(np.float32)
    beta = rng.random(T).astype(np.float32)
    S0 = np.zeros((K, V), np.float32)
    S0[:KL] = rng.standard_normal((KL, V))
    return q, k, v, g, beta, S0


def write_chunk(name: str, T: int, seed: int) -> None:
    """transformers' torch_chunk_gated_delta_rule (chunk 64, float32, the initial state given,
    use_qk_l2norm_in_kernel off: the inputs are normed already) on chunk_inputs(T, seed)."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import torch_chunk_gated_delta_rule

    q, k, v, g, beta, S0 = chunk_inputs(T, seed)
    t = [torch.from_numpy(a)[None, :, None] for a in (q, k, v, g, beta)]
    o, S = torch_chunk_gated_delta_rule(*t, chunk_size=64, initial_state=torch.from_numpy(S0)[None, None],
                                        output_final_state=True, use_qk_l2norm_in_kernel=False)
    out = {"q": q[:, :128], "k": k[:, :128], "v": v, "g": g, "beta": beta, "S0": S0[:128],
           "o": o[0, :, 0].numpy(), "S": S[0, 0, :128].numpy(), "T": np.int64(T)}
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **out)
    print(name, os.path.getsize(path), "bytes")


CHUNK_CASES = {"chunk_fp32_100": (100, 11)}


def write_prefill(name: str, base: str, T: int) -> None:
    """The stock forward over T tokens at once (transformers' T > 1 path: causal_conv1d_fn and
    torch_chunk_gated_delta_rule from the cached state) on the stack of fixture `base`: every
    layer's output at every position, the argmax at every position, samples of the final states
    (with their indices and the states' largest magnitudes)."""
    m, conv0, rec0, _ = model_of(base)
    hf = synth.to_hf(m)
    toks = np.random.default_rng(3).integers(0, m.dims.vocab, T).astype(np.int64)
    cache = stock.make_cache(hf, conv0, rec0)
    h = hf.model.embed_tokens.weight[torch.from_numpy(toks)][None]
    outs = stock.chip_forward(hf, h, cache)
    trace = torch.stack([o[0].float() for o in outs], 1).numpy()
    preds = stock.head_argmax(hf, outs[-1][0]).numpy().astype(np.int32)
    L = m.dims.n_layers
    conv = np.stack([cache.layers[k].conv_states[0][0].float().numpy() for k in range(L)])
    rec = np.stack([cache.layers[k].recurrent_states[0][0].float().numpy() for k in range(L)])
    rng = np.random.default_rng(1)
    ridx = rng.integers(0, rec.size, 8192)
    out = {"tokens": toks, "preds": preds, "trace": trace, "base": base, "conv": conv,
           "rec_idx": ridx, "rec_sample": rec.reshape(-1)[ridx], "rec_max": np.float32(np.abs(rec).max()),
           "rec_sha": sha_state(rec), "trace_sha": sha(trace)}
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **out)
    print(name, os.path.getsize(path), "bytes", preds.tolist()[:8])


PREFILL_CASES = {"small_fp32_pf100": ("small_fp32_32", 100), "small_bf16_pf100": ("small_bf16_32", 100)}


def write_prefill_c3(name: str, T: int) -> None:
    """The stock forward's T > 1 path over the first T tokens of config 3's first verified-mode
    call (bench.py's warm-up call), on the 37-layer stack at its full shape: the argmax at every
    position; each layer's largest output magnitude and its outputs at 4,096 seeded (position,
    column) samples (bf16 bits: the layers' outputs are bf16); samples of the final states with
    their largest magnitudes. The full trace (37 x T x 3572) is too large to commit."""
    spec = synth.config3()
    m = synth.build(spec)
    conv0, rec0 = synth.init_state(m)
    hf = synth.to_hf(m)
    toks = synth.tokens(spec, 65_536, 0)[:T].astype(np.int64)
    cache = stock.make_cache(hf, conv0, rec0)
    h = hf.model.embed_tokens.weight[torch.from_numpy(toks)][None]
    outs = stock.chip_forward(hf, h, cache)
    trace = torch.stack([o[0].float() for o in outs], 1).numpy()  # (T, L, hidden)
    preds = stock.head_argmax(hf, outs[-1][0]).numpy().astype(np.int32)
    L, H = m.dims.n_layers, m.dims.hidden
    conv = np.stack([cache.layers[k].conv_states[0][0].float().numpy() for k in range(L)])
    rec = np.stack([cache.layers[k].recurrent_states[0][0].float().numpy() for k in range(L)])
    rng = np.random.default_rng(5)
    pos, col = rng.integers(0, T, 4096), rng.integers(0, H, 4096)
    samp = trace[pos, :, col]  # (4096, L)
    assert np.all((samp.view(np.uint32) & 0xffff) == 0)
    ridx, cidx = rng.integers(0, rec.size, 8192), rng.integers(0, conv.size, 8192)
    out = {"tokens": toks, "preds": preds, "pos": pos, "col": col,
           "trace_bf16": (samp.T.copy().view(np.uint32) >> 16).astype(np.uint16),
           "layer_max": np.abs(trace).max(axis=(0, 2)).astype(np.float32),
           "rec_idx": ridx, "rec_sample": rec.reshape(-1)[ridx],
           "rec_max": np.float32(np.abs(rec).max()), "conv_idx": cidx,
           "conv_sample": conv.reshape(-1)[cidx], "conv_max": np.float32(np.abs(conv).max()),
           "trace_sha": sha(trace), "transformers": __import__("transformers").__version__}
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **out)
    print(name, os.path.getsize(path), "bytes", preds.tolist()[:8])


PREFILL_C3_CASES = {"c3_pf64": 64}


def main():
    torch.set_grad_enabled(False)
    names = sys.argv[1:] or list(CASES) + list(CHUNK_CASES) + list(PREFILL_CASES) + \
        list(PREFILL_C3_CASES)
    for name in names:
        if name in CHUNK_CASES:
            write_chunk(name, *CHUNK_CASES[name])
            continue
        if name in PREFILL_CASES:
            write_prefill(name, *PREFILL_CASES[name])
            continue
        if name in PREFILL_C3_CASES:
            write_prefill_c3(name, PREFILL_C3_CASES[name])
            continue
        _, n, full = CASES[name]
        m, conv0, rec0, start = model_of(name)
        hf = synth.to_hf(m)
        preds, trace, conv, rec = stock.decode(hf, conv0, rec0, [start], n)
        rng = np.random.default_rng(0)
        ridx = rng.integers(0, rec.size, 4096)
        out = {"preds": preds, "start": np.int64(start), "n": np.int64(n),
               "conv_sha": sha(conv), "rec_sha": sha_state(rec), "rec_idx": ridx,
               "rec_sample": rec.reshape(-1)[ridx], "trace_sha": sha(trace),
               "conv_sample": conv.reshape(-1)[rng.integers(0, conv.size, 4096)],
               "conv_idx": rng.integers(0, conv.size, 4096)}
        out["conv_sample"] = conv.reshape(-1)[out["conv_idx"]]
        if full:
            out["trace"] = trace
        if m.dims.dtype == "bf16" and not full:
            # the contract (IEEE, no flushing) against the stock trace: the elements that differ
            # (oneDNN's bf16 GEMM flushes denormals on this host; the oracle's flush mode models it)
            ox.build()
            om = ox.OracleModel(m)
            ox.set_flush(False)
            c, r = conv0.copy(), rec0.copy()
            _, _, tr = om.decode(c, r, [start], n, trace=True)
            diff = tr.view(np.uint32) != np.ascontiguousarray(trace, np.float32).view(np.uint32)
            out["contract_diff"] = np.int64(diff.sum())
            out["contract_diff_max_abs"] = np.float32(
                max(np.abs(tr[diff]).max(initial=0), np.abs(trace[diff]).max(initial=0)))
            out["host_cpu_capability"] = torch.backends.cpu.get_cpu_capability()
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **out)
        print(name, os.path.getsize(path), "bytes", preds.tolist()[:8])


if __name__ == "__main__":
    main()
