"""Write the golden vectors: the stock forward's outputs on small seeded inputs.

The stock forward is transformers 5.15.0's Qwen3_5 decoder layers (torch fallbacks; neither
fla nor the hub kernels are installed) in lx/lx/hf.py's chip view, run token by token on the CPU
by oracle/stock.py; the reference pins 5.19.0 (requirements.txt:4), whose qwen3_5 code path for
these ops is the same. Nothing of the reference repository is imported.

    python tests/golden/make_golden.py      # rewrites tests/golden/*.npz

Each fixture holds the inputs' seeds and shapes (rebuilt by linuxformer_amd.synth), the greedy
stream, every step's per-layer residual (float32) or a hash of it, and the final states' hashes
plus a sample of their values.
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from linuxformer_amd import synth  # noqa: E402
from oracle import stock  # noqa: E402

CASES = {
    # name: (spec builder, steps, keep full traces)
    "c1_64": (lambda: synth.config1(), 64, False),
    "small_bf16_32": (lambda: synth.small(), 32, True),
    "small_fp32_32": (lambda: synth.small(dtype="fp32", seed=3), 32, True),
    "tiny_fp32_8": (lambda: "tiny_fp32", 8, True),
    "tiny_bf16_8": (lambda: "tiny_bf16", 8, True),
}


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


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


def main():
    torch.set_grad_enabled(False)
    for name, (_, n, full) in CASES.items():
        m, conv0, rec0, start = model_of(name)
        hf = synth.to_hf(m)
        preds, trace, conv, rec = stock.decode(hf, conv0, rec0, [start], n)
        rng = np.random.default_rng(0)
        ridx = rng.integers(0, rec.size, 4096)
        out = {"preds": preds, "start": np.int64(start), "n": np.int64(n),
               "conv_sha": sha(conv), "rec_sha": sha(rec), "rec_idx": ridx,
               "rec_sample": rec.reshape(-1)[ridx], "trace_sha": sha(trace),
               "conv_sample": conv.reshape(-1)[rng.integers(0, conv.size, 4096)],
               "conv_idx": rng.integers(0, conv.size, 4096)}
        out["conv_sample"] = conv.reshape(-1)[out["conv_idx"]]
        if full:
            out["trace"] = trace
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **out)
        print(name, os.path.getsize(path), "bytes", preds.tolist()[:8])


if __name__ == "__main__":
    main()
