"""The verified-mode outputs at config 3's shape against the stock T > 1 forward's golden
(tests/golden/c3_pf64.npz, written by tests/golden/make_golden.py): the bounds shared by the
oracle's test (test_oracle.py) and the kernel's (test_gpu_prefill.py)."""

import os

import numpy as np


def c3_stock_fixture():
    return dict(np.load(os.path.join(os.path.dirname(__file__), "golden", "c3_pf64.npz")))


def check_against_stock_c3(traces, preds, conv, rec, g):
    """The verified-mode outputs at config 3's shape against the stock T > 1 forward's
    (tests/golden/c3_pf64.npz): the same argmax at every position; each layer's outputs within
    1e-6 of that layer's largest magnitude at the fixture's 4,096 samples (the north star's
    per-layer bound; the decode form and the chunked form round their fp32 sums apart, measured
    <= 1.6e-7 over every value); the final recurrent states within 1e-6 of their largest
    magnitude (measured 7.5e-8); the conv windows (bf16 projections) within one bf16 step of
    their largest magnitude, 2^-8 (measured 2.6e-4)."""
    assert preds.tolist() == g["preds"].tolist()
    want = (g["trace_bf16"].astype(np.uint32) << 16).view(np.float32)  # (L, 4096)
    for L in range(want.shape[0]):
        got = traces[L][g["pos"], g["col"]]
        assert np.abs(got - want[L]).max() <= 1e-6 * float(g["layer_max"][L]), L
    assert np.abs(rec.reshape(-1)[g["rec_idx"]] - g["rec_sample"]).max() <= 1e-6 * float(g["rec_max"])
    assert np.abs(conv.reshape(-1)[g["conv_idx"]] - g["conv_sample"]).max() <= \
        2.0 ** -8 * float(g["conv_max"])

