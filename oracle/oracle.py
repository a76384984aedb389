"""TEST INFRASTRUCTURE ONLY: ctypes access to the C oracle (oracle/lx_oracle.c).

The oracle restates the stock decode of the chip layers (transformers' Qwen3_5 decoder layer in
lx/lx/hf.py:169-184's chip view) on the CPU. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may use it, and only as the checker.

The oracle builds its own CSR tables from a ``linuxformer_amd.synth.SparseModel``'s coordinate
tensors (sorted by row then column), independently of the product's packer.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liblxoracle.so")

I32, F32, PTR = ctypes.c_int, ctypes.c_float, ctypes.c_void_p

ELEM = {"exp": 0, "silu": 1, "sigmoid": 2, "softplus": 3, "rsqrt": 4, "log1p": 5, "bf16": 6}


class Dims(ctypes.Structure):
    _fields_ = [(n, I32) for n in ("hidden", "n_layers", "nk", "kd", "nv", "vd", "conv", "inter",
                                   "vocab", "bf16")] + [("rms_eps", F32), ("gated_eps", F32)]


class Csr(ctypes.Structure):
    _fields_ = [("nrows", I32), ("ncols", I32), ("ptr", PTR), ("col", PTR), ("val", PTR),
                ("blocks", I32), ("pad", I32)]


class Layer(ctypes.Structure):
    _fields_ = [(n, Csr) for n in ("qkv", "z", "b", "a", "out", "gate", "up", "down")] + \
        [(n, PTR) for n in ("conv_w", "A_log", "dt_bias", "gnorm", "ln_in", "ln_post")]


class Model(ctypes.Structure):
    _fields_ = [("d", Dims), ("layers", PTR), ("embed", Csr), ("final_norm", PTR)]


def build(force: bool = False) -> str:
    src = os.path.join(HERE, "lx_oracle.c")
    if force or not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(src):
        subprocess.run(["make", "-s", "-B", "-C", HERE], check=True)
    return LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
        _lib.ox_expf.restype = F32
        _lib.ox_expf.argtypes = [F32]
        _lib.ox_sum_h.restype = F32
        _lib.ox_sum_h.argtypes = [PTR, I32]
        _lib.ox_sum_64.restype = F32
        _lib.ox_sum_64.argtypes = [PTR, I32]
        _lib.ox_elem.argtypes = [I32, PTR, PTR, ctypes.c_long]
        _lib.ox_decode.restype = I32
        _lib.ox_decode.argtypes = [PTR, PTR, PTR, PTR, I32, I32, PTR, PTR, PTR]
        _lib.ox_layer_step.argtypes = [PTR, I32, PTR, PTR, PTR]
        _lib.ox_head.argtypes = [PTR, PTR, I32, PTR, PTR]
        _lib.ox_rec_step.argtypes = [I32, I32, I32] + [PTR] * 7
        _lib.ox_set_flush.argtypes = [I32]
        _lib.ox_row_dot.restype = F32
        _lib.ox_row_dot.argtypes = [I32, I32, PTR, PTR]
    return _lib


def set_flush(on: bool) -> None:
    """Model oneDNN's bf16 GEMM on AMX hosts (denormal inputs and sums flushed to zero) in the
    bf16 matrix products: only for showing that this is all that separates the contract from the
    stock forward on such a host. Off by default."""
    lib().ox_set_flush(int(bool(on)))


def _p(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def elem(fn: str, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().ox_elem(ELEM[fn], _p(x), _p(y), x.size)
    return y


def sum_h(x) -> np.float32:
    x = np.ascontiguousarray(x, np.float32)
    return np.float32(lib().ox_sum_h(_p(x), len(x)))


def sum_64(x) -> np.float32:
    x = np.ascontiguousarray(x, np.float32)
    return np.float32(lib().ox_sum_64(_p(x), len(x)))


def row_dot(x, w, dense: bool) -> np.float32:
    """x . w in a row's order: in order from +0, or (dense) the dense order."""
    x, w = np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32)
    return np.float32(lib().ox_row_dot(64 if dense else 0, len(x), _p(x), _p(w)))


def rec_step(q, k, v, g, beta, S, bf16: bool):
    """One token of torch_recurrent_gated_delta_rule (q, k (nk, 256); v (nv, 128); g, beta (nv);
    S (nv, 256, 128) updated in place). Returns o (nv, 128)."""
    q, k, v, g, beta = (np.ascontiguousarray(a, np.float32) for a in (q, k, v, g, beta))
    assert S.dtype == np.float32 and S.flags.c_contiguous
    o = np.zeros((v.shape[0], 128), np.float32)
    lib().ox_rec_step(q.shape[0], v.shape[0], int(bf16), _p(q), _p(k), _p(v), _p(g), _p(beta),
                      _p(S), _p(o))
    return o


def chunk_gdr(q, k, v, g, beta, S, C: int = 64):
    """torch_chunk_gated_delta_rule for one value head (q, k (T, K) l2-normed; v (T, V); g, beta
    (T)); S (K, V) float32 updated in place to the final state. Returns o (T, V) float32."""
    q, k, v, g, beta = (np.ascontiguousarray(a, np.float32) for a in (q, k, v, g, beta))
    assert S.dtype == np.float32 and S.flags.c_contiguous
    T, K = q.shape
    V = v.shape[1]
    o = np.zeros((T, V), np.float32)
    rc = lib().ox_chunk_gdr(T, K, V, C, _p(q), _p(k), _p(v), _p(g), _p(beta), _p(S), _p(o))
    if rc:
        raise ValueError("chunk_gdr: unsupported sizes")
    return o


class OracleModel:
    """A SparseModel's tensors in the oracle's C layout (owns every array it points to)."""

    def __init__(self, model):
        self.model = model
        d = model.dims
        self.keep = []
        self.dims = Dims(hidden=d.hidden, n_layers=d.n_layers, nk=d.nk, kd=d.kd, nv=d.nv,
                         vd=d.vd, conv=d.conv, inter=d.inter, vocab=d.vocab,
                         bf16=1 if d.dtype == "bf16" else 0, rms_eps=d.rms_eps,
                         gated_eps=d.geps)
        layers = (Layer * max(d.n_layers, 1))()
        for L, ly in enumerate(model.layers):
            o = layers[L]
            for name, coo in (("qkv", ly.in_proj_qkv), ("z", ly.in_proj_z), ("b", ly.in_proj_b),
                              ("a", ly.in_proj_a), ("out", ly.out_proj), ("gate", ly.gate_proj),
                              ("up", ly.up_proj), ("down", ly.down_proj)):
                setattr(o, name, self._csr(coo))
            o.conv_w = self._arr(ly.conv1d)
            o.A_log, o.dt_bias = self._arr(ly.A_log), self._arr(ly.dt_bias)
            o.gnorm = self._arr(ly.norm)
            o.ln_in, o.ln_post = self._arr(ly.input_layernorm), self._arr(ly.post_attention_layernorm)
        self.layers = layers
        self.c = Model(d=self.dims, layers=ctypes.cast(layers, PTR), embed=self._csr(model.embed),
                       final_norm=self._arr(model.norm))

    def _arr(self, a, dt=np.float32):
        a = np.ascontiguousarray(a, dt)
        self.keep.append(a)
        return _p(a)

    def _csr(self, coo) -> Csr:
        rows = np.asarray(coo.rows, np.int64)
        cols, vals = np.asarray(coo.cols), np.asarray(coo.vals)
        dr, dc = np.diff(rows), np.diff(cols.astype(np.int64))
        if not ((dr > 0) | ((dr == 0) & (dc > 0))).all():  # (already in (row, column) order: kept)
            order = np.lexsort((cols, rows))  # (dense matrices keep their explicit zeros)
            rows, cols, vals = rows[order], cols[order], vals[order]
        ptr = np.zeros(coo.shape[0] + 1, np.int64)
        np.cumsum(np.bincount(rows, minlength=coo.shape[0]), out=ptr[1:])
        blocks = int(getattr(coo, "blocks", 0))
        assert blocks in (0, 64)
        if blocks:  # every stored row: a multiple of 64 entries (the oracle aborts otherwise)
            assert (np.diff(ptr) % 64 == 0).all(), "a dense row needs a multiple of 64 entries"
        return Csr(nrows=coo.shape[0], ncols=coo.shape[1], ptr=self._arr(ptr, np.int64),
                   col=self._arr(cols, np.int32), val=self._arr(vals), blocks=blocks)

    def decode(self, conv: np.ndarray, rec: np.ndarray, forced, n: int, trace: bool = False):
        """n greedy steps from forced tokens, conv/rec (float32 numpy, updated in place).
        Returns (preds, inputs, trace or None)."""
        d = self.model.dims
        assert conv.dtype == np.float32 and conv.flags.c_contiguous
        assert rec.dtype == np.float32 and rec.flags.c_contiguous
        f = np.ascontiguousarray(forced, np.int32)
        preds = np.zeros(n, np.int32)
        inputs = np.zeros(n, np.int32)
        tr = np.zeros((n, d.n_layers, d.hidden), np.float32) if trace else None
        rc = lib().ox_decode(ctypes.byref(self.c), _p(conv), _p(rec), _p(f), len(f), n,
                             _p(preds), _p(inputs), _p(tr) if trace else None)
        if rc:
            raise ValueError("oracle: token id out of range")
        return preds, inputs, tr

    def prefill_chunked(self, conv: np.ndarray, rec: np.ndarray, tokens, C: int = 64,
                        trace: bool = False):
        """The stock forward's T > 1 path over tokens (ox_prefill_chunked): conv/rec (float32
        numpy) updated in place. Returns (every position's argmax, the last layer's outputs
        (T, hidden), trace (T, n_layers, hidden) or None)."""
        d = self.model.dims
        assert conv.dtype == np.float32 and conv.flags.c_contiguous
        assert rec.dtype == np.float32 and rec.flags.c_contiguous
        t = np.ascontiguousarray(tokens, np.int32)
        T = len(t)
        h = np.zeros((T, d.hidden), np.float32)
        if lib().ox_embed(ctypes.byref(self.c), _p(t), T, _p(h)):
            raise ValueError("oracle: token id out of range")
        tr = np.zeros((T, d.n_layers, d.hidden), np.float32) if trace else None
        lib().ox_prefill_chunked(ctypes.byref(self.c), _p(conv), _p(rec), _p(h), T, C,
                                 _p(tr) if trace else None)
        return self.head(h), h, tr

    def layer_step(self, L: int, h: np.ndarray, conv_L: np.ndarray, rec_L: np.ndarray):
        """One layer's decode step on residual h (float32, updated in place)."""
        lib().ox_layer_step(ctypes.byref(self.c), L, _p(h), _p(conv_L), _p(rec_L))

    def head(self, h: np.ndarray, logits: bool = False):
        h = np.ascontiguousarray(h, np.float32).reshape(-1, self.model.dims.hidden)
        T = h.shape[0]
        pred = np.zeros(T, np.int32)
        lg = np.zeros((T, self.model.dims.vocab), np.float32) if logits else None
        lib().ox_head(ctypes.byref(self.c), _p(h), T, _p(lg) if logits else None, _p(pred))
        return (pred, lg) if logits else pred
