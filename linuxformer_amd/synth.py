"""Seeded synthetic chip stacks (the benchmark's configurations) as sparse checkpoint tensors.

The reference measures only the real chip, whose 32 GB checkpoint is not available offline, so
every workload here is synthetic and fully determined by a seed. A ``SparseModel`` holds the
same tensors a stock ``Qwen3_5ForCausalLM`` chip model carries (the names of
transformers/models/qwen3_5/modeling_qwen3_5.py:387-430 and :704-793; the tied embedding/head of
lx/lx/hf.py:179-184), but in coordinate form, so that a 37-layer stack at 0.08 % density costs
megabytes instead of the 16 GB its dense bf16 tensors would. ``to_hf`` materialises small
models as a real transformers model (the stock forward used to pin the oracle).

Write gates. Most chip layer-steps leave the recurrent state and the residual stream alone: the
real chip's decode touches ~4.5 state rows per token (lx/results/head_activity.json). The
synthetic stacks reproduce that with one *gate column* per layer at the top of the residual
stream: a layer's query, key and decay projections read only its gate column, no projection
writes gate columns, and a token's embedding row sets the gate columns of p_gate x n_layers
seeded layers (config 2: exactly one). The query/key channels of the benchmark stacks convolve
only the current token (their earlier taps are 0; ``qk_window``), so a layer-step has a nonzero
query, key or decay exactly when its own input token carries that layer's gate, i.e. on
``p_gate`` of layer-steps whatever tokens the greedy stream visits (with earlier taps a gate
would stay open for the following three tokens too). The final norm weight is -1 on gate
columns, so the head's argmax never sees them. Everything else is uniform at the configured density, except that a SwiGLU unit's
up_proj row reads the same (seeded, uniform) columns as its gate_proj row, so that units fire
and the residual stream mixes across layers.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace

import numpy as np

VALS = np.array([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0], dtype=np.float32)

# component ids for per-(layer, component) seeds
_QKV, _Z, _B, _A, _OUT, _CONV, _GATE, _UP, _DOWN, _LIVE, _EMB, _GEMB, _FN, _STATE, _START, \
    _HD, _MERGE = range(17)


@dataclass
class Coo:
    """A sparse matrix: rows, cols (int64), vals (float32, exact in the model dtype), sorted by
    row then column, no duplicates."""
    shape: tuple
    rows: np.ndarray
    cols: np.ndarray
    vals: np.ndarray
    blocks: int = 0  # 64: a dense matrix, rows summed in the dense order (every live column kept)

    @staticmethod
    def build(shape, rows, cols, vals) -> "Coo":
        rows = np.asarray(rows, np.int64)
        cols = np.asarray(cols, np.int64)
        vals = np.asarray(vals, np.float32)
        keep = vals != 0
        rows, cols, vals = rows[keep], cols[keep], vals[keep]
        key = rows * shape[1] + cols
        order = np.argsort(key, kind="stable")
        key = key[order]
        assert len(key) < 2 or np.all(np.diff(key) > 0), "duplicate entries"
        return Coo(tuple(shape), rows[order], cols[order], vals[order])

    @staticmethod
    def from_dense(w) -> "Coo":
        w = np.asarray(w, np.float32)
        r, c = np.nonzero(w)
        return Coo(tuple(w.shape), r.astype(np.int64), c.astype(np.int64), w[r, c])

    @property
    def nnz(self) -> int:
        return len(self.vals)

    def dense(self) -> np.ndarray:
        out = np.zeros(self.shape, np.float32)
        out[self.rows, self.cols] = self.vals
        return out

    def transpose(self) -> "Coo":
        return Coo.build((self.shape[1], self.shape[0]), self.cols, self.rows, self.vals)


@dataclass
class Dims:
    hidden: int
    n_layers: int
    nk: int = 16
    kd: int = 256
    nv: int = 128
    vd: int = 128
    conv: int = 4
    inter: int = 1024
    vocab: int = 4096
    dtype: str = "bf16"  # model dtype: "bf16" or "fp32"
    rms_eps: float = 1e-6
    gated_eps: float | None = None  # the gated norm's eps (None: rms_eps, as the stock layer)

    @property
    def geps(self) -> float:
        return self.rms_eps if self.gated_eps is None else self.gated_eps

    @property
    def n_conv(self) -> int:
        return 2 * self.nk * self.kd + self.nv * self.vd


@dataclass
class Layer:
    in_proj_qkv: Coo
    in_proj_z: Coo
    in_proj_b: Coo
    in_proj_a: Coo
    out_proj: Coo
    conv1d: np.ndarray  # (n_conv, conv) float32
    A_log: np.ndarray  # (nv,)
    dt_bias: np.ndarray  # (nv,)
    norm: np.ndarray  # (vd,) the gated norm's weight
    input_layernorm: np.ndarray  # (hidden,) raw weight w (the module scales by 1 + w)
    post_attention_layernorm: np.ndarray
    gate_proj: Coo
    up_proj: Coo
    down_proj: Coo


@dataclass
class SparseModel:
    dims: Dims
    layers: list
    embed: Coo  # (vocab, hidden), tied to the output head
    norm: np.ndarray  # (hidden,) final norm weight
    meta: dict = field(default_factory=dict)


@dataclass
class Spec:
    """A synthetic stack: shapes, density, gates and seeds (benchmark configs 1, 2, 3 and 5)."""
    name: str
    dims: Dims
    seed: int = 0
    density: float = 0.0008
    p_gate: float = 0.02  # gated fraction of (token, layer) pairs; each token gates p_gate x
    # n_layers layers (rounded up or down at random), so config 2's tokens gate one layer each
    p_live: float = 0.25  # per key head: reads the gate (query/key rows)
    p_decay: float = 0.25  # per value head of a live key head: in_proj_a reads the gate
    p_tap: float = 0.1  # per earlier conv tap of a live channel
    qk_window: bool = False  # query/key channels get earlier taps too (gates stay open 3 more steps)
    gate_gain: float = 64.0  # 1 + input_layernorm weight on gate columns
    dt_bias: float = -112.0  # softplus(dt_bias) == 0 in fp32: no decay without the gate
    emb_nnz: int = 3  # nonzeros per embedding row outside the gate columns
    state: str = "normal"  # initial recurrent state: "normal" (N(0,1)) or "zero"
    n_steps: int = 256
    # dense head columns (the real chip's head has 31: every row nonzero, few distinct values,
    # lx/results/mega_boot.json's head_dense): this many seeded non-gate columns of the tied
    # embedding get a value on (almost) every row, from 4 values per column (the last column
    # from {0, +-1/2, 1}, so it holds zeros too)
    head_dense: int = 0


def config1(seed: int = 1) -> Spec:
    """Benchmark config 1: one chip-shaped GDN + SwiGLU layer, fp32, zero state, 4,096 tokens.
    A single layer at 0.08 % density barely mixes the residual stream, so a quarter of its
    layer-steps are gated on (the delta rule, its writes into the zero state and their reads)."""
    return Spec("c1", Dims(hidden=3572, n_layers=1, vocab=4096, dtype="fp32"), seed=seed,
                state="zero", n_steps=256, p_gate=0.25)


def config2(seed: int = 2) -> Spec:
    """Benchmark config 2: the 37-layer synthetic chip stack, bf16, N(0,1) state; every token
    gates exactly one layer (1/37 = 2.7 % of layer-steps, the benchmark's "about 2 %")."""
    return Spec("c2", Dims(hidden=3572, n_layers=37, vocab=459_982, dtype="bf16"), seed=seed,
                state="normal", n_steps=262_144, p_gate=1.0 / 37)


def config3(seed: int = 2) -> Spec:
    """Benchmark config 3: verified mode (the prefill) over config 2's stack, 65,536 seeded
    uniform token ids per call. A token gates a layer with probability 0.35 % (0.13 gates per
    token over the 37 layers), so a live key head (a quarter of them) is active in a 64-token
    chunk with probability 1 - (1 - 0.0035)^64 = 20 %: 5 % of (key head, chunk) pairs, as the
    config states."""
    s = config2(seed)
    return replace(s, name="c3", p_gate=0.0035, n_steps=65_536)


def config5(seed: int = 2) -> Spec:
    """Benchmark config 5: config 2's stack with gates on for half of the layer-steps."""
    s = config2(seed)
    return replace(s, name="c5", p_gate=0.5, n_steps=65_536)


def small(seed: int = 7, n_layers: int = 3, hidden: int = 192, vocab: int = 512,
          dtype: str = "bf16", p_gate: float = 0.3, density: float = 0.05,
          state: str = "normal") -> Spec:
    """A small stack of the chip's head shapes (KD 256, VD 128) for fast parity tests."""
    return Spec("small", Dims(hidden=hidden, n_layers=n_layers, nk=2, nv=8, inter=48,
                              vocab=vocab, dtype=dtype), seed=seed, density=density,
                p_gate=p_gate, p_live=1.0, p_decay=0.5, p_tap=0.3, emb_nnz=6, state=state,
                n_steps=64, qk_window=True)


def _rng(seed: int, *k: int) -> np.random.Generator:
    return np.random.default_rng([seed, *k])


def _uniform(rng, rows: np.ndarray, cols: np.ndarray, density: float, shape) -> Coo:
    """Nonzeros at round(density * n) seeded uniform positions of the submatrix rows x cols,
    values uniform over VALS."""
    n = len(rows) * len(cols)
    k = int(round(density * n))
    if k == 0 or n == 0:
        return Coo.build(shape, [], [], [])
    pos = rng.choice(n, size=k, replace=False)
    return Coo.build(shape, rows[pos // len(cols)], cols[pos % len(cols)],
                     rng.choice(VALS, size=k))


def _layer(spec: Spec, L: int) -> Layer:
    d, s = spec.dims, spec.seed
    H, nk, kd, nv, vd, R = d.hidden, d.nk, d.kd, d.nv, d.vd, d.nv // d.nk
    C = d.n_conv
    ng = np.arange(H - d.n_layers)  # columns (rows) that are not gate columns
    gcol = H - d.n_layers + L
    # live key heads: their query and key rows read the gate column
    rl = _rng(s, L, _LIVE)
    live = rl.random(nk) < spec.p_live
    if not live.any():
        live[rl.integers(nk)] = True
    qr, qc, qv = [], [], []
    for kh in np.nonzero(live)[0]:
        for base, lo, hi in ((kh * kd, 1, 5), (nk * kd + kh * kd, 1, 3)):
            n = int(rl.integers(lo, hi))
            rows = base + rl.choice(kd, size=n, replace=False)
            qr += list(rows)
            qc += [gcol] * n
            qv += list(rl.choice(VALS, size=n))
    qk = Coo.build((C, H), qr, qc, qv)
    v_rows = np.arange(2 * nk * kd, C)
    v = _uniform(_rng(s, L, _QKV), v_rows, ng, spec.density, (C, H))
    qkv = Coo.build((C, H), np.concatenate([qk.rows, v.rows]), np.concatenate([qk.cols, v.cols]),
                    np.concatenate([qk.vals, v.vals]))
    # conv taps: tap conv-1 (the current input) on every channel with a projection row, earlier
    # taps seeded
    rc = _rng(s, L, _CONV)
    has_row = np.zeros(C, bool)
    has_row[qkv.rows] = True
    conv = np.zeros((C, d.conv), np.float32)
    conv[has_row, d.conv - 1] = rc.choice(VALS, size=int(has_row.sum()))
    extra = (rc.random((C, d.conv - 1)) < spec.p_tap) & has_row[:, None]
    conv[:, :d.conv - 1] = np.where(extra, rc.choice(VALS, size=(C, d.conv - 1)), 0.0)
    if not spec.qk_window:
        conv[:2 * nk * kd, :d.conv - 1] = 0.0
    # decay projections: some value heads of live key heads read the gate
    ra = _rng(s, L, _A)
    vh_live = np.repeat(live, R)
    dec = vh_live & (ra.random(nv) < spec.p_decay)
    a = Coo.build((nv, H), np.nonzero(dec)[0], np.full(int(dec.sum()), gcol),
                  ra.choice(VALS, size=int(dec.sum())))
    vrows_h = np.arange(nv * vd)
    # SwiGLU units: up_proj's row reads the columns its gate_proj row reads (seeded uniform
    # positions, independent values), so a unit fires whenever its inputs are nonzero
    gate = _uniform(_rng(s, L, _GATE), np.arange(d.inter), ng, spec.density, (d.inter, H))
    lay = Layer(
        in_proj_qkv=qkv,
        in_proj_z=_uniform(_rng(s, L, _Z), vrows_h, ng, spec.density, (nv * vd, H)),
        in_proj_b=_uniform(_rng(s, L, _B), np.arange(nv), ng, spec.density, (nv, H)),
        in_proj_a=a,
        out_proj=_uniform(_rng(s, L, _OUT), ng, np.arange(nv * vd), spec.density, (H, nv * vd)),
        conv1d=conv,
        A_log=np.zeros(nv, np.float32),
        dt_bias=np.full(nv, spec.dt_bias, np.float32),
        norm=np.ones(vd, np.float32),
        input_layernorm=np.zeros(H, np.float32),
        post_attention_layernorm=np.zeros(H, np.float32),
        gate_proj=gate,
        up_proj=Coo.build(gate.shape, gate.rows, gate.cols,
                          _rng(s, L, _UP).choice(VALS, size=gate.nnz)),
        down_proj=_uniform(_rng(s, L, _DOWN), ng, np.arange(d.inter), spec.density, (H, d.inter)),
    )
    lay.input_layernorm[H - d.n_layers:] = spec.gate_gain - 1.0
    lay.post_attention_layernorm[H - d.n_layers:] = -1.0
    return lay


def build(spec: Spec, layers: list | None = None) -> SparseModel:
    """The seeded stack of ``spec`` (weights only; see ``init_state`` for the caches). ``layers``:
    the layers of a stack built from a spec that differs from this one only in p_gate (configs
    2, 3 and 5), reused as they are (a layer does not depend on p_gate; only the embedding's
    gate columns do)."""
    d, s = spec.dims, spec.seed
    H, V = d.hidden, d.vocab
    assert d.nv % d.nk == 0 and H > d.n_layers
    if layers is None:
        layers = [_layer(spec, L) for L in range(d.n_layers)]
    assert len(layers) == d.n_layers
    # embedding: emb_nnz distinct non-gate columns per row, plus each layer's gate at p_gate
    re = _rng(s, 0, _EMB)
    hng = H - d.n_layers
    k = min(spec.emb_nnz, hng)
    cols = np.stack([re.choice(hng, size=k, replace=False) for _ in range(min(V, 4096))]) \
        if V <= 4096 else _distinct_cols(re, V, hng, k)
    rows = np.repeat(np.arange(V), k)
    vals = re.choice(VALS, size=V * k)
    # gates: token v sets the gate columns of k_v seeded layers, k_v = floor(g) or floor(g) + 1
    # with mean g = p_gate * n_layers, so every token carries (almost) the same number of gates
    # and the stream's gate rate is p_gate whatever tokens the greedy decode visits
    rg = _rng(s, 0, _GEMB)
    g = spec.p_gate * d.n_layers
    k = np.floor(g).astype(np.int64) + (rg.random(V) < g - np.floor(g))
    order = np.argsort(rg.random((V, d.n_layers)), axis=1)
    on = np.arange(d.n_layers)[None, :] < k[:, None]
    gr = np.repeat(np.arange(V), on.sum(1))
    gc = hng + order[on]
    rows, cols = np.concatenate([rows, gr]), np.concatenate([cols.reshape(-1), gc])
    vals = np.concatenate([vals, rg.choice(VALS, size=len(gr))])
    if spec.head_dense:
        rd = _rng(s, 0, _HD)
        dcols = rd.choice(hng, size=spec.head_dense, replace=False)
        keep = ~np.isin(cols, dcols)
        rows, cols, vals = rows[keep], cols[keep], vals[keep]
        for j, c in enumerate(dcols):
            tab = [-1.0, -0.5, 0.5, 1.0] if j + 1 < len(dcols) else [0.0, -0.5, 0.5, 1.0]
            rows = np.concatenate([rows, np.arange(V)])
            cols = np.concatenate([cols, np.full(V, c)])
            vals = np.concatenate([vals, rd.choice(np.asarray(tab, np.float32), size=V)])
    embed = Coo.build((V, H), rows, cols, vals)
    # final norm: weight 0 or -2 (1 + w = +-1) outside the gates, -1 on them (the head ignores
    # the gates)
    rf = _rng(s, 0, _FN)
    norm = np.where(rf.random(H) < 0.5, -2.0, 0.0).astype(np.float32)
    norm[hng:] = -1.0
    return SparseModel(d, layers, embed, norm, meta={"spec": spec})


def merged(model: SparseModel, offset: int, seed: int = 0) -> SparseModel:
    """The chip stack inside a larger vocabulary, as the reference's merged model holds it
    (lx/lx/merge.py; lx/lx/linux.py:108-109): ``offset`` seeded rows of other tokens (a few
    nonzeros each) before the chip's embedding rows, so chip token t is row offset + t.
    ``Fast(m, rows=slice(offset, offset + vocab))`` and ``Mega(..., offset)`` select the chip's
    rows again; the layers are the chip's."""
    d = model.dims
    r = _rng(seed, 0, _MERGE)
    k = 4
    xc = np.stack([r.choice(d.hidden, size=k, replace=False) for _ in range(offset)]) if offset \
        else np.zeros((0, k), np.int64)
    xr = np.repeat(np.arange(offset), k)
    e = model.embed
    emb = Coo.build((offset + d.vocab, d.hidden), np.concatenate([xr, e.rows + offset]),
                    np.concatenate([xc.reshape(-1), e.cols]),
                    np.concatenate([r.choice(VALS, size=offset * k), e.vals]))
    return SparseModel(replace(d, vocab=offset + d.vocab), model.layers, emb, model.norm,
                       meta={**model.meta, "merged_offset": offset})


def _distinct_cols(rng, V: int, n: int, k: int) -> np.ndarray:
    cols = rng.integers(0, n, size=(V, k))
    while True:
        s = np.sort(cols, axis=1)
        bad = np.nonzero((np.diff(s, axis=1) == 0).any(1))[0]
        if len(bad) == 0:
            return cols
        cols[bad] = rng.integers(0, n, size=(len(bad), k))


def init_state(model: SparseModel, kind: str | None = None, seed: int | None = None):
    """The initial caches: conv windows (n_layers, n_conv, conv) zero and recurrent states
    (n_layers, nv, kd, vd) float32, N(0,1) (seeded per layer, row by row) or zero. Returns
    numpy arrays; conv windows hold values exact in the model dtype."""
    d = model.dims
    spec = model.meta.get("spec")
    kind = kind or (spec.state if spec else "zero")
    seed = seed if seed is not None else (spec.seed if spec else 0)
    conv = np.zeros((d.n_layers, d.n_conv, d.conv), np.float32)
    rec = np.zeros((d.n_layers, d.nv, d.kd, d.vd), np.float32)
    if kind == "normal":
        for L in range(d.n_layers):
            rec[L] = _rng(seed, L, _STATE).standard_normal((d.nv, d.kd, d.vd), np.float32)
    return conv, rec


def tokens(spec: Spec, n: int | None = None, seed: int = 0) -> np.ndarray:
    """n seeded uniform token ids over the vocabulary (config 3's verified-mode input)."""
    n = spec.n_steps if n is None else n
    return _rng(spec.seed, 1 + seed, _START).integers(0, spec.dims.vocab, n).astype(np.int64)


def start_token(spec: Spec) -> int:
    return int(_rng(spec.seed, 0, _START).integers(0, spec.dims.vocab))


def tiny_dense(seed: int = 0, dtype: str = "fp32", hidden: int = 64, n_layers: int = 2,
               nk: int = 4, nv: int = 32, inter: int = 64, vocab: int = 96,
               scale: float = 0.08) -> SparseModel:
    """A small dense random stack (every weight nonzero, N(0, scale) rounded to the dtype):
    every head is live at every step, so every sum of the step has its full length. Used to
    pin the oracle against the stock transformers forward."""
    d = Dims(hidden=hidden, n_layers=n_layers, nk=nk, nv=nv, inter=inter, vocab=vocab,
             dtype=dtype)
    rng = np.random.default_rng([seed, 99])

    def w(*shape, s=scale):
        return _round(rng.standard_normal(shape).astype(np.float32) * s, dtype)

    H, C = hidden, d.n_conv
    layers = []
    for _ in range(n_layers):
        layers.append(Layer(
            in_proj_qkv=Coo.from_dense(w(C, H)), in_proj_z=Coo.from_dense(w(nv * d.vd, H)),
            in_proj_b=Coo.from_dense(w(nv, H, s=0.5)), in_proj_a=Coo.from_dense(w(nv, H, s=0.5)),
            out_proj=Coo.from_dense(w(H, nv * d.vd)),
            conv1d=w(C, d.conv, s=0.5), A_log=w(nv, s=0.5), dt_bias=w(nv, s=0.5),
            norm=1.0 + w(d.vd, s=0.1), input_layernorm=w(H, s=0.1),
            post_attention_layernorm=w(H, s=0.1), gate_proj=Coo.from_dense(w(inter, H, s=0.3)),
            up_proj=Coo.from_dense(w(inter, H, s=0.3)), down_proj=Coo.from_dense(w(H, inter)),
        ))
    embed = Coo.from_dense(w(vocab, H, s=1.0))
    return SparseModel(d, layers, embed, w(H, s=0.1), meta={"tiny": seed})


def _round(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded to the model dtype (bf16: round to nearest even), as float32."""
    if dtype == "fp32":
        return x.astype(np.float32)
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def to_hf(model: SparseModel, dev: str = "cpu"):
    """The model as a stock transformers Qwen3_5ForCausalLM (dense tensors: config 2's stack
    takes 16 GB in bf16 plus 3.3 GB of tied embedding): n_layers linear-attention layers, the
    tied head, the final norm."""
    import torch
    from transformers import Qwen3_5ForCausalLM, Qwen3_5TextConfig

    d = model.dims
    dt = torch.bfloat16 if d.dtype == "bf16" else torch.float32
    cfg = Qwen3_5TextConfig(
        vocab_size=d.vocab, hidden_size=d.hidden, intermediate_size=d.inter,
        num_hidden_layers=d.n_layers, layer_types=["linear_attention"] * d.n_layers,
        linear_key_head_dim=d.kd, linear_value_head_dim=d.vd, linear_num_key_heads=d.nk,
        linear_num_value_heads=d.nv, linear_conv_kernel_dim=d.conv, rms_norm_eps=d.rms_eps,
        tie_word_embeddings=True, hidden_act="silu", num_attention_heads=4,
        num_key_value_heads=1, head_dim=64,
        rope_parameters={"rope_type": "default", "rope_theta": 10000.0,
                         "partial_rotary_factor": 0.25})
    with torch.device("meta"):
        m = Qwen3_5ForCausalLM(cfg)
    sd = {}
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dt)  # noqa: E731

    def dense(coo):  # scattered straight into a zeroed tensor of the model dtype
        w = torch.zeros(coo.shape, dtype=dt)
        if coo.nnz:
            w[torch.from_numpy(coo.rows), torch.from_numpy(coo.cols)] = t(coo.vals)
        return w

    for L, lay in enumerate(model.layers):
        p = f"model.layers.{L}."
        ga = p + "linear_attn."
        sd[ga + "in_proj_qkv.weight"] = dense(lay.in_proj_qkv)
        sd[ga + "in_proj_z.weight"] = dense(lay.in_proj_z)
        sd[ga + "in_proj_b.weight"] = dense(lay.in_proj_b)
        sd[ga + "in_proj_a.weight"] = dense(lay.in_proj_a)
        sd[ga + "out_proj.weight"] = dense(lay.out_proj)
        sd[ga + "conv1d.weight"] = t(lay.conv1d[:, None, :])
        sd[ga + "A_log"] = t(lay.A_log)
        sd[ga + "dt_bias"] = t(lay.dt_bias)
        sd[ga + "norm.weight"] = t(lay.norm)
        sd[p + "input_layernorm.weight"] = t(lay.input_layernorm)
        sd[p + "post_attention_layernorm.weight"] = t(lay.post_attention_layernorm)
        sd[p + "mlp.gate_proj.weight"] = dense(lay.gate_proj)
        sd[p + "mlp.up_proj.weight"] = dense(lay.up_proj)
        sd[p + "mlp.down_proj.weight"] = dense(lay.down_proj)
    sd["model.embed_tokens.weight"] = dense(model.embed)
    sd["model.norm.weight"] = t(model.norm)
    missing, unexpected = m.load_state_dict(sd, strict=False, assign=True)
    assert not unexpected and set(missing) <= {"lm_head.weight"}, (missing[:4], unexpected[:4])
    m.tie_weights()
    from transformers.models.qwen3_5 import modeling_qwen3_5 as q
    m.model.rotary_emb = q.Qwen3_5TextRotaryEmbedding(config=cfg)
    m = m.to(device=dev, dtype=dt).eval()
    if d.gated_eps is not None:  # (the gated norm's own eps, where the stack has one)
        for layer in m.model.layers:
            layer.linear_attn.norm.variance_epsilon = d.gated_eps
    return m


def _coo_rows(w, lo: int, hi: int, block: int = 32768) -> Coo:
    """Rows lo .. hi of a weight tensor in coordinate form, a block of rows at a time (the rows
    are never densified in float32 all at once)."""
    rs, cs, vs = [], [], []
    for a in range(lo, hi, block):
        x = w[a:min(a + block, hi)].detach().float().cpu().numpy()
        r, c = np.nonzero(x)
        rs.append(r.astype(np.int64) + (a - lo))
        cs.append(c.astype(np.int64))
        vs.append(x[r, c])
    cat = lambda z, t: np.concatenate(z) if z else np.zeros(0, t)  # noqa: E731
    return Coo((hi - lo, w.shape[1]), cat(rs, np.int64), cat(cs, np.int64), cat(vs, np.float32))


def from_hf(m, n_chip: int | None = None, rows: slice | None = None) -> SparseModel:
    """A transformers Qwen3_5 chip model's tensors (its first n_chip layers) in coordinate form.
    rows: the head's rows (lx/lx/fast.py:183, the merged model's chip tokens); only those rows of
    the tied embedding are read, and the result's embedding holds them (meta "row0": the first
    one's index in the model)."""
    import torch

    cfg = m.config
    n = n_chip if n_chip is not None else cfg.num_hidden_layers
    dtype = "bf16" if m.dtype == torch.bfloat16 else "fp32"
    w = m.lm_head.weight
    lo = 0 if rows is None else (rows.start or 0)
    hi = w.shape[0] if rows is None or rows.stop is None else min(rows.stop, w.shape[0])
    e = m.model.embed_tokens.weight
    if e.data_ptr() != w.data_ptr() and not all(
            torch.equal(e[a:min(a + 65536, hi)], w[a:min(a + 65536, hi)])
            for a in range(lo, hi, 65536)):
        raise ValueError("the chip path reads one tied table for its inputs and its head: "
                         "lm_head and embed_tokens differ on the chip's rows")
    d = Dims(hidden=cfg.hidden_size, n_layers=n, nk=cfg.linear_num_key_heads,
             kd=cfg.linear_key_head_dim, nv=cfg.linear_num_value_heads,
             vd=cfg.linear_value_head_dim, conv=cfg.linear_conv_kernel_dim,
             inter=cfg.intermediate_size, vocab=hi - lo, dtype=dtype,
             rms_eps=cfg.rms_norm_eps,
             gated_eps=float(m.model.layers[0].linear_attn.norm.variance_epsilon) if n else None)

    def f(x):
        return x.detach().float().cpu().numpy()

    def coo(x):
        return Coo.from_dense(f(x))

    layers = []
    for L in range(n):
        lay = m.model.layers[L]
        ga = lay.linear_attn
        layers.append(Layer(
            in_proj_qkv=coo(ga.in_proj_qkv.weight), in_proj_z=coo(ga.in_proj_z.weight),
            in_proj_b=coo(ga.in_proj_b.weight), in_proj_a=coo(ga.in_proj_a.weight),
            out_proj=coo(ga.out_proj.weight), conv1d=f(ga.conv1d.weight[:, 0]),
            A_log=f(ga.A_log), dt_bias=f(ga.dt_bias), norm=f(ga.norm.weight),
            input_layernorm=f(lay.input_layernorm.weight),
            post_attention_layernorm=f(lay.post_attention_layernorm.weight),
            gate_proj=coo(lay.mlp.gate_proj.weight), up_proj=coo(lay.mlp.up_proj.weight),
            down_proj=coo(lay.mlp.down_proj.weight)))
    return SparseModel(d, layers, _coo_rows(w, lo, hi), f(m.model.norm.weight),
                       meta={"row0": lo})


# ---------------------------------------------------------------------------------------------
# Benchmark config 4: the dense padded text-view stack (lx/lx/merge.py:82-120's layout): key heads
# of dim 256 whose upper 128 dims are zero, 8 value heads per key head of which 2 are live and 6
# zero, bf16 N(0, 0.02) weights on the live blocks. Its projections are dense, so they are summed
# in the dense order (64 groups of a row's entries, then a pairwise tree; the oracle's `blocks`).


@dataclass
class DenseSpec:
    name: str
    hidden: int
    n_layers: int
    nk: int = 16
    kd_live: int = 128      # live dims of each 256-dim key head (the rest zero-padded)
    nv: int = 128
    r_live: int = 2         # live value heads of each key head (the first r_live of its 8)
    inter: int = 9216
    vocab: int = 248_320
    seed: int = 4
    std: float = 0.02
    rms_eps: float = 1e-6
    gated_eps: float = 5e-7
    n_prefill: int = 8192
    n_steps: int = 4096

    def dims(self) -> Dims:
        return Dims(hidden=self.hidden, n_layers=self.n_layers, nk=self.nk, kd=256, nv=self.nv,
                    vd=128, conv=4, inter=self.inter, vocab=self.vocab, dtype="bf16",
                    rms_eps=self.rms_eps, gated_eps=self.gated_eps)


def config4(seed: int = 4) -> DenseSpec:
    """Benchmark config 4: 24 layers, hidden 2560, 16 key heads (256, zero-padded from 128), 128
    value heads (2 live + 6 zero per key head), SwiGLU 9216, gated-norm eps 5e-7, vocabulary
    248,320; an 8,192-token prefill of seeded uniform ids, then 4,096 greedy steps."""
    return DenseSpec("c4", hidden=2560, n_layers=24, seed=seed)


def config4_small(seed: int = 5) -> DenseSpec:
    """Config 4's structure at a size the oracle runs in seconds (the parity tests)."""
    return DenseSpec("c4s", hidden=256, n_layers=2, nk=2, nv=16, inter=512, vocab=1024,
                     seed=seed, n_prefill=24, n_steps=16)


def config4_mid(seed: int = 6) -> DenseSpec:
    """One layer of config 4 at its full widths (hidden 2560, 16 key heads, SwiGLU 9216) with a
    small vocabulary: the parity tests' check of the full row lengths."""
    return DenseSpec("c4m", hidden=2560, n_layers=1, vocab=4096, seed=seed, n_prefill=8, n_steps=8)


@dataclass
class DenseModel:
    """Config 4's tensors on a device: bf16 weights of the live blocks only (the zero-padded
    rows and columns are implicit), float32 small parameters (values exact in bf16)."""
    spec: DenseSpec
    dims: Dims
    layers: list          # dicts of tensors, see build_dense
    embed: object         # (vocab, hidden) bf16, tied to the head
    norm: object          # (hidden,) float32 final norm weight


def build_dense(spec: DenseSpec, device="cpu") -> DenseModel:
    """The seeded dense stack on device (torch generators seeded per (layer, tensor))."""
    import torch

    d = spec.dims()
    H, nk, kl, rl, I = spec.hidden, spec.nk, spec.kd_live, spec.r_live, spec.inter
    dev = torch.device(device)

    def gen(L, c):
        return torch.Generator(device=dev).manual_seed(spec.seed * 1_000_003 + L * 101 + c)

    def w(L, c, *shape, std=None):
        x = torch.randn(*shape, generator=gen(L, c), device=dev, dtype=torch.float32)
        return (x * (spec.std if std is None else std)).to(torch.bfloat16)

    def small(x):
        return x.to(torch.bfloat16).to(torch.float32)

    layers = []
    for L in range(spec.n_layers):
        g = gen(L, 50)
        A = torch.rand(d.nv, generator=g, device=dev) * 15.0 + 1.0
        dt = torch.exp(torch.rand(d.nv, generator=g, device=dev) * (np.log(0.1) - np.log(0.001))
                       + np.log(0.001))
        layers.append({
            "qk": w(L, 0, 2, nk, kl, H),              # query / key rows of the live dims
            "v": w(L, 1, nk, rl, 128, H),             # value rows of the live value heads
            "z": w(L, 2, nk, rl, 128, H),
            "b": w(L, 3, nk, rl, H),
            "a": w(L, 4, nk, rl, H),
            "conv_qk": w(L, 5, 2, nk, kl, 4),
            "conv_v": w(L, 6, nk, rl, 128, 4),
            "A_log": small(torch.log(A)),
            "dt_bias": small(torch.log(torch.expm1(dt))),
            "norm": small(1.0 + w(L, 7, 128).float()),
            "ln_in": small(w(L, 8, H).float()),
            "ln_post": small(w(L, 9, H).float()),
            "out": w(L, 10, H, nk, rl, 128),          # out_proj over the live value dims
            "gate": w(L, 11, I, H),
            "up": w(L, 12, I, H),
            "down": w(L, 13, H, I),
        })
    embed = w(999, 14, spec.vocab, H)
    norm = small(w(999, 15, H).float())
    return DenseModel(spec, d, layers, embed, norm)


def dense_to(dm: DenseModel, device) -> DenseModel:
    """The same model with every tensor on device."""
    return DenseModel(dm.spec, dm.dims, [{k: v.to(device) for k, v in ly.items()} for ly in dm.layers],
                      dm.embed.to(device), dm.norm.to(device))


def dense_state(dm: DenseModel, seed: int | None = None):
    """Initial (conv, rec) for a dense stack as float32 numpy arrays in the padded layout: zero,
    or (seed) N(0, 1) recurrent rows and N(0, 0.02) windows (bf16-exact) on the live heads'
    dims only (the dead heads and padded dims stay zero, as the stock layer keeps them)."""
    sp, d = dm.spec, dm.dims
    R = d.nv // d.nk
    conv = np.zeros((d.n_layers, d.n_conv, 4), np.float32)
    rec = np.zeros((d.n_layers, d.nv, 256, 128), np.float32)
    if seed is None:
        return conv, rec
    rng = np.random.default_rng(seed)
    for kh in range(sp.nk):
        for r in range(sp.r_live):
            vh = kh * R + r
            rec[:, vh, :sp.kd_live] = rng.standard_normal((d.n_layers, sp.kd_live, 128))
            ch = 2 * sp.nk * 256 + vh * 128
            conv[:, ch:ch + 128] = _round(0.02 * rng.standard_normal((d.n_layers, 128, 4)), "bf16")
        for part in (0, 1):
            ch = part * sp.nk * 256 + kh * 256
            conv[:, ch:ch + sp.kd_live] = _round(0.02 * rng.standard_normal((d.n_layers, sp.kd_live, 4)), "bf16")
    return conv, rec


def to_sparse(dm: DenseModel) -> SparseModel:
    """The dense stack as the padded checkpoint tensors in coordinate form, dense matrices marked
    (blocks = 64, every live column kept): the oracle's input. Small stacks only."""
    sp, d = dm.spec, dm.dims
    H, nk, kl, rl, R = sp.hidden, sp.nk, sp.kd_live, sp.r_live, d.nv // d.nk
    C = d.n_conv

    def np32(t):
        return t.float().cpu().numpy()

    def coo_rows(shape, rows, mat, cols):
        rows = np.asarray(rows, np.int64)
        cols = np.asarray(cols, np.int64)
        rr = np.repeat(rows, len(cols))
        cc = np.tile(cols, len(rows))
        vals = np.asarray(mat, np.float32).reshape(-1)
        # (row-major entries of ascending rows and columns are in (row, column) order already)
        if not ((np.diff(rows) > 0).all() and (np.diff(cols) > 0).all()):
            order = np.lexsort((cc, rr))
            rr, cc, vals = rr[order], cc[order], vals[order]
        return Coo(tuple(shape), rr, cc, vals, blocks=64)

    layers = []
    allH = np.arange(H)
    vh_live = np.array([kh * R + r for kh in range(nk) for r in range(rl)], np.int64)
    for ly in dm.layers:
        qk = np32(ly["qk"])          # (2, nk, kl, H)
        qrows = np.array([kh * 256 + i for kh in range(nk) for i in range(kl)], np.int64)
        krows = nk * 256 + qrows
        vrows = 2 * nk * 256 + (vh_live[:, None] * 128 + np.arange(128)[None]).reshape(-1)
        qkv = coo_rows((C, H), np.concatenate([qrows, krows, vrows]),
                       np.concatenate([qk[0].reshape(-1, H), qk[1].reshape(-1, H),
                                       np32(ly["v"]).reshape(-1, H)]), allH)
        conv = np.zeros((C, 4), np.float32)
        conv[qrows] = np32(ly["conv_qk"])[0].reshape(-1, 4)
        conv[krows] = np32(ly["conv_qk"])[1].reshape(-1, 4)
        conv[vrows] = np32(ly["conv_v"]).reshape(-1, 4)
        zrows = (vh_live[:, None] * 128 + np.arange(128)[None]).reshape(-1)
        z = coo_rows((d.nv * 128, H), zrows, np32(ly["z"]).reshape(-1, H), allH)
        b = coo_rows((d.nv, H), vh_live, np32(ly["b"]).reshape(-1, H), allH)
        a = coo_rows((d.nv, H), vh_live, np32(ly["a"]).reshape(-1, H), allH)
        out = coo_rows((H, d.nv * 128), allH, np32(ly["out"]).reshape(H, -1), zrows)
        layers.append(Layer(
            in_proj_qkv=qkv, in_proj_z=z, in_proj_b=b, in_proj_a=a, out_proj=out, conv1d=conv,
            A_log=np32(ly["A_log"]), dt_bias=np32(ly["dt_bias"]), norm=np32(ly["norm"]),
            input_layernorm=np32(ly["ln_in"]), post_attention_layernorm=np32(ly["ln_post"]),
            gate_proj=coo_rows((d.inter, H), np.arange(d.inter), np32(ly["gate"]), allH),
            up_proj=coo_rows((d.inter, H), np.arange(d.inter), np32(ly["up"]), allH),
            down_proj=coo_rows((H, d.inter), allH, np32(ly["down"]), np.arange(d.inter))))
    embed = coo_rows((d.vocab, H), np.arange(d.vocab), np32(dm.embed), allH)
    return SparseModel(d, layers, embed, np32(dm.norm), meta={"dense_spec": sp})


def dense_to_hf(dm: DenseModel):
    """Config 4's stack as the stock transformers Qwen3_5ForCausalLM on the host, in its padded
    layout (lx/lx/merge.py:82-120: 256-dim key heads with zero upper dims, 8 value heads per key
    head of which the first r_live are live; zeros everywhere else), bf16, the gated norm's eps
    set to the spec's. The CPU baseline's model: the reference's stock forward runs it as is."""
    import torch
    from transformers import Qwen3_5ForCausalLM, Qwen3_5TextConfig

    sp, d = dm.spec, dm.dims
    H, nk, kl, rl, R = sp.hidden, sp.nk, sp.kd_live, sp.r_live, d.nv // d.nk
    cfg = Qwen3_5TextConfig(
        vocab_size=d.vocab, hidden_size=H, intermediate_size=d.inter,
        num_hidden_layers=d.n_layers, layer_types=["linear_attention"] * d.n_layers,
        linear_key_head_dim=256, linear_value_head_dim=128, linear_num_key_heads=nk,
        linear_num_value_heads=d.nv, linear_conv_kernel_dim=4, rms_norm_eps=sp.rms_eps,
        tie_word_embeddings=True, hidden_act="silu", num_attention_heads=4,
        num_key_value_heads=1, head_dim=64,
        rope_parameters={"rope_type": "default", "rope_theta": 10000.0,
                         "partial_rotary_factor": 0.25})
    with torch.device("meta"):
        m = Qwen3_5ForCausalLM(cfg)
    bf, cpu = torch.bfloat16, lambda x: x.detach().to("cpu")  # noqa: E731
    vh = torch.tensor([kh * R + r for kh in range(nk) for r in range(rl)])
    vdims = (vh[:, None] * 128 + torch.arange(128)[None]).reshape(-1)
    qrows = torch.tensor([kh * 256 + i for kh in range(nk) for i in range(kl)])
    sd = {}
    for L, ly in enumerate(dm.layers):
        p, ga = f"model.layers.{L}.", f"model.layers.{L}.linear_attn."
        C = 2 * nk * 256 + d.nv * 128
        qkv = torch.zeros(C, H, dtype=bf)
        qk = cpu(ly["qk"]).reshape(2, nk * kl, H)
        qkv[qrows], qkv[nk * 256 + qrows] = qk[0], qk[1]
        qkv[2 * nk * 256 + vdims] = cpu(ly["v"]).reshape(-1, H)
        conv = torch.zeros(C, 1, 4, dtype=bf)
        cqk = cpu(ly["conv_qk"]).reshape(2, nk * kl, 4)
        conv[qrows, 0], conv[nk * 256 + qrows, 0] = cqk[0], cqk[1]
        conv[2 * nk * 256 + vdims, 0] = cpu(ly["conv_v"]).reshape(-1, 4)
        z = torch.zeros(d.nv * 128, H, dtype=bf)
        z[vdims] = cpu(ly["z"]).reshape(-1, H)
        ba = {k: torch.zeros(d.nv, H, dtype=bf) for k in ("b", "a")}
        for k in ba:
            ba[k][vh] = cpu(ly[k]).reshape(-1, H)
        out = torch.zeros(H, d.nv * 128, dtype=bf)
        out[:, vdims] = cpu(ly["out"]).reshape(H, -1)
        sd.update({ga + "in_proj_qkv.weight": qkv, ga + "in_proj_z.weight": z,
                   ga + "in_proj_b.weight": ba["b"], ga + "in_proj_a.weight": ba["a"],
                   ga + "out_proj.weight": out, ga + "conv1d.weight": conv,
                   ga + "A_log": cpu(ly["A_log"]).to(bf), ga + "dt_bias": cpu(ly["dt_bias"]).to(bf),
                   ga + "norm.weight": cpu(ly["norm"]).to(bf),
                   p + "input_layernorm.weight": cpu(ly["ln_in"]).to(bf),
                   p + "post_attention_layernorm.weight": cpu(ly["ln_post"]).to(bf),
                   p + "mlp.gate_proj.weight": cpu(ly["gate"]), p + "mlp.up_proj.weight": cpu(ly["up"]),
                   p + "mlp.down_proj.weight": cpu(ly["down"])})
    sd["model.embed_tokens.weight"] = cpu(dm.embed)
    sd["model.norm.weight"] = cpu(dm.norm).to(bf)
    missing, unexpected = m.load_state_dict(sd, strict=False, assign=True)
    assert not unexpected and set(missing) <= {"lm_head.weight"}, (missing[:4], unexpected[:4])
    m.tie_weights()
    from transformers.models.qwen3_5 import modeling_qwen3_5 as q
    m.model.rotary_emb = q.Qwen3_5TextRotaryEmbedding(config=cfg)
    m = m.to(dtype=bf).eval()
    for layer in m.model.layers:
        layer.linear_attn.norm.variance_epsilon = sp.gated_eps
    return m


def has_dense_order(model) -> bool:
    """Whether any matrix of a SparseModel is marked dense (only the dense path sums those)."""
    cs = [model.embed] + [getattr(ly, n) for ly in model.layers for n in (
        "in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj", "gate_proj", "up_proj",
        "down_proj")]
    return any(getattr(c, "blocks", 0) for c in cs)
