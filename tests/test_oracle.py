"""The oracle (oracle/lx_oracle.c) pinned: its elementary functions against float64 and against
torch's own bf16 kernels, its sum orders against constructed cancellations, and its decode
against the stock forward's golden vectors (tests/golden, written from transformers' Qwen3_5
layers by tests/golden/make_golden.py)."""

import os

import numpy as np
import pytest
import torch

from linuxformer_amd import synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bf16_all():
    return (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_exp_log1p_correctly_rounded(oracle_lib):
    """exp and log1p against float64 rounded once to float32 (the double reference is 2^29
    times finer than a float ulp, so a mismatch would mean a misrounded result)."""
    ox = oracle_lib
    rng = np.random.default_rng(0)
    x = rng.uniform(-103.0, 88.7, 1 << 20).astype(np.float32)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    assert (bits(ox.elem("exp", x)) != bits(ref)).sum() == 0
    y = np.exp(rng.uniform(np.log(1e-30), np.log(1e9), 1 << 20)).astype(np.float32)
    ref = np.log1p(y.astype(np.float64)).astype(np.float32)
    assert (bits(ox.elem("log1p", y)) != bits(ref)).sum() == 0


def test_special_values(oracle_lib):
    ox = oracle_lib
    x = np.array([0.0, -0.0, 1.0, 88.72, 89.5, -103.9, -104.0, -200.0, np.inf, -np.inf], np.float32)
    e = ox.elem("exp", x)
    assert e[0] == 1.0 and e[1] == 1.0 and e[2] == np.float32(np.e)
    assert np.isfinite(e[3]) and e[4] == np.inf and e[5] > 0 and e[6] == 0 and e[7] == 0
    assert e[8] == np.inf and e[9] == 0
    sp = ox.elem("softplus", np.array([21.0, 20.0, -200.0, 0.0], np.float32))
    assert sp[0] == 21.0 and sp[1] == np.float32(np.log1p(np.exp(20.0))) and sp[2] == 0.0
    assert sp[3] == np.float32(np.log(2.0))
    si = ox.elem("silu", np.array([0.0, -0.0, -200.0, 100.0], np.float32))
    assert bits(si[:2]).tolist() == [0, 0x80000000] and si[2] == 0.0 and si[3] == 100.0
    assert ox.elem("rsqrt", np.array([4.0], np.float32))[0] == 0.5
    b = ox.elem("bf16", np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, np.nan], np.float32))
    assert b[0] == 1.0 and b[1] == 1.0 + 2 ** -6 and bits(b[2:]).tolist() == [0x7FC00000]


def test_bf16_elementwise_equals_torch(oracle_lib):
    """On every bf16 input, the oracle's silu, sigmoid, exp and rsqrt rounded to bf16 equal
    torch's bf16 kernels (the vectorised path the chip's 128-head tensors take)."""
    ox = oracle_lib
    x = bf16_all()
    fin = np.isfinite(x)
    xb = torch.from_numpy(x.copy()).to(torch.bfloat16)
    for name, fn in (("silu", torch.nn.functional.silu), ("sigmoid", torch.sigmoid),
                     ("exp", torch.exp), ("rsqrt", torch.rsqrt)):
        mine = ox.elem("bf16", ox.elem(name, x))
        ref = fn(xb).float().numpy()
        same = (bits(mine) == bits(ref)) | (np.isnan(mine) & np.isnan(ref))
        assert (~same & fin).sum() == 0, name


def test_hidden_sum_order(oracle_lib):
    """The 512-lane tree: lane l adds x[4l..4l+3] then x[2048+4l..2048+4l+3] in order; lanes
    pair at offsets 32..1 within a group of 64, then the 8 group totals at 4, 2, 1. Big values
    placed where the documented pairing cancels them first keep the small terms; any other
    order loses them."""
    ox = oracle_lib
    x = np.zeros(3572, np.float32)
    x[0], x[4 * 32] = 1e8, -1e8            # lanes 0 and 32: paired at offset 32 in group 0
    x[4] = 1.0                              # lane 1 meets the pair's exact 0 later
    x[256 * 3], x[256 * 7] = 3e8, -3e8      # groups 3 and 7 (their lane 0) pair at offset 4
    x[2048 + 256 * 5 + 28] = 0.5            # lane 327 (group 5), second part
    assert ox.sum_h(x) == 1.5
    y = np.zeros(3572, np.float32)
    y[20], y[21] = 1e8, 1.0                 # lane 5, in order: 1e8 + 1 rounds to 1e8
    y[2048 + 20] = -1e8                     # lane 5's fifth term
    assert ox.sum_h(y) == 0.0
    z = np.arange(1, 3573, dtype=np.float32)
    assert ox.sum_h(z) == float(z.astype(np.float64).sum())
    h = np.zeros(256, np.float32)
    h[0], h[32], h[1], h[3] = 1e8, -1e8, 1.0, 0.25  # lanes 0 and 32 cancel first
    assert ox.sum_64(h) == 1.25
    h[64] = 1.0  # lane 0 again, after its 1e8: absorbed
    assert ox.sum_64(h) == 1.25


def _load(name):
    return dict(np.load(os.path.join(GOLD, name + ".npz")))


@pytest.mark.parametrize("name,exact,tol", [
    ("c1_256", True, 0.0),           # the chip's shape, all 256 steps: bit for bit
    ("small_fp32_32", False, 1e-6),  # dense-ish rows, 8 value heads: per-layer 1e-6 relative
    ("tiny_fp32_8", False, 1e-5),    # dense layers: per-step 1e-6 errors carried 8 steps in the state
])
def test_oracle_matches_stock_fp32(oracle_lib, name, exact, tol):
    from golden.make_golden import model_of, sha, sha_state

    g = _load(name)
    m, conv0, rec0, start = model_of(name)
    om = oracle_lib.OracleModel(m)
    c, r = conv0.copy(), rec0.copy()
    preds, _, tr = om.decode(c, r, [int(g["start"])], int(g["n"]), trace=True)
    assert preds.tolist() == g["preds"].tolist()
    if exact:
        assert sha(tr) == str(g["trace_sha"])
        assert sha(c) == str(g["conv_sha"]) and sha_state(r) == str(g["rec_sha"])
    else:
        ref = g["trace"]
        rel = np.abs(tr - ref).max(-1) / np.maximum(np.abs(ref).max(-1), 1e-30)
        assert rel.max() <= tol, rel.max()
        rs = r.reshape(-1)[g["rec_idx"]]
        assert np.abs(rs - g["rec_sample"]).max() <= tol * max(1.0, np.abs(g["rec_sample"]).max())


def _decode_c2s(ox, flush: bool):
    from golden.make_golden import model_of, sha, sha_state

    g = _load("c2s_bf16_64")
    m, conv0, rec0, start = model_of("c2s_bf16_64")
    om = ox.OracleModel(m)
    ox.set_flush(flush)
    try:
        c, r = conv0.copy(), rec0.copy()
        preds, _, tr = om.decode(c, r, [int(g["start"])], int(g["n"]), trace=True)
    finally:
        ox.set_flush(False)
    return g, preds, tr, sha(c), sha_state(r), sha


def test_oracle_flush_mode_is_the_stock_bf16_forward(oracle_lib):
    """Config 2's layer shape in bf16 (3 layers, N(0,1) state, a gate open every step), 64
    greedy steps: with oneDNN's bf16 GEMM flushing modelled (denormal inputs and sums of the
    matrix products to zero, as AMX does on the host that wrote the fixture), the oracle IS the
    stock forward bit for bit: the stream, every layer's residual at every step and the final
    conv windows; the final recurrent states element for element (x == y, the reference's own
    state comparison: the sign of a zero state entry is not compared). Every rounding point of
    the bf16 layer is pinned by it (a dropped or added D() anywhere changes residual bits within a
    few steps)."""
    g, preds, tr, csha, rsha, sha = _decode_c2s(oracle_lib, True)
    assert preds.tolist() == g["preds"].tolist()
    assert sha(tr) == str(g["trace_sha"])
    assert csha == str(g["conv_sha"]) and rsha == str(g["rec_sha"])


def test_oracle_contract_vs_stock_bf16_chip_shape(oracle_lib):
    """The contract (IEEE binary32, denormals kept; what the kernels compute) against the same
    stock forward: the same stream and bit-identical final conv windows and recurrent states; the
    residual traces differ in exactly the elements the fixture counted against the stock trace
    (672 of 685,824), all of magnitude below 2^-100: values that the stock host's flushing set to
    zero, and their images through the next norms. Per-layer relative error 0."""
    g, preds, tr, csha, rsha, _ = _decode_c2s(oracle_lib, False)
    _, _, tr_f, _, _, _ = _decode_c2s(oracle_lib, True)  # == the stock trace (test above)
    assert preds.tolist() == g["preds"].tolist()
    assert csha == str(g["conv_sha"]) and rsha == str(g["rec_sha"])
    diff = bits(tr) != bits(tr_f)
    assert int(diff.sum()) == int(g["contract_diff"]) == 672
    big = np.maximum(np.abs(tr[diff]), np.abs(tr_f[diff]))
    assert big.max() < 2.0 ** -100
    rel = np.abs(tr - tr_f).max(-1) / np.abs(tr_f).max(-1)
    assert rel.max() <= 1e-30


def test_flush_mode_changes_only_tiny_values(oracle_lib):
    """The flush mode touches only bf16 matrix products with denormal inputs or sums: on a row
    whose inputs are all normal it is the contract's sum, and a denormal input is dropped."""
    ox = oracle_lib
    x = np.array([1.5, -2.0, 1e-39, 0.75], np.float32)
    w = np.array([1.0, 0.5, 2.0, -2.0], np.float32)
    m = synth.small()
    om = ox.OracleModel(synth.build(m))  # the flag acts in bf16 models' products
    del om
    assert ox.row_dot(x, w, dense=False) == np.float32(1.5 - 1.0 + 2e-39 - 1.5)


@pytest.mark.parametrize("name", ["small_bf16_32", "tiny_bf16_8"])
def test_oracle_matches_stock_bf16(oracle_lib, name):
    """bf16 stacks with long dense sums: torch's summation orders (oneDNN's GEMV, ATen's
    vectorised inner sums) differ from the contract's, so single fp32 roundings can flip a bf16
    result; the stream is identical and most residual values are bit-equal."""
    from golden.make_golden import model_of

    g = _load(name)
    m, conv0, rec0, start = model_of(name)
    om = oracle_lib.OracleModel(m)
    c, r = conv0.copy(), rec0.copy()
    preds, _, tr = om.decode(c, r, [int(g["start"])], int(g["n"]), trace=True)
    assert preds.tolist() == g["preds"].tolist()
    ref = g["trace"]
    assert (tr == ref).mean() >= 0.2
    rel = np.abs(tr - ref).max(-1) / np.maximum(np.abs(ref).max(-1), 1e-30)
    assert rel.max() <= 0.03, rel.max()


def test_layer_step_matches_stock_decoder_layer(oracle_lib):
    """One fully dense decoder layer (fp32) from identical random inputs, against transformers'
    Qwen3_5DecoderLayer: the output within 5e-6 relative -- its out_proj adds 4,096 dense
    terms, which oneDNN sums in its own order (two orders spread by ~sqrt(4096) x 2^-24 =
    3.8e-6) -- and the state and conv window within 1e-6. (The sparse, chip-shaped config 1 is
    bit-identical: test_oracle_matches_stock_fp32; the delta rule alone is bit-identical:
    test_recurrent_step_bit_exact.)"""
    from oracle import stock

    torch.set_grad_enabled(False)
    m = synth.tiny_dense(seed=11, dtype="fp32")
    hf = synth.to_hf(m)
    d = m.dims
    rng = np.random.default_rng(2)
    conv0 = rng.standard_normal((d.n_layers, d.n_conv, 4)).astype(np.float32)
    rec0 = rng.standard_normal((d.n_layers, d.nv, d.kd, d.vd)).astype(np.float32)
    h = rng.standard_normal(d.hidden).astype(np.float32)
    cache = stock.make_cache(hf, conv0, rec0)
    out = hf.model.layers[0](torch.from_numpy(h)[None, None], position_embeddings=None,
                             attention_mask=None, position_ids=None, past_key_values=cache)
    out = (out[0] if isinstance(out, tuple) else out)[0, 0].numpy()
    om = oracle_lib.OracleModel(m)
    hx, c, r = h.copy(), conv0[0].copy(), rec0[0].copy()
    om.layer_step(0, hx, c, r)
    R = cache.layers[0].recurrent_states[0][0].numpy()
    Cs = cache.layers[0].conv_states[0][0].numpy()
    assert np.abs(hx - out).max() / np.abs(out).max() <= 5e-6
    assert np.abs(r - R).max() <= 1e-6 * np.abs(R).max()
    assert np.abs(c - Cs).max() <= 1e-6 * np.abs(Cs).max()


def _bf16_ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|a - b| in bf16 units in the last place of the larger magnitude (8 significant bits)."""
    m = np.maximum(np.abs(a), np.abs(b))
    e = np.floor(np.log2(np.maximum(m, np.float32(1e-38))))
    return np.abs(a.astype(np.float64) - b) / np.exp2(e - 7)


def test_dense_layer_within_one_bf16_ulp_of_stock_at_config4_widths(oracle_lib):
    """Config 4's dense order against the stock bf16 forward, one layer at config 4's full widths
    (hidden 2560, 16 key heads of 256 dims with 128 live, 2 live of 8 value heads each, SwiGLU
    9216) from identical inputs and a live state: transformers' Qwen3_5DecoderLayer on the host
    (oneDNN's bf16 GEMV order) against the oracle's dense order (64 groups, pairwise tree). Each
    dense row is the fp32 sum of the same exact bf16 products rounded once to bf16, so two
    orders can differ only where that sum lies within the orders' fp32 spread of a bf16
    rounding boundary: the residual output and the conv window agree to within one bf16 unit in
    the last place everywhere and bit for bit on at least 99.9 % of their values, and the fp32
    recurrent state bit for bit on at least 99.9 % and within 1e-6 of its largest value. (On
    this seed: the residual and the state bit-equal, one conv value of 98,304 one unit apart.)
    A mistake planted in the oracle's input (one out_proj weight dropped) is caught."""
    from oracle import stock

    torch.set_grad_enabled(False)
    dm = synth.build_dense(synth.config4_mid(), "cpu")
    sm = synth.to_sparse(dm)
    hf = synth.dense_to_hf(dm)
    conv0, rec0 = synth.dense_state(dm, seed=3)
    rng = np.random.default_rng(5)
    h = synth._round(rng.standard_normal(sm.dims.hidden).astype(np.float32) * 0.5, "bf16")
    cache = stock.make_cache(hf, conv0, rec0)
    out = hf.model.layers[0](torch.from_numpy(h)[None, None].to(torch.bfloat16),
                             position_embeddings=None, attention_mask=None, position_ids=None,
                             past_key_values=cache)
    out = (out[0] if isinstance(out, tuple) else out)[0, 0].float().numpy()
    R = cache.layers[0].recurrent_states[0][0].float().numpy()
    Cs = cache.layers[0].conv_states[0][0].float().numpy()
    del hf, cache, dm

    def step(model):
        hx, c, r = h.copy(), conv0[0].copy(), rec0[0].copy()
        oracle_lib.OracleModel(model).layer_step(0, hx, c, r)
        return hx, c, r

    def agrees(hx, c, r):
        return (_bf16_ulps(hx, out).max() <= 1.0 and (hx == out).mean() >= 0.999 and
                _bf16_ulps(c, Cs).max() <= 1.0 and (c == Cs).mean() >= 0.999 and
                (r == R).mean() >= 0.999 and np.abs(r - R).max() <= 1e-6 * np.abs(R).max())

    hx, c, r = step(sm)
    assert agrees(hx, c, r), (_bf16_ulps(hx, out).max(), (hx == out).mean(),
                              _bf16_ulps(c, Cs).max(), (c == Cs).mean(), (r == R).mean())
    op = sm.layers[0].out_proj
    k = int(np.argmax(np.abs(op.vals)))
    v = op.vals[k]
    op.vals[k] = 0.0
    try:
        assert not agrees(*step(sm))
    finally:
        op.vals[k] = v


def _rec_inputs(dtype, dense, chip, seed):
    rng = np.random.default_rng(seed)
    nk, nv = 16, 128
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32

    def rnd(shape, p):
        if chip:  # dyadic values, as the chip's circuit values are
            x = rng.choice(synth.VALS, shape).astype(np.float32)
        else:
            x = rng.standard_normal(shape).astype(np.float32)
        x[rng.random(shape) > p] = 0
        return torch.from_numpy(x).to(tdt).float().numpy()

    qv = rnd((nk, 256), 1.0 if dense else 0.02)
    kv = rnd((nk, 256), 1.0 if dense else 0.01)
    qv[3] = 0
    kv[3] = 0  # an idle head
    vv = torch.from_numpy(rng.standard_normal((nv, 128)).astype(np.float32)).to(tdt).float().numpy()
    beta = torch.from_numpy(rng.random(nv).astype(np.float32)).to(tdt).float().numpy()
    if chip:  # decays exp(g) in {1, 1/2, 0}
        g = rng.choice(np.array([0.0, -np.log(2.0), -200.0], np.float32), nv).astype(np.float32)
    else:
        g = np.where(rng.random(nv) < 0.3, -rng.random(nv), 0.0).astype(np.float32)
    S0 = rng.standard_normal((nv, 256, 128)).astype(np.float32)
    return qv, kv, vv, g, beta, S0, tdt


def _stock_rec(qv, kv, vv, g, beta, S0, tdt):
    from transformers.models.qwen3_5 import modeling_qwen3_5 as q

    R = vv.shape[0] // qv.shape[0]
    T = lambda a: torch.from_numpy(a).to(tdt)  # noqa: E731
    o, S = q.torch_recurrent_gated_delta_rule(
        T(qv)[None, None].repeat_interleave(R, dim=2), T(kv)[None, None].repeat_interleave(R, dim=2),
        T(vv)[None, None], g=torch.from_numpy(g)[None, None], beta=T(beta)[None, None],
        initial_state=torch.from_numpy(S0.copy())[None], output_final_state=True,
        use_qk_l2norm_in_kernel=True)
    return o[0, 0].float().numpy(), S[0].numpy()


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("dense", [False, True])
def test_recurrent_step_bit_exact(oracle_lib, dtype, dense):
    """The delta rule (l2norm in the model dtype, decay, kv, delta, write, output) equals
    transformers' torch_recurrent_gated_delta_rule bit for bit at the chip's 16 key x 8 value
    heads, in the chip's regime (dyadic query/key values, decays exp(g) in {1, 1/2, 0}) with
    random state, values and betas; sparse (as the chip's) or dense queries and keys."""
    torch.set_grad_enabled(False)
    qv, kv, vv, g, beta, S0, tdt = _rec_inputs(dtype, dense, True, 7 + dense)
    o_t, S_t = _stock_rec(qv, kv, vv, g, beta, S0, tdt)
    S = S0.copy()
    o = oracle_lib.rec_step(qv, kv, vv, g, beta, S, dtype == "bf16")
    assert (o == o_t).all()
    assert (S == S_t).all()


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_recurrent_step_generic_inputs(oracle_lib, dtype):
    """Random (non-dyadic) inputs: torch's fp32 l2norm sums 256 terms in its vector-width order
    and its Sleef exp is 1 ulp off on ~1 % of decays, so fp32 results agree within 1e-6
    relative; in bf16 the outputs are bit-identical and the state differs only on heads whose
    exp(g) torch rounds differently."""
    torch.set_grad_enabled(False)
    qv, kv, vv, g, beta, S0, tdt = _rec_inputs(dtype, True, False, 21)
    o_t, S_t = _stock_rec(qv, kv, vv, g, beta, S0, tdt)
    S = S0.copy()
    o = oracle_lib.rec_step(qv, kv, vv, g, beta, S, dtype == "bf16")
    same_e = oracle_lib.elem("exp", g) == torch.exp(torch.from_numpy(g)).numpy()
    assert np.abs(o - o_t).max() <= 1e-6 * np.abs(o_t).max() + (0 if dtype == "fp32" else 1e-2)
    assert np.abs(S - S_t).max() <= 1e-6 * np.abs(S_t).max()
    if dtype == "bf16":
        assert (S[same_e] == S_t[same_e]).all()


def test_dense_order_sums_exact_integers(oracle_lib):
    """Small integers: every order gives the exact sum, so a dropped, doubled or misplaced term
    (a wrong group bound) shows."""
    ox = oracle_lib
    rng = np.random.default_rng(0)
    for n in (64, 2560, 9216):
        x = rng.integers(-8, 9, n).astype(np.float32)
        w = rng.integers(-8, 9, n).astype(np.float32)
        exact = float(np.dot(x.astype(np.int64), w.astype(np.int64)))
        assert float(ox.row_dot(x, w, dense=True)) == exact
        assert float(ox.row_dot(x, w, dense=False)) == exact


def test_dense_order_is_the_group_tree(oracle_lib):
    """Terms 1, 2^24, 1 in groups 0, 1 and 32 of a 64-entry row: the tree adds group 32 to group
    0 first (1 + 1 = 2), then group 1 last: 2 + 2^24 = 16777218, exact; in order, 1 + 2^24
    rounds to 2^24 and so does + 1. Both values follow from the definitions by hand."""
    ox = oracle_lib
    x = np.zeros(64, np.float32)
    w = np.ones(64, np.float32)
    x[0], x[1], x[32] = 1.0, 2.0 ** 24, 1.0
    assert float(ox.row_dot(x, w, dense=True)) == 16777218.0
    assert float(ox.row_dot(x, w, dense=False)) == 16777216.0


def _chunk_fixture():
    g = _load("chunk_fp32_100")
    pad = lambda a, n: np.concatenate([a, np.zeros((a.shape[0], n - a.shape[1]), np.float32)], 1)
    q, k = pad(g["q"], 256), pad(g["k"], 256)
    S0 = np.zeros((256, 128), np.float32)
    S0[:128] = g["S0"]
    return g, q, k, S0


def test_chunk_form_matches_stock_chunk(oracle_lib):
    """The oracle's chunked delta rule against transformers' torch_chunk_gated_delta_rule (chunk
    64, float32) on one value head over 100 positions (a full chunk and a padded one): outputs and
    final state within 1e-6 of the largest magnitude (the matrix products' orders are MKL's)."""
    g, q, k, S0 = _chunk_fixture()
    S = S0.copy()
    o = oracle_lib.chunk_gdr(q, k, g["v"], g["g"], g["beta"], S, 64)
    assert np.abs(o - g["o"]).max() <= 1e-6 * np.abs(g["o"]).max()
    assert np.abs(S[:128] - g["S"]).max() <= 1e-6 * np.abs(g["S"]).max()
    assert not S[128:].any()


def test_chunk_form_planted_mistakes_fail(oracle_lib):
    """What the fixture comparison catches: a dropped decay (g = 0), a dropped beta, and the
    recurrent form itself differ from the stock chunk output by far more than its tolerance."""
    g, q, k, S0 = _chunk_fixture()
    ref = g["o"]
    tol = 1e-6 * np.abs(ref).max()
    o1 = oracle_lib.chunk_gdr(q, k, g["v"], np.zeros_like(g["g"]), g["beta"], S0.copy(), 64)
    o2 = oracle_lib.chunk_gdr(q, k, g["v"], g["g"], np.ones_like(g["beta"]), S0.copy(), 64)
    assert np.abs(o1 - ref).max() > 1e3 * tol and np.abs(o2 - ref).max() > 1e3 * tol


@pytest.mark.parametrize("C", [64, 16])
def test_chunk_form_exact_regime_equals_recurrent(oracle_lib, C):
    """In the chip's exact regime (one-hot keys and queries, beta in {0, 1}, no decay, dyadic
    values) every product and sum is exact, so the chunked form (any chunk size) equals the
    delta rule's recurrence S <- S + k (x) (v - S^T k) beta, o = S^T q / 16, run position by
    position, bit for bit (outputs and final state)."""
    from golden.make_golden import chunk_inputs

    q, k, v, g, beta, S0 = chunk_inputs(150, 4, exact=True)
    S = S0.copy()
    o = oracle_lib.chunk_gdr(q, k, v, g, beta, S, C)
    Sr = S0.astype(np.float64)
    orr = np.zeros(o.shape, np.float64)
    for t in range(len(q)):
        Sr = Sr * np.exp(float(g[t]))
        Sr = Sr + np.outer(k[t], (v[t] - Sr.T @ k[t]) * beta[t])
        orr[t] = Sr.T @ (q[t] / 16.0)
    assert (o.astype(np.float64) == orr).all()
    assert (S.astype(np.float64) == Sr).all()
    assert np.abs(orr).max() > 0 and (beta == 1).any() and (beta == 0).any()


@pytest.mark.parametrize("name,tol", [("small_fp32_pf100", 1e-6), ("small_bf16_pf100", 0.0)])
def test_oracle_prefill_chunked_matches_stock_T_gt_1(oracle_lib, name, tol):
    """The oracle's restatement of the stock T > 1 forward (ox_prefill_chunked: the decode step's
    arithmetic per position, the delta rule as torch_chunk_gated_delta_rule per value head)
    against transformers' own forward over the same 100 tokens at once: the same argmax at every
    position; every layer's output within tol of its row's largest magnitude (fp32: 1e-6; the
    bf16 stack: bit for bit); final recurrent states within 1e-6 of their largest magnitude; the
    final conv windows (the last projections) within 2e-6 of each window's largest magnitude in
    fp32 (oneDNN's GEMM sums in its own order), and in bf16 bit for bit except values below
    2^-40 (2 of 24,576: the host's flushing of denormal products)."""
    from golden.make_golden import model_of

    g = _load(name)
    m, conv0, rec0, _ = model_of(str(g["base"]))
    om = oracle_lib.OracleModel(m)
    c, r = conv0.copy(), rec0.copy()
    preds, _, tr = om.prefill_chunked(c, r, g["tokens"], trace=True)
    assert preds.tolist() == g["preds"].tolist()
    ref = g["trace"]
    rel = np.abs(tr - ref).max(-1) / np.maximum(np.abs(ref).max(-1), 1e-30)
    assert rel.max() <= tol, rel.max()
    assert np.abs(r.reshape(-1)[g["rec_idx"]] - g["rec_sample"]).max() <= 1e-6 * float(g["rec_max"])
    cr = g["conv"]
    if tol:
        crel = np.abs(c - cr).max(-1) / np.maximum(np.abs(cr).max(-1), 1e-30)
        assert crel.max() <= 2e-6, crel.max()
    else:
        diff = bits(c) != bits(cr)
        assert diff.sum() <= 4
        assert np.maximum(np.abs(c[diff]), np.abs(cr[diff])).max(initial=0.0) < 2.0 ** -40


def test_oracle_prefill_chunked_differs_from_forced_decode(oracle_lib):
    """The two forms are different restatements: on the fp32 stack the chunked prefill's final
    states differ from those of the same tokens as forced decode steps (by rounding only)."""
    from golden.make_golden import model_of

    g = _load("small_fp32_pf100")
    m, conv0, rec0, _ = model_of(str(g["base"]))
    om = oracle_lib.OracleModel(m)
    c1, r1 = conv0.copy(), rec0.copy()
    om.prefill_chunked(c1, r1, g["tokens"])
    c2, r2 = conv0.copy(), rec0.copy()
    om.decode(c2, r2, g["tokens"], len(g["tokens"]))
    d = np.abs(r1 - r2).max() / np.abs(r2).max()
    assert 0 < d < 1e-5


def test_decode_form_within_stock_T_gt_1_at_config3_shape(oracle_lib):
    """The oracle's decode form (what the verified-mode kernels compute, bit for bit) against
    the stock T > 1 forward at config 3's full shape over 64 tokens (tests/golden/c3_pf64.npz):
    the bounds the GPU test applies to the kernel (test_gpu_prefill.py) hold here; a decay left
    out of one layer (its dt_bias moved) breaks them."""
    import c3_check as gpf

    ox = oracle_lib
    g = gpf.c3_stock_fixture()
    spec = synth.config3()
    m = synth.build(spec)
    conv0, rec0 = synth.init_state(m)
    om = ox.OracleModel(m)
    c, r = conv0.copy(), rec0.copy()
    toks = [int(x) for x in g["tokens"]]
    preds, _, tr = om.decode(c, r, toks, len(toks), trace=True)
    gpf.check_against_stock_c3([tr[:, L] for L in range(m.dims.n_layers)], preds, c, r, g)
    # a planted mistake: the recurrent states left undecayed where a decay acts
    m.layers[5].dt_bias[:] = 0.0
    om = ox.OracleModel(m)
    c, r = conv0.copy(), rec0.copy()
    preds, _, tr = om.decode(c, r, toks, len(toks), trace=True)
    with pytest.raises(AssertionError):
        gpf.check_against_stock_c3([tr[:, L] for L in range(m.dims.n_layers)], preds, c, r, g)
