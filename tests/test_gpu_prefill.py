"""Parity of the HIP verified-mode forward (the prefill: Fast.forward / layer / head_argmax /
decode) with the oracle, on an MI355X, through the C ABI.

Each position sees exactly the stock decode step, so a prefill over T positions must leave what
T forced decode steps of the oracle leave: every position's prediction, every layer's residual
at every position, the conv windows and the recurrent states, compared bit for bit. At full
config-3 size the prefill is checked against the decode kernel driven by the same tokens (two
independent GPU paths of the same semantics).
"""

import numpy as np
import pytest
import torch

from linuxformer_amd import fast, mega, mk_build, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cuda():
    assert torch.cuda.is_available(), "the gpu tests need an MI355X"
    mk_build.load()  # the native library, never a fallback
    return torch.device("cuda", 0)


def _specs():
    return {"small": synth.small(), "small_fp32": synth.small(dtype="fp32", seed=3),
            "c1": synth.config1(), "c2": synth.config2(), "c3": synth.config3(),
            "c5": synth.config5()}


_MODELS = {}


def model(name):
    if name not in _MODELS:
        spec = _specs()[name]
        m = synth.build(spec)
        conv0, rec0 = synth.init_state(m)
        _MODELS[name] = (spec, m, conv0, rec0, fast.Fast(m))
    return _MODELS[name]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def check(name, tokens, conv0=None, per_layer=True):
    """The prefill over tokens from the model's initial state against the oracle's forced
    decode of the same tokens, bit for bit."""
    from oracle import oracle as ox

    spec, m, c0, r0, f = model(name)
    conv0 = c0 if conv0 is None else conv0
    tokens = [int(x) for x in tokens]
    T, d = len(tokens), m.dims
    print(f"[gpu-test] prefill {name}: T={T} per_layer={per_layer}", flush=True)
    cache = fast.StateCache(conv0, r0, d.dtype, "cuda")
    pf = f.prefill("cuda")
    if per_layer:
        pf.embed(tokens)
        traces = []
        for L in range(d.n_layers):
            pf.layers(T, cache, L, L + 1)
            traces.append(pf.from_tiles(T).float().cpu().numpy())
        preds = pf.head(T).cpu().numpy()
    else:
        preds = f.verify(tokens, cache).cpu().numpy()
    om = ox.OracleModel(m)
    c, r = conv0.copy(), r0.copy()
    po, _, tro = om.decode(c, r, tokens, T, trace=per_layer)
    if per_layer:
        for L in range(d.n_layers):
            same = bits(traces[L]) == bits(tro[:, L])
            assert same.all(), (L, np.argwhere(~same)[:5].tolist())
    assert preds.tolist() == po.tolist()
    assert (bits(cache.conv_numpy()) == bits(c)).all()
    assert (bits(cache.rec_numpy()) == bits(r)).all()
    return preds


def _toks(name, T, seed=0):
    spec = _specs()[name]
    return synth.tokens(spec, T, seed)


def test_prefill_small(cuda):
    check("small", _toks("small", 37))


def test_prefill_small_fp32(cuda):
    check("small_fp32", _toks("small_fp32", 30))


def test_prefill_config1(cuda):
    """Benchmark config 1's layer (fp32): 256 positions, a quarter of them gated."""
    check("c1", _toks("c1", 256))


def test_prefill_config2(cuda):
    """The 37-layer bf16 stack from its N(0,1) state: 48 positions, every layer's residual."""
    check("c2", _toks("c2", 48))


def test_prefill_config5(cuda):
    """Half of the layer-steps gated: 16 positions."""
    check("c5", _toks("c5", 16))


def test_prefill_short_from_live_windows(cuda):
    """1, 2, 3 and 5 positions from nonzero windows on every channel: the first positions'
    convs read the windows the cache held, and short calls shift them."""
    spec, m, c0, r0, f = model("small")
    rng = np.random.default_rng(11)
    conv0 = synth._round(rng.standard_normal(c0.shape).astype(np.float32), "bf16")
    for T in (1, 2, 3, 5):
        check("small", _toks("small", T, seed=T), conv0=conv0)


def test_prefill_calls_continue(cuda):
    """Two calls (10, then 27 positions) leave the states of one call of 37 and the same
    predictions."""
    from oracle import oracle as ox

    spec, m, c0, r0, f = model("small")
    toks = [int(x) for x in _toks("small", 37, seed=4)]
    cache = fast.StateCache(c0, r0, m.dims.dtype, "cuda")
    p1 = f.verify(toks[:10], cache).cpu().numpy().tolist()
    p2 = f.verify(toks[10:], cache).cpu().numpy().tolist()
    c, r = c0.copy(), r0.copy()
    po, _, _ = ox.OracleModel(m).decode(c, r, toks, 37)
    assert p1 + p2 == po.tolist()
    assert (bits(cache.conv_numpy()) == bits(c)).all()
    assert (bits(cache.rec_numpy()) == bits(r)).all()


def test_fast_api_forward_decode_head(cuda):
    """The reference's Fast API on residual tensors: forward (1, T, hidden), decode (1, 1,
    hidden), head_argmax (int64) agree with the oracle's layer steps and head."""
    from oracle import oracle as ox

    spec, m, c0, r0, f = model("small")
    d = m.dims
    toks = [int(x) for x in _toks("small", 9, seed=2)]
    emb = m.embed.dense()[toks]  # exact in bf16
    h = torch.from_numpy(emb).to("cuda", torch.bfloat16)[None]
    cache = fast.StateCache(c0, r0, d.dtype, "cuda")
    assert f.to("cuda") is f  # (the tables on the device; the calls below use them)
    out = f.forward(h[:, :8], cache)
    out1 = f.decode(h[:, 8:], cache)
    hs = torch.cat([out, out1], 1)[0]
    preds = f.head_argmax(hs)
    om = ox.OracleModel(m)
    c, r = c0.copy(), r0.copy()
    want = np.zeros((9, d.hidden), np.float32)
    for i in range(9):
        x = emb[i].astype(np.float32).copy()
        for L in range(d.n_layers):
            om.layer_step(L, x, c[L], r[L])
        want[i] = x
    assert (bits(hs.float().cpu().numpy()) == bits(want)).all()
    assert preds.dtype == torch.int64
    assert preds.cpu().numpy().tolist() == om.head(want).tolist()
    assert (bits(cache.rec_numpy()) == bits(r)).all()


def test_prefill_token_out_of_range(cuda):
    spec, m, c0, r0, f = model("small")
    cache = fast.StateCache(c0, r0, m.dims.dtype, "cuda")
    with pytest.raises(ValueError):
        f.verify([0, m.dims.vocab], cache)


def test_prefill_device_tokens_and_caches(cuda):
    """Tokens already on the device give the host path's predictions and states; a call on
    another cache and size in between (the parameter blocks are kept per buffers and state
    arrays) changes nothing; a device token out of range sets the error word, with no raise."""
    spec, m, c0, r0, f = model("small")
    toks = np.asarray(_toks("small", 40), np.int32)
    print("[gpu-test] prefill device tokens", flush=True)
    ca = fast.StateCache(c0, r0, m.dims.dtype, "cuda")
    want = f.verify([int(x) for x in toks], ca).cpu().numpy()
    want_conv, want_rec = ca.conv_numpy(), ca.rec_numpy()
    pf = f.prefill("cuda")
    td = torch.from_numpy(toks).to("cuda")
    cb = fast.StateCache(c0, r0, m.dims.dtype, "cuda")
    pb = pf.verify(td, cb).cpu().numpy()
    cc = fast.StateCache(c0, r0, m.dims.dtype, "cuda")
    pf.verify([int(x) for x in toks[:7]], ca)
    pc = pf.verify(td, cc).cpu().numpy()
    assert pb.tolist() == want.tolist() and pc.tolist() == want.tolist()
    for cx in (cb, cc):
        assert (bits(cx.conv_numpy()) == bits(want_conv)).all()
        assert (bits(cx.rec_numpy()) == bits(want_rec)).all()
    assert int(pf.err.item()) == 0
    bad = torch.tensor([0, m.dims.vocab], dtype=torch.int32, device="cuda")
    pf.verify(bad, fast.StateCache(c0, r0, m.dims.dtype, "cuda"))
    assert int(pf.err.item()) != 0
    # a good call after the bad one: the error word starts from zero again, the results are whole
    cd = fast.StateCache(c0, r0, m.dims.dtype, "cuda")
    pd = pf.verify(td, cd).cpu().numpy()
    assert int(pf.err.item()) == 0
    assert pd.tolist() == want.tolist()
    assert (bits(cd.rec_numpy()) == bits(want_rec)).all()


def test_config3_full_matches_decode_kernel(cuda):
    """Benchmark config 3 at full size: 65,536 uniform tokens through the 37-layer stack. The
    prefill's predictions and final states equal those of the decode kernel forced through
    the same tokens (65,536 steps), bit for bit."""
    spec, m, c0, r0, f = model("c3")
    toks = _toks("c3", 65_536)
    print("[gpu-test] c3 prefill 65,536", flush=True)
    cache = fast.StateCache(c0, r0, "bf16", "cuda")
    preds = f.verify(toks, cache).cpu().numpy()
    conv_p, rec_p = cache.conv_numpy(), cache.rec_numpy()
    del cache
    print("[gpu-test] c3 decode kernel 65,536", flush=True)
    cache2 = fast.StateCache(c0, r0, "bf16", "cuda")
    mg = mega.Mega(f, m, cache2, 0)
    want = mg.run(toks.tolist(), len(toks))
    assert preds.tolist() == want
    assert (bits(cache2.conv_numpy()) == bits(conv_p)).all()
    assert (bits(cache2.rec_numpy()) == bits(rec_p)).all()


def test_verify_matches_stock_T_gt_1_forward(cuda):
    """Verified mode against the stock forward it names, transformers' T > 1 path (one forward
    over all 100 tokens: causal_conv1d_fn and torch_chunk_gated_delta_rule from the cached
    state; the committed fixture tests/golden/small_bf16_pf100.npz): the same argmax at every
    position, and final recurrent states within 1e-6 of their largest magnitude (the chunked
    and recurrent forms round apart by ~3e-7 there)."""
    from golden.make_golden import model_of

    g = dict(np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                                "small_bf16_pf100.npz")))
    m, conv0, rec0, _ = model_of(str(g["base"]))
    print("[gpu-test] verify vs stock T>1: small_bf16_pf100", flush=True)
    cache = fast.StateCache(conv0, rec0, m.dims.dtype, "cuda")
    got = fast.Fast(m).verify([int(t) for t in g["tokens"]], cache).cpu().numpy()
    assert got.tolist() == g["preds"].tolist()
    r = cache.rec_numpy()
    assert np.abs(r.reshape(-1)[g["rec_idx"]] - g["rec_sample"]).max() <= 1e-6 * float(g["rec_max"])


def test_config3_shape_matches_stock_T_gt_1_forward(cuda):
    """Verified mode at config 3's full shape (37 layers, hidden 3,572, the c3 stack and its
    N(0,1) state) over the first 64 tokens of bench.py's first call, layer by layer, against the
    stock T > 1 forward (transformers' own modules; tests/golden/c3_pf64.npz)."""
    from c3_check import check_against_stock_c3, c3_stock_fixture

    g = c3_stock_fixture()
    spec, m, c0, r0, f = model("c3")
    tokens = [int(x) for x in g["tokens"]]
    T = len(tokens)
    print(f"[gpu-test] c3 shape vs stock T>1: T={T}", flush=True)
    cache = fast.StateCache(c0, r0, m.dims.dtype, "cuda")
    pf = f.prefill("cuda")
    pf.embed(tokens)
    traces = []
    for L in range(m.dims.n_layers):
        pf.layers(T, cache, L, L + 1)
        traces.append(pf.from_tiles(T).float().cpu().numpy())
    preds = pf.head(T).cpu().numpy()
    check_against_stock_c3(traces, preds, cache.conv_numpy(), cache.rec_numpy(), g)
