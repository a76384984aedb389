"""Parity of the HIP decode kernel with the oracle, on an MI355X, through the C ABI.

Bit-exact: predictions, each step's input, every layer's residual after every step, the conv
windows and the recurrent states (compared bit for bit). The oracle runs the same seeded inputs
on the CPU; the configs are the benchmark's (config 1, 2, 5) and a small stack of the chip's head
shapes. Full-size runs are checked by properties the decode must keep.
"""

import ctypes

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
    import dataclasses

    return {"small": synth.small(), "small_fp32": synth.small(dtype="fp32", seed=3),
            "small_hd": dataclasses.replace(synth.small(seed=11), head_dense=5),
            "small_hd_fp32": dataclasses.replace(synth.small(dtype="fp32", seed=12), head_dense=3),
            "c1": synth.config1(), "c2": synth.config2(), "c5": synth.config5()}


_MODELS = {}


def model(name):
    if name not in _MODELS:
        spec = _specs()[name]
        # (configs 2 and 5 share their layers: only the embedding's gate columns differ)
        other = {"c2": "c5", "c5": "c2"}.get(name)
        m = synth.build(spec, layers=_MODELS[other][1].layers if other in _MODELS else None)
        conv0, rec0 = synth.init_state(m)
        _MODELS[name] = (spec, m, conv0, rec0)
    return _MODELS[name]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def check(name, n, forced=None, launches=None, conv0=None, trace=True, merged=None):
    """Run the kernel and the oracle from the same state; compare everything bit for bit.
    merged (offset, via): the chip's rows at offset in a larger embedding (synth.merged), the
    kernel built through Fast(rows=...) and Mega(offset) from the coordinate model (via "coo")
    or from a transformers model of it (via "hf"); the oracle runs the chip-only model."""
    from oracle import oracle as ox

    spec, m, c0, r0 = model(name)
    conv0 = c0 if conv0 is None else conv0
    print(f"[gpu-test] {name}: n={n} forced={None if forced is None else len(forced)} "
          f"launches={launches} merged={merged}", flush=True)
    forced = [synth.start_token(spec)] if forced is None else list(forced)
    cache = fast.StateCache(conv0, r0, m.dims.dtype, "cuda")
    if merged is None:
        mg = mega.Mega(fast.Fast(m), m, cache, 0)
    else:
        off, via = merged
        mm = synth.merged(m, off)
        src = mm if via == "coo" else synth.to_hf(mm)
        f = fast.Fast(src, m.dims.n_layers, slice(off, off + m.dims.vocab))
        mg = mega.Mega(f, src, cache, off)
    d = m.dims
    tr = torch.zeros(n, d.n_layers, d.hidden, device="cuda") if trace else None
    inp = torch.zeros(n, dtype=torch.int32, device="cuda")
    preds = []
    done = 0
    for k in launches or [n]:
        f = forced[done:] if done < len(forced) else [preds[-1]]
        sub_tr = tr[done:done + k] if trace else None
        sub_in = inp[done:done + k]
        preds += mg.run(f, k, inputs=sub_in, trace=sub_tr)
        done += k
    om = ox.OracleModel(m)
    c, r = conv0.copy(), r0.copy()
    po, io, tro = om.decode(c, r, forced, n, trace=trace)
    assert preds == po.tolist()
    assert inp.cpu().numpy().tolist() == io.tolist()
    if trace:
        assert (bits(tr.cpu().numpy()) == bits(tro)).all()
    assert (bits(cache.conv_numpy()) == bits(c)).all()
    assert (bits(cache.rec_numpy()) == bits(r)).all()
    return preds


def test_device_math_matches_oracle(cuda):
    """The kernels' exp, log1p, silu, sigmoid, softplus, rsqrt and bf16 rounding equal the
    oracle's on every bf16 value and on 1M random floats per function."""
    from oracle import oracle as ox

    lib = mk_build.load()
    rng = np.random.default_rng(3)
    allb = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for fn, code in ox.ELEM.items():
        lo, hi = (0.0, 1e9) if fn in ("log1p", "rsqrt") else (-120.0, 100.0)
        x = np.concatenate([allb, rng.uniform(lo, hi, 1 << 20).astype(np.float32)])
        if fn == "bf16":  # every exponent: denormals, rounding into infinity, NaNs
            x = np.concatenate([x, rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64)
                                .astype(np.uint32).view(np.float32)])
        if fn == "log1p":
            x = np.abs(x)
        xd = torch.from_numpy(x).to(cuda)
        yd = torch.empty_like(xd)
        assert lib.lxm_t_elem(code, ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(yd.data_ptr()),
                              x.size, st) == 0
        y = yd.cpu().numpy()
        ref = ox.elem(fn, x)
        same = (bits(y) == bits(ref)) | (np.isnan(y) & np.isnan(ref))
        assert same.all(), (fn, int((~same).sum()))


def test_device_silu_bf16_fast_path_is_exact(cuda):
    """The decode's fast silu for bf16 models (hardware exp2 and reciprocal; the exact sequence
    near a bf16 rounding boundary and for |x| >= 64) equals bf16(silu(x)) of the oracle on every
    one of the 65,536 bf16 inputs: the whole input space, so the equality is complete."""
    from oracle import oracle as ox

    lib = mk_build.load()
    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    xd = torch.from_numpy(x).to(cuda)
    yd = torch.empty_like(xd)
    assert lib.lxm_t_elem(7, ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(yd.data_ptr()),
                          x.size, st) == 0
    y = yd.cpu().numpy()
    ref = ox.elem("bf16", ox.elem("silu", x))
    same = (bits(y) == bits(ref)) | (np.isnan(y) & np.isnan(ref))
    assert same.all(), int((~same).sum())


@pytest.mark.parametrize("kind,n", [(0, 3572), (0, 192), (1, 128), (1, 256)])
def test_device_sums_match_oracle(cuda, kind, n):
    from oracle import oracle as ox

    lib = mk_build.load()
    rng = np.random.default_rng(kind * 1000 + n)
    rows = 64
    x = (rng.standard_normal((rows, n)) * np.exp(rng.uniform(-8, 8, (rows, n)))).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda)
    out = torch.zeros(rows, device=cuda)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.lxm_t_sum(kind, ctypes.c_void_p(xd.data_ptr()), n, rows,
                         ctypes.c_void_p(out.data_ptr()), st) == 0
    ref = [ox.sum_h(x[i]) if kind == 0 else ox.sum_64(x[i]) for i in range(rows)]
    assert (bits(out.cpu().numpy()) == bits(np.array(ref, np.float32))).all()


def test_small_stack(cuda):
    check("small", 64)


def test_small_stack_fp32(cuda):
    check("small_fp32", 48)


def test_config1_greedy(cuda):
    """Benchmark config 1: 256 greedy steps of one chip-shaped fp32 layer."""
    check("c1", 256)


def test_config1_forced_inputs(cuda):
    """Config 1 driven by 256 seeded inputs (a quarter of its layer-steps gated)."""
    rng = np.random.default_rng(5)
    check("c1", 256, forced=rng.integers(0, 4096, 256).tolist())


def test_config2(cuda):
    """Benchmark config 2 (37 layers, bf16, N(0,1) state): 20 steps, every layer's residual."""
    check("c2", 20)


def test_config5(cuda):
    """Benchmark config 5 (half of the layer-steps gated): 8 steps."""
    check("c5", 8)


def test_dense_head_columns(cuda):
    """A head with dense columns (every row nonzero there; 2-bit codes in the helpers' LDS, the
    reference's head_dense), one with zeros: bf16 and fp32 stacks."""
    spec, m, _, _ = model("small_hd")
    assert mega.pack(fast.Fast(m), 0, 256).n_hd == 5
    check("small_hd", 48)
    check("small_hd_fp32", 40)


@pytest.mark.parametrize("via", ["coo", "hf"])
def test_merged_model_offset(cuda, via):
    """The merged model's call path (lx/lx/linux.py:108-109, :222): Fast(model, n_chip,
    rows=slice(offset, offset + VOCAB)) and Mega(fast, model, cache, offset), here with 300 rows
    of other tokens before the chip's; the inputs are chip token ids."""
    check("small_hd", 40, merged=(300, via), launches=[17, 23])


def test_merged_model_verified_mode(cuda):
    """Verified mode (Fast.verify) through the merged model's Fast (transformers model, rows)
    against the oracle's forced decode of the chip-only model."""
    from oracle import oracle as ox

    spec, m, c0, r0 = model("small_hd")
    off = 300
    hf = synth.to_hf(synth.merged(m, off))
    f = fast.Fast(hf, m.dims.n_layers, slice(off, off + m.dims.vocab))
    toks = [int(t) for t in synth.tokens(spec, 29, 3)]
    print("[gpu-test] merged verified mode: 29 tokens", flush=True)
    cache = fast.StateCache(c0, r0, m.dims.dtype, "cuda")
    got = f.verify(toks, cache).cpu().numpy().tolist()
    c, r = c0.copy(), r0.copy()
    want, _, _ = ox.OracleModel(m).decode(c, r, toks, len(toks))
    assert got == want.tolist()
    assert (bits(cache.conv_numpy()) == bits(c)).all()
    assert (bits(cache.rec_numpy()) == bits(r)).all()


def test_launches_continue_the_stream(cuda):
    """Three launches (5, 3 and 40 steps, each fed the last prediction) leave the same stream
    and states as one launch of 48: the windows written at a launch's end are the next's."""
    check("small", 48, launches=[5, 3, 40])


def test_short_launch_with_live_windows(cuda):
    """A launch shorter than the conv window, from nonzero windows on every channel (dead ones
    included): the first steps read the windows left before the launch."""
    spec, m, c0, r0 = model("small")
    rng = np.random.default_rng(9)
    conv0 = synth._round(rng.standard_normal(c0.shape).astype(np.float32), "bf16")
    check("small", 2, conv0=conv0)
    check("small", 9, launches=[1, 1, 1, 6], conv0=conv0)


def test_window_writer_waves_spanning_two_layers(cuda):
    """The launch's last conv windows are written by waves whose lanes can hold two layers'
    channels (the small stack's 6,144 channels over 256 workgroups: 24 a workgroup). Layer 1's
    first 24 query rows here also read ordinary columns, so their windows differ from what
    layer 0's ring rows would give: each lane has to read its own layer's rows. The test checks
    that such a wave exists and that its layer-1 channels hold nonzero windows, then compares
    the whole run with the oracle bit for bit."""
    import dataclasses

    from oracle import oracle as ox

    spec, m0, c0, r0 = model("small")
    d = m0.dims
    q = m0.layers[1].in_proj_qkv
    rng = np.random.default_rng(21)
    have = set(zip(q.rows.tolist(), q.cols.tolist()))
    rows, cols = [], []
    for r in range(24):
        for c in rng.choice(d.hidden - d.n_layers, size=3, replace=False):  # not a gate column
            if (r, int(c)) not in have:
                rows.append(r)
                cols.append(int(c))
    vals = rng.choice(np.array([0.5, -0.25, 0.75, -1.0], np.float32), size=len(rows))
    q2 = synth.Coo.build(q.shape, np.concatenate([q.rows, rows]), np.concatenate([q.cols, cols]),
                         np.concatenate([q.vals, vals]))
    layers = list(m0.layers)
    layers[1] = dataclasses.replace(layers[1], in_proj_qkv=q2)
    m = dataclasses.replace(m0, layers=layers)
    n = 64
    print("[gpu-test] window writer across layers: small, n=64", flush=True)
    cache = fast.StateCache(c0, r0, d.dtype, "cuda")
    mg = mega.Mega(fast.Fast(m), m, cache, 0)
    start = [synth.start_token(spec)]
    preds = mg.run(start, n)
    om = ox.OracleModel(m)
    c, r = c0.copy(), r0.copy()
    po, _, _ = om.decode(c, r, start, n)
    # a wave whose lane 0 holds a layer-0 channel and whose later lanes hold layer-1 query
    # channels with nonzero windows (the workgroups' channel ranges as the kernel deals them)
    per = -(-(d.n_layers * d.n_conv) // mg.ncta)
    b = d.n_conv // per
    w0 = b * per + 64 * ((d.n_conv - b * per) // 64)
    assert w0 < d.n_conv, "no wave spans layers 0 and 1"
    hi = min(w0 + 64, (b + 1) * per) - d.n_conv
    assert np.any(c[1, :hi] != 0), "the spanning wave's layer-1 windows are all zero"
    assert preds == po.tolist()
    assert (bits(cache.conv_numpy()) == bits(c)).all()
    assert (bits(cache.rec_numpy()) == bits(r)).all()


def test_forced_token_out_of_range(cuda):
    spec, m, c0, r0 = model("small")
    cache = fast.StateCache(c0, r0, m.dims.dtype, "cuda")
    mg = mega.Mega(fast.Fast(m), m, cache, 0)
    with pytest.raises(ValueError):
        mg.run([m.dims.vocab], 4)


def test_config2_long_run_properties(cuda):
    """4,096 steps of config 2: every input is the previous prediction (input purity), every
    prediction is a token, and the state of value heads no live gate reaches is untouched."""
    spec, m, c0, r0 = model("c2")
    cache = fast.StateCache(c0, r0, "bf16", "cuda")
    f = fast.Fast(m)
    mg = mega.Mega(f, m, cache, 0)
    n = 4096
    inp = torch.zeros(n, dtype=torch.int32, device="cuda")
    preds = mg.run([synth.start_token(spec)], n, inputs=inp)
    inp = inp.cpu().numpy()
    assert (inp[1:] == np.array(preds[:-1])).all()
    assert min(preds) >= 0 and max(preds) < m.dims.vocab
    rec = cache.rec_numpy()
    R = m.dims.nv // m.dims.nk
    for L in (0, 18, 36):
        touched = set()
        for kh in f.dec[L]["kh"]:
            touched.update(range(kh * R, kh * R + R))
        touched.update(int(v) for v in f.dec[L]["decays"])
        idle = [v for v in range(m.dims.nv) if v not in touched]
        assert idle and (bits(rec[L][idle]) == bits(r0[L][idle])).all()


@pytest.mark.parametrize("name,golden", [("c2", "c2_chunk.json"), ("c5", "c5_run.json")])
def test_whole_run_equals_oracle(cuda, name, golden):
    """Benchmark config 2's whole 262,144-token greedy chunk, and config 5's 65,536-token run
    (half of the layer-steps gated: long chains of GDN events and MLP redos), each from its start
    token and initial state, in four launches continuing one stream: the prediction stream and
    the final conv windows and recurrent states hash to what the CPU oracle's run of the same
    tokens hashes (tests/golden/c2_chunk.json and c5_run.json, written by
    tests/golden/make_chunk.py; the reference pins its boot the same way:
    lx/tools/mega_boot.py:74-75, lx/results/mega_boot.json's stream_sha256)."""
    import hashlib
    import json
    import os

    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", golden)))
    spec, m, conv0, rec0 = model(name)
    assert g["config"] == spec.name and g["start"] == synth.start_token(spec)
    print(f"[gpu-test] {name} whole run: {g['chunk']} tokens", flush=True)
    cache = fast.StateCache(conv0, rec0, m.dims.dtype, "cuda")
    mg = mega.Mega(fast.Fast(m), m, cache, 0)
    preds, tok = [], g["start"]
    n = g["chunk"] // 4
    for _ in range(4):
        preds += mg.run([tok], n)
        tok = preds[-1]
        print(f"[gpu-test] {name} whole run: {len(preds)} tokens", flush=True)
    assert preds[:256] == g["first_preds"] and preds[-16:] == g["last_preds"]
    assert hashlib.sha256(np.asarray(preds, "<i4").tobytes()).hexdigest() == g["stream_sha256"]
    hc, hr = hashlib.sha256(), hashlib.sha256()
    for ly in cache.layers:
        hc.update(ly.conv_states[0][0].float().cpu().numpy().tobytes())
        hr.update((ly.recurrent_states[0][0].cpu().numpy() + np.float32(0.0)).tobytes())
    assert hc.hexdigest() == g["conv_sha256"]
    assert hr.hexdigest() == g["rec_sha256"]
