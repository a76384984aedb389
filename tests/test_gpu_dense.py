"""Parity of the HIP dense decode (benchmark config 4's structure) with the oracle on an MI355X,
through the C ABI (the persistent run, lxm_dn_run, the per-step kernels, lxm_dn_step, and the
batched prefill, lxm_dn_prefill, followed by steps): predictions and final states bit for bit. The dense projections are summed in
the dense order the oracle restates for matrices marked dense (64 groups of a row's entries in
order from +0, then the pairwise tree); everything else follows the stock decode as in the
sparse paths. Sizes: config 4's layout scaled down (hidden 256, 2 layers) so the oracle runs in
seconds; the full config is measured by bench.py (--legs dense).
"""

import numpy as np
import pytest
import torch

from linuxformer_amd import dense, fast, mk_build, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cuda():
    assert torch.cuda.is_available(), "the gpu tests need an MI355X"
    mk_build.load()
    return torch.device("cuda", 0)


_M = {}


def model(name="small"):
    if name not in _M:
        spec = synth.config4_small() if name == "small" else synth.config4_mid()
        dm_cpu = synth.build_dense(spec, "cpu")
        _M[name] = (spec, dm_cpu, synth.to_sparse(dm_cpu))
    return _M[name]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def check(n_forced, n, seed=None, graph=True, name="small", mode="persistent"):
    from oracle import oracle as ox

    spec, dm_cpu, sm = model(name)
    conv0, rec0 = synth.dense_state(dm_cpu, seed)
    forced = [int(x) for x in np.random.default_rng(7 + n_forced).integers(0, spec.vocab, n_forced)]
    print(f"[gpu-test] dense {spec.name}: forced={n_forced} n={n} seed={seed} mode={mode} "
          f"graph={graph}", flush=True)
    dm = synth.dense_to(dm_cpu, "cuda")
    cache = fast.StateCache(conv0, rec0, "bf16", "cuda")
    dd = dense.DenseDecode(dm, cache)
    preds = dd.run(forced, n, graph=graph, mode=mode)
    c, r = conv0.copy(), rec0.copy()
    po, _, _ = ox.OracleModel(sm).decode(c, r, forced, n)
    assert preds == po.tolist()
    assert (bits(cache.conv_numpy()) == bits(c)).all()
    assert (bits(cache.rec_numpy()) == bits(r)).all()
    return preds


MODES = ["persistent", "steps"]


@pytest.mark.parametrize("mode", MODES)
def test_dense_small_greedy(cuda, mode):
    check(1, 24, mode=mode)


@pytest.mark.parametrize("mode", MODES)
def test_dense_small_forced_then_greedy(cuda, mode):
    """A forced prefix (the config's prefill, scaled down), then greedy steps."""
    check(16, 32, mode=mode)


def test_dense_small_live_state_eager(cuda):
    """From N(0, 1) states and nonzero windows on the live heads, eager steps (no graph)."""
    check(4, 12, seed=3, graph=False, mode="steps")


def test_dense_small_live_state_graph(cuda):
    check(4, 12, seed=3, graph=True, mode="steps")


def test_dense_persistent_phase_clock(cuda):
    """The profiling build's persistent run (its phase clock on) predicts what the oracle does and
    fills the clock: every workgroup's six phases, each use counted in ticks."""
    from oracle import oracle as ox

    spec, dm_cpu, sm = model("small")
    conv0, rec0 = synth.dense_state(dm_cpu, 3)
    forced = [int(x) for x in np.random.default_rng(11).integers(0, spec.vocab, 3)]
    print(f"[gpu-test] dense {spec.name}: persistent run with the phase clock", flush=True)
    dm = synth.dense_to(dm_cpu, "cuda")
    cache = fast.StateCache(conv0, rec0, "bf16", "cuda")
    dd = dense.DenseDecode(dm, cache, subprof=True)
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    prof = torch.zeros(32 * ncu, dtype=torch.int64, device="cuda")
    preds = dd.run(forced, 10, mode="persistent", prof=prof)
    c, r = conv0.copy(), rec0.copy()
    po, _, _ = ox.OracleModel(sm).decode(c, r, forced, 10)
    assert preds == po.tolist()
    assert (bits(cache.rec_numpy()) == bits(r)).all()
    acc = prof.view(ncu, 32)[:, :18].cpu().numpy().reshape(ncu, 6, 3)
    assert (acc[:, :, 1:].sum(axis=2) > 0).all()  # every phase's rows and barrier took time
    assert (acc >= 0).all() and (acc[:, 5, 1] > 0).all()  # the head's rows on every workgroup
    with pytest.raises(ValueError):
        dd.run(forced, 2, mode="persistent", prof=prof[:16])


def test_dense_small_live_state_persistent(cuda):
    check(4, 12, seed=3)


@pytest.mark.parametrize("mode", MODES)
def test_dense_full_widths(cuda, mode):
    """Config 4's full row lengths (hidden 2560: 40 entries per lane; SwiGLU 9216: 144; 16 key
    heads x 2 live value heads: 4096 out_proj entries, 64) over one layer, from live states."""
    check(3, 6, seed=5, name="mid", mode=mode)


def check_prefill(T, n, seed=None, name="small"):
    """lxm_dn_prefill over T - 1 forced tokens, then n steps from the last one: the predictions
    and states of T - 1 + n steps of the oracle with the same T forced tokens."""
    from oracle import oracle as ox

    spec, dm_cpu, sm = model(name)
    conv0, rec0 = synth.dense_state(dm_cpu, seed)
    toks = [int(x) for x in np.random.default_rng(11 + T).integers(0, spec.vocab, T)]
    print(f"[gpu-test] dense prefill {spec.name}: T={T} n={n} seed={seed}", flush=True)
    dm = synth.dense_to(dm_cpu, "cuda")
    cache = fast.StateCache(conv0, rec0, "bf16", "cuda")
    dd = dense.DenseDecode(dm, cache)
    dd.prefill(toks[:-1])
    preds = dd.run(toks[-1:], n)
    c, r = conv0.copy(), rec0.copy()
    po, _, _ = ox.OracleModel(sm).decode(c, r, toks, T - 1 + n)
    assert preds == po.tolist()[T - 1:]
    assert (bits(cache.conv_numpy()) == bits(c)).all()
    assert (bits(cache.rec_numpy()) == bits(r)).all()


@pytest.mark.parametrize("T,seed", [(40, None), (3, 3), (34, 3)])
def test_dense_prefill_small(cuda, T, seed):
    """Batches of 16 (the last one partial), a prompt shorter than the conv window, live states."""
    check_prefill(T, 6, seed=seed)


def test_dense_prefill_full_widths(cuda):
    check_prefill(21, 3, seed=5, name="mid")


def test_dense_prefill_equals_steps_config4(cuda):
    """At config 4's full size (24 layers, hidden 2560, vocabulary 248,320): a 40-token prompt
    through lxm_dn_prefill and one step leaves the prediction and every state and window that
    40 forced steps leave, bit for bit (two native paths, each pinned to the oracle above on the
    scaled-down stacks)."""
    spec = synth.config4()
    dm = synth.build_dense(spec, "cuda")
    d = dm.dims
    toks = [int(x) for x in np.random.default_rng(9).integers(0, spec.vocab, 40)]
    print(f"[gpu-test] dense prefill config 4 full size: T={len(toks)}", flush=True)
    out = []
    for batched in (False, True):
        conv0 = np.zeros((d.n_layers, d.n_conv, 4), np.float32)
        rec0 = np.zeros((d.n_layers, d.nv, 256, 128), np.float32)
        cache = fast.StateCache(conv0, rec0, "bf16", "cuda")
        dd = dense.DenseDecode(dm, cache, max_steps=64)
        if batched:
            dd.prefill(toks[:-1])
            p = dd.run(toks[-1:], 1)
        else:
            p = dd.run(toks, len(toks))[-1:]
        out.append((p, [l.conv_states[0].clone() for l in cache.layers],
                    [l.recurrent_states[0].clone() for l in cache.layers]))
        del dd, cache
    (p0, c0, r0), (p1, c1, r1) = out
    assert p0 == p1
    for a, b in zip(c0, c1):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    for a, b in zip(r0, r1):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert any(bool(r.any()) for r in r1)  # (the prompt moved the live states)


def test_dense_prefill_rejects_bad_token(cuda):
    spec, dm_cpu, _ = model()
    conv0, rec0 = synth.dense_state(dm_cpu)
    dd = dense.DenseDecode(synth.dense_to(dm_cpu, "cuda"), fast.StateCache(conv0, rec0, "bf16", "cuda"))
    with pytest.raises(ValueError, match="out of range"):
        dd.prefill([1, spec.vocab])


def test_dense_rejects_dead_state(cuda):
    """A nonzero state on a dead value head would not stay zero as the kernels assume."""
    spec, dm_cpu, sm = model()
    conv0, rec0 = synth.dense_state(dm_cpu)
    rec0[0, 2, 0, 0] = 1.0  # value head 2 of key head 0: dead (r_live = 2)
    cache = fast.StateCache(conv0, rec0, "bf16", "cuda")
    with pytest.raises(AssertionError):
        dense.DenseDecode(synth.dense_to(dm_cpu, "cuda"), cache)


def check_prefill_chunked(T, n, seed=None, name="small"):
    """lxm_dn_prefill_chunked over T - 1 tokens (the stock T > 1 path: chunks of 64, the delta
    rule on the matrix cores), then n steps from the last token, against the oracle's restatement
    of the same (ox_prefill_chunked, then ox_decode). The chunked delta rule sums in its own order
    (MFMA tiles), so its outputs match the oracle's to about 1e-6 before they round to bf16: a
    rare output rounds the other way and moves the residual by one bf16 step, which the later
    layers carry. Bounds: the first layer's recurrent states (its inputs are the embeddings, so
    only the delta rule's own arithmetic differs) within 1e-6 of each head's largest magnitude
    (measured <= 2e-7; the oracle's recurrent and chunked forms differ by up to 9e-7); later
    layers within 5e-3 (measured <= 9e-4; the oracle's two forms differ by up to 1.3e-3 there);
    at least 99 % of the conv windows' values bit for bit (measured: all) and the rest within
    2^-6 relative; the same greedy predictions."""
    from oracle import oracle as ox

    spec, dm_cpu, sm = model(name)
    conv0, rec0 = synth.dense_state(dm_cpu, seed)
    toks = [int(x) for x in np.random.default_rng(23 + T).integers(0, spec.vocab, T)]
    print(f"[gpu-test] dense chunked prefill {spec.name}: T={T} n={n} seed={seed}", flush=True)
    dm = synth.dense_to(dm_cpu, "cuda")
    cache = fast.StateCache(conv0, rec0, "bf16", "cuda")
    dd = dense.DenseDecode(dm, cache)
    dd.prefill(toks[:-1], mode="chunked")
    gc_, gr = cache.conv_numpy().copy(), cache.rec_numpy().copy()
    preds = dd.run(toks[-1:], n)
    om = ox.OracleModel(sm)
    c, r = conv0.copy(), rec0.copy()
    om.prefill_chunked(c, r, toks[:-1])
    diff = bits(gc_) != bits(c)
    assert diff.mean() <= 0.01, diff.mean()
    assert (np.abs(gc_ - c) <= 2.0 ** -6 * np.abs(c)).all()
    for L in range(r.shape[0]):
        bound = 1e-6 if L == 0 else 5e-3
        for h in range(r.shape[1]):
            ref = np.abs(r[L, h]).max()
            assert np.abs(gr[L, h] - r[L, h]).max() <= bound * max(ref, 1e-30), (L, h)
    po, _, _ = om.decode(c, r, toks[-1:], n)
    assert preds == po.tolist()
    # the prompt moved the live heads' states (the chunked path ran)
    assert not np.array_equal(gr, rec0)
    return gr


@pytest.mark.parametrize("T,seed", [(150, None), (66, 3), (20, 3)])
def test_dense_prefill_chunked_small(cuda, T, seed):
    """Chunks of 64 with a ragged last one, exactly one chunk plus a token, a prompt shorter than
    one chunk; from zero and from live states."""
    check_prefill_chunked(T, 6, seed=seed)


def test_dense_prefill_chunked_full_widths(cuda):
    check_prefill_chunked(70, 3, seed=5, name="mid")


def test_dense_prefill_chunked_close_to_batched(cuda):
    """The chunked and the batched (recurrent, bit-exact to forced steps) prompts on the same
    tokens: the same states up to rounding: the first layer within 2e-6 of each head's largest
    magnitude (the two forms' own arithmetic), the later ones within 5e-3 (rare bf16 outputs
    rounding the other way, carried)."""
    spec, dm_cpu, sm = model("small")
    conv0, rec0 = synth.dense_state(dm_cpu, 3)
    toks = [int(x) for x in np.random.default_rng(5).integers(0, spec.vocab, 100)]
    dm = synth.dense_to(dm_cpu, "cuda")
    out = []
    for mode in ("batched", "chunked"):
        cache = fast.StateCache(conv0, rec0, "bf16", "cuda")
        dense.DenseDecode(dm, cache).prefill(toks, mode=mode)
        out.append(cache.rec_numpy())
    a, b = out
    for L in range(a.shape[0]):
        bound = 2e-6 if L == 0 else 5e-3
        for h in range(a.shape[1]):
            assert np.abs(a[L, h] - b[L, h]).max() <= bound * max(np.abs(a[L, h]).max(), 1e-30)
    assert not np.array_equal(a, b)  # different forms, different roundings
