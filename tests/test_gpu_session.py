"""The non-mega decode as replayed graphs (Session.step / Session.free, lx/lx/session.py:148-225)
against the oracle's greedy decode, on an MI355X, through the C ABI.

Session.step(start) then Session.free(n) runs the tokens start, p0, p1, ..., each the prediction
of the one before, through the single-token step graph and the graph of run_k steps fed back on
the GPU: the predictions, the final conv windows and the final recurrent states must equal the
oracle's n + 1 greedy steps bit for bit. Graphs are replayed several times with eager work and
synchronisations between the replays, and a verified-mode call of another length on the same
Fast between two replays must not disturb them (the session owns its run buffers).
"""

import numpy as np
import pytest
import torch

from linuxformer_amd import fast, mk_build, synth
from linuxformer_amd.session import Session

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cuda():
    assert torch.cuda.is_available(), "the gpu tests need an MI355X"
    mk_build.load()
    return torch.device("cuda", 0)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _model(name):
    spec = {"small": synth.small(), "small_fp32": synth.small(dtype="fp32", seed=3),
            "c1": synth.config1(), "c5": synth.config5()}[name]
    m = synth.build(spec)
    conv0, rec0 = synth.init_state(m)
    return spec, m, conv0, rec0


@pytest.mark.parametrize("name,n", [("small", 64 + 9), ("small_fp32", 2 * 64 + 3), ("c1", 256),
                                    ("c5", 64 + 5)])
def test_session_free_equals_oracle(cuda, name, n):
    from oracle import oracle as ox

    spec, m, conv0, rec0 = _model(name)
    start = synth.start_token(spec)
    print(f"[gpu-test] session {name}: n={n}", flush=True)
    f = fast.Fast(m)
    cache = fast.StateCache(conv0, rec0, m.dims.dtype, cuda)
    s = Session(f, cache)
    p0 = s.step(start)
    out = s.free(n)
    torch.cuda.synchronize()
    om = ox.OracleModel(m)
    c, r = conv0.copy(), rec0.copy()
    want, inputs, _ = om.decode(c, r, [start], n + 1)
    assert p0 == int(want[0])
    assert out == want[:n].tolist()
    assert s.next == int(want[n])
    assert inputs.tolist() == [start] + out
    assert (bits(cache.conv_numpy()) == bits(c)).all()
    assert (bits(cache.rec_numpy()) == bits(r)).all()


def test_session_replays_survive_other_calls(cuda):
    """Three replays of the run graph with eager work between them, and a verified-mode call of
    another length on the same Fast (its own buffers) between two replays."""
    from oracle import oracle as ox

    spec, m, conv0, rec0 = _model("small")
    start = synth.start_token(spec)
    f = fast.Fast(m)
    cache = fast.StateCache(conv0, rec0, m.dims.dtype, cuda)
    other = fast.StateCache(conv0, rec0, m.dims.dtype, cuda)
    s = Session(f, cache)
    s.step(start)
    k = s.run_k
    out = s.free(k)
    x = torch.randn(1000, device=cuda).sum()  # eager work between the replays
    torch.cuda.synchronize()
    out += s.free(k)
    f.verify([int(t) for t in synth.tokens(spec, 37)], other)  # another T on the same Fast
    torch.cuda.synchronize()
    out += s.free(k)
    del x
    om = ox.OracleModel(m)
    c, r = conv0.copy(), rec0.copy()
    want, _, _ = om.decode(c, r, [start], 3 * k + 1)
    assert out == want[:3 * k].tolist()
    assert (bits(cache.conv_numpy()) == bits(c)).all()
    assert (bits(cache.rec_numpy()) == bits(r)).all()


def test_session_forced_steps_equal_oracle(cuda):
    """step() with tokens the caller chooses (the typed path): each prediction is the oracle's
    for the same forced inputs."""
    from oracle import oracle as ox

    spec, m, conv0, rec0 = _model("small")
    toks = [int(t) for t in synth.tokens(spec, 12, 5)]
    f = fast.Fast(m)
    cache = fast.StateCache(conv0, rec0, m.dims.dtype, cuda)
    s = Session(f, cache)
    got = [s.step(t) for t in toks]
    om = ox.OracleModel(m)
    c, r = conv0.copy(), rec0.copy()
    want, _, _ = om.decode(c, r, toks, len(toks))
    assert got == want.tolist()
    assert (bits(cache.rec_numpy()) == bits(r)).all()
    with pytest.raises(ValueError):
        s.step(m.dims.vocab)
