"""The model-alone driver loop (linuxformer_amd.alone, lx/lx/linux.py:230-310's run_alone) on an
MI355X: its launches replayed on the oracle give the same stream and states bit for bit, the
launch sizes double from the first to the cap while nothing is answered, keystroke batches land
at record boundaries, and every launch's inputs pass the purity check."""

import numpy as np
import pytest
import torch

from linuxformer_amd import alone, fast, mega, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup():
    assert torch.cuda.is_available(), "the gpu tests need an MI355X"
    spec = synth.small()
    m = synth.build(spec)
    conv0, rec0 = synth.init_state(m)
    return spec, m, conv0, rec0


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def replay(m, conv0, rec0, launches):
    """The same launches on the oracle: the stream of inputs, and the final states."""
    from oracle import oracle as ox

    om = ox.OracleModel(m)
    c, r = conv0.copy(), rec0.copy()
    stream = []
    for forced, n in launches:
        preds, _, _ = om.decode(c, r, forced, n)
        preds = preds.tolist()
        stream += list(forced) + preds[len(forced) - 1:n - 1]
    return stream, c, r


def test_alone_decodes_its_own_stream(setup):
    spec, m, conv0, rec0 = setup
    cache = fast.StateCache(conv0, rec0, m.dims.dtype, "cuda")
    mg = mega.Mega(fast.Fast(m), m, cache, 0)
    print("[gpu-test] alone: one batch, 300 tokens, launches 16..64", flush=True)
    r = alone.run_alone(mg, [[int(synth.start_token(spec))]], final=lambda t: True,
                        done=lambda st, b: len(st) >= 300, first_launch=16, max_launch=64)
    assert r["launch_sizes"][:3] == [16, 32, 64] and set(r["launch_sizes"][2:]) <= {64, 1}
    assert r["input_purity"]["passed"] and r["tokens"] >= 300
    want, c, rr = replay(m, conv0, rec0, r["launches"])
    assert r["stream"] == want
    assert (bits(cache.conv_numpy()) == bits(c)).all()
    assert (bits(cache.rec_numpy()) == bits(rr)).all()


def test_alone_types_at_record_boundaries(setup):
    spec, m, conv0, rec0 = setup
    cache = fast.StateCache(conv0, rec0, m.dims.dtype, "cuda")
    mg = mega.Mega(fast.Fast(m), m, cache, 0)
    vocab = m.dims.vocab
    batches = [[3, 5, 7], [11], [13, 17]]
    final = lambda t: t % 4 == 0  # noqa: E731  (a record boundary: a quarter of the tokens)
    print("[gpu-test] alone: three batches at boundaries", flush=True)
    r = alone.run_alone(mg, batches, final=final,
                        done=lambda st, b: len(st) >= 60 * (b + 1), first_launch=8,
                        max_launch=32)
    assert all(0 <= t < vocab for t in r["stream"])
    for i, at in enumerate(r["typed_at"]):
        assert r["stream"][at:at + len(batches[i])] == batches[i]
        assert at == 0 or final(r["stream"][at - 1])
    assert r["input_purity"]["keystrokes"] == 6 and r["input_purity"]["passed"]
    want, c, rr = replay(m, conv0, rec0, r["launches"])
    assert r["stream"] == want
    assert (bits(cache.rec_numpy()) == bits(rr)).all()
