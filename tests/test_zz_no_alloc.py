"""lxm_run_noalloc (the decode launch whose run buffers live in the library's static per-device
scratch) against lxm_run (Mega.run, caller-allocated run buffers): predictions, each step's input
and the final conv windows and recurrent states, bit for bit, over calls in a row whose inputs
shrink, across two models (the scratch keeps the previous call's contents)."""

import numpy as np
import pytest
import torch

from linuxformer_amd import fast, mega, synth

pytestmark = pytest.mark.gpu


def _pair(spec):
    m = synth.build(spec)
    conv0, rec0 = synth.init_state(m)
    dev = torch.device("cuda", 0)
    ca = fast.StateCache(conv0, rec0, m.dims.dtype, dev)
    cb = fast.StateCache(conv0, rec0, m.dims.dtype, dev)
    ma = mega.Mega(fast.Fast(m), m, ca, 0, device="cuda:0")
    mb = mega.Mega(fast.Fast(m), m, cb, 0, device="cuda:0")
    return m, ma, mb, ca, cb


def _same_states(ca, cb):
    for la, lb in zip(ca.layers, cb.layers):
        assert torch.equal(la.conv_states[0].view(torch.int16) if la.conv_states[0].dtype == torch.bfloat16
                           else la.conv_states[0].view(torch.int32),
                           lb.conv_states[0].view(torch.int16) if lb.conv_states[0].dtype == torch.bfloat16
                           else lb.conv_states[0].view(torch.int32))
        assert torch.equal(la.recurrent_states[0].view(torch.int32), lb.recurrent_states[0].view(torch.int32))


def _noalloc(mb, forced, n):
    dev = mb.dev
    ft = torch.tensor(np.asarray(forced, np.int32), device=dev)
    preds = torch.full((n,), -1, dtype=torch.int32, device=dev)
    inputs = torch.full((n,), -1, dtype=torch.int32, device=dev)
    err = torch.full((1,), 7, dtype=torch.int32, device=dev)  # the call clears it
    mb.run_noalloc(ft, n, preds, err, inputs=inputs)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    return preds.cpu().tolist(), inputs.cpu().tolist()


@pytest.mark.parametrize("name", ["small", "c1"])
def test_noalloc_equals_run_on_shrinking_calls(name):
    spec = synth.small() if name == "small" else synth.config1()
    m, ma, mb, ca, cb = _pair(spec)
    start = synth.start_token(spec)
    tok_a = tok_b = start
    for n in (40, 9):  # the second call smaller than the first
        print(f"[no_alloc] {name}: {n} tokens", flush=True)
        inp = torch.zeros(n, dtype=torch.int32, device=ma.dev)
        want = ma.run([tok_a], n, inputs=inp)
        got, got_in = _noalloc(mb, [tok_b], n)
        assert got == want
        assert got_in == inp.cpu().tolist()
        _same_states(ca, cb)
        tok_a, tok_b = want[-1], got[-1]
    # a forced stream through both entry points
    toks = synth.tokens(spec, 12, 5).tolist()
    want = ma.run(toks, 12)
    got, _ = _noalloc(mb, toks, 12)
    assert got == want
    _same_states(ca, cb)


def test_noalloc_rejects_shapes_beyond_its_scratch():
    from linuxformer_amd import mk_build

    spec = synth.small()
    m, ma, mb, ca, cb = _pair(spec)
    lib = mk_build.load()
    rs, cs = mb._state_ptrs_cached()
    ft = torch.zeros(1, dtype=torch.int32, device=mb.dev)
    preds = torch.zeros(4, dtype=torch.int32, device=mb.dev)
    err = torch.zeros(1, dtype=torch.int32, device=mb.dev)
    import ctypes

    st = ctypes.c_void_p(torch.cuda.current_stream(mb.dev).cuda_stream)
    p = mb._params(rs, cs, ft, 1, 4, preds)
    p.err = err.data_ptr()
    p.n_layers = 65  # beyond LXM_SCRATCH_MAXL: refused before anything is launched
    assert lib.lxm_run_noalloc(ctypes.byref(p), mb.ncta, mb.lds, st) != 0
    p.n_layers = m.dims.n_layers
    p.err = None  # the error word is the caller's
    assert lib.lxm_run_noalloc(ctypes.byref(p), mb.ncta, mb.lds, st) != 0
