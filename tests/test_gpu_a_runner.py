"""The C-only binding (csrc/lxm_runner.cpp): a packed decode replayed through liblxm.so's C ABI
by a process with no Python, as a foreign host (C, cgo, JNI) would drive it: dlopen, the
parameter block filled from the dumped tables, lxm_run. Its stream must be the oracle's.

The runner's cooperative launch is refused (hipErrorIllegalState, 401) while another process
that has made cooperative launches holds the device, so the runner runs in a child of a process
that has made none: this file sorts before the other GPU tests, and the test skips itself, with
that reason, when this process has already launched cooperatively (it is run after the others).
"""

import json
import os
import subprocess

import pytest
import torch

from linuxformer_amd import fast, mega, mk_build, synth

pytestmark = pytest.mark.gpu


def test_native_runner_continues_the_stream(tmp_path):
    from oracle import oracle as ox

    assert torch.cuda.is_available(), "the gpu tests need an MI355X"
    mk_build.load()
    if mk_build.cooperative_launches:
        pytest.skip("this process has made cooperative launches: the runner's would be refused "
                    "with hipErrorIllegalState (401) while it holds the device")
    assert os.path.exists(mk_build.RUNNER), "lxm_runner is built by mk_build.build()"
    spec = synth.small()
    m = synth.build(spec)
    conv0, rec0 = synth.init_state(m)
    start = synth.start_token(spec)
    cache = fast.StateCache(conv0, rec0, m.dims.dtype, "cuda")
    mg = mega.Mega(fast.Fast(m), m, cache, 0)  # packs and uploads; launches nothing
    n = 24
    mg.dump(str(tmp_path), [start], n)
    del mg, cache
    torch.cuda.synchronize()
    print(f"[gpu-test] lxm_runner: 2 launches of {n} tokens", flush=True)
    r = subprocess.run([mk_build.RUNNER, str(tmp_path), "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    want, _, _ = ox.OracleModel(m).decode(conv0.copy(), rec0.copy(), [start], 2 * n)
    assert out["tokens_per_launch"] == n and out["launches"] == 2
    assert out["last_pred"] == int(want[-1])
    assert out["tok_per_s"] > 0
