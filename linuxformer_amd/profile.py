"""In-kernel cycle counters of the decode kernel (lx.mega's prof buffer and MK_SUBPROF build):

    python -m linuxformer_amd.profile --config c2 --tokens 4096 [--subprof]
    python -m linuxformer_amd.profile --config c4 --tokens 1024 [--mode chunked|batched]
    python -m linuxformer_amd.profile --config c4 --tokens 256 --mode phases

Runs one launch of --tokens greedy steps from the config's start token and initial state with
the phase counters on, and prints one JSON object: cycles per token of each chain phase
(embedding, stage A, stage B, GDN events, stage C1, stage C2, final norm, head wait), the
helpers' mean and max cycles per token in each of their parts, and with --subprof (the library
built with -DLXM_SUBPROF) each chain wave's busy and waiting cycles per layer in each stage.
The counters are the chain's own clock cycle counter; `clock_mhz` is the chain's cycles per token
over the launch's wall time per token (the launch's set-up included).

--config c4 runs only config 4's prompt (--tokens seeded uniform ids from a zero state) through
DenseDecode.prefill in the given mode, once to warm up and once timed: the process to put under
rocprofv3 for the prompt's kernels (few enough dispatches for counter collection). With
--mode phases it runs config 4's persistent decode (lxm_dn_run, the LXM_SUBPROF build) for
--tokens greedy steps after a 64-token prompt and prints the phase clock: per phase, the
microseconds per use from its start (the barrier before it passed) to its input staged, to every
wave's rows summed, and to the next barrier passed, for workgroup 0 (a delta-rule workgroup),
the last workgroup, and the mean over workgroups."""

from __future__ import annotations

import argparse
import json
import sys
import time

import torch

from . import fast, mega, synth


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c5", "small", "c4"])
    ap.add_argument("--tokens", type=int, default=4096)
    ap.add_argument("--subprof", action="store_true")
    ap.add_argument("--mode", default="chunked", choices=["chunked", "batched", "phases"])
    a = ap.parse_args()
    if a.config == "c4":
        return dense_phases(a.tokens) if a.mode == "phases" else dense_prompt(a.tokens, a.mode)
    spec = {"c1": synth.config1(), "c2": synth.config2(), "c5": synth.config5(),
            "small": synth.small()}[a.config]
    m = synth.build(spec)
    conv0, rec0 = synth.init_state(m)
    dev = torch.device("cuda", 0)
    cache = fast.StateCache(conv0, rec0, m.dims.dtype, dev)
    mg = mega.Mega(fast.Fast(m), m, cache, 0, subprof=a.subprof)
    start = synth.start_token(spec)
    mg.run([start], 256)  # warm-up (first touch of the tables)
    prof = torch.zeros(mg.prof_size, dtype=torch.int64, device=dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    mg.run([start], a.tokens, prof=prof)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    rep = mg.phase_report(prof)
    chain = sum(v for k, v in rep.items() if k in mega.Mega.PHASES)
    rep["chain cycles per token"] = round(chain, 1)
    rep["us per token"] = round(wall * 1e6 / a.tokens, 2)
    rep["clock_mhz"] = round(chain / (wall * 1e6 / a.tokens), 1)
    rep["config"] = spec.name
    rep["subprof"] = a.subprof
    print(json.dumps(rep))
    return 0


def dense_prompt(n: int, mode: str) -> int:
    import numpy as np

    from . import dense

    spec = synth.config4()
    dev = torch.device("cuda", 0)
    dm = synth.build_dense(spec, "cuda")
    d = dm.dims
    toks = np.random.default_rng(spec.seed).integers(0, spec.vocab, n).tolist()
    times = []
    for _ in range(2):
        conv0 = np.zeros((d.n_layers, d.n_conv, 4), np.float32)
        rec0 = np.zeros((d.n_layers, d.nv, 256, 128), np.float32)
        cache = fast.StateCache(conv0, rec0, "bf16", dev)
        dd = dense.DenseDecode(dm, cache, max_steps=2)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dd.prefill(toks, mode=mode)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        del dd, cache
    print(json.dumps({"config": "c4", "mode": mode, "tokens": n, "s": [round(x, 4) for x in times],
                      "tok_s": round(n / times[-1], 1)}))
    return 0


def dense_phases(n: int) -> int:
    import numpy as np

    from . import dense

    spec = synth.config4()
    dev = torch.device("cuda", 0)
    dm = synth.build_dense(spec, "cuda")
    d = dm.dims
    conv0 = np.zeros((d.n_layers, d.n_conv, 4), np.float32)
    rec0 = np.zeros((d.n_layers, d.nv, 256, 128), np.float32)
    cache = fast.StateCache(conv0, rec0, "bf16", dev)
    dd = dense.DenseDecode(dm, cache, max_steps=n + 64, subprof=True)
    toks = np.random.default_rng(spec.seed).integers(0, spec.vocab, 64).tolist()
    dd.prefill(toks[:-1])
    p1 = dd.run(toks[-1:], 1, graph=False)
    dd.run([p1[-1]], 8, mode="persistent")  # warm-up
    ncu = torch.cuda.get_device_properties(dev).multi_processor_count
    prof = torch.zeros(32 * ncu, dtype=torch.int64, device=dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dd.run([p1[-1]], n, mode="persistent", prof=prof)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    acc = prof.view(ncu, 32)[:, :18].cpu().numpy().reshape(ncu, 6, 3).astype(np.float64) * 0.01
    rep = {"config": "c4", "steps": n, "us_per_token": round(wall * 1e6 / n, 1),
           "segments": ["input staged", "rows summed", "barrier passed"]}
    for k, name in enumerate(["projections", "delta rule", "out_proj", "SwiGLU", "down_proj",
                              "head"]):
        per = n * (d.n_layers if k < 5 else 1)
        a = acc[:, k, :] / per
        rep[name] = {"wg0": [round(x, 2) for x in a[0]], "wg_last": [round(x, 2) for x in a[-1]],
                     "mean": [round(x, 2) for x in a.mean(0)],
                     "rows_max": round(float(a[:, 1].max()), 2)}
    print(json.dumps(rep))
    return 0


if __name__ == "__main__":
    sys.exit(main())
