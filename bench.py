"""Benchmark: greedy decode tok/s of the 37-layer synthetic sparse chip stack on one MI355X, and
verified-prefill tok/s of the same stack (BASELINE's two metrics).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--tokens T] [--config c2]
                    [--legs decode,prefill,dense] [--pf-calls N] [--pf-tokens T]

Decode (the headline `value`): a step is one launch of the persistent decode kernel over one
chunk of T tokens (default 262,144), continuing the same greedy stream launch
after launch, as lx/tools/mega_boot.py runs the boot in 262,144-token launches. The model is the
seeded synthetic stack (synth.config2: 37 layers, hidden 3572, bf16, 0.08 % density, N(0,1)
state); it is built and packed on the host, then every input is resident in HBM before the
timed region.

Verified prefill (`verified_prefill`): BASELINE config 3, calls of 65,536 seeded uniform tokens
through the same stack (synth.config3: 0.35 % of token-layers gated, 5 % of (key head, 64-token
chunk) pairs active), each call embedding, running all 37 layers and taking every position's
argmax (lx.fast's verified mode), timed with HIP events on the stream after two warm-up calls.

Dense decode (`dense_decode`): BASELINE config 4, the dense padded text-view stack
(synth.config4: 24 layers, hidden 2560, SwiGLU 9216); an 8,192-token prompt of seeded uniform ids
(the batched prefill, then one step), then 4,096 greedy steps timed.

One JSON line on stdout (the driver's contract); everything else goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "greedy decode tok/s, 37-layer sparse chip stack, 1 MI355X; verified prefill tok/s"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3  # MI355X's published fp32 peak


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def survey_bytes_per_token(model, f_out: float) -> float:
    """The algorithmic bytes of one decoded token, SURVEY 8(d)'s formula for config 2:
    sum over layers of 4 B per nonzero of in_proj_qkv, b, a, gate, up, down, plus 4 B x the
    fraction of layer-steps with output x (in_proj_z + out_proj nonzeros), plus 16 B per live
    conv channel (window read + write), plus 4 B per head nonzero, plus the 2 B x hidden
    embedding row. (The recurrent-state term is left out: at ~2 % activity it is < 1 %.)"""
    import numpy as np

    tot = 0.0
    w1 = np.float32(1.0) + np.asarray(model.norm, np.float32)
    for ly in model.layers:
        tot += 4 * (ly.in_proj_qkv.nnz + ly.in_proj_b.nnz + ly.in_proj_a.nnz +
                    ly.gate_proj.nnz + ly.up_proj.nnz + ly.down_proj.nnz)
        tot += 4 * f_out * (ly.in_proj_z.nnz + ly.out_proj.nnz)
        live = int((np.asarray(ly.conv1d) != 0).any(1).sum())
        tot += 16 * live
    hk = np.nonzero(w1 != 0)[0]
    mask = np.zeros(model.dims.hidden, bool)
    mask[hk] = True
    tot += 4 * int(mask[model.embed.cols].sum())
    tot += 2 * model.dims.hidden
    return tot


def measured_traffic(config: str, kind: str = "decode", key: str = "hbm_bytes_per_token"):
    """HBM bytes per unit (a decoded token, a prefill position) of a path, from the committed
    rocprofv3 counter summary (profiles/pmc_lxm_<kind>_<config>.txt: FETCH_SIZE and WRITE_SIZE
    per dispatch, each scaled by the same counter's reading for a plain copy of known size), or
    None."""
    path = os.path.join(HERE, "profiles", f"pmc_lxm_{kind}_{config}.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith(key + ":"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(model, conv0, rec0, start: int, n: int):
    """The C oracle (a single-threaded port of the stock decode) on the first n tokens."""
    from oracle import oracle as ox

    ox.build()
    om = ox.OracleModel(model)
    c, r = conv0.copy(), rec0.copy()
    om.decode(c, r, [start], 2)  # warm-up (page-in)
    c, r = conv0.copy(), rec0.copy()
    t = time.perf_counter()
    preds, _, _ = om.decode(c, r, [start], n)
    dt = time.perf_counter() - t
    return n / dt, preds


# The fastest grid-wide synchronisation measured on MI355X: 256 workgroups (one per CU) arriving
# on eight per-XCD counter copies whose sum the waiters poll, 1.6 us per barrier.
T_BAR_US = 1.6


def latency_roofline(n_layers: int, us_per_token: float) -> dict:
    """The decode's latency term: a token's dependent chain is two phases per layer (the GDN, then
    the MLP that reads its residual) and the head, and with the rarely-writing GDN phases paired
    with their MLP about n_layers + 1 grid-wide synchronisations; at the measured barrier cost
    that bounds a design that syncs the grid per phase. This kernel runs the chain on one
    workgroup instead and syncs across workgroups only for the head and GDN events."""
    p = n_layers + 1
    t = p * T_BAR_US
    return {"dependent_syncs_per_token": p, "t_bar_us": T_BAR_US, "t_roof_us": round(t, 1),
            "t_measured_us": round(us_per_token, 2), "frac": round(t / us_per_token, 4)}


def prefill_leg(calls: int, T: int, cpu_tokens: int) -> dict:
    """verified-mode calls of T seeded uniform tokens; tok/s over the timed
    calls (HIP events around each call on the current stream, inputs resident)."""
    import numpy as np
    import torch

    from linuxformer_amd import fast, synth

    spec = synth.config3()
    t0 = time.time()
    model = synth.build(spec)
    conv0, rec0 = synth.init_state(model)
    f = fast.Fast(model)
    dev = torch.device("cuda", 0)
    cache = fast.StateCache(conv0, rec0, model.dims.dtype, dev)
    pf = f.prefill(dev)
    d = model.dims
    log(f"[bench] c3: built and packed in {time.time() - t0:.1f}s; {json.dumps({k: v for k, v in pf.stats.items() if not isinstance(v, list)})}")
    stream = torch.cuda.current_stream(dev)
    first = synth.tokens(spec, T, 0)
    p0 = pf.verify(first, cache).cpu().numpy()  # warm-up calls (the first is the parity sample)
    cand = pf.count.cpu().numpy()[:d.n_layers].astype(np.int64)
    pf.verify(synth.tokens(spec, T, 1000), cache)
    torch.cuda.synchronize()
    ms = []
    for k in range(calls):
        toks = synth.tokens(spec, T, 1 + k)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        pf.verify(toks, cache)
        e1.record(stream)
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
        nc = int(pf.count[:d.n_layers].sum())
        log(f"[bench] verified-prefill call {k + 1}/{calls}: {T} tokens in {ms[-1]:.2f} ms "
            f"({nc} candidate positions over the layers)")
    call_ms = sum(ms) / len(ms)
    # algorithmic bytes per position: the residual read and written per layer (bf16), the head's
    # normed input, and each value-head slot's state read and written once per layer per call
    slots = sum(int(pf.layers_h[L].n_vs) for L in range(d.n_layers))
    esz = 2 if d.dtype == "bf16" else 4
    b_pos = d.n_layers * 2 * esz * d.hidden + 2 * esz * d.hidden + 2 * 4 * 256 * 128 * slots / T
    achieved = b_pos * T / (call_ms * 1e-3) / 1e9
    t_pos = measured_traffic("c3", "prefill", "hbm_bytes_per_position")
    out = {"metric": "verified prefill tok/s, 37-layer sparse chip stack, 1 MI355X",
           "value": round(T / (call_ms * 1e-3), 1), "unit": "tok/s", "calls": calls,
           "ms_per_call": round(call_ms, 3), "call_ms": [round(x, 2) for x in ms],
           "tokens_per_call": T,
           "config": {"workload": f"c3: verified mode over the c2 stack, {T} seeded uniform tokens "
                                  f"per call, p_gate {spec.p_gate}",
                      "candidates_per_layer": round(float(cand.mean()), 1),
                      "value_head_slots": slots},
           "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5),
                        "bytes_per_position": round(b_pos),
                        "traffic": None if t_pos is None else round(t_pos * T)}}
    if cpu_tokens > 0:
        from oracle import oracle as ox

        ox.build()
        om = ox.OracleModel(model)
        c, r = conv0.copy(), rec0.copy()
        t = time.perf_counter()
        po, _, _ = om.decode(c, r, [int(x) for x in first[:cpu_tokens]], cpu_tokens)
        dt = time.perf_counter() - t
        out["cpu_baseline"] = {"value": round(cpu_tokens / dt, 2), "unit": "tok/s", "cores": 1,
                               "kind": "port", "sample": f"the first {cpu_tokens} positions of "
                               "the warm-up call (C oracle's forced decode, one thread)"}
        out["check"] = {"oracle_positions": cpu_tokens,
                        "preds_match": bool(po.tolist() == p0[:cpu_tokens].tolist())}
    return out


def dense_cpu_tok_s(dm, n: int) -> float:
    """The dense stack's decode step restated with torch's eager ops in float32 on the host cores
    (weights copied from the GPU once; the stock forward's structure, not its bit order): tok/s
    over n greedy steps from a zero state. A reported baseline only."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    sp, d = dm.spec, dm.dims
    H, nk, kl, rl = sp.hidden, sp.nk, sp.kd_live, sp.r_live
    torch.set_num_threads(os.cpu_count() or 1)
    L = [{k: v.float().cpu() for k, v in ly.items()} for ly in dm.layers]
    E = dm.embed.float().cpu()
    wf = dm.norm.float().cpu()
    S = [torch.zeros(nk * rl, 256, 128) for _ in L]
    win = [torch.zeros(2 * nk * kl + nk * rl * 128, 4) for _ in L]

    def rms(x, w, eps):
        return (x * torch.rsqrt(x.pow(2).mean() + eps)) * (1.0 + w)

    tok = 0
    t = time.perf_counter()
    for _ in range(n):
        h = E[tok].clone()
        for i, ly in enumerate(L):
            x = rms(h, ly["ln_in"], sp.rms_eps)
            qk = ly["qk"].reshape(-1, H) @ x
            v = ly["v"].reshape(-1, H) @ x
            z = (ly["z"].reshape(-1, H) @ x).view(nk * rl, 128)
            b = ly["b"].reshape(-1, H) @ x
            a = ly["a"].reshape(-1, H) @ x
            P = torch.cat([qk, v])
            win[i] = torch.cat([win[i][:, 1:], P[:, None]], 1)
            taps = torch.cat([ly["conv_qk"].reshape(-1, 4), ly["conv_v"].reshape(-1, 4)])
            y = F.silu((win[i] * taps).sum(1))
            q = F.normalize(y[:nk * kl].view(nk, kl), dim=-1).repeat_interleave(rl, 0) / 16.0
            k = F.normalize(y[nk * kl:2 * nk * kl].view(nk, kl), dim=-1).repeat_interleave(rl, 0)
            vv = y[2 * nk * kl:].view(nk * rl, 128)
            R = d.nv // nk
            vh = torch.tensor([kh * R + r for kh in range(nk) for r in range(rl)])
            g = torch.exp(-torch.exp(ly["A_log"][vh]) * F.softplus(a + ly["dt_bias"][vh]))
            St = S[i][:, :kl] * g[:, None, None]
            kv = (St * k[:, :, None]).sum(1)
            St = St + k[:, :, None] * ((vv - kv) * torch.sigmoid(b)[:, None])[:, None, :]
            S[i][:, :kl] = St
            o = (St * q[:, :, None]).sum(1)
            on = (o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + sp.gated_eps)) * ly["norm"] * F.silu(z)
            h = h + ly["out"].reshape(H, -1) @ on.reshape(-1)
            xm = rms(h, ly["ln_post"], sp.rms_eps)
            h = h + ly["down"] @ (F.silu(ly["gate"] @ xm) * (ly["up"] @ xm))
        tok = int(torch.argmax(E @ rms(h, wf, sp.rms_eps)))
    return n / (time.perf_counter() - t)


def dense_leg(n_prefill: int, n_steps: int, cpu_tokens: int, graph: bool = True,
              persistent: bool = True, batched: bool = True) -> dict:
    """the dense padded text-view stack; a prompt of n_prefill seeded uniform
    tokens from a zero state (batched: lxm_dn_prefill over all but the last, then one step;
    else n_prefill forced steps), then n_steps greedy steps, timed (HIP events on the stream)."""
    import numpy as np
    import torch

    from linuxformer_amd import dense, fast, synth

    spec = synth.config4()
    t0 = time.time()
    dm = synth.build_dense(spec, "cuda")
    d = dm.dims
    conv0 = np.zeros((d.n_layers, d.n_conv, 4), np.float32)
    rec0 = np.zeros((d.n_layers, d.nv, 256, 128), np.float32)
    cache = fast.StateCache(conv0, rec0, "bf16", torch.device("cuda", 0))
    dd = dense.DenseDecode(dm, cache, max_steps=max(n_prefill, n_steps) + 1)
    torch.cuda.synchronize()
    log(f"[bench] c4: built in {time.time() - t0:.1f}s")
    toks = np.random.default_rng(spec.seed).integers(0, spec.vocab, n_prefill).tolist()
    t = time.perf_counter()
    if batched:
        dd.prefill(toks[:-1])  # lxm_dn_prefill: the same states as forced steps, bit for bit
        p1 = dd.run(toks[-1:], 1, graph=graph)
    else:
        p1 = dd.run(toks, n_prefill, graph=graph)
    pre_s = time.perf_counter() - t
    log(f"[bench] c4: prefill of {n_prefill} tokens in {pre_s:.2f}s "
        f"({'batched, then one step' if batched else 'forced steps'})")
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    p2 = dd.run([p1[-1]], n_steps, graph=graph)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    # the same steps as one persistent launch (lxm_dn_run), timed the same way
    n_per = max(1, n_steps // 4)
    ms_per = None
    if persistent:
        e2, e3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e2.record(stream)
        dd.run([p2[-1]], n_per, mode="persistent")
        e3.record(stream)
        torch.cuda.synchronize()
        ms_per = e2.elapsed_time(e3)
    H, I, nk, kl, rl = spec.hidden, spec.inter, spec.nk, spec.kd_live, spec.r_live
    nvr = nk * rl * 128
    w_layer = 2 * ((2 * nk * kl + 2 * nvr + 2 * nk * rl) * H + H * nvr + 3 * I * H)
    state = 2 * nk * rl * 256 * 128 * 4
    b_tok = d.n_layers * (w_layer + state) + 2 * spec.vocab * H
    pad_layer = 2 * ((2 * nk * 256 + 2 * d.nv * 128 + 2 * d.nv) * H + H * d.nv * 128 + 3 * I * H)
    achieved = b_tok * n_steps / (ms * 1e-3) / 1e9
    t_tok = measured_traffic("c4", "dense")
    # fused multiply-adds per prompt token: every live weight of every layer once
    fma_tok = d.n_layers * ((2 * nk * kl + 2 * nvr + 2 * nk * rl) * H + H * nvr + 3 * I * H)
    out = {"metric": "dense padded decode tok/s, 24-layer text-view stack, 1 MI355X",
           "value": round(n_steps / (ms * 1e-3), 1), "unit": "tok/s",
           "ms_per_token": round(ms / n_steps, 4), "steps": n_steps,
           "prefill": {"tokens": n_prefill, "s": round(pre_s, 2),
                       "tok_s": round(n_prefill / pre_s, 1),
                       "mode": "lxm_dn_prefill (batches of 16) + one step" if batched
                               else "forced steps",
                       # the prompt's row sums are fp32 fused ops on the VALU (bf16 x bf16
                       # products, summed in the decode's order); packed fp32 is not used, so
                       # the vector rate available is half the published fp32 peak
                       "roofline": {"bound": "valu", "achieved": round(2 * fma_tok * n_prefill / pre_s / 1e12, 2),
                                    "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                                    "frac": round(2 * fma_tok * n_prefill / pre_s / 1e12 / FP32_PEAK_TFLOPS, 4),
                                    "flops_per_token": 2 * fma_tok}},
           "config": {"workload": "c4: 24 layers, hidden 2560, 16 key heads (256, 128 live), 128 "
                                  "value heads (2 live per key head), SwiGLU 9216, vocab 248,320, "
                                  "bf16 N(0, 0.02); zero state"},
           "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                        "bytes_per_token": b_tok,
                        "traffic": None if t_tok is None else round(t_tok * n_steps),
                        "padded_bytes_per_token": d.n_layers * (pad_layer + state) + 2 * spec.vocab * H},
           "distinct_predictions": len(set(p2)),
           "persistent": None if ms_per is None else
                         {"steps": n_per, "tok_s": round(n_per / (ms_per * 1e-3), 1),
                          "note": "lxm_dn_run, continuing from the greedy run's states"}}
    if cpu_tokens > 0:
        out["cpu_baseline"] = {"value": round(dense_cpu_tok_s(dm, cpu_tokens), 3), "unit": "tok/s",
                               "cores": os.cpu_count(), "kind": "port",
                               "sample": f"{cpu_tokens} greedy steps from a zero state, torch eager "
                                         "float32 on the host"}
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--tokens", type=int, default=262_144)
    ap.add_argument("--warmup-tokens", type=int, default=4096)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c5", "small"])
    ap.add_argument("--cpu-tokens", type=int, default=256, help="CPU baseline sample (0: skip)")
    ap.add_argument("--legs", default="decode,prefill,dense",
                    help="comma-separated: decode (config 2), prefill (config 3), dense (config 4)")
    ap.add_argument("--pf-calls", type=int, default=5)
    ap.add_argument("--pf-tokens", type=int, default=65_536)
    ap.add_argument("--pf-cpu-tokens", type=int, default=48)
    ap.add_argument("--dn-prefill", type=int, default=8192)
    ap.add_argument("--dn-steps", type=int, default=4096)
    ap.add_argument("--dn-cpu-tokens", type=int, default=4)
    ap.add_argument("--dn-graph", type=int, default=1,
                    help="1: the dense steps replayed from a captured graph; 0: launched eagerly")
    ap.add_argument("--dn-batched", type=int, default=1,
                    help="config 4's prompt through lxm_dn_prefill (0: as forced steps)")
    ap.add_argument("--dn-persistent", type=int, default=1,
                    help="1: also time the persistent run (lxm_dn_run); 0: skip it")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the decode is one sequential chain per stream and this "
              f"build runs on a single MI355X (asked for --gpus {args.gpus}).", file=sys.stderr)
        return 2

    legs = set(args.legs.split(","))
    if "decode" not in legs:
        out = {}
        if "prefill" in legs:
            out["verified_prefill"] = prefill_leg(args.pf_calls, args.pf_tokens, args.pf_cpu_tokens)
        if "dense" in legs:
            out["dense_decode"] = dense_leg(args.dn_prefill, args.dn_steps, args.dn_cpu_tokens,
                                            bool(args.dn_graph), bool(args.dn_persistent), bool(args.dn_batched))
        print(json.dumps(out), flush=True)
        return 0

    import numpy as np
    import torch

    from linuxformer_amd import fast, mega, synth

    spec = {"c1": synth.config1(), "c2": synth.config2(), "c5": synth.config5(),
            "small": synth.small()}[args.config]
    t0 = time.time()
    model = synth.build(spec)
    conv0, rec0 = synth.init_state(model)
    start = synth.start_token(spec)
    f = fast.Fast(model)
    dev = torch.device("cuda", 0)
    cache = fast.StateCache(conv0, rec0, model.dims.dtype, dev)
    mg = mega.Mega(f, model, cache, 0)
    torch.cuda.synchronize()
    log(f"[bench] {spec.name}: built and packed in {time.time() - t0:.1f}s; "
        f"{json.dumps({k: v for k, v in mg.stats.items() if not isinstance(v, list)})}")

    stream = torch.cuda.current_stream(dev)
    # warm-up launches continue the stream from the start token; their first predictions are
    # checked against the CPU oracle below
    tok = start
    first_preds = None
    for w in range(args.warmup):
        preds = mg.run([tok], args.warmup_tokens)
        if first_preds is None:
            first_preds = preds
        tok = preds[-1]
        log(f"[bench] warm-up launch {w + 1}/{args.warmup}: {args.warmup_tokens} tokens")
    torch.cuda.synchronize()
    # timed: K launches of T tokens, events on the launch stream around each
    evs = []
    t_start = time.perf_counter()
    for k in range(args.steps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        preds = mg.run([tok], args.tokens)
        e1.record(stream)
        evs.append((e0, e1))
        tok = preds[-1]
        log(f"[bench] timed launch {k + 1}/{args.steps}: {args.tokens} tokens, "
            f"distinct predictions {len(set(preds))}")
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    kern_ms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
    n_tok = args.steps * args.tokens
    value = n_tok / wall
    # roofline: SURVEY 8(d)'s algorithmic bytes per token x tokens per launch / launch time
    b_tok = survey_bytes_per_token(model, spec.p_gate)
    achieved = b_tok * args.tokens / (kern_ms * 1e-3) / 1e9
    t_tok = measured_traffic(spec.name)
    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall * 1e3 / args.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16" if model.dims.dtype == "bf16" else "fp32",
        "data": "synthetic (seeded config stack, random weights and state; no checkpoint)",
        "config": {"workload": f"{spec.name}: {model.dims.n_layers}-layer synthetic sparse chip stack, "
                               f"hidden {model.dims.hidden}, vocab {model.dims.vocab}, greedy decode "
                               f"chunks of {args.tokens} tokens at batch 1",
                   "tokens_per_step": args.tokens, "batch": 1, "p_gate": spec.p_gate,
                   "density": spec.density, "parallelism": "single GPU (one chain workgroup + "
                   f"{mg.ncta - 1} head workgroups)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5),
                     "traffic": None if t_tok is None else round(t_tok * args.tokens),
                     "bytes_per_token": round(b_tok), "kernel_ms_per_launch": round(kern_ms, 3)},
        "latency_roofline": latency_roofline(model.dims.n_layers, kern_ms * 1e3 / args.tokens),
    }
    if args.cpu_tokens > 0:
        cps, cpreds = cpu_baseline(model, conv0, rec0, start, args.cpu_tokens)
        m = min(len(cpreds), len(first_preds or []))
        match = bool(m > 0 and list(cpreds[:m]) == list(first_preds[:m]))
        out["cpu_baseline"] = {"value": round(cps, 2), "unit": "tok/s", "cores": 1, "kind": "port",
                               "sample": f"first {args.cpu_tokens} tokens of the {spec.name} stream "
                                         f"(C oracle, one thread)"}
        out["check"] = {"oracle_tokens": m, "preds_match": match}
    if "prefill" in legs:
        del mg, cache
        torch.cuda.empty_cache()
        out["verified_prefill"] = prefill_leg(args.pf_calls, args.pf_tokens, args.pf_cpu_tokens)
    if "dense" in legs:
        torch.cuda.empty_cache()
        out["dense_decode"] = dense_leg(args.dn_prefill, args.dn_steps, args.dn_cpu_tokens,
                                        bool(args.dn_graph), bool(args.dn_persistent), bool(args.dn_batched))
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
