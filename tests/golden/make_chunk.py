"""Write tests/golden/c2_chunk.json (or c5_run.json): the CPU oracle's run of a whole greedy chunk.

Config 2: one 262,144-token greedy chunk of the 37-layer synthetic stack
(linuxformer_amd.synth.config2); config 5 (--config c5): the same stack with half of the
layer-steps gated, 65,536 greedy tokens (benchmark config 5's run). Each starts from its config's
start token and initial state and is decoded by the C oracle (oracle/lx_oracle.c, the stock
decode restated). The fixture holds the sha256 of the prediction stream (int32, little-endian),
of the final conv windows and of the final recurrent states (float32, the stacked (L, C, 4) and
(L, nv, 256, 128) arrays; the states with every zero made +0), and the stream's first
predictions. The GPU test and bench.py compare
the decode kernel's chunk against it (the reference pins its boot the same way:
lx/tools/mega_boot.py:74-75, lx/results/mega_boot.json's stream_sha256).

    OMP_NUM_THREADS=8 python tests/golden/make_chunk.py [--config c2|c5] [--chunk N] [--ckpt DIR]

About 1-2 hours on 8 host threads for config 2, about 35 minutes for config 5. With --ckpt the run saves its progress every piece and resumes
from it.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from linuxformer_amd import synth  # noqa: E402
from oracle import oracle as ox  # noqa: E402


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", choices=("c2", "c5"), default="c2")
    ap.add_argument("--chunk", type=int, default=None, help="tokens (default: the config's run)")
    ap.add_argument("--piece", type=int, default=4096)
    ap.add_argument("--ckpt", default=None, help="directory for resumable progress")
    ap.add_argument("--out", default=None)
    args = ap.parse_args()

    spec = synth.config2() if args.config == "c2" else synth.config5()
    if args.chunk is None:
        args.chunk = spec.n_steps
    if args.out is None:
        args.out = os.path.join(HERE, "c2_chunk.json" if args.config == "c2" else "c5_run.json")
    model = synth.build(spec)
    conv, rec = synth.init_state(model)
    start = synth.start_token(spec)
    ox.build()
    om = ox.OracleModel(model)
    preds = np.zeros(0, np.int32)
    if args.ckpt:
        os.makedirs(args.ckpt, exist_ok=True)
        f = os.path.join(args.ckpt, "progress.npz")
        if os.path.exists(f):
            z = np.load(f)
            preds, conv, rec = z["preds"], z["conv"].copy(), z["rec"].copy()
            print(f"resumed at {len(preds)} tokens", flush=True)
    t0 = time.time()
    while len(preds) < args.chunk:
        tok = start if len(preds) == 0 else int(preds[-1])
        n = min(args.piece, args.chunk - len(preds))
        p, _, _ = om.decode(conv, rec, [tok], n)
        preds = np.concatenate([preds, p])
        el = time.time() - t0
        print(f"{len(preds)}/{args.chunk} tokens, {el:.0f}s", flush=True)
        if args.ckpt:
            tmp = os.path.join(args.ckpt, "progress.tmp.npz")
            np.savez(tmp, preds=preds, conv=conv, rec=rec)
            os.replace(tmp, os.path.join(args.ckpt, "progress.npz"))
    out = {"config": spec.name, "chunk": args.chunk, "start": start,
           "stream_sha256": hashlib.sha256(preds.astype("<i4").tobytes()).hexdigest(),
           "conv_sha256": hashlib.sha256(np.ascontiguousarray(conv, np.float32).tobytes()).hexdigest(),
           # the sign of a zero state entry is not compared (the reference's x.ne(y),
           # lx/tests/check_mega.py:34-36): x + 0 makes every zero +0
           "rec_sha256": hashlib.sha256((np.ascontiguousarray(rec, np.float32)
                                         + np.float32(0.0)).tobytes()).hexdigest(),
           "distinct_predictions": int(len(np.unique(preds))),
           "first_preds": preds[:256].tolist(), "last_preds": preds[-16:].tolist(),
           "writer": "oracle/lx_oracle.c (ox_decode) via tests/golden/make_chunk.py"}
    with open(args.out, "w") as fh:
        json.dump(out, fh, indent=1)
    print(json.dumps({k: v for k, v in out.items() if "preds" not in k}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
