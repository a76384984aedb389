"""Pack a configuration and write it for the native runner (csrc/lxm_runner.cpp):

    python -m linuxformer_amd.dump --config c2 --out /tmp/lxm_c2 --tokens 262144
    linuxformer_amd/_lib/lxm_runner /tmp/lxm_c2 <launches> [tokens]

The runner replays the decode through the C ABI without Python (the process rocprofv3 traces)."""

import argparse
import sys

import torch

from . import fast, mega, synth


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c5", "small"])
    ap.add_argument("--out", required=True)
    ap.add_argument("--tokens", type=int, default=262_144)
    ap.add_argument("--prof", action="store_true")
    a = ap.parse_args()
    spec = {"c1": synth.config1(), "c2": synth.config2(), "c5": synth.config5(),
            "small": synth.small()}[a.config]
    m = synth.build(spec)
    conv0, rec0 = synth.init_state(m)
    cache = fast.StateCache(conv0, rec0, m.dims.dtype, torch.device("cuda", 0))
    mg = mega.Mega(fast.Fast(m), m, cache, 0)
    mg.dump(a.out, [synth.start_token(spec)], a.tokens, prof=a.prof)
    print(f"dumped {a.config} to {a.out}", file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
