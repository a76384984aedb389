"""Build and load the native library (lx/lx/mk_build.py's role: nvcc + ctypes there, hipcc for
gfx950 here). The library is built in-tree, so it travels with the repository to the GPU box;
loading never compiles, and a missing library is an error, never a fallback."""

from __future__ import annotations

import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "_lib")
LIB = os.path.join(LIBDIR, "liblxm.so")
# the same kernel with the per-wave sub-phase counters (-DLXM_SUBPROF; lx.mega's MK_SUBPROF build)
LIB_SUBPROF = os.path.join(LIBDIR, "liblxm_subprof.so")
RUNNER = os.path.join(LIBDIR, "lxm_runner")
SOURCES = ["lxm_decode.hip", "lxm_prefill.hip", "lxm_dense.hip", "lxm_chunk.hip", "lxm_probe.hip"]
HEADERS = ["lxm_math.h", os.path.join("..", "..", "include", "lxm.h"),
           os.path.join("..", "..", "include", "lxm_prefill.h"),
           os.path.join("..", "..", "include", "lxm_dense.h"),
           os.path.join("..", "..", "include", "lxm_chunk.h")]
# -ffp-contract=off: no a*b+c is fused (the rounding contract); packed fp32 ops disabled
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if c and (os.path.isabs(c) and os.path.exists(c) or not os.path.isabs(c)):
            return c
    return "hipcc"


def _compile(out: str, extra: list, verbose: bool) -> None:
    tmp = out + ".tmp"
    cmd = [hipcc(), *FLAGS, *extra, "-o", tmp, *[os.path.join(CSRC, s) for s in SOURCES]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{r.stderr[-4000:]}")
    if verbose and r.stderr:
        print(r.stderr)
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    """Compile the library (and its sub-phase profiling twin) for gfx950 (always compiles)."""
    os.makedirs(LIBDIR, exist_ok=True)
    from concurrent.futures import ThreadPoolExecutor

    with ThreadPoolExecutor(2) as ex:
        for f in [ex.submit(_compile, LIB, [], verbose),
                  ex.submit(_compile, LIB_SUBPROF, ["-DLXM_SUBPROF"], verbose)]:
            f.result()
    # the runner has a kernel of its own (the copy that calibrates the byte counters): gfx950
    r = subprocess.run([hipcc(), "--offload-arch=gfx950", "-O2", "-std=c++17", "-Xclang",
                        "-target-feature", "-Xclang", "-packed-fp32-ops", "-o", RUNNER + ".tmp",
                        os.path.join(CSRC, "lxm_runner.cpp"), "-ldl"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc (runner) failed ({r.returncode}):\n{r.stderr[-4000:]}")
    os.replace(RUNNER + ".tmp", RUNNER)
    return LIB


_libs = {}
# cooperative launches this process has made (lxm_run, lxm_run_noalloc, lxm_dn_run, lxm_t_sync):
# on the GPU boxes a cooperative launch from another process is refused (hipErrorIllegalState)
# while one that has made them holds the device
cooperative_launches = 0


def note_cooperative() -> None:
    global cooperative_launches
    cooperative_launches += 1


def load(subprof: bool = False) -> ctypes.CDLL:
    """The built library (ctypes), or its sub-phase profiling twin. Raises if it has not been
    built."""
    path = LIB_SUBPROF if subprof else LIB
    if path not in _libs:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run linuxformer_amd.mk_build.build() (or "
                               "__graft_entry__.build()) first")
        lib = ctypes.CDLL(path)
        P, I = ctypes.c_void_p, ctypes.c_int
        lib.lxm_run.argtypes = [P, P, I, I, P]
        lib.lxm_run.restype = I
        lib.lxm_run_noalloc.argtypes = [P, I, I, P]
        lib.lxm_run_noalloc.restype = I
        for n in ("lxm_lds_base", "lxm_max_lds", "lxm_last_error", "lxm_device_cus"):
            getattr(lib, n).restype = I
            getattr(lib, n).argtypes = []
        lib.lxm_max_blocks.argtypes = [I]
        lib.lxm_max_blocks.restype = I
        lib.lxm_t_elem.argtypes = [I, P, P, ctypes.c_long, P]
        lib.lxm_t_elem.restype = I
        lib.lxm_t_sum.argtypes = [I, P, I, I, P, P]
        lib.lxm_t_sum.restype = I
        lib.lxm_helper_lds.argtypes = [I]
        lib.lxm_helper_lds.restype = I
        for n in ("lxm_pf_head", "lxm_pf_embed"):
            getattr(lib, n).argtypes = [P, P, P]
            getattr(lib, n).restype = I
        lib.lxm_pf_layers.argtypes = [P, P, I, I, P]
        lib.lxm_pf_layers.restype = I
        lib.lxm_pf_tiles.argtypes = [P, P, P, I, P]
        lib.lxm_pf_tiles.restype = I
        lib.lxm_pf_lds.argtypes = [I, I, I]
        lib.lxm_pf_lds.restype = I
        lib.lxm_dn_step.argtypes = [P, P, P]
        lib.lxm_dn_step.restype = I
        lib.lxm_dn_run.argtypes = [P, P, I, P]
        lib.lxm_dn_run.restype = I
        lib.lxm_dn_prefill.argtypes = [P, P, I, P, P]
        lib.lxm_dn_prefill.restype = I
        lib.lxm_dn_prefill_chunked.argtypes = [P, P, I, P, P]
        lib.lxm_dn_prefill_chunked.restype = I
        lib.lxm_gdn_chunk.argtypes = [P, P]
        lib.lxm_gdn_chunk.restype = I
        lib.lxm_t_sync.argtypes = [I, I, I, I, P, P, P, P]
        lib.lxm_t_sync.restype = I
        _libs[path] = lib
    return _libs[path]


EXPORTS = ("lxm_run", "lxm_lds_base", "lxm_helper_lds", "lxm_max_blocks", "lxm_max_lds",
           "lxm_last_error", "lxm_device_cus", "lxm_t_elem", "lxm_t_sum", "lxm_pf_layers",
           "lxm_pf_head", "lxm_pf_embed", "lxm_pf_tiles", "lxm_pf_lds", "lxm_dn_step", "lxm_dn_run",
           "lxm_dn_prefill", "lxm_t_sync", "lxm_run_noalloc", "lxm_gdn_chunk",
           "lxm_dn_prefill_chunked")
