"""The stock forward's chunked delta rule on the matrix cores (csrc/lxm_chunk.hip, C ABI
include/lxm_chunk.h): torch_chunk_gated_delta_rule (transformers qwen3_5 :249-327; the reference's
fla chunk_gated_delta_rule call, lx/lx/fast.py:342-345) for value heads over T positions, in
chunks of 64 from position 0, the state carried from chunk to chunk.

    o = gated_delta_chunked(q, k, v, g, beta, S)   # S updated in place
"""

from __future__ import annotations

import ctypes

import torch

from . import mk_build

CHUNK = 64


class ChunkIO(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("q", "k", "v", "beta", "g", "S", "o")] + \
        [(n, ctypes.c_int64) for n in ("qk_ts", "qk_hs", "v_ts", "g_ts", "g_hs", "gl_ts", "o_ts")] + \
        [(n, ctypes.c_int32) for n in ("n", "n_slots", "rl", "rfull", "kl", "o_bf16")]


@torch.no_grad()
def gated_delta_chunked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                        beta: torch.Tensor, S: torch.Tensor, kl: int = 128,
                        o_bf16: bool = False) -> torch.Tensor:
    """q, k (T, nk, 256) float32 (l2-normed; q already times 1/16), v (T, nv, 128), g (T, nv) log
    decays, beta (T, nv), S (nv, 256, 128) float32 updated in place (value head h reads key head
    h // (nv // nk)). Only the first kl key dims may be nonzero. Returns o (T, nv, 128) float32."""
    lib = mk_build.load()
    T, nk, K = q.shape
    nv = v.shape[1]
    assert K == 256 and v.shape == (T, nv, 128) and k.shape == q.shape
    assert g.shape == (T, nv) and beta.shape == (T, nv) and S.shape == (nv, 256, 128)
    assert nv % nk == 0 and 0 < kl <= 128 and kl % 16 == 0
    for t in (q, k, v, g, beta, S):
        assert t.dtype == torch.float32 and t.is_contiguous() and t.is_cuda
    o = torch.zeros(T, nv, 128, dtype=torch.float32, device=q.device)
    st = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
    for c0 in range(0, T, CHUNK):
        n = min(CHUNK, T - c0)
        io = ChunkIO(q=q[c0].data_ptr(), k=k[c0].data_ptr(), v=v[c0].data_ptr(),
                     beta=beta[c0].data_ptr(), g=g[c0].data_ptr(), S=S.data_ptr(),
                     o=o[c0].data_ptr(), qk_ts=nk * 256, qk_hs=256, v_ts=nv * 128, g_ts=nv,
                     g_hs=1, gl_ts=nv, o_ts=nv * 128, n=n, n_slots=nv, rl=nv // nk,
                     rfull=nv // nk, kl=kl, o_bf16=int(o_bf16))
        e = lib.lxm_gdn_chunk(ctypes.byref(io), st)
        if e:
            raise RuntimeError(f"lxm_gdn_chunk failed: hipError {e}")
    return o
