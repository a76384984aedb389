"""The chunked delta rule on the matrix cores (lxm_gdn_chunk) against the oracle's restatement of
torch_chunk_gated_delta_rule, on an MI355X, through the C ABI.

Random regime: outputs and final states within 2e-6 of each head's largest magnitude (the MFMA
tiles and the blocked triangular inverse sum in their own orders; the oracle itself is within 1e-6
of transformers' function, tests/test_oracle.py). Exact regime (one-hot keys and queries, beta in
{0, 1}, no decay, dyadic values): bit for bit. Sequences of one partial chunk, whole chunks and a
ragged tail; several key heads with several value heads each.
"""

import numpy as np
import pytest
import torch

from linuxformer_amd import mk_build
from linuxformer_amd.chunk import gated_delta_chunked

pytestmark = pytest.mark.gpu

TOL = 2e-6


@pytest.fixture(scope="module")
def cuda():
    assert torch.cuda.is_available(), "the gpu tests need an MI355X"
    mk_build.load()
    return torch.device("cuda", 0)


def _inputs(T, nk, R, seed, exact=False):
    from golden.make_golden import chunk_inputs

    nv = nk * R
    q = np.zeros((T, nk, 256), np.float32)
    k = np.zeros((T, nk, 256), np.float32)
    v = np.zeros((T, nv, 128), np.float32)
    g = np.zeros((T, nv), np.float32)
    beta = np.zeros((T, nv), np.float32)
    S = np.zeros((nv, 256, 128), np.float32)
    for kh in range(nk):
        qi, ki, _, _, _, _ = chunk_inputs(T, seed + 100 * kh, exact)
        q[:, kh], k[:, kh] = qi, ki
    for vh in range(nv):
        _, _, vi, gi, bi, Si = chunk_inputs(T, seed + 7 * vh + 1, exact)
        v[:, vh], g[:, vh], beta[:, vh], S[vh] = vi, gi, bi, Si
    return q, k, v, g, beta, S


def _oracle(q, k, v, g, beta, S, R):
    from oracle import oracle as ox

    T, nv = v.shape[0], v.shape[1]
    o = np.zeros((T, nv, 128), np.float32)
    S = S.copy()
    for vh in range(nv):
        Sv = np.ascontiguousarray(S[vh])
        o[:, vh] = ox.chunk_gdr(q[:, vh // R], k[:, vh // R], v[:, vh], g[:, vh], beta[:, vh], Sv, 64)
        S[vh] = Sv
    return o, S


def _run(cuda, q, k, v, g, beta, S):
    t = [torch.from_numpy(np.ascontiguousarray(a)).to(cuda) for a in (q, k, v, g, beta, S)]
    t[0] = t[0] * 0.0625  # the kernel takes the query already scaled by 1/sqrt(256)
    o = gated_delta_chunked(*t)
    torch.cuda.synchronize()
    return o.cpu().numpy(), t[5].cpu().numpy()


@pytest.mark.parametrize("T,nk,R", [(37, 1, 1), (64, 2, 2), (200, 4, 2), (130, 16, 2)])
def test_chunk_random_regime(cuda, T, nk, R):
    print(f"[gpu-test] chunk random T={T} nk={nk} R={R}", flush=True)
    q, k, v, g, beta, S = _inputs(T, nk, R, 3)
    o_ref, S_ref = _oracle(q, k, v, g, beta, S, R)
    o, Sg = _run(cuda, q, k, v, g, beta, S)
    for vh in range(nk * R):
        assert np.abs(o[:, vh] - o_ref[:, vh]).max() <= TOL * np.abs(o_ref[:, vh]).max()
        assert np.abs(Sg[vh] - S_ref[vh]).max() <= TOL * np.abs(S_ref[vh]).max()
    assert not Sg[:, 128:].any()


@pytest.mark.parametrize("T", [50, 192])
def test_chunk_exact_regime_bit_exact(cuda, T):
    print(f"[gpu-test] chunk exact T={T}", flush=True)
    q, k, v, g, beta, S = _inputs(T, 2, 2, 9, exact=True)
    o_ref, S_ref = _oracle(q, k, v, g, beta, S, 2)
    o, Sg = _run(cuda, q, k, v, g, beta, S)
    assert (o == o_ref).all()
    assert (Sg == S_ref).all()
    assert np.abs(o_ref).max() > 0
