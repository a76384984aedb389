"""Host-side pieces, no GPU: the seeded generator, the packer's tables (decoded back and compared
with the model's tensors), the C ABI's exports, bench.py's one-GPU contract."""

import ctypes
import hashlib
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from linuxformer_amd import fast, mega, mk_build, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def digest(m) -> str:
    h = hashlib.sha256()
    for ly in m.layers:
        for c in (ly.in_proj_qkv, ly.in_proj_z, ly.out_proj, ly.gate_proj, ly.up_proj, ly.down_proj):
            h.update(c.rows.tobytes())
            h.update(c.vals.tobytes())
        h.update(ly.conv1d.tobytes())
    h.update(m.embed.cols.tobytes())
    return h.hexdigest()


def test_generator_is_deterministic():
    assert digest(synth.build(synth.small())) == digest(synth.build(synth.small()))
    assert digest(synth.build(synth.small(seed=8))) != digest(synth.build(synth.small()))


def test_config2_shape_and_gates():
    spec = synth.config2()
    m = synth.build(spec)
    d = m.dims
    assert (d.hidden, d.n_layers, d.nk, d.kd, d.nv, d.vd, d.inter, d.vocab) == \
        (3572, 37, 16, 256, 128, 128, 1024, 459_982)
    ng = d.hidden - d.n_layers
    for L in (0, 17, 36):
        ly = m.layers[L]
        for c in (ly.in_proj_z, ly.out_proj, ly.gate_proj, ly.up_proj, ly.down_proj):
            assert abs(c.nnz / (c.shape[0] * c.shape[1] * ng / d.hidden) - 0.0008) < 2e-5
            assert set(np.unique(c.vals)) <= set(synth.VALS.tolist())
        # no projection writes a gate column; query/key/decay rows read only the layer's gate
        assert ly.out_proj.rows.max() < ng and ly.down_proj.rows.max() < ng
        qk = ly.in_proj_qkv.rows < 2 * d.nk * d.kd
        assert (ly.in_proj_qkv.cols[qk] == ng + L).all() and (ly.in_proj_a.cols == ng + L).all()
    gates = m.embed.cols >= ng
    per_tok = np.bincount(m.embed.rows[gates], minlength=d.vocab)
    assert (per_tok == 1).all()  # every token gates exactly one layer: 1/37 of layer-steps
    assert (np.bincount(m.embed.rows[~gates], minlength=d.vocab) == 3).all()
    c5 = synth.build(synth.config5())
    g5 = np.bincount(c5.embed.rows[c5.embed.cols >= ng], minlength=d.vocab)
    assert set(np.unique(g5)) == {18, 19} and abs(g5.mean() / 37 - 0.5) < 0.01


class _FakeLib:
    """The library calls the packer makes, answered as an MI355X would (no GPU needed)."""

    def lxm_device_cus(self):
        return 256

    def lxm_lds_base(self):
        return 141_000

    def lxm_max_lds(self):
        return 163_840

    def lxm_helper_lds(self, head_lds):
        return head_lds + 43_856

    def lxm_max_blocks(self, lds):
        return 256


@pytest.fixture
def packed(monkeypatch):
    monkeypatch.setattr(mk_build, "_lib", _FakeLib())

    def make(spec):
        m = synth.build(spec)
        return m, mega.Mega(fast.Fast(m), device="cpu")
    return make


def _ent(blob: bytes, off: int, i: int, scale: int = 4):
    """A packed e4 entry: (index, value); gather tables store the index as a byte offset."""
    w = int.from_bytes(blob[off + 4 * i:off + 4 * i + 4], "little")
    assert (w & 0xffff) % scale == 0
    return (w & 0xffff) // scale, np.uint32((w >> 16) << 16).view(np.float32)


def test_packer_tables_decode_to_the_model(packed):
    """Every packed MLP row, down row, gate row and head row decodes back to the model's
    tensors: same columns, same values, same order (ascending), nothing dropped."""
    m, mg = packed(synth.small())
    blob = bytes(mg.blob.numpy())
    descs = (mega.LayerDesc * m.dims.n_layers).from_buffer_copy(bytes(mg.layers_d.numpy()))
    for L, ly in enumerate(m.layers):
        base = descs[L].hot
        hot = mega.Hot.from_buffer_copy(blob[base:base + 64])
        assert hot.size <= mega.HOT_MAX
        units = mg.unit_order[L]  # the live units (lx/lx/fast.py:242-248), by row length
        assert sorted(units.tolist()) == sorted(np.asarray(fast.Fast(m).dec[L]["units"]).tolist())
        assert hot.n_units == len(units)
        meta = np.frombuffer(blob[base + hot.unit:base + hot.unit + 4 * hot.n_units], np.uint32)
        for j, u in enumerate(units):
            st, ng, nu = int(meta[j] & 0xffff), int((meta[j] >> 16) & 255), int(meta[j] >> 24)
            for rows, k0, cnt in ((ly.gate_proj, st, ng), (ly.up_proj, st + ng, nu)):
                sel = rows.rows == u
                got = [_ent(blob, base + hot.gu_ent, k0 + k) for k in range(cnt)]
                assert [c for c, _ in got] == rows.cols[sel].tolist()
                assert [float(v) for _, v in got] == rows.vals[sel].tolist()
        # down rows: units ascending, all of a row's live terms
        dptr = np.frombuffer(blob[base + hot.down_ptr:base + hot.down_ptr + 2 * (m.dims.hidden + 1)], np.uint16)
        uidx = {int(u): j for j, u in enumerate(units)}
        dn = ly.down_proj
        for i in range(m.dims.hidden):
            want = [(uidx[int(c)], float(v)) for c, v in zip(dn.cols[dn.rows == i], dn.vals[dn.rows == i])
                    if int(c) in uidx]
            got = [_ent(blob, base + hot.down_ent, k) for k in range(dptr[i], dptr[i + 1])]
            assert [(int(c), float(v)) for c, v in got] == want
        # out_proj by residual row over every value dim, ascending
        oc = ly.out_proj
        optr = np.frombuffer(blob[descs[L].out_ptr:descs[L].out_ptr + 4 * (m.dims.hidden + 1)], np.int32)
        for i in range(m.dims.hidden):
            sel = oc.rows == i
            order = np.argsort(oc.cols[sel], kind="stable")
            want = list(zip(oc.cols[sel][order].tolist(), oc.vals[sel][order].tolist()))
            got = [_ent(blob, descs[L].out_ent, k, 1) for k in range(optr[i], optr[i + 1])]
            assert [(int(c), float(v)) for c, v in got] == want
    # head: rows x columns with a nonzero final weight
    hptr = mg.head_ptr.numpy()
    hent = bytes(mg.head_ent.numpy())
    w1 = 1.0 + m.norm
    E = m.embed
    for v in (0, 7, m.dims.vocab - 1):
        want = [(int(c), float(x)) for c, x in zip(E.cols[E.rows == v], E.vals[E.rows == v]) if w1[c] != 0]
        got = [_ent(hent, 0, k) for k in range(hptr[v], hptr[v + 1])]
        assert [(int(c), float(x)) for c, x in got] == want


def test_packer_fits_every_config(packed):
    for spec in (synth.config1(), synth.config2()):
        m, mg = packed(spec)
        assert max(mg.stats["hot_bytes"]) <= mega.HOT_MAX
        assert mg.stats["qk_total"] <= mega.MAXQK
        assert mg.lds <= 163_840
        assert mg.e4  # every packed value is exact in bf16: 4-byte entries


def test_c_abi_exports_every_declared_symbol(native_lib):
    """The library loads and exports each entry point include/lxm.h declares (no GPU call)."""
    hdr = open(os.path.join(ROOT, "include", "lxm.h")).read()
    names = re.findall(r"^int (lxm_\w+)\(", hdr, re.M)
    assert len(names) >= 8
    lib = ctypes.CDLL(mk_build.LIB)
    for n in names:
        assert hasattr(lib, n), n
    assert set(mk_build.EXPORTS) <= set(names)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
