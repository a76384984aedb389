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

from linuxformer_amd import chain, fast, mega, mk_build, synth

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
    """The library calls the packer makes, answered as an MI355X would (no GPU needed): LDS
    sizes from the built library itself (pure functions), the device's shape from MI355X."""

    def __init__(self, real):
        self.real = real

    def lxm_device_cus(self):
        return 256

    def lxm_lds_base(self):
        return self.real.lxm_lds_base()

    def lxm_max_lds(self):
        return 163_840

    def lxm_helper_lds(self, head_lds):
        return self.real.lxm_helper_lds(head_lds)

    def lxm_max_blocks(self, lds):
        return 256 if lds <= 163_840 else 0


@pytest.fixture
def packed(monkeypatch, native_lib):
    fake = _FakeLib(native_lib)
    monkeypatch.setattr(mk_build, "load", lambda subprof=False: fake)

    def make(spec):
        m = synth.build(spec)
        return m, mega.Mega(fast.Fast(m), device="cpu")
    return make


def _ent(blob: bytes, off: int, i: int, scale: int = 4):
    """A packed e4 entry: (index, value); gather tables store the index as a byte offset."""
    w = int.from_bytes(blob[off + 4 * i:off + 4 * i + 4], "little")
    assert (w & 0xffff) % scale == 0
    return (w & 0xffff) // scale, np.uint32((w >> 16) << 16).view(np.float32)


def _slot_ent(S, s):
    """Entry at slot s of one lane's e4 slots: (index, value)."""
    w = int(S[s])
    assert (w & 0xffff) % 4 == 0
    return (w & 0xffff) // 4, float(np.uint32((w >> 16) << 16).view(np.float32))


def _chain_rows(mg, m, L, blob, desc):
    """The chain tables of layer L decoded as the kernel reads them: {act index: (gate entries,
    up entries)} and {row: down entries}, each an ordered list of (index, value) without the
    padding, plus the checks on the padding and on the wave-uniform bounds."""
    f = chain.fmt(mg.e4)
    assert f.e4
    S = chain.decode_ptt(f, blob[desc.ptt:desc.ptt + 16 * f.WORDS * chain.NT])
    g = mega.Gate.from_buffer_copy(blob[desc.gate:desc.gate + 64])
    a_u, a_r, a_e = desc.gate + g.long_u, desc.gate + g.long_r, desc.gate + g.long_ent
    lu = np.frombuffer(blob[a_u:a_u + 32 * g.n_long_u], np.int32).reshape(-1, 8)
    lr = np.frombuffer(blob[a_r:a_r + 16 * g.n_long_r], np.int32).reshape(-1, 4)
    units, rows = {}, {}

    def trim(lst, n):  # entries past the row's own are padding: index 0, value 0
        assert all(e == (0, 0.0) for e in lst[n:])
        return lst[:n]

    for lane in range(chain.NT):
        m0, m1, m2 = (int(x) for x in S[lane, f.MA:f.MA + 3])
        wave = S[(lane // 64) * 64:(lane // 64 + 1) * 64, f.MA + 2]
        assert (wave == m2).all()
        mb3 = int(S[lane, f.MB + 3])
        wave = S[(lane // 64) * 64:(lane // 64 + 1) * 64, f.MB + 3]
        assert ((wave >> 16) == (mb3 >> 16)).all()
        for p, base in ((0, f.U0), (1, f.U1)):
            if not (m0 >> (16 * p)) & 0x8000:
                continue
            k = (m0 >> (16 * p)) & 0xfff
            G = (m2 >> (4 * p)) & 15
            gl = [_slot_ent(S[lane], base + 2 * j) for j in range(G)]
            ul = [_slot_ent(S[lane], base + 2 * j + 1) for j in range(G)]
            if (m2 >> (8 + p)) & 1:  # shared columns: the up slots hold bare weights
                assert all(c == 0 for c, _ in ul)
                ul = [(gl[j][0] if ul[j] != (0, 0.0) else 0, ul[j][1]) for j in range(G)]
            ng = len(m.layers[L].gate_proj.cols[m.layers[L].gate_proj.rows == mg.unit_order[L][k]])
            nu = len(m.layers[L].up_proj.cols[m.layers[L].up_proj.rows == mg.unit_order[L][k]])
            if (m2 >> (8 + p)) & 1:  # shared columns
                assert [c for c, _ in gl] == [c for c, _ in ul]
            assert k not in units
            units[k] = (trim(gl, ng), trim(ul, nu))
        mask = (mb3 >> 16) & 255
        for q, ln in enumerate(f.DLEN):
            wo = (int(S[lane, f.MB + q // 2]) >> (16 * (q & 1))) & 0xffff
            if wo == 4 * 4096 + 4 * lane:  # the lane's dummy slot: no row in this pass
                continue
            assert wo % 4 == 0 and wo < 4 * m.dims.hidden
            row = wo // 4
            assert mask & (1 << q)
            ents = [_slot_ent(S[lane], f.D + f.doff[q] + j) for j in range(ln)]
            n = len(m.layers[L].down_proj.cols[m.layers[L].down_proj.rows == row])
            assert row not in rows
            rows[row] = [e for e in ents if e != (0, 0.0)]
        li, ri = m1 & 0xffff, mb3 & 0xffff
        if li != 0xffff:
            assert (m2 >> 10) & 1
            k, gs, gn, us, un = (int(x) for x in lu[li][:5])
            units[k] = ([_ent(blob, a_e, gs + j) for j in range(gn)],
                        [_ent(blob, a_e, us + j) for j in range(un)])
            units[k] = tuple([(int(c), float(v)) for c, v in r] for r in units[k])
        if ri != 0xffff:
            assert (mb3 >> 24) & 1
            row, st, n = (int(x) for x in lr[ri][:3])
            rows[row] = [(int(c), float(v)) for c, v in
                         (_ent(blob, a_e, st + j) for j in range(n))]
    return S, units, rows


def test_packer_tables_decode_to_the_model(packed):
    """Every packed MLP row, down row, gate row and head row decodes back to the model's
    tensors: same columns, same values, same order (ascending), nothing dropped; every table
    slot past a row is padding that adds +0."""
    for spec in (synth.small(), synth.config1()):
        m, mg = packed(spec)
        blob = bytes(mg.blob.numpy())
        descs = (mega.LayerDesc * m.dims.n_layers).from_buffer_copy(bytes(mg.layers_d.numpy()))
        H = m.dims.hidden
        for L, ly in enumerate(m.layers):
            S, units, rows = _chain_rows(mg, m, L, blob, descs[L])
            order = mg.unit_order[L]  # the live units (lx/lx/fast.py:242-248), model order
            assert order.tolist() == np.asarray(fast.Fast(m).dec[L]["units"]).tolist()
            assert sorted(units) == list(range(len(order)))
            for k, u in enumerate(order):
                for coo, got in ((ly.gate_proj, units[k][0]), (ly.up_proj, units[k][1])):
                    sel = coo.rows == u
                    assert [c for c, _ in got] == coo.cols[sel].tolist()
                    assert [v for _, v in got] == coo.vals[sel].tolist()
            # down rows: live units in the model's order, all of a row's live terms
            uidx = {int(u): j for j, u in enumerate(order)}
            dn = ly.down_proj
            for i in range(H):
                want = [(uidx[int(c)], float(v)) for c, v in
                        zip(dn.cols[dn.rows == i], dn.vals[dn.rows == i]) if int(c) in uidx]
                assert rows.get(i, []) == want, (L, i)
            # the MLP norm's weights of each thread's rows
            f = chain.fmt(mg.e4)
            w = np.zeros(4096, np.float32)
            w[:H] = ly.post_attention_layernorm
            for t in (0, 1, 300, 511):
                rr = [4 * t + k for k in range(4)] + [2048 + 4 * t + k for k in range(4)]
                bits16 = [(int(S[t, f.W1 + k // 2]) >> (16 * (k % 2))) & 0xffff for k in range(8)]
                assert [np.uint32(b << 16).view(np.float32) for b in bits16] == w[rr].tolist()
            # each wave loads every word its passes read
            ww = int(descs[L].pt_words)
            for wv in range(8):
                nu, nb = (ww >> (8 * wv)) & 15, (ww >> (8 * wv + 4)) & 15
                lanes = S[64 * wv:64 * wv + 64]
                used_u = np.nonzero(lanes[:, f.U0:f.MB].any(0))[0]
                used_b = np.nonzero(lanes[:, f.MB:].any(0))[0]
                assert len(used_u) == 0 or used_u.max() // 4 < nu
                assert used_b.max() // 4 < nb
            # the gate tables: live query/key channels and their rows, in column order
            gate = mega.Gate.from_buffer_copy(blob[descs[L].gate:descs[L].gate + 64])
            qk = (mega.QkC * gate.n_qk).from_buffer_copy(
                blob[descs[L].gate + gate.qk:descs[L].gate + gate.qk + 32 * gate.n_qk])
            qkv = ly.in_proj_qkv
            live = np.nonzero((np.asarray(ly.conv1d)[:2 * m.dims.nk * 256] != 0).any(1))[0]
            assert [q.chan for q in qk] == live.tolist()
            for q in qk:
                sel = qkv.rows == q.chan
                got = [_ent(blob, descs[L].gate + gate.ent, q.start + k) for k in range(q.len)]
                assert [(int(c), float(v)) for c, v in got] == \
                    list(zip(qkv.cols[sel].tolist(), qkv.vals[sel].tolist()))
            # out_proj by residual row over every value dim, ascending
            oc = ly.out_proj
            optr = np.frombuffer(blob[descs[L].out_ptr:descs[L].out_ptr + 4 * (H + 1)], np.int32)
            for i in range(0, H, 7):
                sel = oc.rows == i
                o2 = np.argsort(oc.cols[sel], kind="stable")
                want = list(zip(oc.cols[sel][o2].tolist(), oc.vals[sel][o2].tolist()))
                got = [_ent(blob, descs[L].out_ent, k, 1) for k in range(optr[i], optr[i + 1])]
                assert [(int(c), float(v)) for c, v in got] == want
        # head: rows x columns with a nonzero final weight
        hptr = mg.head_ptr.numpy()
        hent = bytes(mg.head_ent.numpy())
        w1 = 1.0 + m.norm
        E = m.embed
        for v in (0, 7, m.dims.vocab - 1):
            want = [(int(c), float(x)) for c, x in zip(E.cols[E.rows == v], E.vals[E.rows == v])
                    if w1[c] != 0]
            got = [_ent(hent, 0, k) for k in range(hptr[v], hptr[v + 1])]
            assert [(int(c), float(x)) for c, x in got] == want


def test_packer_fits_every_config(packed):
    for spec in (synth.config1(), synth.config2()):
        m, mg = packed(spec)
        assert mg.gate_bytes <= mega.GATE_MAX
        assert mg.stats["qk_total"] <= mega.MAXQK
        assert mg.lds <= 163_840
        assert mg.e4  # every packed value is exact in bf16: 4-byte entries


def test_c_abi_exports_every_declared_symbol(native_lib):
    """The library loads and exports each entry point include/*.h declares (no GPU call)."""
    hdrs = sorted(f for f in os.listdir(os.path.join(ROOT, "include")) if f.endswith(".h"))
    assert {"lxm.h", "lxm_prefill.h", "lxm_dense.h", "lxm_chunk.h"} <= set(hdrs)
    hdr = "".join(open(os.path.join(ROOT, "include", h)).read() for h in hdrs)
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


@pytest.mark.parametrize("name", ["small", "tiny"])
def test_prefill_entries_carry_their_norm_weights(name):
    """The prefill packer (host only): every entry of an MLP unit's gate/up row carries the
    post-attention norm weight 1 + w of its column, every entry of a query/key row and of a decay
    row the input norm's; other entries carry 0. The tile kernel forms D((x r) w1) from them as
    it gathers, so a wrong weight here would change the units' and the gates' inputs. (tiny:
    random norm weights on every column, where the two norms differ everywhere.)"""
    from linuxformer_amd import fast, prefill

    m = synth.build(synth.small()) if name == "small" else synth.tiny_dense(3, "bf16")
    f = fast.Fast(m)
    for L in range(m.dims.n_layers):
        ly = m.layers[L]
        blob = prefill._Blob()
        pl = prefill.pack_layer(m, f, L, blob)
        raw = blob.bytes()

        def arr(off, dtype, n):
            return np.frombuffer(raw, dtype=dtype, count=n, offset=off)

        n_ent = (pl.entn - pl.ent) // prefill.ENT.itemsize  # ent is followed by entn
        ent = arr(pl.ent, prefill.ENT, n_ent)
        entn = arr(pl.entn, np.float32, n_ent)
        w1_in = np.float32(1.0) + np.asarray(ly.input_layernorm, np.float32)
        w1_post = np.float32(1.0) + np.asarray(ly.post_attention_layernorm, np.float32)
        want = np.zeros(n_ent, np.float32)
        units = arr(pl.units, np.int32, 4 * pl.n_units).reshape(-1, 4)
        for gs, gn, us, un in units:
            for a, n in ((gs, gn), (us, un)):
                want[a:a + n] = w1_post[ent["off"][a:a + n] // 16]
        qk = arr(pl.qk, np.dtype([("chan", "<i4"), ("kslot", "<i4"), ("pos", "<i4"),
                                  ("start", "<i4"), ("len", "<i4"), ("pad", "<i4", 3),
                                  ("taps", "<f4", 4)]), pl.n_qk)
        dec = arr(pl.dec, np.dtype([("vslot", "<i4"), ("start", "<i4"), ("len", "<i4"),
                                    ("dt_bias", "<f4"), ("A_log", "<f4"), ("pad", "<i4", 3)]),
                  pl.n_dec)
        for a, n in list(zip(qk["start"], qk["len"])) + list(zip(dec["start"], dec["len"])):
            want[a:a + n] = w1_in[ent["off"][a:a + n] // 16]
        assert pl.n_units > 0 and pl.n_qk > 0
        assert (entn.view(np.uint32) == want.view(np.uint32)).all(), L


def test_alone_rejects_bad_launch_sizes():
    from linuxformer_amd import alone

    with pytest.raises(ValueError):
        alone.run_alone(None, [[1]], final=lambda t: True, done=lambda s, b: True,
                        first_launch=0)
    with pytest.raises(ValueError):
        alone.run_alone(None, [[1]], final=lambda t: True, done=lambda s, b: True,
                        first_launch=64, max_launch=32)


def test_runner_refuses_more_tokens_than_the_dump_holds(tmp_path, native_lib):
    """lxm_runner checks the token count against the dumped prediction buffer (and inputs and
    trace) before it touches the GPU: a launch of more tokens would write past them."""
    from linuxformer_amd import mega

    if not os.path.exists(mk_build.RUNNER):
        mk_build.build()
    p = mega.Params(hidden=64, n_layers=2, n_tokens=10)
    (tmp_path / "params.bin").write_bytes(bytes(p))
    (tmp_path / "lib.txt").write_text(mk_build.LIB + "\n")
    (tmp_path / "manifest.txt").write_text("launch x 256 1024\nzero preds 40\nzero inputs 40\n")
    for n, ok in (("11", False), ("0", False)):
        r = subprocess.run([mk_build.RUNNER, str(tmp_path), "1", n], capture_output=True,
                           text=True, timeout=60)
        assert r.returncode == 2 and "hold 10 predictions" in r.stderr, (n, r.stderr)
    (tmp_path / "manifest.txt").write_text("launch x 256 1024\nzero preds 8\n")
    r = subprocess.run([mk_build.RUNNER, str(tmp_path), "1"], capture_output=True, text=True,
                       timeout=60)  # the dumped count itself (10) exceeds a 2-token buffer
    assert r.returncode == 2 and "hold 2 predictions" in r.stderr, r.stderr


def test_prefill_head_table_rows():
    """pf_head's table (host only): each row holds its kept entries (columns whose final-norm
    factor is nonzero) in column order, its first four at 4 x row and the rest of a longer row at
    its (start, count), then zero-weight entries at column hidden up to a multiple of 4 and at
    least 4 (an empty row too); the slices cover the rows in order."""
    from types import SimpleNamespace
    from linuxformer_amd import prefill
    hidden = 12
    rows = [[], [(1, 0.5)], [(0, 1.0), (3, -2.0), (5, 0.25), (7, 4.0), (9, -1.0)], [(4, 3.0)],
            [(2, 1.5), (6, 2.5), (8, -0.5), (10, 0.75)]]
    ptr = np.cumsum([0] + [len(r) for r in rows]).astype(np.int64)
    cols = np.asarray([c for r in rows for c, _ in r], np.int64)
    vals = np.asarray([v for r in rows for _, v in r], np.float32)
    er = SimpleNamespace(n=len(rows), ptr=ptr, cols=cols, vals=vals)
    w1f = np.ones(hidden, np.float32)
    w1f[4] = 0.0  # a column the final norm zeroes: dropped from every row
    w1f[9] = 0.0
    sl, more, hent = prefill.head_table(er, w1f, hidden)
    assert more.shape == (len(rows), 2)
    n_all = 4 * len(rows) + int(more[:, 1].sum())
    assert len(hent) == n_all + 4
    for i, r in enumerate(rows):
        kept = [(c, v) for c, v in r if w1f[c] != 0]
        s, n = int(more[i, 0]), int(more[i, 1])
        e = np.concatenate([hent[4 * i:4 * i + 4], hent[s:s + n]])  # the row as the kernel reads it
        assert n % 4 == 0 and (n == 0) == (len(kept) <= 4) and len(e) - len(kept) < 4 + (4 if not kept else 0)
        assert n == 0 or s >= 4 * len(rows)
        assert [(int(o) // 16, float(w)) for o, w in e[:len(kept)]] == [(c, v) for c, v in kept]
        assert (e["off"][len(kept):] == 16 * hidden).all() and (e["w"][len(kept):] == 0).all()
    assert (hent["off"][n_all:] == 16 * hidden).all() and (hent["w"][n_all:] == 0).all()
    assert sl[0] == 0 and sl[-1] == len(rows) and (np.diff(sl) >= 0).all()
    assert len(sl) == prefill.SLICES + 1


def _head_dense_back(pl, H):
    """The packed head (entries plus coded dense columns) as a dense (vocab, hidden) array."""
    V = pl.vocab
    out = np.zeros((V, H), np.float32)
    ent = np.frombuffer(pl.head_ent, np.uint32)[:pl.head_ptr[-1]]
    rows = np.repeat(np.arange(V), np.diff(pl.head_ptr))
    out[rows, (ent & 0xffff) // 4] = ((ent >> 16) << 16).view(np.float32)
    for j in range(pl.n_hd):
        codes = ((pl.head_code >> np.uint64(2 * j)) & np.uint64(3)).astype(np.int64)
        out[:, pl.head_dcol[j]] = pl.head_dtab[4 * j + codes]
    return out


def test_dense_head_columns_decode_to_the_model(native_lib):
    """A head with dense columns (every row nonzero there, 4 values; one column with zeros): the
    coded columns and the remaining entries decode back to the tied head's rows exactly, and the
    coded columns are exactly the dense ones."""
    import dataclasses

    m = synth.build(dataclasses.replace(synth.small(), head_dense=5))
    pl = mega.pack(fast.Fast(m), 0, 256, native_lib)
    assert pl.n_hd == 5
    w1 = 1.0 + m.norm
    want = m.embed.dense() * (w1 != 0)[None]
    assert np.array_equal(_head_dense_back(pl, m.dims.hidden), want)
    cnt = (want != 0).sum(0)
    assert set(pl.head_dcol[:5].tolist()) == set(np.nonzero(cnt * 2 >= m.dims.vocab)[0].tolist())
    assert (np.diff(pl.head_dcol[:5]) > 0).all()
    # without dense columns nothing is coded
    pl0 = mega.pack(fast.Fast(synth.build(synth.small())), 0, 256, native_lib)
    assert pl0.n_hd == 0 and pl0.summary()["head_dense_cols"] == 0


def test_merged_layout_packs_the_chip_rows(native_lib):
    """The chip inside a larger vocabulary (lx/lx/linux.py:108-109's rows = slice(offset,
    offset + VOCAB), Mega's offset): the packed tables equal the chip-only model's, through the
    coordinate model and through a transformers model (only the chip's rows of its head read);
    an offset that is not where the rows start is refused."""
    m = synth.build(synth.small())
    off = 300
    mm = synth.merged(m, off)
    want = mega.pack(fast.Fast(m), 0, 256, native_lib)
    rows = slice(off, off + m.dims.vocab)
    f = fast.Fast(mm, rows=rows)
    got = mega.pack(f, off, 256, native_lib)
    hf = synth.to_hf(mm)
    fh = fast.Fast(hf, m.dims.n_layers, rows)
    assert fh.sm.embed.shape == (m.dims.vocab, m.dims.hidden)  # only the chip's rows were read
    via_hf = mega.pack(fh, off, 256, native_lib)
    for pl in (got, via_hf):
        assert pl.blob == want.blob and pl.emb_ent == want.emb_ent and pl.head_ent == want.head_ent
        assert np.array_equal(pl.emb_ptr, want.emb_ptr) and np.array_equal(pl.head_ptr, want.head_ptr)
        assert pl.vocab == m.dims.vocab
    with pytest.raises(ValueError, match="offset"):
        mega.pack(f, 0, 256, native_lib)
    with pytest.raises(ValueError, match="offset"):
        mega.pack(fast.Fast(m), 5, 256, native_lib)
    # the verified-mode tables read the same rows
    pf_rows = f.embed_rows()
    assert pf_rows.n == m.dims.vocab and np.array_equal(pf_rows.cols, fast.Fast(m).embed_rows().cols)


def test_real_chip_sizes(native_lib):
    """The reference's real chip against the decode kernel's limits, from its published table
    statistics (lx/results/mega_boot.json: 459,982 head rows, 31 dense head columns, 4,133,751
    other head nonzeros; fast_boot.json: hidden 2560, 37 layers, up to 8,102 live MLP units in
    one layer). The head now fits a helper's LDS (its dense columns as 2-bit codes, not 14.3M
    entries), and the packer names the limit the MLP units break (LXM_MAXU)."""
    import dataclasses

    d = synth.Dims(hidden=2560, n_layers=1, vocab=459_982, inter=1024)
    spec = dataclasses.replace(synth.small(), dims=d, emb_nnz=9, head_dense=31, density=0.0008,
                               p_live=0.25, p_decay=0.25, p_tap=0.1)
    m = synth.build(spec)
    e = m.embed
    dense_cols = np.nonzero(np.bincount(e.cols, minlength=d.hidden) == d.vocab)[0]
    assert len(dense_cols) >= 30
    pl = mega.pack(fast.Fast(m), 0, 256, native_lib).check()
    assert pl.n_hd == 31
    assert abs(pl.summary()["head_nnz"] - 4_133_751) / 4_133_751 < 0.02  # the other columns
    # (about 140 KB a helper: 89 KB of head tables, 14 KB of them the codes; the same rows as
    # 4-byte entries would need ~290 KB)
    assert pl.lds <= mega.MAX_LDS_MI355X and pl.lds_helper <= mega.MAX_LDS_MI355X
    # a layer with the real chip's largest live-unit count
    ly = m.layers[0]
    rng = np.random.default_rng(0)
    U, d2 = 8102, dataclasses.replace(d, inter=9216)
    cols = np.stack([rng.choice(d.hidden - 1, 3, replace=False) for _ in range(U)]).reshape(-1)
    gate = synth.Coo.build((d2.inter, d.hidden), np.repeat(np.arange(U), 3), cols,
                           np.ones(3 * U, np.float32))
    down = synth.Coo.build((d.hidden, d2.inter), rng.integers(0, d.hidden - 1, U), np.arange(U),
                           np.ones(U, np.float32))
    big = dataclasses.replace(ly, gate_proj=gate, up_proj=gate, down_proj=down)
    m2 = synth.SparseModel(d2, [big], m.embed, m.norm, meta=m.meta)
    with pytest.raises(mega.PackError, match="LXM_MAXU"):
        mega.pack(fast.Fast(m2), 0, 256, native_lib)
