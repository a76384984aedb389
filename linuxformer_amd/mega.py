"""The chip layers' decode as one persistent HIP kernel (csrc/lxm_decode.hip) on MI355X.

The drop-in for lx.mega (lx/lx/mega.py): the same class, constructor and ``run`` signature,
the same cache tensors updated in place, the same predictions.

    m = Mega(fast, model, cache, offset)
    preds = m.run(forced, n)   # n steps: inputs forced[0..], then each step's own prediction

The packer here turns the model's sparse tensors (from ``Fast``) into one byte blob of tables the
kernel reads: per layer a per-thread table (norm weights, MLP rows, down rows; chain.py) that
the chain workgroup prefetches into its registers one layer ahead, the gates' tables (the live
query/key channels and decays, resident in the chain's LDS), and "cold" tables (value rows, z,
beta, out_proj by residual row) read only when a head is active; the head's rows split over the
helper workgroups, each staging its own in LDS.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import synth, chain, mk_build

NT, MAXH, KD, VD, RMAX = 512, 4096, 256, 128, 8
MAXU, MAXQK, MAXQKL, MAXDEC, GATE_MAX, NSYNC, OUT_MAX = 2048, 1024, 512, 512, 65536, 19456, 1024
OUT_HELPERS, OUT_ROWS = 64, 64

I32, I64, F32, PTR = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class Gate(ctypes.Structure):
    _fields_ = [(n, I32) for n in ("n_qk", "n_dec", "qk_base", "qk", "dec", "ent", "ent_w1",
                                   "size")] + [("eps", F32), ("geps", F32)] + \
        [(n, I32) for n in ("long_u", "long_r", "long_ent", "n_long_u", "n_long_r", "pad")]


class QkC(ctypes.Structure):
    _fields_ = [("slot", I32), ("chan", I32), ("start", I32), ("len", I32), ("taps", F32 * 4)]


class Dec(ctypes.Structure):
    _fields_ = [("vh", I32), ("start", I32), ("len", I32), ("dt_bias", F32), ("A_log", F32),
                ("pad", I32 * 3)]


class Chan(ctypes.Structure):
    _fields_ = [("start", I32), ("len", I32), ("taps", F32 * 4)]


class LayerDesc(ctypes.Structure):
    _fields_ = [(n, I64) for n in ("ptt", "pt_words", "gate")] + \
        [(n, I64) for n in ("chan", "qkv_ent", "b_row", "b_ent", "z_row", "z_ent", "out_ptr",
                            "out_ent", "gnorm", "w1_in")]


class Params(ctypes.Structure):
    _fields_ = [(n, I32) for n in ("hidden", "n_layers", "nk", "kd", "nv", "vd", "n_conv",
                                   "vocab", "bf16", "n_blocks")] + \
        [("rms_eps", F32), ("head_lds", I32), ("e4", I32), ("gate_bytes", I32)] + \
        [(n, PTR) for n in ("layers", "blob", "gates", "rec", "conv", "emb_ptr", "emb_ent",
                            "w1_final", "head_rows", "head_ptr", "head_ent", "forced")] + \
        [("n_forced", I32), ("n_tokens", I32)] + \
        [(n, PTR) for n in ("preds", "inputs", "trace", "ring", "rring", "hn", "sync", "keys", "err",
                            "prof", "mb_task", "mb_e", "mb_qk", "ybuf", "xo")] + \
        [("n_qk_total", I32), ("n_hd", I32)] + \
        [(n, PTR) for n in ("head_dcol", "head_dtab", "head_code")]


assert ctypes.sizeof(Gate) == 64 and ctypes.sizeof(QkC) == 32 and ctypes.sizeof(Dec) == 32
assert ctypes.sizeof(Chan) == 24 and ctypes.sizeof(LayerDesc) == 104


def _bf16_bits(v: np.ndarray) -> np.ndarray:
    """float32 values exactly representable in bf16 -> their 16 bits (uint32)."""
    u = np.ascontiguousarray(v, np.float32).view(np.uint32)
    assert np.all((u & 0xffff) == 0), "a value is not exact in bf16"
    return u >> 16


class _Blob:
    """A growing byte buffer with 16-byte aligned sections."""

    def __init__(self):
        self.parts, self.n = [], 0

    def add(self, b: bytes) -> int:
        off = self.n
        b = bytes(b)
        pad = -len(b) % 16
        self.parts.append(b + bytes(pad))
        self.n += len(b) + pad
        return off

    def bytes(self) -> bytes:
        return b"".join(self.parts)


class _Csr:
    """Rows of a Coo (sorted by row, then column): ptr, cols, vals."""

    def __init__(self, coo, keep_rows=None):
        rows, cols, vals = coo.rows, coo.cols, coo.vals
        self.n = coo.shape[0]
        self.ptr = np.zeros(self.n + 1, np.int64)
        np.cumsum(np.bincount(rows, minlength=self.n), out=self.ptr[1:])
        self.cols, self.vals = cols, vals

    def row(self, r):
        a, b = self.ptr[r], self.ptr[r + 1]
        return self.cols[a:b], self.vals[a:b]

    def count(self, r):
        return int(self.ptr[r + 1] - self.ptr[r])


def _bf16_exact(v) -> bool:
    return bool(np.all((np.ascontiguousarray(v, np.float32).view(np.uint32) & 0xffff) == 0))


def model_e4(sm) -> bool:
    """Whether every value the packer stores is exact in bf16 (the 4-byte entry format)."""
    if sm.dims.dtype == "bf16":
        return True
    for ly in sm.layers:
        for c in (ly.in_proj_qkv, ly.in_proj_z, ly.in_proj_b, ly.in_proj_a, ly.out_proj,
                  ly.gate_proj, ly.up_proj, ly.down_proj):
            if not _bf16_exact(c.vals):
                return False
        if not (_bf16_exact(ly.input_layernorm) and _bf16_exact(ly.post_attention_layernorm)):
            return False
    return _bf16_exact(sm.embed.vals)


class Packer:
    def __init__(self, e4: bool):
        self.bf16 = e4

    def ent(self, idx: np.ndarray, vals: np.ndarray, scale: int = 4) -> bytes:
        """Entries: e4 one uint32 (index | bf16 << 16), else two uint32 (index, float). The index
        is stored times ``scale``: 4 (a byte offset into the float vector the row is applied to,
        which the kernel adds to the vector's base) for every table but out_proj's."""
        idx = np.asarray(idx, np.int64) * scale
        if self.bf16:
            assert len(idx) == 0 or idx.max() < 1 << 16
            return (idx.astype(np.uint32) | (_bf16_bits(vals) << 16)).astype(np.uint32).tobytes()
        out = np.empty((len(idx), 2), np.uint32)
        out[:, 0] = idx
        out[:, 1] = np.asarray(vals, np.float32).view(np.uint32)
        return out.tobytes()

    @property
    def esz(self) -> int:
        return 4 if self.bf16 else 8

    def w1(self, w: np.ndarray) -> bytes:
        """A norm's weights: bf16 models the raw weight's bits (the kernel adds 1 in fp32, as
        (1.0 + weight.float()) does), fp32 models 1 + w in fp32."""
        w = np.asarray(w, np.float32)
        if self.bf16:
            return _bf16_bits(w).astype(np.uint16).tobytes()
        return (np.float32(1.0) + w).astype(np.float32).tobytes()


class PackError(ValueError):
    """A model the decode kernel's tables cannot hold; the message names the limit."""


def _cap(ok: bool, msg: str) -> None:
    if not ok:
        raise PackError(msg)


MAX_LDS_MI355X = 163_840  # LDS bytes one workgroup may use on gfx950 (160 KB per CU)
HEAD_DENSE = 32           # dense head columns, at most (LXM_HEAD_DENSE)


def head_dense_columns(rows, cols, vals, n_rows: int, hidden: int):
    """The head columns kept as 2-bit codes (the reference's dense head columns,
    lx/lx/mega.py:354-376, lx/csrc/mega.cu:96-101): a column nonzero in at least half of the
    rows with at most 4 distinct values (zero counted where the column has one), the fullest
    first, at most HEAD_DENSE of them. Returns (columns ascending, (n, 4) float32 tables: each
    column's values ascending, padded with the first)."""
    cnt = np.bincount(cols, minlength=hidden)
    cand = np.nonzero(2 * cnt >= max(n_rows, 1))[0]
    if len(cand) == 0:
        return np.zeros(0, np.int64), np.zeros((0, 4), np.float32)
    sel = np.isin(cols, cand)
    c_s, v_s = cols[sel], vals[sel]
    order = np.argsort(c_s, kind="stable")
    c_s, v_s = c_s[order], v_s[order]
    bounds = np.searchsorted(c_s, cand), np.searchsorted(c_s, cand, side="right")
    picked = []
    for k in np.argsort(-cnt[cand], kind="stable"):
        c = int(cand[k])
        v = np.unique(v_s[bounds[0][k]:bounds[1][k]].astype(np.float32))
        if cnt[c] < n_rows:
            v = np.unique(np.concatenate([v, np.zeros(1, np.float32)]))
        if len(v) <= 4:
            picked.append((c, v))
        if len(picked) == HEAD_DENSE:
            break
    picked.sort()
    tabs = np.zeros((len(picked), 4), np.float32)
    for j, (_, v) in enumerate(picked):
        tabs[j, :len(v)] = v
        tabs[j, len(v):] = v[0]
    return np.array([c for c, _ in picked], np.int64), tabs


class Plan:
    """The decode's packed tables and launch sizes, built on the host (``pack``); ``Mega``
    uploads them. ``check(max_lds)`` raises PackError naming a limit the plan breaks."""

    def check(self, max_lds: int = MAX_LDS_MI355X) -> "Plan":
        _cap(self.lds <= max_lds,
             f"a workgroup needs {self.lds} B of LDS (chain {self.lds_chain}, helper "
             f"{self.lds_helper} with {self.head_lds} B of head tables) > {max_lds}")
        return self

    def summary(self) -> dict:
        return {k: v for k, v in self.stats.items() if not isinstance(v, list)}


def pack(fast, offset: int = 0, ncta: int = 256, lib=None) -> Plan:
    """Pack ``fast``'s chip layers for the decode kernel on ncta workgroups (the chain and
    ncta - 1 helpers). Host work only: the tables as bytes and arrays, the LDS each workgroup
    needs (lib: the native library, for its LDS constants). Raises PackError when the model
    breaks one of the kernel's limits (include/lxm.h)."""
    lib = lib or mk_build.load()
    sm = fast.sm
    if synth.has_dense_order(sm):
        raise ValueError("a dense-order stack (config 4) runs on linuxformer_amd.dense")
    d = sm.dims
    pl = Plan()
    pl.dims, pl.ncta = d, ncta
    _cap(ncta >= 2, "the decode needs the chain workgroup and at least one helper")
    _cap(ncta <= 256, "at most 256 workgroups (the sync area's per-helper stamps)")
    nh = ncta - 1
    _cap(d.nv <= nh, f"{d.nv} value heads: each needs its own helper workgroup ({nh})")
    _cap(-(-d.hidden // min(nh, OUT_HELPERS)) <= OUT_ROWS, "too many out_proj rows per helper")
    _cap(d.kd == KD and d.vd == VD and d.conv == 4, "key dim 256, value dim 128, conv 4")
    _cap(d.nv % d.nk == 0 and d.nv // d.nk <= RMAX, f"at most {RMAX} value heads per key head")
    _cap(d.hidden <= MAXH, f"hidden {d.hidden} > {MAXH} (LXM_MAXH)")
    _cap(d.nv <= 256 and d.nk <= 64 and d.n_layers <= 64,
         "at most 256 value heads, 64 key heads and 64 layers")
    pl.bf = d.dtype == "bf16"
    pl.e4 = model_e4(sm)
    pk = Packer(pl.e4)
    blob = _Blob()
    descs = (LayerDesc * d.n_layers)()
    H, R, C = d.hidden, d.nv // d.nk, d.n_conv
    qk_total = 0
    pl.stats = {"layers": d.n_layers, "units": [], "qk": [], "dec": [], "chain": []}
    pl.unit_order = []  # per layer: the model's unit index of each packed unit
    cf = chain.fmt(pl.e4)
    gate_blobs, gate_off = [], 0
    ptts, longs = [], []
    for L, ly in enumerate(sm.layers):
        # ---- live MLP units (gate row, up row and down column nonzero; lx/lx/fast.py:242-248),
        # in the model's order (the act index of a unit is its position here)
        g, u, dn = _Csr(ly.gate_proj), _Csr(ly.up_proj), _Csr(ly.down_proj.transpose())
        gc = np.diff(g.ptr)
        uc = np.diff(u.ptr)
        dc = np.diff(dn.ptr)
        units = np.nonzero((gc > 0) & (uc > 0) & (dc > 0))[0]
        _cap(len(units) <= MAXU, f"layer {L}: {len(units)} live MLP units > {MAXU} (LXM_MAXU)")
        pl.unit_order.append(units)
        uidx = np.full(d.inter, -1, np.int64)
        uidx[units] = np.arange(len(units))
        # down_proj by residual row over the live units, in the model's unit order (the sum's
        # order), each entry naming the unit's packed index
        dcoo = ly.down_proj
        keep = uidx[dcoo.cols] >= 0
        drows, dunits, dvals = dcoo.rows[keep], uidx[dcoo.cols[keep]], dcoo.vals[keep]
        order = np.lexsort((dcoo.cols[keep], drows))
        drows, dunits, dvals = drows[order], dunits[order], dvals[order]
        dptr = np.zeros(H + 1, np.int64)
        np.cumsum(np.bincount(drows, minlength=H), out=dptr[1:])
        ct = chain.pack_layer(
            cf, H, units, [g.row(k) for k in units], [u.row(k) for k in units],
            [(dunits[dptr[r]:dptr[r + 1]], dvals[dptr[r]:dptr[r + 1]]) for r in range(H)],
            np.asarray(ly.post_attention_layernorm, np.float32))
        # ---- the gates: live query/key channels (nonzero conv taps) and decaying heads
        qkv = _Csr(ly.in_proj_qkv)
        taps = np.asarray(ly.conv1d, np.float32)
        ent_parts, ent_w1, epos = [], [], 0
        qks = []
        w1in = np.asarray(ly.input_layernorm, np.float32)
        for c in np.nonzero((taps[:2 * d.nk * KD] != 0).any(1))[0]:
            kh, rem = divmod(int(c) % (d.nk * KD), KD)
            isk = int(c) >= d.nk * KD
            cols, vals = qkv.row(c)
            q = QkC(slot=kh * 512 + (256 if isk else 0) + rem, chan=int(c), start=epos,
                    len=len(cols))
            q.taps[:] = [float(x) for x in taps[c]]
            qks.append(q)
            ent_parts.append(pk.ent(cols, vals))
            ent_w1.append(w1in[cols])
            epos += len(cols)
        _cap(len(qks) <= MAXQKL, f"layer {L}: {len(qks)} live query/key channels > {MAXQKL} (LXM_MAXQKL)")
        acsr = _Csr(ly.in_proj_a)
        decs = []
        for vh in range(d.nv):
            cols, vals = acsr.row(vh)
            # softplus(dt_bias) is exactly 0 only when exp(dt_bias) underflows (< -103.97)
            if len(cols) == 0 and not float(ly.dt_bias[vh]) > -103.9:
                continue
            decs.append(Dec(vh=vh, start=epos, len=len(cols), dt_bias=float(ly.dt_bias[vh]),
                            A_log=float(ly.A_log[vh])))
            ent_parts.append(pk.ent(cols, vals))
            ent_w1.append(w1in[cols])
            epos += len(cols)
        _cap(len(decs) <= MAXDEC, f"layer {L}: {len(decs)} decaying value heads > {MAXDEC} (LXM_MAXDEC)")
        # one gate item per chain lane: the channels on the top waves, the decays below them
        _cap(-(-len(qks) // 64) * 64 + len(decs) <= NT, f"layer {L}: {len(qks)} query/key channels and {len(decs)} decays exceed the chain's {NT} gate lanes")
        gb = _Blob()
        gb.add(bytes(64))
        o_qk = gb.add(b"".join(bytes(q) for q in qks))
        o_dec = gb.add(b"".join(bytes(x) for x in decs))
        o_ent = gb.add(b"".join(ent_parts) + bytes(4 * pk.esz))
        # the GDN norm's weight at each of those entries' columns
        o_entw = gb.add((pk.w1(np.concatenate(ent_w1)) if ent_w1 else b"") + bytes(16))
        # the chain's long units and rows (too long for its register passes)
        o_lu = gb.add(ct.long_u)
        o_lr = gb.add(ct.long_r)
        o_le = gb.add(ct.long_ent)
        gate = Gate(n_qk=len(qks), n_dec=len(decs), qk_base=qk_total, qk=o_qk, dec=o_dec,
                    ent=o_ent, ent_w1=o_entw, size=gb.n, eps=d.rms_eps, geps=d.geps,
                    long_u=o_lu, long_r=o_lr, long_ent=o_le, n_long_u=len(ct.long_u) // 32,
                    n_long_r=len(ct.long_r) // 16)
        gb.parts[0] = bytes(gate)
        gate_blobs.append(gb.bytes())
        descs[L].gate = gate_off  # (made absolute below)
        gate_off += gb.n
        qk_total += len(qks)
        ptts.append(ct)
        pl.stats["chain"].append(ct.stats)
        desc = descs[L]
        # ---- cold tables
        chans = np.zeros(C, dtype=[("start", "<i4"), ("len", "<i4"), ("taps", "<f4", (4,))])
        chans["start"] = qkv.ptr[:-1]
        chans["len"] = np.diff(qkv.ptr)
        chans["taps"] = taps
        desc.chan = blob.add(chans.tobytes())
        desc.qkv_ent = blob.add(pk.ent(qkv.cols, qkv.vals))
        b = _Csr(ly.in_proj_b)
        desc.b_row = blob.add(np.stack([b.ptr[:-1], np.diff(b.ptr)], 1).astype(np.int32).tobytes())
        desc.b_ent = blob.add(pk.ent(b.cols, b.vals))
        z = _Csr(ly.in_proj_z)
        desc.z_row = blob.add(np.stack([z.ptr[:-1], np.diff(z.ptr)], 1).astype(np.int32).tobytes())
        desc.z_ent = blob.add(pk.ent(z.cols, z.vals))
        # out_proj by residual row over all value dims (vh * vd + j), ascending; each
        # helper workgroup stages the entries of its slice of rows
        oc = _Csr(ly.out_proj)
        optr = oc.ptr
        rp = -(-H // min(nh, OUT_HELPERS))
        for r0 in range(0, H, rp):
            n_e = int(optr[min(r0 + rp, H)] - optr[r0])
            _cap(n_e <= OUT_MAX, f"layer {L}: {n_e} out_proj entries in {rp} rows > {OUT_MAX} (LXM_OUT_MAX)")
        desc.out_ptr = blob.add(optr.astype(np.int32).tobytes())
        desc.out_ent = blob.add(pk.ent(oc.cols, oc.vals, scale=1))
        desc.gnorm = blob.add(np.asarray(ly.norm, np.float32).tobytes())
        desc.w1_in = blob.add(pk.w1(ly.input_layernorm))
        pl.stats["units"].append(len(units))
        pl.stats["qk"].append(len(qks))
        pl.stats["dec"].append(len(decs))
    _cap(qk_total <= MAXQK, f"{qk_total} live query/key channels > {MAXQK} (LXM_MAXQK)")
    _cap(gate_off <= GATE_MAX, f"the gate tables ({gate_off} B) exceed {GATE_MAX} B of the chain's LDS (LXM_GATE_MAX)")
    pl.gate_bytes = gate_off
    gsec = blob.add(b"".join(gate_blobs))
    pl.gate_sec = gsec
    for L, ct in enumerate(ptts):
        desc = descs[L]
        desc.gate += gsec
        desc.ptt = blob.add(ct.ptt)
        desc.pt_words = ct.wave_words
    blob.add(bytes(4096))  # padding past the last table
    pl.blob = blob.bytes()
    pl.layers = bytes(descs)
    pl.n_qk_total = qk_total
    # ---- embedding (the chip's rows, all columns) and the head
    emb = fast.embed_rows(offset)
    V = emb.n
    _cap(V <= 1 << 19, f"{V} vocabulary rows > 2^19 (the head keys carry a 19-bit index)")
    pl.emb_ptr = emb.ptr.astype(np.int64)
    pl.emb_ent = pk.ent(emb.cols, emb.vals)
    w1f = (np.float32(1.0) + np.asarray(sm.norm, np.float32)).astype(np.float32)
    w1pad = np.ones(MAXH, np.float32)  # the chain reads every thread's rows (<= MAXH)
    w1pad[:H] = w1f
    pl.w1_final = w1pad
    hmask = w1f != 0  # a column whose (1 + w) is 0 adds only zeros
    keep = hmask[emb.cols]
    hrows = np.repeat(np.arange(V), np.diff(emb.ptr))[keep]
    hcols, hvals = emb.cols[keep], emb.vals[keep]
    # dense columns as 2-bit codes per row; the other columns as entries
    dcols, dtabs = head_dense_columns(hrows, hcols, hvals, V, H)
    nd = len(dcols)
    code = np.zeros(V, np.uint64)
    if nd:
        jof = np.full(H, -1, np.int64)
        jof[dcols] = np.arange(nd)
        isd = jof[hcols] >= 0
        for j in range(nd):
            zc = int(np.nonzero(dtabs[j] == 0.0)[0][0]) if (dtabs[j] == 0.0).any() else 0
            code |= np.uint64(zc) << np.uint64(2 * j)  # rows with no entry there: the zero's code
        r_d, j_d, v_d = hrows[isd], jof[hcols[isd]], hvals[isd].astype(np.float32)
        c_d = np.zeros(len(r_d), np.uint64)
        for j in range(nd):
            m = j_d == j
            c_d[m] = np.searchsorted(dtabs[j], v_d[m]).astype(np.uint64)
            assert np.all(dtabs[j][c_d[m].astype(np.int64)] == v_d[m])
        # clear each coded column's default, then set its code
        clear = np.zeros(len(r_d), np.uint64)
        for j in range(nd):
            clear[j_d == j] = np.uint64(3) << np.uint64(2 * j)
        np.bitwise_and.at(code, r_d, ~clear)
        np.bitwise_or.at(code, r_d, c_d << (2 * j_d).astype(np.uint64))
        hrows, hcols, hvals = hrows[~isd], hcols[~isd], hvals[~isd]
    hptr = np.zeros(V + 1, np.int64)
    np.cumsum(np.bincount(hrows, minlength=V), out=hptr[1:])
    pl.head_ptr = hptr
    pl.head_ent = pk.ent(hcols, hvals) + bytes(16)
    pl.n_hd = nd
    pl.head_dcol = np.zeros(HEAD_DENSE, np.int32)
    pl.head_dcol[:nd] = dcols
    pl.head_dtab = np.zeros(4 * HEAD_DENSE, np.float32)
    pl.head_dtab[:4 * nd] = dtabs.reshape(-1)
    if pl.e4 and nd:
        _bf16_bits(dtabs)  # (the e4 kernel's coded values are bf16-exact, as the entries)
    pl.head_code = code if nd else np.zeros(1, np.uint64)
    # block 0 is the chain (no head rows); helper b covers cuts[b - 1] .. cuts[b]
    cuts = np.linspace(0, V, nh + 1).round().astype(np.int64)
    bounds = np.concatenate([[0], cuts])
    pl.head_rows = bounds.astype(np.int32)
    a16 = lambda n: (int(n) + 15) // 16 * 16  # noqa: E731
    need = 0
    for b in range(1, ncta):
        r0, r1 = bounds[b], bounds[b + 1]
        ne = hptr[r1] - hptr[r0]
        nb = a16((r1 - r0 + 1) * 4) + a16(ne * pk.esz)
        if nd:
            nb += a16(8 * (r1 - r0)) + a16(H) + 768
        need = max(need, nb)
    pl.head_lds = a16(need)
    pl.lds_chain = int(lib.lxm_lds_base())
    pl.lds_helper = int(lib.lxm_helper_lds(pl.head_lds))
    pl.lds = (max(pl.lds_chain, pl.lds_helper) + 255) // 256 * 256
    pl.vocab = V
    pl.stats.update({"ctas": ncta, "lds": pl.lds, "head_lds": pl.head_lds,
                     "blob_bytes": len(pl.blob), "qk_total": qk_total,
                     "head_nnz": int(hptr[-1]), "head_dense_cols": nd, "vocab": V})
    return pl


class Mega:
    """lx.mega.Mega (lx/lx/mega.py:198-574) on MI355X.

    fast: a ``linuxformer_amd.fast.Fast``; model: the model it was built from (unused beyond
    what Fast holds, kept for the signature); cache: per layer ``conv_states[0]`` (1, n_conv, 4)
    in the model dtype and ``recurrent_states[0]`` (1, nv, kd, vd) float32 on the device,
    updated in place; offset: the first chip token's row in the embedding. ``spec`` and
    ``pair_layers`` are accepted for compatibility: this kernel computes each layer's gates
    before its MLP, so it never speculates and never redoes work.
    """

    def __init__(self, fast, model=None, cache=None, offset: int = 0, ncta: int | None = None,
                 subprof: bool = False, spec: bool = True, pair_layers=None, device=None):
        self.lib = mk_build.load(subprof)
        self.subprof = subprof
        self.fast, self.model, self.cache, self.offset = fast, model, cache, offset
        dev = torch.device(device) if device is not None else torch.device("cuda")
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.dev = dev
        pl = pack(fast, offset, ncta or int(self.lib.lxm_device_cus()), self.lib)
        pl.check(int(self.lib.lxm_max_lds()))
        if int(self.lib.lxm_max_blocks(pl.lds)) < pl.ncta:
            raise PackError("the grid is not co-resident")
        self.plan = pl
        d = self.dims = pl.dims
        self.ncta, self.bf, self.e4 = pl.ncta, pl.bf, pl.e4
        self.lds = self.smem = pl.lds  # (smem: lx.mega.Mega's name for the launch's LDS)
        self.head_lds, self.gate_bytes, self.gate_sec = pl.head_lds, pl.gate_bytes, pl.gate_sec
        self.n_qk_total, self.vocab, self.n_hd = pl.n_qk_total, pl.vocab, pl.n_hd
        self.unit_order, self.stats = pl.unit_order, pl.stats

        def up(b, dtype=torch.uint8):
            return torch.frombuffer(bytearray(b), dtype=torch.uint8).view(dtype).to(dev)

        self.blob = up(pl.blob)
        self.layers_d = up(pl.layers)
        self.emb_ptr = torch.from_numpy(pl.emb_ptr).to(dev)
        self.emb_ent = up(pl.emb_ent)
        self.w1_final = torch.from_numpy(pl.w1_final).to(dev)
        self.head_ptr = torch.from_numpy(pl.head_ptr).to(dev)
        self.head_ent = up(pl.head_ent)
        self.head_rows = torch.from_numpy(pl.head_rows).to(dev)
        self.head_dcol = torch.from_numpy(pl.head_dcol).to(dev)
        self.head_dtab = torch.from_numpy(pl.head_dtab).to(dev)
        self.head_code = torch.from_numpy(pl.head_code.view(np.int64)).to(dev)
        # ---- run buffers (the library allocates nothing)
        self.ring = torch.zeros(4 * d.n_layers * MAXH, dtype=torch.float32, device=dev)
        self.rring = torch.zeros(4 * d.n_layers, dtype=torch.float32, device=dev)
        self.mb_task = torch.zeros(d.nv, dtype=torch.int32, device=dev)
        self.mb_e = torch.zeros(d.nv, dtype=torch.float32, device=dev)
        self.mb_qk = torch.zeros(MAXQKL, dtype=torch.float32, device=dev)
        # stamped words (a float low, the event's number high), zeroed for every launch
        self.ybuf = torch.zeros(d.nv * VD, dtype=torch.int64, device=dev)
        self.xo = torch.zeros(MAXH, dtype=torch.float32, device=dev)
        self.hn = torch.zeros(MAXH, dtype=torch.float32, device=dev)
        self.sync = torch.zeros(NSYNC, dtype=torch.int32, device=dev)
        self.keys = torch.zeros(2, dtype=torch.int64, device=dev)
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)

    PHASES = ("embedding", "residual + sums (stage C2, +trace)", "norms (stage A)",
              "gates + MLP units (stage B)", "GDN events + MLP redo",
              "down_proj rows (stage C1)", "final norm + publish", "head argmax wait")
    HELPER = ("wait", "head rows", "value head", "out_proj rows")

    SUB_STAGES = ("stage A (norms)", "stage B (units + gates)", "stage C1 (down rows)",
                  "stage C2 (residual + sums)")

    @property
    def prof_size(self) -> int:
        return 32 + 4 * self.ncta + (16 * len(self.SUB_STAGES) + 4 + 12 * self.ncta
                                     if self.subprof else 0)

    def phase_report(self, prof: torch.Tensor) -> dict:
        """prof counters -> cycles per token of each chain phase, and the helpers' mean (and
        max) cycles per token in each of their parts."""
        c = prof.cpu().tolist()
        n = max(c[17], 1)
        out = {name: round(c[k] / n, 1) for k, name in enumerate(self.PHASES)}
        out["GDN events per token"] = round(c[16] / n, 3)
        out["MLP redos per token"] = round(c[18] / n, 3)  # (events with a live query)
        for k, name in enumerate(self.HELPER):
            v = [c[32 + 4 * b + k] for b in range(1, self.ncta)]
            out[f"helper {name}"] = round(sum(v) / len(v) / n, 1)
            out[f"helper {name} max"] = round(max(v) / n, 1)
        out["tokens"] = n
        if self.subprof:
            base = 32 + 4 * self.ncta
            for s, name in enumerate(self.SUB_STAGES):
                busy = [round(c[base + 16 * s + w] / n / self.dims.n_layers) for w in range(8)]
                wait = [round(c[base + 16 * s + 8 + w] / n / self.dims.n_layers) for w in range(8)]
                out[f"per layer, {name}: busy by wave"] = busy
                out[f"per layer, {name}: wait by wave"] = wait
            ev = base + 16 * len(self.SUB_STAGES)
            ne = c[ev + 2]
            if ne:
                post = c[ev] / ne  # mean wall-clock ticks (10 ns) of the events' posts
                us = lambda x: round((x / ne - post) / 100.0, 3)  # noqa: E731
                seen = [us(c[ev + 4 + 4 * b]) for b in range(1, self.ncta)]
                own = [us(c[ev + 4 + 4 * b + 1]) for b in range(1, min(self.ncta, self.dims.nv + 1))]
                outs = [b for b in range(1, self.ncta) if c[ev + 4 + 4 * b + 2]]
                cvh = [us(c[ev + 4 + 4 * b + 2]) for b in outs]
                odone = [us(c[ev + 4 + 4 * b + 3]) for b in outs]
                out["GDN event timeline (us after the post, mean over events)"] = {
                    "events": ne, "helpers saw it (mean, max)": [round(sum(seen) / len(seen), 3), max(seen)],
                    "value head stored (mean, max)": [round(sum(own) / len(own), 3), max(own)] if own else None,
                    "out_proj helpers had every head and their rows (mean, max)": [round(sum(cvh) / len(cvh), 3), max(cvh)] if cvh else None,
                    "out_proj rows stored (mean, max)": [round(sum(odone) / len(odone), 3), max(odone)] if odone else None,
                    "chain saw every helper": us(c[ev + 1])}
                gb = ev + 4 + 4 * self.ncta
                rows = []
                for b in range(1, min(self.ncta, self.dims.nv + 1)):
                    g = c[gb + 8 * b: gb + 8 * b + 8]
                    if g[5]:
                        rows.append([round(g[k] / g[5] / 100.0, 2) for k in range(5)] +
                                    [g[5], round(g[6] / max(g[7], 1) / 100.0, 2), g[7]])
                if rows:
                    worst = max(rows, key=lambda r: r[4])
                    out["value head step (us from its start: q/k in, v/z/beta in, tile computed, "
                        "state stored, output stored; steps; mean decaying step; decaying steps)"] = {
                        "mean over heads": [round(sum(r[k] for r in rows) / len(rows), 2) for k in range(8)],
                        "slowest head": worst}
        return out

    def _bufs(self) -> dict:
        return dict(ring=self.ring.data_ptr(), rring=self.rring.data_ptr(),
                    hn=self.hn.data_ptr(), sync=self.sync.data_ptr(),
                    keys=self.keys.data_ptr(), err=self.err.data_ptr(),
                    mb_task=self.mb_task.data_ptr(), mb_e=self.mb_e.data_ptr(),
                    mb_qk=self.mb_qk.data_ptr(), ybuf=self.ybuf.data_ptr(),
                    xo=self.xo.data_ptr())

    def dump(self, path: str, forced, n: int, prof: bool = False) -> None:
        """Write everything a launch needs (tables, states, parameter block, manifest) to path,
        for csrc/lxm_runner.cpp to replay through the C ABI without Python."""
        import os

        os.makedirs(path, exist_ok=True)
        d = self.dims
        lines = [f"launch x {self.ncta} {self.lds}"]

        def buf(name, t):
            fn = name + ".bin"
            with open(os.path.join(path, fn), "wb") as f:
                f.write(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes())
            lines.append(f"buf {name} {fn}")

        for name in ("layers_d", "blob", "emb_ptr", "emb_ent", "w1_final", "head_rows",
                     "head_ptr", "head_ent", "head_dcol", "head_dtab", "head_code"):
            buf({"layers_d": "layers"}.get(name, name), getattr(self, name))
        buf("forced", torch.tensor([int(forced[0])], dtype=torch.int32))
        for field, attr in (("rec", "recurrent_states"), ("conv", "conv_states")):
            files = []
            for L in range(d.n_layers):
                fn = f"{field}{L}.bin"
                t = getattr(self.cache.layers[L], attr)[0]
                with open(os.path.join(path, fn), "wb") as f:
                    f.write(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes())
                files.append(fn)
            lines.append(f"ptrs {field} {d.n_layers} " + " ".join(files))
        for name, nbytes in (("preds", 4 * n), ("ring", self.ring.numel() * 4),
                             ("rring", self.rring.numel() * 4),
                             ("hn", self.hn.numel() * 4), ("sync", NSYNC * 4), ("keys", 16),
                             ("err", 4), ("mb_task", self.mb_task.numel() * 4),
                             ("mb_e", self.mb_e.numel() * 4), ("mb_qk", self.mb_qk.numel() * 4),
                             ("ybuf", self.ybuf.numel() * 8), ("xo", self.xo.numel() * 4)):
            lines.append(f"zero {name} {nbytes}")
        if prof:
            lines.append(f"zero prof {8 * self.prof_size}")
        p = Params(hidden=d.hidden, n_layers=d.n_layers, nk=d.nk, kd=KD, nv=d.nv, vd=VD,
                   n_conv=d.n_conv, vocab=self.vocab, bf16=int(self.bf), n_blocks=self.ncta,
                   rms_eps=d.rms_eps, head_lds=self.head_lds, e4=int(self.e4), n_forced=1,
                   n_tokens=n, n_qk_total=self.n_qk_total, gate_bytes=self.gate_bytes,
                   n_hd=self.n_hd)
        lines.append(f"sub gates blob {self.gate_sec}")
        with open(os.path.join(path, "params.bin"), "wb") as f:
            f.write(bytes(p))
        with open(os.path.join(path, "manifest.txt"), "w") as f:
            f.write("\n".join(lines) + "\n")
        with open(os.path.join(path, "lib.txt"), "w") as f:
            f.write(mk_build.LIB + "\n")

    def _state_ptrs(self):
        rs, cs = [], []
        d = self.dims
        for L in range(d.n_layers):
            cl = self.cache.layers[L]
            r, c = cl.recurrent_states[0], cl.conv_states[0]
            assert r.is_contiguous() and c.is_contiguous() and r.dtype == torch.float32
            assert tuple(r.shape[-3:]) == (d.nv, KD, VD) and c.shape[-1] == 4
            assert c.dtype == (torch.bfloat16 if self.bf else torch.float32)
            assert r.device == self.dev and c.device == self.dev
            rs.append(r.data_ptr())
            cs.append(c.data_ptr())
        return (torch.tensor(rs, dtype=torch.int64, device=self.dev),
                torch.tensor(cs, dtype=torch.int64, device=self.dev))

    def sync_bitmaps(self) -> None:
        """lx.mega's nonzero-row bitmaps are not used: decays scale the whole state tile."""

    def _params(self, rs, cs, ft, n_forced: int, n: int, preds, inputs=None, trace=None,
                prof=None, bufs: dict | None = None) -> Params:
        d = self.dims
        return Params(hidden=d.hidden, n_layers=d.n_layers, nk=d.nk, kd=KD, nv=d.nv, vd=VD,
                      n_conv=d.n_conv, vocab=self.vocab, bf16=int(self.bf), n_blocks=self.ncta,
                      rms_eps=d.rms_eps, head_lds=self.head_lds, e4=int(self.e4),
                      gate_bytes=self.gate_bytes, layers=self.layers_d.data_ptr(),
                      blob=self.blob.data_ptr(), gates=self.blob.data_ptr() + self.gate_sec,
                      rec=rs.data_ptr(), conv=cs.data_ptr(), emb_ptr=self.emb_ptr.data_ptr(),
                      emb_ent=self.emb_ent.data_ptr(), w1_final=self.w1_final.data_ptr(),
                      head_rows=self.head_rows.data_ptr(), head_ptr=self.head_ptr.data_ptr(),
                      head_ent=self.head_ent.data_ptr(), forced=ft.data_ptr(), n_forced=n_forced,
                      n_tokens=n, preds=preds.data_ptr(),
                      inputs=inputs.data_ptr() if inputs is not None else None,
                      trace=trace.data_ptr() if trace is not None else None,
                      prof=prof.data_ptr() if prof is not None else None,
                      n_qk_total=self.n_qk_total, n_hd=self.n_hd,
                      head_dcol=self.head_dcol.data_ptr(), head_dtab=self.head_dtab.data_ptr(),
                      head_code=self.head_code.data_ptr(), **(bufs or {}))

    @torch.no_grad()
    def run(self, forced, n: int, dbg=None, dbg_tok: int = 0, dbg_items=None, prof=None,
            inputs: torch.Tensor | None = None, trace: torch.Tensor | None = None) -> list:
        """n steps; step i's input is forced[i] (i < len(forced)) or step i - 1's prediction.
        Returns the n predictions (chip token ids). inputs (n,) int32: each step's input as the
        kernel embedded it. trace (n, n_layers, hidden) float32: the residual after each
        layer of each step. prof (``prof_size``) int64: phase cycle counters (see
        ``phase_report``). lx.mega's item dumps (dbg, dbg_items: its per-item shared-memory
        layout) have no counterpart in this kernel and raise; ``trace`` records every layer's
        residual instead."""
        if dbg is not None or dbg_items is not None:
            raise NotImplementedError("Mega.run: dbg/dbg_items dump lx.mega's per-item shared "
                                      "memory, which this kernel does not have; use trace=")
        assert len(forced) >= 1 and n >= 1
        f = np.asarray(forced, np.int64)
        if f.min() < 0 or f.max() >= self.vocab:
            raise ValueError("forced token out of range")
        self._check_events(n)
        d = self.dims
        rs, cs = self._state_ptrs()
        ft = torch.tensor(f.astype(np.int32), device=self.dev)
        preds = torch.zeros(n, dtype=torch.int32, device=self.dev)
        if inputs is not None:
            assert inputs.dtype == torch.int32 and inputs.numel() >= n and inputs.device == self.dev
        if prof is not None:
            assert prof.dtype == torch.int64 and prof.numel() >= self.prof_size
            assert prof.device == self.dev
        if trace is not None:
            assert trace.dtype == torch.float32 and trace.is_contiguous()
            assert trace.numel() >= n * d.n_layers * d.hidden and trace.device == self.dev
        self.sync.zero_()
        self.keys.zero_()
        self.err.zero_()
        self.ybuf.zero_()
        p = self._params(rs, cs, ft, len(f), n, preds, inputs, trace, prof, self._bufs())
        pd = torch.frombuffer(bytearray(bytes(p)), dtype=torch.uint8).to(self.dev)
        self._keep = (rs, cs, ft, pd)
        st = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        mk_build.note_cooperative()
        e = self.lib.lxm_run(ctypes.byref(p), ctypes.c_void_p(pd.data_ptr()), self.ncta,
                             self.lds, st)
        if e:
            raise RuntimeError(f"mega launch failed: hipError {e}")
        out = preds.tolist()  # syncs
        e = self.lib.lxm_last_error()
        if e:
            raise RuntimeError(f"mega failed: hipError {e}")
        err = int(self.err.item())
        if err:
            raise RuntimeError(f"mega failed: a grid wait timed out (code {err})")
        return out

    def run_noalloc(self, forced: torch.Tensor, n: int, preds: torch.Tensor, err: torch.Tensor,
                    inputs: torch.Tensor | None = None) -> None:
        """``run`` through lxm_run_noalloc, for callers that cannot allocate device memory: the
        forced tokens (int32, device), the predictions (int32, device, >= n) and the error word
        (int32, device, 1; nonzero after the run when a wait timed out) are the caller's; the
        run buffers are the library's static per-device scratch. Asynchronous on the current
        stream (nothing here allocates or synchronizes); calls that overlap on one GPU race."""
        for t in (forced, preds, err):
            assert t.dtype == torch.int32 and t.device == self.dev and t.is_contiguous()
        assert forced.numel() >= 1 and n >= 1 and preds.numel() >= n and err.numel() >= 1
        self._check_events(n)
        if inputs is not None:
            assert inputs.dtype == torch.int32 and inputs.numel() >= n and inputs.device == self.dev
        rs, cs = self._state_ptrs_cached()
        p = self._params(rs, cs, forced, forced.numel(), n, preds, inputs)
        p.err = err.data_ptr()
        st = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        mk_build.note_cooperative()
        e = self.lib.lxm_run_noalloc(ctypes.byref(p), self.ncta, self.lds, st)
        if e:
            raise RuntimeError(f"mega launch failed: hipError {e}")

    def _check_events(self, n: int) -> None:
        """A launch numbers its events (n_layers + 1 per token) in 24 bits, as the stamped
        words carry them."""
        if n * (self.dims.n_layers + 1) >= 1 << 24:
            raise ValueError(f"{n} tokens: at most {((1 << 24) - 1) // (self.dims.n_layers + 1)} "
                             "per launch")

    def _state_ptrs_cached(self):
        """The state pointer arrays, built once per set of state tensors (keyed by every layer's
        recurrent and conv pointers; a new set goes through _state_ptrs' checks)."""
        key = tuple((self.cache.layers[L].recurrent_states[0].data_ptr(),
                     self.cache.layers[L].conv_states[0].data_ptr())
                    for L in range(self.dims.n_layers))
        if getattr(self, "_ptrs_key", None) != key:
            self._ptrs = self._state_ptrs()
            self._ptrs_key = key
        return self._ptrs
