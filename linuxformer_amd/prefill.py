"""The verified-mode forward of the chip layers on the native prefill kernels
(csrc/lxm_prefill.hip, C ABI include/lxm_prefill.h): lx.fast's Fast.forward, Fast.layer,
Fast.head_argmax and Fast.decode (lx/lx/fast.py:252-361, :365-540, :544-550) for T positions.

Semantics: every position sees exactly the stock decode step, so a call over T positions leaves
the residuals, predictions, conv windows and recurrent states that T forced decode steps leave
(``Mega.run(tokens, T)``), bit for bit. This module packs each layer's sparse rows into the
kernels' tables (one device blob) and drives the entry points over caller-owned buffers.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import mk_build, synth

TT, KD, VD, NT = 4, 256, 128, 512
MAXKS, MAXVS, UPT, SLICES = 16, 128, 4, 8

ENT = np.dtype([("off", "<i4"), ("w", "<f4")])


class PfLayer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("ent", "w1_in", "w1_post", "units", "drows", "qk",
                                              "dec", "vs", "vc", "zrow", "brow", "orows", "cc",
                                              "gnorm", "entn")] + \
        [(n, ctypes.c_int32) for n in ("n_units", "n_drows", "n_qk", "n_dec", "n_ks", "n_vs",
                                       "n_orows", "rec_bytes")] + \
        [("kh", ctypes.c_int32 * MAXKS), ("eps", ctypes.c_float), ("geps", ctypes.c_float),
         ("reach", ctypes.c_int32), ("pad", ctypes.c_int32)]


class PfParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("hidden", "n_layers", "nk", "nv", "n_conv", "vocab",
                                              "bf16", "T", "ntiles", "max_rec")] + \
        [("rms_eps", ctypes.c_float), ("head_long", ctypes.c_int32)] + \
        [(n, ctypes.c_void_p) for n in ("layers", "layers_host", "blob", "rec", "conv", "w1_final",
                                        "emb_ptr", "emb_ent", "head_slice", "head_more", "head_ent",
                                        "tokens", "h", "hn", "r1", "mask", "cand", "cmask", "count",
                                        "recs", "keys", "preds", "err")]


def rec_bytes(n_ks: int, n_vs: int) -> int:
    """A candidate record: header, qn/kn per key slot, v/z per value slot, beta, e, proc."""
    n = 16 + 2 * 4 * KD * n_ks + 2 * 4 * VD * n_vs + 3 * 4 * n_vs
    return (n + 15) // 16 * 16


class _Blob:
    def __init__(self):
        self.parts, self.size = [], 0

    def add(self, a) -> int:
        b = a.tobytes() if isinstance(a, np.ndarray) else bytes(a)
        off = self.size
        pad = (-len(b)) % 16
        self.parts.append(b + b"\0" * pad)
        self.size += len(b) + pad
        return off

    def bytes(self) -> bytes:
        return b"".join(self.parts)


class _Ents:
    """One layer's entry array, built row group by row group."""

    def __init__(self):
        self.offs, self.ws, self.nws, self.n = [], [], [], 0

    def add(self, offs, ws, nw=None) -> int:
        """Entries (16 x column, weight); nw: the norm weight of each entry's column when the
        row reads a norm's output (applied as the tile kernel gathers), else 0."""
        start = self.n
        self.offs.append(np.asarray(offs, np.int64))
        self.ws.append(np.asarray(ws, np.float32))
        k = len(self.offs[-1])
        self.nws.append(np.zeros(k, np.float32) if nw is None else np.asarray(nw, np.float32))
        assert len(self.nws[-1]) == k
        self.n += k
        return start

    def add4(self, offs, ws, nw, zero: int) -> int:
        """add() for a row that the tile kernel sums four entries at a time with no test: padded
        to a multiple of 4 by entries (off = zero, w = 0, norm weight 0), zero being 16 x a
        column that holds +0 (adding +0 x 0 to a sum from +0 changes no bits: such a sum is
        never -0). The row's length stays its own."""
        offs, ws = np.asarray(offs, np.int64), np.asarray(ws, np.float32)
        p = (-len(offs)) % 4
        nw = np.zeros(len(offs), np.float32) if nw is None else np.asarray(nw, np.float32)
        return self.add(np.concatenate([offs, np.full(p, zero, np.int64)]),
                        np.concatenate([ws, np.zeros(p, np.float32)]),
                        np.concatenate([nw, np.zeros(p, np.float32)]))

    def pad(self) -> None:
        """Four entries (off 0, w 0) closing a group: a row's last load of four entries reads
        its own group or these, never a table of another vector."""
        self.add(np.zeros(4, np.int64), np.zeros(4, np.float32))

    def array(self) -> np.ndarray:
        e = np.zeros(self.n + 4, ENT)  # four padding entries (off 0, w 0) after the table
        if self.n:
            e["off"][:self.n] = np.concatenate(self.offs)
            e["w"][:self.n] = np.concatenate(self.ws)
        return e

    def norms(self) -> np.ndarray:
        """The entries' norm weights, padded like array()."""
        n = np.zeros(self.n + 4, np.float32)
        if self.n:
            n[:self.n] = np.concatenate(self.nws)
        return n


class _Csr:
    """Row access to a Coo (sorted by row, then column)."""

    def __init__(self, coo):
        self.cols, self.vals = np.asarray(coo.cols), np.asarray(coo.vals, np.float32)
        self.ptr = np.zeros(coo.shape[0] + 1, np.int64)
        np.cumsum(np.bincount(np.asarray(coo.rows), minlength=coo.shape[0]), out=self.ptr[1:])

    def row(self, r):
        a, b = self.ptr[r], self.ptr[r + 1]
        return self.cols[a:b], self.vals[a:b]

    def rows(self, rs):
        """Concatenated entries of rows rs (in that order), with each row's start and length."""
        rs = np.asarray(rs, np.int64)
        lens = self.ptr[rs + 1] - self.ptr[rs]
        idx = np.concatenate([np.arange(self.ptr[r], self.ptr[r + 1]) for r in rs]) \
            if len(rs) else np.zeros(0, np.int64)
        starts = np.cumsum(lens) - lens
        return self.cols[idx], self.vals[idx], starts, lens


def _may_decay(ly, has_a: np.ndarray) -> np.ndarray:
    """Value heads whose exp(g) can differ from 1: an in_proj_a row, or a dt_bias (a = 0) whose
    softplus is not 0 in fp32 (exp(x) rounds to 0 below -104), or an A_log whose exp overflows."""
    dt = np.asarray(ly.dt_bias, np.float32)
    al = np.asarray(ly.A_log, np.float32)
    return has_a | (dt > -104.0) | (al > 88.0)


def pack_layer(sm, fast, L: int, blob: _Blob) -> PfLayer:
    d, ly = sm.dims, sm.layers[L]
    H, nk, nv = d.hidden, d.nk, d.nv
    R = nv // nk
    dec_info = fast.dec[L]
    E = _Ents()
    pl = PfLayer()
    # ---- MLP: live units sorted by length (thread-strided, similar lengths per wave); the tile
    # kernel's rows (units, down_proj, query/key channels, decays) padded to multiples of 4 at a
    # zero column (column hidden of the residual tile, column n_units of the units' outputs)
    g, u = _Csr(ly.gate_proj), _Csr(ly.up_proj)
    w1_in = np.float32(1.0) + np.asarray(ly.input_layernorm, np.float32)
    w1_post = np.float32(1.0) + np.asarray(ly.post_attention_layernorm, np.float32)
    units = np.asarray(dec_info["units"], np.int64)
    assert len(units) <= UPT * NT, f"layer {L}: {len(units)} MLP units > {UPT * NT}"
    glen = g.ptr[units + 1] - g.ptr[units]
    ulen = u.ptr[units + 1] - u.ptr[units]
    order = np.argsort(-(glen + ulen), kind="stable")
    units = units[order]
    pos = np.full(d.inter, -1, np.int64)
    pos[units] = np.arange(len(units))
    ut = np.zeros((len(units), 4), np.int32)
    for i, un in enumerate(units):
        c, v = g.row(un)
        ut[i, 0], ut[i, 1] = E.add4(16 * c, v, w1_post[c], 16 * H), len(c)
        c, v = u.row(un)
        ut[i, 2], ut[i, 3] = E.add4(16 * c, v, w1_post[c], 16 * H), len(c)
    E.pad()
    # down_proj rows over the live units, entries in ascending unit order (16 x position)
    dcoo = ly.down_proj
    keep = pos[np.asarray(dcoo.cols)] >= 0
    drows_r = np.asarray(dcoo.rows)[keep]
    dcols = pos[np.asarray(dcoo.cols)[keep]]
    dvals = np.asarray(dcoo.vals, np.float32)[keep]
    rows_u, rcount = np.unique(drows_r, return_counts=True)
    rstart_src = np.concatenate([[0], np.cumsum(rcount)[:-1]]) if len(rcount) else np.zeros(0, np.int64)
    dorder = np.argsort(-rcount, kind="stable")
    dt = np.zeros((len(rows_u), 4), np.int32)
    for i, k in enumerate(dorder):
        a, n = rstart_src[k], rcount[k]
        dt[i] = (rows_u[k], E.add4(16 * dcols[a:a + n], dvals[a:a + n], None, 16 * len(units)),
                 n, 0)
    E.pad()
    # ---- gates: live key heads' query/key channels with a nonzero tap
    qkv = _Csr(ly.in_proj_qkv)
    taps = np.asarray(ly.conv1d, np.float32)
    kh = np.asarray(dec_info["kh"], np.int64)
    assert len(kh) <= MAXKS
    kslot = np.full(nk, -1, np.int64)
    kslot[kh] = np.arange(len(kh))
    qk_rows, reach = [], 0
    for s, k in enumerate(kh):
        for part in (0, 1):
            for i in range(KD):
                ch = part * nk * KD + k * KD + i
                tp = taps[ch]
                if not (tp != 0).any():
                    continue
                reach = max(reach, 3 - int(np.nonzero(tp)[0][0]))
                c, v = qkv.row(ch)
                qk_rows.append((ch, s, part * KD + i, E.add4(16 * c, v, w1_in[c], 16 * H), len(c),
                                tp))
    qkt = np.zeros(len(qk_rows), np.dtype([("chan", "<i4"), ("kslot", "<i4"), ("pos", "<i4"),
                                           ("start", "<i4"), ("len", "<i4"), ("pad", "<i4", 3),
                                           ("taps", "<f4", 4)]))
    for i, (ch, s, p, st, n, tp) in enumerate(qk_rows):
        qkt[i] = (ch, s, p, st, n, (0, 0, 0), tp)
    # ---- value-head slots: the live key heads' value heads and the heads that may decay
    acsr = _Csr(ly.in_proj_a)
    has_a = acsr.ptr[1:] > acsr.ptr[:-1]
    decays = np.nonzero(_may_decay(ly, has_a))[0]
    slots = np.union1d((kh[:, None] * R + np.arange(R)).reshape(-1), decays).astype(np.int64)
    assert len(slots) <= MAXVS
    vslot = np.full(nv, -1, np.int64)
    vslot[slots] = np.arange(len(slots))
    dslot = np.full(nv, -1, np.int64)
    dslot[decays] = np.arange(len(decays))
    vst = np.zeros((len(slots), 4), np.int32)
    for i, vh in enumerate(slots):
        vst[i] = (vh, kslot[vh // R], dslot[vh], 0)
    dect = np.zeros(len(decays), np.dtype([("vslot", "<i4"), ("start", "<i4"), ("len", "<i4"),
                                           ("dt_bias", "<f4"), ("A_log", "<f4"),
                                           ("pad", "<i4", 3)]))
    for i, vh in enumerate(decays):
        c, v = acsr.row(vh)
        dect[i] = (vslot[vh], E.add4(16 * c, v, w1_in[c], 16 * H), len(c), ly.dt_bias[vh],
                   ly.A_log[vh], (0, 0, 0))
    zcsr, bcsr = _Csr(ly.in_proj_z), _Csr(ly.in_proj_b)
    vct = np.zeros(len(slots) * VD, np.dtype([("start", "<i4"), ("len", "<i4"), ("taps", "<f4", 4)]))
    zt = np.zeros((len(slots) * VD, 2), np.int32)
    bt = np.zeros((len(slots), 2), np.int32)
    for i, vh in enumerate(slots):
        if kslot[vh // R] < 0:
            continue
        for j in range(VD):
            ch = 2 * nk * KD + vh * VD + j
            c, v = qkv.row(ch)
            vct[i * VD + j] = (E.add(16 * c, v), len(c), taps[ch])
            c, v = zcsr.row(vh * VD + j)
            zt[i * VD + j] = (E.add(16 * c, v), len(c))
        c, v = bcsr.row(vh)
        bt[i] = (E.add(16 * c, v), len(c))
    E.pad()
    # ---- out_proj rows over the value dims of slots with a live key head, ascending dims
    oc = ly.out_proj
    ocols = np.asarray(oc.cols)
    ovh = ocols // VD
    okeep = (vslot[ovh] >= 0) & (kslot[np.maximum(ovh // R, 0)] >= 0)
    orow_r = np.asarray(oc.rows)[okeep]
    ooff = 4 * (vslot[ovh[okeep]] * VD + ocols[okeep] % VD)
    oval = np.asarray(oc.vals, np.float32)[okeep]
    orr, ocount = np.unique(orow_r, return_counts=True)
    ostart = np.concatenate([[0], np.cumsum(ocount)[:-1]]) if len(ocount) else np.zeros(0, np.int64)
    ot = np.zeros((len(orr), 4), np.int32)
    for i in range(len(orr)):
        a, n = ostart[i], ocount[i]
        ot[i] = (orr[i], E.add(ooff[a:a + n], oval[a:a + n]), n, 0)
    E.pad()
    # ---- every conv channel's row (the windows left after the call)
    cc = np.zeros((d.n_conv, 2), np.int32)
    cc[:, 0] = E.n + qkv.ptr[:-1]
    cc[:, 1] = qkv.ptr[1:] - qkv.ptr[:-1]
    E.add(16 * qkv.cols, qkv.vals)
    ents = E.array()
    assert len(ents) < 2 ** 31
    pl.ent = blob.add(ents)
    pl.entn = blob.add(E.norms())
    pl.w1_in = blob.add(w1_in)
    pl.w1_post = blob.add(w1_post)
    pl.units = blob.add(ut)
    pl.drows = blob.add(dt)
    pl.qk = blob.add(qkt)
    pl.dec = blob.add(dect)
    pl.vs = blob.add(vst)
    pl.vc = blob.add(vct)
    pl.zrow = blob.add(zt)
    pl.brow = blob.add(bt)
    pl.orows = blob.add(ot)
    pl.cc = blob.add(cc)
    pl.gnorm = blob.add(np.asarray(ly.norm, np.float32))
    pl.n_units, pl.n_drows, pl.n_qk, pl.n_dec = len(units), len(rows_u), len(qk_rows), len(decays)
    pl.n_ks, pl.n_vs, pl.n_orows = len(kh), len(slots), len(orr)
    pl.rec_bytes = rec_bytes(len(kh), len(slots))
    for s, k in enumerate(kh):
        pl.kh[s] = int(k)
    pl.eps, pl.geps, pl.reach = d.rms_eps, d.geps, reach
    return pl


class PfBuffers:
    """The run buffers of T positions (device, caller-owned; include/lxm_prefill.h)."""

    NAMES = ("tokens", "h", "hn", "r1", "mask", "cand", "cmask", "count", "recs", "keys",
             "preds", "err")

    def __init__(self, dims, max_rec: int, T: int, dev):
        nt = (T + TT - 1) // TT
        dt = torch.bfloat16 if dims.dtype == "bf16" else torch.float32
        self.T = T
        self.h = torch.zeros(nt * dims.hidden * TT, dtype=dt, device=dev)
        self.hn = torch.zeros_like(self.h)
        self.r1 = torch.zeros(T, dtype=torch.float32, device=dev)
        self.mask = torch.zeros(T, dtype=torch.int32, device=dev)
        self.cand = torch.zeros(T, dtype=torch.int32, device=dev)
        self.cmask = torch.zeros(T, dtype=torch.int32, device=dev)
        self.count = torch.zeros(dims.n_layers + 1, dtype=torch.int32, device=dev)
        self.recs = torch.zeros(T * max_rec, dtype=torch.uint8, device=dev)
        self.keys = torch.zeros(T, dtype=torch.int64, device=dev)
        self.preds = torch.zeros(T, dtype=torch.int32, device=dev)
        self.tokens = torch.zeros(T, dtype=torch.int32, device=dev)
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)


def head_table(er, w1f: np.ndarray, hidden: int):
    """The tied head's rows for pf_head: the embedding rows' entries at columns whose final-norm
    factor (1 + weight) is nonzero, as (slices, more, entries). Entries: off = 16 x column, w =
    value. Row r's first four entries sit at 4 r (a row's place is its index: no row pointer to
    wait for), padded by entries of weight 0 at column hidden (the head kernel's zero column);
    the rest of a longer row, padded the same way to a multiple of 4, sits after the 4 x vocab
    first entries at more[r] = (start, count), (0, 0) for a row of at most four. A row's sum
    takes its entries four at a time with no test (adding +0 to a sum from +0 changes no bits:
    such a sum is never -0; an empty row's logit stays +0). Slices: row ranges of about equal
    work (rows + entries), one per XCD."""
    keep = w1f[er.cols] != 0
    rows = np.repeat(np.arange(er.n), np.diff(er.ptr))[keep]
    cols, vals = er.cols[keep], er.vals[keep]
    cnt = np.bincount(rows, minlength=er.n)
    rank = np.arange(len(rows)) - np.repeat(np.cumsum(cnt) - cnt, cnt)  # entry's place in its row
    extra = np.maximum(0, (cnt - 4 + 3) // 4 * 4)  # the rest of each row, padded
    start = 4 * er.n + np.concatenate([[0], np.cumsum(extra)[:-1]]) if er.n else np.zeros(0, np.int64)
    total = 4 * er.n + int(extra.sum())
    if total + 4 >= 2**31:  # the head kernel indexes entries with 32-bit words
        raise ValueError("head table: more than 2^31 entries")
    hent = np.zeros(total + 4, ENT)
    hent["off"][:] = 16 * hidden
    first = rank < 4
    pos = np.where(first, 4 * rows + rank, start[rows] + rank - 4)
    hent["off"][pos] = 16 * cols
    hent["w"][pos] = vals
    more = np.zeros((er.n, 2), np.int32)
    more[:, 0] = np.where(extra > 0, start, 0)
    more[:, 1] = extra
    work = np.cumsum(4 + extra + 2)
    tot = work[-1] if len(work) else 0
    sl = [0] + [int(np.searchsorted(work, tot * k / SLICES)) for k in range(1, SLICES)] + [er.n]
    sl = np.maximum.accumulate(np.asarray(sl, np.int64))
    return sl, more, hent


class Prefill:
    """The packed tables of a Fast's layers and head on one device, and the drivers."""

    def __init__(self, fast, device="cuda", offset: int | None = None):
        self.fast = fast
        sm = fast.sm
        if synth.has_dense_order(sm):
            raise ValueError("a dense-order stack (config 4) runs on linuxformer_amd.dense")
        d = self.dims = sm.dims
        self.dev = torch.device(device)
        self.bf = d.dtype == "bf16"
        self.lib = mk_build.load()
        blob = _Blob()
        self.layers_h = (PfLayer * max(d.n_layers, 1))()
        for L in range(d.n_layers):
            self.layers_h[L] = pack_layer(sm, fast, L, blob)
        self.max_rec = max([self.layers_h[L].rec_bytes for L in range(d.n_layers)] + [16])
        self.umax = max([self.layers_h[L].n_units for L in range(d.n_layers)] + [0])
        self.blob = torch.frombuffer(bytearray(blob.bytes() + b"\0" * 64), dtype=torch.uint8).to(self.dev)
        self.layers_d = torch.frombuffer(bytearray(bytes(self.layers_h)), dtype=torch.uint8).to(self.dev)
        # embedding and the tied head over the chip rows
        er = fast.embed_rows(offset)
        self.vocab = er.n
        ent = np.zeros(len(er.cols) + 4, ENT)
        ent["off"][:len(er.cols)] = er.cols
        ent["w"][:len(er.cols)] = er.vals
        self.emb_ptr = torch.from_numpy(er.ptr.astype(np.int64)).to(self.dev)
        self.emb_ent = torch.from_numpy(ent.view(np.uint8)).to(self.dev)
        w1f = np.float32(1.0) + np.asarray(sm.norm, np.float32)
        sl, more, hent = head_table(er, w1f, d.hidden)
        self.head_slice = torch.from_numpy(sl.astype(np.int32)).to(self.dev)
        self.head_more = torch.from_numpy(more).to(self.dev)
        self.head_long = int((more[:, 1] > 0).any())  # (else the head kernel reads no head_more)
        self.head_ent = torch.from_numpy(hent.view(np.uint8)).to(self.dev)
        self.w1_final = torch.from_numpy(w1f).to(self.dev)
        self._T = None
        self.stats = {"units": [self.layers_h[L].n_units for L in range(d.n_layers)],
                      "key_slots": [self.layers_h[L].n_ks for L in range(d.n_layers)],
                      "value_slots": [self.layers_h[L].n_vs for L in range(d.n_layers)],
                      "blob_bytes": blob.size, "record_bytes": self.max_rec}

    # ------------------------------------------------------------------------------------------
    def lds_ok(self) -> bool:
        return self.lib.lxm_pf_lds(int(self.bf), self.dims.hidden, self.umax) <= 160 * 1024

    def buffers(self, T: int) -> "PfBuffers":
        """A new set of run buffers for T positions (a caller that captures the launches in a
        graph keeps its own set, which later calls of other sizes never reallocate)."""
        return PfBuffers(self.dims, self.max_rec, T, self.dev)

    def _buffers(self, T: int) -> None:
        if self._T == T:
            return
        self.buf = self.buffers(T)
        for name in PfBuffers.NAMES:
            setattr(self, name, getattr(self.buf, name))
        self._T = T

    def _state_ptrs(self, cache):
        """The cache's state pointer arrays on the device (kept per set of pointers: the cache's
        tensors stay where they are, so later calls copy nothing to the device)."""
        key = tuple((cache.layers[L].recurrent_states[0].data_ptr(),
                     cache.layers[L].conv_states[0].data_ptr()) for L in range(self.dims.n_layers))
        memo = self.__dict__.setdefault("_ptrs_memo", {})
        if key not in memo:
            memo.clear()
            memo[key] = self._state_ptrs_new(cache)
        return memo[key]

    def _state_ptrs_new(self, cache):
        rs, cs = [], []
        d = self.dims
        for L in range(d.n_layers):
            cl = cache.layers[L]
            r, c = cl.recurrent_states[0], cl.conv_states[0]
            assert r.is_contiguous() and c.is_contiguous() and r.dtype == torch.float32
            assert tuple(r.shape[-3:]) == (d.nv, KD, VD) and tuple(c.shape[-2:]) == (d.n_conv, 4)
            assert c.dtype == (torch.bfloat16 if self.bf else torch.float32)
            assert r.device == self.dev and c.device == self.dev
            rs.append(r.data_ptr())
            cs.append(c.data_ptr())
        return (torch.tensor(rs, dtype=torch.int64, device=self.dev),
                torch.tensor(cs, dtype=torch.int64, device=self.dev))

    def params(self, T: int, cache=None, buf: "PfBuffers | None" = None):
        """The parameter block for T positions (host struct, device copy) over buf (default: the
        Prefill's own buffers for T)."""
        p, pd, keep = self.bind(T, cache, buf)
        self._keep = keep
        return p, pd

    def bind(self, T: int, cache=None, buf: "PfBuffers | None" = None):
        """(host block, device block, tensors the blocks point into that the caller keeps). The
        blocks are kept per (T, buffers, state pointers): a repeated call copies nothing."""
        if buf is None:
            self._buffers(T)
            buf = self.buf
        assert buf.T == T
        rs, cs = self._state_ptrs(cache) if cache is not None else (None, None)
        # (kept with the buffers, which it points into, by the addresses of the state arrays it
        # points to: the arrays at those addresses are the current ones)
        key = None if rs is None else (rs.data_ptr(), cs.data_ptr())
        memo = buf.__dict__.setdefault("_bind_memo", {})
        if key not in memo:
            if len(memo) > 8:
                memo.clear()
            memo[key] = self._bind_new(T, buf, rs, cs)
        p, pd = memo[key]
        return p, pd, (rs, cs, pd, buf)

    def _bind_new(self, T: int, buf: "PfBuffers", rs, cs):
        d = self.dims
        p = PfParams(hidden=d.hidden, n_layers=d.n_layers, nk=d.nk, nv=d.nv, n_conv=d.n_conv,
                     vocab=self.vocab, bf16=int(self.bf), T=T, ntiles=(T + TT - 1) // TT,
                     max_rec=self.max_rec, rms_eps=d.rms_eps, head_long=self.head_long,
                     layers=self.layers_d.data_ptr(),
                     layers_host=ctypes.cast(self.layers_h, ctypes.c_void_p).value,
                     blob=self.blob.data_ptr(),
                     rec=rs.data_ptr() if rs is not None else None,
                     conv=cs.data_ptr() if cs is not None else None,
                     w1_final=self.w1_final.data_ptr(), emb_ptr=self.emb_ptr.data_ptr(),
                     emb_ent=self.emb_ent.data_ptr(), head_slice=self.head_slice.data_ptr(),
                     head_more=self.head_more.data_ptr(), head_ent=self.head_ent.data_ptr(),
                     **{n: getattr(buf, n).data_ptr() for n in PfBuffers.NAMES})
        pd = torch.frombuffer(bytearray(bytes(p)), dtype=torch.uint8).to(self.dev)
        return p, pd

    def _stream(self):
        return ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)

    @staticmethod
    def _check(e: int, what: str) -> None:
        if e:
            raise RuntimeError(f"{what} failed: hipError {e}")

    # ------------------------------------------------------------------------------------------
    def to_tiles(self, x: torch.Tensor) -> None:
        """x (T, hidden) row-major, model dtype -> the residual tiles (self.h)."""
        T = x.shape[0]
        p, _ = self.params(T)
        x = x.contiguous()
        self._check(self.lib.lxm_pf_tiles(ctypes.byref(p), ctypes.c_void_p(x.data_ptr()),
                                          ctypes.c_void_p(self.h.data_ptr()), 0, self._stream()),
                    "prefill tiles")

    def from_tiles(self, T: int, src: torch.Tensor | None = None) -> torch.Tensor:
        d = self.dims
        p, _ = self.params(T)
        out = torch.empty(T, d.hidden, dtype=self.h.dtype, device=self.dev)
        src = self.h if src is None else src
        self._check(self.lib.lxm_pf_tiles(ctypes.byref(p), ctypes.c_void_p(src.data_ptr()),
                                          ctypes.c_void_p(out.data_ptr()), 1, self._stream()),
                    "prefill tiles")
        return out

    def embed(self, tokens) -> int:
        """The tokens' embedding rows into the residual tiles. Returns T. Tokens already on the
        device (an int32 tensor) are copied there and range-checked by the kernel, which sets the
        error word (``err``, zeroed here at the start of every call, nonzero after it when a
        token was out of range; nothing synchronizes; the layers still run on such a call and
        change the cache); host tokens are checked here and raise."""
        if isinstance(tokens, torch.Tensor) and tokens.device == self.dev:
            if tokens.dtype != torch.int32 or tokens.numel() == 0:
                raise ValueError("device tokens: a non-empty int32 tensor")
            T = int(tokens.numel())
            p, pd = self.params(T)
            self.err.zero_()
            self.tokens.copy_(tokens.reshape(-1))
            self._check(self.lib.lxm_pf_embed(ctypes.byref(p), ctypes.c_void_p(pd.data_ptr()),
                                              self._stream()), "prefill embed")
            return T
        t = torch.as_tensor(tokens, dtype=torch.int64)
        T = int(t.numel())
        if T == 0:
            raise ValueError("no tokens")
        lo, hi = int(t.min()), int(t.max())
        if lo < 0 or hi >= self.vocab:
            raise ValueError("token out of range")
        p, pd = self.params(T)
        self.err.zero_()
        self.tokens.copy_(t.to(torch.int32).reshape(-1))
        self._check(self.lib.lxm_pf_embed(ctypes.byref(p), ctypes.c_void_p(pd.data_ptr()),
                                          self._stream()), "prefill embed")
        return T

    def layers(self, T: int, cache, l0: int = 0, l1: int | None = None) -> None:
        """Layers [l0, l1) over the T positions in the residual tiles, updating the cache."""
        l1 = self.dims.n_layers if l1 is None else l1
        if l0 >= l1:
            return
        if not self.lds_ok():
            raise RuntimeError("prefill: a layer's MLP units exceed the tile kernel's LDS")
        p, pd = self.params(T, cache)
        self._check(self.lib.lxm_pf_layers(ctypes.byref(p), ctypes.c_void_p(pd.data_ptr()), l0, l1,
                                           self._stream()), "prefill layers")

    def head(self, T: int) -> torch.Tensor:
        """The final norm and the head's first maximum at each of the T positions (int32)."""
        p, pd = self.params(T)
        self._check(self.lib.lxm_pf_head(ctypes.byref(p), ctypes.c_void_p(pd.data_ptr()),
                                         self._stream()), "prefill head")
        return self.preds

    def verify(self, tokens, cache) -> torch.Tensor:
        """Every position's prediction (int32, on the device) after the tokens, all layers."""
        T = self.embed(tokens)
        self.layers(T, cache)
        return self.head(T)
