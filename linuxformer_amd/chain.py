"""The chain workgroup's per-layer tables (the packer half of csrc/lxm_decode.hip's chain).

The chain is the one workgroup (512 threads) that runs a token's 37 layers back to back. Each
layer's tables are prefetched from global memory into its threads' registers one layer ahead, so
the chain never stages tables through LDS: thread t reads words t, NT + t, 2 NT + t, ... of the
layer's *per-thread table*, i.e. a wave reads 1 KB runs. A thread's words are slots (uint32) in a
fixed layout, the same for every layer:

    w1     the MLP norm's weights of the thread's residual rows 4t..4t+3, 2048+4t..2048+4t+3
    meta A its units' act indices, its long unit, the wave's unit pass bounds
    P0, P1 two unit passes: a unit whose gate and up rows have at most G0MAX (P0) or G1MAX (P1)
           entries, entry j of the gate row and of the up row interleaved (gate j, up j, ...),
           rows padded with weight-0 entries to the wave's longest row in the pass
    meta B its down rows, its long row, the wave's down passes
    D      down-row passes of fixed lengths (DLEN): one residual row's entries each, padded

The kernel prefetches three regions (w1 + meta A, the unit passes, meta B + the down passes)
each into its own registers right after its last use, in the order the next layer uses them.

Everything a wave does is then at slot positions known at compile time, with wave-uniform loop
bounds, so the kernel keeps the tables in registers and wastes no gather on a dead slot. Units
and rows longer than a pass (rare at the chip's density) are "long": their entries go to small
per-layer tables, resident in the chain's LDS with the gate tables, that a lane walks with a
plain loop.

Sums keep the oracle's order: a unit's gate and up rows in column order (the packer sorts each
row), a residual row's down entries in the model's unit order, each from +0 (padding adds +0).
The chain's gates (the live query/key channels and decays) keep their own small tables, resident
in the chain's LDS for the whole launch.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

NT = 512
NW = NT // 64


@dataclass(frozen=True)
class Fmt:
    """The per-thread table's slot layout for one entry format (csrc/lxm_decode.hip: PT<E4>)."""
    e4: bool
    W1: int
    MA: int
    U0: int
    U1: int
    MB: int
    D: int
    WORDS: int
    G0MAX: int
    G1MAX: int
    DLEN: tuple

    @property
    def esz(self) -> int:  # slots per entry
        return 1 if self.e4 else 2

    @property
    def doff(self) -> tuple:  # entry offset of each down pass
        return tuple(int(x) for x in np.concatenate([[0], np.cumsum(self.DLEN)[:-1]]))


FMT_E4 = Fmt(True, W1=0, MA=4, U0=8, U1=14, MB=40, D=44, WORDS=15, G0MAX=3, G1MAX=13,
             DLEN=(1, 1, 2, 1, 4, 6))
FMT_E8 = Fmt(False, W1=0, MA=8, U0=12, U1=20, MB=36, D=40, WORDS=13, G0MAX=2, G1MAX=4,
             DLEN=(1, 1, 2, 2))
NONE16 = 0xFFFF


def fmt(e4: bool) -> Fmt:
    f = FMT_E4 if e4 else FMT_E8
    assert f.U1 == f.U0 + 2 * f.esz * f.G0MAX and f.MB >= f.U1 + 2 * f.esz * f.G1MAX
    assert f.MB % 4 == 0 and f.U0 % 4 == 0 and f.MA % 4 == 0 and f.D == f.MB + 4
    assert f.D + f.esz * sum(f.DLEN) <= 4 * f.WORDS and f.MA + 4 <= f.U0 and len(f.DLEN) <= 6
    return f


def _bf16_bits(v) -> np.ndarray:
    u = np.ascontiguousarray(v, np.float32).view(np.uint32)
    assert np.all((u & 0xFFFF) == 0), "a value is not exact in bf16"
    return u >> 16


def _slots_of(f: Fmt, off: int, val: float) -> list:
    """One entry as slots: e4 (byte offset | bf16 << 16), else (byte offset, float bits)."""
    u = int(np.float32(val).view(np.uint32))
    if f.e4:
        assert u & 0xFFFF == 0, "a value is not exact in bf16"
        return [int(off) | (u & 0xFFFF0000)]
    return [int(off), u]


@dataclass
class LayerTables:
    ptt: bytes          # WORDS x NT 16-byte words, word j of thread t at (j * NT + t) * 16
    wave_words: int     # byte w: the RU words (low nibble) and RB words (high nibble) wave w loads
    long_u: bytes       # lxm_longu[n]
    long_r: bytes       # lxm_longr[n]
    long_ent: bytes     # their entries (unit: byte offsets into xm; row: into act)
    stats: dict


def pack_layer(f: Fmt, H: int, units, gate_rows, up_rows, down_rows, w_post) -> LayerTables:
    """The chain tables of one layer.

    units: the live units' model indices in packed (act) order; gate_rows / up_rows: per packed
    unit (cols, vals) sorted by column; down_rows: per residual row r < H, (act indices, vals) in
    the model's unit order; w_post: the MLP norm's raw weights (H,)."""
    assert H <= 8 * NT
    S = np.zeros((NT, 4 * f.WORDS), np.uint64)
    esz = f.esz

    # ---- w1: the thread's rows 4t..4t+3 and 2048+4t..2048+4t+3
    w = np.zeros(8 * NT, np.float32)
    w[:H] = w_post
    rows = np.concatenate([4 * np.arange(NT)[:, None] + np.arange(4)[None],
                           2048 + 4 * np.arange(NT)[:, None] + np.arange(4)[None]], 1)
    wt = w[rows]  # (NT, 8)
    if f.e4:  # the raw weights' bf16 bits, two per slot (the kernel forms 1 + w in fp32)
        b = _bf16_bits(wt).astype(np.uint64)
        for k in range(4):
            S[:, f.W1 + k] = b[:, 2 * k] | (b[:, 2 * k + 1] << 16)
    else:  # 1 + w in fp32, as (1.0 + weight.float()) forms it
        S[:, f.W1:f.W1 + 8] = (np.float32(1.0) + wt).astype(np.float32).view(np.uint32)

    # ---- units: passes P0 (rows <= G0MAX) and P1 (<= G1MAX), the rest long
    n = len(units)
    gl = np.array([len(c) for c, _ in gate_rows], np.int64)
    ul = np.array([len(c) for c, _ in up_rows], np.int64)
    m = np.maximum(gl, ul) if n else np.zeros(0, np.int64)
    shared = np.array([len(gate_rows[k][0]) == len(up_rows[k][0]) and
                       np.array_equal(gate_rows[k][0], up_rows[k][0]) for k in range(n)], bool)
    order = np.argsort(m, kind="stable")
    p0 = [int(k) for k in order if m[k] <= f.G0MAX][:NT]
    in0 = set(p0)
    rest = [int(k) for k in order[::-1] if m[k] <= f.G1MAX and k not in in0]
    p1, longu = rest[:NT], rest[NT:] + [k for k in range(n) if m[k] > f.G1MAX]
    meta0 = np.zeros(NT, np.uint64)
    G = np.zeros((2, NW), np.int64)
    sh = np.ones((2, NW), bool)
    # lanes: P1 longest first over waves 3, 1, 0, 2, 4, 5, 6, 7 (wave w issues on SIMD w % 4, so
    # the longest units go to wave 3, whose SIMD partner is the query/key wave 7 with one P0
    # entry, and wave 6, the decays' wave, takes the shortest); P0 longest first over waves
    # 1..5, then wave 0 and the top two waves (the gates). Measured against P1 from lane 0: config
    # 2 6,778 -> 6,834 tok/s, config 5 2,396 -> 2,429.
    lanes0 = list(range(64, NT - 128)) + list(range(64)) + list(range(NT - 128, NT))
    lanes1 = [64 * w + lane for w in (3, 1, 0, 2, 4, 5, 6, 7) for lane in range(64)]
    p0 = sorted(p0, key=lambda k: -m[k])
    placed = ((p0, lanes0, f.U0), (p1, lanes1, f.U1))
    for p, (lst, lanes, base) in enumerate(placed):
        for k, lane in zip(lst, lanes):
            wv = lane // 64
            G[p, wv] = max(G[p, wv], m[k])
            sh[p, wv] &= bool(shared[k])
    # "fly": every unit pass of the layer shares its columns (and no unit is long, 4-byte
    # entries): the kernel forms the MLP norm's output per gathered column from the residual,
    # D((h * r) * (1 + w)), instead of writing it for every row first; the up slot's free low
    # half then carries the column's raw norm weight w (bf16 bits)
    fly = bool(f.e4 and sh.all() and len(p0) + len(p1) == n)
    wbits = _bf16_bits(np.asarray(w_post, np.float32)) if fly else None
    for p, (lst, lanes, base) in enumerate(placed):
        for k, lane in zip(lst, lanes):
            wv = lane // 64
            meta0[lane] |= np.uint64((k | 0x8000) << (16 * p))
            for j, (c, v) in enumerate(zip(*gate_rows[k])):
                S[lane, base + 2 * esz * j:base + 2 * esz * j + esz] = _slots_of(f, 4 * c, v)
            # (a wave whose pass shares columns reads the up slots as bare weights: offset 0,
            # or in a fly layer the column's norm weight)
            bare = f.e4 and sh[p, wv]
            for j, (c, v) in enumerate(zip(*up_rows[k])):
                sl = _slots_of(f, 0 if bare else 4 * c, v)
                if fly:
                    sl = [int(sl[0]) | int(wbits[c])]
                S[lane, base + 2 * esz * j + esz:base + 2 * esz * (j + 1)] = sl
    assert n < 1 << 12
    S[:, f.MA + 0] = meta0

    # ---- down rows: passes of fixed lengths, the rest long
    dl = np.array([len(down_rows[r][0]) for r in range(H)], np.int64)
    nq = len(f.DLEN)
    # the longest pass fills from the top lane down (the top wave has the fewest unit slots),
    # the others from lane 0 up
    free = [list(range(NT))[::-1] if f.DLEN[q] == max(f.DLEN) and q > 0 else list(range(NT))
            for q in range(nq)]
    place = {}
    longr = []
    for r in np.argsort(-dl, kind="stable"):
        if dl[r] == 0:
            break
        qs = sorted((q for q in range(nq) if f.DLEN[q] >= dl[r] and free[q]),
                    key=lambda q: (f.DLEN[q], q))
        if not qs:
            longr.append(int(r))
            continue
        q = qs[0]
        place[int(r)] = (q, free[q].pop(0))
    # where each pass's sum goes: the byte offset from dsum of its row, else of the lane's dummy
    # slot (the kernel's L_DUMMY follows dsum's 4096 rows)
    rowf = np.tile((4 * 4096 + 4 * np.arange(NT, dtype=np.uint64))[:, None], (1, 6))
    dmask = np.zeros(NW, np.int64)
    doff = f.doff
    for r, (q, lane) in place.items():
        rowf[lane, q] = 4 * r
        dmask[lane // 64] |= 1 << q
        for j, (a, v) in enumerate(zip(*down_rows[r])):
            s0 = f.D + esz * (doff[q] + j)
            S[lane, s0:s0 + esz] = _slots_of(f, 4 * int(a), v)
    for k in range(3):
        S[:, f.MB + k] = rowf[:, 2 * k] | (rowf[:, 2 * k + 1] << 16)

    # ---- long units and rows: tables of global entries, one item per lane
    assert len(longu) <= NT and len(longr) <= NT, "too many long units or rows"
    lu, lr, ents = [], [], []
    epos = 0

    def add(cols, vals, scale=4):
        nonlocal epos
        start = epos
        for c, v in zip(cols, vals):
            ents.append(_slots_of(f, scale * int(c), v))
        epos += len(cols)
        return start

    # long item i on lane NT - 1 - i: the top wave has the fewest unit passes (P1 fills from lane
    # 0, its longest units first)
    long_u_idx = np.full(NT, NONE16, np.uint64)
    long_r_idx = np.full(NT, NONE16, np.uint64)
    for i, k in enumerate(longu):
        gs = add(*gate_rows[k])
        us = add(*up_rows[k])
        lu.append(np.array([k, gs, len(gate_rows[k][0]), us, len(up_rows[k][0]), 0, 0, 0], np.int32))
        long_u_idx[NT - 1 - i] = i
    for i, r in enumerate(longr):
        s0 = add(*down_rows[r])
        lr.append(np.array([r, s0, len(down_rows[r][0]), 0], np.int32))
        long_r_idx[NT - 1 - i] = i
    S[:, f.MA + 1] = long_u_idx
    for _ in range(8):  # the long loop reads up to 4 entries past a row's end
        ents.append([0] * esz)
    anyu = np.zeros(NW, bool)
    anyr = np.zeros(NW, bool)
    anyu[(NT - 1 - np.arange(len(longu))) // 64] = True
    anyr[(NT - 1 - np.arange(len(longr))) // 64] = True

    # ---- the wave-uniform words (meta A +2; meta B +3 above its lane's long row)
    for wv in range(NW):
        wa = (int(G[0, wv]) | (int(G[1, wv]) << 4) | (int(sh[0, wv]) << 8) |
              (int(sh[1, wv]) << 9) | (int(anyu[wv]) << 10) | (int(fly) << 11))
        S[wv * 64:(wv + 1) * 64, f.MA + 2] = wa
        wb = (int(dmask[wv]) << 16) | (int(anyr[wv]) << 24)
        S[wv * 64:(wv + 1) * 64, f.MB + 3] = long_r_idx[wv * 64:(wv + 1) * 64] | np.uint64(wb)

    # ---- the words each wave loads of the unit and down regions (its passes' last slots)
    ru_a, rb_a = f.U0 // 4, f.MB // 4
    wave_words = 0
    for wv in range(NW):
        last_u = -1
        if G[1, wv]:
            last_u = f.U1 + 2 * esz * int(G[1, wv]) - 1
        elif G[0, wv]:
            last_u = f.U0 + 2 * esz * int(G[0, wv]) - 1
        nu = 0 if last_u < 0 else last_u // 4 - ru_a + 1
        last_d = f.MB + 3
        for q in range(nq):
            if dmask[wv] >> q & 1:
                last_d = max(last_d, f.D + esz * (doff[q] + f.DLEN[q]) - 1)
        nb = last_d // 4 - rb_a + 1
        assert nu <= (f.MB - f.U0) // 4 < 16 and nb <= f.WORDS - rb_a < 16
        wave_words |= (nu | (nb << 4)) << (8 * wv)
    assert S.max() < 1 << 32
    # thread-interleaved words: word j of thread t at (j * NT + t)
    words = S.astype(np.uint32).reshape(NT, f.WORDS, 4).transpose(1, 0, 2)
    used_g = sum(len(gate_rows[k][0]) + len(up_rows[k][0]) for k in p0 + p1)
    slots_g = sum(2 * int(G[p, wv]) * 64 for p in range(2) for wv in range(NW))
    stats = {"p0": len(p0), "p1": len(p1), "long_units": len(longu), "long_rows": len(longr),
             "unit_fill": round(used_g / max(slots_g, 1), 3), "G": G.tolist(),
             "down_mask": dmask.tolist(), "fly": fly}
    ent_arr = np.array(ents, np.uint32).reshape(-1) if ents else np.zeros(0, np.uint32)
    # 16-byte words a thread loads per layer, averaged over the waves
    stats["words_per_thread"] = sum(f.U0 // 4 + ((wave_words >> (8 * w)) & 15) +
                                    ((wave_words >> (8 * w + 4)) & 15) for w in range(NW)) / NW
    return LayerTables(ptt=words.tobytes(), wave_words=wave_words,
                       long_u=b"".join(x.tobytes() for x in lu),
                       long_r=b"".join(x.tobytes() for x in lr),
                       long_ent=ent_arr.tobytes(), stats=stats)


def decode_ptt(f: Fmt, ptt: bytes) -> np.ndarray:
    """The per-thread slots (NT, 4 WORDS) of a packed table (tests)."""
    a = np.frombuffer(ptt, np.uint32).reshape(f.WORDS, NT, 4).transpose(1, 0, 2)
    return a.reshape(NT, 4 * f.WORDS)
