"""The chip layers without the zeros (lx/lx/fast.py's role): which rows, columns, units and heads
of the checkpoint tensors are live, and the tables the decode kernel is packed from.

    f = Fast(model, n_chip, rows)    # model: a transformers Qwen3_5ForCausalLM, or a SparseModel
    m = Mega(f, model, cache, offset)

What is skipped, and why that changes nothing (lx/lx/fast.py:8-19): weight rows and columns that
are all zero (a dead output is exactly 0, a dead input contributes exactly 0), MLP units whose
gate row, up row or down column is zero (lx/lx/fast.py:242-248), head columns the final norm
zeroes, and key heads whose query, key and decay are all zero at a step (their state stays as it
is and their output is exactly 0).
"""

from __future__ import annotations

import numpy as np
import torch

from . import synth


# the chip layers' projection modules (the weights Fast packs from)
PROJ = ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj", "gate_proj", "up_proj",
        "down_proj")


def place_lean(model, n_chip: int, dev) -> None:
    """lx.fast.place_lean (lx/lx/fast.py:33-46): a transformers model moved to dev except its
    first n_chip layers' projections (the chip's 0.08 %-dense weights, which Fast packs and the
    device never needs in full); build Fast from the model first, then Fast.to(dev)."""
    kept = []
    for layer in model.model.layers[:n_chip]:
        for mod in layer.modules():
            for name in PROJ:
                lin = getattr(mod, name, None)
                if isinstance(lin, torch.nn.Linear):
                    kept.append((lin, lin.weight))
                    lin.weight = None  # (a None parameter is skipped by Module.to)
    model.to(dev)
    for lin, w in kept:
        lin.weight = w


class Rows:
    """CSR rows (ptr, cols, vals) of a Coo's row range."""

    def __init__(self, coo, lo: int = 0, hi: int | None = None):
        hi = coo.shape[0] if hi is None else hi
        sel = (coo.rows >= lo) & (coo.rows < hi)
        rows, self.cols, self.vals = coo.rows[sel] - lo, coo.cols[sel], coo.vals[sel]
        self.n = hi - lo
        self.ptr = np.zeros(self.n + 1, np.int64)
        np.cumsum(np.bincount(rows, minlength=self.n), out=self.ptr[1:])


class Fast:
    """lx.fast.Fast (lx/lx/fast.py:172-185): built once from the model's tensors."""

    def __init__(self, model, n_chip: int | None = None, rows: slice | None = None):
        self.model = model
        if isinstance(model, synth.SparseModel):
            self.sm, self.row0 = model, 0
        else:
            # only the chip's rows of the head are read (lx/lx/fast.py:183's lm_head.weight[rows]):
            # the coordinate model's embedding holds rows row0 .. row0 + vocab of the model's
            self.sm = synth.from_hf(model, n_chip, rows)
            self.row0 = int(self.sm.meta.get("row0", 0))
        d = self.sm.dims
        self.n_chip = d.n_layers
        self.nk, self.nv, self.kd, self.vd = d.nk, d.nv, d.kd, d.vd
        self.r = d.nv // d.nk
        self.rows = rows
        n_all = self.row0 + d.vocab  # rows of the model's embedding this Fast can see
        lo = 0 if rows is None else (rows.start or 0)
        hi = n_all if rows is None or rows.stop is None else rows.stop
        if (rows is not None and rows.step not in (None, 1)) or not self.row0 <= lo < hi <= n_all:
            raise ValueError(f"rows {rows}: not a range of the embedding's rows "
                             f"{self.row0} .. {n_all}")
        self.head_range = (lo, hi)
        w1 = np.float32(1.0) + np.asarray(self.sm.norm, np.float32)
        self.head_cols = np.nonzero(w1 != 0)[0]
        self.dec = [self._live(L) for L in range(self.n_chip)]

    lean = False       # lx.fast's flags (lx/lx/fast.py:388-397): the projections are not on the
    head_block = None  # device (place_lean); the head's row block (the kernel picks its own)

    def to(self, dev) -> "Fast":
        """Fast.to (lx/lx/fast.py:399-418): everything Fast needs on dev (the packed tables of
        the verified-mode kernels, built from host memory), so the model's own projections may
        stay on the host (place_lean)."""
        self.prefill(dev)
        return self

    def init_cache(self, cache, dev) -> None:
        """Fast.init_cache (lx/lx/fast.py:420-430): the chip layers' states as the stock forward
        of one zero token leaves them, all zero (conv windows in the model dtype, recurrent states
        float32). cache: a transformers DynamicCache or a StateCache."""
        d = self.sm.dims
        conv = torch.zeros(1, d.n_conv, 1, dtype=self._dtype(), device=dev)
        rec = torch.zeros(1, d.nv, d.kd, d.vd, dtype=torch.float32, device=dev)
        for L in range(self.n_chip):
            if hasattr(cache, "update_conv_state"):
                cache.update_conv_state(conv, L, conv_kernel_size=d.conv)
                ly = cache.layers[L]
                if hasattr(ly, "update_recurrent_state"):
                    ly.update_recurrent_state(rec.clone())
                else:
                    cache.update_recurrent_state(rec.clone(), L)
            else:
                ly = cache.layers[L]
                ly.conv_states[0] = torch.zeros(1, d.n_conv, d.conv, dtype=self._dtype(),
                                                device=dev)
                ly.recurrent_states[0] = rec.clone()

    def _live(self, L: int) -> dict:
        """A layer's live parts (lx/lx/fast.py:187-248): key heads with a live query or key
        channel, value heads that can decay, MLP units, out_proj rows."""
        ly, d = self.sm.layers[L], self.sm.dims
        taps = np.asarray(ly.conv1d)
        live = (taps != 0).any(1)
        nq = d.nk * d.kd
        kh = np.nonzero(live[:nq].reshape(d.nk, d.kd).any(1) |
                        live[nq:2 * nq].reshape(d.nk, d.kd).any(1))[0]
        g = np.bincount(ly.gate_proj.rows, minlength=d.inter) > 0
        u = np.bincount(ly.up_proj.rows, minlength=d.inter) > 0
        dn = np.bincount(ly.down_proj.cols, minlength=d.inter) > 0
        return {"kh": kh, "units": np.nonzero(g & u & dn)[0],
                "decays": np.unique(ly.in_proj_a.rows),
                "out_rows": np.unique(ly.out_proj.rows)}

    # ---- verified mode: the native prefill (linuxformer_amd/prefill.py)
    def prefill(self, device="cuda"):
        """The packed prefill tables on device (built once per device)."""
        from .prefill import Prefill

        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        if getattr(self, "_pf", None) is None or self._pf.dev != dev:
            self._pf = Prefill(self, dev)
        return self._pf

    def _dtype(self):
        return torch.bfloat16 if self.sm.dims.dtype == "bf16" else torch.float32

    @torch.no_grad()
    def forward(self, h: torch.Tensor, cache) -> torch.Tensor:
        """h (1, T, hidden) -> (1, T, hidden), updating the cache's conv and recurrent states
        (lx/lx/fast.py:252-258). Each position sees exactly the stock decode step."""
        assert h.dim() == 3 and h.shape[0] == 1 and h.shape[2] == self.sm.dims.hidden
        pf = self.prefill(h.device)
        T = h.shape[1]
        pf.to_tiles(h[0].to(self._dtype()))
        pf.layers(T, cache)
        return pf.from_tiles(T)[None]

    @torch.no_grad()
    def layer(self, L: int, h: torch.Tensor, cache) -> None:
        """One chip layer on h (T, hidden), in place (lx/lx/fast.py:260-269)."""
        assert h.dim() == 2 and h.shape[1] == self.sm.dims.hidden and h.dtype == self._dtype()
        pf = self.prefill(h.device)
        T = h.shape[0]
        pf.to_tiles(h)
        pf.layers(T, cache, L, L + 1)
        h.copy_(pf.from_tiles(T))

    @torch.no_grad()
    def head_argmax(self, h: torch.Tensor, block: int | None = None) -> torch.Tensor:
        """The final norm and the tied head's first maximum at each position of h (T, hidden)
        or (1, T, hidden): int64 (T,) (lx/lx/fast.py:544-550; block sizes are the kernel's
        own)."""
        x = h.reshape(-1, self.sm.dims.hidden).to(self._dtype())
        pf = self.prefill(h.device)
        pf.to_tiles(x)
        return pf.head(x.shape[0]).to(torch.int64).clone()

    @torch.no_grad()
    def decode(self, h: torch.Tensor, cache) -> torch.Tensor:
        """One decode step of every chip layer on h (1, 1, hidden) (lx/lx/fast.py:365-540):
        the forward of a single position."""
        return self.forward(h, cache)

    @torch.no_grad()
    def verify(self, tokens, cache) -> torch.Tensor:
        """Verified mode end to end: the tokens' embedding rows, every layer, the head; returns
        each position's prediction (int32, on the device; prediction i is for token i + 1)."""
        return self.prefill().verify(tokens, cache)

    def embed_rows(self, offset: int | None = None) -> Rows:
        """The chip tokens' embedding rows (all columns): the head's rows (``rows``, or every row),
        which are also the inputs' rows, chip token t at row offset + t (lx/csrc/mega.cu:647-651's
        embed[tok + offset]); a given offset must be where those rows start."""
        lo, hi = self.head_range
        if offset is not None and offset != lo:
            raise ValueError(f"offset {offset}: the chip's rows start at {lo} (Fast's rows="
                             f"{self.rows}); the tied head and the inputs share them")
        return Rows(self.sm.embed, lo - self.row0, hi - self.row0)


class _CacheLayer:
    def __init__(self, conv: torch.Tensor, rec: torch.Tensor):
        self.conv_states = {0: conv}
        self.recurrent_states = {0: rec}


class StateCache:
    """The chip layers' states in transformers' LinearAttentionLayer layout
    (transformers/cache_utils.py:998-1080): layers[L].conv_states[0] (1, n_conv, 4) in the model
    dtype, layers[L].recurrent_states[0] (1, nv, kd, vd) float32."""

    def __init__(self, conv: np.ndarray, rec: np.ndarray, dtype: str, device):
        dt = torch.bfloat16 if dtype == "bf16" else torch.float32
        self.layers = [
            _CacheLayer(torch.from_numpy(np.ascontiguousarray(conv[L]))[None].to(device=device, dtype=dt),
                        torch.from_numpy(np.ascontiguousarray(rec[L]))[None].to(device=device))
            for L in range(conv.shape[0])]

    def conv_numpy(self) -> np.ndarray:
        return np.stack([l.conv_states[0][0].float().cpu().numpy() for l in self.layers])

    def rec_numpy(self) -> np.ndarray:
        return np.stack([l.recurrent_states[0][0].cpu().numpy() for l in self.layers])
