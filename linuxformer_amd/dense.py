"""Greedy decode of the dense padded text-view stack (benchmark config 4) on the native dense
kernels (csrc/lxm_dense.hip, C ABI include/lxm_dense.h).

    dd = DenseDecode(model, cache)            # model: synth.DenseModel on the GPU
    preds = dd.run(forced, n)                 # lx.mega's run semantics: step i's input is
                                              # forced[i] (i < len(forced)), else pred[i - 1]
    dd.prefill(prompt[:-1]); dd.run(prompt[-1:], n)   # the same states and predictions from the
                                              # last prompt token on, the prompt in batches

By default ``run`` calls lxm_dn_step per step (embedding, 24 layers, the head's argmax, the token
fed back), whose step counter and fed-back token live on the device, so it captures a step in a
graph once and replays it per token; mode "persistent" makes all n steps in one launch
(lxm_dn_run: one workgroup per CU, grid barriers between the layers' phases). The cache
holds the states in transformers' layout (conv (1, n_conv, 4) bf16, recurrent (1, nv, 256, 128)
fp32) and is updated in place.
"""

from __future__ import annotations

import ctypes

import torch

from . import mk_build

P64 = ctypes.c_void_p


class DnLayer(ctypes.Structure):
    _fields_ = [(n, P64) for n in ("proj", "conv_qk", "conv_v", "A_log", "dt_bias", "gnorm",
                                   "ln_in", "ln_post", "out", "gate", "up", "down", "rec",
                                   "conv")]


class DnPbuf(ctypes.Structure):
    _fields_ = [(n, P64) for n in ("h", "xn", "P", "qk", "v", "g", "live", "o", "ys", "act", "gl")]


PB = 16  # tokens per prefill batch (LXM_DN_PB)
CHUNK = 64  # tokens per chunk of the chunked prompt (LXM_CHUNK)


class DnParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("hidden", "n_layers", "nk", "kl", "nv", "rl",
                                              "inter", "vocab", "n_conv")] + \
        [("rms_eps", ctypes.c_float), ("geps", ctypes.c_float)] + \
        [(n, ctypes.c_int32) for n in ("n_forced", "n_steps", "pad")] + \
        [(n, P64) for n in ("layers", "layers_host", "embed", "w_final", "forced", "preds", "step",
                            "tok", "h", "xn", "P", "on", "keys", "err", "sync", "prof")]


def interleave(w):
    """Rows (n, K) bf16 in the kernels' order: each lane's K / 64 entries in 8-entry chunks,
    chunk q of lane l at (q * 64 + l) * 8 (K / 64 = 4: unchanged)."""
    n, K = w.shape
    G = K // 64
    assert K % 64 == 0 and (G == 4 or G % 8 == 0), K
    if G == 4:
        return w.contiguous()
    return w.reshape(n, 64, G // 8, 8).transpose(1, 2).contiguous().reshape(n, K)


class DenseDecode:
    """The packed weights of a DenseModel and the decode driver over a cache."""

    def __init__(self, model, cache, max_steps: int = 1 << 16, subprof: bool = False):
        self.model, self.cache = model, cache
        sp, d = model.spec, model.dims
        self.spec, self.dims = sp, d
        self.dev = model.embed.device
        self.lib = mk_build.load(subprof)  # (subprof: the build with the phase clocks)
        H, nk, kl, rl, I = sp.hidden, sp.nk, sp.kd_live, sp.r_live, sp.inter
        R = d.nv // d.nk
        self.nproj = 2 * nk * kl + 2 * nk * rl * 128 + 2 * nk * rl
        self._keep = []
        self.layers_h = (DnLayer * d.n_layers)()
        for L, ly in enumerate(model.layers):
            proj = torch.cat([ly["qk"][0].reshape(-1, H), ly["qk"][1].reshape(-1, H),
                              ly["v"].reshape(-1, H), ly["z"].reshape(-1, H),
                              ly["b"].reshape(-1, H), ly["a"].reshape(-1, H)]).contiguous()
            assert proj.shape[0] == self.nproj
            tens = dict(proj=interleave(proj), conv_qk=ly["conv_qk"].contiguous(),
                        conv_v=ly["conv_v"].contiguous(), A_log=ly["A_log"].contiguous(),
                        dt_bias=ly["dt_bias"].contiguous(), gnorm=ly["norm"].contiguous(),
                        ln_in=ly["ln_in"].contiguous(), ln_post=ly["ln_post"].contiguous(),
                        out=interleave(ly["out"].reshape(H, -1)), gate=interleave(ly["gate"]),
                        up=interleave(ly["up"]), down=interleave(ly["down"]))
            self._keep.append(tens)
            cl = cache.layers[L]
            rec, conv = cl.recurrent_states[0], cl.conv_states[0]
            assert rec.dtype == torch.float32 and rec.is_contiguous() and rec.device == self.dev
            assert conv.dtype == torch.bfloat16 and conv.is_contiguous() and conv.device == self.dev
            # the zero value heads and the zero-padded key dims must hold zero state and windows
            # (the kernels leave them alone; the stock layer keeps them zero)
            rv = rec[0].view(nk, R, 256, 128)
            cv = conv[0]
            assert not rv[:, rl:].any() and not rv[:, :rl, kl:].any(), "dead heads' state != 0"
            qk = cv[:2 * nk * 256].view(2, nk, 256, 4)
            vv = cv[2 * nk * 256:].view(nk, R, 128, 4)
            assert not qk[:, :, kl:].any() and not vv[:, rl:].any(), "dead channels' windows != 0"
            lay = self.layers_h[L]
            for k, t in tens.items():
                setattr(lay, k, t.data_ptr())
            lay.rec, lay.conv = rec.data_ptr(), conv.data_ptr()
        self.layers_d = torch.frombuffer(bytearray(bytes(self.layers_h)), dtype=torch.uint8).to(self.dev)
        self.embed = interleave(model.embed)  # (the head's rows, and the embedding through it)
        dev = self.dev
        self.h = torch.zeros(H, dtype=torch.float32, device=dev)
        self.xn = torch.zeros(H + I, dtype=torch.float32, device=dev)
        self.P = torch.zeros(self.nproj, dtype=torch.float32, device=dev)
        self.on = torch.zeros(nk * rl * 128, dtype=torch.float32, device=dev)
        self.keys = torch.zeros(2, dtype=torch.int64, device=dev)
        self.sync = torch.zeros(256, dtype=torch.int32, device=dev)
        self.step = torch.zeros(1, dtype=torch.int32, device=dev)
        self.tok = torch.zeros(1, dtype=torch.int32, device=dev)
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)
        self.preds = torch.zeros(max_steps, dtype=torch.int32, device=dev)
        self.forced = torch.zeros(max_steps, dtype=torch.int32, device=dev)
        self.max_steps = max_steps
        self.graph = None
        self._pb = None

    def _params(self, n_forced: int, prof: int = 0):
        sp, d = self.spec, self.dims
        p = DnParams(hidden=sp.hidden, n_layers=d.n_layers, nk=sp.nk, kl=sp.kd_live, nv=d.nv,
                     rl=sp.r_live, inter=sp.inter, vocab=sp.vocab, n_conv=d.n_conv,
                     rms_eps=sp.rms_eps, geps=sp.gated_eps, n_forced=n_forced,
                     n_steps=self.max_steps, layers=self.layers_d.data_ptr(),
                     layers_host=ctypes.cast(self.layers_h, P64).value,
                     embed=self.embed.data_ptr(), w_final=self.model.norm.data_ptr(),
                     forced=self.forced.data_ptr(), preds=self.preds.data_ptr(),
                     step=self.step.data_ptr(), tok=self.tok.data_ptr(), h=self.h.data_ptr(),
                     xn=self.xn.data_ptr(), P=self.P.data_ptr(), on=self.on.data_ptr(),
                     keys=self.keys.data_ptr(), err=self.err.data_ptr(),
                     sync=self.sync.data_ptr(), prof=prof)
        pd = torch.frombuffer(bytearray(bytes(p)), dtype=torch.uint8).to(self.dev)
        return p, pd

    def _pbuf(self, chunked: bool = False):
        """The prompt's buffers (allocated on first use): PB tokens for the batched prefill,
        CHUNK tokens (and the log decays) for the chunked one."""
        key = "_pbc" if chunked else "_pb"
        if getattr(self, key, None) is None:
            sp = self.spec
            H, nk, rl, I = sp.hidden, sp.nk, sp.r_live, sp.inter
            nvr = nk * rl * 128
            sizes = dict(h=H, xn=H, P=self.nproj, qk=nk * 2 * 256, v=nvr, g=nk * rl * 2,
                         live=nk * 2, o=nvr, ys=nvr, act=I)
            if chunked:
                sizes["gl"] = nk * rl
            bf = ("xn", "ys", "act")  # (the row kernels' inputs, bf16)
            nt = CHUNK if chunked else PB
            ts = {k: torch.zeros(nt * n, device=self.dev,
                                 dtype=torch.bfloat16 if k in bf else torch.float32)
                  for k, n in sizes.items()}
            setattr(self, key + "_t", ts)
            setattr(self, key, DnPbuf(**{k: t.data_ptr() for k, t in ts.items()}))
        return getattr(self, key)

    def prefill(self, tokens, mode: str = "batched") -> None:
        """The tokens through every layer without the head; no predictions are made. A caller
        then steps from the next token: run([next], n).

        mode "batched" (lxm_dn_prefill: batches of PB tokens, each weight row read once per
        batch): the cache's states and windows afterwards are those of len(tokens) forced steps
        of run(), bit for bit. mode "chunked" (lxm_dn_prefill_chunked): the stock forward's
        T > 1 path, the delta rule in chunks of 64 on the matrix cores
        (torch_chunk_gated_delta_rule); every other sum as in "batched", the delta rule's outputs
        and states those of the chunked form."""
        if mode not in ("batched", "chunked"):
            raise ValueError(f"prefill mode {mode!r}: 'batched' or 'chunked'")
        t = torch.as_tensor(tokens, dtype=torch.int64)
        if t.numel() == 0:
            return
        if int(t.min()) < 0 or int(t.max()) >= self.spec.vocab:
            raise ValueError("prefill token out of range")
        chunked = mode == "chunked"
        pb = self._pbuf(chunked)
        tok = t.to(torch.int32).to(self.dev)
        self.err.zero_()
        p, _ = self._params(1)
        st = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        fn = self.lib.lxm_dn_prefill_chunked if chunked else self.lib.lxm_dn_prefill
        e = fn(ctypes.byref(p), ctypes.c_void_p(tok.data_ptr()), int(t.numel()), ctypes.byref(pb), st)
        if e:
            raise RuntimeError(f"dense prefill launch failed: hipError {e}")
        torch.cuda.synchronize(self.dev)
        if int(self.err.item()):
            raise RuntimeError("dense prefill: a token out of range")

    def _step(self) -> None:
        st = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        e = self.lib.lxm_dn_step(ctypes.byref(self._p), ctypes.c_void_p(self._pd.data_ptr()), st)
        if e:
            raise RuntimeError(f"dense decode launch failed: hipError {e}")

    @torch.no_grad()
    def run(self, forced, n: int, graph: bool = True, mode: str = "steps", prof=None) -> list:
        """n greedy steps from the cache's states (updated in place); step i's input is forced[i]
        for i < len(forced), else step i - 1's prediction. Returns the n predictions. mode
        "steps": lxm_dn_step per step (graph: the first step eagerly, one step captured
        (capturing runs nothing) and replayed for the others; the step reads its index and input
        from device memory); "persistent": one launch of lxm_dn_run for all n steps (the same
        results; for callers that cannot capture graphs). prof: with a DenseDecode built with
        subprof=True and mode "persistent", an int64 tensor of 32 x (workgroups) that receives
        the run's phase clock (include/lxm_dense.h)."""
        f = torch.as_tensor(forced, dtype=torch.int64)
        if len(f) == 0 or n < 1 or n > self.max_steps or len(f) > self.max_steps:
            raise ValueError("forced tokens and steps: 1 .. max_steps")
        if int(f.min()) < 0 or int(f.max()) >= self.spec.vocab:
            raise ValueError("forced token out of range")
        if mode not in ("persistent", "steps"):
            raise ValueError(f"mode: persistent or steps, not {mode!r}")
        self.forced[:len(f)].copy_(f.to(torch.int32))
        self.step.zero_()
        self.err.zero_()
        self.keys.zero_()
        self.sync.zero_()
        if prof is not None:
            ncu = torch.cuda.get_device_properties(self.dev).multi_processor_count
            if prof.dtype != torch.int64 or not prof.is_cuda or prof.numel() < 32 * ncu:
                raise ValueError("prof: an int64 device tensor of at least 32 x (the device's "
                                 "CUs) entries")
        pp = 0 if prof is None else prof.data_ptr()
        if getattr(self, "_nf", None) != len(f) or getattr(self, "_pp", 0) != pp:
            self._p, self._pd = self._params(len(f), pp)
            self._nf, self._pp, self.graph = len(f), pp, None
        if mode == "persistent":
            st = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
            mk_build.note_cooperative()
            e = self.lib.lxm_dn_run(ctypes.byref(self._p), ctypes.c_void_p(self._pd.data_ptr()), n, st)
            if e:
                raise RuntimeError(f"dense decode launch failed: hipError {e}")
        else:
            self._step()
            if graph and n > 1:
                if self.graph is None:
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g):
                        self._step()
                    self.graph = g
                for _ in range(n - 1):
                    self.graph.replay()
            else:
                for _ in range(n - 1):
                    self._step()
        torch.cuda.synchronize(self.dev)
        err = int(self.err.item())
        if err == 1:
            raise RuntimeError("dense decode: a forced token out of range")
        if err:
            raise RuntimeError(f"dense decode: a wait timed out (error {err})")
        return self.preds[:n].cpu().tolist()
