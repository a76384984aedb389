"""The non-mega decode as replayed HIP graphs: lx.session.Session's model-alone stepping
(lx/lx/session.py:148-225) on the verified-mode kernels at one position.

    s = Session(fast, cache)        # fast: a Fast; cache: the chip layers' states (in place)
    nxt = s.step(t)                 # token t alone (one graph replay); the model's prediction
    toks = s.free(n)                # n tokens, each the prediction of the one before

`step` replays one captured graph of a single-token step: the token's embedding row
(lxm_pf_embed, which reads the token from device memory), every chip layer (lxm_pf_layers at
T = 1: the kernels compute only the positions whose key heads or decays are live, so a value
head whose query, key and decay are all zero keeps its state and outputs 0, as
lx/lx/fast_kernels.py:1-6's idle-skip step does) and the head's first maximum (lxm_pf_head).
`free` replays a graph of run_k such steps in which each step's prediction is copied on the GPU
into the next step's token (lx/lx/session.py:196-205's `_capture_run`): one host synchronisation
per run_k tokens. The states afterwards, and every prediction, are those of the same forced or
greedy steps through `Mega.run`, bit for bit: the kernels are the prefill's, whose every position
is the stock decode step.

The graphs own their run buffers (one PfBuffers of one position), so other calls on the same
Fast (a verified-mode call of any length) never move them. The cache's state tensors must stay
where they are while the Session lives (the graphs hold their addresses); capture runs the step
eagerly once first and restores the states it changed.
"""

from __future__ import annotations

import ctypes

import torch


class Session:
    run_k = 64  # free() replays this many steps per graph, fed back on the GPU

    def __init__(self, fast, cache, device=None):
        dev = torch.device(device) if device is not None else \
            torch.device("cuda", torch.cuda.current_device())
        self.fast, self.cache, self.dev = fast, cache, dev
        self.pf = fast.prefill(dev)
        self.lib = self.pf.lib
        self.buf = self.pf.buffers(1)
        self._p, self._pd, self._keep = self.pf.bind(1, cache, self.buf)
        self.g_run = torch.zeros(self.run_k, dtype=torch.int32, device=dev)
        self.graph = None
        self.run_graph = None
        self.next = None  # the model's prediction after the last token run
        self.last = None  # the last token run
        self.n = 0        # tokens run

    # ------------------------------------------------------------------------------------------
    def _check(self, e: int, what: str) -> None:
        if e:
            raise RuntimeError(f"{what} failed: hipError {e}")

    def _body(self) -> None:
        """One step on the current stream: buf.tokens[0] -> every layer -> buf.preds[0]."""
        st = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        p, pd = ctypes.byref(self._p), ctypes.c_void_p(self._pd.data_ptr())
        self._check(self.lib.lxm_pf_embed(p, pd, st), "session embed")
        self._check(self.lib.lxm_pf_layers(p, pd, 0, self.pf.dims.n_layers, st), "session layers")
        self._check(self.lib.lxm_pf_head(p, pd, st), "session head")

    def _states(self):
        return [(ly.conv_states[0].clone(), ly.recurrent_states[0].clone())
                for ly in self.cache.layers]

    def _restore(self, saved) -> None:
        for ly, (c, r) in zip(self.cache.layers, saved):
            ly.conv_states[0].copy_(c)
            ly.recurrent_states[0].copy_(r)

    @torch.no_grad()
    def _capture(self) -> None:
        """The single-token step graph (lx/lx/session.py:148-163). The eager warm-up step changes
        the state: it is saved and put back."""
        saved = self._states()
        self._body()  # eager: the launchers' one-time set-up happens outside the capture
        torch.cuda.synchronize(self.dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._body()
        self._restore(saved)
        torch.cuda.synchronize(self.dev)

    @torch.no_grad()
    def _capture_run(self) -> None:
        """run_k steps in one graph, each step's prediction copied into the next step's token on
        the GPU (lx/lx/session.py:196-205)."""
        if self.graph is None:
            self._capture()
        self.run_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.run_graph):
            for i in range(self.run_k):
                self._body()
                self.g_run[i:i + 1].copy_(self.buf.preds[:1])
                self.buf.tokens.copy_(self.buf.preds[:1])

    def _token(self, t: int) -> None:
        if not 0 <= t < self.pf.vocab:
            raise ValueError(f"token {t} out of range [0, {self.pf.vocab})")
        self.buf.tokens.fill_(t)

    def _err(self) -> None:
        if int(self.buf.err.item()):
            raise RuntimeError("session: a token out of range reached the embedding")

    @torch.no_grad()
    def step(self, t: int) -> int:
        """Run token t alone (one graph replay); returns the model's next prediction
        (lx/lx/session.py:165-174)."""
        if self.graph is None:
            self._capture()
        self._token(t)
        self.graph.replay()
        self.next, self.last = int(self.buf.preds[0]), t
        self._err()
        self.n += 1
        return self.next

    @torch.no_grad()
    def free(self, n: int, stop=None, first: int | None = None) -> list:
        """Feed the model its own predictions for n tokens (or until stop(tokens) is true),
        starting from `first` (default: the last prediction); returns the tokens run
        (lx/lx/session.py:207-225)."""
        if first is not None:
            self.next = first
        if self.next is None:
            raise ValueError("free: no prediction to start from (step a token, or pass first)")
        out = []
        while stop is None and n - len(out) >= self.run_k:
            if self.run_graph is None:
                self._capture_run()
            self._token(self.next)
            self.run_graph.replay()
            pred = self.g_run.tolist()
            self._err()
            fed = [self.next] + pred[:-1]
            out += fed
            self.next, self.last = pred[-1], fed[-1]
            self.n += len(fed)
        while len(out) < n:
            t = self.next
            self.step(t)
            out.append(t)
            if stop and stop(out):
                break
        return out
