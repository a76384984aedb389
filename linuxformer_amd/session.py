"""The non-mega decode as replayed HIP graphs: lx.session.Session's model-alone stepping
(lx/lx/session.py:148-225) on the verified-mode kernels at one position.

    s = Session(fast, cache)        # fast: a Fast; cache: the chip layers' states (in place)
    nxt = s.step(t)                 # token t alone (one graph replay); the model's prediction
    toks = s.free(n)                # n tokens, each the prediction of the one before

A step is the token's embedding row (lxm_pf_embed), every chip layer (lxm_pf_layers at T = 1:
the kernels compute only the positions whose key heads or decays are live, so a value head whose
query, key and decay are all zero keeps its state and outputs 0, as lx/lx/fast_kernels.py:1-6's
idle-skip step does) and the head's first maximum (lxm_pf_head). The states afterwards, and every
prediction, are those of the same forced or greedy steps through `Mega.run`, bit for bit: the
kernels are the prefill's, whose every position is the stock decode step.

The chain of steps lives in one device ring of int32 words:

    ring[0]          the error word of every step (0: no error)
    ring[1 + i]      the token step i runs
    ring[2 + i]      step i's prediction, which is also step i + 1's token

Step i's parameter block points its token at ring[1 + i] and its prediction at ring[2 + i], so
a prediction is the next step's input where it is written: nothing is copied between steps. A
graph of k steps (captured once per k: k = 1 for `step`, k = run_k for `free`) is replayed after
one host write of (0, token) into ring[0:2], and one host read of ring[0 : k + 2] returns the
error word, the k tokens run and the prediction after them.

The session owns its run buffers (one position), so other calls on the same Fast (a
verified-mode call of any length) never move them. The cache's state tensors must stay where
they are while the Session lives (the graphs hold their addresses); a capture runs one step
eagerly first (the launchers' one-time set-up) and restores the states it changed.
"""

from __future__ import annotations

import copy
import ctypes

import torch


class Session:
    run_k = 64  # steps per replay in free()

    def __init__(self, fast, cache, device=None):
        dev = torch.device(device) if device is not None else \
            torch.device("cuda", torch.cuda.current_device())
        self.fast, self.cache, self.dev = fast, cache, dev
        self.pf = fast.prefill(dev)
        self.lib = self.pf.lib
        self.ring = torch.zeros(self.run_k + 2, dtype=torch.int32, device=dev)
        base = self.pf.buffers(1)
        self._blocks = [self._block(base, i) for i in range(self.run_k)]
        self._graphs: dict = {}
        self.next = None  # the model's prediction after the last token run
        self.last = None  # the last token run
        self.n = 0        # tokens run

    def _block(self, base, i: int):
        """Step i's parameter block: base's run buffers with the token, prediction and error
        words in the ring. Returns (host block, device block, what they point into)."""
        view = copy.copy(base)
        view.__dict__.pop("_bind_memo", None)
        view.tokens = self.ring[1 + i:2 + i]
        view.preds = self.ring[2 + i:3 + i]
        view.err = self.ring[0:1]
        return self.pf.bind(1, self.cache, view)

    # ------------------------------------------------------------------------------------------
    def _launch(self, k: int) -> None:
        """Steps 0 .. k-1 on the current stream."""
        st = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        nl = self.pf.dims.n_layers
        for p, pd, _ in self._blocks[:k]:
            hp, dp = ctypes.byref(p), ctypes.c_void_p(pd.data_ptr())
            for e, what in ((self.lib.lxm_pf_embed(hp, dp, st), "embed"),
                            (self.lib.lxm_pf_layers(hp, dp, 0, nl, st), "layers"),
                            (self.lib.lxm_pf_head(hp, dp, st), "head")):
                if e:
                    raise RuntimeError(f"session {what} failed: hipError {e}")

    def _graph(self, k: int):
        g = self._graphs.get(k)
        if g is None:
            saved = [(ly.conv_states[0].clone(), ly.recurrent_states[0].clone())
                     for ly in self.cache.layers]
            self._launch(1)
            torch.cuda.synchronize(self.dev)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._launch(k)
            for ly, (c, r) in zip(self.cache.layers, saved):
                ly.conv_states[0].copy_(c)
                ly.recurrent_states[0].copy_(r)
            torch.cuda.synchronize(self.dev)
            self._graphs[k] = g
        return g

    @torch.no_grad()
    def _run(self, t: int, k: int) -> list:
        """k steps from token t (one replay): returns the k tokens run, and sets next/last/n."""
        if not 0 <= t < self.pf.vocab:
            raise ValueError(f"token {t} out of range [0, {self.pf.vocab})")
        g = self._graph(k)
        self.ring[:2].copy_(torch.tensor([0, t], dtype=torch.int32))
        g.replay()
        words = self.ring[:k + 2].tolist()
        if words[0]:
            raise RuntimeError(f"session: the kernels set error word {words[0]}")
        fed = words[1:k + 1]
        self.next, self.last = words[k + 1], fed[-1]
        self.n += k
        return fed

    def step(self, t: int) -> int:
        """Run token t alone (one graph replay); returns the model's next prediction
        (lx/lx/session.py:165-174)."""
        self._run(t, 1)
        return self.next

    def free(self, n: int, stop=None, first: int | None = None) -> list:
        """Feed the model its own predictions for n tokens (or until stop(tokens) is true),
        starting from `first` (default: the last prediction); returns the tokens run
        (lx/lx/session.py:207-225). Without a stop, n // run_k replays of the run_k-step graph
        come first; the rest (or, with a stop, every token) go one step at a time."""
        if first is not None:
            self.next = first
        if self.next is None:
            raise ValueError("free: no prediction to start from (step a token, or pass first)")
        out = []
        for _ in range(0 if stop is not None else n // self.run_k):
            out += self._run(self.next, self.run_k)
        for _ in range(n - len(out)):
            out += self._run(self.next, 1)
            if stop is not None and stop(out):
                break
        return out
