"""The model-alone driver loop around the decode kernel: the host side of lx/lx/linux.py:230-310
(``Linux.run_alone``) and tools/mega_boot.py:61-84, with the machine's token vocabulary given as
callables so the loop needs nothing of the reference's machine.

    r = alone.run_alone(mg, batches, final=..., done=..., first_launch=4096, max_launch=65536)

``mg`` is a ``mega.Mega`` (its cache and stream continue from launch to launch). Each keystroke
batch (a list of token ids, already in the machine's typing tokens) is forced at the start of a
launch once the stream's last token is ``final`` (a record boundary, where the host may type);
between batches the kernel decodes its own predictions in launches of ``first_launch`` tokens,
doubling up to ``max_launch`` while nothing waits (the reference's 4k -> 64k), then one token at
a time once ``done(stream)`` holds, until a record boundary comes. Every launch's inputs are read
back and checked (``input purity``): step 0 takes the batch's first token or the last
prediction, each forced token its own position, every other step the prediction before it.
"""

from __future__ import annotations

import time
from typing import Callable, Sequence

import torch


class PurityError(AssertionError):
    """A launch's inputs were not the forced tokens and the kernel's own predictions."""


def run_alone(mg, batches: Sequence[Sequence[int]], *, final: Callable[[int], bool],
              done: Callable[[list, int], bool], start: int | None = None,
              first_launch: int = 4096, max_launch: int = 1 << 16, max_tokens: int = 60_000_000,
              progress: Callable | None = None) -> dict:
    """Type each batch at a record boundary and decode the model's own stream after it.

    final(tok): the token ends a record (typing may follow). done(stream, batch): batch
    (0-based) has been answered (the reference: the typed bytes were consumed and, after the
    last batch, the console shows the prompt with the CPU idle), judged on the stream so far.
    start: the token the first launch takes when there is no batch (else the first batch's
    first token). Returns the stream (every step's input), the predictions' last token, the
    timeline (seconds, tokens), each launch's forced tokens and size, where each batch was typed,
    and the purity counts."""
    if first_launch < 1 or max_launch < first_launch:
        raise ValueError("launch sizes: 1 <= first_launch <= max_launch")
    cap = max_launch + max((len(b) for b in batches), default=1)
    inp = torch.zeros(cap, dtype=torch.int32, device=mg.dev)
    stream: list = []
    nxt = start
    sizes, timeline, typed_at, launches = [], [], [], []
    pure = {"inputs_checked": 0, "keystrokes": 0, "launches": 0}
    torch.cuda.synchronize(mg.dev)
    t0 = time.time()
    todo = list(batches) if batches else [[]]
    for bi, batch in enumerate(todo):
        if stream and not final(stream[-1]):
            raise ValueError(f"batch {bi}: the stream's last token {stream[-1]} ends no record")
        forced = list(batch) if batch else [nxt]
        if forced[0] is None:
            raise ValueError("the first launch needs a batch or a start token")
        typed_at.append(len(stream))
        m, keys = first_launch, len(batch)
        while len(stream) < max_tokens:
            n = len(forced) + m - 1
            preds = mg.run(forced, n, inputs=inp)
            got = inp[:n].tolist()
            if got[:len(forced)] != forced:
                raise PurityError(f"launch {pure['launches']}: forced inputs {forced} read back "
                                  f"as {got[:len(forced)]}")
            if got[len(forced):] != preds[len(forced) - 1:n - 1]:
                i = next(i for i in range(len(forced), n) if got[i] != preds[i - 1])
                raise PurityError(f"launch {pure['launches']}: step {i}'s input {got[i]} is not "
                                  f"the prediction before it ({preds[i - 1]})")
            pure["inputs_checked"] += n
            pure["keystrokes"] += keys
            pure["launches"] += 1
            keys = 0
            sizes.append(n)
            launches.append((list(forced), n))
            stream += got
            nxt = preds[-1]
            forced = [nxt]
            timeline.append((round(time.time() - t0, 3), len(stream)))
            if progress:
                progress(time.time() - t0, len(stream))
            answered = done(stream, bi)
            if answered and final(stream[-1]):
                break
            m = 1 if answered else min(2 * m, max_launch)
    torch.cuda.synchronize(mg.dev)
    dt = time.time() - t0
    pure["passed"] = pure["inputs_checked"] == len(stream) and \
        pure["keystrokes"] == sum(len(b) for b in batches)
    return {"stream": stream, "next": nxt, "tokens": len(stream), "seconds": round(dt, 3),
            "tok_per_s": round(len(stream) / dt) if dt > 0 else None, "launch_sizes": sizes,
            "launches": launches, "typed_at": typed_at, "timeline": timeline,
            "input_purity": pure}
