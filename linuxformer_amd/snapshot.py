"""Session snapshots: every chip layer's conv window and recurrent state, plus the session's
scalars and the proposer's fields, in the reference's formats (lx/lx/session.py:228-292).

    snapshot.save(path, cache, next=t, last=u, n=k, waiting=w, ref=machine)
    d = snapshot.load(path)        # {"state": [(conv, recurrent), ...], "next", "last", "n",
                                   #  "waiting", "ref"}
    snapshot.restore(d, cache)     # the states into a cache, in place

``cache`` is any cache whose ``layers[L].conv_states[0]`` and ``layers[L].recurrent_states[0]``
are tensors (this package's ``fast.StateCache``, transformers' cache): conv (1, C, 4) in the
model dtype, recurrent (1, nv, 256, 128) float32, stored as they are.

.safetensors, the pickle-free form (the reference's save_safe / load_safe, session.py:258-292):

    tensor ``conv.{L}``           conv window of layer L, (1, C, 4), the model dtype
    tensor ``recurrent.{L}``      recurrent state of layer L, (1, nv, 256, 128), float32
    tensor ``ref.{name}``         a bytes / bytearray field of the proposer, uint8 (1-D)
    metadata ``"lx.session"``     JSON: {"next", "last", "n", "waiting": the session's scalars,
                                  "ref": the proposer's other fields, "bytes": {name: "bytes" |
                                  "bytearray"} for the ref.{name} tensors}

for L = 0 .. n-1. A file the reference wrote loads here, and one written here loads in the
reference's load_safe.

.pt: the same dict through ``torch.save``, the proposer as a plain dict of its fields (this
package has no ``lx.ref.Machine``), loaded with ``weights_only=True`` (bytes and bytearray
allowed). A .pt the reference wrote
pickles a ``Machine`` object; loading it would run code from the file, so it is refused with a
``ValueError`` (convert it to .safetensors with the reference's own ``save_safe``).
"""

from __future__ import annotations

import json
import re
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import torch

KEY = "lx.session"
SCALARS = ("next", "last", "n", "waiting")


def _fields(ref) -> dict:
    """The proposer's fields: a dict, an object's attributes, or none."""
    if ref is None:
        return {}
    if isinstance(ref, dict):
        return dict(ref)
    return dict(vars(ref))


def state_of(cache) -> list:
    """[(conv, recurrent)] per layer, copied to host memory (Session._state, session.py:228-230)."""
    return [(l.conv_states[0].detach().to("cpu", copy=True),
             l.recurrent_states[0].detach().to("cpu", copy=True)) for l in cache.layers]


def restore(d: dict, cache) -> None:
    """The snapshot's states into cache, in place (Session._set_state, session.py:232-235):
    every layer's shapes and dtypes must match."""
    st = d["state"]
    if len(st) != len(cache.layers):
        raise ValueError(f"snapshot holds {len(st)} layers, the cache {len(cache.layers)}")
    for L, (cs, rs) in enumerate(st):
        c, r = cache.layers[L].conv_states[0], cache.layers[L].recurrent_states[0]
        for name, dst, src in (("conv", c, cs), ("recurrent", r, rs)):
            if tuple(dst.shape) != tuple(src.shape) or dst.dtype != src.dtype:
                raise ValueError(f"layer {L} {name}: snapshot {tuple(src.shape)} {src.dtype}, "
                                 f"cache {tuple(dst.shape)} {dst.dtype}")
            dst.copy_(src)


def save(path, cache=None, *, state=None, next=None, last=None, n=0, waiting=None,
         ref=None) -> None:
    """Write a snapshot (Session.save, session.py:237-246): the states of cache (or state, a
    list of (conv, recurrent) tensors), the scalars, and the proposer's fields. The suffix picks
    the format (.safetensors, else torch.save)."""
    if state is None:
        if cache is None:
            raise ValueError("save needs a cache or a state")
        state = state_of(cache)
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    d = {"state": [(cs.cpu(), rs.cpu()) for cs, rs in state], "next": next, "last": last,
         "n": n, "waiting": waiting, "ref": _fields(ref)}
    if path.suffix == ".safetensors":
        _save_safe(d, path)
    else:
        torch.save(d, path)


def load(path) -> dict:
    """Read a snapshot (Session.load's file part, session.py:248-256): {"state": [(conv,
    recurrent)], "next", "last", "n", "waiting", "ref"}; ref is a namespace of the proposer's
    fields, its byte fields as bytes or bytearray as they were saved."""
    path = Path(path)
    if path.suffix == ".safetensors":
        return _load_safe(path)
    try:
        # (bytes and bytearray rebuild from their own data: allowlisting them runs nothing else)
        with torch.serialization.safe_globals([bytes, bytearray]):
            d = torch.load(path, map_location="cpu", weights_only=True)
    except Exception as e:  # an unpickling error: the file holds objects beyond tensors and data
        raise ValueError(f"{path}: not loadable without running code from the file ({e}); "
                         "a snapshot the reference pickled converts with its save_safe") from e
    if not isinstance(d, dict) or "state" not in d:
        raise ValueError(f"{path}: not a session snapshot")
    d = dict(d)
    d["ref"] = SimpleNamespace(**_fields(d.get("ref")))
    d["state"] = [(cs, rs) for cs, rs in d["state"]]
    return d


_LAYER_KEY = re.compile(r"^(conv|recurrent)\.(\d+)$")


def _byte_tensor(v) -> torch.Tensor:
    """A bytes-like value as a 1-D uint8 tensor (owning its memory; empty for b"")."""
    return torch.from_numpy(np.frombuffer(bytes(v), dtype=np.uint8).copy())


def _save_safe(d: dict, path: Path) -> None:
    """The .safetensors layout (the module docstring's table): states as conv.L / recurrent.L,
    byte-valued proposer fields as ref.NAME uint8 tensors, the rest as JSON metadata."""
    from safetensors.torch import save_file

    tensors = {}
    for L, (cs, rs) in enumerate(d["state"]):
        tensors[f"conv.{L}"] = cs.contiguous()
        tensors[f"recurrent.{L}"] = rs.contiguous()
    fields = d["ref"]
    byte_kind = {k: type(v).__name__ for k, v in fields.items()
                 if isinstance(v, (bytes, bytearray))}
    tensors.update({f"ref.{k}": _byte_tensor(fields[k]) for k in byte_kind})
    meta = {"next": d["next"], "last": d["last"], "n": d["n"], "waiting": d["waiting"],
            "ref": {k: v for k, v in fields.items() if k not in byte_kind},
            "bytes": byte_kind}
    save_file(tensors, str(path), metadata={KEY: json.dumps(meta)})


def _load_safe(path: Path) -> dict:
    """Read the .safetensors layout back; the layers are the conv.L / recurrent.L pairs, which
    must number 0 .. n-1 with both halves present."""
    from safetensors import safe_open

    with safe_open(str(path), "pt") as f:
        md = f.metadata() or {}
        if KEY not in md:
            raise ValueError(f"{path}: no {KEY!r} metadata: not a session snapshot")
        meta = json.loads(md[KEY])
        keys = list(f.keys())
        layers: dict = {}
        for k in keys:
            hit = _LAYER_KEY.match(k)
            if hit:
                layers.setdefault(int(hit.group(2)), {})[hit.group(1)] = f.get_tensor(k)
        kinds = meta.get("bytes", {})
        fields = dict(meta.get("ref", {}))
        for name, kind in kinds.items():
            raw = f.get_tensor(f"ref.{name}").numpy().tobytes()
            fields[name] = bytearray(raw) if kind == "bytearray" else raw
    if sorted(layers) != list(range(len(layers))) or \
            any(set(v) != {"conv", "recurrent"} for v in layers.values()):
        raise ValueError(f"{path}: the conv.L / recurrent.L tensors do not form layers 0..n-1")
    out = {k: meta.get(k) for k in SCALARS}
    out["state"] = [(layers[L]["conv"], layers[L]["recurrent"]) for L in range(len(layers))]
    out["ref"] = SimpleNamespace(**fields)
    return out
