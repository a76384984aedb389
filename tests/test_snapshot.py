"""Session snapshots (linuxformer_amd.snapshot) in the reference's formats, lx/lx/session.py:228-292.

The .safetensors layout is pinned two ways: a file built key by key as the reference's save_safe
lays it out (session.py:258-275: conv.{L} / recurrent.{L} tensors, ref.{field} uint8 tensors for
byte fields, JSON metadata under "lx.session" with "ref" and "bytes") loads here with every
state bit and field intact; and a file written here holds exactly those keys and metadata, so the
reference's load_safe (session.py:278-292) reads it.
"""

import json
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from linuxformer_amd import fast, snapshot


def _cache(seed=0, n_layers=3, n_conv=24, nv=4):
    rng = np.random.default_rng(seed)
    conv = rng.standard_normal((n_layers, n_conv, 4)).astype(np.float32)
    rec = rng.standard_normal((n_layers, nv, 256, 128)).astype(np.float32)
    rec[0, 1, 7, 9] = -0.0  # a negative zero survives as such
    return fast.StateCache(conv, rec, "bf16", "cpu")


def _bits(t):
    return t.contiguous().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


def _same_state(a, b):
    assert len(a) == len(b)
    for (ca, ra), (cb, rb) in zip(a, b):
        assert ca.dtype == cb.dtype and ra.dtype == rb.dtype
        assert tuple(ca.shape) == tuple(cb.shape) and tuple(ra.shape) == tuple(rb.shape)
        assert torch.equal(_bits(ca), _bits(cb)) and torch.equal(_bits(ra), _bits(rb))


def _machine():
    return SimpleNamespace(mem=bytearray(b"\x00\x01\xfe\xff" * 3), rom=b"boot", empty=b"", pc=17,
                           regs=[1, 2, 3], csr={"mtvec": 256, "mstatus": 8}, name="hart0")


@pytest.mark.parametrize("suffix", [".safetensors", ".pt"])
def test_round_trip(tmp_path, suffix):
    cache = _cache()
    path = tmp_path / f"s{suffix}"
    snapshot.save(path, cache, next=301, last=300, n=12345, waiting=[7, 8], ref=_machine())
    d = snapshot.load(path)
    _same_state(d["state"], snapshot.state_of(cache))
    assert (d["next"], d["last"], d["n"], d["waiting"]) == (301, 300, 12345, [7, 8])
    m, want = d["ref"], _machine()
    for k, v in vars(want).items():
        got = getattr(m, k)
        assert got == v and type(got) is type(v), k
    other = _cache(seed=1)
    snapshot.restore(d, other)
    _same_state(snapshot.state_of(other), snapshot.state_of(cache))


def test_reference_layout_loads(tmp_path):
    """A file laid out as session.py:258-275 writes it."""
    from safetensors.torch import save_file

    cache = _cache(seed=2, n_layers=2)
    st = snapshot.state_of(cache)
    t = {}
    for L, (cs, rs) in enumerate(st):
        t[f"conv.{L}"], t[f"recurrent.{L}"] = cs, rs
    t["ref.mem"] = torch.tensor([5, 6, 7], dtype=torch.uint8)
    t["ref.tape"] = torch.zeros(0, dtype=torch.uint8)
    meta = {"next": 9, "last": 8, "n": 2, "waiting": 0, "ref": {"pc": 3, "csr": {"a": 1}},
            "bytes": {"mem": "bytearray", "tape": "bytes"}}
    path = tmp_path / "ref.safetensors"
    save_file(t, str(path), metadata={"lx.session": json.dumps(meta)})
    d = snapshot.load(path)
    _same_state(d["state"], st)
    assert (d["next"], d["last"], d["n"], d["waiting"]) == (9, 8, 2, 0)
    assert d["ref"].mem == bytearray(b"\x05\x06\x07") and type(d["ref"].mem) is bytearray
    assert d["ref"].tape == b"" and type(d["ref"].tape) is bytes
    assert d["ref"].pc == 3 and d["ref"].csr == {"a": 1}


def test_written_layout_is_the_reference_one(tmp_path):
    """What load_safe (session.py:278-292) reads: the tensor keys and the metadata's fields."""
    from safetensors import safe_open

    cache = _cache(seed=3, n_layers=2)
    path = tmp_path / "ours.safetensors"
    snapshot.save(path, cache, next=1, last=0, n=5, waiting=None, ref=_machine())
    with safe_open(str(path), "pt") as f:
        keys = set(f.keys())
        meta = json.loads(f.metadata()["lx.session"])
        assert f.get_tensor("conv.0").dtype == torch.bfloat16
        assert f.get_tensor("recurrent.1").dtype == torch.float32
        assert tuple(f.get_tensor("recurrent.1").shape) == (1, 4, 256, 128)
        assert f.get_tensor("ref.mem").dtype == torch.uint8
    assert keys == {"conv.0", "conv.1", "recurrent.0", "recurrent.1", "ref.mem", "ref.rom",
                    "ref.empty"}
    assert set(meta) == {"next", "last", "n", "waiting", "ref", "bytes"}
    assert meta["bytes"] == {"mem": "bytearray", "rom": "bytes", "empty": "bytes"}
    assert meta["ref"] == {"pc": 17, "regs": [1, 2, 3], "csr": {"mtvec": 256, "mstatus": 8},
                           "name": "hart0"}


class _Pickled:
    pass


def test_pickled_pt_is_refused(tmp_path):
    """A .pt holding a pickled object (what the reference's torch.save of a Machine writes)
    is not loaded: weights_only loading refuses it."""
    path = tmp_path / "obj.pt"
    torch.save({"state": [], "ref": _Pickled()}, path)
    with pytest.raises(ValueError, match="running code"):
        snapshot.load(path)


def test_restore_checks_shapes(tmp_path):
    cache = _cache(n_layers=2)
    path = tmp_path / "s.safetensors"
    snapshot.save(path, cache)
    with pytest.raises(ValueError, match="layers"):
        snapshot.restore(snapshot.load(path), _cache(n_layers=3))
    with pytest.raises(ValueError, match="recurrent"):
        snapshot.restore(snapshot.load(path), _cache(n_layers=2, nv=8))


def test_not_a_snapshot(tmp_path):
    from safetensors.torch import save_file

    path = tmp_path / "w.safetensors"
    save_file({"x": torch.zeros(2)}, str(path))
    with pytest.raises(ValueError, match="lx.session"):
        snapshot.load(path)
