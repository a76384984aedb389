"""Every name a function of the driver-facing scripts and the package reads is bound somewhere it
can resolve (its own scope, an enclosing one, the module, or builtins): a static check, run on
the CPU, for the class of mistake that otherwise only shows on the GPU box (a NameError at the
end of a long bench run)."""

import builtins
import glob
import os
import symtable

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FILES = ["bench.py", "__graft_entry__.py"] + sorted(
    os.path.relpath(p, ROOT) for p in glob.glob(os.path.join(ROOT, "linuxformer_amd", "*.py")))


def _unbound(path):
    src = open(os.path.join(ROOT, path)).read()
    top = symtable.symtable(src, path, "exec")
    module = {s.get_name() for s in top.get_symbols() if s.is_assigned() or s.is_imported()
              or s.is_namespace()}
    known = module | set(dir(builtins)) | {"__file__", "__name__", "__doc__"}
    bad = []

    def walk(tab):
        for ch in tab.get_children():
            if ch.get_type() == "function":
                for s in ch.get_symbols():
                    if s.is_referenced() and s.is_global() and s.get_name() not in known:
                        bad.append(f"{ch.get_name()}:{s.get_name()}")
            walk(ch)

    walk(top)
    return bad


@pytest.mark.parametrize("path", FILES)
def test_every_global_name_is_bound(path):
    assert _unbound(path) == []
