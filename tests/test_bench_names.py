"""Static check of bench.py and __graft_entry__.py: every name a function
reads as a global is bound at module level or is a builtin (a function-local
import that goes missing shows up here, not as a NameError on the GPU host)."""
import builtins
import pathlib
import symtable

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _unbound_globals(path: pathlib.Path):
    top = symtable.symtable(path.read_text(), str(path), "exec")
    bound = {s.get_name() for s in top.get_symbols() if s.is_assigned() or s.is_imported()}
    bound |= set(dir(builtins)) | {"__file__", "__name__", "__doc__"}
    missing = []

    def walk(table, where):
        for s in table.get_symbols():
            if s.is_global() and s.is_referenced() and s.get_name() not in bound:
                missing.append(f"{where}: {s.get_name()}")
        for child in table.get_children():
            walk(child, f"{where}.{child.get_name()}")

    for child in top.get_children():
        walk(child, child.get_name())
    return missing


@pytest.mark.parametrize("name", ["bench.py", "__graft_entry__.py"])
def test_function_globals_are_bound(name):
    assert _unbound_globals(ROOT / name) == []


def test_the_check_finds_a_missing_import(tmp_path):
    p = tmp_path / "m.py"
    p.write_text("import os\n\ndef f():\n    return os.sep + native.X\n\ndef g():\n    from x import native\n"
                 "    return native\n")
    assert _unbound_globals(p) == ["f: native"]
