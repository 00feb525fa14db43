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


def _bench_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("copies", [1, 2, 5, 12, 13])
@pytest.mark.parametrize("warmup", [0, 1, 5, 12, 40])
@pytest.mark.parametrize("steps", [1, 5, 11, 12, 20, 25, 400])
def test_every_timed_plan_is_warmed(steps, warmup, copies):
    """No plan is launched for the first time inside a timed region: the
    layer-set steps and the one-plan-per-step loop both launch only plans
    that the warm-up launched."""
    b = _bench_module()
    warmed = set(b.warmup_schedule(steps, warmup, copies))
    timed = b.plan_schedule(steps, copies) + b.one_plan_schedule(steps, copies)
    assert set(timed) <= warmed
    # the timed schedules run exactly `steps` steps over the rotation
    n = sum(copies if k == ("round",) else k[1] for k in b.plan_schedule(steps, copies))
    assert n == steps
    assert len(b.one_plan_schedule(steps, copies)) == steps
    # the warm-up holds at least the requested warm-up steps
    w = sum(copies if k == ("round",) else k[1] for k in b.plan_schedule(max(warmup, 1), copies))
    assert w == max(warmup, 1)


def test_settle_replays_until_its_time_has_passed():
    """bench.settle (the untimed replays before a leg samples a plan) calls
    its replay at least once and keeps calling it until the time budget has
    passed, then stops."""
    import time
    b = _bench_module()
    calls = []
    t0 = time.perf_counter()
    b.settle(lambda: calls.append(time.perf_counter()), seconds=0.02)
    assert len(calls) > 1 and calls[-2] - calls[0] < 0.02 <= time.perf_counter() - t0
    calls.clear()
    b.settle(lambda: calls.append(1), seconds=0.0)
    assert calls == [1]
