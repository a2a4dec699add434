import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "omni-rs_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    return oracle_lib.Oracle()


class Knobs:
    """Per-test overrides of the library's tuning knobs (OMNI_W8A8_TILE and
    the like), which it reads from the environment once per process:
    ``set(name, value)`` pins one, ``unset(name)`` makes it read as unset;
    every knob touched returns to the environment's value after the test."""

    def __init__(self):
        self.touched = set()

    def _call(self, name, mode, value):
        from omni_int8 import _lib
        st = _lib.lib().omni_int8_set_tuning(name.encode(), mode, value)
        assert st == 0, _lib.last_error()
        self.touched.add(name)

    def set(self, name, value):
        self._call(name, 2, int(value))

    def unset(self, name):
        self._call(name, 1, 0)

    def restore(self):
        from omni_int8 import _lib
        for name in self.touched:
            _lib.lib().omni_int8_set_tuning(name.encode(), 0, 0)
        self.touched.clear()


@pytest.fixture
def knobs():
    k = Knobs()
    yield k
    k.restore()


def pytest_terminal_summary(terminalreporter):
    """The fp16-output tests' worst errors per file: the bar these tests
    assert (denominator floored at 0.1 x the output RMS) and the
    reference's own measure (floored at 0.1, quant.rs:552)."""
    import tolerance
    if not tolerance.RECORD:
        return
    worst = {}
    for test, truth, err, clamp in tolerance.RECORD:
        key = (test.split("::")[0], "f64 truth" if truth else "other rounded routes")
        w = worst.setdefault(key, [0, 0.0, 0.0, ""])
        w[0] += 1
        w[1] = max(w[1], err)
        if clamp > w[2]:
            w[2], w[3] = clamp, test
    terminalreporter.write_sep("-", "fp16 output errors (max per file)")
    for (f, against), (n, err, clamp, where) in sorted(worst.items()):
        terminalreporter.write_line(f"{f} vs {against}: {n} checks, rms-floored {err:.3e}, "
                                    f"|ref|.max(0.1) {clamp:.3e} at {where}")
