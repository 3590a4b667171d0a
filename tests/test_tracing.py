"""roctx ranges of the host-side phases (vllm_gr_amd.tracing): the library
binds, ranges nest and pop on exceptions, and VLLM_GR_ROCTX=0 turns them off.
No GPU is needed: roctx records nothing without a profiler attached."""

import pytest

from vllm_gr_amd import tracing


class _Spy:
    """Counts pushes and pops; stands in for libroctx64 in the nesting tests."""

    def __init__(self):
        self.depth = 0
        self.names = []

    def roctxRangePushA(self, name):
        self.depth += 1
        self.names.append(name.decode())
        return self.depth - 1

    def roctxRangePop(self):
        self.depth -= 1
        return self.depth


def test_roctx_library_binds():
    # the image ships roctx with ROCm; the real calls return a nesting level
    if not tracing.available():
        pytest.skip("roctx library not found")
    lib = tracing._roctx()
    assert lib.roctxRangePushA(b"test") >= 0
    assert lib.roctxRangePop() >= 0
    with tracing.roctx_range("outer"):
        with tracing.roctx_range("inner"):
            pass


def test_ranges_nest_and_pop_on_error(monkeypatch):
    spy = _Spy()
    monkeypatch.setattr(tracing, "_roctx", lambda: spy)
    monkeypatch.setenv("VLLM_GR_ROCTX", "1")
    with tracing.roctx_range("a"):
        assert spy.depth == 1
        with tracing.roctx_range("b"):
            assert spy.depth == 2
    assert spy.depth == 0 and spy.names == ["a", "b"]
    with pytest.raises(ValueError):
        with tracing.roctx_range("c"):
            raise ValueError("x")
    assert spy.depth == 0


def test_disabled_by_env(monkeypatch):
    spy = _Spy()
    monkeypatch.setattr(tracing, "_roctx", lambda: spy)
    monkeypatch.setenv("VLLM_GR_ROCTX", "0")
    with tracing.roctx_range("a"):
        pass
    assert spy.names == []
