"""NoGradTrack's thread-local switch (gradtrack/no_grad_track.rs:16-235) in the
host library: host logic only, no device call (CPU).  The reference's own
tests (no_grad_track.rs:260-420) fix the behaviour: enabled by default,
guards nest and restore the enclosing state, set_grad_enabled replaces the
innermost state, an unbalanced drop restores the default, and every thread
has its own stack."""
from __future__ import annotations

import threading

import train_station_amd as T


def _reset():
    while not T.is_grad_enabled():
        T.native_gradtrack.ts_no_grad_pop()
    T.native_gradtrack.ts_no_grad_pop()  # unbalanced: back to the default [true]


def test_default_and_nesting():
    _reset()
    assert T.is_grad_enabled()
    with T.NoGradTrack():
        assert not T.is_grad_enabled()
        with T.NoGradTrack():
            assert not T.is_grad_enabled()
        assert not T.is_grad_enabled()        # the outer guard still holds
    assert T.is_grad_enabled()


def test_set_grad_enabled_replaces_the_innermost_state():
    _reset()
    T.set_grad_enabled(False)
    assert not T.is_grad_enabled()
    with T.NoGradTrack():
        T.set_grad_enabled(True)              # inside a guard: only its own level
        assert T.is_grad_enabled()
    assert not T.is_grad_enabled()            # the base level keeps False
    T.set_grad_enabled(True)
    assert T.is_grad_enabled()


def test_unbalanced_pop_restores_the_default():
    _reset()
    T.set_grad_enabled(False)
    T.native_gradtrack.ts_no_grad_pop()       # no_grad_track.rs:117-127: stack becomes [true]
    assert T.is_grad_enabled()


def test_with_no_grad_returns_the_value():
    _reset()
    assert T.with_no_grad(lambda: (T.is_grad_enabled(), 7)) == (False, 7)
    assert T.is_grad_enabled()


def test_the_switch_is_per_thread():
    _reset()
    seen = {}

    def worker():
        seen["start"] = T.is_grad_enabled()
        T.native_gradtrack.ts_no_grad_push()
        seen["inside"] = T.is_grad_enabled()

    with T.NoGradTrack():
        th = threading.Thread(target=worker)
        th.start()
        th.join()
        assert not T.is_grad_enabled()
    assert seen == {"start": True, "inside": False}
    assert T.is_grad_enabled()                # the other thread's push did not leak here
