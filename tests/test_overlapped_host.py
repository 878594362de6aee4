"""Layer readiness on the CPU (reference behaviour: reelcache/overlapped_restore.py:70-316):
release order, several sources, typed failures, cancellation, time-outs and the layer view."""

import threading
import time

import pytest

from reelcache_amd import errors
from reelcache_amd.overlapped_restore import (RAW, RESTORE, LayerReadiness, start_overlapped_install)


def test_layers_release_when_every_source_marked():
    readiness = LayerReadiness(3, sources=(RESTORE, RAW))
    readiness.mark(0, source=RESTORE)
    assert not readiness.ready(0) and readiness.is_marked(0, RESTORE) and not readiness.is_marked(0)
    readiness.mark(0, source=RAW)
    assert readiness.ready(0) and readiness.is_marked(0)
    readiness.mark(0, source=RAW)  # repeated marks are ignored
    readiness.wait(0)
    assert not readiness.ready(1)
    with pytest.raises(errors.ConfigurationError):
        readiness.mark(1)  # two sources: the source must be named
    with pytest.raises(errors.ConfigurationError):
        readiness.mark(1, source="other")


def test_install_marks_layers_in_order_and_joins():
    seen = []
    readiness = start_overlapped_install(lambda layer: seen.append(layer), layers=5)
    for layer in range(5):
        readiness.layer(layer).wait()
    info = readiness.join(timeout=10)
    assert seen == [0, 1, 2, 3, 4] and readiness.done
    assert info["overlapped"] and info["sources"] == [RAW]
    marks = readiness.timeline()["marked_at"]
    assert all(m is not None for m in marks) and marks == sorted(marks)


def test_failure_is_delivered_typed_and_stops_the_source():
    issued = []
    consumed = threading.Event()

    def raw(layer):
        if layer == 2:
            consumed.wait(10)  # the consumer has read layers 0 and 1
            raise errors.IntegrityError("bad rows")
        issued.append(layer)

    readiness = start_overlapped_install(raw, layers=6)
    readiness.wait(0)
    readiness.wait(1)
    consumed.set()
    # After the failure every wait raises it, also for layers released before it.
    with pytest.raises(errors.IntegrityError):
        readiness.wait(2)
    with pytest.raises(errors.IntegrityError):
        readiness.join(timeout=10)
    assert issued == [0, 1] and not readiness.ready(3)
    # Anything that is not a package error becomes a StateError.
    bad = start_overlapped_install(lambda layer: 1 / 0, layers=2)
    with pytest.raises(errors.StateError):
        bad.join(timeout=10)


def test_cancel_stops_at_the_next_layer():
    gate = threading.Event()

    def raw(layer):
        if layer == 1:
            gate.wait(10)

    readiness = start_overlapped_install(raw, layers=4)
    readiness.wait(0)
    readiness.cancel()
    gate.set()
    assert readiness.quiesce(timeout=10) is False
    assert readiness.cancelled and readiness.done
    with pytest.raises(errors.StateError):
        readiness.wait(3)


def test_wait_times_out_with_state_error():
    readiness = LayerReadiness(2, timeout=0.05)
    begin = time.perf_counter()
    with pytest.raises(errors.StateError):
        readiness.wait(1)
    assert time.perf_counter() - begin < 5


def test_validation():
    with pytest.raises(errors.ConfigurationError):
        LayerReadiness(0)
    with pytest.raises(errors.ConfigurationError):
        LayerReadiness(2, timeout=0)
    with pytest.raises(errors.ConfigurationError):
        LayerReadiness(2, sources=("a", "a"))
    readiness = LayerReadiness(2)
    with pytest.raises(errors.ConfigurationError):
        readiness.layer(2)
