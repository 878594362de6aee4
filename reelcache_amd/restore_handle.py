"""Completion handles of restore calls and the parking of inputs that outlive their handle.

:class:`RestoreHandle` keeps the contract of reelcache/restore_kernels.py:876-954 (``event``,
``stream``, ``released``, ``stats``, ``query``, ``synchronize``, ``wait``, ``release``): a call's
inputs, tables and temporaries stay referenced until the GPU work that reads them has completed.

The mechanism here is a finalizer rather than ``__del__``: each handle owns a small
:class:`_Hold` (the completion event and the referenced objects) and registers
``weakref.finalize(handle, _PARKING.park, hold)``.  :meth:`RestoreHandle.release` empties the
hold and detaches the finalizer; a handle collected unreleased hands its hold to the module's
:class:`_Parking`, which drops it once its event reports completion (checked at every
:func:`reconstruct` call and by :func:`pending_deferred`).  A call that fails after enqueuing
work parks its inputs the same way.
"""

from __future__ import annotations

import threading
import weakref

import torch


class _Hold:
    """What a pending call keeps referenced, and the event after which it may be dropped."""

    __slots__ = ("event", "refs")

    def __init__(self, event, refs):
        self.event, self.refs = event, refs

    def done(self):
        return self.refs is None or self.event is None or self.event.query()


class _Parking:
    """Holds of collected or failed calls whose GPU work may still be running."""

    def __init__(self):
        self._lock = threading.Lock()
        self._holds: list = []

    def park(self, hold):
        if not _capturing() and hold.done():
            return
        with self._lock:
            self._holds.append(hold)

    def sweep(self):
        """Drop every hold whose event has completed; returns how many remain.  Nothing is
        queried while this thread's stream captures a HIP graph (a capture forbids it)."""
        with self._lock:
            if self._holds and not _capturing():
                self._holds = [hold for hold in self._holds if not hold.done()]
            return len(self._holds)

    def __len__(self):
        with self._lock:
            return len(self._holds)


_PARKING = _Parking()


def _capturing():
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def _sweep_deferred():
    """Drop the inputs of collected-but-unreleased handles whose GPU work has finished."""
    _PARKING.sweep()


def pending_deferred():
    """Number of collected handles whose inputs are still held until their event completes."""
    return len(_PARKING)


def park_failed(stream, refs):
    """Keep ``refs`` until the work already enqueued on ``stream`` has completed (a call that
    raised after launching)."""
    event = torch.cuda.Event()
    event.record(stream)
    _PARKING.park(_Hold(event, refs))


class RestoreHandle:
    """Completion of one :func:`reconstruct` call.

    ``event`` is recorded on the execution stream after the last write (None for
    host execution).  The handle keeps all inputs, tables and temporaries alive
    until :meth:`release`; a handle collected before release parks them until its
    event completes.
    """

    __slots__ = ("__weakref__", "_finalizer", "_hold", "_released", "_stream", "stats")

    def __init__(self, *, event, stream, keepalive, stats):
        self._hold = _Hold(event, keepalive)
        self._stream = stream
        self._released = False
        self.stats = stats
        self._finalizer = weakref.finalize(self, _PARKING.park, self._hold) if keepalive is not None else None

    @property
    def event(self):
        return self._hold.event

    @property
    def stream(self):
        return self._stream

    @property
    def released(self):
        return self._released

    def query(self):
        """True once the call's GPU work has completed (always for host execution)."""
        event = self._hold.event
        return event is None or event.query()

    def synchronize(self):
        """Block the host until the call's GPU work has completed."""
        if self._hold.event is not None:
            self._hold.event.synchronize()

    def wait(self, stream=None):
        """Make ``stream`` (default: current) wait for completion without blocking the host."""
        event = self._hold.event
        if event is not None:
            (torch.cuda.current_stream(self._stream.device) if stream is None else stream).wait_event(event)

    def release(self):
        """Wait for completion, then drop every retained input and temporary."""
        if self._released:
            return
        self.synchronize()
        if self._finalizer is not None:
            self._finalizer.detach()
        self._hold.refs = None
        self._released = True
        _PARKING.sweep()
