"""Layer-overlapped restore: a history's KV layers are restored on a private stream while the
model's forward reads the layers already written.

Consumer/producer contract of ``reelcache/overlapped_restore.py:70-316`` (class and method
names, sources, typed failures, report keys):

* a :class:`LayerReadiness` per restore, with one or more named producers ("sources", e.g. the
  compressed restore and a RAW install); each producer calls :meth:`LayerReadiness.mark` after
  it has *issued* a layer's writes on its stream and :meth:`LayerReadiness.fail` on an error;
* the consumer (the attention of layer ``L``) calls :meth:`LayerReadiness.wait` before reading
  the layer: a host wait until every source issued it, then a device-side wait of the consumer's
  stream on each source's event, so the device never reads a layer before its writes complete
  and the host is blocked only until they are issued;
* a failure reaches every later ``wait`` and :meth:`LayerReadiness.join` with its class kept for
  this package's errors (``StateError`` otherwise), and stops the other producers at their next
  layer; :meth:`LayerReadiness.cancel` and :meth:`LayerReadiness.quiesce` stop and drain.

Design: the readiness is one state machine under one condition variable.  Each layer holds a
bit mask of the sources that have not marked it yet and one HIP event per source (recorded at
the mark on the producer's stream); the run state is ``running`` -> ``stopping`` (cancelled)
or ``failed``.  Host waits are ``Condition.wait_for`` on "this layer's mask is empty, or the
run failed"; producers are :class:`_Producer` threads that check the state before each layer.

:func:`start_overlapped_restore` is the compressed-restore producer for this package's hot
path: it takes the per-layer ``ReconstructionJob`` lists (e.g. from
``archive_restore.history_jobs``) and runs one :func:`restore_kernels.reconstruct` call per layer,
in layer order, on a private stream.  The reference's version drives a ``LineageRestorer`` over
the lineage store, which is outside this package; the readiness object and its semantics are the
same.  :func:`start_overlapped_install` runs any per-layer callable (a RAW install) the same way.
"""

from __future__ import annotations

import contextlib
import threading
import time
from typing import Any, Callable, Sequence

import torch

from ._checks import need
from .errors import ConfigurationError, ReelCacheError, StateError

#: Source names of the compressed restore and of the RAW install (reference constants).
RESTORE, RAW = "restore", "raw"

_RUNNING, _STOPPING, _FAILED = "running", "stopping", "failed"


def _since(origin, stamps):
    return [None if stamp is None else stamp - origin for stamp in stamps]


class LayerReadiness:
    """Per-layer readiness of a destination whose layers are still being written.

    ``marked_at[i]``: ``time.perf_counter()`` when the last source marked layer ``i``;
    ``waited_seconds[i]``: the consumer's host wait for it; ``info``: the producers' report.
    """

    def __init__(self, layers: int, device: Any = None, *, timeout: float = 600.0,
                 sources: Sequence[str] = (RESTORE,)) -> None:
        names = tuple(sources)
        need(type(layers) is int and layers >= 1, "layer readiness needs a positive layer count")
        need(timeout > 0, "the layer wait timeout must be positive")
        need(names and len(set(names)) == len(names) and all(isinstance(n, str) and n for n in names),
             "readiness sources must be distinct non-empty names")
        self.layers, self.sources, self.timeout = layers, names, float(timeout)
        self.device = torch.device("cpu") if device is None else torch.device(device)
        self._bit = {name: 1 << index for index, name in enumerate(names)}
        self._cond = threading.Condition()
        self._state = _RUNNING
        self._cancelled = False
        self._error: BaseException | None = None
        self._unmarked = [(1 << len(names)) - 1] * layers
        gpu = self.device.type == "cuda"
        # Timing events: the consumer orders after them, and they date each layer's release.
        self._events = [[torch.cuda.Event(enable_timing=True) if gpu else None for _ in names] for _ in range(layers)]
        self._threads: dict[str, threading.Thread] = {}
        self._finished: dict[str, float] = {}
        self.streams: dict[str, Any] = {}
        self.stream = None
        self.created_at = self.called_at = time.perf_counter()
        self.marked_at: list[float | None] = [None] * layers
        self.source_marked_at = {name: [None] * layers for name in names}
        self.waited_seconds = [0.0] * layers
        self.info: dict[str, Any] = {}

    def _name(self, source: str | None) -> str:
        if source is None:
            need(len(self.sources) == 1, f"name the source of a readiness with sources {self.sources}")
            return self.sources[0]
        need(source in self._bit, f"unknown readiness source {source!r} (sources {self.sources})")
        return source

    # -- producers ------------------------------------------------------------------------------
    def mark(self, layer: int, stream: Any = None, source: str | None = None) -> None:
        """``source`` has issued layer ``layer``'s writes on ``stream`` (None: the current
        stream); the layer is released once every source has marked it.  Ignored after a
        failure or a repeated mark."""
        name = self._name(source)
        bit = self._bit[name]
        with self._cond:
            if self._state == _FAILED or not self._unmarked[layer] & bit:
                return
            event = self._events[layer][self.sources.index(name)]
            if event is not None:
                event.record(torch.cuda.current_stream(self.device) if stream is None else stream)
            stamp = time.perf_counter()
            self.source_marked_at[name][layer] = stamp
            self._unmarked[layer] &= ~bit
            if not self._unmarked[layer]:
                self.marked_at[layer] = stamp
                self._cond.notify_all()

    def fail(self, error: BaseException) -> None:
        """A source failed: every later wait and :meth:`join` raise it; the producers stop."""
        with self._cond:
            if self._error is None:
                self._error = error
            self._state = _FAILED
            self._cond.notify_all()

    def attach(self, thread: threading.Thread, source: str | None = None) -> None:
        self._threads[self._name(source)] = thread

    def is_marked(self, layer: int, source: str | None = None) -> bool:
        """Whether layer ``layer`` is released (``source`` None) or ``source`` has marked it."""
        if source is None:
            return self.marked_at[layer] is not None
        return not self._unmarked[layer] & self._bit[self._name(source)]

    @property
    def stopping(self) -> bool:
        """Cancelled or failed: producers stop at their next layer."""
        return self._state != _RUNNING

    # -- consumer -------------------------------------------------------------------------------
    def wait(self, layer: int, stream: Any = None) -> None:
        """Before reading layer ``layer``: wait on the host until every source issued it, then
        order ``stream`` (None: the current stream) after every source's writes.  Raises the
        failure (typed) or ``StateError`` after ``timeout`` seconds."""
        begin = time.perf_counter()
        with self._cond:
            released = self._cond.wait_for(lambda: self._state == _FAILED or not self._unmarked[layer], self.timeout)
        if not released:
            raise StateError(f"layer {layer} of the overlapped restore was not issued within {self.timeout} s")
        self.waited_seconds[layer] += time.perf_counter() - begin
        if self._error is not None:
            raise self._failure() from self._error
        events = [event for event in self._events[layer] if event is not None]
        if events:
            consumer = torch.cuda.current_stream(self.device) if stream is None else stream
            for event in events:
                consumer.wait_event(event)

    def ready(self, layer: int) -> bool:
        return not self._unmarked[layer] and self._error is None

    def layer(self, layer: int) -> "LayerWait":
        """Per-layer view (``wait()`` / ``ready()``) for the attention cache of ``layer``."""
        need(type(layer) is int and 0 <= layer < self.layers, f"layer must be an integer in [0, {self.layers})")
        return LayerWait(self, layer)

    @property
    def error(self) -> BaseException | None:
        return self._error

    @property
    def cancelled(self) -> bool:
        return self._cancelled

    @property
    def done(self) -> bool:
        """Every source's producer thread has finished (successfully, failed or cancelled)."""
        return set(self._threads) == set(self.sources) and all(not t.is_alive() for t in self._threads.values())

    def cancel(self) -> None:
        """Stop every producer at its next layer; no later layer is released."""
        with self._cond:
            self._cancelled = True
            if self._state == _RUNNING:
                self._state = _STOPPING

    def _drain(self, timeout: float | None, message: str) -> None:
        """Join every producer thread within one deadline; ``StateError(message)`` past it."""
        deadline = time.perf_counter() + (self.timeout if timeout is None else timeout)
        for thread in list(self._threads.values()):
            thread.join(max(0.0, deadline - time.perf_counter()))
            need(not thread.is_alive(), message, StateError)

    def quiesce(self, timeout: float | None = None) -> bool:
        """Leave no restore work in flight: cancel unless finished, join the producers, and
        synchronize their streams.  Never raises the restore's failure; True when it completed."""
        if not self.done:
            self.cancel()
        self._drain(timeout, "the overlapped restore did not quiesce")
        streams = {id(s): s for s in (*self.streams.values(), self.stream) if s is not None}
        for stream in streams.values():
            stream.synchronize()
        return self._error is None

    def join(self, timeout: float | None = None) -> dict[str, Any]:
        """Wait for every producer; raise a failure (typed); return the report."""
        self._drain(timeout, "the overlapped restore did not finish")
        if self._error is not None:
            raise self._failure() from self._error
        return dict(self.info)

    def _failure(self) -> ReelCacheError:
        """The failure re-raised to the consumer: the package error's own class, else StateError."""
        error = self._error
        message = f"overlapped restore failed: {type(error).__name__}: {error}"
        kind = type(error) if isinstance(error, ReelCacheError) else StateError
        try:
            return kind(message)
        except Exception:  # noqa: BLE001 - an error class with another constructor
            return StateError(message)

    def _finish(self, source: str) -> None:
        with self._cond:
            self._finished[source] = time.perf_counter()
            complete = len(self._finished) == len(self.sources) and self._error is None
        if not complete:
            return
        marks = [stamp - self.called_at for stamp in self.marked_at if stamp is not None]
        self.info.update(overlapped=True, sources=list(self.sources),
                         first_layer_ready_seconds_from_call=min(marks) if marks else None,
                         last_layer_ready_seconds_from_call=max(marks) if marks else None,
                         restore_complete_seconds_from_call=max(self._finished.values()) - self.called_at)

    def device_ready_ms(self, since: Any) -> list[float | None]:
        """Per layer, device milliseconds from the timing event ``since`` (recorded by the caller
        before the restore started) to the end of the layer's writes on every source's stream: the
        latest source event.  None for a layer not released on a GPU stream.  Call after the
        restore finished (e.g. after :meth:`quiesce`)."""
        ready: list[float | None] = []
        for layer in range(self.layers):
            marked = [event for event in self._events[layer] if event is not None]
            if self.marked_at[layer] is None or len(marked) != len(self.sources):
                ready.append(None)
                continue
            ready.append(max(since.elapsed_time(event) for event in marked))
        return ready

    def timeline(self) -> dict[str, Any]:
        """Marks (seconds after creation) and the consumer's host waits, per layer."""
        record = {"marked_at": _since(self.created_at, self.marked_at), "waited_seconds": list(self.waited_seconds)}
        if len(self.sources) > 1:
            record["sources"] = {name: _since(self.created_at, stamps)
                                 for name, stamps in self.source_marked_at.items()}
        return record


class LayerWait:
    """The view of one layer that its attention cache holds."""

    def __init__(self, readiness: LayerReadiness, index: int) -> None:
        self.readiness = readiness
        self.index = index

    def wait(self, stream: Any = None) -> None:
        self.readiness.wait(self.index, stream)

    def ready(self) -> bool:
        return self.readiness.ready(self.index)


class _Producer(threading.Thread):
    """Issues one source's layers in order on its stream (None on the CPU), marking each; stops
    when the readiness is stopping; reports any error to the readiness.  The caller's grad and
    inference modes carry over to the thread."""

    def __init__(self, readiness, source, layers, issue, stream, wait_event):
        super().__init__(name=f"reelcache-overlapped-{source}", daemon=True)
        self.readiness, self.source, self.layers, self.issue = readiness, source, layers, issue
        self.stream, self.wait_event = stream, wait_event
        self.modes = (torch.is_inference_mode_enabled(), torch.is_grad_enabled())

    def _issue_all(self):
        readiness, stream = self.readiness, self.stream
        if stream is not None and self.wait_event is not None:
            stream.wait_event(self.wait_event)
        results = []
        for layer in self.layers:
            if readiness.stopping:
                raise StateError("overlapped restore cancelled" if readiness.cancelled
                                 else "another source of the overlapped restore failed")
            results.append(self.issue(layer, stream))
            readiness.mark(layer, stream, self.source)
        if stream is not None:
            stream.synchronize()  # every layer's work completed before the producer reports done
        for result in results:
            getattr(result, "release", lambda: None)()

    def run(self):
        inference, grad = self.modes
        try:
            with torch.inference_mode(inference), torch.set_grad_enabled(grad), \
                    (torch.cuda.stream(self.stream) if self.stream is not None else contextlib.nullcontext()):
                self._issue_all()
        except BaseException as error:  # noqa: BLE001 - delivered to the consumer, typed
            self.readiness.fail(error)
        finally:
            self.readiness._finish(self.source)


def _producer(readiness: LayerReadiness, source: str, layers: Sequence[int], issue: Callable[[int, Any], Any],
              stream: Any, wait_event: Any) -> None:
    thread = _Producer(readiness, source, layers, issue, stream, wait_event)
    readiness.attach(thread, source)
    thread.start()


def _stream_for(readiness: LayerReadiness, source: str):
    """A private stream (default priority) for ``source`` on a GPU readiness; None on the CPU."""
    if readiness.device.type != "cuda":
        return None
    stream = readiness.streams[source] = torch.cuda.Stream(readiness.device)
    if readiness.stream is None or source == RESTORE:
        readiness.stream = stream
    return stream


def _checked(readiness, layers, source, device, timeout):
    if readiness is None:
        return LayerReadiness(layers, device, timeout=timeout, sources=(source,))
    if readiness.layers != layers or source not in readiness.sources:
        raise ConfigurationError(f"the readiness must cover {layers} layers and have a {source!r} source")
    return readiness


def start_overlapped_restore(layer_jobs: Sequence[Sequence[Any]], *, device: Any = None, precision: str = "auto",
                             config: dict | None = None, timeout: float = 600.0, wait_event: Any = None,
                             readiness: LayerReadiness | None = None) -> LayerReadiness:
    """Restore ``layer_jobs[L]`` (the ``ReconstructionJob`` list of layer ``L``) for every layer in
    increasing order on a private stream, marking each layer once its launches are issued;
    returns the readiness at once.  ``wait_event``: orders the first launch after the caller's
    preparation.  ``readiness``: an existing readiness with a ``"restore"`` source (a mixed
    history with a RAW install as the other source)."""
    from . import restore_kernels as rk

    readiness = _checked(readiness, len(layer_jobs), RESTORE, device, timeout)

    def issue(layer: int, on: Any):
        jobs = list(layer_jobs[layer])
        return rk.reconstruct(jobs, stream=on, precision=precision, config=config) if jobs else None

    _producer(readiness, RESTORE, range(len(layer_jobs)), issue, _stream_for(readiness, RESTORE), wait_event)
    return readiness


def start_overlapped_install(raw: Callable[[int], Any], *, layers: int, device: Any = None, timeout: float = 600.0,
                             wait_event: Any = None, readiness: LayerReadiness | None = None,
                             source: str = RAW) -> LayerReadiness:
    """Run ``raw(layer)`` for every layer in order on a private stream (a RAW install: dense
    K / V copied and stored by the caller's function), marking each layer."""
    readiness = _checked(readiness, layers, source, device, timeout)
    _producer(readiness, source, range(layers), lambda layer, on: raw(layer), _stream_for(readiness, source),
              wait_event)
    return readiness
