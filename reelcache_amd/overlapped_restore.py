"""Layer-overlapped restore: a history's KV layers are restored on a private stream while the
model's forward reads the layers already written.

Mirrors the consumer/producer contract of ``reelcache/overlapped_restore.py:70-316``:

* a :class:`LayerReadiness` per restore, with one or more named producers ("sources", e.g. the
  compressed restore and a RAW install); each producer calls :meth:`LayerReadiness.mark` after
  it has *issued* a layer's writes on its stream (an event is recorded there) and
  :meth:`LayerReadiness.fail` on an error;
* the consumer (the attention of layer ``L``) calls :meth:`LayerReadiness.wait` before reading
  the layer: a host wait until every source issued it, then a device-side wait of the consumer's
  stream on each source's event, so the device never reads a layer before its writes complete
  and the host is blocked only until they are issued;
* a failure reaches every later ``wait`` and :meth:`LayerReadiness.join` with its class kept for
  this package's errors (``StateError`` otherwise), and stops the other producers at their next
  layer; :meth:`LayerReadiness.cancel` and :meth:`LayerReadiness.quiesce` stop and drain.

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

from .errors import ConfigurationError, ReelCacheError, StateError

#: Source names of the compressed restore and of the RAW install (reference constants).
RESTORE, RAW = "restore", "raw"


class LayerReadiness:
    """Per-layer readiness of a destination whose layers are still being written.

    ``marked_at[i]``: ``time.perf_counter()`` when the last source marked layer ``i``;
    ``waited_seconds[i]``: the consumer's host wait for it; ``info``: the producers' report.
    """

    def __init__(self, layers: int, device: Any = None, *, timeout: float = 600.0,
                 sources: Sequence[str] = (RESTORE,)) -> None:
        if type(layers) is not int or layers < 1:
            raise ConfigurationError("layer readiness needs a positive layer count")
        if not timeout > 0:
            raise ConfigurationError("the layer wait timeout must be positive")
        names = tuple(sources)
        if not names or len(set(names)) != len(names) or any(not isinstance(n, str) or not n for n in names):
            raise ConfigurationError("readiness sources must be distinct non-empty names")
        self.layers = layers
        self.sources = names
        self.device = torch.device(device) if device is not None else torch.device("cpu")
        self.timeout = float(timeout)
        on_gpu = self.device.type == "cuda"
        self._lock = threading.Lock()
        self._released = [threading.Event() for _ in range(layers)]
        self._missing = [set(names) for _ in range(layers)]
        self._events = [{n: (torch.cuda.Event() if on_gpu else None) for n in names} for _ in range(layers)]
        self._error: BaseException | None = None
        self._stop = threading.Event()
        self._cancelled = threading.Event()
        self._threads: dict[str, threading.Thread] = {}
        self._finished: dict[str, float] = {}
        self.streams: dict[str, Any] = {}
        self.stream = None
        self.created_at = self.called_at = time.perf_counter()
        self.marked_at: list[float | None] = [None] * layers
        self.source_marked_at = {n: [None] * layers for n in names}
        self.waited_seconds = [0.0] * layers
        self.info: dict[str, Any] = {}

    def _name(self, source: str | None) -> str:
        if source is None:
            if len(self.sources) != 1:
                raise ConfigurationError(f"name the source of a readiness with sources {self.sources}")
            return self.sources[0]
        if source not in self.sources:
            raise ConfigurationError(f"unknown readiness source {source!r} (sources {self.sources})")
        return source

    # -- producers ------------------------------------------------------------------------------
    def mark(self, layer: int, stream: Any = None, source: str | None = None) -> None:
        """``source`` has issued layer ``layer``'s writes on ``stream`` (None: the current
        stream); the layer is released once every source has marked it.  Ignored after a
        failure or a repeated mark."""
        name = self._name(source)
        with self._lock:
            if self._error is not None or name not in self._missing[layer]:
                return
            event = self._events[layer][name]
            if event is not None:
                event.record(stream if stream is not None else torch.cuda.current_stream(self.device))
            now = time.perf_counter()
            self._missing[layer].discard(name)
            self.source_marked_at[name][layer] = now
            released = not self._missing[layer]
            if released:
                self.marked_at[layer] = now
        if released:
            self._released[layer].set()

    def fail(self, error: BaseException) -> None:
        """A source failed: every later wait and :meth:`join` raise it; the producers stop."""
        with self._lock:
            if self._error is None:
                self._error = error
        self._stop.set()
        for flag in self._released:
            flag.set()

    def attach(self, thread: threading.Thread, source: str | None = None) -> None:
        self._threads[self._name(source)] = thread

    def is_marked(self, layer: int, source: str | None = None) -> bool:
        """Whether layer ``layer`` is released (``source`` None) or ``source`` has marked it."""
        if source is None:
            return self.marked_at[layer] is not None
        return self._name(source) not in self._missing[layer]

    @property
    def stopping(self) -> bool:
        """Cancelled or failed: producers stop at their next layer."""
        return self._stop.is_set()

    # -- consumer -------------------------------------------------------------------------------
    def wait(self, layer: int, stream: Any = None) -> None:
        """Before reading layer ``layer``: wait on the host until every source issued it, then
        order ``stream`` (None: the current stream) after every source's writes.  Raises the
        failure (typed) or ``StateError`` after ``timeout`` seconds."""
        begin = time.perf_counter()
        if not self._released[layer].wait(self.timeout):
            raise StateError(f"layer {layer} of the overlapped restore was not issued within {self.timeout} s")
        self.waited_seconds[layer] += time.perf_counter() - begin
        if self._error is not None:
            raise self._failure() from self._error
        consumer = None
        for event in self._events[layer].values():
            if event is None:
                continue
            if consumer is None:
                consumer = stream if stream is not None else torch.cuda.current_stream(self.device)
            consumer.wait_event(event)

    def ready(self, layer: int) -> bool:
        return self._released[layer].is_set() and self._error is None

    def layer(self, layer: int) -> "LayerWait":
        """Per-layer view (``wait()`` / ``ready()``) for the attention cache of ``layer``."""
        if type(layer) is not int or not 0 <= layer < self.layers:
            raise ConfigurationError(f"layer must be an integer in [0, {self.layers})")
        return LayerWait(self, layer)

    @property
    def error(self) -> BaseException | None:
        return self._error

    @property
    def cancelled(self) -> bool:
        return self._cancelled.is_set()

    @property
    def done(self) -> bool:
        """Every source's producer thread has finished (successfully, failed or cancelled)."""
        threads = list(self._threads.values())
        return len(threads) == len(self.sources) and not any(t.is_alive() for t in threads)

    def cancel(self) -> None:
        """Stop every producer at its next layer; no later layer is released."""
        self._cancelled.set()
        self._stop.set()

    def _join_threads(self, timeout: float | None, message: str) -> None:
        deadline = time.perf_counter() + (self.timeout if timeout is None else timeout)
        for thread in list(self._threads.values()):
            thread.join(max(0.0, deadline - time.perf_counter()))
            if thread.is_alive():
                raise StateError(message)

    def quiesce(self, timeout: float | None = None) -> bool:
        """Leave no restore work in flight: cancel unless finished, join the producers, and
        synchronize their streams.  Never raises the restore's failure; True when it completed."""
        if not self.done:
            self.cancel()
        self._join_threads(timeout, "the overlapped restore did not quiesce")
        streams = [s for s in self.streams.values() if s is not None]
        if self.stream is not None and all(s is not self.stream for s in streams):
            streams.append(self.stream)
        for stream in streams:
            stream.synchronize()
        return self._error is None

    def join(self, timeout: float | None = None) -> dict[str, Any]:
        """Wait for every producer; raise a failure (typed); return the report."""
        self._join_threads(timeout, "the overlapped restore did not finish")
        if self._error is not None:
            raise self._failure() from self._error
        return dict(self.info)

    def _failure(self) -> ReelCacheError:
        error = self._error
        message = f"overlapped restore failed: {type(error).__name__}: {error}"
        if isinstance(error, ReelCacheError):
            with contextlib.suppress(Exception):
                return type(error)(message)
        return StateError(message)

    def _finish(self, source: str) -> None:
        with self._lock:
            self._finished[source] = time.perf_counter()
            last = len(self._finished) == len(self.sources)
        if last and self._error is None:
            marks = [t for t in self.marked_at if t is not None]
            self.info.update({
                "overlapped": True, "sources": list(self.sources),
                "first_layer_ready_seconds_from_call": (min(marks) - self.called_at) if marks else None,
                "last_layer_ready_seconds_from_call": (max(marks) - self.called_at) if marks else None,
                "restore_complete_seconds_from_call": max(self._finished.values()) - self.called_at})

    def timeline(self) -> dict[str, Any]:
        """Marks (seconds after creation) and the consumer's host waits, per layer."""
        record = {"marked_at": [None if t is None else t - self.created_at for t in self.marked_at],
                  "waited_seconds": list(self.waited_seconds)}
        if len(self.sources) > 1:
            record["sources"] = {n: [None if t is None else t - self.created_at for t in marks]
                                 for n, marks in self.source_marked_at.items()}
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


def _producer(readiness: LayerReadiness, source: str, layers: Sequence[int], issue: Callable[[int, Any], Any],
              stream: Any, wait_event: Any) -> None:
    """Issue layers in order on ``stream`` (None on the CPU), marking each; stop when asked."""
    grad = torch.is_grad_enabled()
    inference = torch.is_inference_mode_enabled()

    def run() -> None:
        try:
            with torch.inference_mode(inference), torch.set_grad_enabled(grad), \
                    (torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()):
                if wait_event is not None and stream is not None:
                    stream.wait_event(wait_event)
                keep = []
                for layer in layers:
                    if readiness.stopping:
                        raise StateError("overlapped restore cancelled" if readiness.cancelled
                                         else "another source of the overlapped restore failed")
                    keep.append(issue(layer, stream))
                    readiness.mark(layer, stream, source)
                if stream is not None:
                    stream.synchronize()  # every layer's work completed before the producer reports done
                for item in keep:
                    release = getattr(item, "release", None)
                    if release is not None:
                        release()
        except BaseException as error:  # noqa: BLE001 - delivered to the consumer, typed
            readiness.fail(error)
        finally:
            readiness._finish(source)

    thread = threading.Thread(target=run, name=f"reelcache-overlapped-{source}", daemon=True)
    readiness.attach(thread, source)
    thread.start()


def _stream_for(readiness: LayerReadiness, source: str):
    if readiness.device.type != "cuda":
        return None
    stream = torch.cuda.Stream(readiness.device)
    readiness.streams[source] = stream
    if readiness.stream is None or source == RESTORE:
        readiness.stream = stream
    return stream


def start_overlapped_restore(layer_jobs: Sequence[Sequence[Any]], *, device: Any = None, precision: str = "auto",
                             config: dict | None = None, timeout: float = 600.0, wait_event: Any = None,
                             readiness: LayerReadiness | None = None) -> LayerReadiness:
    """Restore ``layer_jobs[L]`` (the ``ReconstructionJob`` list of layer ``L``) for every layer in
    increasing order on a private stream, marking each layer once its launches are issued;
    returns the readiness at once.  ``wait_event``: orders the first launch after the caller's
    preparation.  ``readiness``: an existing readiness with a ``"restore"`` source (a mixed
    history with a RAW install as the other source)."""
    from . import restore_kernels as rk

    layers = len(layer_jobs)
    if readiness is None:
        readiness = LayerReadiness(layers, device, timeout=timeout, sources=(RESTORE,))
    elif readiness.layers != layers or RESTORE not in readiness.sources:
        raise ConfigurationError("the readiness must cover the restored layers and have a 'restore' source")
    stream = _stream_for(readiness, RESTORE)

    def issue(layer: int, on: Any):
        jobs = list(layer_jobs[layer])
        if not jobs:
            return None
        return rk.reconstruct(jobs, stream=on, precision=precision, config=config)

    _producer(readiness, RESTORE, range(layers), issue, stream, wait_event)
    return readiness


def start_overlapped_install(raw: Callable[[int], Any], *, layers: int, device: Any = None, timeout: float = 600.0,
                             wait_event: Any = None, readiness: LayerReadiness | None = None,
                             source: str = RAW) -> LayerReadiness:
    """Run ``raw(layer)`` for every layer in order on a private stream (a RAW install: dense
    K / V copied and stored by the caller's function), marking each layer."""
    if readiness is None:
        readiness = LayerReadiness(layers, device, timeout=timeout, sources=(source,))
    elif readiness.layers != layers or source not in readiness.sources:
        raise ConfigurationError(f"the readiness must cover {layers} layers and have a {source!r} source")
    stream = _stream_for(readiness, source)
    _producer(readiness, source, range(layers), lambda layer, on: raw(layer), stream, wait_event)
    return readiness
