"""Owner-thread GPU fitting on MI355X: batched Gram (MFMA) -> eigh -> stored FP16 basis -> projection.

Public surface of ``reelcache/gpu_fitting.py``: GPU_FIT_METHODS, EIGH_SOLVERS, BoundedEigh
(:100-235), select_eigh_solver (:238-273), gram_bases (:276-295) and GPUFitter (:298-522) with
``prefit`` / ``fit`` / ``plan_chunk`` / ``adopt_current_thread`` / ``clear_prefit``.

MI355X design:
* the Gram of every source is one launch of the hand-written HIP kernel (``rch_fit_gram``:
  exact 16-bit products on MFMA, fp32 accumulation, only lower-triangle tiles computed,
  written exactly symmetric, so the reference's ``(G + G^T) / 2`` is the identity);
* the batched symmetric eigensolve is rocSOLVER through ``torch.linalg.eigh`` on the stacked
  batch (ascending values, columns transposed to rows), sub-batched by :class:`BoundedEigh`
  exactly as the reference sub-batches cuSOLVER; cuSOLVER's ctypes binding does not exist on
  ROCm and is refused loudly;
* projection, residual and source energies are the FP64-MFMA kernels of
  :mod:`reelcache_amd.factorization`.

There is no CPU path: host tensors and a missing HIP library raise UnsupportedError.
"""

from __future__ import annotations

import contextlib
import os
import threading
import time

import torch

from . import fit_kernels
from .errors import CapacityError, ConfigurationError, StateError, UnsupportedError
from .factorization import (
    Factors, _canonical_signs, all_finite, fast_condition_bound, project_onto_basis, validate_matrix, validate_rank,
)

GPU_FIT_METHODS = ("gesvd", "gesvdj", "gesvda", "torch_lowrank", "cupy", "randomized", "gram", "gram_batched")
EIGH_SOLVERS = ("auto", "torch_batched", "cusolver_ctypes", "torch_loop")
#: Methods this build runs (the SVD backends of the reference are CUDA library calls, not part of this path).
SUPPORTED_FIT_METHODS = ("gram", "gram_batched")
#: Torch versions whose CUDA build sends a stacked eigh to cusolverDnXsyevBatched (kept for callers
#: that test it; a ROCm build never does).
TORCH_BATCHED_XSYEV_MIN_VERSION = (2, 13)
#: Share of the device memory one eigensolver call may use (input copy, vectors, workspace).
EIGH_MEMORY_FRACTION = 0.125
#: Batches above this many Gram elements are split when the solver's workspace cannot be queried.
EIGH_UNQUERIED_ELEMENT_LIMIT = 1 << 29
#: From this matrix size on, every matrix is solved in its own call by default.
PER_MATRIX_EIGH_MIN_N = 4096


def _torch_version() -> tuple[int, int]:
    head = torch.__version__.split("+")[0].split(".")
    try:
        return int(head[0]), int(head[1])
    except (IndexError, ValueError) as error:
        raise UnsupportedError(f"cannot parse the running Torch version {torch.__version__!r}") from error


def torch_batched_eigh_is_xsyevbatched() -> bool:
    """True when this Torch build sends a batched CUDA eigh to cusolverDnXsyevBatched (never on ROCm)."""
    return torch.version.cuda is not None and _torch_version() >= TORCH_BATCHED_XSYEV_MIN_VERSION


def torch_batched_eigh_is_rocsolver() -> bool:
    """True on a ROCm Torch build: a stacked ``torch.linalg.eigh`` runs rocSOLVER on the device."""
    return torch.version.hip is not None


def _torch_rows_eigh(grams):
    values, columns = torch.linalg.eigh(grams)
    return values, columns.transpose(1, 2)


def _torch_loop_eigh(grams):
    pairs = [torch.linalg.eigh(gram) for gram in grams]
    return torch.stack([values for values, _ in pairs]), torch.stack([columns.T for _, columns in pairs])


def default_eigh_sub_batch(n: int) -> int | None:
    """One matrix per call from PER_MATRIX_EIGH_MIN_N on, else None (the whole batch in one call)."""
    return 1 if n >= PER_MATRIX_EIGH_MIN_N else None


def xsyevbatched_workspace_bytes(batch: int, n: int, device) -> int | None:
    """cuSOLVER's workspace query; there is no cuSOLVER on ROCm."""
    raise UnsupportedError("the cusolverDnXsyevBatched buffer-size query needs CUDA's cuSOLVER (absent on ROCm)")


class BoundedEigh:
    """A batched eigensolver called on sub-batches that the memory bound admits.

    The solver never changes.  ``sub_batch_size(n)`` (default :func:`default_eigh_sub_batch`)
    fixes the sub-batch of ``n x n`` problems: every call then runs ``ceil(b / s)`` calls of
    exactly ``s`` matrices, the last padded with identity matrices whose results are dropped,
    so a matrix's eigenpairs never depend on what it is solved with.  A fixed sub-batch whose
    copies and workspace exceed the bound still runs (recorded ``over_budget``).  Without a
    fixed size a batch runs in one call, or halves until it fits the bound (``memory_bound``)
    or the solver's size limit (``solver_rejects_batch_size``).  ``calls`` records each call's
    ``batch``, ``n``, ``sub_batch``, ``solver_calls``, ``reason`` (plus ``padded`` /
    ``over_budget``); ``last`` the latest.
    """

    def __init__(self, label: str, solver, *, memory_fraction: float = EIGH_MEMORY_FRACTION, workspace=None,
                 total_memory: int | None = None, sub_batch_size=None):
        if not 0 < memory_fraction <= 1:
            raise ConfigurationError("eigh memory fraction must be in (0, 1]")
        if total_memory is not None and (type(total_memory) is not int or total_memory <= 0):
            raise ConfigurationError("total_memory must be a positive byte count")
        if sub_batch_size is not None and not callable(sub_batch_size):
            raise ConfigurationError("sub_batch_size must map n to a fixed sub-batch size or None")
        self.label, self.solver, self.memory_fraction = label, solver, memory_fraction
        self._workspace = workspace  # (batch, n, device) -> bytes, or None when the solver rejects the size
        self.total_memory = total_memory
        self.sub_batch_size = default_eigh_sub_batch if sub_batch_size is None else sub_batch_size
        self.calls: list[dict] = []
        self.last: dict | None = None

    def derive(self, *, memory_fraction: float | None = None, total_memory: int | None = None) -> "BoundedEigh":
        """The same solver and sub-batch policy under another memory bound."""
        return BoundedEigh(self.label, self.solver,
                           memory_fraction=self.memory_fraction if memory_fraction is None else memory_fraction,
                           workspace=self._workspace, total_memory=total_memory, sub_batch_size=self.sub_batch_size)

    def _workspace_bytes(self, batch: int, n: int, device) -> int | None:
        if self._workspace is not None:
            return self._workspace(batch, n, device)
        return None if batch * n * n > EIGH_UNQUERIED_ELEMENT_LIMIT else 4 * batch * n * n

    def _budget(self, device) -> float | None:
        if self.total_memory is None and device.type != "cuda":
            return None
        total = self.total_memory or torch.cuda.get_device_properties(device).total_memory
        return self.memory_fraction * total

    @staticmethod
    def _need(size: int, n: int, workspace: int) -> int:
        return 8 * size * n * n + 4 * size * n + workspace  # input copy + vectors, values, workspace

    def sub_batch(self, batch: int, n: int, device) -> tuple[int, str]:
        return self._sub_batch(batch, n, device)[:2]

    def _sub_batch(self, batch: int, n: int, device) -> tuple[int, str, bool]:
        device = torch.device(device)
        fixed = self.sub_batch_size(n)
        budget = self._budget(device)
        if fixed is not None:
            if type(fixed) is not int or fixed < 1:
                raise ConfigurationError(f"sub_batch_size({n}) must be a positive integer or None")
            reason = "per_matrix" if fixed == 1 else "fixed_sub_batch"
            if budget is None:
                return fixed, reason, False
            workspace = self._workspace_bytes(fixed, n, device)
            if workspace is None:
                raise UnsupportedError(f"the batched eigensolver rejects the fixed sub-batch of {fixed} {n}x{n} matrices")
            return fixed, reason, self._need(fixed, n, workspace) > budget
        if budget is None:
            return batch, "whole_batch", False
        size, reason = batch, "whole_batch"
        while True:
            workspace = self._workspace_bytes(size, n, device)
            if workspace is None:
                reason = "solver_rejects_batch_size"
            elif self._need(size, n, workspace) > budget:
                reason = "memory_bound"
            else:
                return size, reason, False
            if size == 1:
                if workspace is None:
                    raise UnsupportedError(f"the batched eigensolver rejects even one {n}x{n} matrix")
                return 1, reason, True
            size = (size + 1) // 2

    def __call__(self, grams: torch.Tensor):
        batch, n = int(grams.shape[0]), int(grams.shape[1])
        size, reason, over_budget = self._sub_batch(batch, n, grams.device)
        fixed = reason in ("per_matrix", "fixed_sub_batch")
        padded = 0
        if size == batch:
            values, vectors = self.solver(grams)
        else:
            values = vectors = None
            for start in range(0, batch, size):
                part = grams[start:start + size]
                count = int(part.shape[0])
                if fixed and count < size:
                    padded = size - count
                    identity = torch.eye(n, dtype=grams.dtype, device=grams.device).expand(padded, n, n)
                    part = torch.cat((part, identity))
                part_values, part_vectors = self.solver(part.contiguous())
                if values is None:
                    values = part_values.new_empty((batch, *part_values.shape[1:]))
                    vectors = part_vectors.new_empty((batch, *part_vectors.shape[1:]))
                values[start:start + count] = part_values[:count]
                vectors[start:start + count] = part_vectors[:count]
        record = {"batch": batch, "n": n, "sub_batch": size if fixed else min(size, batch),
                  "solver_calls": -(-batch // size), "reason": reason}
        if padded:
            record["padded"] = padded
        if over_budget:
            record["over_budget"] = True
        self.last = record
        self.calls.append(record)
        return values, vectors


def select_eigh_solver(solver="auto", *, sub_batch_size=None):
    """``(label, eigh)`` for stacked FP32 Grams; never a silent downgrade.

    ``auto`` / ``torch_batched``: one stacked ``torch.linalg.eigh`` per (sub-)batch, which on
    ROCm runs rocSOLVER on the device (:class:`BoundedEigh`).  ``cusolver_ctypes`` raises
    UnsupportedError (no cuSOLVER on ROCm).  ``torch_loop`` is the explicit per-matrix
    diagnostic.  ``eigh`` maps ``[b, n, n]`` to ascending values and row eigenvectors.
    """
    if solver not in EIGH_SOLVERS:
        raise ConfigurationError(f"eigh solver must be one of {EIGH_SOLVERS}")
    if solver in ("auto", "torch_batched"):
        if torch_batched_eigh_is_rocsolver():
            label = "torch_linalg_eigh_batched_rocsolver"
            return label, BoundedEigh(label, _torch_rows_eigh, sub_batch_size=sub_batch_size)
        if torch_batched_eigh_is_xsyevbatched():
            label = "torch_linalg_eigh_batched_xsyevbatched"
            return label, BoundedEigh(label, _torch_rows_eigh, sub_batch_size=sub_batch_size)
        raise UnsupportedError(f"Torch {torch.__version__} has no batched device eigensolver for this build")
    if solver == "cusolver_ctypes":
        raise UnsupportedError("the ctypes cusolverDnXsyevBatched binding needs CUDA's cuSOLVER, which ROCm does not "
                               "provide; use eigh_solver='auto' (rocSOLVER)")
    return "torch_eigh_loop_explicit", _torch_loop_eigh


def gram_bases(sources, ranks, *, eigh=None):
    """Top-``rank`` right singular bases of each ``[rows, n]`` source via one batched Gram eigh.

    Returns FP32 ``[rank, n]`` bases in descending energy, canonical signs not yet applied.
    The Grams are one launch of the MFMA Gram kernel; ``eigh`` maps ``[b, n, n]`` to
    ``(values, row_vectors)`` (default: ``torch.linalg.eigh``, columns transposed to rows).
    """
    if not sources or len(sources) != len(ranks):
        raise ConfigurationError("batched Gram fitting needs one rank per source")
    if len({int(x.shape[1]) for x in sources}) != 1:
        raise ConfigurationError("one Gram batch must share the channel count")
    grams = fit_kernels.gram(list(sources))
    if eigh is None:
        _, columns = torch.linalg.eigh(grams)
        vectors = columns.transpose(1, 2)
    else:
        _, vectors = eigh(grams)
    return [vectors[index, -rank:].flip(0) for index, rank in enumerate(ranks)]


def _stored_bases(bases) -> list[torch.Tensor]:
    """Canonical signs, FP16 rounding, and one finiteness read for the whole group."""
    stored = [_canonical_signs(basis).to(dtype=torch.float16).contiguous() for basis in bases]
    finite = torch.stack([torch.isfinite(basis).all() for basis in stored]).cpu()
    if not bool(finite.all()):
        raise ConfigurationError("fitted basis is not finite in stored FP16")
    return stored


class GPUFitter:
    """Owner-thread GPU fitting facade (``method="gram_batched"``: batched prefit + per-matrix fit)."""

    def __init__(self, *, gpu_id, gpu_uuid, method="randomized", max_workspace_bytes=2 * 1024**3, seed=0,
                 power_iterations=2, batch_size=60, side_stream=False, shared=False, eigh_solver="auto"):
        if type(gpu_id) is not int or gpu_id < 0 or not isinstance(gpu_uuid, str) or not gpu_uuid.startswith("GPU-"):
            raise ConfigurationError("GPU fitting requires an explicit visible device index and UUID")
        if method not in GPU_FIT_METHODS:
            raise ConfigurationError("unsupported GPU fitting backend")
        if type(max_workspace_bytes) is not int or max_workspace_bytes <= 0:
            raise ConfigurationError("GPU fitting workspace budget must be positive")
        if type(seed) is not int or seed < 0 or type(power_iterations) is not int or not 0 <= power_iterations <= 8:
            raise ConfigurationError("invalid GPU fitting seed or iteration count")
        if type(batch_size) is not int or not 1 <= batch_size <= 256:
            raise ConfigurationError("GPU fitting batch size must be an integer in [1, 256]")
        if type(side_stream) is not bool:
            raise ConfigurationError("side_stream must be boolean")
        if type(shared) is not bool:
            raise ConfigurationError("shared must be boolean")
        if eigh_solver not in EIGH_SOLVERS:
            raise ConfigurationError(f"eigh_solver must be one of {EIGH_SOLVERS}")
        self.gpu_id, self.gpu_uuid, self.method = gpu_id, gpu_uuid, method
        self.max_workspace_bytes, self.seed, self.power_iterations = max_workspace_bytes, seed, power_iterations
        self.batch_size = batch_size
        self.eigh_solver = eigh_solver
        # ``shared`` lets worker threads call ``fit``: calls serialize on a lock and run on the
        # fitter's private stream (default priority), never on the caller's forward stream.
        self.shared = shared
        self.side_stream = side_stream or shared
        self._stream = None
        self._lock = threading.Lock()
        self.owner = (os.getpid(), threading.get_ident())
        self._prefit: dict = {}
        self.prefit_stats = {"batches": 0, "matrices": 0, "hits": 0, "misses": 0, "solver": None}

    def adopt_current_thread(self):
        """Move ownership to the calling thread (not while fitting)."""
        self.clear_prefit()
        self.owner = (os.getpid(), threading.get_ident())

    def _check_owner(self):
        if self.shared:
            if self.owner[0] != os.getpid():
                raise StateError("a shared GPU fitter cannot cross processes")
            return
        if self.owner != (os.getpid(), threading.get_ident()):
            raise StateError("GPU fitting must run on its configured owner thread, not the CPU encoder pool")

    def _device(self):
        if self.gpu_id >= torch.cuda.device_count():
            raise UnsupportedError("GPU fitting device is unavailable")
        device = torch.device("cuda", self.gpu_id)
        actual = str(torch.cuda.get_device_properties(device).uuid)
        if actual.startswith("GPU-"):
            actual = actual[len("GPU-"):]
        if actual != self.gpu_uuid[len("GPU-"):]:
            raise ConfigurationError("GPU fitting device differs from the granted UUID")
        return device

    def _check_method(self):
        if self.method not in SUPPORTED_FIT_METHODS:
            raise UnsupportedError(f"GPU fitting method {self.method!r} is a CUDA library SVD backend; this MI355X "
                                   f"build fits with {SUPPORTED_FIT_METHODS}")

    def _scope(self, device):
        if self.side_stream and self._stream is None:
            self._stream = torch.cuda.Stream(device)
        return torch.cuda.stream(self._stream) if self.side_stream else contextlib.nullcontext()

    @staticmethod
    def _identity(tensor, context, rank):
        return (tensor.untyped_storage().data_ptr(), tensor.storage_offset(), tuple(tensor.shape), tuple(tensor.stride()),
                tensor.dtype, str(tensor.device), tensor._version, context, rank)

    @torch.no_grad()
    def prefit(self, items):
        """Batch-solve bases for ``{key: (tensor, context, rank)}`` ahead of per-matrix ``fit``.

        Only ``gram_batched`` batches; other methods return immediately.  A cached basis is
        consumed by the next ``fit`` of the same, unmodified tensor with the same context and
        rank; the tensor is referenced until consumed or :meth:`clear_prefit`.
        """
        self._check_owner()
        self.clear_prefit()
        if self.method != "gram_batched" or not items:
            return
        prepared = []
        for tensor, context, rank in items.values():
            validate_matrix(tensor, context, lossy=True, check_values=False)
            validate_rank(rank, tuple(tensor.shape))
            prepared.append((tensor, context, rank))
        channels = max(int(t.shape[1]) for t, _, _ in prepared)
        rows = max(int(t.shape[0]) for t, _, _ in prepared)
        per_item = 3 * 4 * channels * channels
        if 8 * rows * channels + per_item > self.max_workspace_bytes:
            raise CapacityError("GPU batched fitting exceeds its declared logical workspace budget")
        batch = min(self.batch_size, max(1, (self.max_workspace_bytes - 8 * rows * channels) // per_item))
        device = self._device()
        label, solver = select_eigh_solver(self.eigh_solver)
        self.prefit_stats["solver"] = label
        with torch.cuda.device(device):
            for start in range(0, len(prepared), batch):
                group = prepared[start:start + batch]
                began, ended = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                began.record()
                sources = [validate_matrix(tensor.to(device), context, check_values=False) for tensor, context, _ in group]
                if not all_finite(sources):
                    raise ConfigurationError("lossy input must be finite and representable in FP32")
                bases = _stored_bases(gram_bases(sources, [rank for _, _, rank in group], eigh=solver))
                ended.record()
                ended.synchronize()
                share = began.elapsed_time(ended) / 1e3 / len(group)
                del sources
                for (tensor, context, rank), basis in zip(group, bases):
                    self._prefit[self._identity(tensor, context, rank)] = (tensor, basis, share)
                self.prefit_stats["batches"] += 1
                self.prefit_stats["matrices"] += len(group)

    def clear_prefit(self):
        self._prefit.clear()

    @torch.no_grad()
    def fit(self, tensor, context, rank, *, reuse_basis=None, reuse_threshold=None):
        self._check_owner()
        if self.shared:
            with self._lock:
                return self._fit(tensor, context, rank, reuse_basis=reuse_basis, reuse_threshold=reuse_threshold)
        return self._fit(tensor, context, rank, reuse_basis=reuse_basis, reuse_threshold=reuse_threshold)

    def _fit(self, tensor, context, rank, *, reuse_basis=None, reuse_threshold=None):
        validate_matrix(tensor, context, lossy=True, check_values=False)
        validate_rank(rank, tuple(tensor.shape))
        rows, channels = tensor.shape
        estimated = 32 * (rows * channels + channels * channels + rows * rank)
        if estimated > self.max_workspace_bytes:
            raise CapacityError("GPU fitting exceeds its declared logical workspace budget")
        device = self._device()
        if reuse_basis is not None or reuse_threshold is not None:
            raise UnsupportedError("explicit GPU solver comparisons currently require fresh bases")
        self._check_method()
        started = time.perf_counter()
        events = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        with torch.cuda.device(device), self._scope(device):
            events[0].record()
            source = tensor.to(device)
            events[1].record()
            factors = self._fit_gram_batched(source, tensor, context, rank)
            events[2].record()
            basis = factors.basis.cpu()
            coefficients = factors.coefficients.cpu()
            events[3].record()
            events[3].synchronize()
        metrics = {
            **factors.metrics, "gpu_fitting_backend": self.method, "gpu_fitting_uuid": self.gpu_uuid,
            "gpu_fitting_workspace_estimate": estimated,
            "gpu_fitting_h2d_ms": events[0].elapsed_time(events[1]),
            "gpu_fitting_compute_ms": events[1].elapsed_time(events[2]),
            "gpu_fitting_d2h_ms": events[2].elapsed_time(events[3]),
            "gpu_fitting_wall_seconds": time.perf_counter() - started,
            "reuse_attempts": 0, "reuse_accepted": False, "reuse_rejections": 0,
            "reuse_reason": "gpu_fresh_basis", "reuse_seconds": 0.0,
            "total_factorization_seconds": time.perf_counter() - started,
            "canonical_basis_rank": rank, "view_rank": rank,
        }
        return Factors(basis=basis, coefficients=coefficients, rank=rank, metrics=metrics)

    def _fit_gram_batched(self, source, tensor, context, rank):
        """The prefit basis when available; otherwise a single-matrix Gram eigh."""
        started = time.perf_counter()
        cached = self._prefit.pop(self._identity(tensor, context, rank), None) if self.method == "gram_batched" else None
        if cached is not None:
            validate_matrix(source, context)
            self.prefit_stats["hits"] += 1
            basis, decomposition_seconds = cached[1], cached[2]
            algorithm = "batched_fp32_gram_eigh"
        else:
            if self.method == "gram_batched":
                self.prefit_stats["misses"] += 1
            decomposition_started = time.perf_counter()
            (basis,) = gram_bases([validate_matrix(source, context)], [rank])
            (basis,) = _stored_bases([basis])
            decomposition_seconds = time.perf_counter() - decomposition_started
            algorithm = "fp32_gram_eigh" if self.method == "gram_batched" else "custom_fp32_gram_eigh"
        projection = project_onto_basis(source, basis, rank=rank, _condition_bound=fast_condition_bound(basis))
        return Factors(basis=basis, coefficients=projection.coefficients, rank=rank, metrics={
            "factorization_method": algorithm, "factorization_seed": self.seed,
            "sketch_rank": None, "power_iterations": 0, "decomposition_count": 1,
            "svd_count": 0, "eigh_count": 1, "qr_count": 0,
            "decomposition_seconds": decomposition_seconds,
            "projection_count": 1, "projection_seconds": projection.seconds,
            "projection_relative_residual": projection.relative_residual,
            "basis_condition_bound": projection.condition_bound,
            "basis_condition_method": "fp32_neumann_upper_bound",
            "zero_input": projection.zero_input,
            "fit_seconds": time.perf_counter() - started,
            "prefit_batched": cached is not None,
        })

    @torch.no_grad()
    def plan_chunk(self, config, view, sources, contexts, bindings, parent_rows, *, chunk_id, source_ids,
                   orthogonalizer="householder", max_working_bytes=None):
        """Energy-target chunk plan on this fitter's device and owner thread (see
        :class:`reelcache_amd.rank_method.GramPlanner`)."""
        from .rank_method import GramPlanner
        self._check_owner()
        device = self._device()
        label, solver = select_eigh_solver(self.eigh_solver)
        planner = GramPlanner(config, view, device=device, eigh=solver, eigh_label=label,
                              orthogonalizer=orthogonalizer, max_working_bytes=max_working_bytes)
        scope = self._lock if self.shared else contextlib.nullcontext()
        with scope, torch.cuda.device(device), self._scope(device):
            plan = planner.plan(sources, contexts, bindings, parent_rows, chunk_id=chunk_id, source_ids=source_ids)
        self.prefit_stats["solver"] = label
        return plan


__all__ = ["BoundedEigh", "EIGH_SOLVERS", "GPUFitter", "GPU_FIT_METHODS", "default_eigh_sub_batch", "gram_bases",
           "select_eigh_solver", "torch_batched_eigh_is_rocsolver", "torch_batched_eigh_is_xsyevbatched"]
