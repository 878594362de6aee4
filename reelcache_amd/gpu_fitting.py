"""Owner-thread GPU fitting on MI355X: batched Gram (MFMA) -> eigh -> stored FP16 basis -> projection.

Public surface of ``reelcache/gpu_fitting.py``: GPU_FIT_METHODS, EIGH_SOLVERS, BoundedEigh
(:100-235), select_eigh_solver (:238-273), gram_bases (:276-295) and GPUFitter (:298-522) with
``prefit`` / ``fit`` / ``plan_chunk`` / ``adopt_current_thread`` / ``clear_prefit``; the record
and metrics keys are that interface.

MI355X design:
* the Gram of every source is one launch of the hand-written HIP kernel (``rch_fit_gram``:
  exact 16-bit products on MFMA, fp32 accumulation, only lower-triangle tiles computed,
  written exactly symmetric, so the reference's ``(G + G^T) / 2`` is the identity);
* the batched symmetric eigensolve is rocSOLVER through ``torch.linalg.eigh`` on the stacked
  batch (ascending values, columns transposed to rows).  :class:`BoundedEigh` schedules it: a
  fixed sub-batch pads the batch's tail with identity matrices once and solves equal chunks; a
  memory- or solver-bounded batch takes the first size of its halving sequence that fits.
  cuSOLVER's ctypes binding does not exist on ROCm and is refused loudly;
* projection, residual and source energies are the FP64-MFMA kernels of
  :mod:`reelcache_amd.factorization`.

There is no CPU path: host tensors and a missing HIP library raise UnsupportedError.
"""

from __future__ import annotations

import contextlib
import os
import threading
import time
from typing import NamedTuple

import torch

from . import fit_kernels
from ._checks import need
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
    """(major, minor) of the running Torch."""
    release = torch.__version__.partition("+")[0]
    try:
        major, minor = release.split(".")[:2]
        return int(major), int(minor)
    except ValueError as error:
        raise UnsupportedError(f"cannot parse the running Torch version {torch.__version__!r}") from error


def torch_batched_eigh_is_xsyevbatched() -> bool:
    """True when this Torch build sends a batched CUDA eigh to cusolverDnXsyevBatched (never on ROCm)."""
    return torch.version.cuda is not None and _torch_version() >= TORCH_BATCHED_XSYEV_MIN_VERSION


def torch_batched_eigh_is_rocsolver() -> bool:
    """True on a ROCm Torch build: a stacked ``torch.linalg.eigh`` runs rocSOLVER on the device."""
    return torch.version.hip is not None


def _torch_rows_eigh(grams):
    """Stacked eigh: ascending values and eigenvectors as rows."""
    values, columns = torch.linalg.eigh(grams)
    return values, columns.mT


def _torch_loop_eigh(grams):
    """One eigh per matrix (the explicit diagnostic solver), stacked like :func:`_torch_rows_eigh`."""
    solved = [_torch_rows_eigh(gram[None]) for gram in grams]
    return torch.cat([values for values, _ in solved]), torch.cat([rows for _, rows in solved])


def default_eigh_sub_batch(n: int) -> int | None:
    """One matrix per call from PER_MATRIX_EIGH_MIN_N on, else None (the whole batch in one call)."""
    return 1 if n >= PER_MATRIX_EIGH_MIN_N else None


def xsyevbatched_workspace_bytes(batch: int, n: int, device) -> int | None:
    """cuSOLVER's workspace query; there is no cuSOLVER on ROCm."""
    raise UnsupportedError("the cusolverDnXsyevBatched buffer-size query needs CUDA's cuSOLVER (absent on ROCm)")


class _Schedule(NamedTuple):
    """How one batch is solved: chunks of ``size`` matrices, why, and whether the size exceeds the
    memory bound (a fixed sub-batch, or one matrix that still does not fit)."""

    size: int
    reason: str
    over_budget: bool = False


def _halvings(batch):
    """batch, ceil(batch / 2), ... down to 1."""
    size = batch
    while True:
        yield size
        if size == 1:
            return
        size = (size + 1) // 2


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
        need(0 < memory_fraction <= 1, "eigh memory fraction must be in (0, 1]")
        need(total_memory is None or (type(total_memory) is int and total_memory > 0),
             "total_memory must be a positive byte count")
        need(sub_batch_size is None or callable(sub_batch_size),
             "sub_batch_size must map n to a fixed sub-batch size or None")
        self.label, self.solver = label, solver
        self.memory_fraction, self.total_memory = memory_fraction, total_memory
        self._workspace = workspace  # (batch, n, device) -> bytes, or None when the solver rejects the size
        self.sub_batch_size = sub_batch_size or default_eigh_sub_batch
        self.calls: list[dict] = []
        self.last: dict | None = None

    def derive(self, *, memory_fraction: float | None = None, total_memory: int | None = None) -> "BoundedEigh":
        """The same solver and sub-batch policy under another memory bound."""
        fraction = self.memory_fraction if memory_fraction is None else memory_fraction
        return BoundedEigh(self.label, self.solver, memory_fraction=fraction, workspace=self._workspace,
                           total_memory=total_memory, sub_batch_size=self.sub_batch_size)

    def _workspace_bytes(self, size: int, n: int, device) -> int | None:
        if self._workspace is not None:
            return self._workspace(size, n, device)
        elements = size * n * n
        return None if elements > EIGH_UNQUERIED_ELEMENT_LIMIT else 4 * elements

    def _budget(self, device) -> float | None:
        """Bytes one solver call may use; None (unbounded) for host solves without a stated total."""
        if self.total_memory is not None:
            return self.memory_fraction * self.total_memory
        if device.type != "cuda":
            return None
        return self.memory_fraction * torch.cuda.get_device_properties(device).total_memory

    @staticmethod
    def _need(size: int, n: int, workspace: int) -> int:
        """Input copy and eigenvectors (2 x 4 bytes per element), values, and the solver workspace."""
        return size * n * (8 * n + 4) + workspace

    def _fits(self, size, n, device, budget):
        """(reason the size fails, or None when it fits; its workspace bytes)."""
        workspace = self._workspace_bytes(size, n, device)
        if workspace is None:
            return "solver_rejects_batch_size", None
        if budget is not None and self._need(size, n, workspace) > budget:
            return "memory_bound", workspace
        return None, workspace

    def sub_batch(self, batch: int, n: int, device) -> tuple[int, str]:
        return tuple(self._schedule(batch, n, device)[:2])

    def _schedule(self, batch: int, n: int, device) -> _Schedule:
        device = torch.device(device)
        budget = self._budget(device)
        fixed = self.sub_batch_size(n)
        if fixed is not None:
            need(type(fixed) is int and fixed >= 1, f"sub_batch_size({n}) must be a positive integer or None")
            reason = "per_matrix" if fixed == 1 else "fixed_sub_batch"
            if budget is None:
                return _Schedule(fixed, reason)
            failure, _ = self._fits(fixed, n, device, budget)
            need(failure != "solver_rejects_batch_size",
                 f"the batched eigensolver rejects the fixed sub-batch of {fixed} {n}x{n} matrices", UnsupportedError)
            return _Schedule(fixed, reason, failure is not None)
        if budget is None:
            return _Schedule(batch, "whole_batch")
        reason = "whole_batch"
        for size in _halvings(batch):
            failure, _ = self._fits(size, n, device, budget)
            if failure is None:
                return _Schedule(size, reason)
            reason = failure
        need(failure != "solver_rejects_batch_size", f"the batched eigensolver rejects even one {n}x{n} matrix",
             UnsupportedError)
        return _Schedule(1, reason, True)

    def __call__(self, grams: torch.Tensor):
        batch, n = int(grams.shape[0]), int(grams.shape[1])
        plan = self._schedule(batch, n, grams.device)
        fixed = plan.reason in ("per_matrix", "fixed_sub_batch")
        padding = (-batch) % plan.size if fixed else 0
        if padding:
            identities = torch.eye(n, dtype=grams.dtype, device=grams.device).expand(padding, n, n)
            grams = torch.cat((grams, identities))
        if plan.size >= grams.shape[0]:
            values, vectors = self.solver(grams)
        else:
            parts = [self.solver(chunk.contiguous()) for chunk in torch.split(grams, plan.size)]
            values, vectors = (torch.cat([part[i] for part in parts]) for i in (0, 1))
        if padding:
            values, vectors = values[:batch], vectors[:batch]
        record = {"batch": batch, "n": n, "sub_batch": plan.size if fixed else min(plan.size, batch),
                  "solver_calls": -(-batch // plan.size), "reason": plan.reason}
        record.update({"padded": padding} if padding else {})
        record.update({"over_budget": True} if plan.over_budget else {})
        self.calls.append(record)
        self.last = record
        return values, vectors


def select_eigh_solver(solver="auto", *, sub_batch_size=None):
    """``(label, eigh)`` for stacked FP32 Grams; never a silent downgrade.

    ``auto`` / ``torch_batched``: one stacked ``torch.linalg.eigh`` per (sub-)batch, which on
    ROCm runs rocSOLVER on the device (:class:`BoundedEigh`).  ``cusolver_ctypes`` raises
    UnsupportedError (no cuSOLVER on ROCm).  ``torch_loop`` is the explicit per-matrix
    diagnostic.  ``eigh`` maps ``[b, n, n]`` to ascending values and row eigenvectors.
    """
    need(solver in EIGH_SOLVERS, f"eigh solver must be one of {EIGH_SOLVERS}")
    if solver == "torch_loop":
        return "torch_eigh_loop_explicit", _torch_loop_eigh
    need(solver != "cusolver_ctypes", "the ctypes cusolverDnXsyevBatched binding needs CUDA's cuSOLVER, which ROCm "
         "does not provide; use eigh_solver='auto' (rocSOLVER)", UnsupportedError)
    for backend, available in (("rocsolver", torch_batched_eigh_is_rocsolver),
                               ("xsyevbatched", torch_batched_eigh_is_xsyevbatched)):
        if available():
            label = f"torch_linalg_eigh_batched_{backend}"
            return label, BoundedEigh(label, _torch_rows_eigh, sub_batch_size=sub_batch_size)
    raise UnsupportedError(f"Torch {torch.__version__} has no batched device eigensolver for this build")


def gram_bases(sources, ranks, *, eigh=None):
    """Top-``rank`` right singular bases of each ``[rows, n]`` source via one batched Gram eigh.

    Returns FP32 ``[rank, n]`` bases in descending energy, canonical signs not yet applied.
    The Grams are one launch of the MFMA Gram kernel; ``eigh`` maps ``[b, n, n]`` to
    ``(values, row_vectors)`` (default: ``torch.linalg.eigh``, columns transposed to rows).
    """
    need(sources and len(sources) == len(ranks), "batched Gram fitting needs one rank per source")
    need(len({int(x.shape[1]) for x in sources}) == 1, "one Gram batch must share the channel count")
    _, rows = (eigh or _torch_rows_eigh)(fit_kernels.gram(list(sources)))
    # Ascending eigenvalues: the top-rank rows are the last ones, reversed into descending energy.
    return [rows[index, -rank:].flip(0) for index, rank in enumerate(ranks)]


def _stored_bases(bases) -> list[torch.Tensor]:
    """Canonical signs, FP16 rounding, and one finiteness read for the whole group."""
    stored = [_canonical_signs(basis).to(dtype=torch.float16).contiguous() for basis in bases]
    finite = torch.stack([torch.isfinite(basis).all() for basis in stored]).cpu()
    need(bool(finite.all()), "fitted basis is not finite in stored FP16")
    return stored


def _fitter_rules(gpu_id, gpu_uuid, method, max_workspace_bytes, seed, power_iterations, batch_size, side_stream,
                  shared, eigh_solver):
    """``(holds, message)`` rules of the :class:`GPUFitter` options, in order."""
    yield (type(gpu_id) is int and gpu_id >= 0 and isinstance(gpu_uuid, str) and gpu_uuid.startswith("GPU-"),
           "GPU fitting requires an explicit visible device index and UUID")
    yield method in GPU_FIT_METHODS, "unsupported GPU fitting backend"
    yield type(max_workspace_bytes) is int and max_workspace_bytes > 0, "GPU fitting workspace budget must be positive"
    yield (type(seed) is int and seed >= 0 and type(power_iterations) is int and 0 <= power_iterations <= 8,
           "invalid GPU fitting seed or iteration count")
    yield type(batch_size) is int and 1 <= batch_size <= 256, "GPU fitting batch size must be an integer in [1, 256]"
    yield type(side_stream) is bool, "side_stream must be boolean"
    yield type(shared) is bool, "shared must be boolean"
    yield eigh_solver in EIGH_SOLVERS, f"eigh_solver must be one of {EIGH_SOLVERS}"


def _tensor_identity(tensor, context, rank):
    """Key of a prefit basis: the same storage view, unmodified (version counter), same context and rank."""
    return (tensor.untyped_storage().data_ptr(), tensor.storage_offset(), tuple(tensor.shape), tuple(tensor.stride()),
            tensor.dtype, str(tensor.device), tensor._version, context, rank)


def _prefit_bytes(rows, channels):
    """(bytes of the largest staged source, bytes per batched matrix: Gram, vectors and workspace)."""
    return 8 * rows * channels, 12 * channels * channels


def _fit_bytes(rows, channels, rank):
    """Logical workspace of one per-matrix fit (source, Gram, coefficients; FP64-sized with copies)."""
    return 32 * (rows * channels + channels * channels + rows * rank)


# Metrics every fresh-basis GPU fit reports about basis reuse (the GPU path never reuses).
_NO_REUSE = {"reuse_attempts": 0, "reuse_accepted": False, "reuse_rejections": 0, "reuse_reason": "gpu_fresh_basis",
             "reuse_seconds": 0.0}


class GPUFitter:
    """Owner-thread GPU fitting facade (``method="gram_batched"``: batched prefit + per-matrix fit).

    ``shared=True`` lets worker threads call :meth:`fit`: calls serialize on a lock and run on
    the fitter's private stream (default priority), never on the caller's forward stream.
    """

    def __init__(self, *, gpu_id, gpu_uuid, method="randomized", max_workspace_bytes=2 * 1024**3, seed=0,
                 power_iterations=2, batch_size=60, side_stream=False, shared=False, eigh_solver="auto"):
        for holds, message in _fitter_rules(gpu_id, gpu_uuid, method, max_workspace_bytes, seed, power_iterations,
                                            batch_size, side_stream, shared, eigh_solver):
            need(holds, message)
        self.gpu_id, self.gpu_uuid, self.method, self.eigh_solver = gpu_id, gpu_uuid, method, eigh_solver
        self.max_workspace_bytes, self.batch_size = max_workspace_bytes, batch_size
        self.seed, self.power_iterations = seed, power_iterations
        self.shared, self.side_stream = shared, side_stream or shared
        self._stream = None
        self._lock = threading.Lock()
        self.owner = (os.getpid(), threading.get_ident())
        self._prefit: dict = {}
        self.prefit_stats = {"batches": 0, "matrices": 0, "hits": 0, "misses": 0, "solver": None}

    # -- ownership and device -------------------------------------------------

    def adopt_current_thread(self):
        """Move ownership to the calling thread (not while fitting)."""
        self.clear_prefit()
        self.owner = (os.getpid(), threading.get_ident())

    def _check_owner(self):
        pid, thread = self.owner
        need(pid == os.getpid(), "a shared GPU fitter cannot cross processes" if self.shared else
             "GPU fitting must run on its configured owner thread, not the CPU encoder pool", StateError)
        need(self.shared or thread == threading.get_ident(),
             "GPU fitting must run on its configured owner thread, not the CPU encoder pool", StateError)

    def _device(self):
        """The granted device, checked against the UUID the fitter was configured with."""
        need(self.gpu_id < torch.cuda.device_count(), "GPU fitting device is unavailable", UnsupportedError)
        device = torch.device("cuda", self.gpu_id)
        actual = str(torch.cuda.get_device_properties(device).uuid).removeprefix("GPU-")
        need(actual == self.gpu_uuid.removeprefix("GPU-"), "GPU fitting device differs from the granted UUID")
        return device

    def _scope(self, device):
        """The fitter's private stream when it has one, else the caller's current stream."""
        if not self.side_stream:
            return contextlib.nullcontext()
        if self._stream is None:
            self._stream = torch.cuda.Stream(device)
        return torch.cuda.stream(self._stream)

    _identity = staticmethod(_tensor_identity)

    # -- batched prefit -------------------------------------------------------

    def _prefit_batch(self, prepared):
        """Matrices per eigh batch under the workspace budget (at least one, at most ``batch_size``)."""
        staged, per_matrix = _prefit_bytes(max(int(t.shape[0]) for t, _, _ in prepared),
                                           max(int(t.shape[1]) for t, _, _ in prepared))
        spare = self.max_workspace_bytes - staged
        if spare < per_matrix:
            raise CapacityError("GPU batched fitting exceeds its declared logical workspace budget")
        return min(self.batch_size, spare // per_matrix)

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
        prepared = list(items.values())
        for tensor, context, rank in prepared:
            validate_matrix(tensor, context, lossy=True, check_values=False)
            validate_rank(rank, tuple(tensor.shape))
        batch = self._prefit_batch(prepared)
        device = self._device()
        label, solver = select_eigh_solver(self.eigh_solver)
        self.prefit_stats["solver"] = label
        with torch.cuda.device(device):
            for first in range(0, len(prepared), batch):
                self._solve_group(prepared[first:first + batch], device, solver)

    def _solve_group(self, group, device, solver):
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        marks[0].record()
        sources = [validate_matrix(tensor.to(device), context, check_values=False) for tensor, context, _ in group]
        need(all_finite(sources), "lossy input must be finite and representable in FP32")
        bases = _stored_bases(gram_bases(sources, [rank for _, _, rank in group], eigh=solver))
        marks[1].record()
        marks[1].synchronize()
        seconds_each = marks[0].elapsed_time(marks[1]) / 1e3 / len(group)
        for (tensor, context, rank), basis in zip(group, bases):
            self._prefit[_tensor_identity(tensor, context, rank)] = (tensor, basis, seconds_each)
        self.prefit_stats["batches"] += 1
        self.prefit_stats["matrices"] += len(group)

    def clear_prefit(self):
        self._prefit.clear()

    # -- per-matrix fit -------------------------------------------------------

    @torch.no_grad()
    def fit(self, tensor, context, rank, *, reuse_basis=None, reuse_threshold=None):
        self._check_owner()
        with self._lock if self.shared else contextlib.nullcontext():
            return self._fit(tensor, context, rank, reuse_basis=reuse_basis, reuse_threshold=reuse_threshold)

    def _fit(self, tensor, context, rank, *, reuse_basis=None, reuse_threshold=None):
        validate_matrix(tensor, context, lossy=True, check_values=False)
        validate_rank(rank, tuple(tensor.shape))
        estimate = _fit_bytes(*tensor.shape, rank)
        need(estimate <= self.max_workspace_bytes, "GPU fitting exceeds its declared logical workspace budget",
             CapacityError)
        device = self._device()
        need(reuse_basis is None and reuse_threshold is None,
             "explicit GPU solver comparisons currently require fresh bases", UnsupportedError)
        need(self.method in SUPPORTED_FIT_METHODS, f"GPU fitting method {self.method!r} is a CUDA library SVD "
             f"backend; this MI355X build fits with {SUPPORTED_FIT_METHODS}", UnsupportedError)
        started = time.perf_counter()
        # Marks after: nothing, the upload, the fit, the download.
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        with torch.cuda.device(device), self._scope(device):
            marks[0].record()
            source = tensor.to(device)
            marks[1].record()
            factors = self._fit_gram_batched(source, tensor, context, rank)
            marks[2].record()
            basis, coefficients = factors.basis.cpu(), factors.coefficients.cpu()
            marks[3].record()
            marks[3].synchronize()
        h2d, compute, d2h = (marks[i].elapsed_time(marks[i + 1]) for i in range(3))
        wall = time.perf_counter() - started
        metrics = dict(factors.metrics)
        metrics.update(gpu_fitting_backend=self.method, gpu_fitting_uuid=self.gpu_uuid,
                       gpu_fitting_workspace_estimate=estimate, gpu_fitting_h2d_ms=h2d,
                       gpu_fitting_compute_ms=compute, gpu_fitting_d2h_ms=d2h, gpu_fitting_wall_seconds=wall,
                       **_NO_REUSE, total_factorization_seconds=wall, canonical_basis_rank=rank, view_rank=rank)
        return Factors(basis=basis, coefficients=coefficients, rank=rank, metrics=metrics)

    def _basis_for(self, source, tensor, context, rank):
        """(stored basis, decomposition seconds, algorithm label, from the prefit cache)."""
        batched = self.method == "gram_batched"
        cached = self._prefit.pop(_tensor_identity(tensor, context, rank), None) if batched else None
        if cached is not None:
            validate_matrix(source, context)
            self.prefit_stats["hits"] += 1
            return cached[1], cached[2], "batched_fp32_gram_eigh", True
        if batched:
            self.prefit_stats["misses"] += 1
        clock = time.perf_counter()
        (basis,) = _stored_bases(gram_bases([validate_matrix(source, context)], [rank]))
        return basis, time.perf_counter() - clock, "fp32_gram_eigh" if batched else "custom_fp32_gram_eigh", False

    def _fit_gram_batched(self, source, tensor, context, rank):
        """The prefit basis when available; otherwise a single-matrix Gram eigh; then the projection."""
        started = time.perf_counter()
        basis, decomposition, algorithm, prefit = self._basis_for(source, tensor, context, rank)
        projection = project_onto_basis(source, basis, rank=rank, _condition_bound=fast_condition_bound(basis))
        metrics = {
            "factorization_method": algorithm, "factorization_seed": self.seed, "sketch_rank": None,
            "power_iterations": 0, "decomposition_count": 1, "svd_count": 0, "eigh_count": 1, "qr_count": 0,
            "decomposition_seconds": decomposition, "projection_count": 1, "projection_seconds": projection.seconds,
            "projection_relative_residual": projection.relative_residual,
            "basis_condition_bound": projection.condition_bound, "basis_condition_method": "fp32_neumann_upper_bound",
            "zero_input": projection.zero_input, "prefit_batched": prefit,
        }
        metrics["fit_seconds"] = time.perf_counter() - started
        return Factors(basis=basis, coefficients=projection.coefficients, rank=rank, metrics=metrics)

    # -- chunk planning -------------------------------------------------------

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
        with self._lock if self.shared else contextlib.nullcontext(), torch.cuda.device(device), \
                self._scope(device):
            plan = planner.plan(sources, contexts, bindings, parent_rows, chunk_id=chunk_id, source_ids=source_ids)
        self.prefit_stats["solver"] = label
        return plan


__all__ = ["BoundedEigh", "EIGH_SOLVERS", "GPUFitter", "GPU_FIT_METHODS", "default_eigh_sub_batch", "gram_bases",
           "select_eigh_solver", "torch_batched_eigh_is_rocsolver", "torch_batched_eigh_is_xsyevbatched"]
