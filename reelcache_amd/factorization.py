"""Stored-basis projection and energy measurement of the fit path (GPU, HIP kernels).

The public names, arguments, results and errors are those of ``reelcache/factorization.py``
(Projection :164-175, Factors :178-183, validate_matrix :206-239, validate_rank :242-245,
validate_stored_basis :248-260, basis_condition_bound :271-292, fast_condition_bound
:294-315, project_onto_basis :318-434, _canonical_signs :437-441, SourceEnergy :562-571,
measure_source_energy :692-724).  A stored basis is FP16 and coefficients follow
``P = X.float() @ B.float().T``; the direct residual and source energies accumulate in FP64.

MI355X design: one launch each for max|X| (which is also the finite scan), the projection
(exact products summed in FP64 on MFMA, rounded once to fp32, with the per-column extrema of P
fused in) and the residual / source energies (FP64 MFMA reconstruction, per-64-row partials,
fixed-order totals); the host reads the scalars it needs in one transfer.  ``tile_rows`` is
validated but does not change the result beyond FP64 summation order.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass, field
from typing import Any

import torch

from . import fit_kernels
from .errors import ConfigurationError, UnsupportedError
from .types import canonical_dtype


@dataclass(frozen=True)
class Projection:
    coefficients: torch.Tensor
    relative_residual: float
    source_norm: float
    residual_norm: float
    zero_input: bool
    condition_bound: float
    seconds: float
    coefficient_seconds: float = 0.0
    guard_seconds: float = 0.0
    condition_seconds: float = 0.0


@dataclass(frozen=True)
class Factors:
    basis: torch.Tensor
    coefficients: torch.Tensor
    rank: int
    metrics: dict[str, Any] = field(default_factory=dict)


@dataclass(frozen=True)
class SourceEnergy:
    """max|X|, the FP64 energy of X / max|X| and the derived norm and energy of X."""

    scale: float
    scaled_energy: float
    source_norm: float
    source_energy: float
    zero_input: bool
    seconds: float


def _is_context(context) -> bool:
    try:
        return (isinstance(context.shape, tuple) and isinstance(context.dtype, str)
                and context.key.target in ("K", "V") and isinstance(context.key_space, str))
    except AttributeError:
        return False


def validate_matrix(tensor: torch.Tensor, context, *, lossy: bool = True, check_values: bool = True) -> torch.Tensor:
    """Geometry and key-space checks of one [tokens, channels] matrix against its context.

    ``context`` is any object with the TensorContext attributes (``shape``, ``dtype``,
    ``key.target``, ``key_space``), e.g. ``reelcache_amd.types.TensorContext``.  Lossy
    arithmetic needs finite values; the scan runs on the tensor's device (the absmax kernel on
    a GPU) unless ``check_values`` is False.
    """
    if not _is_context(context):
        raise ConfigurationError("context must be a TensorContext")
    if not isinstance(tensor, torch.Tensor) or tensor.layout != torch.strided:
        raise ConfigurationError("tensor must be a dense strided torch.Tensor")
    if tensor.device.type == "meta":
        raise ConfigurationError("meta tensors have no encodable values")
    if tensor.ndim != 2 or tuple(tensor.shape) != tuple(context.shape):
        raise ConfigurationError(f"tensor shape must equal context shape {context.shape}")
    if canonical_dtype(tensor.dtype) != context.dtype:
        raise ConfigurationError("tensor dtype differs from the declared matrix dtype")
    if context.key.target == "K":
        if context.key_space not in ("pre_rope", "post_rope"):
            raise ConfigurationError("K requires an explicit pre_rope or post_rope key_space")
        if lossy and context.key_space != "pre_rope":
            raise ConfigurationError("SVD requires normalized pre-RoPE K; post-RoPE K is RAW-only")
    elif context.key_space != "none":
        raise ConfigurationError("V must be direct values with key_space='none'")
    result = tensor.detach()
    if lossy and check_values and not all_finite([result]):
        raise ConfigurationError("lossy input must be finite and representable in FP32")
    return result


def all_finite(matrices) -> bool:
    """Whether every element of every matrix is finite (one device scan and one read on a GPU)."""
    if matrices[0].device.type == "cuda" and all(m.dtype in fit_kernels._DTYPE_CODES for m in matrices):
        keys = fit_kernels.absmax(matrices)
        return bool((keys.cpu() < fit_kernels.NONFINITE_BITS).all())
    return all(bool(torch.isfinite(m).all()) and bool(torch.isfinite(m.float()).all()) for m in matrices)


def validate_rank(rank: int, shape: tuple[int, int]) -> int:
    if type(rank) is not int or not 1 <= rank <= min(shape):
        raise ConfigurationError(f"rank must be an integer in [1, {min(shape)}]")
    return rank


def validate_stored_basis(basis: torch.Tensor, channels: int) -> torch.Tensor:
    if not isinstance(basis, torch.Tensor) or basis.layout != torch.strided:
        raise ConfigurationError("reuse basis must be a dense torch.Tensor")
    if basis.device.type == "meta" or basis.dtype != torch.float16:
        raise ConfigurationError("reuse basis must be the actual stored FP16 basis")
    if basis.ndim != 2 or basis.shape[1] != channels or not 1 <= basis.shape[0] <= channels:
        raise ConfigurationError("stored basis must have shape [canonical_rank, channels]")
    if not bool(torch.isfinite(basis).all()):
        raise ConfigurationError("stored basis must be finite")
    return basis.detach()


def _canonical_signs(basis: torch.Tensor) -> torch.Tensor:
    """Rows flipped so that the first entry of largest magnitude of each row is positive; a
    ``[..., rows, C]`` batch is handled in one reduction (rows along the last dimension)."""
    pivot = basis.gather(-1, basis.abs().argmax(dim=-1, keepdim=True))
    return basis * torch.where(pivot < 0, -1.0, 1.0).to(basis.dtype)


@torch.no_grad()
def basis_condition_bound(basis: torch.Tensor) -> float:
    """Infinity-norm condition bound ||G|| ||G^-1|| of G = B B^T in FP64 via Cholesky
    (inf for a singular basis)."""
    rounded = basis.to(dtype=torch.float64)
    gram = rounded @ rounded.T
    factor, info = torch.linalg.cholesky_ex(gram, check_errors=False)
    if int(info.item()) != 0 or not bool(torch.isfinite(factor).all()):
        return math.inf
    inverse = torch.cholesky_inverse(factor)
    condition = float((gram.abs().sum(1).max() * inverse.abs().sum(1).max()).item())
    return condition if math.isfinite(condition) else math.inf


@torch.no_grad()
def fast_condition_bound(basis: torch.Tensor) -> float:
    """Upper bound (1 + eta) / (1 - eta) on :func:`basis_condition_bound`, eta = ||B B^T - I||_inf
    plus the rigorous fp32 summation slack (fp16 products are exact in fp32).  Falls back to the
    exact FP64 bound when eta >= 1/3 (the basis is not near orthonormal)."""
    rounded = basis.to(dtype=torch.float32)
    rows, channels = rounded.shape
    gram = rounded @ rounded.T
    largest = float(gram.diagonal().abs().max())
    gram.diagonal().sub_(1.0)
    eta = float(gram.abs().sum(1).max())
    unit = 2.0 ** -24
    gamma = channels * unit / (1 - channels * unit)
    eta += rows * gamma * largest + rows * unit
    if not math.isfinite(eta) or eta >= 1 / 3:
        return basis_condition_bound(basis)
    return (1 + eta) / (1 - eta)


def _check_projection_input(tensor) -> None:
    if (not isinstance(tensor, torch.Tensor) or tensor.layout != torch.strided or tensor.ndim != 2
            or min(tensor.shape) < 1 or not tensor.is_floating_point() or tensor.device.type == "meta"):
        raise ConfigurationError("projection requires a nonempty finite FP32-compatible matrix")
    if tensor.device.type != "cuda":
        raise UnsupportedError("projection runs on the GPU (HIP kernels); move the matrix to a cuda device")
    if tensor.dtype not in fit_kernels._DTYPE_CODES:
        raise UnsupportedError("projection takes bfloat16, float16 or float32 matrices")


@torch.no_grad()
def project_onto_basis(tensor: torch.Tensor, basis: torch.Tensor, *, rank: int | None = None, tile_rows: int = 1024,
                       max_condition: float = 1e6, _condition_bound: float | None = None,
                       _work: dict | None = None) -> Projection:
    """Project once onto the stored FP16 basis and measure the direct residual in FP64."""
    started = time.perf_counter()
    _check_projection_input(tensor)
    stored = validate_stored_basis(basis, tensor.shape[1])
    rank = stored.shape[0] if rank is None else rank
    validate_rank(rank, tuple(tensor.shape))
    if rank > stored.shape[0]:
        raise ConfigurationError("requested rank exceeds the immutable stored basis")
    if type(tile_rows) is not int or tile_rows < 1:
        raise ConfigurationError("tile_rows must be a positive integer")
    if (isinstance(max_condition, bool) or not isinstance(max_condition, (int, float))
            or not math.isfinite(max_condition) or max_condition < 1):
        raise ConfigurationError("max_condition must be finite and at least one")
    view = stored[:rank].to(device=tensor.device)
    condition_started = time.perf_counter()
    condition = basis_condition_bound(view) if _condition_bound is None else _condition_bound
    condition_seconds = time.perf_counter() - condition_started
    if not math.isfinite(condition) or condition > max_condition:
        raise ConfigurationError("stored basis is singular or ill-conditioned")
    coefficient_started = time.perf_counter()
    keys = fit_kernels.absmax([tensor])
    (coefficients,), extrema = fit_kernels.project([tensor], [view], [rank], extrema=True)
    totals = fit_kernels.energies([tensor], keys, bases=[view], ranks=[rank], coefficients=[coefficients])
    bits, low, high = _read_scalars(keys, extrema, rank)
    coefficient_seconds = time.perf_counter() - coefficient_started
    if bits >= fit_kernels.NONFINITE_BITS:
        raise ConfigurationError("projection requires a nonempty finite FP32-compatible matrix")
    if not (math.isfinite(low) and math.isfinite(high)):
        raise ConfigurationError("projection overflowed FP32")
    guard_started = time.perf_counter()
    source_squared, error_squared = (float(v) for v in totals[0].cpu())
    scale = float(torch.tensor(bits, dtype=torch.int32).view(torch.float32))
    if not math.isfinite(source_squared) or not math.isfinite(error_squared):
        raise ConfigurationError("nonfinite direct residual energy")
    zero = scale == 0.0
    residual = 0.0 if zero else math.sqrt(error_squared / source_squared)
    if not math.isfinite(residual):
        raise ConfigurationError("nonfinite relative projection residual")
    guard_seconds = time.perf_counter() - guard_started
    return Projection(
        coefficients=coefficients.contiguous(), relative_residual=residual,
        source_norm=scale * math.sqrt(source_squared), residual_norm=scale * math.sqrt(error_squared),
        zero_input=zero, condition_bound=condition, seconds=time.perf_counter() - started,
        coefficient_seconds=coefficient_seconds, guard_seconds=guard_seconds, condition_seconds=condition_seconds,
    )


def _read_scalars(keys: torch.Tensor, extrema: torch.Tensor, rank: int) -> tuple[int, float, float]:
    """One device->host read: (absmax bits, min of P, max of P)."""
    host = torch.cat((keys.view(-1), extrema.view(-1))).cpu().numpy()
    low, high = fit_kernels.split_keys(host[1:], rank)
    return int(host[0]), float(low.min()), float(high.max())


@torch.no_grad()
def measure_source_energy(tensor: torch.Tensor, *, tile_rows: int = 1024) -> SourceEnergy:
    """max|X| and the FP64 energy of X / max|X| (no FP32 pre-round of the values)."""
    started = time.perf_counter()
    if (not isinstance(tensor, torch.Tensor) or tensor.layout != torch.strided or tensor.device.type == "meta"
            or tensor.ndim != 2 or min(tensor.shape) < 1 or not tensor.is_floating_point()):
        raise ConfigurationError("source energy requires a nonempty floating matrix")
    if type(tile_rows) is not int or tile_rows < 1:
        raise ConfigurationError("tile_rows must be a positive integer")
    _check_projection_input(tensor)
    keys = fit_kernels.absmax([tensor])
    totals = fit_kernels.energies([tensor], keys)
    host = torch.cat((keys.to(torch.float64).view(-1), totals.view(-1))).cpu()
    bits = int(host[0])
    if bits >= fit_kernels.NONFINITE_BITS:
        raise ConfigurationError("source energy requires finite input")
    scale = float(torch.tensor(bits, dtype=torch.int32).view(torch.float32))
    scaled = float(host[1]) if scale else 0.0
    if not math.isfinite(scaled) or (scale != 0 and scaled <= 0):
        raise ConfigurationError("invalid original source energy")
    norm = scale * math.sqrt(scaled)
    energy = norm * norm
    if not math.isfinite(norm) or not math.isfinite(energy):
        raise ConfigurationError("original source energy exceeds FP64")
    return SourceEnergy(scale, scaled, norm, energy, scale == 0, time.perf_counter() - started)


__all__ = ["Factors", "Projection", "SourceEnergy", "basis_condition_bound", "fast_condition_bound",
           "measure_source_energy", "project_onto_basis", "validate_matrix", "validate_rank", "validate_stored_basis"]
