"""Builders of seeded restore jobs shared by the CPU and GPU tests.

Each builder returns the product's ``ReconstructionJob`` (tensors on the
requested device) and the oracle's float64 view of the same inputs, so tests
compare the product's output with ``oracle.restore`` on identical data.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from oracle import quantize as oq
from oracle import restore as orc
from reelcache_amd import restore_kernels as rk

TORCH_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def random_affine(rank, rng):
    """Affine of a random coefficient range, as the reference tests draw it
    (tests/test_restore_kernels.py:287-291): lo ~ U(-4, 0), hi = lo + U(0.5, 6)."""
    lo = rng.uniform(-4, 0, size=rank).astype(np.float32)
    hi = (lo.astype(np.float64) + rng.uniform(0.5, 6, size=rank)).astype(np.float32)
    affine = oq.covering_affine(lo, hi)
    return affine[0].copy(), affine[1].copy()


def orthonormal_basis(rows, channels, rng, dtype=torch.float16):
    """Rows of a random orthonormal matrix (QR of a Gaussian), rounded to ``dtype``."""
    q, _ = np.linalg.qr(rng.standard_normal((channels, rows)))
    return torch.from_numpy(q.T.copy()).to(dtype)


@dataclass
class Case:
    job: rk.ReconstructionJob
    coefficients: np.ndarray      # float32 [N, rank] the job reconstructs from
    basis: np.ndarray             # float64 [rank, C] (the basis values)
    heads: int
    rope: tuple | None            # per-token (cos, sin) float64 or None
    out_dtype: str


def destination(layout, tokens, heads, head_dim, dtype, device, *, offset=0, extra=0, fill=0.0):
    total = offset + tokens + extra
    shape = {"BTHD": (1, total, heads, head_dim), "THD": (total, heads, head_dim),
             "BHTD": (1, heads, total, head_dim)}[layout]
    return torch.full(shape, fill, dtype=TORCH_DTYPES[dtype], device=device)


def make_case(rng, *, grid, heads, head_dim, rank, basis_rows=None, source="uint8", rope="separable",
              layout="BTHD", out_dtype="bfloat16", device="cpu", basis_dtype=torch.float16, token_offset=0,
              view=None, basis=None, table=None, rope_rows=None, coefficient_dtype=torch.float32, code_pitch=None,
              picture_origin=(2, 3), picture_pad=(3, 5)):
    """One job with random inputs; ``view`` (a NativeView) overrides the destination.

    ``code_pitch``: uint8 codes live in the first ``rank`` columns of ``[N, code_pitch]`` rows
    whose padding holds nonzero bytes (they must not leak into the product)."""
    tokens = int(np.prod(grid))
    channels = heads * head_dim
    if basis is None:
        basis = orthonormal_basis(max(rank, basis_rows or rank), channels, rng, basis_dtype).to(device)
    basis_values = basis[:rank].double().cpu().numpy()
    if view is None:
        tensor = destination(layout, tokens, heads, head_dim, out_dtype, device, offset=token_offset, extra=3,
                             fill=-123.0)
        view = rk.NativeView(tensor, layout, token_offset=token_offset)
    if source in ("uint8", "pictures"):
        codes = rng.integers(0, 256, size=(tokens, rank), dtype=np.uint8)
        scale, offset = random_affine(rank, rng)
        coefficients = orc.dequantize(codes, scale, offset)
        if source == "uint8":
            stored = codes
            if code_pitch is not None:
                stored = np.full((tokens, code_pitch), 0xA5, dtype=np.uint8)
                stored[:, :rank] = codes
            values = torch.from_numpy(stored).to(device)[:, :rank]
            src = rk.CoefficientSource(values, scale, offset)
        else:
            layout_v1 = oq.video_layout(grid[0], grid[1], grid[2], rank, "yuv444p")
            canvas, indices = orc.pack_pictures(codes, layout_v1, origin=picture_origin, pad=picture_pad)
            src = rk.PictureSource.from_canvases(torch.from_numpy(canvas).to(device), layout_v1, indices,
                                                 tuple(picture_origin), scale, offset)
    elif source == "float":
        values = torch.from_numpy(rng.standard_normal((tokens, rank)).astype(np.float32) * 3).to(coefficient_dtype)
        coefficients = values.float().numpy()
        src = rk.CoefficientSource(values.to(device))
    else:
        raise ValueError(source)
    positions = None
    rope_values = None
    if rope != "none":
        if table is None:
            if rope == "separable":
                freqs = torch.from_numpy(orc.wan_freqs(head_dim, 64))
                table = rk.RopeTable.from_complex(freqs)
            else:
                angles = rng.uniform(0, 2 * np.pi, size=(tokens + 9, head_dim // 2))
                table = rk.RopeTable.from_cos_sin(torch.from_numpy(np.cos(angles)).float(),
                                                  torch.from_numpy(np.sin(angles)).float())
        if rope_rows is None:
            rope_rows = (3, 1, 2) if table.sections is not None else 5
        positions = rk.RopePositions(table, rope_rows)
        # The kernels use FP32 tables; the expected values use the same FP32 table values.
        cos32 = table.cos.float().double().numpy()
        sin32 = table.sin.float().double().numpy()
        rope_values = orc.rope_cos_sin(cos32, sin32, table.sections, positions.rows, grid)
    job = rk.ReconstructionJob(src, view, grid, basis, rank, positions)
    return Case(job, coefficients, basis_values, heads, rope_values, out_dtype)


def written(case):
    """The destination slot as float64 [N, C]."""
    job = case.job
    return job.destination.slot(job.tokens).reshape(job.tokens, -1).double().cpu().numpy()


def expected(case, precision):
    """Oracle ``(y*, bound)`` for a case (float64)."""
    return orc.error_bound(case.coefficients, case.basis, case.heads, case.rope, precision, case.out_dtype)
