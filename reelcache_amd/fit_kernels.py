"""Host side of the fit kernels (``rch_fit_*``, ``rch_column_extrema``, ``rch_quantize``).

Each function builds the ``rch_fit_matrix`` descriptor table of a batch, allocates the device
outputs (torch is used for memory and streams only) and launches on the current stream of the
sources' device.  Every result stays on the device; callers read what they need once.  CPU
tensors and a missing library raise :class:`UnsupportedError` -- there is no host fallback.

Layout rules the kernels rely on (violating inputs are copied into zero-padded buffers here):
rows of X and Q start 16-byte aligned with unit column stride, and channels % 8 == 0.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .errors import ConfigurationError, UnsupportedError

_DTYPE_CODES = {torch.bfloat16: _lib.DT_BF16, torch.float16: _lib.DT_F16, torch.float32: _lib.DT_F32}
#: fp32 bits of +inf: an absmax key at or above it marks a non-finite source element.
NONFINITE_BITS = 0x7F800000
_ROW_TILE = 64  # rows per partial energy


def _device(tensors) -> torch.device:
    devices = {tensor.device for tensor in tensors}
    if len(devices) != 1:
        raise ConfigurationError("one fit batch must live on one device")
    (device,) = devices
    if device.type != "cuda":
        raise UnsupportedError("the fit kernels run on the GPU (HIP, gfx950); move the matrices to a cuda device")
    _lib.library()  # raises UnsupportedError with the reason when the library is unavailable
    return device


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def padded(channels: int) -> int:
    return -(-channels // 8) * 8


def _aligned(x: torch.Tensor, channels: int) -> torch.Tensor:
    """``x`` when the kernels can read it in place, else a copy into a zero-padded buffer."""
    size = x.element_size()
    if (x.shape[1] == channels and x.stride(1) == 1 and x.stride(0) >= channels
            and (x.stride(0) * size) % 16 == 0 and x.data_ptr() % 16 == 0):
        return x
    out = torch.zeros((x.shape[0], channels), dtype=x.dtype, device=x.device)
    out[:, :x.shape[1]].copy_(x)
    return out


def _check_sources(sources) -> tuple[list[torch.Tensor], int, int]:
    if not sources:
        raise ConfigurationError("a fit batch needs at least one matrix")
    shapes = [x.shape for x in sources]  # each tensor's shape, strides and address read once
    channels = {int(shape[1]) for shape in shapes}
    if len(channels) != 1:
        raise ConfigurationError("one fit batch must share the channel count")
    dtypes = {x.dtype for x in sources}
    if len(dtypes) != 1 or next(iter(dtypes)) not in _DTYPE_CODES:
        raise UnsupportedError("the fit kernels take one of bfloat16, float16 or float32 per batch")
    for shape in shapes:
        if len(shape) != 2 or shape[0] < 1 or shape[1] < 1:
            raise ConfigurationError("fit sources must be nonempty 2-D matrices")
    (c,) = channels
    c8 = padded(c)
    if c != c8:
        return [_aligned(x, c8) for x in sources], c, c8
    size = sources[0].element_size()
    aligned = []
    for x in sources:
        stride = x.stride()
        # _aligned's in-place rule (the channel count is c8 here).
        if stride[1] == 1 and stride[0] >= c8 and (stride[0] * size) % 16 == 0 and x.data_ptr() % 16 == 0:
            aligned.append(x)
        else:
            aligned.append(_aligned(x, c8))
    return aligned, c, c8


def _table(count: int) -> np.ndarray:
    return np.zeros(count, dtype=_lib.FIT_DTYPE)


def _upload(table: np.ndarray, device: torch.device) -> torch.Tensor:
    """The descriptor table on the device, copied from pinned memory on the current stream without
    a host wait (a pageable copy would drain the stream first).  The pinned block stays reserved
    until the copy has run (torch's host allocator records it on the stream)."""
    staged = torch.from_numpy(table.view(np.int64)).pin_memory()
    return staged.to(device, non_blocking=True)


def _fill_sources(table: np.ndarray, sources) -> None:
    """Source columns of a descriptor table, filled column by column (not row by row); one batch
    has one dtype (``_check_sources``)."""
    table["src_ptr"] = [x.data_ptr() for x in sources]
    table["src_dtype"] = _DTYPE_CODES[sources[0].dtype]
    table["rows"] = [x.shape[0] for x in sources]
    table["src_stride"] = [x.stride(0) for x in sources]


def decode_max_keys(keys) -> np.ndarray:
    """fp32 values of order-preserving keys (the per-column maxima)."""
    k = np.asarray(keys, dtype=np.int64).astype(np.uint32)
    bits = np.where(k & np.uint32(0x80000000), k & np.uint32(0x7FFFFFFF), ~k)
    return bits.astype(np.uint32).view(np.float32)


def decode_min_keys(keys) -> np.ndarray:
    """fp32 values of inverted order-preserving keys (the per-column minima)."""
    return decode_max_keys(~np.asarray(keys, dtype=np.int64).astype(np.uint32))


# ---------------------------------------------------------------------------------------------
# Batched entry points
# ---------------------------------------------------------------------------------------------


def absmax(sources) -> torch.Tensor:
    """int32 [n]: fp32 bits of max|X| of each source (>= NONFINITE_BITS when X holds inf/nan)."""
    device = _device(sources)
    aligned, _, c8 = _check_sources(sources)
    keys = torch.zeros(len(aligned), dtype=torch.int32, device=device)
    table = _table(len(aligned))
    _fill_sources(table, aligned)
    table["absmax_ptr"] = keys.data_ptr() + 4 * np.arange(len(aligned))
    descriptors = _upload(table, device)
    max_rows = max(int(x.shape[0]) for x in aligned)
    _lib.call("rch_fit_absmax", descriptors.data_ptr(), len(aligned), c8, max_rows, _DTYPE_CODES[aligned[0].dtype],
              _stream(device))
    return keys


def gram(sources) -> torch.Tensor:
    """fp32 [n, C, C]: exactly symmetric X^T X of each source (MFMA, exact products)."""
    device = _device(sources)
    aligned, channels, c8 = _check_sources(sources)
    grams = torch.empty((len(aligned), c8, c8), dtype=torch.float32, device=device)
    table = _table(len(aligned))
    _fill_sources(table, aligned)
    table["gram_ptr"] = grams.data_ptr() + 4 * c8 * c8 * np.arange(len(aligned))
    table["gram_stride"] = c8
    descriptors = _upload(table, device)
    _lib.call("rch_fit_gram", descriptors.data_ptr(), len(aligned), c8, _DTYPE_CODES[aligned[0].dtype], _stream(device))
    return grams if c8 == channels else grams[:, :channels, :channels]


def _basis_rows(basis: torch.Tensor, rank: int, c8: int, keep: list) -> tuple[int, int]:
    """(address, row stride) of ``basis[:rank]`` as the kernels read it: the basis itself when its
    rows can be read in place (``_aligned``'s rule; a row prefix keeps the address and stride), else
    a zero-padded copy appended to ``keep``."""
    if basis.dtype != torch.float16:
        raise ConfigurationError("the stored basis must be float16")
    stride = basis.stride()
    address = basis.data_ptr()
    if basis.shape[1] == c8 and stride[1] == 1 and stride[0] >= c8 and (stride[0] * 2) % 16 == 0 and address % 16 == 0:
        return address, stride[0]
    q = _aligned(basis[:rank], c8)
    keep.append(q)
    return q.data_ptr(), q.stride(0)


def project(sources, bases, ranks, *, extrema: bool = False):
    """``(coefficients, keys)``: fp32 P = X Q[:rank]^T per source (FP64-accumulated MFMA) and,
    with ``extrema``, int32 [n, 2 * max_rank] order keys of the columns of P: row i holds
    ~key(min) of its columns in [0, rank_i) and key(max) in [rank_i, 2 rank_i) (see :func:`split_keys`)."""
    device = _device(sources)
    aligned, _, c8 = _check_sources(sources)
    if len(bases) != len(aligned) or len(ranks) != len(aligned):
        raise ConfigurationError("projection needs one basis and one rank per source")
    table = _table(len(aligned))
    _fill_sources(table, aligned)
    keep, outputs = [], []
    max_rank = max(int(r) for r in ranks)
    keys = torch.zeros((len(aligned), 2 * max_rank), dtype=torch.int32, device=device) if extrema else None
    ranks = [int(rank) for rank in ranks]
    rows = [int(x.shape[0]) for x in aligned]
    strides = [-(-rank // 4) * 4 for rank in ranks]
    sizes = [count * stride for count, stride in zip(rows, strides)]
    storage = torch.empty(sum(sizes), dtype=torch.float32, device=device)  # every P of the batch, 16-byte rows
    storage_address = storage.data_ptr()
    first = 0
    basis_ptr, basis_stride, coef_ptr = [], [], []
    for index, (basis, rank) in enumerate(zip(bases, ranks)):
        shape = basis.shape
        if not 1 <= rank <= shape[0] or shape[1] > c8 or basis.device != device:
            raise ConfigurationError("projection basis does not match its source")
        address, stride = _basis_rows(basis, rank, c8, keep)
        basis_ptr.append(address)
        basis_stride.append(stride)
        # P of source index: rows x stride fp32 at element offset `first` of the storage.
        outputs.append(torch.as_strided(storage, (rows[index], rank), (strides[index], 1), first))
        coef_ptr.append(storage_address + 4 * first)
        first += sizes[index]
    table["basis_ptr"] = basis_ptr
    table["basis_stride"] = basis_stride
    table["rank"] = ranks
    table["coef_ptr"] = coef_ptr
    table["coef_stride"] = strides
    if extrema:
        table["extrema_ptr"] = keys.data_ptr() + 4 * 2 * max_rank * np.arange(len(aligned))
    descriptors = _upload(table, device)
    max_rows = max(int(x.shape[0]) for x in aligned)
    _lib.call("rch_fit_project", descriptors.data_ptr(), len(aligned), c8, max_rows, max_rank,
              _DTYPE_CODES[aligned[0].dtype], _stream(device))
    del keep
    return outputs, keys


def split_keys(keys_row, rank: int) -> tuple[np.ndarray, np.ndarray]:
    """Host fp32 (min, max) of each of the ``rank`` columns from one row of :func:`project` keys."""
    row = np.asarray(keys_row)
    return decode_min_keys(row[:rank]), decode_max_keys(row[rank:2 * rank])


def split_keys_many(keys_rows, ranks) -> tuple[list, list, list]:
    """:func:`split_keys` of every row of a ``[n, width]`` key block at once (one vectorized decode
    per rank): per row the fp32 (min, max) arrays and whether both are finite."""
    rows = np.asarray(keys_rows)
    lows, highs, finite = [None] * len(ranks), [None] * len(ranks), [False] * len(ranks)
    by_rank: dict = {}
    for index, rank in enumerate(ranks):
        by_rank.setdefault(int(rank), []).append(index)
    for rank, members in by_rank.items():
        block = rows[members]
        low, high = decode_min_keys(block[:, :rank]), decode_max_keys(block[:, rank:2 * rank])
        ok = np.isfinite(low).all(1) & np.isfinite(high).all(1)
        for position, index in enumerate(members):
            lows[index], highs[index], finite[index] = low[position], high[position], bool(ok[position])
    return lows, highs, finite


def energies(sources, absmax_keys: torch.Tensor, *, bases=None, ranks=None, coefficients=None,
             residuals: bool = False):
    """float64 [n, 2]: sum (X/s)^2 and sum ((X - P Q)/s)^2 per source, s = max|X| from ``absmax_keys``
    (FP64, fixed-order sums); without bases only the source energy (second column = first).
    With ``residuals`` returns ``(totals, [fp32 X - P Q per source])``."""
    device = _device(sources)
    aligned, _, c8 = _check_sources(sources)
    n = len(aligned)
    if absmax_keys.shape != (n,) or absmax_keys.dtype != torch.int32 or absmax_keys.device != device:
        raise ConfigurationError("energies need the int32 absmax keys of the same batch")
    with_basis = bases is not None
    if with_basis and not (len(bases) == len(ranks) == len(coefficients) == n):
        raise ConfigurationError("residual energies need one basis, rank and coefficient matrix per source")
    table = _table(n)
    _fill_sources(table, aligned)
    tiles = [-(-int(x.shape[0]) // _ROW_TILE) for x in aligned]
    partials = torch.empty(2 * sum(tiles), dtype=torch.float64, device=device)
    totals = torch.empty((n, 2), dtype=torch.float64, device=device)
    table["absmax_ptr"] = absmax_keys.data_ptr() + 4 * np.arange(n)
    table["energy_ptr"] = totals.data_ptr() + 16 * np.arange(n)
    table["partial_ptr"] = partials.data_ptr() + 16 * np.concatenate(([0], np.cumsum(tiles)[:-1]))
    keep, outputs = [], []
    if residuals:
        for index, x in enumerate(aligned):
            r = torch.empty((x.shape[0], c8), dtype=torch.float32, device=device)
            table[index]["resid_ptr"] = r.data_ptr()
            outputs.append(r[:, :sources[index].shape[1]])
    if with_basis:
        columns = {"basis_ptr": [], "basis_stride": [], "rank": [], "coef_ptr": [], "coef_stride": []}
        for index, (x, basis, rank, p) in enumerate(zip(aligned, bases, ranks, coefficients)):
            rank = int(rank)
            if not 1 <= rank <= basis.shape[0] or p.shape != (x.shape[0], rank) or p.dtype != torch.float32:
                raise ConfigurationError("residual coefficients do not match their source and rank")
            basis_address, basis_stride = _basis_rows(basis, rank, c8, keep)
            p_stride = p.stride()
            p_address = p.data_ptr()
            if p_stride[1] != 1 or (p_stride[0] * 4) % 16 or p_address % 16:
                stride = -(-rank // 4) * 4
                copy = torch.zeros((p.shape[0], stride), dtype=torch.float32, device=device)
                copy[:, :rank].copy_(p)
                keep.append(copy)
                p_stride, p_address = copy.stride(), copy.data_ptr()
            columns["basis_ptr"].append(basis_address)
            columns["basis_stride"].append(basis_stride)
            columns["rank"].append(rank)
            columns["coef_ptr"].append(p_address)
            columns["coef_stride"].append(p_stride[0])
        for name, values in columns.items():
            table[name] = values
    descriptors = _upload(table, device)
    _lib.call("rch_fit_residual", descriptors.data_ptr(), n, c8, max(int(x.shape[0]) for x in aligned),
              _DTYPE_CODES[aligned[0].dtype], _stream(device))
    del keep
    return (totals, outputs) if residuals else totals


CHOLESKY_MAX_K = 128  # RCH_CHOLESKY_MAX_K: one k x k FP64 matrix per workgroup, held in LDS


def cholesky_inverse(gram: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``(inverse, info)`` of a batch ``[n, k, k]`` of FP64 symmetric positive definite matrices on
    the device (k <= :data:`CHOLESKY_MAX_K`): ``inverse = R^-1`` with ``A = R^T R`` (R upper, only
    the upper triangle of A read) and int32 ``info`` (0, or j + 1 when the leading minor of order
    j + 1 is not positive definite; that member's inverse is the identity), in one launch."""
    if (gram.ndim != 3 or gram.shape[1] != gram.shape[2] or gram.dtype != torch.float64
            or gram.device.type != "cuda" or not 1 <= gram.shape[1] <= CHOLESKY_MAX_K or gram.shape[0] < 1):
        raise ConfigurationError(f"cholesky_inverse takes a device float64 [n, k, k] batch with k <= {CHOLESKY_MAX_K}")
    a = gram.contiguous()
    inverse = torch.empty_like(a)
    info = torch.empty(a.shape[0], dtype=torch.int32, device=a.device)
    _lib.call("rch_cholesky_inverse", a.data_ptr(), inverse.data_ptr(), info.data_ptr(), int(a.shape[0]),
              int(a.shape[1]), _stream(a.device))
    return inverse, info


def gaussian(blocks) -> None:
    """Fill each ``(view, seed)`` of ``blocks`` with seeded standard normals in one launch: ``view``
    an fp32 ``[rows, cols]`` device tensor with unit column stride (e.g. the trailing columns of a
    start block), ``seed`` a 64-bit integer; the values depend only on the seed and the shape."""
    blocks = list(blocks)
    if not blocks:
        return
    device = _device([view for view, _ in blocks])
    table = np.zeros(len(blocks), dtype=_lib.GAUSS_DTYPE)
    for row, (view, seed) in zip(table, blocks):
        if view.dtype != torch.float32 or view.ndim != 2 or view.stride(1) != 1 or min(view.shape) < 1:
            raise ConfigurationError("Gaussian blocks are nonempty fp32 [rows, cols] views with unit column stride")
        row["dst_ptr"], row["rows"], row["cols"], row["stride"] = view.data_ptr(), view.shape[0], view.shape[1], \
            view.stride(0)
        row["seed"] = np.int64(np.uint64(int(seed) % 2 ** 64).astype(np.int64))
    descriptors = _upload(table, device)
    _lib.call("rch_fit_gaussian", descriptors.data_ptr(), len(blocks), int((table["rows"] * table["cols"]).max()),
              _stream(device))


def column_extrema(values: torch.Tensor) -> torch.Tensor:
    """int32 [2 * cols] order keys of every column of an fp32 matrix: ~key(min) then key(max)
    (the layout :func:`split_keys` reads with ``rank = cols``)."""
    device = _device([values])
    if values.dtype != torch.float32 or values.ndim != 2 or min(values.shape) < 1 or values.stride(1) != 1:
        raise ConfigurationError("column extrema take a nonempty fp32 matrix with unit column stride")
    keys = torch.zeros(2 * values.shape[1], dtype=torch.int32, device=device)
    _lib.call("rch_column_extrema", values.data_ptr(), values.shape[0], values.shape[1], values.stride(0),
              keys.data_ptr(), _stream(device))
    return keys


def quantize(values: torch.Tensor, scale: torch.Tensor, offset: torch.Tensor) -> torch.Tensor:
    """uint8 codes clamp(rint((v - offset) / scale), 0, 255) in FP64 (0 where scale == 0)."""
    device = _device([values])
    if values.dtype != torch.float32 or values.ndim != 2 or min(values.shape) < 1 or values.stride(1) != 1:
        raise ConfigurationError("quantization takes a nonempty fp32 matrix with unit column stride")
    cols = values.shape[1]
    for vector in (scale, offset):
        if vector.dtype != torch.float64 or vector.shape != (cols,) or vector.device != device:
            raise ConfigurationError("quantization needs float64 scale and offset vectors per column")
    scale, offset = scale.contiguous(), offset.contiguous()
    codes = torch.empty(values.shape, dtype=torch.uint8, device=device)
    _lib.call("rch_quantize", values.data_ptr(), values.shape[0], cols, values.stride(0), scale.data_ptr(),
              offset.data_ptr(), codes.data_ptr(), codes.stride(0), _stream(device))
    return codes


def quantize_batched(values, affines) -> list[torch.Tensor]:
    """:func:`quantize` of many fp32 matrices in one launch: ``affines[i]`` is the float64
    ``[2, cols_i]`` host (scale; offset) of ``values[i]``; one host-to-device copy for all."""
    device = _device(values)
    if len(values) != len(affines) or not values:
        raise ConfigurationError("batched quantization needs one affine per matrix")
    shapes = [v.shape for v in values]
    parts = []
    for v, shape, affine in zip(values, shapes, affines):
        affine = np.asarray(affine, dtype=np.float64)
        if (v.dtype != torch.float32 or len(shape) != 2 or min(shape) < 1 or v.stride(1) != 1
                or affine.shape != (2, shape[1])):
            raise ConfigurationError("batched quantization takes nonempty fp32 matrices and [2, cols] affines")
        parts.append(affine.reshape(-1))  # a copy when the affine is a strided view
    rows = [int(shape[0]) for shape in shapes]
    cols = [int(shape[1]) for shape in shapes]
    host = torch.from_numpy(np.concatenate(parts))
    device_affine = host.to(device)
    # Every matrix's codes in one allocation: matrix i's [rows, cols] block at element offset first_i.
    sizes = [r * c for r, c in zip(rows, cols)]
    firsts = np.concatenate(([0], np.cumsum(sizes[:-1], dtype=np.int64)))
    storage = torch.empty(int(sum(sizes)), dtype=torch.uint8, device=device)
    codes = [torch.as_strided(storage, (r, c), (c, 1), int(first)) for r, c, first in zip(rows, cols, firsts)]
    table = np.zeros(len(values), dtype=_lib.QUANTIZE_DTYPE)
    table["values_ptr"] = [v.data_ptr() for v in values]
    table["rows"] = rows
    table["cols"] = cols
    table["stride"] = [v.stride(0) for v in values]
    table["affine_ptr"] = device_affine.data_ptr() + 16 * np.concatenate(([0], np.cumsum(cols[:-1], dtype=np.int64)))
    table["codes_ptr"] = storage.data_ptr() + firsts
    table["code_stride"] = cols
    descriptors = _upload(table, device)
    _lib.call("rch_quantize_batched", descriptors.data_ptr(), len(values), max(rows), _stream(device))
    return codes
