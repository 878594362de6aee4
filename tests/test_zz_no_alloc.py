"""GPU test of rch_restore_noalloc, the restore entry point that allocates nothing: the packed
bases live in the library's static device array.  Called through the C ABI (the planner's
``static_scratch`` mode), its output must equal rch_basis_pack + rch_restore's bit for bit, on
two calls in a row (the second smaller), and sizes beyond the array are refused."""

import ctypes

import numpy as np
import pytest
import torch

from reelcache_amd import _lib
from reelcache_amd import restore_kernels as rk
from reelcache_amd.errors import ConfigurationError

from restore_cases import expected, make_case, written

pytestmark = pytest.mark.gpu


def _cases(rng, device, grid, heads, ranks, basis_rows, layout="BTHD"):
    """K (RoPE) and V jobs sharing one basis per target, like one layer call."""
    channels = heads * 128
    cases = []
    for target, rank in zip("KV", ranks):
        basis = torch.from_numpy(np.linalg.qr(rng.standard_normal((channels, basis_rows)))[0].T.copy()) \
            .to(torch.bfloat16).to(device)
        for _ in range(2):
            cases.append(make_case(rng, grid=grid, heads=heads, head_dim=128, rank=rank, source="uint8",
                                   rope="separable" if target == "K" else "none", layout=layout, device=device,
                                   basis=basis))
    return cases


def _pair(cases, **kwargs):
    """Restore the cases twice -- default entry points, then the no-allocation one -- and return
    both outputs."""
    for case in cases:
        case.job.destination.tensor.fill_(-5.0)
    handle = rk.reconstruct([case.job for case in cases], **kwargs)
    handle.synchronize()
    first = [written(case) for case in cases]
    for case in cases:
        case.job.destination.tensor.fill_(-5.0)
    handle = rk.reconstruct([case.job for case in cases], config={"static_scratch": True}, **kwargs)
    handle.synchronize()
    second = [written(case) for case in cases]
    return first, second


def test_noalloc_matches_the_allocating_entry_points(device):
    rng = np.random.default_rng(71)
    big = _cases(rng, device, (3, 10, 13), 12, (128, 192), 192)
    first, second = _pair(big)
    for case, a, b in zip(big, first, second):
        np.testing.assert_array_equal(a, b)
        values, bound = expected(case, "fp16x2")
        assert float((np.abs(b - values) - bound).max()) <= 0
    # A second, smaller call: the array keeps the first call's contents, which must not leak.
    small = _cases(rng, device, (1, 6, 7), 4, (40, 72), 80, layout="THD")
    first, second = _pair(small, precision="fp16")
    for case, a, b in zip(small, first, second):
        np.testing.assert_array_equal(a, b)
        values, bound = expected(case, "fp16")
        assert float((np.abs(b - values) - bound).max()) <= 0


def test_noalloc_with_one_basis_in_two_launch_groups(device):
    """One basis shared by jobs of two rank classes (two launch groups) at different pack positions
    in each group: the no-allocation call must read each group's own copy."""
    rng = np.random.default_rng(73)
    heads = 4
    first = torch.from_numpy(np.linalg.qr(rng.standard_normal((heads * 128, 128)))[0].T.copy()).to(torch.bfloat16)
    second = torch.from_numpy(np.linalg.qr(rng.standard_normal((heads * 128, 192)))[0].T.copy()).to(torch.bfloat16)
    first, second = first.to(device), second.to(device)
    cases = [make_case(rng, grid=(1, 6, 9), heads=heads, head_dim=128, rank=rank, source="uint8", rope="none",
                       device=device, basis=basis)
             for rank, basis in ((128, first), (120, second), (40, second), (56, first))]
    one, two = _pair(cases)
    for case, a, b in zip(cases, one, two):
        np.testing.assert_array_equal(a, b)
        values, bound = expected(case, "fp16x2")
        assert float((np.abs(b - values) - bound).max()) <= 0


def _pack(rank, channels):
    pack = np.zeros(1, dtype=_lib.PACK_DTYPE)
    pack["src_dtype"], pack["rank"], pack["channels"], pack["row_stride"] = _lib.DT_F16, rank, channels, channels
    pack["ksteps"], pack["nblocks"] = (rank + 15) // 16, 2 * ((channels + 63) // 64)
    return pack


def test_noalloc_refuses_sizes_beyond_the_array(device):
    words = torch.zeros(64, dtype=torch.int32, device=device)  # stands in for descriptors; nothing launches
    address = words.data_ptr()
    stream = torch.cuda.current_stream(device).cuda_stream
    too_big = _pack(4096, 8192)  # 256 steps x 256 blocks x 1 KB = 64 MiB of fragments
    with pytest.raises(ConfigurationError, match="static scratch holds"):
        _lib.call("rch_restore_noalloc", too_big.ctypes.data, 1, address, 1, address, 1, address, 1, 8192, 128,
                  _lib.SRC_U8, _lib.DT_BF16, 4, 256, 0, stream)
    many = np.concatenate([_pack(16, 128)] * 9)
    with pytest.raises(ConfigurationError, match="at most 8"):
        _lib.call("rch_restore_noalloc", many.ctypes.data, 9, address, 1, address, 1, address, 1, 128, 128,
                  _lib.SRC_U8, _lib.DT_BF16, 4, 1, 0, stream)
    # Stream slabs must have the depth of the stream variant that runs (4, 8, 12 or 16 rank steps):
    # these are refused before anything is launched.
    fp16x2, flags = _lib.PRECISION_CODES["fp16x2"], _lib.GF_FAST | _lib.GF_STREAM
    for ksteps, max_ksteps in ((6, 6), (8, 10), (16, 4)):
        slab = _pack(16 * max_ksteps, 256)
        slab["kind"], slab["ksteps"], slab["nblocks"] = _lib.PACK_STREAM, ksteps, 8
        with pytest.raises(ConfigurationError, match="stream slabs"):
            _lib.call("rch_restore_noalloc", slab.ctypes.data, 1, address, 1, address, 1, address, 1, 256, 128,
                      _lib.SRC_U8, _lib.DT_BF16, fp16x2, max_ksteps, flags, stream)
    with pytest.raises(ConfigurationError, match="stream slabs"):  # fragments in a stream group
        _lib.call("rch_restore_noalloc", _pack(64, 256).ctypes.data, 1, address, 1, address, 1, address, 1, 256,
                  128, _lib.SRC_U8, _lib.DT_BF16, fp16x2, 4, flags, stream)
    torch.cuda.synchronize(device)
