"""GPU parity of the staged comparison backend (``backend="staged"``, the reference's
``_staged_group``: reelcache/restore_kernels.py:2192-2248) against the oracle.

The HIP unpack (``rch_staged_unpack``) writes each GEMM group's dequantized, prescaled coefficients
into a dense work matrix, the BLAS library multiplies it with FP32 output, and the HIP store
(``rch_staged_store``) undoes the prescale, rotates, casts and stores.  Every output element must lie
within the oracle's ``error_bound`` for the precision (reelcache/restore_kernels.py:1208-1227), which
holds for any FP32 summation order; neighbours of the slots stay untouched.
"""

import dataclasses
import zlib

import numpy as np
import pytest
import torch

from reelcache_amd import restore_kernels as rk

from restore_cases import expected, make_case, written

pytestmark = pytest.mark.gpu

STAGED = ("fp32", "fp16", "bf16")


def _check(case, precision):
    values, bound = expected(case, precision)
    excess = np.abs(written(case) - values) - bound
    assert float(excess.max()) <= 0, f"{precision}: {int((excess > 0).sum())} elements exceed the bound"


@pytest.mark.parametrize("precision", STAGED)
@pytest.mark.parametrize("source", ["uint8", "pictures", "float32", "bfloat16"])
def test_staged_sources_layouts_and_rope(device, precision, source):
    rng = np.random.default_rng(zlib.crc32(f"staged/{precision}/{source}".encode()))
    kind = "float" if source in ("float32", "bfloat16") else source
    dtype = torch.bfloat16 if source == "bfloat16" else torch.float32
    for layout, rope, out_dtype in (("BTHD", "separable", "bfloat16"), ("THD", "dense", "float16"),
                                    ("BHTD", "none", "float32")):
        case = make_case(rng, grid=(2, 5, 13), heads=3, head_dim=32, rank=37, source=kind, rope=rope, layout=layout,
                         out_dtype=out_dtype, device=device, token_offset=4, coefficient_dtype=dtype)
        stages = []
        handle = rk.reconstruct([case.job], backend="staged", precision=precision, stage_events=stages)
        handle.synchronize()
        assert handle.stats["backend"] == "staged" and handle.stats["precision"] == precision
        assert [name for name, _ in stages if name in ("unpack", "gemm", "rope_store")] == \
            ["unpack", "gemm", "rope_store"]
        _check(case, precision)
        tensor = case.job.destination.tensor
        canonical = (tensor.transpose(1, 2) if layout == "BHTD" else tensor).reshape(-1, 96)
        assert bool((canonical[:4] == -123.0).all()) and bool((canonical[4 + 130:] == -123.0).all())


def test_staged_layer_call_groups_gemms(device):
    """One call like a layer restore: K jobs (RoPE) on one basis at two ranks, V jobs on another,
    and a dense job; the GEMM groups stack their jobs' rows, every slot within the bound."""
    rng = np.random.default_rng(91)
    heads = 4
    channels = heads * 64
    bases = [torch.from_numpy(np.linalg.qr(rng.standard_normal((channels, rows)))[0].T.copy()).half().to(device)
             for rows in (96, 128)]
    cases = []
    for rank, basis, rope in ((80, bases[0], "separable"), (80, bases[0], "separable"), (48, bases[0], "separable"),
                              (128, bases[1], "none"), (100, bases[1], "none")):
        cases.append(make_case(rng, grid=(1, 9, 17), heads=heads, head_dim=64, rank=rank, source="uint8", rope=rope,
                               device=device, basis=basis))
    dense_values = torch.from_numpy(rng.standard_normal((153, channels)).astype(np.float32)).to(device)
    dense_slot = torch.full((1, 160, heads, 64), -7.0, dtype=torch.bfloat16, device=device)
    dense = rk.ReconstructionJob(rk.DenseSource(dense_values), rk.NativeView(dense_slot, "BTHD"), (1, 9, 17))
    handle = rk.reconstruct([case.job for case in cases] + [dense], backend="staged", precision="fp16")
    handle.synchronize()
    for case in cases:
        _check(case, "fp16")
    assert torch.equal(dense_slot[0, :153].reshape(153, -1), dense_values.to(torch.bfloat16))
    assert bool((dense_slot[0, 153:] == -7.0).all())


def test_staged_fp16_device_bound(device):
    """Float coefficients without a host bound in fp16: the device bound sets the prescale."""
    rng = np.random.default_rng(17)
    for scale in (1.0, 3e4, 2e-3):
        base = make_case(rng, grid=(1, 7, 19), heads=2, head_dim=64, rank=50, source="float", rope="separable",
                         device=device, out_dtype="float32")
        values = base.job.source.values * scale
        job = base.job
        scaled = rk.ReconstructionJob(rk.CoefficientSource(values), job.destination, job.grid, job.basis, job.rank,
                                      job.rope)
        case = dataclasses.replace(base, job=scaled, coefficients=values.float().cpu().numpy())
        rk.reconstruct([case.job], backend="staged", precision="fp16").synchronize()
        _check(case, "fp16")


def test_staged_native_rope(device):
    """native_rope with the staged backend: pre-RoPE K reconstructed by the staged path, then the
    engine's rotation (here the oracle's own formula on the device)."""
    rng = np.random.default_rng(23)
    case = make_case(rng, grid=(1, 6, 11), heads=2, head_dim=64, rank=40, source="uint8", rope="separable",
                     device=device, out_dtype="float32")
    cos, sin = (torch.from_numpy(part).float().to(device) for part in case.rope)

    def rotate(values, job):
        pairs = values.float().reshape(values.shape[0], -1, 2)
        c = cos.repeat(1, values.shape[1])
        s = sin.repeat(1, values.shape[1])
        even, odd = pairs[..., 0], pairs[..., 1]
        return torch.stack((even * c - odd * s, even * s + odd * c), dim=-1).reshape(values.shape)

    handle = rk.reconstruct([case.job], backend="staged", precision="fp32", native_rope=rotate)
    handle.synchronize()
    _check(case, "fp32")


def test_staged_refuses_what_it_cannot_run(device):
    rng = np.random.default_rng(29)
    case = make_case(rng, grid=(1, 4, 8), heads=2, head_dim=32, rank=8, device=device)
    for precision in ("auto", "fp16x2", "tf32", "tf32x3"):
        with pytest.raises(rk.UnsupportedError):
            rk.reconstruct([case.job], backend="staged", precision=precision)
