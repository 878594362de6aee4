"""CPU tests of the staged comparison backend's host side (reelcache/restore_kernels.py:2153-2248).

* The staged GEMM asks the BLAS library for an FP32 product exactly once and never retries with a
  16-bit output: a Torch that rejects ``out_dtype`` gives :class:`UnsupportedError` chained to the
  original error; any other error propagates unchanged (the reference's ``StagedGemmTests``,
  tests/test_restore_kernels.py:553-596).
* The precision check refuses what the process-wide torch settings forbid, before any work.
* The planner's GEMM groups: jobs sharing a basis view and rank stack their coefficient rows into
  one work matrix in job order (reelcache/restore_kernels.py:2198-2213).
"""

from unittest import mock

import numpy as np
import pytest
import torch

from reelcache_amd import restore_kernels as rk
from reelcache_amd import restore_plan as rp
from reelcache_amd.errors import UnsupportedError
from reelcache_amd.restore_plan import job_desc
from restore_cases import make_case, orthonormal_basis

COEFFICIENTS = torch.randn(6, 4, generator=torch.Generator().manual_seed(1)).half()
BASIS = torch.randn(4, 8, generator=torch.Generator().manual_seed(2)).half()


def _run_with(behaviour, precision="fp16"):
    calls = []

    def fake_mm(*args, **kwargs):
        calls.append(kwargs)
        return behaviour(*args, **kwargs)

    with mock.patch.object(torch, "mm", fake_mm):
        try:
            return rk._staged_gemm(COEFFICIENTS, BASIS, precision), calls
        except Exception as error:  # noqa: BLE001 - inspected by the caller
            return error, calls


def test_staged_gemm_requests_fp32_output_once():
    for precision in ("fp16", "bf16"):
        result, calls = _run_with(lambda a, b, out_dtype=None: (a.double() @ b.double()).to(out_dtype), precision)
        assert calls == [{"out_dtype": torch.float32}]
        assert result.dtype == torch.float32
    result, calls = _run_with(lambda a, b: a @ b, "fp32")  # FP32 operands: a plain product
    assert calls == [{}]


def test_staged_gemm_never_retries_with_a_16_bit_output():
    def raiser(error):
        def behaviour(*args, **kwargs):
            raise error
        return behaviour

    for error in (TypeError("mm() got an unexpected keyword argument 'out_dtype'"),
                  NotImplementedError("Could not run 'aten::mm.dtype'")):
        result, calls = _run_with(raiser(error))
        assert isinstance(result, UnsupportedError) and result.__cause__ is error
        assert "out_dtype=torch.float32" in str(result) and len(calls) == 1
    out_of_memory = RuntimeError("HIP out of memory")
    result, calls = _run_with(raiser(out_of_memory))
    assert result is out_of_memory and len(calls) == 1


def test_staged_precision_follows_process_settings():
    for precision in ("fp16x2", "tf32x3"):
        with pytest.raises(UnsupportedError, match="supports fp32, tf32, fp16 and bf16"):
            rk._check_staged_precision(precision)
    with pytest.raises(UnsupportedError, match="no TF32"):
        rk._check_staged_precision("tf32")
    rk._check_staged_precision("bf16")
    matmul = torch.backends.cuda.matmul
    if hasattr(matmul, "allow_fp16_accumulation"):
        saved = matmul.allow_fp16_accumulation
        try:
            matmul.allow_fp16_accumulation = True
            with pytest.raises(UnsupportedError, match="FP16 accumulation"):
                rk._check_staged_precision("fp16")
        finally:
            matmul.allow_fp16_accumulation = saved
    rk._check_staged_precision("fp16")
    saved = rk.fp32_matmul_precision("cuda")
    if saved == "ieee":
        rk._check_staged_precision("fp32")
    try:
        if hasattr(matmul, "fp32_precision"):
            matmul.fp32_precision = "tf32"
        else:
            torch.set_float32_matmul_precision("high")
        with pytest.raises(UnsupportedError, match="ieee"):
            rk._check_staged_precision("fp32")
    finally:
        if hasattr(matmul, "fp32_precision"):
            matmul.fp32_precision = saved if saved != "ieee" else "ieee"
        else:
            torch.set_float32_matmul_precision("highest")
    assert rk.fp32_matmul_precision("cuda") == saved


def test_staged_layout_stacks_gemm_groups_in_job_order(monkeypatch):
    monkeypatch.setattr(rp, "_compute_units", lambda device: 256)
    monkeypatch.setattr(rp, "_occupancy", lambda *args: 2)
    rng = np.random.default_rng(11)
    heads = 2
    first = orthonormal_basis(64, heads * 32, rng)
    second = orthonormal_basis(48, heads * 32, rng)
    specs = [((1, 4, 5), 40, first), ((2, 3, 4), 40, first), ((1, 2, 7), 36, first), ((1, 5, 5), 40, second),
             ((1, 3, 3), 40, first)]
    cases = [make_case(rng, grid=grid, heads=heads, head_dim=32, rank=rank, rope="none", basis=basis)
             for grid, rank, basis in specs]
    descs = [job_desc(case.job) for case in cases]
    groups = [0, 0, 0, 3, 0]  # first job of each basis view
    layout = rp._Layout(descs, [0] * len(descs), groups, "fp16", dict(rp.DEFAULT_MERGED), "cpu", staged=True)
    assert layout.variants == ["staged"] and not len(layout.pack_rows)
    (plan,) = layout.plans
    gemms = {(tuple(g["members"]), g["rank"]): g["rows"] for g in plan["gemms"]}
    # basis `first` at rank 40: jobs 0, 1, 4 (20 + 24 + 9 rows); rank 36: job 2; basis `second`: job 3.
    assert gemms == {((0, 1, 4), 40): 53, ((2,), 36): 14, ((3,), 40): 25}
    assert layout.staged_rows.tolist() == [0, 20, 0, 0, 44]
    image = layout.template
    at = layout.staged_rows_offset
    assert image[at:at + 8 * len(descs)].view(np.int64).tolist() == [0, 20, 0, 0, 44]
    for gemm in plan["gemms"]:
        tiles = image[gemm["tiles"]:gemm["tiles"] + 8 * gemm["n_tiles"]].view(np.int32).reshape(-1, 2)
        assert sorted(set(tiles[:, 0].tolist())) == sorted(gemm["members"])
        assert all(tiles[i, 1] % rp.TILE_TOKENS == 0 for i in range(len(tiles)))
