"""CPU tests of the fit path's host logic: contract types, eigensolver sub-batching, the fitter's
validation and owner thread, the planner's byte / bucket / crossing rules, key decoding, the
packet mosaic, and that every device entry point refuses host tensors (no CPU fallback).

Mirrors the reference's host-side tests of these functions (tests/test_gpu_fitting_batched.py
:64-241 BoundedEigh / dispatch / owner thread; tests/test_step4_rank_method.py byte estimates).
"""

import hashlib
import math
import threading

import numpy as np
import pytest
import torch

from oracle import fit as of
from oracle import restore as orc
from reelcache_amd import factorization as fz
from reelcache_amd import fit_kernels as fk
from reelcache_amd import gpu_fitting as gf
from reelcache_amd import node_packets as npk
from reelcache_amd import quantize as pq
from reelcache_amd import rank_method as rm
from reelcache_amd.errors import CapacityError, ConfigurationError, StateError, UnsupportedError
from reelcache_amd.types import (CodecSpec, EnergyTargets, MatrixKey, ModelIdentity, TensorContext, canonical_digest,
                                 energy_targets)


def _context(target="K", tokens=64, channels=32, dtype="bfloat16", key_space=None):
    model = ModelIdentity("m", "f" * 64, 2, channels, "THD", dtype)
    return TensorContext(model, MatrixKey(0, target), 0, 1, tokens, 1,
                         key_space or ("pre_rope" if target == "K" else "none"))


# ---------------------------------------------------------------------------
# Contract types
# ---------------------------------------------------------------------------


def test_types_validate_and_canonicalize():
    context = _context("V", tokens=12, channels=40, dtype="bf16")
    assert context.shape == (12, 40) and context.dtype == "bfloat16"
    with pytest.raises(ConfigurationError):
        _context("V", key_space="pre_rope")
    with pytest.raises(ConfigurationError):
        ModelIdentity("m", "f", 2, {"K": 8}, "THD", "bfloat16")
    assert CodecSpec("svd", 4, "global", 0.7).protected_fraction == 0.0
    assert CodecSpec("svd", 4, "per_channel", 0.2).protected_fraction == 1.0
    with pytest.raises(ConfigurationError):
        CodecSpec("raw", 4)
    with pytest.raises(ConfigurationError):
        CodecSpec("svd", 4, inter_prediction=True)
    targets = energy_targets("causvid")
    assert (targets.for_target("K"), targets.for_target("V")) == (0.98, 0.95)
    with pytest.raises(ConfigurationError):
        energy_targets("unknown-model")
    with pytest.raises(ConfigurationError):
        EnergyTargets("p", 1.5, 0.9, False)


def test_canonical_digest_is_sha256_of_sorted_compact_json():
    value = {"b": [1, 2.5, "x"], "a": {"z": None, "y": True}}
    text = '{"a":{"y":true,"z":null},"b":[1,2.5,"x"]}'
    assert canonical_digest(value) == hashlib.sha256(text.encode()).hexdigest()
    with pytest.raises(ValueError):
        canonical_digest({"x": math.nan})


# ---------------------------------------------------------------------------
# Eigensolver selection and sub-batching (host logic, CPU solver)
# ---------------------------------------------------------------------------


def _grams(count, n, seed=0):
    a = torch.from_numpy(np.random.default_rng(seed).standard_normal((count, n, n))).float()
    return a @ a.transpose(1, 2)


def test_bounded_eigh_halves_rejected_batches():
    grams = _grams(5, 6)
    solver = gf.BoundedEigh("cpu", gf._torch_rows_eigh, workspace=lambda b, n, d: 0 if b <= 2 else None,
                            total_memory=1 << 40)
    values, rows = solver(grams)
    assert solver.last == {"batch": 5, "n": 6, "sub_batch": 2, "solver_calls": 3,
                           "reason": "solver_rejects_batch_size"}
    for index in range(5):
        expected, columns = torch.linalg.eigh(grams[index])
        torch.testing.assert_close(values[index], expected)
        torch.testing.assert_close(rows[index].abs(), columns.T.abs())


def test_bounded_eigh_fixed_sub_batch_pads_with_identities():
    grams = _grams(3, 4, seed=1)
    seen = []

    def solver(batch):
        seen.append(int(batch.shape[0]))
        return gf._torch_rows_eigh(batch)

    bounded = gf.BoundedEigh("cpu", solver, sub_batch_size=lambda n: 2)
    values, _ = bounded(grams)
    assert seen == [2, 2] and bounded.last["padded"] == 1 and bounded.last["reason"] == "fixed_sub_batch"
    torch.testing.assert_close(values[2], torch.linalg.eigh(grams[2])[0])
    assert gf.default_eigh_sub_batch(4096) == 1 and gf.default_eigh_sub_batch(1536) is None


def test_bounded_eigh_memory_bound():
    bounded = gf.BoundedEigh("cpu", gf._torch_rows_eigh, total_memory=5_000, memory_fraction=1.0)  # 8 need 6400 B
    assert bounded.sub_batch(8, 8, "cpu") == (4, "memory_bound")
    with pytest.raises(ConfigurationError):
        gf.BoundedEigh("cpu", gf._torch_rows_eigh, memory_fraction=0.0)


def test_select_eigh_solver_never_degrades_silently():
    with pytest.raises(ConfigurationError):
        gf.select_eigh_solver("bogus")
    with pytest.raises(UnsupportedError):
        gf.select_eigh_solver("cusolver_ctypes")
    assert gf.select_eigh_solver("torch_loop")[0] == "torch_eigh_loop_explicit"
    label, solver = gf.select_eigh_solver("auto")
    assert label == "torch_linalg_eigh_batched_rocsolver" and isinstance(solver, gf.BoundedEigh)
    assert not gf.torch_batched_eigh_is_xsyevbatched()


# ---------------------------------------------------------------------------
# GPUFitter contract
# ---------------------------------------------------------------------------


def test_gpu_fitter_validation():
    good = {"gpu_id": 0, "gpu_uuid": "GPU-0000"}
    for bad in ({"gpu_uuid": "0000"}, {"method": "svd"}, {"max_workspace_bytes": 0}, {"batch_size": 0},
                {"power_iterations": 9}, {"eigh_solver": "magma"}, {"side_stream": 1}):
        with pytest.raises(ConfigurationError):
            gf.GPUFitter(**{**good, **bad})
    fitter = gf.GPUFitter(**good, method="gram_batched", shared=True)
    assert fitter.side_stream and gf.GPU_FIT_METHODS[-1] == "gram_batched"


def test_gpu_fitter_owner_thread_and_budget():
    fitter = gf.GPUFitter(gpu_id=0, gpu_uuid="GPU-0000", method="gram_batched")
    x = torch.zeros((64, 32), dtype=torch.bfloat16)
    context = _context("K", 64, 32)
    outcome = []

    def other():
        try:
            fitter.fit(x, context, 4)
        except StateError:
            outcome.append("refused")

    thread = threading.Thread(target=other)
    thread.start()
    thread.join()
    assert outcome == ["refused"]
    small = gf.GPUFitter(gpu_id=0, gpu_uuid="GPU-0000", method="gram_batched", max_workspace_bytes=1000)
    with pytest.raises(CapacityError):
        small.fit(x, context, 4)
    with pytest.raises(ConfigurationError):
        fitter.fit(x, context, 40)  # rank above min(shape)
    if torch.cuda.device_count() == 0:
        with pytest.raises(UnsupportedError):
            fitter.fit(x, context, 4)


# ---------------------------------------------------------------------------
# Validation, signs and no host fallback
# ---------------------------------------------------------------------------


def test_validate_matrix_rules():
    context = _context("K", 64, 32)
    x = torch.zeros((64, 32), dtype=torch.bfloat16)
    assert fz.validate_matrix(x, context) is not None
    with pytest.raises(ConfigurationError):
        fz.validate_matrix(x.float(), context)  # dtype differs from the context
    with pytest.raises(ConfigurationError):
        fz.validate_matrix(x[:10], context)
    with pytest.raises(ConfigurationError):
        fz.validate_matrix(x, _context("K", 64, 32, key_space="post_rope"))
    bad = x.clone()
    bad[3, 3] = float("nan")
    with pytest.raises(ConfigurationError):
        fz.validate_matrix(bad, context)
    with pytest.raises(ConfigurationError):
        fz.validate_matrix(x, object())


def test_canonical_signs_match_oracle():
    rows = np.random.default_rng(3).standard_normal((9, 17)).astype(np.float32)
    rows[0, :2] = [0.5, -0.5]  # tie: the first index decides
    np.testing.assert_array_equal(fz._canonical_signs(torch.from_numpy(rows)).numpy(), of.canonical_signs(rows))


def test_device_entry_points_refuse_host_tensors():
    x = torch.zeros((64, 32), dtype=torch.bfloat16)
    q = torch.zeros((4, 32), dtype=torch.float16)
    q[:, :4] = torch.eye(4)
    for call in (lambda: fk.gram([x]), lambda: fk.absmax([x]), lambda: fk.project([x], [q], [4]),
                 lambda: fz.project_onto_basis(x, q), lambda: fz.measure_source_energy(x),
                 lambda: gf.gram_bases([x], [4]), lambda: npk.quantize_device(x.float(), CodecSpec("svd", 4))):
        with pytest.raises(UnsupportedError):
            call()


def test_order_key_decoding():
    keys = np.array([0xBF800000, 0x3FFFFFFF, 0x80000000, 0x7FFFFFFF, 0xFF800000], dtype=np.uint32)
    np.testing.assert_array_equal(fk.decode_max_keys(keys), np.array([1.0, -2.0, 0.0, -0.0, np.inf], np.float32))
    np.testing.assert_array_equal(fk.decode_min_keys(~keys), fk.decode_max_keys(keys))


# ---------------------------------------------------------------------------
# Planner rules
# ---------------------------------------------------------------------------


def _config(**kwargs):
    return rm.RankMethodConfig(energy_targets("causvid"), CodecSpec("svd_hevc", 1), **kwargs)


def test_planner_config_and_binding_rules():
    assert _config().solver_id() == "fp32_gram_topk_rr.v1:m64:s3"  # the reference's default solver
    assert _config(solver="gram_eigh").solver_id() == "fp32_gram_eigh.v1"
    assert _config(solver="warm_start").solver_id(warm=True) == "fp32_gram_warm_rr.v1:s1"
    assert _config(refit_rule="cumulative").refit_rule == "cumulative"
    with pytest.raises(ConfigurationError):
        _config(solver="power")
    with pytest.raises(ConfigurationError):
        _config(decision_band=0.1)
    with pytest.raises(ConfigurationError):
        rm.ActiveBasisBinding(version_ref="manifest:" + "a" * 64, total_rank=8, group_id="nothex")
    with pytest.raises(ConfigurationError):
        rm.ActiveBasisBinding(fresh_rank=8)
    rm.ActiveBasisBinding(version_ref="manifest:" + "a" * 64, total_rank=8, group_id="b" * 64,
                          fresh_rank=8, fresh_chunk_id="c0")


def test_estimate_bytes_terms():
    config = _config()
    context = _context("K", 4680, 1536)
    binding = rm.ActiveBasisBinding()
    estimate = rm.estimate_bytes(config, context, 64, 32, binding)
    layout = pq.normalization_layout(64, "per_channel", 1.0)
    assert estimate["estimate_type"] == "factor_byte_proxy" and estimate["coefficient_rate"] == 1.0
    assert estimate["coefficient_bytes"] == 4680 * 64
    assert estimate["basis_bytes"] == 2 * 1536 * 32
    assert estimate["scale_bytes"] == 4 * layout["affine_shape"][0] * layout["affine_shape"][1] == 512
    assert estimate["total_bytes"] == 4680 * 64 + 2 * 1536 * 32 + 512 + 4096
    measured = rm.ActiveBasisBinding(coefficient_rate=0.5, rate_identity=rm.rate_identity(context, config.spec_for(64)))
    assert rm.estimate_bytes(config, context, 64, 0, measured)["estimate_type"] == "measured_coefficient_rate"
    svd = rm.RankMethodConfig(energy_targets("causvid"), CodecSpec("svd", 1))
    assert rm.estimate_bytes(svd, context, 10, 0, binding)["coefficient_bytes"] == 4.0 * 4680 * 10


def test_refit_debt_rule():
    fresh = {"coefficient_bytes": 100.0, "scale_bytes": 0, "basis_bytes": 50, "total_bytes": 150}
    larger = {"coefficient_bytes": 120.0, "scale_bytes": 0, "basis_bytes": 10, "total_bytes": 160}
    assert rm.refit_debt_test(0.0, larger, fresh) == (True, 20.0, 40)
    assert rm.refit_debt_test(30.0, larger, fresh)[0] is True
    assert rm.refit_debt_test(10.0, larger, fresh)[0] is False


def test_bucket_prefixes_and_crossing():
    assert [rm._bucket(r, 32, 1536) for r in (1, 10, 32, 33, math.inf)] == [32, 32, 32, 64, 1536]
    assert rm._legal_prefixes(96, 32) == [32, 64, 96]
    assert rm._legal_prefixes(70, 32) == [32, 64, 70]
    rng = np.random.default_rng(4)
    energies = np.sort(rng.exponential(size=50))[::-1].copy()
    directions = rm.DirectionSet(torch.zeros(50, 3), torch.from_numpy(energies), float(energies.sum() * 1.01), True, "x")
    for fraction in (0.3, 0.9, 0.99, 0.995):
        assert directions.crossing(fraction) == of.crossing(energies, energies.sum() * 1.01, fraction)


def test_crossing_edges_and_shared_fp16_rows():
    """Crossings at the exact boundary and past the last direction; FP16 rows from the batch's shared
    conversion equal a per-set conversion, for every prefix and position."""
    energies = torch.tensor([4.0, 2.0, 1.0, 1.0], dtype=torch.float64)
    directions = rm.DirectionSet(torch.zeros(4, 3), energies, 10.0, False, "x")
    assert [directions.crossing(f) for f in (0.4, 0.41, 0.6, 0.8, 0.81, 1.0)] == [1, 2, 2, 4, None, None]
    assert rm.DirectionSet(torch.zeros(0, 3), energies[:0], 0.0, True, "x").crossing(0.5) == 0
    batch = torch.randn(3, 5, 7, generator=torch.Generator().manual_seed(3)) * 100
    half = rm._HalfRows(batch)
    for position in range(3):
        shared = rm.DirectionSet(batch[position], energies, 10.0, False, "x", half=(half, position))
        alone = rm.DirectionSet(batch[position], energies, 10.0, False, "x")
        for count in (1, 3, 5):
            assert torch.equal(shared.rows16(count), alone.rows16(count))
            assert shared.rows16(count).is_contiguous() and shared.rows16(count).dtype == torch.float16
    assert sorted(half.prefixes) == [1, 3, 5]


def test_batch_view_only_for_consecutive_slices():
    base = torch.arange(5 * 4 * 3, dtype=torch.float32).reshape(5, 4, 3)
    view = rm._batch_view([base[1], base[2], base[3]])
    assert view is not None and torch.equal(view, base[1:4]) and view.data_ptr() == base[1].data_ptr()
    sliced = rm._batch_view([base[0][:2], base[1][:2]])  # sub-blocks keep their strides
    assert sliced is not None and torch.equal(sliced, base[:2, :2])
    spaced = rm._batch_view([base[0], base[2], base[4]])  # evenly spaced blocks: a strided view
    assert spaced is not None and torch.equal(spaced, base[0::2])
    for tensors in ([base[0], base[1], base[3]], [base[2], base[1]], [base[1], base[2].clone()],
                    [base[1][:2], base[2]], [base[1], base[2].double()]):
        assert rm._batch_view(tensors) is None
    grams = [base[0], base[2], base[1]]
    assert torch.equal(rm._stack_grams(grams, [0, 2]), base[:2])
    assert torch.equal(rm._stack_grams(grams, [1, 2]), torch.stack([base[2], base[1]]))


def test_mosaic_matches_the_oracle_packer():
    rng = np.random.default_rng(5)
    for shape, fmt in (((3, 6, 8, 40), "yuv444p"), ((2, 4, 4, 100), "yuv420p"), ((1, 5, 3, 7), "yuv444p")):
        video = pq.video_layout(*shape, fmt)
        codes = rng.integers(0, 256, size=(shape[0] * shape[1] * shape[2], shape[3]), dtype=np.uint8)
        canvas, _ = orc.pack_pictures(codes, video, origin=(0, 0), pad=(0, 0), fill=0)
        np.testing.assert_array_equal(npk.mosaic_device(torch.from_numpy(codes), video).numpy(), canvas)
