"""GPU tests of the fitting facade (``reelcache_amd.gpu_fitting``) against the FP64 oracle.

Mirrors the reference's GramBasesTests / GPUFitterBatchedContractTests
(tests/test_gpu_fitting_batched.py:24-62, :97-241): Gram bases span the SVD subspace in
descending energy, the stored basis is canonical-signed FP16, prefit bases are consumed by the
matching ``fit``, and the projection / residual follow the stored basis.
"""

import numpy as np
import pytest
import torch

from oracle import fit as of
from reelcache_amd import gpu_fitting as gf
from reelcache_amd.errors import StateError, UnsupportedError
from reelcache_amd.types import MatrixKey, ModelIdentity, TensorContext

pytestmark = pytest.mark.gpu


def _spectrum(seed, rows, channels):
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(of.decaying_spectrum(rng, rows, channels)).to(torch.bfloat16)
    return x, x.float().numpy()


def _subspace_gap(rows, reference):
    a = np.asarray(rows, dtype=np.float64)
    return float(np.abs(a.T @ a - reference.T @ reference).max())


def test_gram_bases_span_the_svd_subspace(device):
    sources, hosts = zip(*[_spectrum(20 + i, 1000 + 100 * i, 256) for i in range(3)])
    ranks = [8, 3, 12]
    bases = gf.gram_bases([x.to(device) for x in sources], ranks)
    for basis, host, rank in zip(bases, hosts, ranks):
        assert basis.dtype == torch.float32 and tuple(basis.shape) == (rank, 256)
        _, reference = of.gram_bases(host, rank)
        assert _subspace_gap(basis.cpu().numpy(), reference) < 1e-3
        np.testing.assert_allclose(basis.cpu().numpy() @ basis.cpu().numpy().T, np.eye(rank), atol=1e-5)
        # Descending energy: the Rayleigh quotients of the rows decrease.
        energies = np.square(host.astype(np.float64) @ basis.cpu().numpy().T.astype(np.float64)).sum(0)
        assert np.all(np.diff(energies) <= 1e-9 * energies[0])


def test_select_eigh_solver_on_rocm(device):
    label, solver = gf.select_eigh_solver("auto")
    assert label == "torch_linalg_eigh_batched_rocsolver" and isinstance(solver, gf.BoundedEigh)
    with pytest.raises(UnsupportedError):
        gf.select_eigh_solver("cusolver_ctypes")
    grams = torch.randn(3, 40, 40, device=device)
    grams = grams @ grams.transpose(1, 2)
    values, rows = solver(grams)
    np.testing.assert_allclose((rows @ grams @ rows.transpose(1, 2)).diagonal(dim1=1, dim2=2).cpu().numpy(),
                               values.cpu().numpy(), rtol=1e-4, atol=1e-3)
    assert solver.last["reason"] == "whole_batch"


def _context(layer, target, tokens, channels):
    model = ModelIdentity("synthetic", "f" * 64, 4, channels, "THD", "bfloat16")
    frames, height = 1, tokens
    return TensorContext(model, MatrixKey(layer, target), 0, frames, height, 1,
                         "pre_rope" if target == "K" else "none")


def test_gpu_fitter_prefit_and_fit(device):
    uuid = str(torch.cuda.get_device_properties(device).uuid)
    uuid = uuid if uuid.startswith("GPU-") else "GPU-" + uuid
    fitter = gf.GPUFitter(gpu_id=device.index or 0, gpu_uuid=uuid, method="gram_batched")
    items = {}
    hosts = {}
    for layer, target, rank in ((0, "K", 16), (0, "V", 8), (1, "K", 32)):
        x, host = _spectrum(30 + layer, 700, 128)
        context = _context(layer, target, 700, 128)
        items[(layer, target)] = (x, context, rank)
        hosts[(layer, target)] = host
    fitter.prefit(items)
    assert fitter.prefit_stats["matrices"] == 3 and fitter.prefit_stats["solver"].startswith("torch_linalg_eigh")
    for key, (x, context, rank) in items.items():
        factors = fitter.fit(x, context, rank)
        assert factors.metrics["prefit_batched"] is True
        basis = factors.basis.numpy()
        assert basis.dtype == np.float16 and basis.shape == (rank, 128)
        np.testing.assert_array_equal(of.canonical_signs(basis), basis)
        _, reference = of.gram_bases(hosts[key], rank)
        assert _subspace_gap(basis, reference) < 2e-3
        expected = of.project(hosts[key], basis)
        assert (factors.coefficients.numpy() == expected).mean() >= 0.999
        scale, source, error = of.energies(hosts[key], basis, factors.coefficients.numpy())
        assert factors.metrics["projection_relative_residual"] == pytest.approx(np.sqrt(error / source), rel=1e-9)
    assert fitter.prefit_stats["hits"] == 3
    # A fit without a prefit basis solves its own Gram.
    x, context, rank = items[(0, "K")]
    assert fitter.fit(x, context, rank).metrics["factorization_method"] == "fp32_gram_eigh"
    assert fitter.prefit_stats["misses"] == 1


def test_gpu_fitter_owner_thread(device):
    import threading

    uuid = str(torch.cuda.get_device_properties(device).uuid)
    uuid = uuid if uuid.startswith("GPU-") else "GPU-" + uuid
    fitter = gf.GPUFitter(gpu_id=device.index or 0, gpu_uuid=uuid, method="gram_batched")
    x, _ = _spectrum(40, 64, 64)
    context = _context(0, "V", 64, 64)
    outcome = []

    def other_thread():
        try:
            fitter.fit(x, context, 4)
            outcome.append("fitted")
        except StateError:
            outcome.append("refused")

    thread = threading.Thread(target=other_thread)
    thread.start()
    thread.join()
    assert outcome == ["refused"]
    fitter.adopt_current_thread()
    assert fitter.fit(x.to(device), context, 4).rank == 4


def _causvid_chunk(rng):
    """The BASELINE configs[2] chunk: 60 matrices [4680, 1536] bf16, six decaying spectra
    (sigma_i = i^-p, p = 0.8 .. 1.8, plus noise) used by ten row-permuted, row-sign-flipped copies
    each (the same Gram up to summation order, so the same crossing)."""
    from reelcache_amd.types import TensorContext as Context

    model = ModelIdentity("synthetic", "f" * 64, 30, 1536, "THD", "bfloat16")
    sources, contexts, family, hosts = {}, {}, {}, []
    for index, exponent in enumerate((0.8, 1.0, 1.2, 1.4, 1.6, 1.8)):
        sigma = np.arange(1, 1537, dtype=np.float64) ** -exponent
        u, _ = np.linalg.qr(rng.standard_normal((4680, 1536)))
        v, _ = np.linalg.qr(rng.standard_normal((1536, 1536)))
        x = (u * sigma) @ v.T + rng.standard_normal((4680, 1536)) * (1e-3 * sigma[0] / np.sqrt(4680))
        base = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
        hosts.append(base.float().numpy())
        for copy in range(10):
            number = index * 10 + copy
            key = MatrixKey(number // 2, "K" if number % 2 == 0 else "V")
            order = torch.from_numpy(rng.permutation(4680))
            signs = torch.from_numpy(rng.choice(np.array([-1.0, 1.0], dtype=np.float32), 4680)).to(torch.bfloat16)
            sources[key] = base[order] * signs[:, None] if copy else base
            contexts[key] = Context(model, key, 0, 3, 30, 52, "pre_rope" if key.target == "K" else "none")
            family[key] = index
    return sources, contexts, family, hosts


def test_gpu_fitter_plan_chunk_from_two_threads(device):
    """``GPUFitter.plan_chunk`` (reelcache/gpu_fitting.py:499-522, the entry point of the reference's
    LineageCommitJob.plan, lineage_commit.py:552) on the 60-matrix CausVid chunk: a ``shared=True``
    fitter planned from two worker threads at once (the calls serialize on the fitter's lock and run
    on its private stream); every matrix's observed rank is the oracle's FP64 crossing and its stored
    energy is within 1e-9 of the oracle's measurement of the returned FP16 rows.  An unshared
    fitter refuses a call from another thread."""
    import threading

    from reelcache_amd import rank_method as rm
    from reelcache_amd.types import CodecSpec, energy_targets

    rng = np.random.default_rng(62)
    sources, contexts, family, hosts = _causvid_chunk(rng)
    on_device = {key: tensor.to(device) for key, tensor in sources.items()}
    bindings = {key: rm.ActiveBasisBinding() for key in sources}
    parents = {key: None for key in sources}
    source_ids = {key: f"s{key.layer}{key.target}" for key in sources}
    config = rm.RankMethodConfig(energy_targets("causvid"), CodecSpec("svd_hevc", 1))
    uuid = str(torch.cuda.get_device_properties(device).uuid)
    uuid = uuid if uuid.startswith("GPU-") else "GPU-" + uuid
    fitter = gf.GPUFitter(gpu_id=device.index or 0, gpu_uuid=uuid, method="gram_batched", shared=True)
    torch.cuda.synchronize(device)
    plans, errors = {}, []

    def worker(name):
        try:
            plans[name] = fitter.plan_chunk(config, None, on_device, contexts, bindings, parents, chunk_id="c1",
                                            source_ids=source_ids)
        except BaseException as error:  # noqa: BLE001 - reported by the main thread
            errors.append(error)

    threads = [threading.Thread(target=worker, args=(name,)) for name in ("a", "b")]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join()
    assert not errors, errors
    assert fitter.prefit_stats["solver"].startswith("torch_linalg_eigh")
    crossings = {}
    for name, plan in plans.items():
        assert plan.counters["decision_fresh"] == 60 and len(plan.plans) == 60
        for key, matrix_plan in plan.plans.items():
            host = hosts[family[key]]
            target = 0.98 if key.target == "K" else 0.95
            if (family[key], target) not in crossings:
                values, _ = of.gram_bases(host, 1)
                crossings[family[key], target] = of.crossing(values, float(np.square(host.astype(np.float64)).sum()),
                                                             target)
            assert matrix_plan.observed_rank == crossings[family[key], target]
            if family[key] * 10 == 2 * key.layer + (key.target == "V"):  # the base matrix of each spectrum
                rows = matrix_plan.new_rows.numpy()
                scale, source, error = of.energies(host, rows, of.project(host, rows))
                assert matrix_plan.decision_energy == pytest.approx(1.0 - error / source, abs=1e-9)
            assert matrix_plan.decision_energy >= target + 1e-6
    # The two threads' plans agree (same chunk, same seeds); the calls did not interleave.
    for key in sources:
        assert plans["a"].plans[key].observed_rank == plans["b"].plans[key].observed_rank
        assert plans["a"].plans[key].decision_energy == pytest.approx(plans["b"].plans[key].decision_energy,
                                                                      abs=1e-12)
    owned = gf.GPUFitter(gpu_id=device.index or 0, gpu_uuid=uuid, method="gram_batched")
    refused = []

    def other():
        try:
            owned.plan_chunk(config, None, on_device, contexts, bindings, parents, chunk_id="c1",
                             source_ids=source_ids)
        except StateError:
            refused.append(True)

    thread = threading.Thread(target=other)
    thread.start()
    thread.join()
    assert refused == [True]
