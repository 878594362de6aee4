"""GPU tests of the energy-target planner (``reelcache_amd.rank_method.GramPlanner``).

Decisions are checked against the FP64 oracle on inputs built so that each branch is taken with
a wide margin (``decision_band`` 1e-6 against energy gaps >= 1e-3): fresh fits land on the
bucket grid with the oracle's crossing as observed rank; an inherited basis that still holds
the energy is shared (shortest verified prefix); a chunk with new directions is augmented with
rows orthogonal to the inherited span, or refitted when the augmented bytes exceed a fresh fit's;
zero matrices and full-width diagnostics take their own branches.  Stored energies agree with
the oracle's measurement of the returned FP16 rows to 1e-9.  Mirrors the reference's
SketchTests / FreshFitTests / ReuseTests (tests/test_step4_rank_method.py:80-318).
"""

import numpy as np
import pytest
import torch

from oracle import fit as of
from oracle import quantize as oq
from reelcache_amd import fit_kernels as fk
from reelcache_amd import node_packets as npk
from reelcache_amd import rank_method as rm
from reelcache_amd.types import CodecSpec, EnergyTargets, MatrixKey, ModelIdentity, TensorContext, energy_targets

pytestmark = pytest.mark.gpu

PARENT = "manifest:" + "a" * 64
GROUP = "b" * 64


def _model(channels, layers=4):
    return ModelIdentity("synthetic", "f" * 64, layers, channels, "THD", "bfloat16")


def _context(model, key, frames, height, width):
    return TensorContext(model, key, 0, frames, height, width, "pre_rope" if key.target == "K" else "none")


def _stored_energy(host, rows16):
    scale, source, error = of.energies(host, rows16, of.project(host, rows16))
    return 1.0 if scale == 0 else 1.0 - error / source


def _spectrum(rng, rows, channels, sigma, v=None, noise=1e-3):
    u, _ = np.linalg.qr(rng.standard_normal((rows, channels)))
    if v is None:
        v, _ = np.linalg.qr(rng.standard_normal((channels, channels)))
    x = (u * sigma) @ v.T + rng.standard_normal((rows, channels)) * (noise * sigma[0] / np.sqrt(rows))
    tensor = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    return tensor, tensor.float().numpy(), v


def _plan(config, device, sources, contexts, parents=None, bindings=None):
    keys = list(sources)
    parents = parents or {key: None for key in keys}
    bindings = bindings or {key: rm.ActiveBasisBinding() for key in keys}
    planner = rm.GramPlanner(config, device=device)
    return planner.plan({k: sources[k].to(device) for k in keys}, contexts, bindings, parents, chunk_id="c1",
                        source_ids={k: f"s{k.layer}{k.target}" for k in keys})


def _config(targets=None, **kwargs):
    return rm.RankMethodConfig(targets or energy_targets("causvid"), CodecSpec("svd_hevc", 1), **kwargs)


@pytest.mark.parametrize("solver", ["topk_rr", "gram_eigh"])
def test_fresh_chunk_at_causvid_shape(device, solver):
    rng = np.random.default_rng(50)
    model = _model(1536)
    sigma = np.arange(1, 1537, dtype=np.float64) ** -1.2
    sources, hosts, contexts = {}, {}, {}
    for layer, target in ((0, "K"), (0, "V"), (1, "K"), (1, "V")):
        key = MatrixKey(layer, target)
        sources[key], hosts[key], _ = _spectrum(rng, 4680, 1536, sigma)
        contexts[key] = _context(model, key, 3, 30, 52)
    plan = _plan(_config(solver=solver), device, sources, contexts)
    assert plan.counters["decision_fresh"] == 4 and plan.eigh_solver
    for key, matrix_plan in plan.plans.items():
        host = hosts[key]
        target = 0.98 if key.target == "K" else 0.95
        values, _ = of.gram_bases(host, 1)
        assert matrix_plan.observed_rank == of.crossing(values, float(np.square(host.astype(np.float64)).sum()), target)
        assert matrix_plan.rank_view == matrix_plan.bucket_rank == 32
        rows = matrix_plan.new_rows.numpy()
        assert rows.dtype == np.float16 and rows.shape == (32, 1536)
        np.testing.assert_array_equal(of.canonical_signs(rows), rows)
        assert matrix_plan.decision_energy == pytest.approx(_stored_energy(host, rows), abs=1e-9)
        assert matrix_plan.decision_energy >= target + 1e-6
    # The chunk's codes: projection onto the planned rows, then the device quantizer == oracle.
    key = MatrixKey(0, "K")
    rows = plan.plans[key].new_rows.to(device)
    (p,), keys = fk.project([sources[key].to(device)], [rows], [32], extrema=True)
    codes, affine, _ = npk.quantize_with_extrema(p, keys[0].cpu().numpy(), CodecSpec("svd_hevc", 32))
    o_codes, o_affine, _ = oq.quantize(of.project(hosts[key], rows.cpu().numpy()), "per_channel")
    np.testing.assert_array_equal(affine, o_affine)
    np.testing.assert_array_equal(codes.cpu().numpy(), o_codes)


def _parent_rows(host, count):
    _, rows = of.gram_bases(host, count)
    return torch.from_numpy(of.stored_basis(rows))


def test_share_shortest_verified_prefix(device):
    rng = np.random.default_rng(51)
    model = _model(256)
    sigma = np.arange(1, 257, dtype=np.float64) ** -1.2
    key = MatrixKey(0, "K")
    first, first_host, v = _spectrum(rng, 1000, 256, sigma)
    second, second_host, _ = _spectrum(rng, 1000, 256, sigma, v=v)
    parent = _parent_rows(first_host, 64)
    binding = rm.ActiveBasisBinding(PARENT, 64, GROUP, 64, "c0")
    plan = _plan(_config(), device, {key: second}, {key: _context(model, key, 1, 1000, 1)}, {key: parent},
                 {key: binding}).plans[key]
    assert plan.decision == "share" and plan.new_rows is None and plan.parent_version_ref == PARENT
    assert plan.rank_view == 32
    assert plan.decision_energy == pytest.approx(_stored_energy(second_host, parent[:32].numpy()), abs=1e-9)
    assert plan.decision_energy >= 0.98 + 1e-6


def _boosted(rng, v, sigma):
    boosted = sigma.copy()
    boosted[40:48] = 0.3  # eight directions outside the inherited top-32 span carry new energy
    return _spectrum(rng, 1000, 256, boosted, v=v)


@pytest.mark.parametrize("solver", ["topk_rr", "gram_eigh"])
@pytest.mark.parametrize("fresh_rank,decision", [(None, "augment"), (32, "refit")])
def test_augment_or_refit(device, fresh_rank, decision, solver):
    rng = np.random.default_rng(52)
    model = _model(256)
    sigma = np.arange(1, 257, dtype=np.float64) ** -1.2
    key = MatrixKey(1, "V")
    _, first_host, v = _spectrum(rng, 1000, 256, sigma)
    second, second_host, _ = _boosted(rng, v, sigma)
    parent = _parent_rows(first_host, 32)
    assert _stored_energy(second_host, parent.numpy()) < 0.9  # certification fails by a wide margin
    binding = rm.ActiveBasisBinding(PARENT, 32, GROUP, fresh_rank, None if fresh_rank is None else "c0")
    config = _config(EnergyTargets("t", 0.98, 0.98, False), solver=solver)
    plan = _plan(config, device, {key: second}, {key: _context(model, key, 1, 1000, 1)}, {key: parent},
                 {key: binding}).plans[key]
    assert plan.decision == decision
    rows = plan.new_rows.numpy()
    if decision == "augment":
        assert plan.reason == "residual_fit_appended" and plan.estimate["reason"] == "no_fresh_rank_estimate"
        assert plan.rank_view == 32 + rows.shape[0] and rows.shape[0] % 32 == 0
        overlap = np.abs(parent.numpy().astype(np.float64) @ rows.astype(np.float64).T).max()
        assert overlap < 5e-3  # orthogonal to the inherited span up to FP16 rounding
        stored = np.concatenate((parent.numpy(), rows))
    else:
        assert plan.reason == "augmented_bytes_exceed_fresh" and plan.parent_version_ref is None
        stored = rows
    assert plan.decision_energy == pytest.approx(_stored_energy(second_host, stored), abs=1e-9)
    assert plan.decision_energy >= 0.98 + 1e-6


def test_zero_and_diagnostic_branches(device):
    model = _model(64)
    zero_key, diag_key = MatrixKey(0, "K"), MatrixKey(0, "V")
    rng = np.random.default_rng(53)
    sources = {zero_key: torch.zeros((96, 64), dtype=torch.bfloat16),
               diag_key: _spectrum(rng, 96, 64, np.arange(1, 65, dtype=np.float64) ** -1.0)[0]}
    contexts = {key: _context(model, key, 1, 96, 1) for key in sources}
    plan = _plan(_config(EnergyTargets("d", 0.98, 1.0, False)), device, sources, contexts).plans
    assert plan[zero_key].decision == "zero_input" and plan[zero_key].zero_input
    assert plan[zero_key].new_rows.tolist()[0][:2] == [1.0, 0.0]
    assert plan[diag_key].decision == "diagnostic_full_width" and plan[diag_key].rank_view == 64


def test_topk_directions_match_the_full_eigendecomposition(device):
    """Top-k Rayleigh-Ritz (k = bucket + margin) against the full Gram eigh of the same matrices:
    the leading Ritz values and subspaces agree, and the extender doubles the set up to the
    exact full decomposition."""
    rng = np.random.default_rng(54)
    sigma = np.arange(1, 513, dtype=np.float64) ** -1.2
    sources = [_spectrum(rng, 2000, 512, sigma)[0].to(device) for _ in range(3)]
    totals = [float(x.double().square().sum()) for x in sources]
    seeds = [11, 12, 13]
    topk = rm.topk_directions(sources, totals, [32] * 3, [None] * 3, seeds, margin=64, steps=3, align=32)
    full = rm.gram_directions(sources, totals)
    for fast, exact in zip(topk, full):
        assert fast.width == 96 and not fast.complete and exact.complete
        top = slice(0, 16)
        np.testing.assert_allclose(fast.energies[top].cpu().numpy(), exact.energies[top].cpu().numpy(), rtol=1e-4)
        a = fast.rows[:16].double().cpu().numpy()
        b = exact.rows[:16].double().cpu().numpy()
        assert np.abs(a.T @ a - b.T @ b).max() < 1e-3
        assert fast.crossing(0.9) == exact.crossing(0.9)
    wider = topk[0].extender(topk[0], 32)
    assert wider.width == 192 and not wider.complete
    widest = wider.extender(wider, 32)
    assert widest.width == 384
    assert widest.extender(widest, 32).complete  # k reaches C: the full eigendecomposition


def test_sixty_matrix_chunk_matches_the_oracle_per_matrix(device):
    """The BASELINE configs[2] batch: one chunk of 60 matrices [4680, 1536] planned in one
    batched call (the launch the bench times).  Six spectra (decay exponents 0.8 .. 1.8), each
    used by ten matrices that are row permutations with random row signs of one base matrix
    (the same Gram up to summation order, so the same crossing, rows and energies): every
    matrix's observed rank is the oracle's FP64 crossing of its spectrum, and its stored energy
    is within 1e-9 of the oracle's measurement of the returned rows on the base matrix; the
    copies' leading rows agree to fp16 rounding (no cross-talk between batch members)."""
    rng = np.random.default_rng(61)
    model = _model(1536, layers=30)
    exponents = (0.8, 1.0, 1.2, 1.4, 1.6, 1.8)
    sources, hosts, contexts, family = {}, {}, {}, {}
    for index, exponent in enumerate(exponents):
        sigma = np.arange(1, 1537, dtype=np.float64) ** -exponent
        base, host, _ = _spectrum(rng, 4680, 1536, sigma)
        hosts[index] = host
        for copy in range(10):
            number = index * 10 + copy
            key = MatrixKey(number // 2, "K" if number % 2 == 0 else "V")
            order = torch.from_numpy(rng.permutation(4680))
            signs = torch.from_numpy(rng.choice(np.array([-1.0, 1.0], dtype=np.float32), 4680)).to(torch.bfloat16)
            sources[key] = base[order] * signs[:, None] if copy else base
            contexts[key] = _context(model, key, 3, 30, 52)
            family[key] = index
    assert len(sources) == 60
    plan = _plan(_config(), device, sources, contexts)
    assert plan.counters["decision_fresh"] == 60
    crossings, first = {}, {}
    for key, matrix_plan in plan.plans.items():
        index = family[key]
        host = hosts[index]
        target = 0.98 if key.target == "K" else 0.95
        if (index, target) not in crossings:
            values, _ = of.gram_bases(host, 1)
            crossings[index, target] = of.crossing(values, float(np.square(host.astype(np.float64)).sum()), target)
        assert matrix_plan.observed_rank == crossings[index, target]
        rows = matrix_plan.new_rows.numpy()
        # Signs are made canonical on the FP32 rows before the FP16 rounding (as the reference
        # does, factorization.py:437-441 then .to(float16)): after rounding, a row's largest
        # magnitude can be a tie, and then one of the tied entries is positive.
        magnitude = np.abs(rows.astype(np.float32))
        pivots = np.where(magnitude == magnitude.max(axis=1, keepdims=True), rows.astype(np.float32), -np.inf)
        assert (pivots.max(axis=1) > 0).all()
        assert matrix_plan.decision_energy == pytest.approx(_stored_energy(host, rows), abs=1e-9)
        assert matrix_plan.decision_energy >= target + 1e-6
        reference = first.setdefault((index, target), rows)
        assert rows.shape == reference.shape
        # The leading directions (well-separated eigenvalues: sigma_i^2 ratios >= 1.3 up to i = 4)
        # agree between copies up to the sign of rows whose pivot is a tie; the tail's nearly
        # degenerate eigenvectors are only fixed as a span, which the energies above pin.
        lead, head = rows[:4].astype(np.float32), reference[:4].astype(np.float32)
        np.testing.assert_allclose(lead * np.sign((lead * head).sum(axis=1))[:, None], head, atol=2e-3)
