"""GPU tests of the planner's anchor sketches, rank predictions, warm-start refits and cumulative
refit rule (reelcache/rank_method.py:591-631, :688-729, :1246-1280, :1370-1505).

* Sketches: orthonormal ``[C, m]`` columns whose captured energy equals the FP64 host measurement
  ``||X S||^2 / ||X||^2``, never exceeds the ideal top-m share (Eckart-Young) and, after q = 2
  power steps on a decaying spectrum, comes within 1e-3 of it; a seed fixes the sketch.
* Warm start: from the exact top directions of a matrix, the warm Rayleigh-Ritz directions
  reproduce the full eigendecomposition's leading energies; growth keeps them.
* Predictions: a fresh chunk planned against the priors records each fit's prediction and a
  FitObservation whose label is at most a bucket above the oracle's exact crossing (Ritz values
  interlace below the eigenvalues); after the registry learns them the next plan of the same
  matrices predicts closer to the labels.
* Cumulative rule: its estimates follow ``refit_debt_test`` (debt below / reaching the cost, no
  fresh rank), refits reset the debt, and ``refit_debt_on_share`` refits a shared chunk.
"""

import numpy as np
import pytest
import torch

from oracle import fit as of
from reelcache_amd import rank_method as rm
from reelcache_amd import rank_predictor as rp
from reelcache_amd.types import CodecSpec, EnergyTargets, MatrixKey, ModelIdentity, TensorContext

pytestmark = pytest.mark.gpu

PARENT = "manifest:" + "a" * 64
GROUP = "b" * 64


def _spectrum(rng, rows, channels, sigma, v=None, noise=1e-3):
    u, _ = np.linalg.qr(rng.standard_normal((rows, channels)))
    if v is None:
        v, _ = np.linalg.qr(rng.standard_normal((channels, channels)))
    x = (u * sigma) @ v.T + rng.standard_normal((rows, channels)) * (noise * sigma[0] / np.sqrt(rows))
    tensor = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    return tensor, tensor.float().numpy().astype(np.float64), v


def _stored_energy(host, rows16):
    scale, source, error = of.energies(host, rows16, of.project(host, rows16))
    return 1.0 if scale == 0 else 1.0 - error / source


def _context(model, key, rows):
    return TensorContext(model, key, 0, 1, rows, 1, "pre_rope" if key.target == "K" else "none")


def _plan(config, device, sources, contexts, parents=None, bindings=None, view=None, chunk="c1"):
    keys = list(sources)
    parents = parents or {key: None for key in keys}
    bindings = bindings or {key: rm.ActiveBasisBinding() for key in keys}
    planner = rm.GramPlanner(config, view, device=device)
    return planner.plan({k: sources[k].to(device) for k in keys}, contexts, bindings, parents, chunk_id=chunk,
                        source_ids={k: f"s{k.layer}{k.target}" for k in keys})


def _config(target=0.98, **kwargs):
    return rm.RankMethodConfig(EnergyTargets("t", target, target, False), CodecSpec("svd_hevc", 1), **kwargs)


def test_anchor_sketches_capture_the_leading_span(device):
    rng = np.random.default_rng(70)
    sigma = np.arange(1, 513, dtype=np.float64) ** -1.0
    tensors, hosts = zip(*[_spectrum(rng, 2000, 512, sigma)[:2] for _ in range(3)])
    sources = [t.to(device) for t in tensors]
    totals = [float(np.square(h).sum()) for h in hosts]
    results = rm.anchor_sketches(sources, totals, [5, 6, 7], anchor_rank=32, power_iterations=2)
    again = rm.anchor_sketches(sources, totals, [5, 6, 7], anchor_rank=32, power_iterations=2)
    for host, total, result, repeat in zip(hosts, totals, results, again):
        sketch = result["sketch"].double().cpu().numpy()
        assert sketch.shape == (512, 32) and result["width"] == 32
        np.testing.assert_allclose(sketch.T @ sketch, np.eye(32), atol=1e-5)
        measured = float(np.square(host @ sketch).sum()) / total
        assert result["captured_energy"] == pytest.approx(measured, abs=1e-6)
        values = np.linalg.eigvalsh(host.T @ host)[::-1]
        ideal = float(values[:32].sum()) / total
        assert measured <= ideal + 1e-9 and result["captured_energy"] > ideal - 1e-3
        assert torch.equal(repeat["sketch"], result["sketch"])
    # The captured share does not depend on the scale the energies are quoted on.
    (scaled,) = rm.anchor_sketches([sources[0]], [totals[0] / 4.0], [5], anchor_rank=32, power_iterations=2,
                                   scales=[2.0])
    assert scaled["captured_energy"] == pytest.approx(results[0]["captured_energy"], rel=1e-9)


def test_warm_start_directions_reproduce_the_leading_eigenpairs(device):
    rng = np.random.default_rng(71)
    sigma = np.arange(1, 257, dtype=np.float64) ** -1.1
    tensor, host, _ = _spectrum(rng, 1500, 256, sigma)
    source = tensor.to(device)
    total = float(np.square(host).sum())
    values, rows = of.gram_bases(host, 64)
    parent = torch.from_numpy(of.stored_basis(rows))
    warm = rm.warm_start_directions(source, total, parent, steps=1, pad=32, seed=9)
    assert warm.width == 96 and not warm.complete and warm.solver == "fp32_gram_warm_rr.v1"
    exact = np.linalg.eigvalsh(host.T @ host)[::-1]
    np.testing.assert_allclose(warm.energies[:32].numpy(), exact[:32], rtol=1e-4)
    gram_rows = warm.rows.double().cpu().numpy()
    np.testing.assert_allclose(gram_rows @ gram_rows.T, np.eye(96), atol=1e-4)
    grown = warm.extender(warm, 32)
    assert grown.width == 128
    np.testing.assert_allclose(grown.energies[:32].numpy(), exact[:32], rtol=1e-4)
    assert grown.crossing(0.9) == warm.crossing(0.9)


def test_predictions_observations_and_learning(device):
    rng = np.random.default_rng(72)
    model = ModelIdentity("predict-test", "9" * 64, 2, 512, "THD", "bfloat16")
    sigma = np.arange(1, 513, dtype=np.float64) ** -0.7
    sources, hosts, contexts = {}, {}, {}
    for layer, target in ((0, "K"), (0, "V"), (1, "K"), (1, "V")):
        key = MatrixKey(layer, target)
        sources[key], hosts[key], _ = _spectrum(rng, 2000, 512, sigma)
        contexts[key] = _context(model, key, 2000)
    config = _config(0.98)
    registry = rp.RankPredictorRegistry("predict-test", anchor_rank=config.anchor_rank)
    first = _plan(config, device, sources, contexts, view=registry.pin())
    assert first.pinned_sequence == 0
    observations = []
    for key, plan in first.plans.items():
        host = hosts[key]
        label = of.crossing(np.linalg.eigvalsh(host.T @ host)[::-1], float(np.square(host).sum()), 0.98)
        # Ritz energies interlace below the exact ones, so a top-k label is at or above the exact
        # crossing (within a bucket here).
        assert plan.decision == "fresh" and 32 < label <= plan.observed_rank <= label + 32
        assert plan.bucket_rank >= label
        (prediction,) = plan.predictions
        assert prediction["kind"] in ("log_linear", "log_linear_clamped") and prediction["x"] > 0
        assert prediction["initial_width"] % 32 == 0 and 0 <= prediction["anchor_energy"] < 0.98
        (observation,) = plan.observations
        assert observation.observed_rank == plan.observed_rank and observation.key.regime == "fresh"
        assert observation.key == config.predictor_key(contexts[key], "fresh")
        assert plan.decision_energy == pytest.approx(_stored_energy(host, plan.new_rows.numpy()), abs=1e-9)
        assert plan.decision_energy >= 0.98 + 1e-6
        observations.append(observation)
    assert registry.observe(observations) == (True,) * 4
    assert registry.observe(observations) == (False,) * 4  # a retried report is a no-op
    second = _plan(config, device, sources, contexts, view=registry.pin(), chunk="c2")
    assert second.pinned_sequence == 4
    for key in sources:
        before, after = first.plans[key], second.plans[key]
        assert abs(after.bucket_rank - before.bucket_rank) <= 32
        label = before.observed_rank
        assert (abs(after.predictions[0]["predicted_rank"] - label)
                < abs(before.predictions[0]["predicted_rank"] - label))
        assert after.predictions[0]["predictor"]["state"]["revision"] >= 1


def _boosted(rng, v, sigma):
    boosted = sigma.copy()
    boosted[40:48] = 0.3  # eight directions outside the inherited top-32 span carry new energy
    return _spectrum(rng, 1000, 256, boosted, v=v)


def _inherit_case(seed):
    rng = np.random.default_rng(seed)
    model = ModelIdentity("refit-test", "8" * 64, 2, 256, "THD", "bfloat16")
    sigma = np.arange(1, 257, dtype=np.float64) ** -1.2
    key = MatrixKey(1, "V")
    _, first_host, v = _spectrum(rng, 1000, 256, sigma)
    second, second_host, _ = _boosted(rng, v, sigma)
    _, rows = of.gram_bases(first_host, 32)
    parent = torch.from_numpy(of.stored_basis(rows))
    return key, model, second, second_host, parent


@pytest.mark.parametrize("fresh_rank,debt", [(None, 0.0), (64, 0.0), (64, 100.0), (64, 1e7), (32, 0.0)])
def test_cumulative_rule_follows_the_debt_test(device, fresh_rank, debt):
    key, model, second, host, parent = _inherit_case(73)
    binding = rm.ActiveBasisBinding(PARENT, 32, GROUP, fresh_rank, None if fresh_rank is None else "c0",
                                    refit_debt=debt)
    config = _config(0.98, refit_rule="cumulative")
    plan = _plan(config, device, {key: second}, {key: _context(model, key, 1000)}, {key: parent},
                 {key: binding}).plans[key]
    estimate = plan.estimate
    assert estimate["schema"] == "reelcache.refit_estimate.v2" and estimate["rule"] == "cumulative"
    assert estimate["debt_before"] == debt
    if fresh_rank is None:
        assert plan.decision == "augment" and estimate["reason"] == "no_fresh_rank_estimate"
        assert plan.refit_debt == debt
    else:
        refit, excess, cost = rm.refit_debt_test(debt, estimate["augmented"], estimate["fresh"])
        assert (estimate["excess"], estimate["cost"]) == (excess, cost)
        assert plan.decision == ("refit" if refit else "augment")
        expected_reason = (("refit_debt_reaches_cost" if refit else "refit_debt_below_cost") if debt > 0
                           else ("augmented_bytes_exceed_fresh" if refit else "augmented_bytes_within_fresh"))
        assert plan.reason == expected_reason if refit else estimate["reason"] == expected_reason
        assert plan.refit_debt == (0.0 if refit else debt + max(0.0, excess))
    stored = plan.new_rows.numpy() if plan.decision == "refit" else np.concatenate((parent.numpy(), plan.new_rows))
    assert plan.decision_energy == pytest.approx(_stored_energy(host, stored), abs=1e-9)
    assert plan.decision_energy >= 0.98 + 1e-6
    if debt == 1e7:
        assert plan.decision == "refit"  # a large debt always refits


def test_debt_on_share_refits_a_shared_chunk(device):
    rng = np.random.default_rng(74)
    model = ModelIdentity("share-test", "7" * 64, 2, 256, "THD", "bfloat16")
    sigma = np.arange(1, 257, dtype=np.float64) ** -1.2
    key = MatrixKey(0, "K")
    _, first_host, v = _spectrum(rng, 1000, 256, sigma)
    second, second_host, _ = _spectrum(rng, 1000, 256, sigma, v=v)
    _, rows = of.gram_bases(first_host, 64)
    parent = torch.from_numpy(of.stored_basis(rows))
    config = _config(0.98, refit_rule="cumulative", refit_debt_on_share=True)
    contexts = {key: _context(model, key, 1000)}
    low = rm.ActiveBasisBinding(PARENT, 64, GROUP, 32, "c0", refit_debt=1.0)
    plan = _plan(config, device, {key: second}, contexts, {key: parent}, {key: low}).plans[key]
    assert plan.decision == "share" and plan.estimate["decision"] == "share"
    assert plan.refit_debt == pytest.approx(1.0 + max(0.0, plan.estimate["excess"]))
    high = rm.ActiveBasisBinding(PARENT, 64, GROUP, 32, "c0", refit_debt=1e9)
    plan = _plan(config, device, {key: second}, contexts, {key: parent}, {key: high}).plans[key]
    assert plan.decision == "refit" and plan.reason == "refit_debt_reaches_cost" and plan.refit_debt == 0.0
    assert plan.decision_energy == pytest.approx(_stored_energy(second_host, plan.new_rows.numpy()), abs=1e-9)
    assert plan.decision_energy >= 0.98 + 1e-6


@pytest.mark.parametrize("solver", ["warm_start", "topk_rr"])
def test_refit_from_the_parent_basis(device, solver):
    key, model, second, host, parent = _inherit_case(75)
    binding = rm.ActiveBasisBinding(PARENT, 32, GROUP, 32, "c0")
    config = _config(0.98, solver=solver)
    chunk = _plan(config, device, {key: second}, {key: _context(model, key, 1000)}, {key: parent}, {key: binding})
    plan = chunk.plans[key]
    assert plan.decision == "refit" and plan.parent_version_ref is None
    if solver == "warm_start":
        assert chunk.counters["warm_start_count"] == 1
    label = of.crossing(np.linalg.eigvalsh(host.T @ host)[::-1], float(np.square(host).sum()), 0.98)
    assert label <= plan.observed_rank <= label + 32 and plan.bucket_rank >= -(-label // 32) * 32
    assert plan.decision_energy == pytest.approx(_stored_energy(host, plan.new_rows.numpy()), abs=1e-9)
    assert plan.decision_energy >= 0.98 + 1e-6


def test_bounded_working_set_plans_in_groups(device):
    """``max_working_bytes`` splits the chunk into consecutive groups whose planning tensors fit
    half the budget (reelcache/rank_method.py:1152-1168); the decisions and verified ranks equal the
    unbounded plan's."""
    rng = np.random.default_rng(76)
    model = ModelIdentity("bounded-test", "6" * 64, 2, 512, "THD", "bfloat16")
    sigma = np.arange(1, 513, dtype=np.float64) ** -0.9
    sources, contexts = {}, {}
    for layer, target in ((0, "K"), (0, "V"), (1, "K"), (1, "V")):
        key = MatrixKey(layer, target)
        sources[key] = _spectrum(rng, 2000, 512, sigma)[0]
        contexts[key] = _context(model, key, 2000)
    config = _config(0.98)
    keys = list(sources)
    bindings = {key: rm.ActiveBasisBinding() for key in keys}
    parents = {key: None for key in keys}
    ids = {k: f"s{k.layer}{k.target}" for k in keys}
    whole = rm.GramPlanner(config, device=device).plan({k: sources[k].to(device) for k in keys}, contexts, bindings,
                                                       parents, chunk_id="c1", source_ids=ids)
    per_matrix = 3 * 4 * 2000 * 512 + 3 * 4 * 512 * 512 + 3 * 8 * 1024 * 512
    bounded = rm.GramPlanner(config, device=device, max_working_bytes=2 * (2 * per_matrix)).plan(
        {k: sources[k].to(device) for k in keys}, contexts, bindings, parents, chunk_id="c1", source_ids=ids)
    assert whole.memory is None
    assert bounded.memory["group_size"] == 2 and bounded.memory["groups"] == 2
    assert bounded.memory["matrix_bytes_estimate"] == per_matrix
    for key in keys:
        a, b = whole.plans[key], bounded.plans[key]
        assert (a.decision, a.bucket_rank) == (b.decision, b.bucket_rank)
        assert b.decision_energy == pytest.approx(a.decision_energy, abs=1e-6)
