"""CPU tests of the online rank predictors (reelcache/predictor_registry.py, the ridge state of
reelcache/types.py:1231-1319) and of the planner configuration's refit rules.

The ridge state is pinned by the reference's own known answers (tests/test_step4_types_registry.py:
144-171: the prior is the zero-data rule a = ln 32, b = 1, so it predicts 32 (1 - E_m) / (1 - E_t))
and, independently of its update formula, by an augmented least-squares problem solved with
``numpy.linalg.lstsq`` (prior rows sqrt(s) [1, 0] -> sqrt(s) ln m and sqrt(s) [0, 1] -> sqrt(s),
one row [1, x] -> ln r per observation).  The registry is checked for idempotent retries,
conflicting payloads, origin-aware duplicates, immutable pinned views, learner isolation, replay
order, pending folds, serialization and concurrency.
"""

import json
import math
import threading

import numpy as np
import pytest

from reelcache_amd import rank_method as rm
from reelcache_amd import rank_predictor as rp
from reelcache_amd.errors import ConfigurationError, IntegrityError, StateError
from reelcache_amd.types import CodecSpec, MatrixKey, canonical_digest, energy_targets


def _key(model="m-v1", layer=0, target="K", rows=4680, regime="fresh"):
    return rp.PredictorKey(model, layer, target, rows, 1536, "fp32_gram_topk_rr.v1:m64:s3",
                           "sketch_qr_subspace.v1:m32:q2", regime)


def _obs(key, source, x, rank, origin=None):
    anchor = 0.5
    target = 1.0 - (1.0 - anchor) / math.exp(x)  # x = ln((1 - anchor) / (1 - target))
    return rp.FitObservation(key, canonical_digest({"source": source}), anchor, target, x, rank, origin=origin)


def test_prior_is_the_zero_data_rule():
    state = rp.OnlineRidgeState.initial()
    assert state.m == (2.0, 0.0, 2.0) and state.v == (pytest.approx(2 * math.log(32)), 2.0)
    a, b = state.coefficients()
    assert a == pytest.approx(math.log(32)) and b == pytest.approx(1.0)
    x = math.log((1 - 0.90) / (1 - 0.98))
    assert state.predict(x) == pytest.approx(32 * (1 - 0.90) / (1 - 0.98))
    assert state.predict(1e6) == math.inf


def test_updates_solve_the_augmented_least_squares_problem():
    rng = np.random.default_rng(3)
    xs = rng.uniform(0.2, 3.0, 25)
    labels = rng.integers(33, 900, 25)
    state = rp.OnlineRidgeState.initial(anchor_rank=48, prior_strength=3.0)
    for x, label in zip(xs, labels):
        state = state.updated(float(x), int(label))
    s = math.sqrt(3.0)
    design = np.vstack([[s, 0.0], [0.0, s], np.stack([np.ones_like(xs), xs], 1)])
    rhs = np.concatenate([[s * math.log(48), s], np.log(labels)])
    expected = np.linalg.lstsq(design, rhs, rcond=None)[0]
    np.testing.assert_allclose(state.coefficients(), expected, rtol=1e-12, atol=1e-12)
    assert (state.observations, state.revision) == (25, 25)
    assert rp.OnlineRidgeState.from_dict(json.loads(json.dumps(state.to_dict()))) == state
    for bad in ((float("nan"), 40), (1.0, 0), (1.0, True)):
        with pytest.raises(ConfigurationError):
            state.updated(*bad)
    with pytest.raises(ConfigurationError):
        rp.OnlineRidgeState((1.0, 2.0, 1.0), (0.0, 0.0))  # not positive definite


def test_observation_validation_and_identity():
    key = _key()
    first = _obs(key, "a", 1.2, 80)
    assert first.observation_id == _obs(key, "a", 2.0, 90).observation_id  # scope + source only
    assert first.payload_digest != _obs(key, "a", 2.0, 90).payload_digest
    assert rp.FitObservation.from_dict(json.loads(json.dumps(first.to_dict()))) == first
    for fields in ({"anchor_energy": 0.99}, {"target_energy": 1.0}, {"x": -1.0}, {"observed_rank": 0},
                   {"source_id": "short"}):
        data = dict(key=key, source_id=first.source_id, anchor_energy=0.5, target_energy=0.98, x=1.0,
                    observed_rank=40)
        data.update(fields)
        with pytest.raises(ConfigurationError):
            rp.FitObservation(**data)
    with pytest.raises(ConfigurationError):
        rp.PredictorKey("m", 0, "Q", 1, 1, "s", "d", "fresh")
    with pytest.raises(ConfigurationError):
        rp.PredictorKey("m", 0, "K", 1, 1, "s", "d", "other")


def test_retries_conflicts_and_origins():
    registry = rp.RankPredictorRegistry("scope")
    key = _key()
    first = _obs(key, "chunk-1", 1.2, 80)
    assert registry.observe([first]) == (True,)
    assert registry.observe([first]) == (False,)
    conflict = rp.FitObservation(key, first.source_id, 0.5, 0.98, 1.2, 81)
    with pytest.raises(IntegrityError):
        registry.observe([conflict])
    assert registry.sequence == 1
    assert registry.stats == {"applied": 1, "duplicates": 1, "rejected": 1, "divergent_duplicates": 0}
    with pytest.raises(ConfigurationError):
        registry.observe([_obs(key, "chunk-2", 1.0, 32)])  # not above the anchor rank
    # Another origin's divergent payload for an applied identity: skipped, first payload wins.
    here, there = "1" * 64, "2" * 64
    registry.observe([_obs(key, "chunk-3", 1.0, 60, origin=here)])
    before = registry.pin().predict(key, 1.0).predicted_rank
    assert registry.observe([_obs(key, "chunk-3", 1.5, 70, origin=there)]) == (False,)
    assert registry.stats["divergent_duplicates"] == 1
    assert registry.pin().predict(key, 1.0).predicted_rank == before
    with pytest.raises(IntegrityError):
        registry.observe([_obs(key, "chunk-3", 1.5, 70, origin=here)])


def test_pinned_views_and_learner_isolation():
    registry = rp.RankPredictorRegistry("scope")
    key = _key()
    view = registry.pin()
    before = view.predict(key, 1.5)
    others = [_key(regime="residual"), _key(model="other"), _key(rows=960)]
    baseline = [view.predict(other, 1.0).predicted_rank for other in others]
    registry.observe([_obs(key, "a", 1.5, 300), _obs(key, "b", 0.7, 90)])
    assert view.predict(key, 1.5).predicted_rank == before.predicted_rank  # the pinned view is immutable
    after = registry.pin().predict(key, 1.5)
    assert after.predicted_rank != before.predicted_rank and after.state.revision == 2
    assert ":r2:" in after.revision_ref and before.to_dict()["state"]["revision"] == 0
    assert [registry.pin().predict(other, 1.0).predicted_rank for other in others] == baseline
    assert registry.pin().digest != view.digest


def test_replay_order_and_pending_folds():
    live = rp.RankPredictorRegistry("live")
    key, other = _key(), _key(layer=1)
    batch = [_obs(key, "a", 1.1, 70), _obs(other, "b", 0.4, 40), _obs(key, "c", 2.0, 300)]
    snapshot = live.to_dict()
    folded = live.pin_with(batch)
    assert live.sequence == 0 and folded.sequence == 3 and len(folded.speculative) == 3
    live.observe(batch)
    assert folded.predict(key, 1.3).predicted_rank == live.pin().predict(key, 1.3).predicted_rank
    replay = rp.RankPredictorRegistry.from_dict(snapshot, mode="replay", expected_order=live.log)
    with pytest.raises(StateError):
        replay.observe([batch[2]])
    assert replay.sequence == 0
    replay.observe(batch[:2])
    replay.observe(batch[2:])
    assert replay.to_dict()["learners"] == live.to_dict()["learners"]
    with pytest.raises(StateError):
        replay.observe([_obs(key, "extra", 1.0, 50)])
    with pytest.raises(ConfigurationError):
        rp.RankPredictorRegistry("x", expected_order=[])


def test_serialization_and_tampering():
    registry = rp.RankPredictorRegistry("scope")
    registry.observe([_obs(_key(), "a", 1.3, 120), _obs(_key(target="V"), "b", 0.9, 64)])
    restored = rp.RankPredictorRegistry.from_dict(json.loads(json.dumps(registry.to_dict())))
    for key in (_key(), _key(target="V")):
        assert restored.pin().predict(key, 0.8).predicted_rank == registry.pin().predict(key, 0.8).predicted_rank
    assert restored.observe([_obs(_key(), "a", 1.3, 120)]) == (False,)
    data = registry.to_dict()
    data["sequence"] = 5
    with pytest.raises(IntegrityError):
        rp.RankPredictorRegistry.from_dict(data)
    data = registry.to_dict()
    data["learners"] = data["learners"][:1]
    with pytest.raises(IntegrityError):
        rp.RankPredictorRegistry.from_dict(data)


def test_concurrent_updates_are_serialized():
    registry = rp.RankPredictorRegistry("shared")
    keys = [_key(layer=layer) for layer in range(4)]

    def worker(index):
        for step in range(25):
            registry.observe([_obs(keys[step % 4], f"{index}-{step}", 0.5 + step / 10, 40 + step)])

    threads = [threading.Thread(target=worker, args=(index,)) for index in range(4)]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join()
    assert registry.sequence == 100 and len(set(registry.log)) == 100
    assert sum(state.observations for state in registry.pin().states.values()) == 100


def test_planner_configuration_of_the_refit_rules_and_solvers():
    base = dict(targets=energy_targets("causvid"), codec=CodecSpec("svd_hevc", 1))
    config = rm.RankMethodConfig(**base, solver="warm_start", refit_rule="cumulative", refit_debt_on_share=True,
                                 refit_hysteresis=2)
    assert config.refit_hysteresis == 2.0 and isinstance(config.refit_hysteresis, float)
    assert config.solver_id() == "fp32_gram_eigh.v1" and config.solver_id(warm=True) == "fp32_gram_warm_rr.v1:s1"
    assert config.detector == "sketch_qr_subspace.v1:m32:q2"
    with pytest.raises(ConfigurationError):
        rm.RankMethodConfig(**base, refit_debt_on_share=True)  # the paper rule carries no debt
    for hysteresis in (0.5, 17, float("nan"), True):
        with pytest.raises(ConfigurationError):
            rm.RankMethodConfig(**base, refit_rule="cumulative", refit_hysteresis=hysteresis)
    # refit_debt_test: the ski-rental rule reduces to the paper test without debt.
    fresh = {"coefficient_bytes": 100.0, "scale_bytes": 10.0, "basis_bytes": 500.0, "total_bytes": 610.0}
    candidate = {"coefficient_bytes": 150.0, "scale_bytes": 10.0, "basis_bytes": 100.0, "total_bytes": 260.0}
    assert rm.refit_debt_test(0.0, candidate, fresh) == (False, 50.0, 400.0)
    assert rm.refit_debt_test(350.0, candidate, fresh) == (True, 50.0, 400.0)
    assert rm.refit_debt_test(349.0, candidate, fresh) == (False, 50.0, 400.0)
    assert rm.refit_debt_test(700.0, candidate, fresh, hysteresis=2.0)[0] is False
    assert rm.refit_debt_test(750.0, candidate, fresh, hysteresis=2.0)[0] is True
    assert MatrixKey(0, "K")  # the planner's keys
