"""Online rank predictors of the planner: the paper's log-linear tail model learned per scope.

A fit's anchor sketch captures ``E_m`` of the energy in ``m`` directions; for a target ``E_t``
the feature is ``x = ln((1 - E_m) / (1 - E_t))`` and the model predicts ``ln r = a + b x``
(reelcache/predictor_registry.py:1-26, the state of reelcache/types.py:1245-1319).  ``(a, b)``
solve a 2 x 2 ridge system ``M (a, b) = v`` with prior ``M0 = s I``, ``v0 = M0 (ln m, 1)``;
every verified observation ``(x, r)`` adds ``z z^T`` to M and ``z ln r`` to v with ``z = (1, x)``.

Interfaces mirrored (names, fields, serialized schemas, errors): PredictorKey
(reelcache/types.py:1185-1228), OnlineRidgeState (:1231-1319), FitObservation (:1322-1385),
PredictorUse / RegistryView / RankPredictorRegistry / observation_origin
(reelcache/predictor_registry.py:42-330).  Planning pins a view; a commit reports its verified
observations afterwards, so a chunk's predictions never depend on the order its own fits finish.
Observation identities bind the learner scope and the source, so retries and replays are
idempotent; a repeated identity with another payload is an integrity error from the same origin
and a skipped duplicate (the first payload wins) from another one.
"""

from __future__ import annotations

import math
import threading
from dataclasses import dataclass
from types import MappingProxyType
from typing import Any, Iterable, Mapping, Sequence

from ._checks import need
from .errors import ConfigurationError, IntegrityError, StateError
from .types import RANK_BUCKET, MatrixKey, canonical_digest

REGISTRY_SCHEMA = "reelcache.rank_predictor_registry.v1"
RIDGE_SCHEMA = "reelcache.online_ridge_state.v1"
OBSERVATION_SCHEMA = "reelcache.fit_observation.v1"
PREDICTOR_REGIMES = ("fresh", "residual")
_LOG_RANK_LIMIT = 700.0  # exp() of more than this overflows a float


def _number(value) -> bool:
    return not isinstance(value, bool) and isinstance(value, (int, float)) and math.isfinite(value)


def _count(value, what: str, *, zero: bool = False) -> None:
    need(type(value) is int and (value >= 0 if zero else value >= 1),
         f"{what} must be a {'nonnegative' if zero else 'positive'} integer")


def _hex64(value, what: str) -> None:
    need(isinstance(value, str) and len(value) == 64 and all(c in "0123456789abcdef" for c in value),
         f"{what} must be a 64-digit hex digest")


@dataclass(frozen=True, order=True)
class PredictorKey:
    """Scope of one learner: model, layer, K or V, geometry, solver, detector and regime (fresh
    fits and augmentation residual fits never share a learner)."""

    model_fingerprint: str
    layer: int
    target: str
    rows: int
    channels: int
    solver: str
    detector: str
    regime: str

    def __post_init__(self) -> None:
        for name in ("model_fingerprint", "solver", "detector"):
            need(isinstance(getattr(self, name), str) and getattr(self, name), f"predictor {name} must be text")
        MatrixKey(self.layer, self.target)
        _count(self.rows, "predictor rows")
        _count(self.channels, "predictor channels")
        need(self.regime in PREDICTOR_REGIMES, f"predictor regime must be one of {PREDICTOR_REGIMES}")

    @property
    def matrix_key(self) -> MatrixKey:
        return MatrixKey(self.layer, self.target)

    def to_dict(self) -> dict[str, Any]:
        return {"model_fingerprint": self.model_fingerprint, "layer": self.layer, "target": self.target,
                "rows": self.rows, "channels": self.channels, "solver": self.solver, "detector": self.detector,
                "regime": self.regime}

    @property
    def digest(self) -> str:
        return canonical_digest(self.to_dict())

    @classmethod
    def from_dict(cls, data: Mapping[str, Any]) -> PredictorKey:
        try:
            return cls(**dict(data))
        except TypeError as exc:
            raise ConfigurationError("invalid predictor key fields") from exc


def _solve2(m: tuple[float, float, float], v: tuple[float, float]) -> tuple[float, float]:
    """``(a, b)`` of the symmetric 2 x 2 system ``[[m0, m1], [m1, m2]] (a, b) = v`` (Cramer)."""
    det = m[0] * m[2] - m[1] * m[1]
    return (m[2] * v[0] - m[1] * v[1]) / det, (m[0] * v[1] - m[1] * v[0]) / det


@dataclass(frozen=True)
class OnlineRidgeState:
    """The 2 x 2 ridge state of one learner; ``m`` holds M's distinct entries (m00, m01, m11)."""

    m: tuple[float, float, float]
    v: tuple[float, float]
    observations: int = 0
    revision: int = 0
    anchor_rank: int = RANK_BUCKET
    prior_strength: float = 2.0

    def __post_init__(self) -> None:
        m, v = tuple(self.m), tuple(self.v)
        need(len(m) == 3 and len(v) == 2 and all(_number(item) for item in m + v),
             "ridge state requires finite M (3 entries) and v (2 entries)")
        object.__setattr__(self, "m", tuple(float(item) for item in m))
        object.__setattr__(self, "v", tuple(float(item) for item in v))
        _count(self.observations, "ridge observations", zero=True)
        _count(self.revision, "ridge revision", zero=True)
        _count(self.anchor_rank, "anchor rank")
        need(_number(self.prior_strength) and self.prior_strength > 0, "ridge prior strength must be finite and positive")
        object.__setattr__(self, "prior_strength", float(self.prior_strength))
        need(self.m[0] > 0 and self.m[0] * self.m[2] - self.m[1] ** 2 > 0, "ridge M must be symmetric positive definite")

    @classmethod
    def initial(cls, anchor_rank: int = RANK_BUCKET, prior_strength: float = 2.0) -> OnlineRidgeState:
        """The prior: ``M0 = s I``, ``v0 = M0 (ln m, 1)`` (a = ln m, b = 1 before any observation)."""
        _count(anchor_rank, "anchor rank")
        s = float(prior_strength)
        return cls((s, 0.0, s), (s * math.log(anchor_rank), s), 0, 0, anchor_rank, s)

    def coefficients(self) -> tuple[float, float]:
        return _solve2(self.m, self.v)

    def log_rank(self, x: float) -> float:
        a, b = self.coefficients()
        return a + b * float(x)

    def predict(self, x: float) -> float:
        """``exp(a + b x)`` unrounded; ``inf`` beyond float range."""
        value = self.log_rank(x)
        return math.inf if value > _LOG_RANK_LIMIT else math.exp(value)

    def updated(self, x: float, observed_rank) -> OnlineRidgeState:
        need(_number(x) and _number(observed_rank) and observed_rank > 0,
             "ridge updates need a finite x and positive observed rank")
        x, y = float(x), math.log(float(observed_rank))
        m, v = self.m, self.v
        return OnlineRidgeState((m[0] + 1.0, m[1] + x, m[2] + x * x), (v[0] + y, v[1] + x * y),
                                self.observations + 1, self.revision + 1, self.anchor_rank, self.prior_strength)

    def to_dict(self) -> dict[str, Any]:
        return {"schema": RIDGE_SCHEMA, "m": list(self.m), "v": list(self.v), "observations": self.observations,
                "revision": self.revision, "anchor_rank": self.anchor_rank, "prior_strength": self.prior_strength}

    @property
    def digest(self) -> str:
        return canonical_digest(self.to_dict())

    @classmethod
    def from_dict(cls, data: Mapping[str, Any]) -> OnlineRidgeState:
        try:
            fields = dict(data)
            need(fields.pop("schema") == RIDGE_SCHEMA, "unsupported ridge state schema")
            return cls(m=tuple(fields.pop("m")), v=tuple(fields.pop("v")), **fields)
        except (KeyError, TypeError) as exc:
            raise ConfigurationError("invalid ridge state fields") from exc


@dataclass(frozen=True)
class FitObservation:
    """One verified training pair ``(x, observed rank)`` of a learner; never a KV matrix.

    ``origin`` names the commit context that produced it (:func:`observation_origin`); it is run
    context, not content, and is not serialized."""

    key: PredictorKey
    source_id: str
    anchor_energy: float
    target_energy: float
    x: float
    observed_rank: int
    predicted_rank: float | None = None
    prediction_revision: int | None = None
    origin: str | None = None

    def __post_init__(self) -> None:
        need(isinstance(self.key, PredictorKey), "observation key must be a PredictorKey")
        _hex64(self.source_id, "observation source id")
        if self.origin is not None:
            _hex64(self.origin, "observation origin")
        need(_number(self.anchor_energy) and 0 <= self.anchor_energy < 1, "anchor energy must be in [0, 1)")
        need(_number(self.target_energy) and 0 <= self.target_energy <= 1, "observation target must be in [0, 1]")
        need(self.target_energy < 1 and self.anchor_energy < self.target_energy,
             "observations come from below-target anchors and sub-unit targets")
        need(_number(self.x) and self.x > 0, "observation x must be finite and positive")
        _count(self.observed_rank, "observed rank")
        predicted = self.predicted_rank
        need(predicted is None or (not isinstance(predicted, bool) and isinstance(predicted, (int, float))
                                   and not math.isnan(predicted) and predicted > 0),
             "predicted rank must be positive or None")
        if self.prediction_revision is not None:
            _count(self.prediction_revision, "prediction revision", zero=True)
        for name in ("anchor_energy", "target_energy", "x"):
            object.__setattr__(self, name, float(getattr(self, name)))

    @property
    def observation_id(self) -> str:
        return canonical_digest({"key": self.key.to_dict(), "source_id": self.source_id})

    @property
    def payload_digest(self) -> str:
        return canonical_digest({"anchor_energy": self.anchor_energy, "target_energy": self.target_energy,
                                 "x": self.x, "observed_rank": self.observed_rank})

    def to_dict(self) -> dict[str, Any]:
        predicted = self.predicted_rank
        return {"schema": OBSERVATION_SCHEMA, "key": self.key.to_dict(), "source_id": self.source_id,
                "anchor_energy": self.anchor_energy, "target_energy": self.target_energy, "x": self.x,
                "observed_rank": self.observed_rank,
                "predicted_rank": predicted if predicted is not None and math.isfinite(predicted) else None,
                "prediction_revision": self.prediction_revision}

    @classmethod
    def from_dict(cls, data: Mapping[str, Any]) -> FitObservation:
        try:
            fields = dict(data)
            need(fields.pop("schema") == OBSERVATION_SCHEMA, "unsupported fit observation schema")
            return cls(key=PredictorKey.from_dict(fields.pop("key")), **fields)
        except (KeyError, TypeError) as exc:
            raise ConfigurationError("invalid fit observation fields") from exc


@dataclass(frozen=True)
class PredictorUse:
    """The learner revision and prediction one fit started from."""

    registry_id: str
    sequence: int
    key: PredictorKey
    state: OnlineRidgeState
    x: float
    log_rank: float
    predicted_rank: float

    @property
    def revision_ref(self) -> str:
        return (f"reelcache-rank-predictor:{self.registry_id}:{self.key.digest[:16]}"
                f":r{self.state.revision}:{self.state.digest[:16]}")

    def to_dict(self) -> dict[str, Any]:
        a, b = self.state.coefficients()
        finite = math.isfinite(self.predicted_rank)
        return {"schema": "reelcache.predictor_use.v1", "registry_id": self.registry_id, "sequence": self.sequence,
                "key": self.key.to_dict(), "state": self.state.to_dict(), "a": a, "b": b, "x": self.x,
                "log_rank": self.log_rank, "predicted_rank": self.predicted_rank if finite else None,
                "predicted_rank_overflow": not finite, "revision_ref": self.revision_ref}


class RegistryView:
    """An immutable revision of the learners, pinned for one commit's predictions."""

    def __init__(self, registry_id: str, sequence: int, states: Mapping[PredictorKey, OnlineRidgeState],
                 anchor_rank: int, prior_strength: float, speculative: Sequence[str] = ()):
        self.registry_id, self.sequence = registry_id, sequence
        self._states = MappingProxyType(dict(states))
        self.anchor_rank, self.prior_strength = anchor_rank, prior_strength
        # Identities of unpublished ancestor observations folded into this view (pipelined commits).
        self.speculative = tuple(speculative)

    @classmethod
    def empty(cls, registry_id: str = "local", *, anchor_rank: int = RANK_BUCKET,
              prior_strength: float = 2.0) -> RegistryView:
        """A view with every learner at its prior (a planner without a shared registry)."""
        return cls(registry_id, 0, {}, anchor_rank, prior_strength)

    @property
    def states(self) -> Mapping[PredictorKey, OnlineRidgeState]:
        return self._states

    def state(self, key: PredictorKey) -> OnlineRidgeState:
        need(isinstance(key, PredictorKey), "predictor lookups require a PredictorKey")
        found = self._states.get(key)
        return OnlineRidgeState.initial(self.anchor_rank, self.prior_strength) if found is None else found

    def predict(self, key: PredictorKey, x: float) -> PredictorUse:
        need(_number(x), "prediction requires a finite anchor feature")
        state = self.state(key)
        return PredictorUse(self.registry_id, self.sequence, key, state, float(x), state.log_rank(x), state.predict(x))

    @property
    def digest(self) -> str:
        return canonical_digest({"registry_id": self.registry_id, "sequence": self.sequence,
                                 "states": sorted([key.digest, state.digest] for key, state in self._states.items())})


def observation_origin(lineage: str, kind: str, node_id: str, view: RegistryView) -> str:
    """Commit context of a fit's observations: lineage, commit kind and node, and the pinned view its
    predictions came from (the same for a retried or replayed commit)."""
    return canonical_digest({"schema": "reelcache.observation_origin.v1", "lineage": lineage, "commit": kind,
                             "node_id": node_id, "registry": view.registry_id, "view": view.digest})


class _Ledger:
    """Applied observation identities in order, with their payload digests and origins."""

    def __init__(self):
        self.order: list[str] = []
        self.payloads: dict[str, str] = {}
        self.origins: dict[str, str | None] = {}

    def known(self, identity: str):
        if identity not in self.payloads:
            return None
        return self.payloads[identity], self.origins.get(identity)

    def add(self, item: FitObservation) -> None:
        self.order.append(item.observation_id)
        self.payloads[item.observation_id] = item.payload_digest
        self.origins[item.observation_id] = item.origin


def _is_duplicate(known: tuple[str, str | None], item: FitObservation) -> bool:
    """True when ``item`` repeats an applied identity harmlessly (same payload, or another origin's
    payload: the first applied one wins); an integrity error when the same origin disagrees."""
    payload, origin = known
    if payload == item.payload_digest or (origin is not None and item.origin is not None and origin != item.origin):
        return True
    raise IntegrityError("conflicting observation payload for an applied source identity")


def _check_batch(items, anchor_rank: int) -> list[FitObservation]:
    batch = list(items)
    for item in batch:
        need(isinstance(item, FitObservation), "registries learn only from FitObservation records")
        need(item.observed_rank > anchor_rank, "only verified fits needing more than the anchor rank are observations")
    return batch


class RankPredictorRegistry:
    """Thread-safe owner of a model's shared learners.

    ``mode="shared"`` applies observations in arrival order; ``mode="replay"`` (qualification)
    continues a recorded order and rejects any deviation, so its predictions depend only on it."""

    def __init__(self, registry_id: str, *, anchor_rank: int = RANK_BUCKET, prior_strength: float = 2.0,
                 mode: str = "shared", expected_order: Sequence[str] | None = None) -> None:
        need(isinstance(registry_id, str) and registry_id, "registry id must be text")
        _count(anchor_rank, "anchor rank")
        OnlineRidgeState.initial(anchor_rank, prior_strength)
        need(mode in ("shared", "replay"), "registry mode must be shared or replay")
        need((mode == "replay") == (expected_order is not None), "only replay registries take a recorded update order")
        self.registry_id, self.anchor_rank, self.prior_strength, self.mode = registry_id, anchor_rank, float(prior_strength), mode
        self._lock = threading.Lock()
        self._states: dict[PredictorKey, OnlineRidgeState] = {}
        self._ledger = _Ledger()
        self._expected = None if expected_order is None else tuple(expected_order)
        if self._expected is not None:
            need(len(set(self._expected)) == len(self._expected)
                 and all(isinstance(item, str) and len(item) == 64 for item in self._expected),
                 "replay order must list unique observation identities")
        self.stats = {"applied": 0, "duplicates": 0, "rejected": 0, "divergent_duplicates": 0}

    @property
    def sequence(self) -> int:
        with self._lock:
            return len(self._ledger.order)

    @property
    def log(self) -> tuple[str, ...]:
        with self._lock:
            return tuple(self._ledger.order)

    def _initial(self) -> OnlineRidgeState:
        return OnlineRidgeState.initial(self.anchor_rank, self.prior_strength)

    def _in_order(self, position: int, identities: Sequence[str]) -> bool:
        return self._expected is None or tuple(self._expected[position:position + len(identities)]) == tuple(identities)

    def pin(self) -> RegistryView:
        """The current revision, immutable, for one commit's predictions."""
        with self._lock:
            return RegistryView(self.registry_id, len(self._ledger.order), self._states, self.anchor_rank,
                                self.prior_strength)

    def state(self, key: PredictorKey) -> OnlineRidgeState:
        return self.pin().state(key)

    def pin_with(self, pending: Iterable[FitObservation]) -> RegistryView:
        """The pinned revision plus a lineage's own verified, unpublished observations (in order,
        skipping applied ones); the shared learners are not changed."""
        batch = _check_batch(pending, self.anchor_rank)
        with self._lock:
            states = dict(self._states)
            seen = {identity: self._ledger.known(identity) for identity in self._ledger.order}
            folded = []
            for item in batch:
                known = seen.get(item.observation_id)
                if known is not None:
                    _is_duplicate(known, item)
                    continue
                if not self._in_order(len(self._ledger.order) + len(folded), [item.observation_id]):
                    raise StateError("replay registry received a pending observation out of its recorded order")
                states[item.key] = states.get(item.key, self._initial()).updated(item.x, item.observed_rank)
                seen[item.observation_id] = (item.payload_digest, item.origin)
                folded.append(item.observation_id)
            return RegistryView(self.registry_id, len(self._ledger.order) + len(folded), states, self.anchor_rank,
                                self.prior_strength, folded)

    def observe(self, observations: Iterable[FitObservation]) -> tuple[bool, ...]:
        """Apply verified observations in order; per item, whether it was applied.  The whole batch is
        checked before any learner changes."""
        batch = _check_batch(observations, self.anchor_rank)
        with self._lock:
            flags, pending, divergent = [], {}, 0
            for item in batch:
                identity = item.observation_id
                known = pending.get(identity) or self._ledger.known(identity)
                if known is not None:
                    try:
                        _is_duplicate(known, item)
                    except IntegrityError:
                        self.stats["rejected"] += 1
                        raise
                    divergent += known[0] != item.payload_digest
                    flags.append(False)
                    continue
                pending[identity] = (item.payload_digest, item.origin)
                flags.append(True)
            new = [item for item, flag in zip(batch, flags) if flag]
            if not self._in_order(len(self._ledger.order), [item.observation_id for item in new]):
                self.stats["rejected"] += 1
                raise StateError("replay registry received an observation out of its recorded order")
            for item in new:
                self._states[item.key] = self._states.get(item.key, self._initial()).updated(item.x, item.observed_rank)
                self._ledger.add(item)
            self.stats["applied"] += len(new)
            self.stats["duplicates"] += len(batch) - len(new)
            self.stats["divergent_duplicates"] += divergent
            return tuple(flags)

    def to_dict(self) -> dict[str, Any]:
        with self._lock:
            ledger = self._ledger
            return {"schema": REGISTRY_SCHEMA, "registry_id": self.registry_id, "anchor_rank": self.anchor_rank,
                    "prior_strength": self.prior_strength, "sequence": len(ledger.order),
                    "learners": [{"key": key.to_dict(), "state": state.to_dict()}
                                 for key, state in sorted(self._states.items(), key=lambda pair: pair[0])],
                    "applied": [[identity, ledger.payloads[identity]]
                                + ([] if ledger.origins.get(identity) is None else [ledger.origins[identity]])
                                for identity in ledger.order]}

    @classmethod
    def from_dict(cls, data: Mapping[str, Any], *, mode: str = "shared",
                  expected_order: Sequence[str] | None = None) -> RankPredictorRegistry:
        """A serialized registry restored (replay mode continues with a recorded order)."""
        try:
            need(data["schema"] == REGISTRY_SCHEMA, "unsupported predictor registry schema")
            registry = cls(data["registry_id"], anchor_rank=data["anchor_rank"], prior_strength=data["prior_strength"],
                           mode=mode, expected_order=expected_order)
            states: dict[PredictorKey, OnlineRidgeState] = {}
            for learner in data["learners"]:
                key = PredictorKey.from_dict(learner["key"])
                if key in states:
                    raise IntegrityError("duplicate learner in a serialized registry")
                states[key] = OnlineRidgeState.from_dict(learner["state"])
            ledger = _Ledger()
            for entry in data["applied"]:
                if not isinstance(entry, (list, tuple)) or len(entry) not in (2, 3):
                    raise IntegrityError("serialized registry observations are [identity, payload(, origin)]")
                if len(entry) == 3 and not (isinstance(entry[2], str) and len(entry[2]) == 64):
                    raise IntegrityError("invalid serialized observation origin")
                ledger.order.append(entry[0])
                ledger.payloads[entry[0]] = entry[1]
                ledger.origins[entry[0]] = entry[2] if len(entry) == 3 else None
            sequence = data["sequence"]
        except (KeyError, TypeError, ValueError) as exc:
            raise IntegrityError("invalid serialized predictor registry") from exc
        applied = len(ledger.order)
        if (type(sequence) is not int or sequence != applied or len(ledger.payloads) != applied
                or sum(state.observations for state in states.values()) != applied):
            raise IntegrityError("serialized registry counts disagree with its applied observations")
        if expected_order is not None and tuple(expected_order[:applied]) != tuple(ledger.order):
            raise StateError("replay order does not start with the snapshot's applied observations")
        registry._states, registry._ledger = states, ledger
        return registry


__all__ = ["FitObservation", "OBSERVATION_SCHEMA", "OnlineRidgeState", "PREDICTOR_REGIMES", "PredictorKey",
           "PredictorUse", "REGISTRY_SCHEMA", "RankPredictorRegistry", "RegistryView", "observation_origin"]
