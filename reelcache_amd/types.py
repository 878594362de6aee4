"""Contract types of the fit path: matrix coordinates, energy targets and codec parameters.

The names, fields and validation rules are those of ``reelcache/types.py`` (ModelIdentity
:78-154, MatrixKey :157-174, TensorContext :177-250, CodecSpec :252-312, RANK_BUCKET :380,
EnergyTargets :531-591), so contexts and specs built by reference callers and by this package
are interchangeable: the fit code reads only their public attributes (``shape``, ``dtype``,
``key.target``, ``key_space``, ``channels`` ...).
"""

from __future__ import annotations

import hashlib
import json
import math
from dataclasses import dataclass
from types import MappingProxyType
from typing import Any, Mapping

from .errors import ConfigurationError

RANK_BUCKET = 32

_DTYPE_NAMES = {
    "bfloat16": "bfloat16", "bf16": "bfloat16",
    "float16": "float16", "half": "float16", "fp16": "float16",
    "float32": "float32", "float": "float32",
    "float64": "float64", "double": "float64",
}
_TARGETS = ("K", "V")


def canonical_dtype(value: Any) -> str:
    """``torch.bfloat16`` / ``"bf16"`` / ... -> the canonical dtype name."""
    name = str(value)
    if name.startswith("torch."):
        name = name[len("torch."):]
    try:
        return _DTYPE_NAMES[name]
    except KeyError:
        raise ConfigurationError(f"unsupported KV dtype: {value!r}") from None


def canonical_digest(value: Any) -> str:
    """SHA-256 hex digest of the canonical JSON of ``value`` (sorted keys, no whitespace, no NaN)."""
    def plain(item):
        kind = type(item)
        if kind is str or kind is int or kind is float or kind is bool or item is None:
            return item  # the common leaves, without the abstract-class checks below
        if kind is dict:
            return {str(key): plain(child) for key, child in item.items()}
        if isinstance(item, Mapping):
            return {str(key): plain(child) for key, child in item.items()}
        if isinstance(item, (list, tuple)):
            return [plain(child) for child in item]
        return item
    text = json.dumps(plain(value), sort_keys=True, separators=(",", ":"), allow_nan=False)
    return hashlib.sha256(text.encode("utf-8")).hexdigest()


def _count(value: Any, name: str, *, zero: bool = False) -> None:
    if type(value) is not int or value < (0 if zero else 1):
        raise ConfigurationError(f"{name} must be a {'nonnegative' if zero else 'positive'} integer")


def _nonempty(value: Any, name: str) -> None:
    if not isinstance(value, str) or not value.strip():
        raise ConfigurationError(f"{name} must be a nonempty string")


def _unit_fraction(value: Any, name: str) -> float:
    if isinstance(value, bool) or not isinstance(value, (int, float)) or not math.isfinite(value) or not 0 < value <= 1:
        raise ConfigurationError(f"{name} must be in (0, 1]")
    return float(value)


@dataclass(frozen=True)
class ModelIdentity:
    """A model's KV geometry: layers, channels per target and the stored dtype."""

    name: str
    fingerprint: str
    layers: int
    kv_channels: int | Mapping[str, int]
    layout: str
    dtype: str | Mapping[str, str]

    def __post_init__(self) -> None:
        _nonempty(self.name, "model name")
        _nonempty(self.fingerprint, "model fingerprint")
        _count(self.layers, "layers")
        _nonempty(self.layout, "layout")
        if isinstance(self.dtype, Mapping):
            keys = set(self.dtype)
            every = {f"{layer}:{target}" for layer in range(self.layers) for target in _TARGETS}
            if keys != set(_TARGETS) and keys != every:
                raise ConfigurationError("dtype mapping must cover K/V or every layer:target matrix")
            object.__setattr__(self, "dtype", MappingProxyType({k: canonical_dtype(v) for k, v in self.dtype.items()}))
        else:
            object.__setattr__(self, "dtype", canonical_dtype(self.dtype))
        if isinstance(self.kv_channels, Mapping):
            if set(self.kv_channels) != set(_TARGETS):
                raise ConfigurationError("kv_channels mapping must contain exactly K and V")
            for target, channels in self.kv_channels.items():
                _count(channels, f"{target} channels")
            object.__setattr__(self, "kv_channels", MappingProxyType(dict(self.kv_channels)))
        else:
            _count(self.kv_channels, "kv_channels")

    def to_dict(self) -> dict[str, Any]:
        """JSON form (the field names of the reference's record)."""
        def plain(value):
            return dict(value) if isinstance(value, Mapping) else value
        return {"name": self.name, "fingerprint": self.fingerprint, "layers": self.layers,
                "kv_channels": plain(self.kv_channels), "layout": self.layout, "dtype": plain(self.dtype)}

    @classmethod
    def from_dict(cls, data: Mapping[str, Any]) -> "ModelIdentity":
        try:
            return cls(**dict(data))
        except (TypeError, KeyError) as error:
            raise ConfigurationError("invalid model identity fields") from error

    def channels_for(self, target) -> int:
        target = target.target if isinstance(target, MatrixKey) else target
        if target not in _TARGETS:
            raise ConfigurationError("target must be K or V")
        return self.kv_channels[target] if isinstance(self.kv_channels, Mapping) else self.kv_channels

    def dtype_for(self, target) -> str:
        key = target if isinstance(target, MatrixKey) else None
        name = key.target if key is not None else target
        if name not in _TARGETS:
            raise ConfigurationError("target must be K or V")
        if key is not None and key.layer >= self.layers:
            raise ConfigurationError("matrix layer is outside the model")
        if not isinstance(self.dtype, Mapping):
            return self.dtype
        if name in self.dtype:
            return self.dtype[name]
        if key is None:
            raise ConfigurationError("layer-specific dtype requires a MatrixKey")
        return self.dtype[f"{key.layer}:{key.target}"]


@dataclass(frozen=True, order=True)
class MatrixKey:
    layer: int
    target: str

    def __post_init__(self) -> None:
        _count(self.layer, "layer", zero=True)
        if self.target not in _TARGETS:
            raise ConfigurationError("matrix target must be K or V")

    def to_dict(self) -> dict[str, Any]:
        return {"layer": self.layer, "target": self.target}

    @classmethod
    def from_dict(cls, data: Mapping[str, Any]) -> "MatrixKey":
        if not isinstance(data, Mapping) or set(data) != {"layer", "target"}:
            raise ConfigurationError("a matrix key is {layer, target}")
        return cls(data["layer"], data["target"])


@dataclass(frozen=True)
class TensorContext:
    """Coordinates of one [frames * height * width, channels] matrix of a chunk."""

    model: ModelIdentity
    key: MatrixKey
    token_start: int
    frames: int
    height: int
    width: int
    key_space: str
    source_dtype: str | None = None

    def __post_init__(self) -> None:
        if not isinstance(self.model, ModelIdentity) or not isinstance(self.key, MatrixKey):
            raise ConfigurationError("context requires ModelIdentity and MatrixKey")
        if self.key.layer >= self.model.layers:
            raise ConfigurationError("matrix layer is outside the model")
        _count(self.token_start, "token_start", zero=True)
        for name in ("frames", "height", "width"):
            _count(getattr(self, name), name)
        if self.key_space not in ("pre_rope", "post_rope", "none"):
            raise ConfigurationError("key_space must be pre_rope, post_rope, or none")
        if self.key.target == "V" and self.key_space != "none":
            raise ConfigurationError("V matrices must use key_space='none'")
        if self.source_dtype is not None:
            object.__setattr__(self, "source_dtype", canonical_dtype(self.source_dtype))

    def to_dict(self) -> dict[str, Any]:
        """JSON form (the field names of the reference's record; ``source_dtype`` only when set)."""
        record = {"model": self.model.to_dict(), "key": self.key.to_dict(), "token_start": self.token_start,
                  "frames": self.frames, "height": self.height, "width": self.width, "key_space": self.key_space}
        if self.source_dtype is not None:
            record["source_dtype"] = self.source_dtype
        return record

    @classmethod
    def from_dict(cls, data: Mapping[str, Any]) -> "TensorContext":
        try:
            fields = dict(data)
            fields["model"] = ModelIdentity.from_dict(fields["model"])
            fields["key"] = MatrixKey.from_dict(fields["key"])
            return cls(**fields)
        except (TypeError, KeyError) as error:
            raise ConfigurationError("invalid tensor context fields") from error

    @property
    def channels(self) -> int:
        return self.model.channels_for(self.key)

    @property
    def dtype(self) -> str:
        return self.model.dtype_for(self.key) if self.source_dtype is None else self.source_dtype

    @property
    def token_count(self) -> int:
        return self.frames * self.height * self.width

    @property
    def token_end(self) -> int:
        return self.token_start + self.token_count

    @property
    def shape(self) -> tuple[int, int]:
        return self.token_count, self.channels


@dataclass(frozen=True)
class CodecSpec:
    """Representation parameters of one matrix; ``protected_fraction`` matters only for
    ``leading_columns`` (canonicalized to 1 for ``per_channel`` and 0 for ``global``)."""

    kind: str = "raw"
    rank: int | None = None
    normalization: str = "per_channel"
    protected_fraction: float = 1.0
    pix_fmt: str = "yuv444p"
    qp: int = 8
    preset: str = "ultrafast"
    ffmpeg_path: str | None = None
    inter_prediction: bool | None = False

    def __post_init__(self) -> None:
        if self.kind not in ("raw", "svd", "svd_hevc"):
            raise ConfigurationError("codec kind must be raw, svd, or svd_hevc")
        if self.kind == "raw":
            if self.rank is not None:
                raise ConfigurationError("raw encoding does not take a rank")
        else:
            _count(self.rank, "rank")
        if self.normalization not in ("per_channel", "global", "leading_columns"):
            raise ConfigurationError("unsupported normalization")
        fraction = self.protected_fraction
        if isinstance(fraction, bool) or not isinstance(fraction, (int, float)) or not math.isfinite(fraction) \
                or not 0 <= fraction <= 1:
            raise ConfigurationError("protected_fraction must be in [0, 1]")
        if self.normalization == "global":
            object.__setattr__(self, "protected_fraction", 0.0)
        elif self.normalization == "per_channel":
            object.__setattr__(self, "protected_fraction", 1.0)
        _nonempty(self.pix_fmt, "pix_fmt")
        _nonempty(self.preset, "preset")
        if self.ffmpeg_path is not None:
            _nonempty(self.ffmpeg_path, "ffmpeg_path")
            if "\x00" in self.ffmpeg_path:
                raise ConfigurationError("ffmpeg_path must not contain NUL")
        if type(self.qp) is not int or not 0 <= self.qp <= 51:
            raise ConfigurationError("qp must be an integer in [0, 51]")
        if self.inter_prediction is not None and type(self.inter_prediction) is not bool:
            raise ConfigurationError("inter_prediction must be a boolean")
        if self.kind != "svd_hevc":
            if self.inter_prediction:
                raise ConfigurationError("inter prediction applies only to svd_hevc coefficient streams")
            object.__setattr__(self, "inter_prediction", False)

    def to_dict(self) -> dict[str, Any]:
        result = {"kind": self.kind, "rank": self.rank, "normalization": self.normalization,
                  "protected_fraction": self.protected_fraction, "pix_fmt": self.pix_fmt, "qp": self.qp,
                  "preset": self.preset, "ffmpeg_path": self.ffmpeg_path}
        if self.kind == "svd_hevc" and self.inter_prediction is not None:
            result["inter_prediction"] = self.inter_prediction
        return result


@dataclass(frozen=True)
class EnergyTargets:
    """Pre-codec energy fractions of normalized pre-RoPE K and direct V."""

    profile: str
    key: float
    value: float
    provisional: bool
    note: str | None = None

    def __post_init__(self) -> None:
        _nonempty(self.profile, "energy profile")
        object.__setattr__(self, "key", _unit_fraction(self.key, "K energy target"))
        object.__setattr__(self, "value", _unit_fraction(self.value, "V energy target"))
        if type(self.provisional) is not bool:
            raise ConfigurationError("provisional must be boolean")
        if self.note is not None:
            _nonempty(self.note, "energy profile note")

    def for_target(self, target) -> float:
        target = target.target if isinstance(target, MatrixKey) else target
        if target == "K":
            return self.key
        if target == "V":
            return self.value
        raise ConfigurationError("energy target selector must be K or V")

    def is_diagnostic(self, target) -> bool:
        return self.for_target(target) == 1.0


_PROVISIONAL = "provisional K98/V95 until the energy sweeps select a model-specific profile"
ENERGY_TARGET_PROFILES = MappingProxyType({
    "causvid": EnergyTargets("causvid", 0.98, 0.95, False, "final: pre-RoPE K 98%, V 95%"),
    "raven": EnergyTargets("raven", 0.98, 0.95, True, _PROVISIONAL),
    "longlive1": EnergyTargets("longlive1", 0.98, 0.95, True, _PROVISIONAL),
    "longlive2": EnergyTargets("longlive2", 0.98, 0.95, True, _PROVISIONAL),
    "longcat_720p": EnergyTargets("longcat_720p", 0.98, 0.95, True, _PROVISIONAL),
})


def energy_targets(profile: str) -> EnergyTargets:
    """A built-in profile; an unknown model is unconfigured (never another model's targets)."""
    try:
        return ENERGY_TARGET_PROFILES[profile]
    except (KeyError, TypeError):
        raise ConfigurationError(f"no energy target profile is configured for {profile!r}") from None


__all__ = ["CodecSpec", "ENERGY_TARGET_PROFILES", "EnergyTargets", "MatrixKey", "ModelIdentity", "RANK_BUCKET",
           "TensorContext", "canonical_digest", "canonical_dtype", "energy_targets"]


def json_copy(value: Any, *, name: str = "metadata") -> Any:
    """A deep copy of a JSON value (dicts, lists, strings, finite numbers, booleans, None); anything
    else is a ConfigurationError naming ``name``."""
    try:
        return json.loads(json.dumps(value, allow_nan=False))
    except (TypeError, ValueError) as error:
        raise ConfigurationError(f"{name} must be JSON data") from error


@dataclass(frozen=True)
class EncodedTensor:
    """An encoded packet: JSON ``metadata``, named byte ``payloads``, optionally the FP16 ``basis``
    bytes of a single-matrix packet and JSON ``metrics`` (reelcache/types.py:349-371)."""

    metadata: Mapping[str, Any]
    payloads: Mapping[str, bytes]
    basis: bytes | None = None
    metrics: Mapping[str, Any] | None = None

    def __post_init__(self) -> None:
        if not isinstance(self.metadata, Mapping) or not isinstance(self.payloads, Mapping):
            raise ConfigurationError("encoded metadata and payloads must be mappings")
        if not self.payloads:
            raise ConfigurationError("encoded tensors require at least one payload")
        for name, payload in self.payloads.items():
            _nonempty(name, "payload name")
            if not isinstance(payload, bytes):
                raise ConfigurationError("encoded payloads must be immutable bytes")
        if self.basis is not None and not isinstance(self.basis, bytes):
            raise ConfigurationError("encoded basis must be immutable bytes")
        if self.metrics is not None and not isinstance(self.metrics, Mapping):
            raise ConfigurationError("metrics must be a mapping")
        object.__setattr__(self, "metadata", json_copy(self.metadata))
        object.__setattr__(self, "payloads", MappingProxyType(dict(self.payloads)))
        if self.metrics is not None:
            object.__setattr__(self, "metrics", json_copy(self.metrics, name="metrics"))
