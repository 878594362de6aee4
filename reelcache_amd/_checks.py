"""Argument checks shared by the contract types of the restore and fit paths.

Every failed check raises :class:`~reelcache_amd.errors.ConfigurationError` (or the error class
given) with a message naming the argument.  The checks are small composable functions so that a
type's ``__post_init__`` reads as a list of rules.
"""

from __future__ import annotations

import math
from typing import Any

import numpy as np
import torch

from .errors import ConfigurationError


def need(condition: Any, message: str, error: type = ConfigurationError) -> None:
    """Raise ``error(message)`` unless ``condition`` holds."""
    if not condition:
        raise error(message)


def count(value: Any, name: str, minimum: int = 0) -> int:
    """An exact ``int`` (not ``bool``) of at least ``minimum``."""
    need(type(value) is int and value >= minimum, f"{name} must be an integer >= {minimum}")
    return value


def strided(value: Any, name: str) -> torch.Tensor:
    """A strided tensor with real storage (no sparse layouts, no meta tensors)."""
    need(isinstance(value, torch.Tensor) and value.layout == torch.strided, f"{name} must be a strided torch.Tensor")
    need(value.device.type != "meta", f"{name} cannot be a meta tensor")
    return value


def matrix(value: Any, name: str, dtypes: tuple, what: str) -> torch.Tensor:
    """A strided 2-D tensor of one of ``dtypes``; ``what`` describes the accepted form."""
    value = strided(value, name)
    need(value.ndim == 2 and value.dtype in dtypes, f"{name} must be {what}")
    return value


def bound(value: Any, name: str) -> float | None:
    """``None`` or a finite nonnegative real number (``bool`` excluded)."""
    if value is None:
        return None
    need(not isinstance(value, bool) and isinstance(value, (int, float)) and math.isfinite(value) and value >= 0,
         f"{name} must be a finite nonnegative upper bound")
    return value


def host_floats(value: Any, length: int, name: str) -> np.ndarray:
    """A read-only finite float32 host copy of a vector of ``length`` entries (the caller's array
    can change afterwards without changing what the holder of the copy reads)."""
    if isinstance(value, torch.Tensor):
        need(value.device.type == "cpu", f"{name} must be a host array; pass the packet affine payload")
        value = value.detach().numpy()
    array = np.asarray(value)
    need(array.dtype == np.float32 and array.shape == (length,),
         f"{name} must be a float32 vector with one entry per rank column")
    need(np.isfinite(array).all(), f"{name} must be finite")
    copy = np.array(array, dtype=np.float32, copy=True, order="C")
    copy.flags.writeable = False
    return copy


def one_of(value: Any, choices: tuple, name: str) -> Any:
    need(value in choices, f"{name} must be one of {choices}")
    return value
