"""Typed failures of the restore and fit paths.

The class names and bases are those callers of ``reelcache.errors`` catch
(reelcache/errors.py:4-33), so code written against the reference handles
these exceptions unchanged.
"""


class ReelCacheError(Exception):
    """Base class of every declared failure."""


class ConfigurationError(ReelCacheError, ValueError):
    """Invalid or incompatible arguments, layouts or identities."""


class IntegrityError(ReelCacheError):
    """Data is corrupt, missing or internally inconsistent."""


class CapacityError(ReelCacheError):
    """A bounded resource cannot admit the request."""


class StateError(ReelCacheError):
    """The operation is invalid in the current state (e.g. the wrong owner thread)."""


class UnsupportedError(ReelCacheError):
    """A requested backend, precision or capability is unavailable (never a silent fallback)."""


__all__ = ["CapacityError", "ConfigurationError", "IntegrityError", "ReelCacheError", "StateError",
           "UnsupportedError"]
