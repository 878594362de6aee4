"""Immutable basis versions: FP16 row blocks and version manifests in a content-addressed store.

Contract of ``reelcache/basis_versions.py`` (``rows_to_bytes`` / ``rows_from_bytes`` :55-70,
``BasisVersionStore`` :73-403, ``detach_basis`` / ``attach_basis`` :406-432) and of the
``BasisVersion`` record (reelcache/types.py:663-750), in the formats the reference stores:

* a row block is the contiguous little-endian FP16 bytes of ``[rows, channels]``, stored as the
  object ``basis:<sha256>``;
* a version is the manifest ``{"type": "basis_version", "version": 1, "record": ...}`` with the
  record's ``reelcache.basis_version.v1`` fields, referencing its row block and its parent; its
  canonical view is the parent's rows followed by its own, bound by ``view_sha256``;
* manifests are canonical JSON ``{"format": "reelcache.manifest.v1", "references": [...],
  "data": ...}`` stored as ``manifest:<sha256>``.

The reference keeps objects in its SQLite/file store, which is outside the restore path; here
:class:`MemoryObjectStore` holds them in process memory with the same addressing (any object
with ``put`` / ``get`` / ``object_size`` / ``put_manifest`` / ``get_manifest_with_references``
and ``verify_reads`` serves).  The restore path reads versions through :meth:`BasisVersionStore.
assemble` (the history gather's :class:`~reelcache_amd.archive_restore.DeviceBasisCache` uploads
each chain tip once and serves every ancestor as a prefix view).

Design: a version's chain is validated once and cached; block bytes are hashed against their
address on read (unless the store verifies reads itself); assembling a prefix copies only the
blocks it needs into one NumPy buffer; an extension's view digest continues the parent's SHA-256
state when this process wrote the parent.
"""

from __future__ import annotations

import hashlib
import json
import re
import sys
from collections import OrderedDict
from dataclasses import dataclass
from typing import Any, Iterable, Mapping

import numpy as np
import torch

from ._checks import need
from .errors import CapacityError, ConfigurationError, IntegrityError
from .types import EncodedTensor, MatrixKey, ModelIdentity, canonical_digest, json_copy

MANIFEST_TYPE = "basis_version"
RECORD_SCHEMA = "reelcache.basis_version.v1"
MANIFEST_FORMAT = "reelcache.manifest.v1"
#: Domain of each target's basis rows (the spaces the reference fits K and V in).
BASIS_DOMAINS = {"K": "normalized_pre_rope_k", "V": "direct_v"}
_EXPONENT_BITS = 0x7C00  # FP16 exponent field: all ones encode Inf / NaN
_REF = re.compile(r"^(blob|basis|manifest):[0-9a-f]{64}$")
_HEX64 = re.compile(r"^[0-9a-f]{64}$")


def _little_endian():
    need(sys.byteorder == "little", "basis row serialization requires a little-endian host")


def _finite_fp16(data) -> bool:
    # A value is inf / nan when its exponent bits are all ones, i.e. when its magnitude bits are
    # at least the exponent mask: one masked maximum decides for the whole block.
    bits = np.frombuffer(data, dtype=np.uint16)
    return bits.size == 0 or int((bits & np.uint16(0x7FFF)).max()) < int(_EXPONENT_BITS)


def rows_to_bytes(rows: torch.Tensor) -> bytes:
    """Row-major little-endian FP16 bytes of a nonempty finite ``[rows, channels]`` tensor."""
    need(isinstance(rows, torch.Tensor) and rows.dtype == torch.float16 and rows.ndim == 2 and min(rows.shape) >= 1,
         "basis row blocks are nonempty FP16 [rows, channels] tensors")
    data = rows.detach().to("cpu").contiguous().numpy().tobytes()
    need(_finite_fp16(data), "basis row blocks must be finite")
    _little_endian()
    return data


def rows_from_bytes(data: bytes, rows: int, channels: int) -> torch.Tensor:
    """A writable FP16 ``[rows, channels]`` tensor of its own from :func:`rows_to_bytes` bytes."""
    need(isinstance(data, (bytes, bytearray)) and len(data) == 2 * rows * channels,
         "basis row block length disagrees with its declared geometry", IntegrityError)
    return torch.from_numpy(np.frombuffer(data, dtype=np.float16).reshape(rows, channels).copy())


def _canonical(value) -> bytes:
    """Manifest bytes: sorted keys, no whitespace, no NaN, and non-ASCII text as raw UTF-8 (not
    ``\\u`` escapes), as the reference store writes them (reelcache/serialization.py:31-34)."""
    return json.dumps(value, sort_keys=True, separators=(",", ":"), ensure_ascii=False,
                      allow_nan=False).encode("utf-8")


def object_ref(value: Any, name: str, *, kinds: tuple = ("manifest",)) -> str:
    """``value`` when it is a ``kind:<sha256>`` reference of one of ``kinds``."""
    need(isinstance(value, str) and _REF.fullmatch(value) is not None and value.split(":", 1)[0] in kinds,
         f"{name} must be an immutable {'/'.join(kinds)} object reference")
    return value


class MemoryObjectStore:
    """Content-addressed objects and manifests in process memory (the reference store's addressing:
    ``kind:<sha256 of the bytes>``; manifests canonical JSON with sorted references).
    ``verify_reads``: re-hash every object read."""

    def __init__(self, *, verify_reads: bool = False):
        need(type(verify_reads) is bool, "verify_reads must be boolean")
        self.verify_reads = verify_reads
        self._objects: dict[str, bytes] = {}
        self.reads = 0

    def _store(self, data: bytes, kind: str) -> str:
        ref = f"{kind}:{hashlib.sha256(data).hexdigest()}"
        self._objects.setdefault(ref, bytes(data))
        return ref

    def put(self, data: bytes, *, kind: str = "blob") -> str:
        need(kind != "manifest", "use put_manifest to register manifest references")
        need(isinstance(data, (bytes, bytearray)), "stored objects are bytes")
        return self._store(data, kind)

    def put_manifest(self, data: Mapping[str, Any], *, references: Iterable[str] = ()) -> str:
        need(isinstance(data, Mapping), "manifest data must be a JSON mapping")
        references = sorted(set(references))
        for reference in references:
            need(reference in self._objects, f"manifest reference {reference} is not stored", IntegrityError)
        return self._store(_canonical({"format": MANIFEST_FORMAT, "references": references, "data": json_copy(data)}),
                           "manifest")

    def get(self, ref: str) -> bytes:
        data = self._objects.get(ref)
        need(data is not None, f"object {ref} is not stored", IntegrityError)
        self.reads += 1
        if self.verify_reads:
            need(hashlib.sha256(data).hexdigest() == ref.split(":", 1)[1], "stored object differs from its address",
                 IntegrityError)
        return data

    def object_size(self, ref: str) -> int:
        data = self._objects.get(ref)
        need(data is not None, f"object {ref} is not stored", IntegrityError)
        return len(data)

    def get_manifest_with_references(self, ref: str) -> tuple[dict[str, Any], tuple[str, ...]]:
        need(isinstance(ref, str) and ref.startswith("manifest:"), "expected a manifest object", IntegrityError)
        value = json.loads(self.get(ref))
        need(isinstance(value, dict) and set(value) == {"format", "references", "data"}
             and value["format"] == MANIFEST_FORMAT and isinstance(value["data"], dict),
             "invalid manifest", IntegrityError)
        return value["data"], tuple(value["references"])


@dataclass(frozen=True)
class BasisVersion:
    """One immutable node of a per-(layer, target) basis DAG: its newly added FP16 row block and its
    parent; the canonical view is the parent's rows followed by the added rows."""

    parent_ref: str | None
    added_rows_ref: str
    added_rank: int
    total_rank: int
    channels: int
    group_id: str
    key: MatrixKey
    model_fingerprint: str
    depth: int
    view_sha256: str
    dtype: str = "float16"

    def __post_init__(self):
        if self.parent_ref is not None:
            object_ref(self.parent_ref, "basis parent version")
        object_ref(self.added_rows_ref, "added basis row block", kinds=("basis",))
        for name in ("added_rank", "total_rank", "channels"):
            need(type(getattr(self, name)) is int and getattr(self, name) >= 1, f"{name} must be a positive integer")
        need(type(self.depth) is int and self.depth >= 0, "basis version depth must be a nonnegative integer")
        need(isinstance(self.key, MatrixKey), "basis version key must be a MatrixKey")
        need(isinstance(self.model_fingerprint, str) and self.model_fingerprint.strip(),
             "basis model fingerprint must be a nonempty string")
        for name in ("group_id", "view_sha256"):
            need(isinstance(getattr(self, name), str) and _HEX64.fullmatch(getattr(self, name)) is not None,
                 f"{name} must be a lowercase SHA256 hex digest")
        need(self.dtype == "float16", "stored basis rows are FP16")
        need(self.total_rank <= self.channels, "basis rank cannot exceed its channel count")
        root = self.parent_ref is None
        need(root == (self.depth == 0), "only a depth-zero root version has no parent")
        need(not root or self.total_rank == self.added_rank, "a root version's total rank equals its block rank")
        need(root or self.total_rank > self.added_rank, "an extension version must add rows to a nonempty parent")

    @property
    def domain(self) -> str:
        return BASIS_DOMAINS[self.key.target]

    @property
    def parent_rank(self) -> int:
        return self.total_rank - self.added_rank

    @property
    def added_bytes(self) -> int:
        return 2 * self.added_rank * self.channels

    @staticmethod
    def root_group_id(model_fingerprint: str, key: MatrixKey, rows_ref: str) -> str:
        return canonical_digest({"model": model_fingerprint, "key": key.to_dict(), "root_rows": rows_ref})

    def to_dict(self) -> dict[str, Any]:
        return {"schema": RECORD_SCHEMA, "parent": self.parent_ref, "added_rows": self.added_rows_ref,
                "added_rank": self.added_rank, "total_rank": self.total_rank, "channels": self.channels,
                "dtype": self.dtype, "group_id": self.group_id, "key": self.key.to_dict(), "domain": self.domain,
                "model_fingerprint": self.model_fingerprint, "depth": self.depth, "view_sha256": self.view_sha256}

    @classmethod
    def from_dict(cls, data: Mapping[str, Any]) -> "BasisVersion":
        try:
            fields = dict(data)
            need(fields.pop("schema") == RECORD_SCHEMA, "unsupported basis version schema")
            domain = fields.pop("domain")
            version = cls(parent_ref=fields.pop("parent"), added_rows_ref=fields.pop("added_rows"),
                          key=MatrixKey.from_dict(fields.pop("key")), **fields)
        except (KeyError, TypeError) as error:
            raise ConfigurationError("invalid basis version fields") from error
        need(domain == version.domain, "basis version domain disagrees with its target")
        return version


class BasisVersionStore:
    """Validated basis-version operations over one object store for one model (see the module
    docstring).  Parsed versions, blocks found finite and the SHA-256 states of views written by
    this process are cached by their immutable references."""

    #: Bound of the view-digest states kept for extensions.
    VIEW_DIGESTS = 16384

    def __init__(self, store, model: ModelIdentity):
        need(isinstance(model, ModelIdentity), "basis versions require a ModelIdentity")
        need(all(hasattr(store, name) for name in ("put", "get", "object_size", "put_manifest",
                                                   "get_manifest_with_references")),
             "basis versions require an object store")
        self.store, self.model = store, model
        self._versions: dict[str, BasisVersion] = {}
        self._finite: set[str] = set()
        self._digests: OrderedDict[str, Any] = OrderedDict()

    def drop_caches(self) -> None:
        self._versions.clear()
        self._finite.clear()
        self._digests.clear()

    # -- writing ----------------------------------------------------------------------------------
    def _rows(self, key: MatrixKey, rows: torch.Tensor) -> bytes:
        need(isinstance(key, MatrixKey) and key.layer < self.model.layers, "basis key is outside the model")
        need(isinstance(rows, torch.Tensor) and rows.ndim == 2 and rows.shape[1] == self.model.channels_for(key),
             "basis rows do not match the model's channel width")
        return rows_to_bytes(rows)

    def _record(self, version: BasisVersion, digest) -> str:
        references = [version.added_rows_ref] + ([] if version.parent_ref is None else [version.parent_ref])
        ref = self.store.put_manifest({"type": MANIFEST_TYPE, "version": 1, "record": version.to_dict()},
                                      references=references)
        self._versions[ref] = version
        self._digests[ref] = digest
        self._digests.move_to_end(ref)
        while len(self._digests) > self.VIEW_DIGESTS:
            self._digests.popitem(last=False)
        return ref

    def put_root(self, key: MatrixKey, rows: torch.Tensor) -> tuple[str, BasisVersion]:
        """Store a new group's first block and its depth-zero version."""
        data = self._rows(key, rows)
        block = self.store.put(data, kind="basis")
        digest = hashlib.sha256(data)
        count = int(rows.shape[0])
        version = BasisVersion(None, block, count, count, int(rows.shape[1]),
                               BasisVersion.root_group_id(self.model.fingerprint, key, block), key,
                               self.model.fingerprint, 0, digest.hexdigest())
        return self._record(version, digest), version

    def put_extension(self, parent_ref: str, rows: torch.Tensor) -> tuple[str, BasisVersion]:
        """Append an immutable row block to ``parent_ref`` (the parent is not modified)."""
        parent = self.load(parent_ref)
        data = self._rows(parent.key, rows)
        count = int(rows.shape[0])
        need(parent.total_rank + count <= parent.channels, "an extension cannot exceed the channel count")
        state = self._digests.get(parent_ref)
        digest = state.copy() if state is not None else hashlib.sha256(self.view_bytes(parent_ref))
        digest.update(data)
        block = self.store.put(data, kind="basis")
        version = BasisVersion(parent_ref, block, count, parent.total_rank + count, parent.channels, parent.group_id,
                               parent.key, parent.model_fingerprint, parent.depth + 1, digest.hexdigest())
        return self._record(version, digest), version

    # -- reading ----------------------------------------------------------------------------------
    def load(self, ref: str) -> BasisVersion:
        """One version after validating it and (once, cached) its whole parent chain."""
        object_ref(ref, "basis version")
        walk = []  # (reference, version) from ``ref`` up to the first validated ancestor or the root
        current = ref
        while current is not None and current not in self._versions:
            version = self._parse(current)
            walk.append((current, version))
            current = version.parent_ref
        for item, version in reversed(walk):  # parents first: each links to a validated parent
            self._link(version)
            self._versions[item] = version
        return self._versions[ref]

    def _parse(self, ref: str) -> BasisVersion:
        data, references = self.store.get_manifest_with_references(ref)
        try:
            need(data.get("type") == MANIFEST_TYPE and data.get("version") == 1 and set(data) == {
                "type", "version", "record"}, "unsupported basis version manifest", IntegrityError)
            version = BasisVersion.from_dict(data["record"])
        except (ConfigurationError, TypeError, AttributeError) as error:
            raise IntegrityError("invalid basis version manifest") from error
        expected = sorted({version.added_rows_ref} | ({version.parent_ref} if version.parent_ref else set()))
        need(list(references) == expected, "basis version references disagree with its parent/block", IntegrityError)
        need(version.model_fingerprint == self.model.fingerprint and version.key.layer < self.model.layers,
             "basis version belongs to another model", IntegrityError)
        need(version.channels == self.model.channels_for(version.key),
             "basis version channel width disagrees with the model", IntegrityError)
        need(self.store.object_size(version.added_rows_ref) == version.added_bytes,
             "basis row block size disagrees with its version", IntegrityError)
        return version

    def _link(self, version: BasisVersion) -> None:
        if version.parent_ref is None:
            need(version.group_id == BasisVersion.root_group_id(version.model_fingerprint, version.key,
                                                                version.added_rows_ref),
                 "root basis group identity is not bound to its first block", IntegrityError)
            return
        parent = self._versions[version.parent_ref]
        consistent = (parent.total_rank + version.added_rank == version.total_rank
                      and parent.depth + 1 == version.depth
                      and (parent.channels, parent.key, parent.group_id, parent.model_fingerprint)
                      == (version.channels, version.key, version.group_id, version.model_fingerprint))
        need(consistent, "basis extension is inconsistent with its parent version", IntegrityError)

    def chain(self, ref: str) -> list[tuple[str, BasisVersion]]:
        """``(reference, version)`` from the group root to ``ref`` (inclusive)."""
        links = []
        while ref is not None:
            version = self.load(ref)
            links.append((ref, version))
            ref = version.parent_ref
        return links[::-1]

    def chain_refs(self, ref: str) -> list[str]:
        return [item for item, _ in self.chain(ref)]

    def total_rank(self, ref: str) -> int:
        return self.load(ref).total_rank

    def blocks(self, ref: str) -> tuple[str, ...]:
        return tuple(version.added_rows_ref for _, version in self.chain(ref))

    def _prefix(self, ref, rows, max_bytes, block_cache):
        """``(version, rows, [(block, bytes taken)])`` of a legal prefix, blocks checked against their
        addresses; the full view also against ``view_sha256`` (unless the store verifies reads)."""
        version = self.load(ref)
        rows = version.total_rank if rows is None else rows
        need(type(rows) is int and 1 <= rows <= version.total_rank,
             "a basis view must be a nonempty legal prefix of its version")
        nbytes = 2 * rows * version.channels
        if max_bytes is not None and nbytes > max_bytes:
            raise CapacityError(f"basis view needs {nbytes} bytes; workspace bound is {max_bytes}")
        verified = bool(getattr(self.store, "verify_reads", False))
        digest = hashlib.sha256() if rows == version.total_rank and not verified else None
        parts, remaining = [], rows
        for _, link in self.chain(ref):
            if remaining <= 0:
                break
            block = link.added_rows_ref
            data = None if block_cache is None else block_cache.get(block)
            if data is None:
                data = self.store.get(block)
                need(verified or hashlib.sha256(data).hexdigest() == block.split(":", 1)[1],
                     "basis row block bytes differ from their content address", IntegrityError)
                if block_cache is not None:
                    block_cache[block] = data
            take = 2 * min(link.added_rank, remaining) * version.channels
            need(len(data) >= take, "basis row block length disagrees with its declared geometry", IntegrityError)
            if digest is not None:
                digest.update(memoryview(data)[:take])
            parts.append((block, data, take))
            remaining -= link.added_rank
        need(digest is None or digest.hexdigest() == version.view_sha256,
             "assembled basis view differs from its version digest", IntegrityError)
        return version, rows, parts

    def assemble(self, ref: str, rows: int | None = None, *, max_bytes: int | None = None,
                 block_cache: dict | None = None) -> torch.Tensor:
        """Contiguous FP16 prefix view ``[rows, channels]`` (host) of the version's blocks; only the
        blocks the prefix needs are read.  ``block_cache`` (caller-owned) keeps checked blocks."""
        version, rows, parts = self._prefix(ref, rows, max_bytes, block_cache)
        view = np.empty(2 * rows * version.channels, dtype=np.uint8)
        at = 0
        for _, data, take in parts:
            view[at:at + take] = np.frombuffer(data, dtype=np.uint8, count=take)
            at += take
        return torch.from_numpy(view.view(np.float16).reshape(rows, version.channels))

    def view_bytes(self, ref: str, rows: int | None = None, *, max_bytes: int | None = None,
                   block_cache: dict | None = None) -> bytes:
        """``rows_to_bytes(assemble(...))`` without tensors; finiteness checked per block (memoized
        for blocks entirely finite)."""
        _little_endian()
        _, _, parts = self._prefix(ref, rows, max_bytes, block_cache)
        chunks = []
        for block, data, take in parts:
            piece = memoryview(data)[:take]
            if block not in self._finite:
                if _finite_fp16(data):
                    self._finite.add(block)
                else:
                    need(_finite_fp16(piece), "basis row blocks must be finite")
            chunks.append(piece)
        return b"".join(chunks)

    def unique_block_bytes(self, refs: Iterable[str]) -> dict[str, int]:
        """Each referenced row block once, with its stored size."""
        sizes: dict[str, int] = {}
        for ref in refs:
            if ref is not None:
                for _, version in self.chain(ref):
                    sizes.setdefault(version.added_rows_ref, version.added_bytes)
        return sizes


def detach_basis(encoded: EncodedTensor):
    """``(metadata, payloads, metrics)`` of a prepared lossy single-matrix packet, its basis bytes
    dropped after checking them against the packet's basis descriptor (kept verbatim)."""
    need(isinstance(encoded, EncodedTensor) and encoded.basis is not None,
         "only lossy single-matrix packets carry a detachable basis")
    descriptor = encoded.metadata.get("basis")
    need(isinstance(descriptor, Mapping) and hashlib.sha256(encoded.basis).hexdigest() == descriptor.get("sha256"),
         "packet basis bytes disagree with their descriptor", IntegrityError)
    metrics = None if encoded.metrics is None else json_copy(encoded.metrics, name="metrics")
    return json_copy(encoded.metadata), dict(encoded.payloads), metrics


def attach_basis(metadata: Mapping[str, Any], payloads: Mapping[str, bytes], basis: bytes, *, rank_view: int,
                 channels: int, check_digest: bool = True) -> EncodedTensor:
    """Re-attach an assembled prefix view after checking it against the packet's descriptor
    (shape, view rank, dtype, length and -- unless ``check_digest`` is False -- SHA-256)."""
    descriptor = metadata.get("basis") if isinstance(metadata, Mapping) else None
    bound = (isinstance(descriptor, Mapping) and descriptor.get("shape") == [rank_view, channels]
             and descriptor.get("view_rank") == rank_view and descriptor.get("dtype") == "float16"
             and descriptor.get("bytes") == len(basis)
             and (not check_digest or hashlib.sha256(basis).hexdigest() == descriptor.get("sha256")))
    need(bound, "assembled basis view differs from the packet's bound prefix", IntegrityError)
    return EncodedTensor(metadata, payloads, basis=basis)


__all__ = ["BASIS_DOMAINS", "BasisVersion", "BasisVersionStore", "MANIFEST_TYPE", "MemoryObjectStore", "attach_basis",
           "detach_basis", "object_ref", "rows_from_bytes", "rows_to_bytes"]
