"""CPU tests of the basis-version store (reelcache/basis_versions.py:55-432, the BasisVersion
record of reelcache/types.py:663-750).

Row serialization follows the reference's own tests (tests/test_step7_cpu_pool.py:90-135): the
bytes of every finite FP16 bit pattern are those patterns (little-endian), non-finite values,
wrong dtypes, shapes and empty blocks are refused with the reference's messages, and bad
lengths are integrity errors.  The store keeps the reference's addressing (``basis:<sha256>``
blocks, canonical-JSON ``manifest:<sha256>`` versions), assembles every prefix of a version chain
equal to the rows it was built from, binds the full view to ``view_sha256`` and refuses
tampered blocks, foreign models and inconsistent chains.
"""

import hashlib
import json

import numpy as np
import pytest
import torch

from reelcache_amd import basis_versions as bv
from reelcache_amd.errors import CapacityError, ConfigurationError, IntegrityError
from reelcache_amd.types import EncodedTensor, MatrixKey, ModelIdentity, canonical_digest

MODEL = ModelIdentity("versions-test", "c" * 64, 3, {"K": 48, "V": 64}, "THD", "bfloat16")


def _rows(rng, count, channels):
    return torch.from_numpy(rng.standard_normal((count, channels))).to(torch.float16)


def test_row_bytes_are_the_fp16_bit_patterns():
    bits = np.arange(1 << 16, dtype=np.uint16)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    rows = torch.from_numpy(finite.view(np.float16).copy()).reshape(-1, 1)
    data = bv.rows_to_bytes(rows)
    assert data == finite.astype("<u2").tobytes()
    restored = bv.rows_from_bytes(data, rows.shape[0], 1)
    assert torch.equal(restored.view(torch.int16), rows.view(torch.int16))
    restored[0, 0] = 1  # a writable tensor of its own
    transposed = _rows(np.random.default_rng(1), 6, 5).t()
    assert bv.rows_to_bytes(transposed) == transposed.contiguous().numpy().tobytes()


def test_row_bytes_rejections():
    for value in (torch.zeros(2, 2), torch.zeros(4, dtype=torch.float16), torch.zeros(0, 3, dtype=torch.float16),
                  "rows"):
        with pytest.raises(ConfigurationError, match="nonempty FP16"):
            bv.rows_to_bytes(value)
    for special in (float("inf"), float("-inf"), float("nan")):
        value = _rows(np.random.default_rng(2), 4, 8)
        value[3, 7] = special
        with pytest.raises(ConfigurationError, match="must be finite"):
            bv.rows_to_bytes(value)
    for data, count, channels in ((b"\x00" * 6, 2, 2), ("text", 1, 1), (b"\x00" * 10, 2, 2)):
        with pytest.raises(IntegrityError):
            bv.rows_from_bytes(data, count, channels)


def test_chain_prefixes_and_addressing():
    rng = np.random.default_rng(3)
    store = bv.MemoryObjectStore()
    versions = bv.BasisVersionStore(store, MODEL)
    key = MatrixKey(1, "V")
    blocks = [_rows(rng, 5, 64), _rows(rng, 3, 64), _rows(rng, 4, 64)]
    root, first = versions.put_root(key, blocks[0])
    mid, _ = versions.put_extension(root, blocks[1])
    tip, last = versions.put_extension(mid, blocks[2])
    fork, _ = versions.put_extension(root, _rows(rng, 2, 64))
    full = torch.cat(blocks)
    assert first.added_rows_ref == "basis:" + hashlib.sha256(bv.rows_to_bytes(blocks[0])).hexdigest()
    assert first.group_id == canonical_digest({"model": MODEL.fingerprint, "key": key.to_dict(),
                                               "root_rows": first.added_rows_ref})
    assert last.view_sha256 == hashlib.sha256(bv.rows_to_bytes(full)).hexdigest()
    assert (last.depth, last.total_rank, last.parent_rank, last.group_id) == (2, 12, 8, first.group_id)
    # The manifest is canonical JSON of the reference's layout, addressed by its SHA-256.
    record, references = store.get_manifest_with_references(tip)
    encoded = json.dumps({"format": "reelcache.manifest.v1", "references": sorted(references), "data": record},
                         sort_keys=True, separators=(",", ":")).encode()
    assert tip == "manifest:" + hashlib.sha256(encoded).hexdigest()
    assert record["record"]["domain"] == "direct_v" and bv.BasisVersion.from_dict(record["record"]) == last
    fresh = bv.BasisVersionStore(store, MODEL)  # validates the chain from the stored objects
    assert fresh.chain_refs(tip) == [root, mid, tip] and fresh.chain_refs(fork) == [root, fork]
    for rows in range(1, 13):
        assert torch.equal(fresh.assemble(tip, rows), full[:rows])
        assert fresh.view_bytes(tip, rows) == bv.rows_to_bytes(full[:rows])
    cache: dict = {}
    fresh.assemble(tip, block_cache=cache)
    reads = store.reads
    fresh.assemble(mid, block_cache=cache)
    assert store.reads == reads and len(cache) == 3  # blocks shared by the chain are read once
    assert fresh.unique_block_bytes([tip, fork]) == {first.added_rows_ref: 640, last.added_rows_ref: 512,
                                                      fresh.load(mid).added_rows_ref: 384,
                                                      fresh.load(fork).added_rows_ref: 256}
    with pytest.raises(CapacityError):
        fresh.assemble(tip, 12, max_bytes=100)
    with pytest.raises(ConfigurationError):
        fresh.assemble(tip, 13)


def test_tampering_and_foreign_versions_are_integrity_errors():
    rng = np.random.default_rng(4)
    store = bv.MemoryObjectStore()
    versions = bv.BasisVersionStore(store, MODEL)
    root, version = versions.put_root(MatrixKey(0, "K"), _rows(rng, 6, 48))
    tip, _ = versions.put_extension(root, _rows(rng, 2, 48))
    store._objects[version.added_rows_ref] = bytes(len(store._objects[version.added_rows_ref]))
    with pytest.raises(IntegrityError):
        bv.BasisVersionStore(store, MODEL).assemble(tip)
    other = ModelIdentity("other", "d" * 64, 3, {"K": 48, "V": 64}, "THD", "bfloat16")
    with pytest.raises(IntegrityError):
        bv.BasisVersionStore(store, other).load(tip)
    with pytest.raises(ConfigurationError):
        versions.put_root(MatrixKey(0, "K"), _rows(rng, 2, 64))  # wrong channel width
    with pytest.raises(ConfigurationError):
        versions.put_extension(root, _rows(rng, 48, 48))  # beyond the channel count


def test_detach_and_attach_single_matrix_basis():
    rows = _rows(np.random.default_rng(7), 4, 48)
    raw = bv.rows_to_bytes(rows)
    metadata = {"basis": {"shape": [4, 48], "view_rank": 4, "dtype": "float16", "bytes": len(raw),
                          "sha256": hashlib.sha256(raw).hexdigest()}}
    encoded = EncodedTensor(metadata, {"coefficients": b"\x01\x02"}, basis=raw, metrics={"x": 1})
    header, payloads, metrics = bv.detach_basis(encoded)
    assert header == metadata and metrics == {"x": 1}
    assert bv.attach_basis(header, payloads, raw, rank_view=4, channels=48).basis == raw
    with pytest.raises(IntegrityError):
        bv.attach_basis(header, payloads, bytes(len(raw)), rank_view=4, channels=48)
    with pytest.raises(IntegrityError):
        bv.attach_basis(header, payloads, raw, rank_view=3, channels=48)


def test_manifests_keep_non_ascii_text_as_utf8():
    """The manifest bytes of a version whose model fingerprint is not ASCII hold the fingerprint's
    UTF-8 bytes, not JSON \\u escapes, so its ``manifest:<sha256>`` address is the reference store's
    (reelcache/serialization.py:31-34 writes ensure_ascii=False)."""
    model = ModelIdentity("versions-test", "modèle-vidéo-ü", 2, {"K": 16, "V": 16}, "THD", "bfloat16")
    store = bv.MemoryObjectStore()
    versions = bv.BasisVersionStore(store, model)
    ref, version = versions.put_root(MatrixKey(0, "K"), _rows(np.random.default_rng(9), 3, 16))
    assert version.model_fingerprint == model.fingerprint
    data = store.get(ref)
    assert model.fingerprint.encode("utf-8") in data and b"\\u00e8" not in data
    # The address is the SHA-256 of exactly those bytes, and re-encoding the parsed record the
    # reference's way gives the same bytes.
    assert ref == "manifest:" + hashlib.sha256(data).hexdigest()
    parsed = json.loads(data.decode("utf-8"))
    assert json.dumps(parsed, sort_keys=True, separators=(",", ":"), ensure_ascii=False,
                      allow_nan=False).encode("utf-8") == data
