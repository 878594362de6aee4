"""CPU tests of the history gather (``reelcache_amd.archive_restore``): basis version chains,
the device basis cache's prefix hits / longest-first uploads / absorption / LRU eviction /
pins (reelcache/archive_restore.py:72-423), and the job gather of a forked history
(reelcache/packed_decode.py:620-636), restored through the CPU reference backend.
"""

import numpy as np
import pytest
import torch

from oracle import restore as orc
from reelcache_amd import archive_restore as ar
from reelcache_amd import restore_kernels as rk
from reelcache_amd.errors import CapacityError, ConfigurationError, IntegrityError, StateError


def _rows(rng, count, channels=16):
    return torch.from_numpy(rng.standard_normal((count, channels)).astype(np.float16))


def _tree(rng, channels=16):
    versions = ar.BasisVersions()
    versions.add("v0", None, _rows(rng, 8, channels))
    versions.add("v1", "v0", _rows(rng, 4, channels))
    versions.add("v2", "v1", _rows(rng, 4, channels))
    versions.add("v1b", "v0", _rows(rng, 2, channels))  # a fork off v0
    return versions


def test_version_chains_append_rows():
    versions = _tree(np.random.default_rng(0))
    assert versions.chain("v2") == ["v0", "v1", "v2"] and versions.chain("v1b") == ["v0", "v1b"]
    assert versions.total_rank("v2") == 16 and versions.total_rank("v1b") == 10
    full = versions.assemble("v2")
    assert torch.equal(full[:12], versions.assemble("v1")) and torch.equal(full[:8], versions.assemble("v0"))
    with pytest.raises(IntegrityError):
        versions.add("v9", "missing", _rows(np.random.default_rng(1), 2))
    with pytest.raises(ConfigurationError):
        versions.add("v0", None, _rows(np.random.default_rng(1), 2))


def test_cache_uploads_longest_first_and_serves_prefixes():
    versions = _tree(np.random.default_rng(2))
    cache = ar.DeviceBasisCache(versions, "cpu", 1 << 20)
    views, tokens = cache.acquire_many([("v0", 8), ("v2", 13), ("v1", 12), ("v1b", 10), ("v0", 5)])
    stats = cache.stats()
    assert stats["uploads"] == 2 and stats["misses"] == 4  # v2 serves v0 and v1; v1b has its own tip
    assert tokens[0] == tokens[1] == tokens[2] == "v2" and tokens[3] == "v1b"
    assert torch.equal(views[1], versions.assemble("v2")[:13])
    assert views[0].data_ptr() == views[2].data_ptr() == views[4].data_ptr()  # prefixes of one tip
    for token in tokens:
        cache.release(token)
    with pytest.raises(StateError):
        cache.release("v2")
    again, tokens = cache.acquire_many([("v1", 3)])
    assert cache.stats()["prefix_hits"] == 1 and tokens == ["v2"]
    cache.release(tokens[0])


def test_cache_absorbs_ancestors_and_evicts_lru():
    rng = np.random.default_rng(3)
    versions = _tree(rng)
    cache = ar.DeviceBasisCache(versions, "cpu", 1 << 20)
    _, tokens = cache.acquire_many([("v0", 8)])
    cache.release(tokens[0])
    _, tokens = cache.acquire_many([("v2", 16)])
    assert cache.stats()["absorbed"] == 1 and cache.stats()["versions"] == 1
    cache.release(tokens[0])
    row_bytes = 16 * 2
    small = ar.DeviceBasisCache(versions, "cpu", 17 * row_bytes)  # room for v2 (16 rows) or v1b (10), not both
    _, tokens = small.acquire_many([("v2", 16)])
    with pytest.raises(CapacityError):
        small.acquire_many([("v1b", 10)])  # v2 is pinned
    small.release(tokens[0])
    _, tokens = small.acquire_many([("v1b", 10)])
    assert small.stats()["evictions"] == 1 and tokens == ["v1b"]
    small.release(tokens[0])
    with pytest.raises(CapacityError):
        ar.DeviceBasisCache(versions, "cpu", 8).acquire("v0", 8)
    with pytest.raises(IntegrityError):
        cache.acquire("v1b", 11)


def test_history_gather_restores_each_node_into_its_range():
    rng = np.random.default_rng(4)
    heads, head_dim = 2, 8
    channels = heads * head_dim
    versions = _tree(rng, channels)
    cache_rows = ar.DeviceBasisCache(versions, "cpu", 1 << 20)
    grid = (1, 2, 3)
    tokens = 6
    nodes, expected = [], {}
    refs = ["v0", "v1", "v2", "v1b", "v2"]
    for index, ref in enumerate(refs):
        matrices = {}
        for target in ("K", "V"):
            rank = int(rng.integers(2, versions.total_rank(ref) + 1))
            codes = torch.from_numpy(rng.integers(0, 256, size=(tokens, rank), dtype=np.uint8))
            scale = rng.uniform(0.01, 0.1, size=rank).astype(np.float32)
            offset = rng.uniform(-1, 0, size=rank).astype(np.float32)
            matrices[(0, target)] = ar.NodeMatrix(codes, scale, offset, ref, rank)
            basis = versions.assemble(ref)[:rank].numpy().astype(np.float64)
            expected[(index, target)] = orc.dequantize(codes.numpy(), scale, offset).astype(np.float64) @ basis
        nodes.append(ar.HistoryNode(f"n{index}", index * tokens, grid, matrices))
    caches = {target: torch.zeros((1, tokens * len(refs), heads, head_dim), dtype=torch.float32)
              for target in ("K", "V")}
    order = [nodes[i] for i in rng.permutation(len(nodes))]  # gather order of a fork path
    jobs, pins = ar.history_jobs(order, 0, caches, cache_rows)
    assert len(jobs) == 2 * len(nodes) and cache_rows.stats()["uploads"] == 2
    rk.reconstruct(jobs)  # host tensors: the CPU reference backend
    for token in pins:
        cache_rows.release(token)
    for (index, target), values in expected.items():
        written = caches[target][0, index * tokens:(index + 1) * tokens].reshape(tokens, channels).numpy()
        np.testing.assert_allclose(written, values.astype(np.float32), rtol=1e-6, atol=1e-6)


def test_batch_uploads_cannot_evict_each_other():
    """A budget that holds one tip but not two: the second upload of one acquire_many call must
    not evict the first (held by the batch), so the call fails with CapacityError and leaves no
    pin behind (reelcache/archive_restore.py:174-175)."""
    rng = np.random.default_rng(5)
    versions = ar.BasisVersions()
    versions.add("a", None, _rows(rng, 8))
    versions.add("b", None, _rows(rng, 6))  # a second root: no prefix sharing
    one_tip = 8 * 16 * 2
    cache = ar.DeviceBasisCache(versions, "cpu", one_tip + 16)
    with pytest.raises(CapacityError):
        cache.acquire_many([("a", 4), ("b", 3)])
    stats = cache.stats()
    assert stats["pinned"] == 0
    # Each alone fits, and nothing leaked: both can be acquired and released in turn.
    view, token = cache.acquire("b", 3)
    assert tuple(view.shape) == (3, 16)
    cache.release(token)
    view, token = cache.acquire("a", 8)
    cache.release(token)
    assert cache.stats()["pinned"] == 0
