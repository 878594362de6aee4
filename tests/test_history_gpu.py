"""GPU test of a fork / rewind restore over basis versions.

A history of 12 CausVid-shape nodes (3 x 30 x 52 tokens, 12 x 128 channels, 30 layers)
references four basis versions per (layer, target): v0 (192 rows), v1 = v0 + 16..64 rows,
v2 = v1 + 16..64 rows and a fork v1b = v0 + 16..64 rows; ranks are ragged in
[64, min(256, version rows)] on the 32-grid.  The nodes are gathered in a seeded random fork
order through the device basis cache (one resident tip per chain, ancestors served as prefixes)
and restored with one call per layer.

The versions come either from the in-memory chain (``BasisVersions``) or from a
``BasisVersionStore`` (content-addressed FP16 row blocks and version manifests, the stored
format), read by the device basis cache through the same interface.

Gather / indexing is checked bit for bit on every layer: the caches equal those of the same
restore given explicit bases built from the test's own rows of each version (not from the
cache's views).  Values of one node per version (v0, v1, the v2 tip and the v1b fork) are
checked against the oracle on the first, a middle and the last layer, both targets
(rel-Frobenius <= 1e-3 against its bf16-cast fp32 reconstruction and the reference's
elementwise bound on a token sample).
"""

import numpy as np
import pytest
import torch

from oracle import restore as orc
from reelcache_amd import archive_restore as ar
from reelcache_amd import basis_versions as bv
from reelcache_amd import restore_kernels as rk
from reelcache_amd.types import MatrixKey, ModelIdentity

from restore_cases import random_affine

pytestmark = pytest.mark.gpu

HEADS, HEAD_DIM, GRID = 12, 128, (3, 30, 52)
TOKENS, CHANNELS = 4680, 1536


def _versions(rng, layers, source="memory"):
    """The product's version source and the test's own rows of every version (root first);
    versions are named by their references (``{layer}{target}:{name}`` in memory, manifest
    references in the store)."""
    if source == "memory":
        versions = ar.BasisVersions()
    else:
        model = ModelIdentity("causvid-history", "a" * 64, layers, CHANNELS, "THD", "bfloat16")
        versions = bv.BasisVersionStore(bv.MemoryObjectStore(), model)
    own, names = {}, {}
    for layer in range(layers):
        for target in ("K", "V"):
            sizes = {"v0": 192, "v1": int(rng.integers(16, 65)), "v2": int(rng.integers(16, 65)),
                     "v1b": int(rng.integers(16, 65))}
            parents = {"v0": None, "v1": "v0", "v2": "v1", "v1b": "v0"}
            total = sum(sizes.values())
            q, _ = np.linalg.qr(rng.standard_normal((CHANNELS, total)))
            rows = torch.from_numpy(q.T.copy()).to(torch.float16)
            start, spans = 0, {}
            for name in ("v0", "v1", "v2", "v1b"):
                block = rows[start:start + sizes[name]]
                parent = None if parents[name] is None else names[f"{layer}{target}:{parents[name]}"]
                if source == "memory":
                    ref = f"{layer}{target}:{name}"
                    versions.add(ref, parent, block)
                elif parent is None:
                    ref, _ = versions.put_root(MatrixKey(layer, target), block)
                else:
                    ref, _ = versions.put_extension(parent, block)
                names[f"{layer}{target}:{name}"] = ref
                spans[name] = (start, start + sizes[name])
                start += sizes[name]
            for name in ("v0", "v1", "v2", "v1b"):
                chain, walk = [], name
                while walk is not None:
                    chain.append(spans[walk])
                    walk = parents[walk]
                own[names[f"{layer}{target}:{name}"]] = torch.cat([rows[a:b] for a, b in reversed(chain)], 0)
    return versions, own, names


def _rank(rng, total):
    high = min(256, total)
    grid = [r for r in range(64, high + 1, 32)]
    return int(rng.choice(grid)) if rng.random() < 0.7 else int(rng.integers(64, high + 1))


LAYERS = 30  # the CausVid shape's layers
VALUE_LAYERS = (0, 15, 29)  # layers whose outputs are also checked against the oracle


@pytest.mark.parametrize("source", ["memory", "store"])
def test_fork_history_gather_is_exact(device, source):
    rng = np.random.default_rng(60)
    versions, own, refs = _versions(rng, LAYERS, source)
    names = ["v0"] * 3 + ["v1"] * 3 + ["v2"] * 3 + ["v1b"] * 3
    nodes = []
    for index, name in enumerate(names):
        matrices = {}
        for layer in range(LAYERS):
            for target in ("K", "V"):
                ref = refs[f"{layer}{target}:{name}"]
                rank = _rank(rng, versions.total_rank(ref))
                codes = torch.randint(0, 256, (TOKENS, rank), dtype=torch.uint8,
                                      generator=torch.Generator().manual_seed(int(rng.integers(1 << 30))))
                scale, offset = random_affine(rank, rng)
                matrices[(layer, target)] = ar.NodeMatrix(codes.to(device), scale, offset, ref, rank)
        nodes.append(ar.HistoryNode(f"n{index}", index * TOKENS, GRID, matrices))
    order = [nodes[i] for i in rng.permutation(len(nodes))]
    table = rk.RopeTable.from_complex(torch.from_numpy(orc.wan_freqs(HEAD_DIM, 64)))
    history = len(nodes) * TOKENS
    cache = ar.DeviceBasisCache(versions, device, 1 << 30)

    def caches():
        return {t: torch.zeros((1, history, HEADS, HEAD_DIM), dtype=torch.bfloat16, device=device) for t in "KV"}

    gathered, explicit = caches(), caches()
    for layer in range(LAYERS):
        for t in "KV":
            gathered[t].zero_()
            explicit[t].zero_()
        jobs, pins = ar.history_jobs(order, layer, gathered, cache, rope_table=table)
        handle = rk.reconstruct(jobs)
        torch.cuda.synchronize(device)  # the pinned basis views are read until the restore completes
        handle.release()
        for token in pins:
            cache.release(token)
        # The same jobs with bases built from the test's own rows of each node's version.
        matrix_of = {f"{node.node_id}:{layer}:{target}": node.matrices[(layer, target)]
                     for node in nodes for target in "KV"}
        copies = []
        for job in jobs:
            matrix = matrix_of[job.label]
            basis = own[matrix.version][:matrix.rank].to(device)
            copies.append(rk.ReconstructionJob(job.source, rk.NativeView(explicit[job.label.split(":")[-1]],
                                                                         token_offset=job.destination.token_offset),
                                               job.grid, basis, job.rank, job.rope, job.label))
        rk.reconstruct(copies).release()
        torch.cuda.synchronize(device)
        for target in "KV":
            assert torch.equal(gathered[target], explicit[target]), (layer, target)
        if layer in VALUE_LAYERS:
            _check_values(nodes, layer, gathered, own, rng)
    stats = cache.stats()
    assert stats["uploads"] == 2 * 2 * LAYERS  # per (layer, target): the v2 chain tip and the v1b fork tip
    assert stats["misses"] == 4 * 2 * LAYERS  # every version missed once, served by its tip thereafter


def _check_values(nodes, layer, gathered, own, rng):
    """Values of one node per version (v0, v1, the v2 tip, the v1b fork) against the oracle."""
    for node in (nodes[i] for i in (0, 3, 6, 9)):
        for target in "KV":
            matrix = node.matrices[(layer, target)]
            basis = own[matrix.version][:matrix.rank].numpy().astype(np.float64)
            coefficients = orc.dequantize(matrix.codes.cpu().numpy(), matrix.scale, matrix.offset)
            rope = None
            if target == "K":
                rope = orc.rope_cos_sin(np.real(orc.wan_freqs(HEAD_DIM, 64)), np.imag(orc.wan_freqs(HEAD_DIM, 64)),
                                        orc.wan_sections(HEAD_DIM // 2), (node.token_start // (30 * 52), 0, 0), GRID)
            values = orc.reconstruct(coefficients, basis, HEADS, rope, compute=np.float32)
            out = gathered[target][0, node.token_start:node.token_start + TOKENS].float().cpu().numpy()
            out = out.reshape(TOKENS, CHANNELS)
            # bf16 cache: compare with the oracle's one bf16 cast of the fp32 reconstruction.
            assert orc.relative_frobenius(out, orc.cast(values, "bfloat16")) <= 1e-3, (layer, node.node_id, target)
            sample = rng.choice(TOKENS, size=128, replace=False)
            exact, bound = orc.error_bound(coefficients[sample], basis, HEADS,
                                           None if rope is None else (rope[0][sample], rope[1][sample]),
                                           "fp16x2", "bfloat16")
            assert float((np.abs(out[sample] - exact) - bound).max()) <= 0, (layer, node.node_id, target)
