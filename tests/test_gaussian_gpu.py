"""GPU tests of the batched seeded Gaussian kernel (``rch_fit_gaussian``) that fills the start
columns of the direction solvers and anchor sketches (the reference draws them from per-matrix
seeded generators, reelcache/rank_method.py:479-484; the values only steer the solvers).

The kernel is pinned three ways: the numpy Philox-4x32-10 below against the published known-answer
vectors of Salmon et al. (SC 2011, Random123 ``kat_vectors``); every device element against that
Philox followed by Box-Muller on the host (within a few FP32 ulps, the device's ``logf``/``cosf``
rounding); and the sample moments of a large block against N(0, 1).
"""

import numpy as np
import pytest
import torch

from reelcache_amd import fit_kernels

pytestmark = pytest.mark.gpu

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
MASK = np.uint64(0xFFFFFFFF)


def philox(counters: np.ndarray, key: tuple[int, int]) -> np.ndarray:
    """Philox-4x32-10 of ``[n, 4]`` uint32 counters under a two-word key."""
    c = counters.astype(np.uint64)
    k0, k1 = np.uint32(key[0]), np.uint32(key[1])
    with np.errstate(over="ignore"):
        for _ in range(10):
            p0 = M0 * c[:, 0]
            p1 = M1 * c[:, 2]
            c = np.stack(((p1 >> np.uint64(32)) ^ c[:, 1] ^ np.uint64(k0), p1 & MASK,
                          (p0 >> np.uint64(32)) ^ c[:, 3] ^ np.uint64(k1), p0 & MASK), axis=1)
            k0, k1 = np.uint32(k0 + W0), np.uint32(k1 + W1)
    return c.astype(np.uint32)


def test_philox_known_answers():
    cases = [((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
             ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
             ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
              (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1))]
    for counter, key, want in cases:
        got = philox(np.array([counter], dtype=np.uint32), key)[0]
        assert tuple(int(x) for x in got) == want


def host_gaussian(rows: int, cols: int, seed: int) -> np.ndarray:
    """Element e = r * cols + c is normal e % 4 of counter e // 4: Box-Muller on word pairs."""
    total = rows * cols
    groups = (total + 3) // 4
    index = np.arange(groups, dtype=np.uint64)
    counters = np.stack((index & MASK, index >> np.uint64(32), np.zeros_like(index), np.zeros_like(index)), axis=1)
    words = philox(counters.astype(np.uint32), (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF))
    scale = np.float32(2.0 ** -32)
    out = np.empty((groups, 4), dtype=np.float64)
    for pair in range(2):
        u1 = ((words[:, 2 * pair].astype(np.float32) + np.float32(1.0)) * scale).astype(np.float64)
        u2 = (words[:, 2 * pair + 1].astype(np.float32) * scale).astype(np.float64)
        radius = np.sqrt(-2.0 * np.log(u1))
        out[:, 2 * pair] = radius * np.cos(2 * np.pi * u2)
        out[:, 2 * pair + 1] = radius * np.sin(2 * np.pi * u2)
    return out.reshape(-1)[:total].reshape(rows, cols)


def test_device_values_match_the_host_restatement(device):
    specs = [(128, 37, 5), (256, 96, 2 ** 63 + 12345), (7, 3, 1), (1024, 160, 987654321)]
    buffers = [torch.full((rows, cols + 8), -9.0, dtype=torch.float32, device=device) for rows, cols, _ in specs]
    fit_kernels.gaussian([(buffer[:, 8:], seed) for buffer, (_, _, seed) in zip(buffers, specs)])
    for buffer, (rows, cols, seed) in zip(buffers, specs):
        got = buffer.cpu().double().numpy()
        assert (got[:, :8] == -9.0).all(), "columns outside the view were written"
        want = host_gaussian(rows, cols, seed)
        assert np.abs(got[:, 8:] - want).max() <= 2e-5 * (1 + np.abs(want).max())


def test_values_depend_only_on_seed_and_shape(device):
    first = torch.empty(64, 40, device=device)
    second = torch.empty(3, 64, 40, device=device)
    fit_kernels.gaussian([(first, 77)])
    fit_kernels.gaussian([(second[0], 76), (second[1], 77), (second[2], 78)])
    assert torch.equal(first, second[1])
    assert not torch.equal(second[0], second[1]) and not torch.equal(second[1], second[2])


def test_sample_moments(device):
    block = torch.empty(2048, 1024, device=device)
    fit_kernels.gaussian([(block, 2024)])
    values = block.double().flatten()
    n = values.numel()
    assert abs(float(values.mean())) < 5 / n ** 0.5
    assert abs(float(values.var()) - 1) < 5 * (2 / n) ** 0.5
    fourth = float((values ** 4).mean())
    assert abs(fourth - 3) < 5 * (96 / n) ** 0.5
    below = float((values < -1.6448536269514722).double().mean())  # P(Z < -1.645) = 0.05
    assert abs(below - 0.05) < 5 * (0.05 * 0.95 / n) ** 0.5


def test_refuses_what_it_cannot_fill(device):
    from reelcache_amd.errors import ConfigurationError

    with pytest.raises(ConfigurationError):
        fit_kernels.gaussian([(torch.empty(8, 8, device=device).T, 1)])
    with pytest.raises(ConfigurationError):
        fit_kernels.gaussian([(torch.empty(8, 8, device=device, dtype=torch.float16), 1)])
