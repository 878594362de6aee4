"""GPU parity at the LongCat layer shape: 32 heads x 128 (4096 channels),
LongCat's [B, H, T, D] cache layout, 4680-token chunks with high per-chunk ranks (256-512 of one
512-row bf16 basis per K/V target), no RoPE (LongCat stores pre-RoPE K,
reelcache/restore_kernels.py:504-506).

Two tests restore three chunks per target, one the full 16-chunk history; the checks are
  * every element of every slot is written (no fill value left) and the tokens around the slots
    are untouched;
  * the oracle's elementwise error bound (reelcache/restore_kernels.py:1208-1227): on every token
    of one job per rank class (512, 384, 256, with rel-Frobenius 1e-3 against the oracle's
    reconstruction cast to bf16), on sampled token rows of the other jobs.
Ranks above 192 (fp16x2) run the rank-halves variant of the straight-line kernel (8-wave
workgroups, two halves of the rank steps reduced through LDS).
"""

import numpy as np
import pytest
import torch

from reelcache_amd import restore_kernels as rk
from oracle import restore as orc

from restore_cases import destination, make_case, orthonormal_basis

pytestmark = pytest.mark.gpu

HEADS, HEAD_DIM, GRID = 32, 128, (3, 30, 52)
RANKS = (512, 384, 256)
FILL = -123.0


def test_longcat_shape_restore(device):
    rng = np.random.default_rng(91)
    tokens = int(np.prod(GRID))
    history = len(RANKS) * tokens
    cases, caches = [], []
    for target in range(2):  # K, V
        cache = destination("BHTD", history, HEADS, HEAD_DIM, "bfloat16", device, offset=7, extra=5, fill=FILL)
        basis = orthonormal_basis(512, HEADS * HEAD_DIM, rng, torch.bfloat16).to(device)
        caches.append(cache)
        for chunk, rank in enumerate(RANKS if target == 0 else RANKS[::-1]):
            view = rk.NativeView(cache, "BHTD", token_offset=7 + chunk * tokens)
            cases.append(make_case(rng, grid=GRID, heads=HEADS, head_dim=HEAD_DIM, rank=rank, rope="none",
                                   view=view, basis=basis, out_dtype="bfloat16", device=device))
    handle = rk.reconstruct([case.job for case in cases])
    handle.release()
    assert handle.stats["variants"] and set(handle.stats["variants"]) == {"split"}, handle.stats["variants"]
    for cache in caches:
        tokens_major = cache[0].transpose(0, 1)  # [T, H, D]
        assert not bool((tokens_major[7:7 + history] == FILL).any()), "a slot element was not written"
        assert bool((tokens_major[:7] == FILL).all()) and bool((tokens_major[7 + history:] == FILL).all())
    for index, case in enumerate(cases):
        got = case.job.destination.slot(tokens).reshape(tokens, -1).double().cpu().numpy()  # [N, H * D]
        if index < len(RANKS):
            # The K jobs, one per rank class (512, 384, 256), on every token: the elementwise bound and
            # rel-Frobenius 1e-3 against the oracle's reconstruction cast to bf16.
            values, bound = orc.error_bound(case.coefficients, case.basis, HEADS, None, "fp16x2", "bfloat16")
            excess = np.abs(got - values) - bound
            assert float(excess.max()) <= 0, f"rank {case.job.rank}: {int((excess > 0).sum())} elements over bound"
            cast = torch.from_numpy(values).float().to(torch.bfloat16).double().numpy()
            assert orc.relative_frobenius(got, cast) <= 1e-3
            continue
        rows = np.unique(np.concatenate(([0, tokens - 1], rng.choice(tokens, 30, replace=False))))
        values, bound = orc.error_bound(case.coefficients[rows], case.basis, HEADS, None, "fp16x2", "bfloat16")
        excess = np.abs(got[rows] - values) - bound
        assert float(excess.max()) <= 0, f"{int((excess > 0).sum())} elements exceed the error bound"


@pytest.mark.parametrize("precision", ["fp16x2", "fp16"])
def test_longcat_shape_beside_a_concurrent_gemm(device, precision):
    """The LongCat layer restored while 4096 x 4096 bf16 GEMMs run on a second stream (the next
    chunk's forward) gives the same bits as the restore alone, within the precision's bound; the
    single-product fp16 mode takes the one-wave kernel at 16 rank steps and rank halves above."""
    rng = np.random.default_rng(92)
    tokens = int(np.prod(GRID))
    history = len(RANKS) * tokens
    cases, caches = [], []
    for target in range(2):
        cache = destination("BHTD", history, HEADS, HEAD_DIM, "bfloat16", device, fill=FILL)
        basis = orthonormal_basis(512, HEADS * HEAD_DIM, rng, torch.bfloat16).to(device)
        caches.append(cache)
        for chunk, rank in enumerate(RANKS):
            view = rk.NativeView(cache, "BHTD", token_offset=chunk * tokens)
            cases.append(make_case(rng, grid=GRID, heads=HEADS, head_dim=HEAD_DIM, rank=rank, rope="none",
                                   view=view, basis=basis, out_dtype="bfloat16", device=device))
    jobs = [case.job for case in cases]
    handle = rk.reconstruct(jobs, precision=precision)
    handle.release()
    expected = {"fp16x2": {"split"}, "fp16": {"split", "fast"}}[precision]
    assert set(handle.stats["variants"]) == expected, handle.stats["variants"]
    alone = [cache.clone() for cache in caches]
    for cache in caches:
        cache.fill_(FILL)
    a = torch.randn(4096, 4096, device=device, dtype=torch.bfloat16)
    b = torch.randn(4096, 4096, device=device, dtype=torch.bfloat16)
    side, main = torch.cuda.Stream(device), torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    main.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        products = [a @ b for _ in range(6)]
    rk.reconstruct(jobs, precision=precision, stream=main).release()
    torch.cuda.synchronize(device)
    del products
    for cache, reference in zip(caches, alone):
        assert torch.equal(cache, reference), "the restore beside a GEMM differs from the restore alone"
    for case in cases:
        rows = np.unique(np.concatenate(([0, tokens - 1], rng.choice(tokens, 16, replace=False))))
        values, bound = orc.error_bound(case.coefficients[rows], case.basis, HEADS, None, precision, "bfloat16")
        got = case.job.destination.slot(tokens)
        got = got[torch.from_numpy(rows).to(got.device)].reshape(len(rows), -1).double().cpu().numpy()
        assert float((np.abs(got - values) - bound).max()) <= 0


def test_longcat_full_history(device):
    """The full configs[4] history of one layer: 16 chunks per target with ranks drawn from the
    32-grid in [256, 512], restored in one call; every slot written, the tokens around untouched,
    sampled rows of every job within the oracle's bound."""
    rng = np.random.default_rng(93)
    chunks = 16
    tokens = int(np.prod(GRID))
    history = chunks * tokens
    cases, caches = [], []
    for target in range(2):
        cache = destination("BHTD", history, HEADS, HEAD_DIM, "bfloat16", device, offset=3, extra=3, fill=FILL)
        basis = orthonormal_basis(512, HEADS * HEAD_DIM, rng, torch.bfloat16).to(device)
        caches.append(cache)
        ranks = rng.choice(np.arange(256, 513, 32), size=chunks)
        for chunk, rank in enumerate(ranks):
            view = rk.NativeView(cache, "BHTD", token_offset=3 + chunk * tokens)
            cases.append(make_case(rng, grid=GRID, heads=HEADS, head_dim=HEAD_DIM, rank=int(rank), rope="none",
                                   view=view, basis=basis, out_dtype="bfloat16", device=device))
    handle = rk.reconstruct([case.job for case in cases])
    handle.release()
    assert set(handle.stats["variants"]) == {"split"}, handle.stats["variants"]
    for cache in caches:
        tokens_major = cache[0].transpose(0, 1)
        assert not bool((tokens_major[3:3 + history] == FILL).any()), "a slot element was not written"
        assert bool((tokens_major[:3] == FILL).all()) and bool((tokens_major[3 + history:] == FILL).all())
    for case in cases:
        rows = np.unique(np.concatenate(([0, tokens - 1], rng.choice(tokens, 12, replace=False))))
        values, bound = orc.error_bound(case.coefficients[rows], case.basis, HEADS, None, "fp16x2", "bfloat16")
        got = case.job.destination.slot(tokens)
        got = got[torch.from_numpy(rows).to(got.device)].reshape(len(rows), -1).double().cpu().numpy()
        assert float((np.abs(got - values) - bound).max()) <= 0
