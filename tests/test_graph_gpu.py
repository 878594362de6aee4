"""GPU test of restores captured in a HIP graph.

A call of K (RoPE) and V jobs is captured once per kernel variant (stream, straight-line with two
or one heads per step or rank halves, channel-slice, general); the graph is replayed several times, with eager work and synchronizations between the
replays and the destinations overwritten before each, and every replay must reproduce the eager
result bit for bit.  Captured calls take their descriptor staging from memory reserved
beforehand (``reserve_capture_staging``); the capture itself allocates no pinned memory and
records no memset.
"""

import numpy as np
import pytest
import torch

from oracle import restore as orc
from reelcache_amd import restore_kernels as rk

from restore_cases import destination, make_case

pytestmark = pytest.mark.gpu


def _jobs(device, ranks=(96, 160)):
    rng = np.random.default_rng(70)
    table = rk.RopeTable.from_complex(torch.from_numpy(orc.wan_freqs(128, 64)))
    heads, head_dim, grid, tokens = 4, 128, (2, 9, 13), 234
    cache_k = destination("BTHD", 2 * tokens, heads, head_dim, "bfloat16", device)
    cache_v = destination("BTHD", 2 * tokens, heads, head_dim, "bfloat16", device)
    jobs = []
    for chunk in range(2):
        jobs.append(make_case(rng, grid=grid, heads=heads, head_dim=head_dim, rank=ranks[0], source="uint8",
                              view=rk.NativeView(cache_k, token_offset=chunk * tokens), table=table,
                              rope_rows=(2 * chunk, 0, 0), out_dtype="bfloat16", device=device).job)
        jobs.append(make_case(rng, grid=grid, heads=heads, head_dim=head_dim, rank=ranks[1], source="uint8",
                              view=rk.NativeView(cache_v, token_offset=chunk * tokens), rope="none",
                              out_dtype="bfloat16", device=device).job)
    return jobs, (cache_k, cache_v)


@pytest.mark.parametrize("config,ranks", [({}, (96, 160)), ({"head_pairs": False}, (96, 160)),
                                          ({"fast_variant": False}, (96, 160)),
                                          ({}, (256, 448)),  # rank halves (8-wave workgroups)
                                          ({"stream_variant": True}, (96, 160)),  # the stream kernel
                                          ({"stream_variant": True, "static_scratch": True}, (96, 160)),
                                          ({"stream_variant": True}, (256, 448))])  # stream (256), rank halves (448)
def test_captured_restore_replays_match_eager(device, config, ranks):
    jobs, caches = _jobs(device, ranks)
    for cache in caches:
        cache.fill_(-3.0)
    rk.reconstruct(jobs, config=config).release()
    torch.cuda.synchronize(device)
    expected = [cache.clone() for cache in caches]

    rk.reserve_capture_staging(1 << 20)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.graph(graph, stream=stream):
        handles = [rk.reconstruct(jobs, config=config)]
    torch.cuda.synchronize(device)
    assert handles[0].stats["launches"] >= 2
    for replay in range(4):
        for cache in caches:
            cache.fill_(float(-replay - 1))
        noise = torch.randn(512, 512, device=device) @ torch.randn(512, 512, device=device)  # eager work
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        for cache, want in zip(caches, expected):
            assert torch.equal(cache, want), f"replay {replay} differs from the eager restore"
        del noise
    del graph, handles


@pytest.mark.parametrize("config", [{}, {"pair_launch": False}])
def test_replays_repack_a_basis_changed_in_place(device, config):
    """Every replay packs the bases again before its restore launch(es).  The bases are doubled in
    place between replays; a power of two only moves the block exponents, so each replay must
    write exactly twice the previous values (a replay that reused the previous fragments or
    exponents would not)."""
    jobs, caches = _jobs(device, (96, 160))
    bases = {job.basis.data_ptr(): job.basis for job in jobs}.values()
    handle = rk.reconstruct(jobs, config=config)
    handle.release()
    torch.cuda.synchronize(device)
    rk.reserve_capture_staging(1 << 20)  # after the RoPE table's first use, before the capture
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.graph(graph, stream=stream):
        handles = [rk.reconstruct(jobs, config=config)]
    torch.cuda.synchronize(device)
    assert handles[0].stats["variants"] == (["pair"] if not config else ["pairs", "pairs"])
    graph.replay()
    torch.cuda.synchronize(device)
    previous = [cache.float().clone() for cache in caches]
    assert all(bool(torch.isfinite(p).all()) and float(p.abs().max()) > 0 for p in previous)
    for replay in range(3):
        for basis in bases:
            basis.mul_(2)
        for cache in caches:
            cache.fill_(0.0)
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        for cache, before in zip(caches, previous):
            assert torch.equal(cache.float(), 2 * before), f"replay {replay + 1} did not repack the doubled bases"
        previous = [cache.float().clone() for cache in caches]
    del graph, handles
