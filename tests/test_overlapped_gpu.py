"""GPU test of the layer-overlapped restore (reelcache/overlapped_restore.py:1-60 contract):
layers are restored on the readiness' private stream while a consumer stream waits for each
layer in turn and reads it (with a matrix product of its own in between, as a forward would);
every layer the consumer read equals the synchronous restore of the same jobs bit for bit."""

import numpy as np
import pytest
import torch

from oracle import restore as orc
from reelcache_amd import restore_kernels as rk
from reelcache_amd.overlapped_restore import start_overlapped_restore

from restore_cases import destination, make_case

pytestmark = pytest.mark.gpu


def _layers(device, count=4):
    rng = np.random.default_rng(91)
    table = rk.RopeTable.from_complex(torch.from_numpy(orc.wan_freqs(128, 64)))
    heads, head_dim, grid, tokens = 4, 128, (2, 9, 13), 234
    layers, caches = [], []
    for _ in range(count):
        cache_k = destination("BTHD", 2 * tokens, heads, head_dim, "bfloat16", device)
        cache_v = destination("BTHD", 2 * tokens, heads, head_dim, "bfloat16", device)
        jobs = []
        for chunk in range(2):
            jobs.append(make_case(rng, grid=grid, heads=heads, head_dim=head_dim, rank=96, source="uint8",
                                  view=rk.NativeView(cache_k, token_offset=chunk * tokens), table=table,
                                  rope_rows=(2 * chunk, 0, 0), out_dtype="bfloat16", device=device).job)
            jobs.append(make_case(rng, grid=grid, heads=heads, head_dim=head_dim, rank=160, source="uint8",
                                  view=rk.NativeView(cache_v, token_offset=chunk * tokens), rope="none",
                                  out_dtype="bfloat16", device=device).job)
        layers.append(jobs)
        caches.append((cache_k, cache_v))
    return layers, caches


def test_overlapped_restore_matches_synchronous(device):
    layers, caches = _layers(device)
    for jobs in layers:
        rk.reconstruct(jobs).release()
    torch.cuda.synchronize(device)
    expected = [(k.clone(), v.clone()) for k, v in caches]
    for k, v in caches:
        k.fill_(-5.0)
        v.fill_(-5.0)
    torch.cuda.synchronize(device)

    readiness = start_overlapped_restore(layers, device=device)
    consumer = torch.cuda.Stream(device)
    seen = []
    with torch.cuda.stream(consumer):
        work = torch.randn(256, 256, device=device)
        for layer, (k, v) in enumerate(caches):
            readiness.layer(layer).wait(consumer)
            seen.append((k.clone(), v.clone()))
            work = work @ work.T / 256  # the forward's own work between layers
    consumer.synchronize()
    info = readiness.join(timeout=120)
    assert info["overlapped"] and readiness.done
    assert readiness.stream is not None and readiness.stream != consumer
    for layer, ((k, v), (want_k, want_v)) in enumerate(zip(seen, expected)):
        assert torch.equal(k, want_k) and torch.equal(v, want_v), f"layer {layer} read before its restore finished"
    assert readiness.quiesce(timeout=60)
