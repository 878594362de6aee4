"""GPU test of the layer-overlapped restore (reelcache/overlapped_restore.py:1-60 contract):
layers are restored on the readiness' private stream while a consumer stream waits for each
layer in turn and reads it (with a matrix product of its own in between, as a forward would).
Every layer the consumer read is checked against the oracle: each slot element within the
reference's error bound for the default fp16x2 precision, and each slot within rel-Frobenius
1e-3 of the oracle's reconstruction cast to bf16 (the BASELINE tolerance).  It also equals the
synchronous restore of the same jobs bit for bit, so no layer was read before its restore ended."""

import numpy as np
import pytest
import torch

from oracle import restore as orc
from reelcache_amd import restore_kernels as rk
from reelcache_amd.overlapped_restore import start_overlapped_restore

from restore_cases import destination, expected, make_case

pytestmark = pytest.mark.gpu


def _layers(device, count=4):
    rng = np.random.default_rng(91)
    table = rk.RopeTable.from_complex(torch.from_numpy(orc.wan_freqs(128, 64)))
    heads, head_dim, grid, tokens = 4, 128, (2, 9, 13), 234
    layers, caches, cases = [], [], []
    for _ in range(count):
        cache_k = destination("BTHD", 2 * tokens, heads, head_dim, "bfloat16", device)
        cache_v = destination("BTHD", 2 * tokens, heads, head_dim, "bfloat16", device)
        layer_cases = []
        for chunk in range(2):
            layer_cases.append((0, chunk * tokens, make_case(
                rng, grid=grid, heads=heads, head_dim=head_dim, rank=96, source="uint8",
                view=rk.NativeView(cache_k, token_offset=chunk * tokens), table=table, rope_rows=(2 * chunk, 0, 0),
                out_dtype="bfloat16", device=device)))
            layer_cases.append((1, chunk * tokens, make_case(
                rng, grid=grid, heads=heads, head_dim=head_dim, rank=160, source="uint8",
                view=rk.NativeView(cache_v, token_offset=chunk * tokens), rope="none", out_dtype="bfloat16",
                device=device)))
        layers.append([case.job for _, _, case in layer_cases])
        caches.append((cache_k, cache_v))
        cases.append(layer_cases)
    return layers, caches, cases


def _check_against_oracle(layer, read, layer_cases):
    """The slots the consumer read (clones of the K and V caches) against the oracle."""
    for target, offset, case in layer_cases:
        tokens = case.job.tokens
        out = read[target][0, offset:offset + tokens].reshape(tokens, -1).double().cpu().numpy()
        values, bound = expected(case, "fp16x2")
        excess = np.abs(out - values) - bound
        assert float(excess.max()) <= 0, f"layer {layer} target {'KV'[target]}: {int((excess > 0).sum())} over bound"
        cast = torch.from_numpy(values).float().to(torch.bfloat16).double().numpy()
        assert orc.relative_frobenius(out, cast) <= 1e-3


def test_overlapped_restore_matches_the_oracle(device):
    layers, caches, cases = _layers(device)
    for jobs in layers:
        rk.reconstruct(jobs).release()
    torch.cuda.synchronize(device)
    synchronous = [(k.clone(), v.clone()) for k, v in caches]
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
    for layer, ((k, v), (want_k, want_v)) in enumerate(zip(seen, synchronous)):
        _check_against_oracle(layer, (k, v), cases[layer])
        assert torch.equal(k, want_k) and torch.equal(v, want_v), f"layer {layer} read before its restore finished"
    assert readiness.quiesce(timeout=60)
