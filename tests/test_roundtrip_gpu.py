"""BASELINE configs[0] on the GPU path: the synthetic runtime round trip.

4 chunks x 2 layers x {K, V}, each chunk a [1560, 1536] bf16 matrix (12 heads x 128,
grid 1 x 30 x 52) drawn as A = U V + eps with U ~ N(0, 1) [1560, 32], V ~ N(0, 1/32) [32, 1536]
and eps ~ N(0, 0.01^2) iid per element, cast to bf16.  Each chunk is planned by
``GramPlanner`` (K 98 % / V 95 %, bucket 32, the default top-k solver), projected onto the
planned rows, quantized to uint8 per channel (codec bypassed: the codes are the raw planes) and
restored with ``reconstruct`` into per-(layer, target) caches.

Checked against the oracle on the same inputs:
  * ranks: the bucket of the FP64 energy crossing of the bf16 matrix (chunk 0);
  * codes and affine: the oracle's quantizer applied to the same coefficients, bit for bit;
  * restored slots: within the oracle's elementwise error bound for the stored codes, affine
    and basis (reelcache/restore_kernels.py:1208-1227);
  * the round trip itself: ||restored - A||_F / ||A||_F within the energy target's residual.
"""

import numpy as np
import pytest
import torch

from oracle import fit as of
from oracle import quantize as oq
from oracle import restore as orc
from reelcache_amd import fit_kernels as fk
from reelcache_amd import node_packets as npk
from reelcache_amd import rank_method as rm
from reelcache_amd import restore_kernels as rk
from reelcache_amd.types import CodecSpec, MatrixKey, ModelIdentity, TensorContext, energy_targets

pytestmark = pytest.mark.gpu

CHUNKS, LAYERS, HEADS, HEAD_DIM, GRID = 4, 2, 12, 128, (1, 30, 52)
TOKENS, CHANNELS = 1560, 1536


def _matrix(rng):
    u = rng.standard_normal((TOKENS, 32))
    v = rng.standard_normal((32, CHANNELS)) / np.sqrt(32)
    a = u @ v + rng.standard_normal((TOKENS, CHANNELS)) * 0.01
    return torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16)


def test_config0_round_trip(device):
    rng = np.random.default_rng(2024)
    config = rm.RankMethodConfig(energy_targets("causvid"), CodecSpec("svd_hevc", 1))
    model = ModelIdentity("roundtrip-synthetic", "d" * 64, LAYERS, CHANNELS, "THD", "bfloat16")
    keys = [MatrixKey(layer, target) for layer in range(LAYERS) for target in "KV"]
    caches = {key: torch.full((1, CHUNKS * TOKENS, HEADS, HEAD_DIM), -7.0, dtype=torch.bfloat16, device=device)
              for key in keys}
    originals = {key: [] for key in keys}
    for chunk in range(CHUNKS):
        sources = {key: _matrix(rng).to(device) for key in keys}
        contexts = {key: TensorContext(model, key, chunk * TOKENS, *GRID, "pre_rope" if key.target == "K" else "none")
                    for key in keys}
        plan = rm.GramPlanner(config, device=device).plan(
            sources, contexts, {key: rm.ActiveBasisBinding() for key in keys}, {key: None for key in keys},
            chunk_id=f"chunk{chunk}", source_ids={key: f"{chunk}{key.layer}{key.target}" for key in keys})
        rows = [plan.plans[key].new_rows.to(device) for key in keys]
        ranks = [int(r.shape[0]) for r in rows]
        coefficients, extrema = fk.project([sources[key] for key in keys], rows, ranks, extrema=True)
        quantized = npk.quantize_many(coefficients, extrema.cpu().numpy(), [config.spec_for(r) for r in ranks])
        jobs, expected = [], []
        for key, row, rank, p, (codes, affine, layout) in zip(keys, rows, ranks, coefficients, quantized):
            host_p = p.float().cpu().numpy()
            want_codes, want_affine, _ = oq.quantize(host_p, "per_channel")
            assert np.array_equal(codes.cpu().numpy(), want_codes), f"{key}: codes differ from the oracle quantizer"
            assert np.array_equal(np.asarray(affine), want_affine), f"{key}: affine differs from the oracle quantizer"
            if chunk == 0:
                x = sources[key].double().cpu().numpy()
                values = np.linalg.eigvalsh(x.T @ x)[::-1]
                target = config.targets.for_target(key.target)
                want = of.bucket(of.crossing(values, float(np.square(x).sum()), target), 32, CHANNELS)
                assert rank == want, f"{key}: rank {rank}, oracle {want}"
            scale, offset = rk.expand_affine(np.asarray(affine), layout, rank)
            jobs.append(rk.ReconstructionJob(rk.CoefficientSource(codes, scale, offset),
                                             rk.NativeView(caches[key], token_offset=chunk * TOKENS), GRID, row, rank))
            expected.append(orc.error_bound(orc.dequantize(want_codes, scale, offset), row.double().cpu().numpy(),
                                            HEADS, None, "fp16x2", "bfloat16"))
            originals[key].append(sources[key].float().cpu().numpy())
        rk.reconstruct(jobs).release()
        for key, (values, bound) in zip(keys, expected):
            got = caches[key][0, chunk * TOKENS:(chunk + 1) * TOKENS].reshape(TOKENS, -1).double().cpu().numpy()
            excess = np.abs(got - values) - bound
            assert float(excess.max()) <= 0, f"{key}: {int((excess > 0).sum())} elements exceed the error bound"
    for key in keys:
        a = np.concatenate(originals[key]).astype(np.float64)
        got = caches[key][0].reshape(CHUNKS * TOKENS, -1).double().cpu().numpy()
        relative = np.linalg.norm(got - a) / np.linalg.norm(a)
        residual = np.sqrt(1.0 - config.targets.for_target(key.target))
        assert relative <= residual, f"{key}: round-trip error {relative:.4f} above the target residual {residual:.4f}"
        assert relative <= 0.05, f"{key}: round-trip error {relative:.4f}"  # noise 1e-4 of the energy + 8-bit codes
