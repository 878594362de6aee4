"""Benchmark: full CausVid-shape history restore on one MI355X.

A step restores the 7-chunk history (32,760 tokens) of all 30 layers, K and V,
into bf16 [1, T, 12, 128] caches: per layer one ``reconstruct`` call of 14 jobs
(uint8 codes [4680, r] with per-column affine, shared bf16 bases r_K = 128 /
r_V = 192, Wan 3-D RoPE on K).  Inputs are synthetic, seeded and resident in HBM
before timing.

The timed step is one full restore step captured once in a HIP graph (its 30 ``reconstruct``
calls: descriptor uploads, basis packs and restore launches) and replayed; every kernel of the
step runs on every replay.  One eager step before it gives the per-layer latency, the kernel
time and the host cost of a ``reconstruct`` call, reported under ``eager``.

Printed JSON line (one): ``value`` = restored KV bytes written per second
(GB/s, whole job), ``ms_per_step``, per-layer latency, the ``roofline`` of the
fused restore kernel (algorithmic bytes per launch / its average duration,
measured with HIP events on the launch stream) and a ``cpu_baseline`` (the
oracle's CPU restatement on a bounded sample, timed on this host).  Beside the headline:
``pictures`` (the same layers restored from picture canvases), ``longcat`` (per-layer restore
time at the BASELINE configs[4] shape, MFMA roofline, alone and beside a concurrent GEMM) and
``fit`` (BASELINE configs[2] chunks per second).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
LAYERS, HEADS, HEAD_DIM = 30, 12, 128
GRID = (3, 30, 52)
CHUNKS = 7
RANK_K, RANK_V = 128, 192
CHANNELS = HEADS * HEAD_DIM
TOKENS = GRID[0] * GRID[1] * GRID[2]
HISTORY = CHUNKS * TOKENS
COPY_PROBE_BYTES = 256 << 20
METRIC = "restored KV GB/s + per-layer restore latency (CausVid shape, 1 GPU); fit chunks/s"


def layer_bytes():
    """Algorithmic HBM bytes of one layer's restore: bf16 K and V written, uint8 codes,
    bf16 bases and fp32 affine read."""
    written = 2 * HISTORY * CHANNELS * 2
    codes = CHUNKS * TOKENS * (RANK_K + RANK_V)
    basis = (RANK_K + RANK_V) * CHANNELS * 2
    affine = CHUNKS * (RANK_K + RANK_V) * 2 * 4
    return written, written + codes + basis + affine


COUNTER_PROFILE = os.path.join(ROOT, "profiles", "restore_causvid_counters.md")


def profile_figures():
    """``{name: value}`` of the machine-readable lines of the committed rocprofv3 summary of the
    restore kernels (copy-calibrated FETCH_SIZE + WRITE_SIZE per launch, trace durations, MFMA
    busy); counters cannot be read from inside this process.  Empty when the file is absent."""
    figures = {}
    try:
        lines = open(COUNTER_PROFILE).read().splitlines()
    except OSError:
        return figures
    for line in lines:
        name, _, value = line.partition(":")
        if name.startswith(("traffic_bytes_per_", "trace_us ", "mfma_busy ")) and value.strip():
            figures[name] = float(value)
    return figures


def launch_bytes(rank):
    """Algorithmic bytes of one restore launch (the 7 jobs of one target): codes, basis and affine
    read, slots written."""
    return CHUNKS * TOKENS * rank + rank * CHANNELS * 2 + CHUNKS * rank * 8 + CHUNKS * TOKENS * CHANNELS * 2


def layer_flops():
    return 2 * CHUNKS * TOKENS * CHANNELS * (RANK_K + RANK_V)


def covering_affine(rank, rng):
    lo = rng.uniform(-4, 0, size=rank).astype(np.float32)
    hi = (lo.astype(np.float64) + rng.uniform(0.5, 6, size=rank)).astype(np.float32)
    from reelcache_amd.quantize import covering_affine as cover

    affine = cover(lo, hi)
    return affine[0].copy(), affine[1].copy()


def build_workload(device, seed=0):
    from reelcache_amd import restore_kernels as rk

    rng = np.random.default_rng(seed)
    generator = torch.Generator(device=device).manual_seed(seed)
    # Wan 3-D RoPE table (theta 10000, sections 22/21/21 pairs), float64 as the model builds it.
    sixth = HEAD_DIM // 6
    parts = []
    for dim in (HEAD_DIM - 4 * sixth, 2 * sixth, 2 * sixth):
        inverse = 1.0 / torch.pow(10000.0, torch.arange(0, dim, 2, dtype=torch.float64) / dim)
        parts.append(torch.polar(torch.ones(64, dim // 2, dtype=torch.float64),
                                 torch.outer(torch.arange(64, dtype=torch.float64), inverse)))
    table = rk.RopeTable.from_complex(torch.cat(parts, dim=1))
    table.kernel_tables(device)
    layers = []
    for layer in range(LAYERS):
        cache_k = torch.empty((1, HISTORY, HEADS, HEAD_DIM), dtype=torch.bfloat16, device=device)
        cache_v = torch.empty_like(cache_k)
        # Orthonormal rows (host QR of a Gaussian), stored as the bf16 basis.
        basis_k = torch.from_numpy(np.linalg.qr(rng.standard_normal((CHANNELS, RANK_K)))[0].T.copy())
        basis_v = torch.from_numpy(np.linalg.qr(rng.standard_normal((CHANNELS, RANK_V)))[0].T.copy())
        basis_k = basis_k.to(device=device, dtype=torch.bfloat16)
        basis_v = basis_v.to(device=device, dtype=torch.bfloat16)
        jobs = []
        for chunk in range(CHUNKS):
            for cache, basis, rank, rope in ((cache_k, basis_k, RANK_K, True), (cache_v, basis_v, RANK_V, False)):
                codes = torch.randint(0, 256, (TOKENS, rank), dtype=torch.uint8, device=device, generator=generator)
                scale, offset = covering_affine(rank, rng)
                jobs.append(rk.ReconstructionJob(
                    rk.CoefficientSource(codes, scale, offset), rk.NativeView(cache, token_offset=chunk * TOKENS),
                    GRID, basis, rank, rk.RopePositions(table, (GRID[0] * chunk, 0, 0)) if rope else None))
        layers.append(jobs)
    torch.cuda.synchronize(device)
    return layers


def restore_step(layers, stream, events=None, precision="auto"):
    from reelcache_amd import restore_kernels as rk

    handles = []
    for index, jobs in enumerate(layers):
        stage = [] if events is not None else None
        handles.append(rk.reconstruct(jobs, stream=stream, stage_events=stage, precision=precision))
        if events is not None:
            events.append(stage)
    return handles


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo), or the platform's processor string."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def host_threads():
    """BLAS threads for the all-threads CPU baselines: the process's OMP_NUM_THREADS share when set
    (the GPU boxes set it to their CPU share), else os.cpu_count()."""
    cores = os.cpu_count() or 1
    try:
        return max(1, min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))
    except ValueError:
        return cores


def _timed_variants(run_one, budget, variants):
    """Run ``run_one(compute)`` repeatedly per (label, compute dtype, BLAS threads) variant for
    about ``budget / len(variants)`` seconds each (at least once); ``{label: (units, seconds)}``."""
    from threadpoolctl import threadpool_limits

    results = {}
    share = budget / len(variants)
    for label, compute, threads in variants:
        with threadpool_limits(limits=threads):
            units, started = 0, time.perf_counter()
            while True:
                run_one(compute)
                units += 1
                elapsed = time.perf_counter() - started
                if elapsed >= share:
                    break
        results[label] = (units, elapsed)
    return results


def cpu_baseline(seconds_budget=20.0, seed=1):
    """The oracle's CPU restatement of the reference restore (``reconstruct_reference``: dequantize,
    the product in FP64 -- the reference's default -- or IEEE FP32, RoPE in the same precision, one
    bf16 cast) on a bounded sample of CausVid jobs (one chunk's K or V matrix each), with all host
    threads and with one BLAS thread."""
    from oracle import restore as orc
    from oracle.quantize import covering_affine as cover

    rng = np.random.default_rng(seed)
    cores = host_threads()
    basis = {rank: np.linalg.qr(rng.standard_normal((CHANNELS, rank)))[0].T.astype(np.float32)
             for rank in (RANK_K, RANK_V)}
    cos, sin = np.real(orc.wan_freqs(HEAD_DIM, 64)), np.imag(orc.wan_freqs(HEAD_DIM, 64))
    jobs = []
    for chunk in range(2):
        for rank, rope in ((RANK_K, True), (RANK_V, False)):
            codes = rng.integers(0, 256, size=(TOKENS, rank), dtype=np.uint8)
            lo = rng.uniform(-4, 0, size=rank).astype(np.float32)
            affine = cover(lo, (lo + rng.uniform(0.5, 6, size=rank)).astype(np.float32))
            jobs.append((codes, affine, rank, orc.rope_cos_sin(cos, sin, orc.wan_sections(HEAD_DIM // 2),
                                                               (GRID[0] * chunk, 0, 0), GRID) if rope else None))
    cursor = [0]

    def one_job(compute):
        codes, affine, rank, rope = jobs[cursor[0] % len(jobs)]
        cursor[0] += 1
        coefficients = orc.dequantize(codes, affine[0], affine[1])
        values = orc.reconstruct(coefficients, basis[rank], HEADS, rope, compute=compute)
        orc.f32_to_bf16_bits(values.astype(np.float32))

    variants = [("fp64_all_threads", np.float64, cores), ("fp32_all_threads", np.float32, cores),
                ("fp64_1_thread", np.float64, 1), ("fp32_1_thread", np.float32, 1)]
    timed = _timed_variants(one_job, seconds_budget, variants)
    job_bytes = TOKENS * CHANNELS * 2  # the bf16 slot a job writes
    rates = {label: {"value": round(units * job_bytes / seconds / 1e9, 4), "jobs": units,
                     "seconds": round(seconds, 2)} for label, (units, seconds) in timed.items()}
    return {"value": rates["fp64_all_threads"]["value"], "unit": "GB/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "variants": rates,
            "sample": "CausVid restore jobs (one chunk's K or V: 4680 x 1536 bf16 slot, r 128 with Wan RoPE / 192) "
                      "through oracle.restore (dequantize, numpy product, RoPE, bf16 cast); value = the reference's "
                      f"default FP64 on all {cores} host threads; FP32 and 1-thread variants beside it"}


# ---------------------------------------------------------------------------------------------
# Fit leg: one chunk = 30 layers x {K, V} matrices [4680, 1536] bf16 with a
# decaying spectrum sigma_i = i ** -1.2 plus noise; planned (Gram -> eigh -> crossing -> verified
# bucket rank), projected onto the planned rows and quantized to uint8 on the device.
# ---------------------------------------------------------------------------------------------

FIT_EXPONENT, FIT_NOISE = 1.2, 1e-3


def fit_workload(device, seed=2, distinct=60):
    """The chunk's 60 source matrices, generated on the device: X = U diag(sigma) V^T + noise with
    U, V the Q factors of seeded Gaussians (per matrix) and noise N(0, (1e-3 sigma_1)^2 / N)."""
    from reelcache_amd.types import MatrixKey, ModelIdentity, TensorContext

    generator = torch.Generator(device=device).manual_seed(seed)
    sigma = torch.arange(1, CHANNELS + 1, dtype=torch.float32, device=device) ** -FIT_EXPONENT
    model = ModelIdentity("causvid-synthetic", "c" * 64, LAYERS, CHANNELS, "THD", "bfloat16")
    sources, contexts = {}, {}
    for index in range(min(distinct, 2 * LAYERS)):
        u = torch.linalg.qr(torch.randn(TOKENS, CHANNELS, device=device, generator=generator)).Q
        v = torch.linalg.qr(torch.randn(CHANNELS, CHANNELS, device=device, generator=generator)).Q
        noise = torch.randn(TOKENS, CHANNELS, device=device, generator=generator) * (FIT_NOISE / math.sqrt(TOKENS))
        x = ((u * sigma) @ v.T.contiguous() + noise).to(torch.bfloat16)
        key = MatrixKey(index // 2, "KV"[index % 2])
        sources[key] = x
        contexts[key] = TensorContext(model, key, 0, *GRID, "pre_rope" if key.target == "K" else "none")
    torch.cuda.synchronize(device)
    return sources, contexts


def _consecutive_host_rows(host_rows):
    """The flat pinned buffer that holds ``host_rows`` back to back in this order, or None."""
    first = host_rows[0]
    base = first._base
    if base is None or not base.is_pinned() or base.dim() != 1:
        return None
    offset = first.storage_offset()
    for rows in host_rows:
        if rows._base is not base or not rows.is_contiguous() or rows.storage_offset() != offset:
            return None
        offset += rows.numel()
    return base[first.storage_offset() - base.storage_offset():offset - base.storage_offset()]


def fit_step(sources, contexts, device):
    """One chunk: plan every matrix, then finalize it on its planned rows (projection, stored and
    span energies, codes; device)."""
    from reelcache_amd import gpu_fitting as gf
    from reelcache_amd import node_packets as npk
    from reelcache_amd import rank_method as rm
    from reelcache_amd.types import CodecSpec, energy_targets

    config = rm.RankMethodConfig(energy_targets("causvid"), CodecSpec("svd_hevc", 1))
    label, solver = gf.select_eigh_solver("auto")
    keys = list(sources)
    plan = rm.GramPlanner(config, device=device, eigh=solver, eigh_label=label).plan(
        sources, contexts, {k: rm.ActiveBasisBinding() for k in keys}, {k: None for k in keys},
        chunk_id="bench", source_ids={k: str(k) for k in keys})
    torch.cuda.synchronize(device)
    planned = time.perf_counter()
    # Final measurement on the planned FP16 rank views: projection, stored and span energies,
    # condition bound and 8-bit codes of all 60 matrices in batched launches.
    # The planned rows (host, one block per matrix) go to the device in one asynchronous copy: the
    # planner leaves them as consecutive views of one pinned buffer (gathered otherwise).
    host_rows = [plan.plans[k].new_rows for k in keys]
    staged = _consecutive_host_rows(host_rows)
    if staged is None:
        staged = torch.cat([rows.reshape(-1) for rows in host_rows]).pin_memory()
    device_rows = staged.to(device, non_blocking=True)
    items, offset = [], 0
    for k, host in zip(keys, host_rows):
        matrix_plan = plan.plans[k]
        rows = device_rows[offset:offset + host.numel()].view(host.shape)
        offset += host.numel()
        items.append(npk.FinalizeItem(sources[k], rows, contexts[k], config.spec_for(int(rows.shape[0])), k,
                                      matrix_plan.target, False, host))
    finalized = npk.finalize_tiles(items, tile_rows=config.tile_rows)
    codes = [pixels for _, pixels in finalized]
    torch.cuda.synchronize(device)
    plan.stages["finalize"] = time.perf_counter() - planned  # finalize_tiles of the chunk
    return plan, codes


def fit_cpu_baseline(seconds_budget=20.0, seed=3):
    """The oracle's CPU restatement of the fit chain per matrix (Gram, LAPACK eigh, crossing,
    FP64-accumulated projection, 8-bit quantization), the Gram and eigh in FP32 (the method's
    arithmetic) or FP64, with all host threads and with one BLAS thread, on CausVid-shape
    matrices generated before the timing."""
    from oracle import fit as of
    from oracle import quantize as oq

    rng = np.random.default_rng(seed)
    cores = host_threads()
    sources = [of.to_bfloat16_values(of.decaying_spectrum(rng, TOKENS, CHANNELS)) for _ in range(2)]
    cursor = [0]

    def one_matrix(compute):
        x = sources[cursor[0] % len(sources)]
        target = 0.98 if cursor[0] % 2 == 0 else 0.95
        cursor[0] += 1
        operand = x.astype(compute)
        values, vectors = np.linalg.eigh(operand.T @ operand)
        values, rows = values[::-1], vectors[:, ::-1].T
        total = float(np.square(x.astype(np.float64)).sum())
        rank = of.bucket(of.crossing(values.astype(np.float64), total, target), 32, CHANNELS)
        oq.quantize(of.project(x, of.stored_basis(rows[:rank])), "per_channel")

    variants = [("fp32_all_threads", np.float32, cores), ("fp64_all_threads", np.float64, cores),
                ("fp32_1_thread", np.float32, 1), ("fp64_1_thread", np.float64, 1)]
    timed = _timed_variants(one_matrix, seconds_budget, variants)
    rates = {label: {"value": round(units / seconds / (2 * LAYERS), 5), "matrices": units,
                     "ms_per_matrix": round(seconds / units * 1e3, 1)} for label, (units, seconds) in timed.items()}
    return {"value": rates["fp32_all_threads"]["value"], "unit": "chunks/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "variants": rates,
            "sample": "CausVid-shape matrices [4680, 1536] (60 per chunk) through oracle.fit: Gram + LAPACK eigh "
                      "(FP32 as the method computes them, or FP64), crossing, FP64 projection, quantizer; value = "
                      f"FP32 on all {cores} host threads; FP64 and 1-thread variants beside it"}


def fit_kernel_probe(device, rank=32):
    """One launch each of the fit chunk's batched device kernels at its shape (60 sources [4680,
    1536] bf16; rank-32 orthonormal bases from a host QR): absmax, Gram, projection, residual
    energies.  Values do not matter to the counters; no eigensolver or QR runs on the device."""
    from reelcache_amd import fit_kernels as fk

    generator = torch.Generator(device=device).manual_seed(9)
    rng = np.random.default_rng(9)
    count = 2 * LAYERS
    sources = [torch.randn(TOKENS, CHANNELS, device=device, generator=generator).to(torch.bfloat16)
               for _ in range(count)]
    basis = torch.from_numpy(np.linalg.qr(rng.standard_normal((CHANNELS, rank)))[0].T.copy()).to(device)
    bases, ranks = [basis.to(torch.float16)] * count, [rank] * count
    torch.cuda.synchronize(device)
    keys = fk.absmax(sources)
    fk.gram(sources)
    coefficients, _ = fk.project(sources, bases, ranks, extrema=True)
    fk.energies(sources, keys, bases=bases, ranks=ranks, coefficients=coefficients)
    torch.cuda.synchronize(device)
    return {"sources": count, "shape": [TOKENS, CHANNELS], "rank": rank,
            "kernels": "absmax, gram, project (with column extrema), energies (source and residual)"}


def fit_leg(device, steps, warmup, cpu_seconds):
    from reelcache_amd import fit_kernels as fk

    sources, contexts = fit_workload(device)
    print(f"fit: {len(sources)} source matrices generated", file=sys.stderr, flush=True)
    for _ in range(warmup):
        fit_step(sources, contexts, device)
        print("fit: warmup chunk done", file=sys.stderr, flush=True)
    stages = {"energy": 0.0, "gram": 0.0, "sketch": 0.0, "predict": 0.0, "topk": 0.0, "eigh": 0.0, "verify": 0.0,
              "finalize": 0.0}
    torch.cuda.synchronize(device)
    began = time.perf_counter()
    plan = None
    for _ in range(steps):
        plan, _codes = fit_step(sources, contexts, device)
        print("fit: timed chunk done", file=sys.stderr, flush=True)
        for name in stages:
            stages[name] += plan.stages.get(name, 0.0)
    seconds = (time.perf_counter() - began) / steps
    matrices = len(sources)
    # The Gram launch alone, timed with events on the launch stream; a device-side wait queued first
    # lets the host enqueue the launches before the start event runs, so host time is not timed.
    batch = list(sources.values())
    fk.gram(batch)
    torch.cuda.synchronize(device)
    gram_runs = []
    for _ in range(3):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)
        start.record()
        for _ in range(3):
            fk.gram(batch)
        stop.record()
        stop.synchronize()
        gram_runs.append(start.elapsed_time(stop) / 3)
    gram_ms = float(np.median(gram_runs))
    unique = TOKENS * CHANNELS * (CHANNELS + 1)
    # Issued MFMA work: 256 x 256 tiles of the lower triangle, 64 x 64 quadrants, the diagonal
    # tiles' 10 lower quadrants only.
    panels = -(-CHANNELS // 256)
    quadrants = 16 * panels * (panels - 1) // 2 + 10 * panels
    issued = 2 * TOKENS * 64 * 64 * quadrants
    ranks = sorted({p.rank_view for p in plan.plans.values()})
    observed = {"K": sorted({p.observed_rank for k, p in plan.plans.items() if k.target == "K"}),
                "V": sorted({p.observed_rank for k, p in plan.plans.items() if k.target == "V"})}
    result = {
        "fit_chunks_per_s": round(1.0 / seconds * (matrices / (2 * LAYERS)), 3),
        "fit": {"chunk_ms": round(seconds * 1e3 * (2 * LAYERS) / matrices, 1), "matrices_per_chunk": 2 * LAYERS,
                "stage_ms_per_chunk": {k: round(v / steps * 1e3, 2) for k, v in stages.items()},
                "eigh_ms_per_matrix": round(stages["eigh"] / steps / matrices * 1e3, 3),
                "solver": "topk_rr: k = 96 Ritz directions per matrix (FP32 Gram products, FP64 CholeskyQR2, "
                          "batched 96 x 96 eigh)",
                "gram_kernel_ms_per_chunk": round(gram_ms, 3),
                "gram_roofline": {"bound": "mfma", "achieved": round(matrices * unique / (gram_ms / 1e3) / 1e12, 1),
                                  "peak": 2500.0, "unit": "TFLOP/s",
                                  "frac": round(matrices * unique / (gram_ms / 1e3) / 1e12 / 2500.0, 4),
                                  "issued_frac": round(matrices * issued / (gram_ms / 1e3) / 1e12 / 2500.0, 4),
                                  "flops": "N*C*(C+1) unique per matrix; issued: 2*N*64^2 per computed 64 x 64 "
                                           f"quadrant ({quadrants} per matrix: 256-tiles of the lower triangle)"},
                "ranks": ranks, "observed_ranks": observed,
                "eigh_solver": plan.eigh_solver,
                "workload": "BASELINE configs[2]: 60 x [4680, 1536] bf16, sigma_i = i^-1.2 + noise 1e-3, "
                            "K 98 % / V 95 %, bucket 32, per-channel 8-bit codes"},
    }
    if cpu_seconds > 0:
        result["fit"]["cpu_baseline"] = fit_cpu_baseline(cpu_seconds)
    return result


# ---------------------------------------------------------------------------------------------
# LongCat leg: layer restores at the LongCat-Video shape, MFMA-bound.
# ---------------------------------------------------------------------------------------------

LC_CHUNKS, LC_HEADS, LC_MAX_RANK = 16, 32, 512


def longcat_leg(device, layers, reps):
    """Per-layer restore time at the LongCat shape: 16 chunks x 4680 tokens of K and V, 32 heads x
    128 in the [1, H, T, D] bf16 cache layout, per-chunk ranks U{256..512} on the 32-grid of one
    512-row orthonormal bf16 basis per layer and target, no RoPE (LongCat stores pre-RoPE K).
    Timed with HIP events on the launch stream (pack -> last restore), alone and while 4096 x 4096
    bf16 GEMMs (the next chunk's forward) run on a second stream for the whole restore; the
    GEMMs' own slowdown is reported beside the restore's."""
    from reelcache_amd import restore_kernels as rk

    rng = np.random.default_rng(5)
    generator = torch.Generator(device=device).manual_seed(5)
    channels = LC_HEADS * HEAD_DIM
    history = LC_CHUNKS * TOKENS
    work = []
    flops = 0
    for _ in range(layers):
        jobs = []
        for _target in range(2):
            cache = torch.empty((1, LC_HEADS, history, HEAD_DIM), dtype=torch.bfloat16, device=device)
            # Orthonormal rows: host QR of a seeded Gaussian (float64), stored as the bf16 basis.
            gauss = rng.standard_normal((channels, LC_MAX_RANK))
            basis = torch.from_numpy(np.linalg.qr(gauss)[0].T.copy()).to(device=device, dtype=torch.bfloat16)
            for chunk in range(LC_CHUNKS):
                rank = int(rng.integers(8, 17)) * 32
                codes = torch.randint(0, 256, (TOKENS, rank), dtype=torch.uint8, device=device, generator=generator)
                scale, offset = covering_affine(rank, rng)
                jobs.append(rk.ReconstructionJob(rk.CoefficientSource(codes, scale, offset),
                                                 rk.NativeView(cache, layout="BHTD", token_offset=chunk * TOKENS),
                                                 GRID, basis, rank, None))
                flops += 2 * TOKENS * channels * rank
        work.append(jobs)
    flops //= layers
    stream = torch.cuda.Stream(device)
    side = torch.cuda.Stream(device)
    a = torch.randn(4096, 4096, device=device, dtype=torch.bfloat16, generator=generator)
    b = torch.randn(4096, 4096, device=device, dtype=torch.bfloat16, generator=generator)

    def products(count):
        """``count`` back-to-back 4096^2 bf16 products on the side stream; (begin, end) events."""
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(side):
            begin.record(side)
            for _ in range(count):
                a @ b
            end.record(side)
        return begin, end

    products(3)
    torch.cuda.synchronize(device)
    gemm_runs = []
    for _ in range(3):
        begin, end = products(10)
        end.synchronize()
        gemm_runs.append(begin.elapsed_time(end) / 10 * 1e3)
    gemm_us = float(np.median(gemm_runs))  # one product alone

    def timed(precision, count):
        """Median restore time per layer (pack -> last launch) with ``count`` side products started
        just before it (0: alone), and the side products' mean time per product."""
        times, side_us, variants = [], [], []
        for _ in range(reps):
            for jobs in work:
                window = None
                if count:
                    side.wait_stream(stream)
                    window = products(count)
                stage = []
                handle = rk.reconstruct(jobs, stream=stream, stage_events=stage, precision=precision)
                handle.release()
                variants = handle.stats["variants"]
                stream.synchronize()
                side.synchronize()
                events = dict(stage)
                times.append(events["pack"].elapsed_time(events["fused"]) * 1e3)
                if window is not None:
                    side_us.append(window[0].elapsed_time(window[1]) * 1e3 / count)
        return float(np.median(times)), (float(np.median(side_us)) if side_us else None), variants

    results = {}
    for precision in ("fp16x2", "fp16"):
        for jobs in work:
            rk.reconstruct(jobs, stream=stream, precision=precision).release()
        torch.cuda.synchronize(device)
        alone, _, variants = timed(precision, 0)
        # Enough side products to cover the whole restore of a layer (and then some), so every
        # restore launch runs beside a GEMM.
        count = max(2, math.ceil(alone / gemm_us) + 1)
        with_gemm, gemm_beside, _ = timed(precision, count)
        achieved = flops / (alone / 1e6) / 1e12
        passes = 2 if precision == "fp16x2" else 1
        results[precision] = {
            "kernel_us_per_layer": round(alone, 1), "kernel_us_per_layer_with_gemm": round(with_gemm, 1),
            "side_gemm": {"products": count, "us_per_product_alone": round(gemm_us, 1),
                          "us_per_product_beside_restore": round(gemm_beside, 1),
                          "gemm_slowdown": round(gemm_beside / gemm_us, 3),
                          "restore_slowdown": round(with_gemm / alone, 3),
                          "what": "bf16 4096^2 products on a second stream, started just before the layer's "
                                  "restore and covering all of it; slowdowns relative to each running alone"},
            "variants": variants,
            "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": 2500.0, "unit": "TFLOP/s",
                         "frac": round(achieved / 2500.0, 4), "mfma_work_tflops": round(passes * achieved, 1)}}
    del work
    torch.cuda.empty_cache()
    headline = results["fp16x2"]
    return {"workload": "BASELINE configs[4] shape: 16 chunks x 4680 tokens x {K,V}, 32x128 BHTD bf16, ranks "
                        "U{256..512} on the 32-grid (one 512-row bf16 basis per layer and target), no RoPE",
            "layers": layers, "gflop_per_layer": round(flops / 1e9, 1), "precision": "fp16x2",
            **headline,
            "fp16": dict(results["fp16"], what="single-product fp16 mode (prescaled codes, one MFMA pass; held "
                                               "to the reference's fp16 bound and rel-Frobenius 1e-3)")}


def pictures_leg(layers, device, reps=3):
    """The same CausVid layers restored from channel_tiles.v1 picture canvases (the decoded-video
    production source; codes laid out by ``node_packets.mosaic_device``) instead of uint8 rows:
    per-layer kernel time with HIP events on the launch stream (pack -> last restore)."""
    from reelcache_amd import node_packets as npk
    from reelcache_amd import restore_kernels as rk
    from reelcache_amd.quantize import video_layout

    work = []
    for jobs in layers:
        pictured = []
        for job in jobs:
            frames = job.grid[0]
            video = video_layout(*job.grid, job.rank, "yuv444p")
            canvases = npk.mosaic_device(job.source.values.contiguous(), video)
            indices = [[segment * frames + frame for frame in range(frames)] for segment in range(video["segments"])]
            source = rk.PictureSource.from_canvases(canvases, video, indices, (0, 0), job.source.scale, job.source.offset)
            pictured.append(rk.ReconstructionJob(source, job.destination, job.grid, job.basis, job.rank, job.rope))
        work.append(pictured)
    stream = torch.cuda.Stream(device)
    for jobs in work:
        rk.reconstruct(jobs, stream=stream).release()
    times, variants = [], []
    for _ in range(reps):
        for jobs in work:
            stage = []
            handle = rk.reconstruct(jobs, stream=stream, stage_events=stage)
            handle.release()
            variants = handle.stats["variants"]
            stream.synchronize()
            events = dict(stage)
            times.append(events["pack"].elapsed_time(events["fused"]) * 1e3)
    kernel_us = float(np.median(times))
    _, algorithmic = layer_bytes()
    return {"workload": "BASELINE configs[1] layers with codes in channel_tiles.v1 yuv444p canvases (one picture per "
                        "frame), gathered in the restore kernel", "layers": len(layers),
            "kernel_us_per_layer": round(kernel_us, 1), "variants": variants,
            "achieved_gbs": round(algorithmic / (kernel_us / 1e6) / 1e9, 1)}


def fp16_leg(layers, device, steps):
    """The same step in the single-product fp16 precision mode (the reference's default is
    fp16x2): coefficients prescaled to fp16, one 32x32x16 f16 product per 16 ranks.  Its parity
    (every element within the oracle's fp16 error bound; rel-Frobenius at most 1e-3 against the
    fp32 reconstruction, the BASELINE tolerance) is tested in tests/test_restore_gpu.py."""
    from reelcache_amd import restore_kernels as rk

    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        for handle in restore_step(layers, stream, precision="fp16"):
            handle.release()
    torch.cuda.synchronize(device)
    rk.reserve_capture_staging(LAYERS * (64 << 10))
    graph = torch.cuda.CUDAGraph()
    capture_stream = torch.cuda.Stream(device)
    capture_stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.graph(graph, stream=capture_stream):
        captured = restore_step(layers, capture_stream, precision="fp16")
    torch.cuda.synchronize(device)
    graph.replay()
    torch.cuda.synchronize(device)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    stop.record()
    torch.cuda.synchronize(device)
    ms = start.elapsed_time(stop) / steps
    written, algorithmic = layer_bytes()
    del graph, captured
    return {"precision": "fp16", "ms_per_step": round(ms, 4),
            "value": round(LAYERS * written / (ms / 1e3) / 1e9, 2),
            "layer_us": round(ms / LAYERS * 1e3, 2),
            "layer_achieved_gbs": round(algorithmic / (ms / LAYERS / 1e3) / 1e9, 1),
            "what": "graph-replayed step in precision='fp16' (not the headline: the reference's default is fp16x2)"}


# Per-layer compute of the first denoise forward for CausVid, c(h) = 2.58 + 0.486 * h ms with h
# history chunks (reelcache/decoded_tier.py:49-50, measured there on another GPU): the deadline
# a layer-overlapped restore has to meet.
CAUSVID_LAYER_MS = (2.58, 0.486)


def vendor_gemm_leg(device, reps=20):
    """The library GEMM (torch.mm -> hipBLASLt) on the shape of each restore launch, as a yardstick
    for the fused kernel: bf16 coefficients [7 x 4680, r] times a bf16 basis [r, 1536] into bf16,
    with nothing else (no dequantization, RoPE or scatter), at the launch's rank r and at 2r (the
    fused fp16x2 product's MFMA work).  Median of ``reps`` launches timed with events."""
    rows = CHUNKS * TOKENS
    generator = torch.Generator(device=device).manual_seed(11)
    out = {}
    for name, rank in (("K", RANK_K), ("V", RANK_V)):
        entry = {}
        for label, inner in (("rank", rank), ("equal_mfma_work", 2 * rank)):
            a = torch.randn(rows, inner, device=device, dtype=torch.bfloat16, generator=generator)
            b = torch.randn(inner, CHANNELS, device=device, dtype=torch.bfloat16, generator=generator)
            for _ in range(3):
                torch.mm(a, b)
            times = []
            for _ in range(reps):
                begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                begin.record()
                torch.mm(a, b)
                end.record()
                end.synchronize()
                times.append(begin.elapsed_time(end) * 1e3)
            entry[label] = {"k": inner, "us": round(float(np.median(times)), 2)}
            del a, b
        out[name] = entry
    torch.cuda.synchronize(device)
    return {"what": "torch.mm (hipBLASLt) bf16 [32760, k] x [k, 1536] -> bf16, k = the launch's rank and twice it "
                    "(the fp16x2 product's MFMA work); compare restore_launch_us (which also dequantizes, "
                    "rotates and scatters)", **out}


def overlap_leg(layers, device, gemm=4096):
    """The CausVid step as a layer-overlapped restore (``overlapped_restore``): a producer thread
    restores the layers in order on a private stream while a consumer stream runs a stand-in
    forward that waits for each layer before computing it.  The stand-in layer is a run of bf16
    [gemm x gemm] products calibrated to the reference's per-layer compute c(h) at this history
    (h = CHUNKS).  Reports the forward alone, the eager restore alone and the overlapped wall time;
    the exposed restore is overlapped - forward."""
    from reelcache_amd.overlapped_restore import start_overlapped_restore

    a = torch.randn(gemm, gemm, device=device, dtype=torch.bfloat16)
    b = torch.randn(gemm, gemm, device=device, dtype=torch.bfloat16)
    consumer = torch.cuda.Stream(device)
    layer_ms = CAUSVID_LAYER_MS[0] + CAUSVID_LAYER_MS[1] * CHUNKS
    with torch.cuda.stream(consumer):
        for _ in range(3):
            a @ b
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(consumer)
        for _ in range(20):
            a @ b
        stop.record(consumer)
    stop.synchronize()
    reps = max(1, round(layer_ms / (start.elapsed_time(stop) / 20)))

    def forward(readiness=None):
        with torch.cuda.stream(consumer):
            out = None
            for layer in range(len(layers)):
                if readiness is not None:
                    readiness.layer(layer).wait(consumer)
                for _ in range(reps):
                    out = a @ b
        return out

    forward()
    torch.cuda.synchronize(device)
    begin = time.perf_counter()
    forward()
    consumer.synchronize()
    forward_ms = (time.perf_counter() - begin) * 1e3
    stream = torch.cuda.Stream(device)
    torch.cuda.synchronize(device)
    begin = time.perf_counter()
    with torch.cuda.stream(stream):
        for handle in restore_step(layers, stream):
            handle.release()
    stream.synchronize()
    restore_ms = (time.perf_counter() - begin) * 1e3
    torch.cuda.synchronize(device)
    begin = time.perf_counter()
    # Device clock of the overlapped run: `origin` on the consumer stream before anything starts
    # (the restore is ordered after it), then per layer the consumer's need (it reached the layer)
    # and its start (the layer's readiness wait passed); the readiness dates each layer's release.
    origin = torch.cuda.Event(enable_timing=True)
    origin.record(consumer)
    readiness = start_overlapped_restore(layers, device=device, wait_event=origin)
    marks = []
    with torch.cuda.stream(consumer):
        for layer in range(len(layers)):
            needed, started = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            needed.record(consumer)
            readiness.layer(layer).wait(consumer)
            started.record(consumer)
            for _ in range(reps):
                a @ b
            marks.append((needed, started))
        finished = torch.cuda.Event(enable_timing=True)
        finished.record(consumer)
    consumer.synchronize()
    overlapped_ms = (time.perf_counter() - begin) * 1e3
    readiness.join(timeout=120)
    readiness.quiesce(timeout=120)
    waits = readiness.timeline()["waited_seconds"]
    ready = readiness.device_ready_ms(origin)
    torch.cuda.synchronize(device)
    per_layer = []
    for layer, ((needed, started), ready_ms) in enumerate(zip(marks, ready)):
        deadline = layer * layer_ms  # the consumer reaches layer L after L layers of compute c(h)
        per_layer.append({"layer": layer, "ready_ms": round(ready_ms, 3), "deadline_ms": round(deadline, 3),
                          "slack_ms": round(deadline - ready_ms, 3),
                          "needed_ms": round(origin.elapsed_time(needed), 3),
                          "stall_ms": round(needed.elapsed_time(started), 3)})
    device_ms = origin.elapsed_time(finished)
    return {"layers": len(layers), "history_chunks": CHUNKS, "deadline_ms_per_layer": round(layer_ms, 3),
            "per_layer": per_layer,
            "layers_ready_by_deadline": sum(entry["slack_ms"] >= 0 for entry in per_layer),
            "min_slack_ms": min(entry["slack_ms"] for entry in per_layer),
            "consumer_stall_ms": round(sum(entry["stall_ms"] for entry in per_layer), 3),
            "overlapped_device_ms": round(device_ms, 3),
            "contention_ms": round(device_ms - forward_ms, 3),
            "forward_stand_in": f"{reps} bf16 [{gemm} x {gemm}] products per layer (c(h) = 2.58 + 0.486 h ms, "
                                "reelcache/decoded_tier.py:49-50)",
            "forward_ms": round(forward_ms, 3), "restore_eager_ms": round(restore_ms, 3),
            "overlapped_ms": round(overlapped_ms, 3),
            "exposed_restore_ms": round(overlapped_ms - forward_ms, 3),
            "consumer_host_wait_ms": round(sum(waits) * 1e3, 3),
            "what": "wall times; the overlapped run restores layer L on a private stream while the "
                    "consumer's layer L waits for it (LayerReadiness).  per_layer (device clock from the "
                    "run's start): ready_ms = the layer's restore writes ended, deadline_ms = L x c(h) "
                    "(when a forward running at c(h) per layer reaches it), needed_ms = when this "
                    "consumer reached it, stall_ms = its wait there; contention_ms = overlapped device "
                    "time - forward alone (the forward slowed by sharing the GPU plus any stalls)"}


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--cpu-seconds", type=float, default=20.0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--fit-steps", type=int, default=8, help="timed fit chunks (0 skips the fit leg)")
    parser.add_argument("--fit-warmup", type=int, default=2)
    parser.add_argument("--longcat-layers", type=int, default=2,
                        help="LongCat-shape layers timed beside the headline (0 skips the leg)")
    parser.add_argument("--no-overlap-leg", dest="overlap_leg", action="store_false",
                        help="skip the layer-overlapped restore beside a stand-in forward")
    parser.add_argument("--no-vendor-gemm-leg", dest="vendor_gemm_leg", action="store_false",
                        help="skip timing the library GEMM on the restore launches' shapes")
    parser.add_argument("--no-fp16-leg", dest="fp16_leg", action="store_false",
                        help="skip the step timed in the single-product fp16 precision mode")
    parser.add_argument("--pictures-layers", type=int, default=4,
                        help="layers restored from picture canvases beside the headline (0 skips the leg)")
    parser.add_argument("--fit-kernel-probe", action="store_true",
                        help="run the fit chunk's device kernels once each on 60 seeded Gaussian sources (absmax, "
                             "Gram, projection, residual energies) without the planner: the dispatches counter "
                             "passes summarize")
    parser.add_argument("--copy-probe", action="store_true",
                        help="after the timed region, run 3 plain device copies of 256 MiB (the calibration "
                             "dispatches for rocprofv3 FETCH_SIZE / WRITE_SIZE passes)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (the restore would shard by layer or head "
                                   "with no exchange between GPUs); run with --gpus 1"}))
        sys.exit(2)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    layers = build_workload(device)
    stream = torch.cuda.Stream(device)
    variants = []
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            for handle in restore_step(layers, stream):
                handle.release()
                variants = handle.stats["variants"]
    torch.cuda.synchronize(device)

    # Eager steps (no graph): the host plans and enqueues every reconstruct call.  Timed without
    # stage events (3 steps, the median), then one step with kernel-stage events on the launch
    # stream for the per-layer latency and kernel time.
    from reelcache_amd import restore_kernels as rk

    eager_runs = []
    for _ in range(3):
        torch.cuda.synchronize(device)
        begin = time.perf_counter()
        with torch.cuda.stream(stream):
            handles = restore_step(layers, stream)
        enqueued_at = time.perf_counter() - begin
        torch.cuda.synchronize(device)
        eager_runs.append((time.perf_counter() - begin, enqueued_at))
        for handle in handles:
            handle.release()
    eager_s, enqueued = sorted(eager_runs)[1]
    stage_log = []
    torch.cuda.synchronize(device)
    with torch.cuda.stream(stream):
        handles = restore_step(layers, stream, stage_log)
    torch.cuda.synchronize(device)
    for handle in handles:
        handle.release()
    layer_ms = []
    kernel_ms = []
    pack_ms = []
    launch_ms = []  # per layer call: duration of each restore launch, in launch order
    for stage in stage_log:
        marks = dict(stage)
        # start -> pack: the basis pack launch; pack -> fused: the restore launches (K, V).
        layer_ms.append(marks["start"].elapsed_time(marks["fused"]))
        kernel_ms.append(marks["pack"].elapsed_time(marks["fused"]))
        pack_ms.append(marks["start"].elapsed_time(marks["pack"]))
        names = [name for name, _ in stage]
        after = [event for name, event in stage[names.index("pack"):] if name == "pack" or name.startswith("launch")]
        launch_ms.append([a.elapsed_time(b) for a, b in zip(after, after[1:])])

    # The timed step: one full restore step (30 reconstruct calls: descriptor upload, basis pack
    # and restore launches per layer) captured once in a HIP graph and replayed, so the step
    # runs at the device's pace instead of the Python planner's.
    rk.reserve_capture_staging(LAYERS * (64 << 10))
    graph = torch.cuda.CUDAGraph()
    capture_stream = torch.cuda.Stream(device)
    capture_stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.graph(graph, stream=capture_stream):
        captured = restore_step(layers, capture_stream)  # kept alive with the graph
    torch.cuda.synchronize(device)
    graph.replay()  # warm replay
    torch.cuda.synchronize(device)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(device)
    begin = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        graph.replay()
    stop.record()
    torch.cuda.synchronize(device)
    wall = time.perf_counter() - begin
    gpu_ms = start.elapsed_time(stop)
    ms_per_step = gpu_ms / args.steps
    written, algorithmic = layer_bytes()
    value = LAYERS * written / (ms_per_step / 1e3) / 1e9
    kernel_avg = float(np.mean(kernel_ms))
    # Live per-launch durations (HIP events on the launch stream around each launch of the
    # stage-event step), the pack before them: one pair launch per layer call (K and V groups
    # together, the default), or K then V when the groups launch one by one.
    launch_us = [float(v) * 1e3 for v in np.mean(np.array(launch_ms), axis=0)]
    pack_us = float(np.mean(pack_ms)) * 1e3
    profile = profile_figures()
    pack_bytes = 2 * (RANK_K + RANK_V) * CHANNELS * 2
    if len(launch_us) == 1:
        launches = (("KV", launch_bytes(RANK_K) + launch_bytes(RANK_V), launch_us[0]),)
        kernel = ("restore_pair_kernel<4, 2, 8, 12>: the K (7 jobs, rank 128, RoPE) and V (7 jobs, rank 192) launch "
                  "groups of a layer call in one launch")
    else:
        launches = (("K", launch_bytes(RANK_K), launch_us[0]), ("V", launch_bytes(RANK_V), launch_us[1]))
        kernel = ("restore_fast_kernel<4, 12, false, 2, 2, 1>: the V launch of a layer call (7 jobs, rank 192), the "
                  "longest of the call's launches")
    split = {}
    for name, nbytes, us in launches + (("pack", pack_bytes, pack_us),):
        entry = {"us": round(us, 2), "algorithmic_bytes": nbytes, "achieved_gbs": round(nbytes / us / 1e3, 1),
                 "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
        if f"traffic_bytes_per_launch {name}" in profile:
            entry["traffic"] = int(profile[f"traffic_bytes_per_launch {name}"])
            entry["rocprof_us"] = profile[f"trace_us {name}"]
        if f"mfma_busy {name}" in profile:
            entry["mfma_busy"] = profile[f"mfma_busy {name}"]
        split[name] = entry
    dominant = split[launches[-1][0]]
    launches_avg = sum(launch_us) / 1e3
    achieved = dominant["achieved_gbs"]
    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u8->fp16x2 MFMA->bf16", "data": "synthetic (seeded codes, orthonormal bases)",
        "config": {"workload": "CausVid/Wan-1.3B-shape restore (BASELINE configs[1]): 30 layers x {K,V}, "
                               "7 chunks x 4680 tokens, 12x128, r_K=128 r_V=192, bf16 basis, Wan 3-D RoPE",
                   "precision": "fp16x2", "layers": LAYERS, "tokens": HISTORY, "channels": CHANNELS},
        "per_layer_latency_us": round(float(np.mean(layer_ms)) * 1e3, 2),
        "per_layer_latency_p50_us": round(float(np.median(layer_ms)) * 1e3, 2),
        "restore_kernel_us": round(kernel_avg * 1e3, 2),
        "pack_us": round(float(np.mean(pack_ms)) * 1e3, 2),
        "restore_launch_us": [round(float(v) * 1e3, 2) for v in np.mean(np.array(launch_ms), axis=0)],
        "wall_s": round(wall, 3),
        "execution": "HIP graph replay of one captured restore step (30 reconstruct calls)",
        "eager": {"ms_per_step": round(eager_s * 1e3, 3),
                  "value": round(LAYERS * written / eager_s / 1e9, 2),
                  "host_us_per_layer_call": round(enqueued / LAYERS * 1e6, 1),
                  "what": "median of 3 eager steps (30 reconstruct calls each, no graph, no stage events): "
                          "host planning + enqueue overlapped with the device"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": dominant.get("traffic"),
                     # The same ratio over the committed rocprofv3 kernel-trace duration of this launch.
                     "rocprof_us": dominant.get("rocprof_us"),
                     "frac_rocprof": round(dominant["algorithmic_bytes"] / dominant["rocprof_us"] / 1e3 / HBM_PEAK_GBS, 4)
                     if dominant.get("rocprof_us") else None,
                     "kernel": kernel,
                     "algorithmic_bytes_per_launch": dominant["algorithmic_bytes"],
                     "launch_us": dominant["us"],
                     "traffic_source": "profiles/restore_causvid_counters.md (rocprofv3 FETCH_SIZE + WRITE_SIZE per "
                                       "dispatch, calibrated on 256 MiB copies)",
                     "split": split,
                     "layer_call": {"launches_us": round(launches_avg * 1e3, 2),
                                    "algorithmic_bytes": algorithmic,
                                    "achieved_gbs": round(algorithmic / (launches_avg / 1e3) / 1e9, 1),
                                    "traffic": int(profile["traffic_bytes_per_layer_call"])
                                    if "traffic_bytes_per_layer_call" in profile else None,
                                    "mfma_tflops": round(2 * layer_flops() / (launches_avg / 1e3) / 1e12, 1)}},
        "layer_gpu": {"us": round(float(np.mean(layer_ms)) * 1e3, 2),
                      "achieved_gbs": round(algorithmic / (float(np.mean(layer_ms)) / 1e3) / 1e9, 1),
                      "what": "one eager layer call on the device, first launch (basis pack) to last restore launch "
                              "(events on the launch stream; includes launch gaps)"},
        "fit_chunks_per_s": None,
    }
    print(f"restore: {ms_per_step:.2f} ms/step, kernel {kernel_avg * 1e3:.1f} us/layer", file=sys.stderr, flush=True)
    if args.fp16_leg:
        result["fp16"] = fp16_leg(layers, device, args.steps)
    if args.overlap_leg:
        result["overlap"] = overlap_leg(layers, device)
    if args.vendor_gemm_leg:
        result["vendor_gemm"] = vendor_gemm_leg(device)
    if args.copy_probe:
        source = torch.empty(COPY_PROBE_BYTES, dtype=torch.uint8, device=device).fill_(7)
        target = torch.empty_like(source)
        for _ in range(3):
            target.copy_(source)
        torch.cuda.synchronize(device)
        del source, target
    del graph, captured
    if args.pictures_layers > 0:
        result["pictures"] = pictures_leg(layers[:args.pictures_layers], device)
    del layers, handles
    torch.cuda.empty_cache()
    if args.longcat_layers > 0:
        result["longcat"] = longcat_leg(device, args.longcat_layers, 3)
    if args.fit_steps > 0:
        result.update(fit_leg(device, args.fit_steps, args.fit_warmup,
                              0.0 if args.no_cpu_baseline else args.cpu_seconds))
    if args.fit_kernel_probe:
        result["fit_kernel_probe"] = fit_kernel_probe(device)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
