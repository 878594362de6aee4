"""GPU parity of the restore paths beside the fused product kernels.

* ``DenseSource`` rows through ``rch_rope_store`` (reelcache/restore_kernels.py:758-767,
  :1557-1585, :2124-2150): every layout x {no RoPE, dense, separable} x output dtype, against
  the oracle's FP64 rotation of the same values (bit-exact cast without RoPE);
* the exact ``native_rope`` path (reelcache/restore_kernels.py:2293-2321): RAW rows and
  factorized sources reconstructed pre-RoPE, handed to the engine's callable, copied into
  the slot, with the callable's arguments recorded as the reference's tests do
  (tests/test_restore_kernels.py:1229-1266);
* ``warmup`` (reelcache/restore_kernels.py:2669-2763): the report, a repeat that does no
  work, and a first real call afterwards within the oracle's bound;
* the separable kernel path with ``RopeTable.from_axes`` tables (per-axis row limits);
* a table's first use on one stream followed at once by a restore on another stream.
"""

import zlib

import numpy as np
import pytest
import torch

from oracle import restore as orc
from reelcache_amd import restore_kernels as rk

from restore_cases import TORCH_DTYPES, destination, expected, make_case, written

pytestmark = pytest.mark.gpu

GRID = (3, 4, 6)


def _rope_table(kind, head_dim, tokens, rng):
    if kind == "separable":
        return rk.RopeTable.from_complex(torch.from_numpy(orc.wan_freqs(head_dim, 64))), (2, 1, 3)
    angles = rng.uniform(0, 2 * np.pi, size=(tokens + 11, head_dim // 2))
    return rk.RopeTable.from_cos_sin(torch.from_numpy(np.cos(angles)).float(),
                                     torch.from_numpy(np.sin(angles)).float()), 7


def _rotation_bound(values, heads, rope, out_dtype):
    """(y*, bound) of the rope-store path: FP64 rotation of the exact input values; the fp32
    rotation without FMA is within 2**-21 (|y_e| + |y_o|) of it, then one cast."""
    tokens, channels = values.shape
    exact = values
    error = np.zeros_like(values)
    if rope is not None:
        exact = orc.apply_rope(values.reshape(tokens, heads, -1), *rope).reshape(tokens, channels)
        pairs = np.abs(exact).reshape(tokens, -1, 2)
        error = 2.0 ** -21 * np.repeat(pairs[..., 0] + pairs[..., 1], 2, axis=-1)
    unit = orc.UNIT_ROUNDOFF[out_dtype]
    return exact, unit * np.abs(exact) + (1 + unit) * error + orc.OUTPUT_FLOOR[out_dtype]


@pytest.mark.parametrize("layout", ["BTHD", "THD", "BHTD"])
@pytest.mark.parametrize("rope_kind", ["none", "dense", "separable"])
@pytest.mark.parametrize("out_dtype", ["bfloat16", "float16", "float32"])
def test_dense_source_rope_store(device, layout, rope_kind, out_dtype):
    rng = np.random.default_rng(zlib.crc32(f"dense/{layout}/{rope_kind}/{out_dtype}".encode()))
    heads, head_dim = 3, 64
    tokens, channels = int(np.prod(GRID)), heads * head_dim
    for source_dtype in (torch.float32, torch.bfloat16, torch.float16):
        values = torch.from_numpy(rng.standard_normal((tokens, channels)).astype(np.float32) * 3).to(source_dtype)
        tensor = destination(layout, tokens, heads, head_dim, out_dtype, device, offset=4, extra=2, fill=-77.0)
        positions, rope = None, None
        if rope_kind != "none":
            table, rows = _rope_table(rope_kind, head_dim, tokens, rng)
            positions = rk.RopePositions(table, rows)
            rope = orc.rope_cos_sin(table.cos.float().double().numpy(), table.sin.float().double().numpy(),
                                    table.sections, positions.rows, GRID)
        job = rk.ReconstructionJob(rk.DenseSource(values.to(device)), rk.NativeView(tensor, layout, token_offset=4),
                                   GRID, rope=positions)
        handle = rk.reconstruct([job])
        handle.synchronize()
        assert handle.stats["backend"] == "fused" and handle.stats["launches"] == 1
        out = job.destination.slot(tokens).reshape(tokens, channels).double().cpu().numpy()
        exact_in = values.double().numpy()
        if rope is None:
            # No rotation: one cast of the source value, bit for bit.
            np.testing.assert_array_equal(out, orc.cast(exact_in, out_dtype))
        else:
            exact, bound = _rotation_bound(exact_in, heads, rope, out_dtype)
            excess = np.abs(out - exact) - bound
            assert float(excess.max()) <= 0, f"{int((excess > 0).sum())} elements exceed the bound"
        canonical = (tensor.transpose(1, 2) if layout == "BHTD" else tensor).reshape(-1, channels)
        assert bool((canonical[:4] == -77.0).all()) and bool((canonical[4 + tokens:] == -77.0).all())


def test_dense_source_odd_head_geometry(device):
    """head_dim 24 (channel tiles of 16 straddle heads), fp32 rows with a padded row stride."""
    rng = np.random.default_rng(3)
    heads, head_dim, grid = 3, 24, (2, 3, 5)
    tokens, channels = 30, 72
    storage = torch.from_numpy(rng.standard_normal((tokens, channels + 8)).astype(np.float32)).to(device)
    values = storage[:, 3:3 + channels]
    table, rows = _rope_table("separable", head_dim, tokens, rng)
    positions = rk.RopePositions(table, rows)
    tensor = torch.zeros(1, tokens, heads, head_dim, dtype=torch.float32, device=device)
    job = rk.ReconstructionJob(rk.DenseSource(values), rk.NativeView(tensor), grid, rope=positions)
    rk.reconstruct([job]).synchronize()
    rope = orc.rope_cos_sin(table.cos.float().double().numpy(), table.sin.float().double().numpy(), table.sections,
                            positions.rows, grid)
    exact, bound = _rotation_bound(values.double().cpu().numpy(), heads, rope, "float32")
    out = tensor.reshape(tokens, channels).double().cpu().numpy()
    assert float((np.abs(out - exact) - bound).max()) <= 0


def _engine_rope(freqs, start):
    """An engine's own RoPE on [N, H, D] pre-RoPE values in their dtype (the callable the
    reference's tests pass): complex multiplication of interleaved pairs by the Wan table rows
    of each token, computed in float64 and returned in the input dtype."""

    def rotate(values, job):
        frames, height, width = job.grid
        f, y, x = orc.token_coordinates(job.grid)
        sections = orc.wan_sections(freqs.shape[1])
        table = np.concatenate([freqs[f + start, :sections[0]],
                                freqs[y, sections[0]:sections[0] + sections[1]],
                                freqs[x, sections[0] + sections[1]:]], axis=1)
        complex_values = values.double().cpu().numpy().reshape(values.shape[0], values.shape[1], -1, 2)
        z = (complex_values[..., 0] + 1j * complex_values[..., 1]) * table[:, None, :]
        out = np.stack((z.real, z.imag), axis=-1).reshape(values.shape)
        return torch.from_numpy(out).to(values.dtype).to(values.device)

    return rotate


def test_native_rope_raw_rows_identity(device):
    heads, head_dim, grid = 2, 16, (2, 3, 4)
    tokens = 24
    freqs = orc.wan_freqs(head_dim, 64)
    table = rk.RopeTable.from_complex(torch.from_numpy(freqs))
    generator = torch.Generator().manual_seed(11)
    raw = (torch.randn(tokens, heads * head_dim, generator=generator) * 4).bfloat16().to(device)
    cache = torch.zeros(1, 2 * tokens, heads, head_dim, dtype=torch.bfloat16, device=device)
    calls = []
    engine = _engine_rope(freqs, 5)

    def native(values, job):
        calls.append((values.dtype, tuple(values.shape), job.label))
        return engine(values, job)

    job = rk.ReconstructionJob(rk.DenseSource(raw), rk.NativeView(cache, token_offset=tokens), grid,
                               rope=rk.RopePositions(table, (5, 0, 0)), label="raw")
    rk.reconstruct([job], native_rope=native).synchronize()
    expected_rows = engine(raw.reshape(tokens, heads, head_dim), job)
    assert torch.equal(cache[0, tokens:], expected_rows)
    assert bool((cache[:, :tokens] == 0).all())
    assert calls == [(torch.bfloat16, (tokens, heads, head_dim), "raw")]


@pytest.mark.parametrize("precision", ["fp16x2", "fp32"])
def test_native_rope_factorized_source(device, precision):
    """uint8 codes reconstructed pre-RoPE into an fp32 temporary by the HIP kernels, rotated by
    the callable, cast into the bf16 slot; a V job of the same call (no RoPE) takes the fused path."""
    rng = np.random.default_rng(12)
    heads, head_dim, grid = 2, 32, (1, 4, 6)
    tokens, rank = 24, 20
    freqs = orc.wan_freqs(head_dim, 64)
    case = make_case(rng, grid=grid, heads=heads, head_dim=head_dim, rank=rank, source="uint8", rope="separable",
                     layout="THD", out_dtype="bfloat16", device=device,
                     table=rk.RopeTable.from_complex(torch.from_numpy(freqs)), rope_rows=(2, 0, 0))
    plain = make_case(rng, grid=grid, heads=heads, head_dim=head_dim, rank=rank, source="uint8", rope="none",
                      layout="THD", out_dtype="bfloat16", device=device)
    calls = []
    engine = _engine_rope(freqs, 2)

    def native(values, job):
        calls.append((values.dtype, tuple(values.shape)))
        return engine(values, job)

    handle = rk.reconstruct([case.job, plain.job], precision=precision, native_rope=native,
                            native_rope_dtype=torch.float32)
    handle.synchronize()
    assert calls == [(torch.float32, (tokens, heads, head_dim))]
    # The pre-RoPE product is within the fp32-output bound of the oracle; the engine's rotation (the
    # float64 table) moves each component's error by at most the pair's summed error, its float32
    # result adds one rounding, and the slot's bf16 cast one more.
    pre, pre_bound = orc.error_bound(case.coefficients, case.basis, heads, None, precision, "float32")
    table = case.job.rope.table
    rope64 = orc.rope_cos_sin(table.cos.numpy(), table.sin.numpy(), table.sections, (2, 0, 0), grid)
    rotated = orc.apply_rope(pre.reshape(tokens, heads, -1), *rope64).reshape(tokens, -1)
    pair_bound = np.repeat(pre_bound.reshape(tokens, -1, 2).sum(-1), 2, axis=-1)
    unit = orc.UNIT_ROUNDOFF["bfloat16"]
    bound = unit * np.abs(rotated) + (1 + unit) * (pair_bound + 2.0 ** -23 * np.abs(rotated)) + 2.0 ** -134
    out = written(case)
    assert float((np.abs(out - rotated) - bound).max()) <= 0
    values, plain_bound = expected(plain, precision)
    assert float((np.abs(written(plain) - values) - plain_bound).max()) <= 0


def test_warmup_then_first_call_matches_oracle(device):
    shapes = [rk.WarmupShape(3, 64, source="uint8", ranks=(16, 200)),
              {"heads": 2, "head_dim": 32, "source": "dense", "rope": "none", "dtype": torch.float32},
              rk.WarmupShape(2, 32, source="pictures", rope="native", native_rope_dtype=torch.float32, ranks=(5, 40))]
    report = rk.warmup(device, shapes, precision=("fp16x2", "fp16"))
    assert report["resolved_backend"] == "fused" and report["precisions"] == ["fp16x2", "fp16"]
    assert report["warmed"] == 6 and report["skipped"] == 0 and report["calls"] > 0 and report["launches"] > 0
    assert not report["repeat"]
    uint8_ranks = report["shapes"][0]["ranks"]
    assert uint8_ranks[0] >= 16 and uint8_ranks[-1] == 200  # one rank per reachable variant class
    again = rk.warmup(device, shapes, precision=("fp16x2", "fp16"))
    assert again["repeat"] and again["calls"] == 0 and again["skipped"] == 6
    # A first real call of a warmed shape.
    rng = np.random.default_rng(44)
    case = make_case(rng, grid=(2, 5, 7), heads=3, head_dim=64, rank=150, source="uint8", rope="separable",
                     device=device, basis_dtype=torch.bfloat16)
    rk.reconstruct([case.job]).synchronize()
    values, bound = expected(case, "fp16x2")
    assert float((np.abs(written(case) - values) - bound).max()) <= 0


def test_from_axes_table_on_the_kernel_path(device):
    """A from_axes table (per-axis rows, NaN elsewhere) through the straight-line kernel."""
    rng = np.random.default_rng(15)
    head_dim = 64
    sections = orc.wan_sections(head_dim // 2)
    axes = []
    for pairs, rows in zip(sections, (9, 5, 8)):
        angles = rng.uniform(-np.pi, np.pi, size=(rows, pairs))
        axes.append(torch.from_numpy(np.cos(angles) + 1j * np.sin(angles)))
    table = rk.RopeTable.from_axes(*axes)
    case = make_case(rng, grid=(3, 4, 6), heads=2, head_dim=head_dim, rank=48, source="uint8", table=table,
                     rope_rows=(6, 1, 2), device=device)
    handle = rk.reconstruct([case.job])
    handle.synchronize()
    assert handle.stats["variants"] == ["pairs"]
    values, bound = expected(case, "fp16x2")
    out = written(case)
    assert np.isfinite(out).all()
    assert float((np.abs(out - values) - bound).max()) <= 0


def test_table_first_used_on_another_stream(device):
    """A table's device copy (and its interleaved pairs) built by a call on stream A is used at
    once by a call on stream B: B must wait for the copy, so its values match the oracle."""
    rng = np.random.default_rng(16)
    for _ in range(3):
        table = rk.RopeTable.from_complex(torch.from_numpy(orc.wan_freqs(128, 64)))
        first = make_case(rng, grid=(3, 10, 12), heads=4, head_dim=128, rank=64, source="uint8", table=table,
                          device=device)
        second = make_case(rng, grid=(3, 10, 12), heads=4, head_dim=128, rank=64, source="uint8", table=table,
                           device=device)
        stream_a, stream_b = torch.cuda.Stream(device), torch.cuda.Stream(device)
        # Keep stream A busy so that its table upload and interleave finish late.
        busy = torch.randn(2048, 2048, device=device)
        with torch.cuda.stream(stream_a):
            for _ in range(8):
                busy = busy @ busy * 1e-3
        handle_a = rk.reconstruct([first.job], stream=stream_a)
        handle_b = rk.reconstruct([second.job], stream=stream_b)
        handle_a.synchronize()
        handle_b.synchronize()
        for case in (first, second):
            values, bound = expected(case, "fp16x2")
            assert float((np.abs(written(case) - values) - bound).max()) <= 0
