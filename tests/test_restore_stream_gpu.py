"""GPU parity of the basis-stationary stream kernel (csrc/restore_stream.h).

fp16x2 launch groups of uint8 code rows with head_dim 128 run it with
``config={"stream_variant": True}``.  Its arithmetic folds the affine into the basis (exact fp16 codes q - 128 times the fp16 hi + lo split of
s_k Q_kc, plus a per-channel FP64 bias), so it is held to the oracle's elementwise fp16x2 bound
(reelcache/restore_kernels.py:1208-1227) and, for fp32 destinations, to the same rel-Frobenius
level as the reference-order kernels -- not to their bits.  Cases cover every layout and output
dtype, bf16 and fp16 bases, ranks from 7 to 256 (tails inside a 16-rank step), ragged last
tiles, padded code rows, several jobs of different affines sharing one basis, affines with
constant columns and large offsets, and untouched neighbours.
"""

import zlib

import numpy as np
import pytest
import torch

from oracle import quantize as oq
from oracle import restore as orc
from reelcache_amd import restore_kernels as rk

from restore_cases import destination, expected, make_case, written

pytestmark = pytest.mark.gpu

STREAM = {"stream_variant": True}

# (layout, heads, rank, rope, grid, token_offset, code_pitch)
SHAPES = [
    ("BTHD", 3, 128, "separable", (3, 7, 11), 5, None),   # ragged last tile (231 tokens)
    ("THD", 2, 33, "dense", (2, 9, 13), 0, 48),             # rank tail inside a 16-rank step
    ("BHTD", 4, 150, "none", (1, 16, 8), 2, 160),            # exactly four tiles, padded rows
    ("BTHD", 12, 192, "none", (1, 20, 26), 0, None),        # V-shaped
    ("BTHD", 1, 7, "separable", (2, 3, 5), 1, 16),           # tiny rank, 30 tokens
    ("BTHD", 2, 256, "separable", (1, 9, 10), 0, None),     # 16 rank steps
]


def _check(case, frobenius=1e-5):
    values, bound = expected(case, "fp16x2")
    out = written(case)
    excess = np.abs(out - values) - bound
    assert float(excess.max()) <= 0, f"{int((excess > 0).sum())} elements exceed the fp16x2 error bound"
    if case.out_dtype == "float32":
        assert orc.relative_frobenius(out, values) <= frobenius


@pytest.mark.parametrize("out_dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("basis_dtype", [torch.bfloat16, torch.float16])
def test_stream_matches_oracle(device, out_dtype, basis_dtype):
    for index, (layout, heads, rank, rope, grid, token_offset, pitch) in enumerate(SHAPES):
        rng = np.random.default_rng(zlib.crc32(f"stream/{out_dtype}/{basis_dtype}/{index}".encode()))
        case = make_case(rng, grid=grid, heads=heads, head_dim=128, rank=rank, source="uint8", rope=rope,
                         layout=layout, out_dtype=out_dtype, device=device, token_offset=token_offset,
                         code_pitch=pitch, basis_dtype=basis_dtype)
        handle = rk.reconstruct([case.job], config=STREAM)
        handle.release()
        assert handle.stats["variants"] == ["stream"], (index, handle.stats["variants"])
        _check(case)
        tensor = case.job.destination.tensor
        canonical = (tensor.transpose(1, 2) if layout == "BHTD" else tensor).reshape(-1, heads * 128)
        tokens = int(np.prod(grid))
        assert bool((canonical[:token_offset] == -123.0).all())
        assert bool((canonical[token_offset + tokens:] == -123.0).all())


def test_stream_layer_call_shares_a_basis(device):
    """A layer call of K and V jobs over 3 chunks (different affines, one basis per target):
    two stream launches, every slot within the bound, and at most a few percent of bf16 outputs
    differ from the reference-order straight-line kernel."""
    rng = np.random.default_rng(81)
    heads, grid = 6, (2, 10, 13)
    tokens = int(np.prod(grid))
    table = rk.RopeTable.from_complex(torch.from_numpy(orc.wan_freqs(128, 64)))
    bases = [torch.from_numpy(np.linalg.qr(rng.standard_normal((heads * 128, r)))[0].T.copy()).to(torch.bfloat16)
             .to(device) for r in (128, 192)]
    caches = [destination("BTHD", 3 * tokens, heads, 128, "bfloat16", device) for _ in range(2)]
    cases = []
    for chunk in range(3):
        cases.append(make_case(rng, grid=grid, heads=heads, head_dim=128, rank=128, source="uint8", table=table,
                               rope_rows=(2 * chunk, 0, 0), view=rk.NativeView(caches[0], token_offset=chunk * tokens),
                               basis=bases[0], device=device))
        cases.append(make_case(rng, grid=grid, heads=heads, head_dim=128, rank=192 - 16 * chunk, source="uint8",
                               rope="none", view=rk.NativeView(caches[1], token_offset=chunk * tokens),
                               basis=bases[1], device=device))
    handle = rk.reconstruct([case.job for case in cases], config=STREAM)
    handle.release()
    assert handle.stats["variants"] == ["stream", "stream"] and handle.stats["launches"] == 3  # pack + K + V
    stream_out = [written(case) for case in cases]
    for case in cases:
        _check(case)
    rk.reconstruct([case.job for case in cases], config={"stream_variant": False}).release()
    for case, ours in zip(cases, stream_out):
        differ = float((written(case) != ours).mean())
        assert differ <= 0.05, f"{differ:.4f} of outputs differ from the reference-order kernel"


def test_stream_affine_edge_cases(device):
    """Constant columns (scale 0), large offsets against small ranges and negative-only ranges:
    the folded bias carries the offsets exactly enough to stay within the bound."""
    rng = np.random.default_rng(82)
    heads, rank, grid = 2, 64, (1, 8, 12)
    tokens = int(np.prod(grid))
    basis = torch.from_numpy(np.linalg.qr(rng.standard_normal((heads * 128, rank)))[0].T.copy()).half().to(device)
    lo = np.concatenate([np.full(16, 3.0), np.full(16, -1000.0), rng.uniform(-4, 0, 32)]).astype(np.float32)
    hi = np.concatenate([np.full(16, 3.0), np.full(16, -999.5), lo[32:] + rng.uniform(0.5, 6, 32)]).astype(np.float32)
    scale, offset = oq.covering_affine(lo, hi)
    codes = rng.integers(0, 256, size=(tokens, rank), dtype=np.uint8)
    out = torch.full((1, tokens, heads, 128), -9.0, dtype=torch.float32, device=device)
    job = rk.ReconstructionJob(rk.CoefficientSource(torch.from_numpy(codes).to(device), scale, offset),
                               rk.NativeView(out), grid, basis, rank)
    handle = rk.reconstruct([job], config=STREAM)
    handle.release()
    assert handle.stats["variants"] == ["stream"]
    coefficients = orc.dequantize(codes, scale, offset)
    values, bound = orc.error_bound(coefficients, basis.double().cpu().numpy(), heads, None, "fp16x2", "float32")
    got = out.reshape(tokens, -1).double().cpu().numpy()
    assert float((np.abs(got - values) - bound).max()) <= 0
    assert orc.relative_frobenius(got, values) <= 1e-6


def test_stream_static_scratch_equals_default(device):
    """The stream groups' slabs packed into the library's static array (rch_restore_noalloc)
    give the same bits as the call-owned buffer."""
    rng = np.random.default_rng(83)
    outs = []
    for config in (STREAM, {**STREAM, "static_scratch": True}):
        rng = np.random.default_rng(83)
        cases = [make_case(rng, grid=(2, 8, 9), heads=4, head_dim=128, rank=rank, source="uint8", rope=rope,
                           device=device) for rank, rope in ((96, "separable"), (160, "none"))]
        handle = rk.reconstruct([case.job for case in cases], config=config)
        handle.release()
        assert handle.stats["variants"] == ["stream", "stream"]
        outs.append([written(case) for case in cases])
        for case in cases:
            _check(case)
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
