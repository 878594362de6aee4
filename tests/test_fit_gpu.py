"""GPU parity of the fit kernels (through the C ABI) against the FP64 oracle.

* absmax: exact; non-finite sources flagged.
* Gram: exactly symmetric; within the fp32 summation bound of the FP64 Gram of the exact values.
* projection: the fp32 rounding of the FP64 dot product -- equal to the oracle except for
  elements within ~1e-13 relative of an fp32 rounding boundary (at most one ulp); the fused
  per-column extrema are exactly the min / max of the returned coefficients.
* energies: FP64, relative 1e-12 of the oracle.
* quantizer: codes bit-exact with the oracle on the same coefficients and affine.
* Cholesky factor and inverse (CholeskyQR): relative 1e-12 of numpy's FP64 factorization;
  LAPACK's info convention for indefinite members.
"""

import functools

import numpy as np
import pytest
import torch

from oracle import fit as of
from oracle import quantize as oq
from reelcache_amd import fit_kernels as fk
from reelcache_amd import quantize as pq

pytestmark = pytest.mark.gpu

DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _source(rng, rows, channels, dtype, device, spectrum=False):
    if spectrum:
        x = of.decaying_spectrum(rng, rows, channels)
    else:
        x = (rng.standard_normal((rows, channels)) * rng.lognormal(0, 1, channels)).astype(np.float32)
    tensor = torch.from_numpy(x).to(DTYPES[dtype]).to(device)
    return tensor, tensor.float().cpu().numpy()


def _basis(rng, rank, channels, device):
    q, _ = np.linalg.qr(rng.standard_normal((channels, rank)))
    basis = of.stored_basis(q.T)
    return torch.from_numpy(basis).to(device), basis


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_absmax_exact_and_nonfinite(device, dtype):
    rng = np.random.default_rng(10)
    a, a_host = _source(rng, 300, 136, dtype, device)
    b, b_host = _source(rng, 65, 136, dtype, device)
    c, _ = _source(rng, 64, 136, dtype, device)
    c[17, 99] = float("inf")
    keys = fk.absmax([a, b, c]).cpu().numpy().astype(np.uint32)
    assert keys[0].view(np.float32) == np.abs(a_host).max()
    assert keys[1].view(np.float32) == np.abs(b_host).max()
    assert keys[2] >= fk.NONFINITE_BITS


@pytest.mark.parametrize("dtype,rows,channels", [("bfloat16", 300, 136), ("float16", 257, 256),
                                                 ("float32", 129, 200), ("bfloat16", 4680, 1536),
                                                 ("float16", 97, 520), ("float32", 70, 392), ("bfloat16", 33, 768)])
def test_gram_symmetric_and_within_fp32_bound(device, dtype, rows, channels):
    rng = np.random.default_rng(11)
    sources, hosts = zip(*[_source(rng, rows - 7 * i, channels, dtype, device) for i in range(2)])
    grams = fk.gram(list(sources)).cpu().numpy()
    for gram, host in zip(grams, hosts):
        np.testing.assert_array_equal(gram, gram.T)  # exactly symmetric
        expected = of.gram(host)
        bound = (host.shape[0] + 2) * 2.0 ** -24 * (np.abs(host).T.astype(np.float64) @ np.abs(host))
        assert np.all(np.abs(gram - expected) <= bound + 1e-30)


def test_gram_pads_unaligned_channels(device):
    rng = np.random.default_rng(12)
    x, host = _source(rng, 50, 13, "float32", device)
    gram = fk.gram([x]).cpu().numpy()
    assert gram.shape == (1, 13, 13)
    np.testing.assert_allclose(gram[0], of.gram(host), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype,rows,channels,rank", [("bfloat16", 300, 136, 40), ("float16", 129, 256, 64),
                                                      ("float32", 100, 64, 7), ("bfloat16", 4680, 1536, 128)])
def test_projection_rounds_the_fp64_product(device, dtype, rows, channels, rank):
    rng = np.random.default_rng(13)
    x, host = _source(rng, rows, channels, dtype, device)
    q, q_host = _basis(rng, rank + 3, channels, device)
    (p,), keys = fk.project([x], [q], [rank], extrema=True)
    p = p.cpu().numpy()
    expected = of.project(host, q_host, rank)
    differ = p != expected
    assert differ.mean() <= 1e-4
    if differ.any():
        ulp = np.abs(p[differ].view(np.int32).astype(np.int64) - expected[differ].view(np.int32).astype(np.int64))
        assert ulp.max() <= 1
    low, high = fk.split_keys(keys[0].cpu().numpy(), rank)
    np.testing.assert_array_equal(low, p.min(0))
    np.testing.assert_array_equal(high, p.max(0))


def test_projection_batch_of_ragged_ranks(device):
    rng = np.random.default_rng(14)
    xs, hosts, qs, q_hosts = [], [], [], []
    ranks = [5, 32, 61]
    for i, rank in enumerate(ranks):
        x, host = _source(rng, 90 + 31 * i, 64, "bfloat16", device)
        q, q_host = _basis(rng, rank, 64, device)
        xs.append(x), hosts.append(host), qs.append(q), q_hosts.append(q_host)
    coefficients, _ = fk.project(xs, qs, ranks)
    for p, host, q_host, rank in zip(coefficients, hosts, q_hosts, ranks):
        expected = of.project(host, q_host, rank)
        assert p.shape == expected.shape
        assert (p.cpu().numpy() == expected).mean() >= 0.999


def test_basis_layouts_read_in_place_or_repadded_give_the_same_values(device):
    """A stored basis is read in place when its rows are unit-stride, 16-byte aligned and 16-byte
    pitched, else through a zero-padded copy.  Row-major, column-major (a transposed view), a row
    block at an odd element offset and a wider pitch must all give the same coefficients and
    energies, bit for bit."""
    rng = np.random.default_rng(41)
    channels, rank = 128, 24
    x, _ = _source(rng, 300, channels, "bfloat16", device, spectrum=True)
    q, _ = _basis(rng, rank, channels, device)
    column_major = q.T.contiguous().T                      # strides (1, rank)
    wide = torch.zeros((rank, channels + 8), dtype=q.dtype, device=device)
    wide[:, :channels] = q
    pitched = wide[:, :channels]                            # row pitch 136 elements (272 bytes)
    shifted_storage = torch.zeros(rank * channels + 1, dtype=q.dtype, device=device)
    shifted = shifted_storage[1:].view(rank, channels)      # address 2 bytes past a 16-byte boundary
    shifted.copy_(q)
    layouts = [q, column_major, pitched, shifted]
    assert column_major.stride() == (1, rank) and shifted.data_ptr() % 16 == 2
    keys = fk.absmax([x] * len(layouts))
    coefficients, extrema = fk.project([x] * len(layouts), layouts, [rank] * len(layouts), extrema=True)
    totals = fk.energies([x] * len(layouts), keys, bases=layouts, ranks=[rank] * len(layouts),
                         coefficients=coefficients).cpu().numpy()
    for p, total, row in zip(coefficients[1:], totals[1:], extrema[1:]):
        assert torch.equal(p, coefficients[0])
        assert np.array_equal(total, totals[0])
        assert torch.equal(row, extrema[0])


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_energies_match_fp64(device, dtype):
    rng = np.random.default_rng(15)
    x, host = _source(rng, 1000, 256, dtype, device, spectrum=True)
    y, y_host = _source(rng, 77, 256, dtype, device)
    q, q_host = _basis(rng, 24, 256, device)
    r, r_host = _basis(rng, 3, 256, device)
    keys = fk.absmax([x, y])
    coefficients, _ = fk.project([x, y], [q, r], [24, 3])
    totals = fk.energies([x, y], keys, bases=[q, r], ranks=[24, 3], coefficients=coefficients).cpu().numpy()
    for total, host_x, basis, p, rank in zip(totals, (host, y_host), (q_host, r_host), coefficients, (24, 3)):
        _, source, error = of.energies(host_x, basis, p.cpu().numpy(), rank)
        assert total[0] == pytest.approx(source, rel=1e-12)
        assert total[1] == pytest.approx(error, rel=1e-12)
    source_only = fk.energies([x], fk.absmax([x])).cpu().numpy()
    assert source_only[0, 0] == pytest.approx(of.energies(host)[1], rel=1e-12)


def test_energies_on_both_rank_paths(device):
    """Ranks up to 64 keep the coefficient block in registers, larger ones stream it: a ragged batch
    over both paths (and a rank that is not a multiple of 4) matches the FP64 oracle, and so does the
    fp32 residual matrix X - P Q (rounded once from its FP64 value)."""
    rng = np.random.default_rng(21)
    ranks = [13, 48, 64, 65, 130]
    sources, hosts, bases, host_bases = [], [], [], []
    for index, rank in enumerate(ranks):
        x, host = _source(rng, 200 + 37 * index, 192, "bfloat16", device, spectrum=True)
        q, q_host = _basis(rng, rank, 192, device)
        sources.append(x)
        hosts.append(host)
        bases.append(q)
        host_bases.append(q_host)
    keys = fk.absmax(sources)
    coefficients, _ = fk.project(sources, bases, ranks)
    totals, residuals = fk.energies(sources, keys, bases=bases, ranks=ranks, coefficients=coefficients,
                                    residuals=True)
    totals = totals.cpu().numpy()
    for total, residual, host, basis, p, rank in zip(totals, residuals, hosts, host_bases, coefficients, ranks):
        p_host = p.cpu().numpy()
        _, source, error = of.energies(host, basis, p_host, rank)
        assert total[0] == pytest.approx(source, rel=1e-12), rank
        assert total[1] == pytest.approx(error, rel=1e-12), rank
        exact = of.as_float(host) - p_host.astype(np.float64) @ np.asarray(basis, np.float16).astype(np.float64)[:rank]
        got = residual.cpu().numpy()
        # FP64 sums in another order: the fp32 rounding agrees except next to a rounding boundary.
        assert (got == exact.astype(np.float32)).mean() >= 0.999, rank
        assert np.abs(got - exact).max() <= 2 ** -23 * np.abs(exact).max(), rank


def test_zero_matrix_energies(device):
    x = torch.zeros((70, 64), dtype=torch.bfloat16, device=device)
    keys = fk.absmax([x])
    assert int(keys.cpu()[0]) == 0
    assert fk.energies([x], keys).cpu().numpy().tolist() == [[0.0, 0.0]]


@functools.lru_cache(maxsize=1)
def _causvid_spectrum():
    rng = np.random.default_rng(16)
    return of.decaying_spectrum(rng, 4680, 1536), np.linalg.qr(rng.standard_normal((1536, 32)))[0].T


@pytest.mark.parametrize("normalization,fraction", [("per_channel", 1.0), ("global", 0.0), ("leading_columns", 0.25)])
def test_quantizer_bit_exact(device, normalization, fraction):
    x_host, rows = _causvid_spectrum()
    x = torch.from_numpy(x_host).to(torch.bfloat16).to(device)
    q = torch.from_numpy(of.stored_basis(rows)).to(device)
    (p,), keys = fk.project([x], [q], [32], extrema=True)
    values = p.contiguous()
    layout = pq.normalization_layout(32, normalization, fraction)
    low, high = fk.split_keys(keys[0].cpu().numpy(), 32)
    affine = pq.affine_from_extrema(low, high, layout)
    scale, offset = pq.expanded_affine(affine, layout, 32)
    codes = fk.quantize(values, torch.from_numpy(np.asarray(scale, np.float64)).to(device),
                        torch.from_numpy(np.asarray(offset, np.float64)).to(device)).cpu().numpy()
    host_p = values.cpu().numpy()
    o_codes, o_affine, _ = oq.quantize(host_p, normalization, fraction)
    np.testing.assert_array_equal(affine, o_affine)
    np.testing.assert_array_equal(codes, o_codes)
    # The standalone extrema kernel agrees with the fused ones.
    low2, high2 = fk.split_keys(fk.column_extrema(values).cpu().numpy(), 32)
    np.testing.assert_array_equal(low2, low)
    np.testing.assert_array_equal(high2, high)


def test_batched_quantizer_matches_single_launches(device):
    rng = np.random.default_rng(17)
    values, affines = [], []
    for rows, cols in ((4680, 32), (700, 64), (1, 5), (129, 96)):
        v = torch.from_numpy((rng.standard_normal((rows, cols)) * 3).astype(np.float32)).to(device)
        lo, hi = v.amin(0).cpu().numpy(), v.amax(0).cpu().numpy()
        affine = pq.covering_affine(lo, hi).astype(np.float64)
        affine[0, 1] = 0.0  # a zero scale maps the column to code 0
        values.append(v)
        affines.append(affine)
    batched = fk.quantize_batched(values, affines)
    for v, affine, codes in zip(values, affines, batched):
        single = fk.quantize(v, torch.from_numpy(affine[0].copy()).to(device), torch.from_numpy(affine[1].copy()).to(device))
        np.testing.assert_array_equal(codes.cpu().numpy(), single.cpu().numpy())
        np.testing.assert_array_equal(codes.cpu().numpy(), oq.quantize_with_affine(v.cpu().numpy(), affine[0], affine[1]))


@pytest.mark.parametrize("k", [1, 7, 96, 128])
def test_cholesky_inverse_matches_fp64_factorization(device, k):
    """The batched factor-and-inverse launch of the planner's CholeskyQR steps against numpy's
    FP64 Cholesky (A = R^T R, R = L^T) and the exact triangular inverse: relative 1e-12 on
    well-conditioned matrices; R^-1 R = I; the lower triangle is zero."""
    from scipy.linalg import solve_triangular

    rng = np.random.default_rng(31 + k)
    batch = []
    for _ in range(5):
        q, _ = np.linalg.qr(rng.standard_normal((k, k)))
        batch.append((q * rng.uniform(1.0, 30.0, k)) @ q.T)  # condition <= 900
    a = np.stack(batch)
    inverse, info = fk.cholesky_inverse(torch.from_numpy(a).to(device))
    inverse, info = inverse.cpu().numpy(), info.cpu().numpy()
    assert (info == 0).all()
    for member, got in zip(a, inverse):
        r = np.linalg.cholesky(member).T
        want = solve_triangular(r, np.eye(k), lower=False)
        assert np.abs(got - want).max() <= 1e-12 * np.abs(want).max()
        assert np.abs(got @ r - np.eye(k)).max() <= 1e-12
        assert (np.tril(got, -1) == 0).all()


def test_cholesky_inverse_flags_indefinite_members(device):
    """LAPACK's info convention: j + 1 for the first leading minor that is not positive definite
    (a negative pivot at order 4, a NaN at order 1); such members come back as the identity and
    do not disturb the others."""
    k = 6
    good = np.diag(np.arange(1.0, k + 1.0))
    indefinite = np.diag([1.0, 2.0, 3.0, -1.0, 5.0, 6.0])
    nan = good.copy()
    nan[0, 0] = np.nan
    inverse, info = fk.cholesky_inverse(torch.from_numpy(np.stack([good, indefinite, nan])).to(device))
    assert info.cpu().tolist() == [0, 4, 1]
    inverse = inverse.cpu().numpy()
    np.testing.assert_allclose(inverse[0], np.diag(1.0 / np.sqrt(np.arange(1.0, k + 1.0))), rtol=1e-15)
    assert (inverse[1] == np.eye(k)).all() and (inverse[2] == np.eye(k)).all()
    with pytest.raises(Exception):
        fk.cholesky_inverse(torch.zeros((1, 129, 129), dtype=torch.float64, device=device))
