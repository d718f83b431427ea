"""Float64 pins of the oracle's multi-chunk softmax statistics and residual
sampler (oracle/vxo.c vxo_row_softmax_stats, vxo_sample_residual).

The reference has no stochastic acceptance (src/paged/spec.rs:25-49 is greedy
only), so these functions are pinned by mathematics instead:

* the row statistics (m, Z) against a float64 log-sum-exp of the same row,
  at vocabularies that span many 8192-element chunks and with the maximum
  placed in the first, a middle, the last full and the partial tail chunk
  (a missing chunk rescale or a dropped chunk moves Z by orders of magnitude);
* the inverse-CDF draw against a float64 prefix sum: the returned index must
  own (up to a rounding band) the CDF interval that u * total falls into,
  with probability mass planted on the elements either side of every 256- and
  8192-element boundary, so an off-by-one at a sub-chunk or chunk edge, or a
  chunk walked out of order, lands on a neighbour whose interval is far away;
* a chi-square test of many draws whose mass straddles those boundaries, for
  both the plain draw (q absent) and the residual max(0, p - q).
"""
import numpy as np
import pytest

import vxo

V_LARGE = 151936  # Qwen3 vocabulary: 18 full chunks of 8192 and a partial one


def lse_f64(row: np.ndarray, inv_t: float):
    x = row.astype(np.float64)
    m = x.max()
    return m, np.exp((x - m) * np.float64(inv_t)).sum()


@pytest.mark.parametrize("where", [3, 5 * 8192 + 17, 17 * 8192 + 4000, V_LARGE - 1])
@pytest.mark.parametrize("inv_t", [np.float32(1) / np.float32(0.8), np.float32(1) / np.float32(0.7), np.float32(1.0)])
def test_softmax_stats_match_float64_lse(where, inv_t):
    rng = np.random.default_rng(where)
    row = rng.normal(0.0, 3.0, size=V_LARGE).astype(np.float32)
    # heavy mass in chunk 0 while the maximum sits elsewhere: every chunk's
    # partial sum has to be rescaled to the global maximum
    row[:64] += 9.0
    row[where] = row.max() + 2.5
    m, z = vxo.row_softmax_stats(row, float(inv_t))
    m64, z64 = lse_f64(row, float(inv_t))
    assert m == np.float32(m64)
    assert abs(z - z64) <= 2e-5 * z64, (z, z64)


def test_softmax_stats_edge_rows():
    inv_t = float(np.float32(1.25))
    # all equal: Z = vocab exactly representable in the chunked sums
    row = np.full(20000, 3.0, np.float32)
    m, z = vxo.row_softmax_stats(row, inv_t)
    assert m == 3.0 and z == 20000.0
    # a single finite element, the rest -inf
    row = np.full(V_LARGE, -np.inf, np.float32)
    row[9 * 8192 + 255] = -4.0
    m, z = vxo.row_softmax_stats(row, inv_t)
    assert m == -4.0 and z == 1.0
    # vocabulary one past a chunk boundary: the tail chunk holds one element
    rng = np.random.default_rng(3)
    row = rng.normal(0, 3, size=8193).astype(np.float32)
    row[8192] = 40.0
    m, z = vxo.row_softmax_stats(row, inv_t)
    m64, z64 = lse_f64(row, inv_t)
    assert m == 40.0 and abs(z - z64) <= 2e-5 * z64


def planted_row(vocab: int, rng, spikes, base_sd=3.0, spike=9.0):
    row = rng.normal(0.0, base_sd, size=vocab).astype(np.float32)
    for j in spikes:
        if j < vocab:
            row[j] = np.float32(spike + rng.uniform(-0.5, 0.5))
    return row


def boundary_spikes(vocab: int):
    out = []
    for b in list(range(256, min(vocab, 3 * 8192), 256))[:40] + list(range(8192, vocab, 8192)):
        out += [b - 1, b]
    out.append(vocab - 1)
    return sorted(set(j for j in out if 0 <= j < vocab))


def residual_f64(lt, ld, inv_t):
    mt, zt = lse_f64(lt, inv_t)
    p = np.exp((lt.astype(np.float64) - mt) * inv_t) / zt
    if ld is None:
        return p
    md, zd = lse_f64(ld, inv_t)
    q = np.exp((ld.astype(np.float64) - md) * inv_t) / zd
    return np.maximum(0.0, p - q)


def check_draw(j, r, u, band):
    """j owns the CDF interval of u * total up to `band` of the total mass."""
    cdf = np.cumsum(r)
    total = cdf[-1]
    t = u * total
    lo = cdf[j - 1] if j > 0 else 0.0
    assert r[j] > 0.0, f"drew index {j} of zero residual mass"
    assert lo - band * total <= t <= cdf[j] + band * total, (j, lo / total, u, cdf[j] / total)


@pytest.mark.parametrize("vocab", [8193, 20000, V_LARGE])
@pytest.mark.parametrize("residual", [False, True])
def test_sample_residual_is_float64_inverse_cdf(vocab, residual):
    inv_t = float(np.float32(1) / np.float32(0.8))
    rng = np.random.default_rng(vocab + residual)
    spikes = boundary_spikes(vocab)
    lt = planted_row(vocab, rng, spikes)
    ld = None
    if residual:
        # the draft puts its own mass on every other spike: their residual
        # vanishes, the rest keep most of theirs
        ld = (lt + rng.normal(0, 1, size=vocab)).astype(np.float32)
        for j in spikes[::2]:
            ld[j] = np.float32(lt[j] + 3.0)
    r = residual_f64(lt, ld, inv_t)
    cdf = np.cumsum(r)
    total = cdf[-1]
    mt, zt = vxo.row_softmax_stats(lt, inv_t)
    md, zd = vxo.row_softmax_stats(ld, inv_t) if residual else (0.0, 1.0)
    # u at the centre of each spike's interval, just inside both of its
    # edges, and at random points
    us = []
    for j in spikes:
        if r[j] > 1e-3 * total:
            lo = cdf[j - 1] if j else 0.0
            us += [(lo + 0.5 * r[j]) / total, (lo + 0.02 * r[j]) / total, (cdf[j] - 0.02 * r[j]) / total]
    us += list(rng.random(64))
    us = [float(np.float32(u)) for u in us if 0.0 <= u < 1.0]
    assert len(us) > 40
    for u in us:
        j = vxo.sample_residual(lt, mt, zt, u, inv_t, ld, md, zd)
        check_draw(j, r, np.float64(u), band=2e-5)
        if (np.abs(cdf / total - u) > 1e-4).all():
            # away from every interval edge the draw is exactly the float64 one
            assert j == int(np.searchsorted(cdf, u * total, side="right")), (u, j)


@pytest.mark.parametrize("residual", [False, True])
def test_draws_straddling_boundaries_follow_the_distribution(residual):
    """Chi-square of 6000 draws on a 20000-token row whose mass sits on the
    elements either side of the 256 / 512 / 8192 / 16384 boundaries."""
    vocab, n = 20000, 6000
    inv_t = 1.0
    spikes = [255, 256, 511, 512, 8191, 8192, 16383, 16384]
    lt = np.full(vocab, -30.0, np.float32)
    vals = np.array([2.0, 1.0, 0.5, 1.5, 0.0, 2.2, 1.2, 0.8], np.float32)
    lt[spikes] = vals
    ld = None
    if residual:
        ld = np.full(vocab, -30.0, np.float32)
        ld[spikes] = np.array([0.5, 2.5, 0.5, 0.0, 1.0, 0.7, 2.0, 0.0], np.float32)
    r = residual_f64(lt, ld, inv_t)
    p = r[spikes] / r.sum()
    mt, zt = vxo.row_softmax_stats(lt, inv_t)
    md, zd = vxo.row_softmax_stats(ld, inv_t) if residual else (0.0, 1.0)
    us = np.random.default_rng(11).random(n).astype(np.float32)
    draws = np.array([vxo.sample_residual(lt, mt, zt, float(u), inv_t, ld, md, zd) for u in us])
    assert np.isin(draws, spikes).all()
    counts = np.array([(draws == j).sum() for j in spikes], np.float64)
    keep = p > 0
    assert (counts[~keep] == 0).all(), "drew a token whose residual is zero"
    exp = n * p[keep]
    chi2 = (((counts[keep] - exp) ** 2) / exp).sum()
    assert chi2 < 30.0, (chi2, counts, exp)  # <= 7 dof, p-value < 1e-4
