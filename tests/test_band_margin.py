"""The banded selection's bin margin (mlx-swift-lm_amd/csrc/bsattn_select.hip,
select_banded): survivors binned by fp32 value over [lim, vmax] into 1024
bins, keys at least D = floor(2e * scale * 1.001) + 3 bins above the K-th
key's bin taken, at least D below dropped, the rest rescored exactly.
The bins are computed here with the kernel's fp32 operations (numpy
float32) on rows whose approximate scores lie within e of exact ones, and
the result is compared with the brute-force top K by (exact score desc,
index asc).  Rows the kernel would hand to its general passes (band over
64, bound over 512 bins, degenerate range) are counted, not checked."""
import numpy as np
import pytest

f32 = np.float32
NB, CAP = 1024, 64


def key(s):
    b = s.astype(f32).view(np.uint32).astype(np.uint64)
    s0 = s.astype(f32)
    return np.where(s0 == 0, np.uint64(0x80000000), np.where(b & 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000))


def exact_topk(s, K):
    order = np.lexsort((np.arange(len(s)), -key(s).astype(np.int64)))
    return np.sort(order[:K])


def banded(v, s, e, lim, K):
    """-> the selected indices, or None where the kernel falls back."""
    vmax = v.max()
    if not vmax > lim:
        return None
    scale = f32(NB - 1) / f32(vmax - lim)
    y = f32(f32(f32(f32(2.0) * e) * scale) * f32(1.001))
    if not (np.isfinite(scale) and y < 512):
        return None
    surv = v >= lim
    bn = np.full(len(v), -1, np.int64)
    bn[surv] = np.minimum(NB - 1, ((v[surv] - lim).astype(f32) * scale).astype(f32).astype(np.int32))
    hist = np.bincount(bn[surv], minlength=NB)
    above = np.concatenate([np.cumsum(hist[::-1])[::-1], [0]])  # keys with bin >= b
    bstar = int(np.nonzero(above[:NB] >= K)[0].max())
    D = int(y) + 3
    inm = surv & (bn >= bstar + D)
    band = surv & ~inm & (bn > bstar - D)
    krem = K - int(inm.sum())
    if band.sum() > CAP:
        return None
    assert krem >= 1 and band.sum() >= krem
    take = inm.copy()
    bidx = np.nonzero(band)[0]
    o = np.lexsort((bidx, -key(s[bidx]).astype(np.int64)))
    take[bidx[o[:krem]]] = True
    return np.nonzero(take)[0]


def row(rng, kind, n, K):
    if kind == "iid":
        s = rng.standard_normal(n) * 11
    elif kind == "ties":
        s = np.round(rng.standard_normal(n) * 4)
    elif kind == "cluster":
        s = 5 + rng.standard_normal(n) * 1e-3
    elif kind == "dups":
        s = rng.standard_normal(n) * 11
        for x in rng.choice(np.argsort(-s)[:K + 20], 5):
            s[rng.choice(n, 20)] = s[x]
    else:  # wide
        s = rng.standard_normal(n) * 1e4
    s = s.astype(f32)
    e = f32(10 ** rng.uniform(-4, 0))
    v = (s.astype(np.float64) + rng.uniform(-0.99, 0.99, n) * float(e)).astype(f32)
    bad = np.abs(v.astype(np.float64) - s) > float(e)
    v[bad] = s[bad]
    t1 = np.sort(v)[::-1][K - 1]
    # the floor certificate: lim <= tau - 2e with tau at most the K-th approximate score
    tau = f32(t1 - abs(rng.standard_normal()) * float(e) * rng.choice([0, 1, 10, 100]))
    return v, s, e, f32(tau - f32(2) * e)


@pytest.mark.parametrize("kind", ["iid", "ties", "cluster", "dups", "wide"])
def test_band_margin_gives_exact_top_k(kind):
    rng = np.random.default_rng(len(kind))
    checked = 0
    for _ in range(300):
        n = int(rng.choice([300, 1000, 4000]))
        K = int(rng.choice([1, 5, 40, 128]))
        v, s, e, lim = row(rng, kind, n, K)
        got = banded(v, s, e, lim, K)
        if got is not None:
            assert np.array_equal(got, exact_topk(s, K)), (kind, n, K)
            checked += 1
    assert checked >= 20, checked
