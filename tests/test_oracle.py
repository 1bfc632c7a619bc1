"""Pins the CPU oracle (oracle/bsattn_oracle.c) against what the mathematics
fixes: library conversions, published RNG vectors, closed forms, hand-derived
IEEE results that tell summation orders apart, brute-force selection, and
independent fp64 / torch attention.  CPU only."""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

rng = np.random.default_rng(12345)


# ---------------------------------------------------------------- formats --

def test_f32_to_f16_matches_numpy():
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) *
        np.float32(10.0) ** rng.integers(-9, 6, 200000).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e-8, 5.96e-8, 2.98e-8, 2.9802322e-08,
                  np.inf, -np.inf, 6.1e-5, 6.097e-5, 1 + 2 ** -11, 1 + 3 * 2 ** -11], np.float32)])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.from_f32(x, "f16"), ref)


def test_f16_to_f32_all_patterns():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = O.to_f32(h, "f16")
    ok = (got == ref) | (np.isnan(got) & np.isnan(ref))
    assert ok.all()


def test_bf16_matches_torch():
    import torch
    x = rng.standard_normal(200000).astype(np.float32) * np.float32(3.0) ** rng.integers(-30, 30, 200000).astype(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -np.inf, 1 + 2 ** -8, 1 + 3 * 2 ** -8], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.from_f32(x, "bf16"), ref)
    h = np.arange(65536, dtype=np.uint16)
    back = torch.from_numpy(h.view(np.int16)).view(torch.bfloat16).float().numpy()
    got = O.to_f32(h, "bf16")
    assert ((got == back) | (np.isnan(got) & np.isnan(back))).all()


def _rne_sig(x: float, bits: int) -> float:
    """Nearest value with `bits` significant bits (ties to even), exact."""
    if x == 0:
        return 0.0
    m, e = math.frexp(x)  # x = m * 2**e, 0.5 <= |m| < 1
    q = Fraction(m) * 2 ** bits
    r = round(q)  # Python rounds Fractions half to even
    return float(Fraction(r) * Fraction(2) ** (e - bits))


def test_f64_to_16_single_rounding():
    L = O.lib()
    xs = list(rng.standard_normal(3000) * 5)
    # exact midpoints +- a hair, where double rounding through fp32 would fail
    for k in range(200):
        base = float(rng.standard_normal())
        b16 = _rne_sig(base, 11)
        ulp = math.ldexp(1.0, math.frexp(b16)[1] - 11)
        xs += [b16 + ulp / 2 + ulp * 2 ** -30, b16 + ulp / 2 - ulp * 2 ** -30]
    for x in xs:
        assert np.uint16(L.orc_f64_to_f16(x)).view(np.float16) == np.float16(x)  # numpy: direct RNE
        assert O.to_f32(np.array([L.orc_f64_to_bf16(x)], np.uint16), "bf16")[0] == _rne_sig(x, 8)


def test_f64_to_16_overflow_boundary():
    """Largest finite + half an ulp (65504 + 16 for fp16, 0x1.FEp+127 +
    2^119 for bf16) is a tie whose even neighbour is the next power of two,
    i.e. infinity; anything below rounds to the largest finite."""
    L = O.lib()
    for conv, mx, half, inf in ((L.orc_f64_to_f16, 65504.0, 16.0, 0x7C00),
                                (L.orc_f64_to_bf16, float.fromhex("0x1.FEp+127"), 2.0 ** 119, 0x7F80)):
        big = inf - 1
        for sgn in (1.0, -1.0):
            s = 0x8000 if sgn < 0 else 0
            assert conv(sgn * mx) == s | big
            assert conv(sgn * (mx + half - half * 2 ** -40)) == s | big
            assert conv(sgn * (mx + half)) == s | inf
            assert conv(sgn * (mx + half * 1.5)) == s | inf
            assert conv(sgn * mx * 4) == s | inf


# -------------------------------------------------------------------- rng --

def test_splitmix64_published_vectors():
    """First outputs of splitmix64 seeded with 0 (Vigna's reference
    generator): state advances by the golden gamma, output = mix(state)."""
    L = O.lib()
    gamma = 0x9E3779B97F4A7C15
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    got = [L.orc_splitmix64((k * gamma) % 2 ** 64) for k in range(4)]
    assert got == want


def test_normal_distribution():
    from scipy import stats
    z = np.array([O.lib().orc_normal(7, 1, i) for i in range(200000)])
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert stats.kstest(z, "norm").pvalue > 1e-3
    # pairs (2p, 2p+1) are the cos / sin of one Box-Muller draw: r^2 = -2 ln u1
    r2 = z[0::2] ** 2 + z[1::2] ** 2
    assert stats.kstest(r2, "expon", args=(0, 2)).pvalue > 1e-3


def test_fill_is_thread_count_independent():
    import os
    a = O.fill_normal(3, 1, 100, (64, 128), "bf16")
    b = np.array([O.lib().orc_f64_to_bf16(O.lib().orc_normal(3, 1, 100 + i)) for i in range(64 * 128)],
                 np.uint16).reshape(64, 128)
    assert np.array_equal(a, b)


def test_choose_positions_distinct():
    p = O.choose_positions(5, 3, 9, 1000, 328)
    assert len(set(p.tolist())) == 328 and p.min() >= 0 and p.max() < 1000


# ---------------------------------------------------------------- summary --

def test_summary_closed_forms():
    for dt in ("f16", "bf16"):
        row = O.fill_normal(1, 1, 0, (1, 128), dt)
        blk = np.repeat(row, 64, axis=0)
        assert np.array_equal(O.summaries(blk, 64, dt)[0], row[0])  # constant block -> the key
        # +x / -x pairs cancel exactly
        k = O.fill_normal(2, 1, 0, (32, 128), dt)
        pm = np.concatenate([k, k ^ np.uint16(0x8000)])
        s = O.to_f32(O.summaries(pm, 64, dt)[0], dt)
        assert np.all(s == 0)


def test_summary_within_one_ulp_of_exact_mean():
    for dt, bits in (("f16", 11), ("bf16", 8)):
        k = O.fill_normal(4, 1, 0, (64 * 200, 128), dt)
        s = O.to_f32(O.summaries(k, 64, dt), dt).astype(np.float64)
        exact = O.to_f32(k, dt).astype(np.float64).reshape(200, 64, 128).mean(axis=1)
        rne = np.vectorize(lambda v: _rne_sig(v, bits))(exact)
        same = np.mean(s == rne)
        assert same > 0.999, same
        spacing = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exact), 1e-30))) - (bits - 1))
        assert np.all(np.abs(s - exact) <= spacing)


def test_summary_sequential_fold_order():
    """One dim of a 64-token fp16 block: 32, 32, 2^-5, then 61 x 2^-19.
    Left fold from token 0 in fp32: 64 + 2^-5 is exact, and each 2^-19 is
    below half an ulp of 64 (2^-18) so it is lost: sum = 64 + 2^-5, mean =
    1 + 2^-11, an fp16 tie -> 1.0.  The exact mean (and any order that adds
    the small terms first) lies above the tie and rounds to 1 + 2^-10."""
    k = np.zeros((64, 128), np.float32)
    k[0, 0], k[1, 0], k[2, 0] = 32.0, 32.0, 2.0 ** -5
    k[3:, 0] = 2.0 ** -19  # fp16 subnormal, exact
    keys = O.from_f32(k, "f16")
    assert np.array_equal(O.to_f32(keys, "f16"), k)
    s = O.summaries(keys, 64, "f16")[0, 0]
    assert s == 0x3C00
    exact = (64 + 2.0 ** -5 + 61 * 2.0 ** -19) / 64
    assert np.float16(exact).view(np.uint16) == 0x3C01


# ---------------------------------------------------------------- scoring --

def _bf(vals):
    return O.from_f32(np.array(vals, np.float32), "bf16")


def _chunk_vec(partials):
    """vector whose chunk c (dims 8c..8c+7) dots to partials[c] against e0-per-chunk."""
    a = np.zeros(128, np.float32)
    b = np.zeros(128, np.float32)
    for c, p in enumerate(partials):
        a[8 * c] = p
        b[8 * c] = 1.0
    return _bf(a), _bf(b)


def test_dot_tree_order():
    big = 2.0 ** 24
    # ((p0+p1)+(p2+p3)): 2^24 + 1 ties to 2^24; 1 - 2^24 is exact; sum = 1
    a, b = _chunk_vec([big, 1.0, 1.0, -big])
    assert O.dot_canonical(a, b, "bf16") == 1.0      # sequential fold would give 0, exact is 2
    # pairing by xor 1 first: (p0+p1) = 0, (p8+p9) = 2 -> 2 ; xor 8 first would give 1
    parts = [0.0] * 16
    parts[0], parts[1], parts[8], parts[9] = big, -big, 1.0, 1.0
    a, b = _chunk_vec(parts)
    assert O.dot_canonical(a, b, "bf16") == 2.0


def test_dot_within_chunk_left_fold():
    big = 2.0 ** 24
    a = np.zeros(128, np.float32)
    a[:4] = [big, 1.0, 1.0, -big]
    b = np.zeros(128, np.float32)
    b[:4] = 1.0
    assert O.dot_canonical(_bf(a), _bf(b), "bf16") == 0.0  # ((2^24+1)+1)-2^24, ties to even


def test_dot_within_chunk_steps_are_fused():
    """Each in-chunk step rounds a*b + acc once: 2^64 * 2^64 = 2^128 leaves
    fp32's range, but added to -2^127 it is 2^127 (a separate multiply
    would give +inf)."""
    a = np.zeros(128, np.float32)
    b = np.zeros(128, np.float32)
    a[0], b[0] = -(2.0 ** 127), 1.0
    a[1], b[1] = 2.0 ** 64, 2.0 ** 64
    assert O.dot_canonical(_bf(a), _bf(b), "bf16") == 2.0 ** 127


def test_dot_exact_on_small_integers_and_error_bound():
    for dt in ("f16", "bf16"):
        ia = rng.integers(-8, 9, (50, 128)).astype(np.float32)
        ib = rng.integers(-8, 9, (50, 128)).astype(np.float32)
        for x, y in zip(ia, ib):
            assert O.dot_canonical(O.from_f32(x, dt), O.from_f32(y, dt), dt) == float(np.dot(x, y))
        xa = O.fill_normal(11, 1, 0, (200, 128), dt)
        xb = O.fill_normal(11, 2, 0, (200, 128), dt)
        fa, fb = O.to_f32(xa, dt).astype(np.float64), O.to_f32(xb, dt).astype(np.float64)
        for i in range(200):
            exact = float(np.dot(fa[i], fb[i]))
            bound = 12 * 2.0 ** -24 * float(np.sum(np.abs(fa[i] * fb[i])))
            assert abs(O.dot_canonical(xa[i], xb[i], dt) - exact) <= bound


def test_score_is_max_over_group():
    q = O.fill_normal(21, 0, 0, (4, 128), "f16")
    summ = O.fill_normal(21, 1, 0, (30, 128), "f16")
    s = O.score_blocks(q, summ, "f16")
    per = np.array([[O.dot_canonical(q[g], summ[j], "f16") for g in range(4)] for j in range(30)],
                   np.float32)
    assert np.array_equal(s, per.max(axis=1))


# -------------------------------------------------------------- selection --

def brute_select(scores, length, Tb, ns, nr, K):
    nb = -(-length // Tb)
    if length <= 0:
        return []
    forced = set(range(min(ns, nb))) | set(range(max(0, nb - nr), nb))
    cand = list(range(ns, nb - nr))
    if len(cand) > K:
        def key(j):
            s = float(scores[j])
            if math.isnan(s):
                return (0, j)
            return (1, -s, j)  # NaN lowest; -0 == +0 in float compare
        cand = sorted(cand, key=lambda j: (0 if math.isnan(scores[j]) else 1, -(scores[j] if not math.isnan(scores[j]) else 0), j),)
        good = [j for j in cand if not math.isnan(scores[j])]
        bad = [j for j in cand if math.isnan(scores[j])]
        good.sort(key=lambda j: (-float(scores[j]), j))
        bad.sort()
        cand = (good + bad)[:K]
    return sorted(forced | set(cand))


@pytest.mark.parametrize("trial", range(40))
def test_select_matches_brute_force(trial):
    r = np.random.default_rng(trial)
    Tb = int(r.choice([32, 64]))
    length = int(r.integers(0, 60 * Tb))
    ns, nr, K = int(r.integers(0, 3)), int(r.integers(1, 4)), int(r.integers(0, 12))
    nb = -(-length // Tb)
    s = r.standard_normal(max(nb, 1)).astype(np.float32)
    if trial % 3 == 0:
        s = np.round(s * 2) / 2  # many ties
    if trial % 5 == 0 and nb > 4:
        s[r.integers(0, nb, 3)] = np.nan
        s[r.integers(0, nb, 2)] = -0.0
        s[r.integers(0, nb, 2)] = 0.0
        s[r.integers(0, nb, 2)] = -np.inf
    idx, n = O.select(s, length, Tb, ns, nr, K)
    want = brute_select(s, length, Tb, ns, nr, K)
    assert n == len(want)
    assert idx[:n].tolist() == want
    assert np.all(idx[n:] == -1)


def test_select_special_cases():
    # all equal -> lowest K candidates
    idx, n = O.select(np.zeros(20, np.float32), 20 * 64, 64, 1, 1, 4)
    assert idx[:n].tolist() == [0, 1, 2, 3, 4, 19]
    # K >= candidates -> all blocks
    idx, n = O.select(np.zeros(5, np.float32), 5 * 64 - 3, 64, 1, 1, 10)
    assert idx[:n].tolist() == [0, 1, 2, 3, 4]
    # forced blocks kept even with -inf scores; partial newest block always kept
    s = np.full(10, -np.inf, np.float32)
    s[5] = 1.0
    idx, n = O.select(s, 9 * 64 + 1, 64, 1, 1, 1)
    assert idx[:n].tolist() == [0, 5, 9]
    # -0 and +0 tie -> lower index
    s = np.array([9, -0.0, 0.0, -1, 9], np.float32)
    idx, n = O.select(s, 5 * 64, 64, 0, 1, 1)
    assert idx[:n].tolist() == [0, 4]
    s = np.array([-5, -0.0, 0.0, -1, 9], np.float32)
    idx, n = O.select(s, 5 * 64, 64, 0, 1, 1)
    assert idx[:n].tolist() == [1, 4]
    # empty sequence
    idx, n = O.select(np.zeros(1, np.float32), 0, 64, 1, 1, 4)
    assert n == 0 and np.all(idx == -1)


def test_score_key_order():
    vals = [np.nan, -np.inf, -3.0, -1e-30, -0.0, 0.0, 1e-30, 2.0, np.inf]
    keys = [O.score_key(v) for v in vals]
    assert keys[0] == 0
    assert keys[4] == keys[5]
    assert all(keys[i] < keys[i + 1] for i in range(1, 4)) and all(keys[i] < keys[i + 1] for i in range(5, 8))


# -------------------------------------------------------------- attention --

def numpy_attention(q, k, v, scale):
    s = (q @ k.T) * scale
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return (p @ v) / p.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_attend_vs_numpy_and_torch(dt):
    import torch
    T, Tb = 1000, 64
    q = O.fill_normal(31, 0, 0, (4, 128), dt)
    k = O.fill_normal(31, 1, 0, (T, 128), dt)
    v = O.fill_normal(31, 2, 0, (T, 128), dt)
    idx = np.array([0, 3, 7, 15], np.int32)
    got = O.attend(q, k, v, Tb, idx, 0.125, dt)
    toks = np.concatenate([np.arange(j * Tb, min((j + 1) * Tb, T)) for j in idx])
    qf, kf, vf = (O.to_f32(a, dt).astype(np.float64) for a in (q, k, v))
    ref = numpy_attention(qf, kf[toks], vf[toks], 0.125)
    assert np.max(np.abs(got - ref)) < 1e-12
    tq = torch.from_numpy(qf)[None, :, None, :]
    tk = torch.from_numpy(kf[toks])[None, None].expand(1, 4, -1, -1)
    tv = torch.from_numpy(vf[toks])[None, None].expand(1, 4, -1, -1)
    tref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, scale=0.125)[0, :, 0].numpy()
    assert np.max(np.abs(got - tref)) < 1e-10


def test_attend_invariants():
    T, Tb = 700, 64
    q = O.fill_normal(41, 0, 0, (4, 128), "bf16")
    k = O.fill_normal(41, 1, 0, (T, 128), "bf16")
    v = np.repeat(O.fill_normal(41, 2, 0, (1, 128), "bf16"), T, axis=0)
    out = O.attend(q, k, v, Tb, np.array([1, 2, 10], np.int32), 0.1, "bf16")
    assert np.allclose(out, O.to_f32(v[:1], "bf16").astype(np.float64), atol=1e-12, rtol=0)  # V constant
    v = O.fill_normal(41, 2, 0, (T, 128), "bf16")
    nb = -(-T // Tb)
    all_blocks = O.attend(q, k, v, Tb, np.arange(nb, dtype=np.int32), 0.1, "bf16")
    assert np.max(np.abs(all_blocks - O.dense(q, k, v, 0.1, "bf16"))) < 1e-12
    # -1 entries and blocks past the end are skipped; empty selection -> zeros
    a = O.attend(q, k, v, Tb, np.array([2, -1, 4, 99, 7, -1], np.int32), 0.1, "bf16")
    b = O.attend(q, k, v, Tb, np.array([2, 4, 7], np.int32), 0.1, "bf16")
    assert np.array_equal(a, b)
    assert np.all(O.attend(q, k, v, Tb, np.array([-1], np.int32), 0.1, "bf16") == 0)


def test_decode_head_composes_stages():
    T, Tb = 64 * 30 + 5, 64
    q = O.fill_normal(51, 0, 0, (4, 128), "f16")
    k = O.fill_normal(51, 1, 0, (T, 128), "f16")
    v = O.fill_normal(51, 2, 0, (T, 128), "f16")
    idx, n, out = O.decode_head(q, k, v, Tb, 1, 1, 6, 0.088, "f16")
    summ = O.summaries(k, Tb, "f16")
    sel, n2 = O.select(O.score_blocks(q, summ, "f16"), T, Tb, 1, 1, 6)
    assert n == n2 == 8 and np.array_equal(idx, sel)
    assert np.array_equal(out, O.attend(q, k, v, Tb, sel, 0.088, "f16"))


def test_block_mass_sums_to_one():
    T = 500
    q = O.fill_normal(61, 0, 0, (128,), "f16")
    kf = O.to_f32(O.fill_normal(61, 1, 0, (T, 128), "f16"), "f16")
    m = O.block_mass(q, kf, 32, 0.1)
    assert abs(m.sum() - 1) < 1e-12 and len(m) == 16
    s = (kf.astype(np.float64) @ O.to_f32(q, "f16").astype(np.float64)) * 0.1
    p = np.exp(s - s.max())
    p /= p.sum()
    assert np.allclose(m, np.add.reduceat(p, np.arange(0, T, 32)), atol=1e-14)


# ------------------------------------------------------------ affine codec --
# The reference quantizes with mlx's affine rule (KVCache.swift:416-417,
# 856-857 call quantized(); the rule lives in the un-vendored mlx).  Each case
# below is derived by hand in fp32 from the published rule: signed scale,
# the larger-magnitude extreme as bias, scale = edge / rint(edge / scale),
# codes from the fp32 scale / bias, rint (half to even), fp16 storage.

def _group(vals, n=64):
    g = np.zeros(n, np.float32)
    g[:len(vals)] = vals
    return g


def _q1(vals, bits):
    """quantize one 128-dim row whose two 64-dim groups both hold `vals`."""
    g = _group(vals)
    c, s, b = O.quantize(O.from_f32(np.concatenate([g, g]), "f16")[None], bits, 64)
    return c[0], int(s[0, 0]), int(b[0, 0])


def test_codec_min_side_positive_scale():
    """|min| > |max|: mn -8, mx 4 -> scale 12/15 = 0.8f, edge -8,
    q0 = rint(-8 / 0.8f) = -10, scale = -8 / -10 = 0.8f, bias -8.
    codes: -8 -> 0, 4 -> rint(12 / 0.8f) = 15, 0 -> rint(8 / 0.8f) = 10.
    fp16(0.8) = 0x3A66, fp16(-8) = 0xC800."""
    c, s, b = _q1([-8, 4], 4)
    assert (s, b) == (0x3A66, 0xC800)
    assert c[0] == 0xAAAAAAF0 and all(c[1:8] == 0xAAAAAAAA)


def test_codec_max_side_negative_scale():
    """|max| >= |min|: mn -4, mx 8 -> scale -(12/15), edge 8, q0 = -10,
    scale = 8 / -10 = -0.8f, bias 8.  codes: 8 -> 0, -4 -> rint(-12 / -0.8f)
    = 15, 0 -> 10.  (bias = min would give 8 -> 15, -4 -> 0, 0 -> 5.)"""
    c, s, b = _q1([8, -4], 4)
    assert (s, b) == (0xBA66, 0x4800)
    assert c[0] == 0xAAAAAAF0


def test_codec_equal_magnitudes_take_max_side():
    """|min| == |max| (4, -4): side is |mn| > |mx|, false, so edge = 4 and
    scale = -(8/15) = -0.53333336f; 4 / scale = -7.4999995 -> q0 = -7,
    scale = 4 / -7 = -0.5714286f (fp16 0xB892), bias 4 (0x4400).
    codes: 4 -> 0, -4 -> rint(-8 / scale) = 14, 0 -> 7."""
    c, s, b = _q1([4, -4], 4)
    assert (s, b) == (0xB892, 0x4400)
    assert c[0] == 0x777777E0 and c[1] == 0x77777777


def test_codec_rounded_q0_and_fp32_scale():
    """mn -1, mx 2.5: scale -(3.5/15), edge 2.5, 2.5 / scale = -10.71 ->
    q0 = -11, scale = 2.5 / -11 = -0.22727273f (fp16 0xB346 = -0.2272949),
    bias 2.5 (0x4100).  codes: -1 -> rint(15.4) = 15, 2.5 -> 0,
    1 -> rint(6.6) = 7, 0.5 -> rint(8.8) = 9, 1.25 -> -1.25 / scale = 5.5
    exactly -> 6 (with the fp16 scale it would be 5.4995 -> 5), 0 -> 11
    (0 = 2.5 + 11 * (2.5 / -11) in exact arithmetic)."""
    c, s, b = _q1([-1, 2.5, 1, 0.5, 1.25], 4)
    assert (s, b) == (0xB346, 0x4100)
    assert c[0] == 0xBBB6970F and c[1] == 0xBBBBBBBB


def test_codec_ties_round_half_to_even():
    """mn -2, mx 5.5: scale -(7.5/15) = -0.5, q0 = -11, scale -0.5 (0xB800),
    bias 5.5 (0x4580); code = rint(11 - 2x): 0.25 -> 10.5 -> 10,
    1.25 -> 8.5 -> 8, 0.75 -> 9.5 -> 10 (half away from zero: 11, 9, 10)."""
    c, s, b = _q1([-2, 5.5, 0.25, 1.25, 0.75], 4)
    assert (s, b) == (0xB800, 0x4580)
    assert c[0] == 0xBBBA8A0F


def test_codec_int8_word():
    """int8, mn -1, mx 2.5: scale -(3.5/255), 2.5 / scale = -182.14 -> q0 =
    -182, scale = 2.5 / -182 = -0.013736264f (fp16 0xA308), bias 2.5;
    codes: -1 -> rint(254.8) = 255, 2.5 -> 0, 0 -> 182; bytes LSB first."""
    c, s, b = _q1([-1, 2.5], 8)
    assert (s, b) == (0xA308, 0x4100)
    assert c[0] == 0xB6B600FF and c[1] == 0xB6B6B6B6


def test_codec_zero_and_constant_groups():
    """all zero: scale = max(0, 1e-7) -> -1e-7 (max side), q0 = 0 -> bias 0;
    fp16(-1e-7) = -2 x 2^-24 = 0x8002.  A constant c: q0 = rint(c / -1e-7)
    != 0, scale = c / q0 ~ -1e-7, bias = c, every code 0, so the group
    dequantizes to c exactly."""
    for bits in (4, 8):
        c, s, b = _q1([], bits)
        assert (s, b) == (0x8002, 0x0000) and not c.any()
        for val, bias in ((0.5, 0x3800), (-3.0, 0xC200), (1000.0, 0x63D0)):
            c, s, b = _q1([val] * 64, bits)
            assert (s, b) == (0x8002, bias) and not c.any()
            deq = O.dequantize(c[None], np.array([[s, s]], np.uint16), np.array([[b, b]], np.uint16), bits, 64)
            assert np.all(deq == np.float32(val))


def test_affine_params_fp32():
    s, b = O.affine_params(_group([-1, 2.5]), 4)
    assert s == float(np.float32(2.5) / np.float32(-11)) and b == 2.5
    s, b = O.affine_params(_group([-8, 4]), 4)
    assert s == float(np.float32(0.8)) and b == -8.0


def test_codec_packing_order():
    """Values 0..15: mx side, scale -1, bias 15, code = 15 - x; element i of
    a row in word i / 8, nibble i % 8 from the least significant end."""
    x = np.tile(np.arange(16, dtype=np.float32), 8)
    codes, scales, biases = O.quantize(O.from_f32(x, "f16")[None], 4, 64)
    assert scales.tolist() == [[0xBC00, 0xBC00]] and biases.tolist() == [[0x4B80, 0x4B80]]
    assert codes[0, 0] == 0x89ABCDEF and codes[0, 1] == 0x01234567
    g = np.arange(64, dtype=np.float32)
    g[63] = 255.0  # range 0..255 -> scale -1, bias 255, code 255 - x
    c8, s8, b8 = O.quantize(O.from_f32(np.concatenate([g, g + 1]), "f16")[None], 8, 64)
    assert O.to_f32(s8, "f16").tolist() == [[-1.0, -1.0]] and O.to_f32(b8, "f16").tolist() == [[255.0, 256.0]]
    assert c8[0, 0] == 0xFCFDFEFF and c8[0, 15] == 0x00C1C2C3 and c8[0, 16] == 0xFCFDFEFF
    assert c8[0, 31] == 0x00C1C2C3


@pytest.mark.parametrize("bits", [4, 8])
def test_codec_round_trip_bound(bits):
    """codes come from the fp32 scale / bias, dequantization uses their fp16
    roundings (within 2^-11 relative, 2^-24 absolute below 2^-14):
    |w - x| <= |s| / 2 + code |s16 - s| + |b16 - b| for values inside the
    code range.  scale = edge / rint(edge / scale0) can be up to half a code
    smaller than scale0, so the far end of a group may fall past the last
    code (by less than one) and is clipped there: error < 1.5 |s|."""
    x = O.fill_normal(71, 1, 0, (300, 128), "f16")
    codes, scales, biases = O.quantize(x, bits, 64)
    deq = O.dequantize(codes, scales, biases, bits, 64).astype(np.float64)
    xf = O.to_f32(x, "f16").astype(np.float64)
    sf = np.abs(np.repeat(O.to_f32(scales, "f16"), 64, axis=1)).astype(np.float64)
    bf = np.abs(np.repeat(O.to_f32(biases, "f16"), 64, axis=1)).astype(np.float64)
    nbins = 2 ** bits - 1
    per = 32 // bits
    code = (codes[:, np.arange(128) // per] >> (bits * (np.arange(128) % per))) & nbins
    rounding = sf * nbins * 2.0 ** -10 + bf * 2.0 ** -10 + 2.0 ** -20
    err = np.abs(deq - xf)
    inside = code < nbins
    assert np.all(err[inside] <= 0.5 * sf[inside] + rounding[inside])
    assert np.all(err <= 1.5 * sf + rounding)
    # clipping happens at the far end only, and not for most groups
    assert np.mean(err > 0.5 * sf + rounding) < 0.01
    # the larger-magnitude end of every group round-trips to within its fp16 bias rounding
    g = xf.reshape(300, 2, 64)
    edge = np.where(np.abs(g.min(-1)) > np.abs(g.max(-1)), g.min(-1), g.max(-1))
    assert np.array_equal(O.to_f32(biases, "f16"), edge.astype(np.float32))
    # constant rows round-trip exactly
    c = np.repeat(x[:1, :1], 128, axis=1)
    cc, cs, cb = O.quantize(np.ascontiguousarray(c), bits, 64)
    assert np.array_equal(O.dequantize(cc, cs, cb, bits, 64), O.to_f32(c, "f16"))


# ------------------------------------------------------- quantized summary --

def _qrow(codes_per_dim, bits):
    """pack one 128-dim row of codes LSB first"""
    per = 32 // bits
    w = np.zeros(128 // per, np.uint32)
    for i, cv in enumerate(codes_per_dim):
        w[i // per] |= np.uint32(int(cv) << (bits * (i % per)))
    return w


@pytest.mark.parametrize("bits", [4, 8])
def test_summary_q_constant_block(bits):
    """Every token dequantizes to w = fmaf(s, c, b) = -0.5 * 3 + 2.25 = 0.75
    (group 0) and fmaf(0.125, 1, -1) = -0.875 (group 1): short fp16 values,
    so the fold of 64 (or 32) equal terms and the 1/Tb scaling are exact and
    the summary is that value."""
    for Tb in (32, 64):
        codes = np.tile(_qrow([3] * 64 + [1] * 64, bits), (Tb, 1))
        sc = np.tile(O.from_f32(np.array([-0.5, 0.125], np.float32), "f16"), (Tb, 1))
        bi = np.tile(O.from_f32(np.array([2.25, -1.0], np.float32), "f16"), (Tb, 1))
        s = O.to_f32(O.summaries_q(codes, sc, bi, Tb, bits, 64)[0], "f16")
        assert np.all(s[:64] == 0.75) and np.all(s[64:] == -0.875)


def test_summary_q_sequential_fold_order():
    """dim 0 of a 64-token int4 block, from codes and per-token scales /
    biases: token 0 16 * 2 + 0 = 32, token 1 -16 * 1 + 48 = 32 (negative
    scale), token 2 2^-6 * 2 + 0 = 2^-5, tokens 3..63 2^-20 * 2 + 0 = 2^-19
    (fp16 subnormals, exact).  The left fold from token 0 is 64 + 2^-5 (each
    2^-19 is below half an ulp of 64 and lost), mean 1 + 2^-11, an fp16 tie
    -> 0x3C00; the exact mean (or any order that adds the small terms first)
    rounds to 0x3C01."""
    Tb, bits = 64, 4
    cd = np.zeros((Tb, 128), np.int64)
    sc = np.zeros((Tb, 2), np.float32)
    bi = np.zeros((Tb, 2), np.float32)
    cd[0, 0], sc[0, 0] = 2, 16.0
    cd[1, 0], sc[1, 0], bi[1, 0] = 1, -16.0, 48.0
    cd[2, 0], sc[2, 0] = 2, 2.0 ** -6
    cd[3:, 0], sc[3:, 0] = 2, 2.0 ** -20
    codes = np.stack([_qrow(r, bits) for r in cd])
    s16, b16 = O.from_f32(sc, "f16"), O.from_f32(bi, "f16")
    assert np.array_equal(O.to_f32(s16, "f16"), sc)
    s = O.summaries_q(codes, s16, b16, Tb, bits, 64)[0]
    assert s[0] == 0x3C00
    exact = (64 + 2.0 ** -5 + 61 * 2.0 ** -19) / 64
    assert np.float16(exact).view(np.uint16) == 0x3C01


@pytest.mark.parametrize("bits", [4, 8])
def test_summary_q_within_one_ulp_of_exact_mean(bits):
    Tb = 32
    k = O.fill_normal(91, 1, 0, (Tb * 100, 128), "f16")
    kq = O.quantize(k, bits, 64)
    s = O.to_f32(O.summaries_q(*kq, Tb, bits, 64), "f16").astype(np.float64)
    deq = O.dequantize(*kq, bits, 64).astype(np.float64)
    exact = deq.reshape(100, Tb, 128).mean(axis=1)
    rne = np.vectorize(lambda v: _rne_sig(v, 11))(exact)
    assert np.mean(s == rne) > 0.999
    ax = np.maximum(np.abs(exact), 2.0 ** -14)
    assert np.all(np.abs(s - exact) <= 2.0 ** (np.floor(np.log2(ax)) - 10))


def test_quantized_attention_matches_dequantized():
    T, Tb = 300, 32
    q = O.fill_normal(81, 0, 0, (16, 128), "f16")
    kq = O.quantize(O.fill_normal(81, 1, 0, (T, 128), "f16"), 8, 64)
    vq = O.quantize(O.fill_normal(81, 2, 0, (T, 128), "f16"), 8, 64)
    idx = np.array([0, 4, 9], np.int32)
    out = O.attend_q(q, kq, vq, Tb, 8, 64, idx, 0.088)
    kd = O.dequantize(*kq, 8, 64).astype(np.float64)
    vd = O.dequantize(*vq, 8, 64).astype(np.float64)
    toks = np.concatenate([np.arange(j * Tb, min((j + 1) * Tb, T)) for j in idx])
    ref = numpy_attention(O.to_f32(q, "f16").astype(np.float64), kd[toks], vd[toks], 0.088)
    assert np.max(np.abs(out - ref)) < 1e-12


# ---------------------------------------------------- parallel layer-step --

@pytest.mark.parametrize("bits", [0, 4, 8])
def test_layer_step_equals_per_head_composition(bits):
    """The OpenMP layer-step (the CPU baseline) is score -> select -> attend
    of every (sequence, kv head), bit for bit what the per-head functions
    give, whatever thread runs a pair."""
    from common import make_workload
    dt = "bf16" if bits == 0 else "f16"
    Tb, T, K = 32, 32 * 24 + 7, 6
    w = make_workload(95 + bits, B=3, Hq=16, Hkv=4, T=T, Tb=Tb, dtype=dt, top_k=K)
    keys, values = np.stack(w.keys), np.stack(w.values)
    if bits:
        kq = [O.quantize(keys[b], bits, 64) for b in range(w.B)]
        vq = [O.quantize(values[b], bits, 64) for b in range(w.B)]
        kqs = tuple(np.stack([k[i] for k in kq]) for i in range(3))
        vqs = tuple(np.stack([v[i] for v in vq]) for i in range(3))
        summ = np.stack([[O.summaries_q(*(a[h] for a in kq[b]), Tb, bits, 64) for h in range(w.Hkv)]
                         for b in range(w.B)])
        idx, out = O.layer_step(w.q, summ, Tb, 1, 1, K, w.scale, dt, kq=kqs, vq=vqs, bits=bits)
    else:
        summ = np.stack([[O.summaries(keys[b, h], Tb, dt) for h in range(w.Hkv)] for b in range(w.B)])
        idx, out = O.layer_step(w.q, summ, Tb, 1, 1, K, w.scale, dt, keys=keys, values=values)
    for b in range(w.B):
        for h in range(w.Hkv):
            q = w.q[b, h * 4:(h + 1) * 4]
            sel, n = O.select(O.score_blocks(q, summ[b, h], dt), T, Tb, 1, 1, K)
            assert np.array_equal(idx[b, h], sel)
            ref = (O.attend_q(q, tuple(a[h] for a in kq[b]), tuple(a[h] for a in vq[b]), Tb, bits, 64,
                              sel[:n], w.scale) if bits else
                   O.attend(q, keys[b, h], values[b, h], Tb, sel[:n], w.scale, dt))
            assert np.array_equal(out[b, h * 4:(h + 1) * 4], ref)
