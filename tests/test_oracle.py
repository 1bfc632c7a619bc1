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

def test_codec_packing_order():
    x = np.arange(16, dtype=np.float32)
    x = np.concatenate([x, x, x, x, x, x, x, x])  # 128 values, groups of 64 hold 0..15 x4
    codes, scales, biases = O.quantize(O.from_f32(x, "f16")[None], 4, 64)
    assert O.to_f32(scales, "f16").tolist() == [[1.0, 1.0]] and O.to_f32(biases, "f16").tolist() == [[0.0, 0.0]]
    assert codes[0, 0] == 0x76543210 and codes[0, 1] == 0xFEDCBA98  # least significant nibble first
    g = np.arange(64, dtype=np.float32)
    g[63] = 255.0  # range 0..255 -> scale 1, bias 0
    c8, s8, b8 = O.quantize(O.from_f32(np.concatenate([g, g + 1]), "f16")[None], 8, 64)
    assert O.to_f32(s8, "f16").tolist() == [[1.0, 1.0]] and O.to_f32(b8, "f16").tolist() == [[0.0, 1.0]]
    assert c8[0, 0] == 0x03020100 and c8[0, 15] == 0xFF3E3D3C and c8[0, 16] == 0x03020100


@pytest.mark.parametrize("bits", [4, 8])
def test_codec_round_trip_bound(bits):
    x = O.fill_normal(71, 1, 0, (300, 128), "f16")
    codes, scales, biases = O.quantize(x, bits, 64)
    deq = O.dequantize(codes, scales, biases, bits, 64)
    xf = O.to_f32(x, "f16")
    sf = np.repeat(O.to_f32(scales, "f16"), 64, axis=1)
    bf = np.repeat(O.to_f32(biases, "f16"), 64, axis=1)
    assert np.all(np.abs(deq - xf) <= 0.5 * sf + np.abs(bf) * 2 ** -10 + 1e-6)
    # constant rows round-trip exactly
    c = np.repeat(x[:1, :1], 128, axis=1)
    cc, cs, cb = O.quantize(np.ascontiguousarray(c), bits, 64)
    assert np.array_equal(O.dequantize(cc, cs, cb, bits, 64), O.to_f32(c, "f16"))


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
    # summaries of dequantized keys: constant-block closed form
    s = O.summaries_q(*kq, Tb, 8, 64)
    assert s.shape == (T // Tb, 128)
