"""The benchmark's input generator (bench.py: counter_normal, round16,
choose_positions, query_inputs, sequence_inputs), run with torch on the CPU,
against the oracle's counter-based generator and the committed input digests
of the decode workloads (tests/golden/input_digests.json)."""
import hashlib
import json
import os
import sys

import numpy as np
import pytest
import torch

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

CPU = torch.device("cpu")


def words(t):
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("seed,stream,start,n", [
    (1002, 1, 0, 4096),
    (1003, 2, 123456 * 128, 8192),
    (7, 0, 1 << 40, 2048),
    (1005, 1, (1 << 63) - 4096, 4096),  # indices near the top of the counter range
])
def test_counter_normal_matches_oracle(dtype, seed, stream, start, n):
    mine = words(bench.round16(bench.counter_normal(seed, stream, start, n, torch, CPU), dtype, torch))
    ref = O.fill_normal(seed, stream, start, (n,), dtype)
    assert np.array_equal(mine, ref)


def test_round16_matches_oracle_at_the_edges():
    ulp_bf = 2.0 ** -7
    xs = [0.0, -0.0, 1.0, -1.0, 3.0,
          1 + ulp_bf / 2, 1 + 3 * ulp_bf / 2, 1 + ulp_bf / 2 + 2.0 ** -40, 1 + ulp_bf / 2 - 2.0 ** -40,
          1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 1 + 2.0 ** -11 + 2.0 ** -45,
          # a double just above a 16-bit midpoint that float32 rounds onto the midpoint
          1 + ulp_bf / 2 + 2.0 ** -30, 1 + 2.0 ** -11 + 2.0 ** -30,
          2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -25, 2.0 ** -25 + 2.0 ** -60, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -26,
          6.1e-5, 1e-7, -3e-6, 2.0 ** -126, 2.0 ** -130, 2.0 ** -133, 2.0 ** -134, 3 * 2.0 ** -134,
          65504.0, 65519.99, 65520.0, 1e6, -1e6, 3.0e38, float.fromhex("0x1.FF8p+127"),
          float.fromhex("0x1.FF7FFFFFp+127"), 1e300]
    x = torch.tensor(xs, dtype=torch.float64)
    got_f16 = words(bench.round16(x, "f16", torch))
    got_bf16 = words(bench.round16(x, "bf16", torch))
    ref_f16 = np.array([O.lib().orc_f64_to_f16(v) for v in xs], np.uint16)
    ref_bf16 = np.array([O.lib().orc_f64_to_bf16(v) for v in xs], np.uint16)
    assert np.array_equal(got_f16, ref_f16), [(v, hex(a), hex(b)) for v, a, b in zip(xs, got_f16, ref_f16) if a != b]
    assert np.array_equal(got_bf16, ref_bf16), [(v, hex(a), hex(b)) for v, a, b in zip(xs, got_bf16, ref_bf16) if a != b]


def test_round16_over_dense_random_doubles():
    # doubles spread over many binades, many of them within a few float32 ulps
    # of a 16-bit midpoint, where a float32 step would round twice
    rng = np.random.default_rng(11)
    e = rng.integers(-30, 20, 20000)
    mant = rng.integers(0, 1 << 16, 20000)
    base = (1.0 + mant / 65536.0 + 2.0 ** -17) * np.exp2(e)
    jitter = rng.integers(-4, 5, 20000) * np.exp2(e - 40.0)
    xs = np.concatenate([base + jitter, -(base + jitter), rng.standard_normal(20000) * 1e-5])
    x = torch.from_numpy(xs)
    for dtype, conv in (("f16", O.lib().orc_f64_to_f16), ("bf16", O.lib().orc_f64_to_bf16)):
        got = words(bench.round16(x, dtype, torch))
        ref = np.array([conv(float(v)) for v in xs], np.uint16)
        assert np.array_equal(got, ref), dtype


def test_choose_positions_matches_oracle():
    keys = list(range(8))
    mine = bench.choose_positions(1002, bench.S_SALIENT, keys, 32768, 328)
    for i, key in enumerate(keys):
        assert np.array_equal(mine[i], O.choose_positions(1002, bench.S_SALIENT, key, 32768, 328))


@pytest.mark.parametrize("key,name", [("c2", "C2"), ("c3", "C3"), ("c5", "C5")])
def test_bench_workload_prefix_matches_committed_digest(key, name):
    """The bench's layer 0 of each workload (its first 256 tokens per
    sequence, q and the lengths) hashes to the committed digest of the
    workload the GPU tests use."""
    cfg = bench.CONFIGS[key]
    with open(os.path.join(ROOT, "tests", "golden", "input_digests.json")) as f:
        ref = json.load(f)[name]
    assert ref["args"]["seed"] == bench.CFG_SEED[key]
    assert (ref["args"]["B"], ref["args"]["Hq"], ref["args"]["Hkv"], ref["args"]["T"]) == (cfg.B, cfg.HQ, cfg.HKV, cfg.T)
    assert ref["args"].get("salient_frac", 0.0) == cfg.salient
    seed = bench.CFG_SEED[key]
    h = hashlib.sha256()
    h.update(np.full(cfg.B, cfg.T, "<i4").tobytes())
    h.update(words(bench.query_inputs(cfg, seed, torch, CPU)).astype("<u2").tobytes())
    for b in range(cfg.B):
        k, v = bench.sequence_inputs(cfg, seed, b, torch, CPU, tokens=ref["prefix_tokens"])
        kw, vw = words(k), words(v)
        for hh in range(cfg.HKV):
            h.update(kw[hh].astype("<u2").tobytes())
            h.update(vw[hh].astype("<u2").tobytes())
    assert h.hexdigest() == ref["prefix_sha256"]
