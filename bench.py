"""Block-sparse decode attention benchmark on one MI355X.

Default workload (the headline configuration, --config c2): B=8 sequences,
Hq=32, Hkv=8, D=128, 32768 tokens each in 64-token blocks (512 blocks), bf16
K/V ~ N(0,1) with 1% of key positions per (sequence, kv head) scaled x8,
top-32 + sink + recent (34 blocks selected), softmax scale 1/sqrt(128).  36
distinct layer caches (one per layer, ~1.1 GB each) so the working set is far
above the 256 MB Infinity Cache.

A step = one decode step through all layers: per layer, block scoring +
top-K select + gathered attention (bsattn_decode).  `value` = microseconds
per layer-step.  Steps are replayed from a HIP graph (captured once) so the
timing is the GPU's, not the Python launcher's; the eager (ctypes per call)
figure is reported alongside.

The default run (no --config) also measures configs c3, c5 and c4 below,
without their CPU legs, and reports them under "other_configs" in the same
JSON line (µs per layer-step, or per step for c4, the attention kernel's µs,
achieved GB/s, fraction of peak and traffic source); --no-others skips them.
The headline's cpu_baseline leg also checks layer 0's GPU output against the
oracle's (output_vs_gpu: raw and net-of-rounding max-abs error).

Other workloads (one JSON line each with --config, not the headline):
  --config c3  int4 affine KV (group 64, fp16 scale / bias): B=4, Hq=32,
               Hkv=8, 131072 tokens, 64-token blocks, top-64 + sink + recent;
  --config c5  int8 affine KV, wide GQA: B=8, Hq=64, Hkv=4 (G=16), 262144
               tokens, 32-token blocks, top-128 + sink + 4 recent; adds the
               per-head recall of the selection against exact dense
               attention mass on two sequences of layer 0;
  --config c4  decode loop with appends: B=32, fp16, lengths U[8192, 65536]
               (seeded counter stream), pages taken from a seeded
               permutation of the free list (shuffled physical order), 256 steps of
               (append one token per sequence, score + top-32 + attend) as
               one appendDecode call each (one launch: the append inside the
               fused decode; the two-call figure is reported beside it); eager, since
               every append changes host-side page tables;
  --config pf  dense causal prefill attention of a 512-token chunk at the end
               of 32768 tokens (B=8, Hq=32, Hkv=8, bf16), MFMA-bound;
  --config pfq the same over int4 affine caches (fp16);
  --config mq  speculative verify at the default geometry: decodeMulti of 4
               query tokens per sequence, against 4 single-token decodes.

roofline: the gather + attention kernel the decode step runs (k_attend /
k_attend_q, with the top-K selection fused into it where the candidates
allow), timed with HIP start/stop events attached to each of its dispatches
on the launch stream (the library's profiling hook) during eager decode
steps; algorithmic bytes per launch = selected K+V bytes (codes and scales /
biases for quantized caches) + q + out + indices.  The same kernel on
precomputed indices (bsattn_attend) is reported as roofline.given_index.
cpu_baseline: the C oracle doing the same layer-step (score given
summaries, select, attend) on layer 0's data, its (sequence, kv head) pairs
over OMP_NUM_THREADS OpenMP threads; the CPU model is reported.
cpu_dense_reference_path: what the reference's own decode path computes on
the CPU for that layer (dense attention over every cached token, float32
numpy with multi-threaded BLAS; the thread count is reported).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from dataclasses import dataclass

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-swift-lm_amd"))

HBM_PEAK_GBPS = 8000.0
D = 128


@dataclass
class Config:
    key: str
    metric: str
    B: int
    HQ: int
    HKV: int
    T: int
    TB: int
    dtype: str      # "bf16" / "f16"
    bits: int       # 0: 16-bit K/V; 4 / 8: affine codes
    top_k: int
    ns: int
    nr: int
    salient: float
    layers: int
    traffic_file: str

    @property
    def G(self):
        return self.HQ // self.HKV

    @property
    def bytes_tok(self):
        """HBM bytes of one token's K + V in one kv head."""
        if self.bits == 0:
            return 2 * D * 2
        return 2 * D * self.bits // 8 + 16   # codes + (k, v) x (scale, bias) x 2 groups fp16


CONFIGS = {
    "c2": Config("c2", "block-sparse decode attn µs/layer-step + achieved HBM GB/s (% of peak), 32k ctx",
                 8, 32, 8, 32768, 64, "bf16", 0, 32, 1, 1, 0.01, 36,
                 "k_attend_b8_ctx32k_bf16_traffic.md"),
    "c3": Config("c3", "block-sparse decode attn µs/layer-step, int4 affine KV, 131k ctx",
                 4, 32, 8, 131072, 64, "f16", 4, 64, 1, 1, 0.0, 36,
                 "k_attend_q_b4_ctx128k_int4_traffic.md"),
    "c5": Config("c5", "block-sparse decode attn µs/layer-step, int8 affine KV, GQA 16, 262k ctx",
                 8, 64, 4, 262144, 32, "f16", 8, 128, 1, 4, 0.0, 12,
                 "k_attend_q_b8_ctx256k_int8_traffic.md"),
}


def profiled_means(layers, kinds, step, reps, torch):
    """Per repetition of step(), each kernel kind's mean dispatch time (us)
    from the library's event timing; lists in repetition order."""
    for cache, _ in layers:
        cache.profile(True)
    last = {name: (0.0, 0) for name in kinds}
    out = {name: [] for name in kinds}
    for _ in range(reps):
        step()
        torch.cuda.synchronize()
        for name, kind in kinds.items():
            tot, n = 0.0, 0
            for cache, _ in layers:
                ms, c = cache.profileRead(kind)
                tot, n = tot + ms, n + c
            dt, dn = tot - last[name][0], n - last[name][1]
            last[name] = (tot, n)
            if dn:
                out[name].append(dt * 1e3 / dn)
    for cache, _ in layers:
        cache.profile(False)
    return out


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", default="c2", choices=["c2", "c3", "c4", "c5", "pf", "pfq", "mq"])
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=0, help="layer caches (0: the config's)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-recall", action="store_true")
    ap.add_argument("--no-others", action="store_true",
                    help="default run: skip the other decode workloads (c3, c5, c4) after the headline")
    ap.add_argument("--counters", action="store_true",
                    help="short run for hardware-counter profiling (rocprofv3 --pmc): build the "
                         "layer caches, run --steps eager decode steps and --steps given-index "
                         "attention passes over every layer, no graph, timing or CPU legs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one plain 256 MiB device copy (a known-traffic dispatch "
                         "for scaling hardware byte counters)")
    return ap.parse_args()


def torch_dtype(torch, cfg):
    return torch.bfloat16 if cfg.dtype == "bf16" else torch.float16


def calibration_copy(torch, dev):
    """One plain 256 MiB device copy, for scaling the hardware byte counters."""
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log("[bench] calibration copy: 256 MiB read + 256 MiB written")
    del src, dst


CFG_SEED = {"c2": 1002, "c3": 1003, "c5": 1005}  # 1000 + the configuration's number


def query_inputs(cfg: Config, seed: int, torch, dev):
    """q [B, Hq, 1, D] of the workload with this seed."""
    q = round16(counter_normal(seed, S_Q, 0, cfg.B * cfg.HQ * D, torch, dev), cfg.dtype, torch)
    return q.view(torch_dtype(torch, cfg)).reshape(cfg.B, cfg.HQ, 1, D)


def sequence_inputs(cfg: Config, seed: int, b: int, torch, dev, tokens=None):
    """Keys and values [Hkv, tokens, D] of sequence b (its first `tokens`
    tokens; all of them by default) of the workload with this seed."""
    import numpy as np
    T, n = cfg.T, cfg.T if tokens is None else tokens
    dt = torch_dtype(torch, cfg)
    if n == T:  # the heads' streams are consecutive
        kx = counter_normal(seed, S_K, b * cfg.HKV * T * D, cfg.HKV * T * D, torch, dev)
        vx = counter_normal(seed, S_V, b * cfg.HKV * T * D, cfg.HKV * T * D, torch, dev)
    else:
        kx = torch.cat([counter_normal(seed, S_K, (b * cfg.HKV + h) * T * D, n * D, torch, dev)
                        for h in range(cfg.HKV)])
        vx = torch.cat([counter_normal(seed, S_V, (b * cfg.HKV + h) * T * D, n * D, torch, dev)
                        for h in range(cfg.HKV)])
    kx = kx.view(cfg.HKV, n, D)
    n_sal = int(round(cfg.salient * T))
    if n_sal:
        pos = choose_positions(seed, S_SALIENT, [b * cfg.HKV + h for h in range(cfg.HKV)], T, n_sal)
        mult = torch.ones(cfg.HKV, T, dtype=torch.float64, device=dev)
        mult.scatter_(1, torch.from_numpy(pos).to(dev), 8.0)
        kx = kx * mult[:, :n, None]
        del mult
    k = round16(kx, cfg.dtype, torch).view(dt)
    del kx
    v = round16(vx, cfg.dtype, torch).view(dt).view(cfg.HKV, n, D)
    return k, v


def make_layer(cfg: Config, layer, dev, torch, bsattn, digest=None):
    """Layer `layer`'s cache and q from the counter-based generator with seed
    CFG_SEED + 1000 * layer (layer 0 is the configuration's committed
    workload).  digest: a dict that receives the SHA-256 of the inputs over
    the lengths (int32), q, then each (sequence, kv head)'s keys and values
    as 16-bit words ("prefix": their first 256 tokens; "full": all of them
    when digest["full"] is set), the order of tests/golden/input_digests.json."""
    import numpy as np
    seed = CFG_SEED[cfg.key] + 1000 * layer
    dt = torch_dtype(torch, cfg)
    cache = bsattn.BlockSparseKVCache(max_seqs=cfg.B, num_q_heads=cfg.HQ, num_kv_heads=cfg.HKV,
                                      head_dim=D, block_size=cfg.TB, dtype=dt, kv_bits=cfg.bits,
                                      top_k=cfg.top_k, sink_blocks=cfg.ns, recent_blocks=cfg.nr,
                                      max_blocks_per_seq=cfg.T // cfg.TB + 2, device=dev.index)
    q = query_inputs(cfg, seed, torch, dev)
    hashes = None
    if digest is not None:
        import hashlib
        hashes = {"prefix": hashlib.sha256()}
        if digest.get("full"):
            hashes["full"] = hashlib.sha256()
        head = np.full(cfg.B, cfg.T, "<i4").tobytes() + host16(q, torch, np).astype("<u2").tobytes()
        for hh in hashes.values():
            hh.update(head)
    for b in range(cfg.B):  # one sequence at a time keeps the temporaries small
        k, v = sequence_inputs(cfg, seed, b, torch, dev)
        if hashes is not None:
            kh, vh = host16(k, torch, np), host16(v, torch, np)
            for h in range(cfg.HKV):
                hashes["prefix"].update(kh[h, :256].astype("<u2").tobytes())
                hashes["prefix"].update(vh[h, :256].astype("<u2").tobytes())
                if "full" in hashes:
                    hashes["full"].update(kh[h].astype("<u2").tobytes())
                    hashes["full"].update(vh[h].astype("<u2").tobytes())
            del kh, vh
        cache.append(k[None].contiguous(), v[None].contiguous(), seq_ids=[b])
        del k, v
    if hashes is not None:
        for name, hh in hashes.items():
            digest[name] = hh.hexdigest()
    return cache, q


def input_check(cfg: Config, digest):
    """Layer 0's input digests against the committed ones of the same
    workload -> {"layer0_sha256": ..., "matches_committed": bool, ...}."""
    name = {"c2": "C2", "c3": "C3", "c5": "C5"}[cfg.key]
    with open(os.path.join(ROOT, "tests", "golden", "input_digests.json")) as f:
        ref = json.load(f)[name]
    out = {"workload": name, "prefix_tokens": 256, "prefix_sha256": digest["prefix"],
           "prefix_matches_committed": digest["prefix"] == ref["prefix_sha256"]}
    if isinstance(digest.get("full"), str):
        out["layer0_sha256"] = digest["full"]
        out["full_matches_committed"] = digest["full"] == ref["sha256"]
    return out


def algorithmic_bytes(cfg: Config, nsel):
    gather = cfg.B * cfg.HKV * nsel * cfg.TB * cfg.bytes_tok
    qo = cfg.B * cfg.HQ * D * 2 * 2
    idx = cfg.B * cfg.HKV * nsel * 4
    summ = cfg.B * cfg.HKV * (cfg.T // cfg.TB) * D * 2
    return gather + qo + idx, summ


def recorded_traffic(cfg: Config):
    """HBM bytes per attention launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (copy-calibrated); None when it is absent."""
    path = os.path.join(ROOT, "profiles", cfg.traffic_file)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1]), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def host16(t, torch, np):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg: Config, cache, q, seconds):
    """Oracle layer-step on layer 0's data: every (sequence, kv head) scores
    its candidate summaries, selects, and attends (over dequantized blocks
    for a quantized cache), the pairs spread over OMP_NUM_THREADS OpenMP
    threads (the C oracle's orc_layer_step).  Repeated for about `seconds`;
    returns (median us per layer-step, repetitions, threads, idx, out) with
    the last repetition's results for the consistency check against the GPU."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    ids = list(range(cfg.B))
    kw = dict(keys=None, values=None, kq=None, vq=None)
    if cfg.bits:
        (k_w, k_s, k_b), (v_w, v_s, v_b) = cache.exportQuantized(ids)
        u32 = lambda t: t.cpu().numpy().view(np.uint32)
        kw["kq"] = (u32(k_w), host16(k_s, torch, np), host16(k_b, torch, np))
        kw["vq"] = (u32(v_w), host16(v_s, torch, np), host16(v_b, torch, np))
    else:
        k, v = cache.export(ids)
        kw["keys"], kw["values"] = host16(k, torch, np), host16(v, torch, np)
    qh = host16(q, torch, np).reshape(cfg.B, cfg.HQ, D)
    summ = np.stack([host16(cache.exportSummaries(b), torch, np) for b in ids])
    scale = 1.0 / math.sqrt(D)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        idx, out = O.layer_step(qh, summ, cfg.TB, cfg.ns, cfg.nr, cfg.top_k, scale, cfg.dtype,
                                bits=cfg.bits, **kw)
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2] * 1e6, len(times), O.omp_threads(), idx, out


def cpu_dense(cfg: Config, cache, q, seconds):
    """What the reference's decode path computes on the CPU for the same
    layer: dense attention of each query over every cached token
    (attentionWithCacheUpdate's SDPA, or quantizedScaledDotProductAttention
    over the dequantized cache), float32 numpy with its multi-threaded BLAS.
    Sample: sequence 0 of layer 0 (all kv heads), scaled by the batch;
    returns (us per layer-step, repetitions, BLAS threads)."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_info
    G, scale = cfg.G, 1.0 / math.sqrt(D)
    if cfg.bits:
        (kw, ks, kb), (vw, vs, vb) = cache.exportQuantized([0])

        def deq(w, sc, bi):
            words = w[0].cpu().numpy().view(np.uint32)          # [Hkv, T, D*bits/32]
            per = 32 // cfg.bits
            sh = (np.arange(per, dtype=np.uint32) * cfg.bits)[None, None, None, :]
            codes = ((words[..., None] >> sh) & ((1 << cfg.bits) - 1)).astype(np.float32) \
                .reshape(words.shape[0], words.shape[1], D)
            sc = sc[0].float().cpu().numpy()                    # [Hkv, T, D/64]
            bi = bi[0].float().cpu().numpy()
            return (codes.reshape(*codes.shape[:2], D // 64, 64) * sc[..., None] + bi[..., None]) \
                .reshape(codes.shape).astype(np.float32)
        K, V = deq(kw, ks, kb), deq(vw, vs, vb)
    else:
        k, v = cache.export([0])
        K, V = k[0].float().cpu().numpy(), v[0].float().cpu().numpy()   # [Hkv, T, D]
    qq = q[0, :, 0, :].float().cpu().numpy()                             # [Hq, D]
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        for h in range(cfg.HKV):
            s_ = (qq[h * G:(h + 1) * G] @ K[h].T) * scale
            s_ -= s_.max(axis=1, keepdims=True)
            p_ = np.exp(s_)
            p_ /= p_.sum(axis=1, keepdims=True)
            _ = p_ @ V[h]
        times.append(time.perf_counter() - t0)
    times.sort()
    threads = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    return times[len(times) // 2] * 1e6 * cfg.B, len(times), threads


def recall_report(cfg: Config, cache, q, idx, seqs):
    """Per-head recall of the selected blocks against exact dense attention
    mass (fp64, over the dequantized keys): for each (sequence, kv head) the
    true top-K candidate blocks by mass summed over the GQA group, recall =
    |selected ∩ true top-K| / K, captured = selected blocks' share of the
    mass; per q head, the captured share of its own mass."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    scale = 1.0 / math.sqrt(D)
    qh = host16(q, torch, np).reshape(cfg.B, cfg.HQ, D)
    idx = idx.cpu().numpy()
    nb = -(-cfg.T // cfg.TB)
    cand = np.arange(cfg.ns, nb - cfg.nr)
    rec, cap_kv, cap_q = [], [], []
    for b in seqs:
        (kw, ks, kb), _ = cache.exportQuantized([b])
        for h in range(cfg.HKV):
            keys = O.dequantize(kw[0, h].cpu().numpy().view(np.uint32), host16(ks[0, h], torch, np),
                                host16(kb[0, h], torch, np), cfg.bits, 64)
            mass = np.stack([O.block_mass(qh[b, h * cfg.G + g], keys, cfg.TB, scale)
                             for g in range(cfg.G)])          # [G, nb]
            sel = idx[b, h][idx[b, h] >= 0]
            tot = mass.sum(axis=0)
            true_top = cand[np.argsort(-tot[cand], kind="stable")[:cfg.top_k]]
            chosen = np.intersect1d(sel, cand)
            rec.append(len(np.intersect1d(chosen, true_top)) / cfg.top_k)
            cap_kv.append(tot[sel].sum() / cfg.G)
            cap_q.extend(mass[:, sel].sum(axis=1).tolist())
    r = lambda a: round(float(a), 4)
    return {"sequences": list(seqs), "kv_heads": cfg.HKV, "q_heads_per_kv": cfg.G,
            "recall_mean": r(np.mean(rec)), "recall_min": r(np.min(rec)),
            "captured_mass_kv_mean": r(np.mean(cap_kv)), "captured_mass_kv_min": r(np.min(cap_kv)),
            "captured_mass_q_mean": r(np.mean(cap_q)), "captured_mass_q_min": r(np.min(cap_q)),
            "note": "mass = exact softmax(q.k * scale) over all tokens of the dequantized keys; "
                    "true top-K ranks candidate blocks (not sink / recent) by mass summed over "
                    "the group's q heads"}


def replay_distribution(run, reps: int, per: int):
    """p10 / p50 / p90 of `reps` individually event-timed calls of `run`
    (one step each), in µs per unit of `per` units per step."""
    import numpy as np
    import torch
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    for a, b in ev:
        a.record()
        run()
        b.record()
    torch.cuda.synchronize()
    us = np.array([a.elapsed_time(b) * 1e3 / per for a, b in ev])
    p10, p50, p90 = np.percentile(us, [10, 50, 90])
    return {"p10": round(float(p10), 3), "p50": round(float(p50), 3), "p90": round(float(p90), 3),
            "reps": reps}


def copy_bandwidth(torch, dev, mib: int = 1024, reps: int = 10) -> dict:
    """Same-run HBM reference point: torch's device copy of `mib` MiB (read +
    written), median of `reps` event-timed copies."""
    src = torch.ones(mib << 18, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        dst.copy_(src)
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b))
    del src, dst
    ms = sorted(ts)[len(ts) // 2]
    gbps = 2 * (mib << 20) / (ms * 1e-3) / 1e9
    return {"value": round(gbps, 1), "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "what": f"torch copy_ of {mib} MiB fp32 on the bench's GPU (read + written bytes / "
                    f"event time), median of {reps}"}


def bench_layers(args, cfg: Config, light: bool = False):
    """One workload's layer-step benchmark -> the result dict.  light: no
    CPU legs, recall or copy reference (the other configurations of the
    default run)."""
    import torch
    import bsattn
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = args.layers or cfg.layers
    t0 = time.time()
    # layer 0's inputs are checked against the committed digests (in full for
    # the headline workload, the 256-token prefixes for the others)
    digest = {"full": cfg.key == "c2" and not light}
    layers = [make_layer(cfg, i, dev, torch, bsattn, digest if i == 0 else None) for i in range(L)]
    torch.cuda.synchronize()
    inputs = input_check(cfg, digest)
    log(f"[bench] {cfg.key}: built {L} layer caches in {time.time() - t0:.1f}s "
        f"({layers[0][0].poolBytes / 2**30:.2f} GiB each); layer 0 inputs: {inputs}")
    scale = 1.0 / math.sqrt(D)

    def step():
        for (cache, q) in layers:
            cache.decode(q, scale)

    # eager warmup + eager timing
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    te = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - te) * 1e3 / args.steps
    log(f"[bench] eager: {eager_ms * 1e3 / L:.2f} us/layer-step")
    if args.counters:
        idx = [cache.selectBlocks(q) for cache, q in layers]
        for _ in range(args.steps):
            for (cache, q), ii in zip(layers, idx):
                cache.attend(q, ii, scale)
        torch.cuda.synchronize()
        log(f"[bench] counters run done: {args.steps} decode steps and {args.steps} given-index "
            f"attention passes over {L} layers")
        if args.copy_calibration:
            calibration_copy(torch, dev)
        return

    # graph of one step (all layers)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    tg = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - tg) * 1e3 / args.steps
    us_per_layer = ms_per_step * 1e3 / L
    log(f"[bench] graph: {us_per_layer:.2f} us/layer-step")
    dist = replay_distribution(graph.replay, max(args.steps, 100), L)
    log(f"[bench] per-step replays: p10 / p50 / p90 = {dist['p10']} / {dist['p50']} / {dist['p90']} "
        f"us/layer-step")

    if args.copy_calibration:
        calibration_copy(torch, dev)

    # kernel times of one decode layer-step (eager, profiled): the median over
    # steps of each step's mean dispatch time (one unprofiled step first)
    kinds = {"score": bsattn._lib.KERNEL_SCORE, "topk": bsattn._lib.KERNEL_TOPK,
             "attend": bsattn._lib.KERNEL_ATTEND, "combine": bsattn._lib.KERNEL_COMBINE}
    step()
    torch.cuda.synchronize()
    per_step = profiled_means(layers, kinds, step, max(9, args.steps // 2), torch)
    decode_kernels = {name: round(statistics.median(v), 3) for name, v in per_step.items() if v}
    log("[bench] decode kernels per step (us): " + "; ".join(
        f"{name} {min(v):.2f}-{max(v):.2f}" for name, v in per_step.items() if v))

    # the given-index gather + attention kernel alone (bsattn_attend on
    # precomputed indices), for comparison with the decode path's kernel.
    # Eager calls with the library's profiling on: each kernel dispatch
    # carries its own HIP start/stop events on the launch stream.
    idx = [cache.selectBlocks(q) for cache, q in layers]
    torch.cuda.synchronize()
    nsel = int((idx[0] >= 0).sum(dim=2).max().item())
    for (cache, q), ii in zip(layers, idx):  # warm
        cache.attend(q, ii, scale)
    torch.cuda.synchronize()

    def given_step():
        for (cache, q), ii in zip(layers, idx):
            cache.attend(q, ii, scale)

    per_rep = profiled_means(layers, {"attend": bsattn._lib.KERNEL_ATTEND,
                                      "combine": bsattn._lib.KERNEL_COMBINE},
                             given_step, max(9, args.steps), torch)
    given_us = statistics.median(per_rep["attend"])
    log(f"[bench] given-index kernels per step (us): attend {min(per_rep['attend']):.2f}-"
        f"{max(per_rep['attend']):.2f}")
    given_combine_us = statistics.median(per_rep["combine"]) if per_rep["combine"] else 0.0
    attn_bytes, summ_bytes = algorithmic_bytes(cfg, nsel)
    given_achieved = attn_bytes / (given_us * 1e-6) / 1e9
    # roofline: the gather + attention kernel the timed decode step runs
    # (selection fused into it where the candidates allow), event-timed on
    # its dispatches during the profiled decode steps above
    attend_us = decode_kernels["attend"]
    combine_us = decode_kernels.get("combine", 0.0)
    achieved = attn_bytes / (attend_us * 1e-6) / 1e9
    layer_bytes = attn_bytes + summ_bytes
    log(f"[bench] decode attend kernel: {attend_us:.2f} us, {achieved:.0f} GB/s "
        f"({100 * achieved / HBM_PEAK_GBPS:.1f}% of peak); combine {combine_us:.2f} us; "
        f"given-index attend {given_us:.2f} us ({100 * given_achieved / HBM_PEAK_GBPS:.1f}%)")

    recall = None
    if cfg.key == "c5" and not args.no_recall and not light:
        t0 = time.time()
        recall = recall_report(cfg, layers[0][0], layers[0][1], idx[0], seqs=[0, 1])
        log(f"[bench] recall ({time.time() - t0:.0f}s): {recall}")

    cpu = None
    cpu_dense_path = None
    if not args.no_cpu and args.cpu_seconds > 0 and not light:
        cpu_us, n, thr, cidx, cout = cpu_baseline(cfg, layers[0][0], layers[0][1], args.cpu_seconds)
        same = bool((cidx == idx[0].cpu().numpy()).all())
        out_check = output_check(cfg, layers[0][0].decode(layers[0][1], scale), cout)
        cpu = {"value": round(cpu_us, 1), "unit": "us/layer-step", "cores": thr, "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"layer 0 of the same workload ({cfg.B} seq x {cfg.HKV} kv heads x {cfg.T} "
                         f"tokens): the C oracle's score + select + attend of every (seq, kv head) "
                         f"given the block summaries, pairs over {thr} OpenMP threads, median of "
                         f"{n} layer-steps",
               "selection_matches_gpu": same, "output_vs_gpu": out_check}
        log(f"[bench] cpu oracle: {cpu_us:.0f} us/layer-step ({thr} threads, {cpu_model()}); "
            f"selection equal to the GPU's: {same}; output {out_check}")
        dense_us, nd, thr = cpu_dense(cfg, layers[0][0], layers[0][1], args.cpu_seconds)
        cpu_dense_path = {"value": round(dense_us, 1), "unit": "us/layer-step", "cores": thr,
                          "kind": "reference path (dense)",
                          "sample": f"the reference's dense decode attention over all {cfg.T} cached tokens "
                                    f"(float32 numpy + BLAS, {thr} threads) for sequence 0 of layer 0, "
                                    f"median of {nd} repetitions, x{cfg.B} sequences"}
        log(f"[bench] cpu dense (reference path): {dense_us:.0f} us/layer-step, {thr} threads")

    copy_bw = None if light else copy_bandwidth(torch, dev)
    if copy_bw:
        log(f"[bench] same-run copy bandwidth: {copy_bw['value']} GB/s")
    traffic, traffic_src = recorded_traffic(cfg)
    kv = cfg.dtype if cfg.bits == 0 else f"int{cfg.bits} affine, group 64, fp16 scale/bias"
    result = {
        "metric": cfg.metric,
        "value": round(us_per_layer, 3),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype if cfg.bits == 0 else f"{cfg.dtype} (int{cfg.bits} KV)",
        "data": "synthetic: counter-based splitmix64 + Box-Muller N(0,1) K/V/q, seed "
                f"{CFG_SEED[cfg.key]} + 1000 x layer"
                + (f", {cfg.salient:.0%} of key positions x8" if cfg.salient else "")
                + "; layer 0 = the committed workload digest",
        "inputs": inputs,
        "config": {"workload": f"block-sparse decode layer-step x{L} distinct layer caches",
                   "batch": cfg.B, "q_heads": cfg.HQ, "kv_heads": cfg.HKV, "head_dim": D,
                   "context": cfg.T, "block_size": cfg.TB, "kv": kv, "top_k": cfg.top_k,
                   "sink_blocks": cfg.ns, "recent_blocks": cfg.nr, "selected_blocks": nsel,
                   "layers": L, "step": "score + top-K + attend"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": ("k_attend" if cfg.bits == 0 else "k_attend_q")
                               + " as the decode step runs it (gather + attention"
                               + ("" if cfg.bits == 0 else ", dequant fused") + ")",
                     "launch_us": round(attend_us, 3),
                     "bytes_per_launch": attn_bytes, "combine_us": round(combine_us, 3),
                     "given_index": {"launch_us": round(given_us, 3),
                                     "achieved": round(given_achieved, 1),
                                     "frac": round(given_achieved / HBM_PEAK_GBPS, 4),
                                     "combine_us": round(given_combine_us, 3)}},
        "decode_kernels_us": decode_kernels,
        "copy_bandwidth": copy_bw,
        "attend_frac_of_copy": round(achieved / copy_bw["value"], 4) if copy_bw else None,
        "layer_step_GBps": round(layer_bytes / (us_per_layer * 1e-6) / 1e9, 1),
        "eager_us_per_layer_step": round(eager_ms * 1e3 / L, 3),
        "us_per_layer_step_distribution": dist,
        "cpu_baseline": cpu,
        "cpu_dense_reference_path": cpu_dense_path,
    }
    if recall is not None:
        result["recall"] = recall
    del layers, idx
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return result


def output_check(cfg: Config, gpu_out, ref):
    """GPU output of a layer against the oracle's fp64 output on the same
    inputs: raw max-abs error, and the error net of the final rounding to
    the output dtype (|gpu - ref| - ulp(ref) / 2), against the bar (2e-3 for
    16-bit caches, 1e-2 for affine ones)."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    dt = cfg.dtype
    got = O.to_f32(host16(gpu_out, torch, np).reshape(ref.shape), dt).astype(np.float64)
    mant = 10 if dt == "f16" else 7
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -14))) - mant)
    raw = float(np.max(np.abs(got - ref)))
    net = float(np.max(np.abs(got - ref) - 0.5 * ulp))
    bar = 2e-3 if cfg.bits == 0 else 1e-2
    return {"max_abs": raw, "max_abs_net_of_output_rounding": net, "bar": bar, "within_bar": net <= bar,
            "out_max_abs": float(np.max(np.abs(ref))), "what": "layer 0's GPU decode output against the "
            "oracle's fp64 output (the cpu_baseline leg's last repetition)"}


def other_summary(r: dict, per: str) -> dict:
    """The figures of a non-headline workload's result kept in the headline line."""
    keep = {"metric": r["metric"], per: r["value"], "config": r["config"]}
    if "roofline" in r:
        ro = r["roofline"]
        keep.update({"attend_kernel": ro["kernel"], "attend_us": ro["launch_us"],
                     "attend_bytes_per_launch": ro["bytes_per_launch"], "attend_achieved_GBps": ro["achieved"],
                     "attend_frac": ro["frac"], "traffic": ro["traffic"], "traffic_source": ro["traffic_source"],
                     "given_index": ro["given_index"], "decode_kernels_us": r["decode_kernels_us"],
                     "layer_step_GBps": r["layer_step_GBps"], "data": r["data"], "inputs": r["inputs"]})
    else:
        keep.update({k: r[k] for k in ("kernels_us_per_step", "kernel_us_per_step_total",
                                       "kernel_GBps", "kernel_frac", "bytes_per_step",
                                       "traffic_note") if k in r})
    return keep


def _mix(x: int) -> int:
    """splitmix64 finaliser on a Python int (mod 2^64)."""
    z = (x + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
    return z ^ (z >> 31)


def _hash3(seed: int, stream: int, index: int) -> int:
    """splitmix64 finaliser chained over (seed, stream, index)."""
    return _mix((_mix((_mix(seed) + stream) & 0xFFFFFFFFFFFFFFFF) + index) & 0xFFFFFFFFFFFFFFFF)


# ---------------------------------------------------------------------------
# The benchmark inputs: the counter-based generator of the decode workloads
# (element i of stream s under seed S is normal(S, s, i); keys of sequence b,
# kv head h, token t, dim d are element ((b Hkv + h) T + t) D + d of stream 1,
# values the same of stream 2, q element (b Hq + hq) D + d of stream 0; a
# salient fraction of each (b, h)'s token positions, drawn on stream 3, have
# their keys scaled by 8 before rounding), computed with torch on the device.
# ---------------------------------------------------------------------------
S_Q, S_K, S_V, S_SALIENT = 0, 1, 2, 3


def _s64(c: int) -> int:
    """A 64-bit pattern as the signed value torch's int64 holds."""
    return c - (1 << 64) if c >= 1 << 63 else c


def _mix_t(z):
    """splitmix64 finaliser on an int64 tensor: products wrap mod 2^64, and the
    right shifts are made logical by masking."""
    z = z + _s64(0x9E3779B97F4A7C15)
    z = (z ^ ((z >> 30) & ((1 << 34) - 1))) * _s64(0xBF58476D1CE4E5B9)
    z = (z ^ ((z >> 27) & ((1 << 37) - 1))) * _s64(0x94D049BB133111EB)
    return z ^ ((z >> 31) & ((1 << 33) - 1))


def counter_normal(seed: int, stream: int, start: int, n: int, torch, dev):
    """normal(seed, stream, start + i), i < n (start and n even), float64:
    Box-Muller in double over the hash pair (2p, 2p + 1) of index pair p,
    u1 = ((a >> 11) + 1) 2^-53 in (0, 1], u2 = (b >> 11) 2^-53; even
    indices take r cos(2 pi u2), odd ones r sin(2 pi u2)."""
    assert start % 2 == 0 and n % 2 == 0
    p2 = 2 * torch.arange(start // 2, (start + n) // 2, device=dev, dtype=torch.int64)
    base = _s64(_mix((_mix(seed) + stream) & 0xFFFFFFFFFFFFFFFF))
    a = _mix_t(p2 + base)
    b = _mix_t(p2 + (base + 1 if base + 1 < 1 << 63 else base + 1 - (1 << 64)))
    del p2
    u1 = (((a >> 11) & ((1 << 53) - 1)) + 1).double() * 2.0 ** -53
    u2 = ((b >> 11) & ((1 << 53) - 1)).double() * 2.0 ** -53
    del a, b
    r = torch.sqrt(-2.0 * torch.log(u1))
    t = 6.283185307179586476925286766559 * u2
    return torch.stack((r * torch.cos(t), r * torch.sin(t)), dim=-1).reshape(-1)


def round16(x, dtype: str, torch):
    """float64 tensor -> bf16 / fp16 storage words (int16), rounded to nearest
    even straight from the double (no float32 step, which would round twice):
    the exponent and top mantissa bits of the double's pattern plus the round
    bit, rebiased; results below the target's normal range are |x| scaled by
    the smallest subnormal, rounded to an integer; beyond the largest finite,
    infinity."""
    mb, eb = (7, 127) if dtype == "bf16" else (10, 15)
    sh = 52 - mb
    bits = x.view(torch.int64)
    sign = (bits < 0).to(torch.int64) << 15
    mag = bits & 0x7FFFFFFFFFFFFFFF
    v = mag >> sh
    rem = mag & ((1 << sh) - 1)
    half = 1 << (sh - 1)
    up = (rem > half) | ((rem == half) & ((v & 1) == 1))
    v = (v + up.to(torch.int64) - ((1023 - eb) << mb)).clamp(max=0xFF << mb if dtype == "bf16" else 0x1F << mb)
    sub = torch.round(x.abs() * 2.0 ** (eb - 1 + mb)).to(torch.int64)
    v = torch.where((mag >> 52) < 1023 - eb + 1, sub, v)
    return (v | sign).to(torch.int16)


def choose_positions(seed: int, stream: int, keys, n: int, count: int):
    """For each key, the first `count` entries of a Fisher-Yates shuffle of
    range(n) whose step i swaps entry i with entry i + hash3(seed, stream,
    (key << 32) | i) mod (n - i) -> int64 array [len(keys), count]."""
    import numpy as np
    c = [np.uint64(x) for x in (0x9E3779B97F4A7C15, 0xBF58476D1CE4E5B9, 0x94D049BB133111EB)]

    def mix_np(z):
        z = z + c[0]
        z = (z ^ (z >> np.uint64(30))) * c[1]
        z = (z ^ (z >> np.uint64(27))) * c[2]
        return z ^ (z >> np.uint64(31))

    base = np.uint64(_mix((_mix(seed) + stream) & 0xFFFFFFFFFFFFFFFF))
    kk = np.asarray(keys, np.uint64) << np.uint64(32)
    rows = np.arange(len(keys))
    perm = np.tile(np.arange(n, dtype=np.int64), (len(keys), 1))
    out = np.empty((len(keys), count), np.int64)
    with np.errstate(over="ignore"):
        for i in range(min(count, n)):
            h = mix_np(base + (kk | np.uint64(i)))
            j = i + (h % np.uint64(n - i)).astype(np.int64)
            t = perm[rows, i].copy()
            perm[rows, i] = perm[rows, j]
            perm[rows, j] = t
            out[:, i] = perm[rows, i]
    return out


def bench_loop(args, light: bool = False):
    """Config 4: decode loop with appends, eager (page tables change every
    step) -> the result dict.  light: only the one-call loop and its kernel
    times (no two-call or graph legs, no copy reference)."""
    import numpy as np
    import torch
    import bsattn
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, HQ, HKV, TB, K, STEPS, SEED = 32, 32, 8, 64, 32, 256, 1004
    steps = args.steps if args.steps != 20 else STEPS
    # lengths U[8192, 65536] from the counter-based stream 4 of seed 1004
    lens = np.array([8192 + _hash3(SEED, 4, b) % (65536 - 8192 + 1) for b in range(B)], np.int64)
    g = torch.Generator(device=dev)
    g.manual_seed(4004)
    mbps = (int(lens.max()) + steps) // TB + 2
    pages = int(sum(-(-(int(n) + steps) // TB) for n in lens)) + B
    cache = bsattn.BlockSparseKVCache(max_seqs=B, num_q_heads=HQ, num_kv_heads=HKV, head_dim=D,
                                      block_size=TB, dtype=torch.float16, top_k=K, sink_blocks=1,
                                      recent_blocks=1, max_blocks_per_seq=mbps, num_pages=pages,
                                      device=0)
    # the physical page order is the free list permuted from the seed (stream
    # 5): every sequence's pages are scattered through the pool
    cache.shuffleFreePages(SEED)
    t0 = time.time()
    for b in range(B):
        n = int(lens[b])
        k = torch.randn(1, HKV, n, D, device=dev, generator=g).half()
        v = torch.randn(1, HKV, n, D, device=dev, generator=g).half()
        cache.append(k, v, seq_ids=[b])
        del k, v
    torch.cuda.synchronize()
    bt = cache.seqPages(0)
    log(f"[bench] c4: seq 0 pages {bt[:6]}... ({len(bt)} pages, ascending runs: "
        f"{sum(1 for a, c in zip(bt, bt[1:]) if c == a + 1)} of {len(bt) - 1})")
    log(f"[bench] c4: prefilled {B} sequences ({int(lens.sum())} tokens) in {time.time() - t0:.1f}s")
    kn = torch.randn(steps + args.warmup, B, HKV, 1, D, device=dev, generator=g).half()
    vn = torch.randn(steps + args.warmup, B, HKV, 1, D, device=dev, generator=g).half()
    qs = torch.randn(steps + args.warmup, B, HQ, 1, D, device=dev, generator=g).half()
    scale = 1.0 / math.sqrt(D)
    # a step = attentionWithCacheUpdate's decode step: appendDecode (here one
    # launch of the fused decode, which also appends the token)
    for i in range(args.warmup):
        cache.appendDecode(kn[i], vn[i], qs[i], scale)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.warmup, args.warmup + steps):
        cache.appendDecode(kn[i], vn[i], qs[i], scale)
    torch.cuda.synchronize()
    us_step = (time.perf_counter() - t0) * 1e6 / steps
    us_two = None
    if not light:
        # the same steps as two calls (append, then decode)
        cache.trim(steps, list(range(B)))
        t0 = time.perf_counter()
        for i in range(args.warmup, args.warmup + steps):
            cache.append(kn[i], vn[i])
            cache.decode(qs[i], scale)
        torch.cuda.synchronize()
        us_two = (time.perf_counter() - t0) * 1e6 / steps
    log(f"[bench] c4: {us_step:.2f} us/step (appendDecode), {us_two} (append + decode)")
    # kernel time per step: the same steps again (trimmed back first), profiled
    cache.trim(steps, list(range(B)))
    cache.profile(True)
    for i in range(args.warmup, args.warmup + steps):
        cache.appendDecode(kn[i], vn[i], qs[i], scale)
    torch.cuda.synchronize()
    kern = {}
    total = 0.0
    names = {"append": bsattn._lib.KERNEL_APPEND, "summary": bsattn._lib.KERNEL_SUMMARY,
             "append+score": bsattn._lib.KERNEL_SCORE, "topk": bsattn._lib.KERNEL_TOPK,
             "attend": bsattn._lib.KERNEL_ATTEND, "combine": bsattn._lib.KERNEL_COMBINE}
    for name, kind in names.items():
        ms, n = cache.profileRead(kind)
        if n:
            kern[name] = {"us_per_step": round(ms * 1e3 / steps, 3), "launches": n}
            total += ms * 1e3 / steps
    cache.profile(False)
    log(f"[bench] c4: {us_step:.2f} us/step eager, kernels {total:.2f} us/step")
    nsel = K + 2
    gather = int(B * HKV * nsel * TB * 2 * D * 2)
    # scoring reads every full block's summary of every (sequence, kv head)
    summ = int(sum(HKV * ((int(n) + steps // 2) // TB) * D * 2 for n in lens))
    per_step = gather + summ + B * HQ * D * 2 * 2
    k_gbps = per_step / (total * 1e-6) / 1e9 if total else None
    result = {
        "metric": "block-sparse decode loop with appends µs/step, B=32 variable lengths",
        "value": round(us_step, 3), "unit": "us/step", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(us_step / 1e3, 5), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic: torch RNG on device, K/V/q ~ N(0,1); lengths from splitmix64 "
                "(seed 1004, stream 4); physical page order shuffled from seed 1004 (stream 5)",
        "config": {"workload": "decode loop: append 1 token per sequence, score + top-K + attend",
                   "batch": B, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
                   "lengths": [int(x) for x in lens], "block_size": TB, "top_k": K,
                   "sink_blocks": 1, "recent_blocks": 1, "pages": pages, "page_order": "shuffled",
                   "timing": "eager wall clock per step (ctypes launches included)",
                   "step_call": "appendDecode (one launch: append, patches and summary fold inside the fused decode)"},
        "kernels_us_per_step": kern, "kernel_us_per_step_total": round(total, 3),
        "gather_bytes_per_step": gather,
        "bytes_per_step": per_step,
        "kernel_GBps": round(k_gbps, 1) if k_gbps else None,
        "kernel_frac": round(k_gbps / HBM_PEAK_GBPS, 4) if k_gbps else None,
        "traffic_note": "bytes_per_step = selected K/V + every full block's summary + q + out; one "
                        "layer cache (4.8 GB of K/V) is re-read every step, so the 37.7 MB of "
                        "summaries can stay in the 256 MB Infinity Cache",
    }
    if light:
        del cache, kn, vn, qs
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        return result
    # the same steps as a HIP graph: reserve pages, capture one [appendStep,
    # decode] step, replay it per step with that step's inputs copied in
    cache.trim(steps, list(range(B)))
    cache.reserve(steps + 1, list(range(B)))
    kb, vb, qb = kn[args.warmup].clone(), vn[args.warmup].clone(), qs[args.warmup].clone()
    cache.appendStep(kb, vb)  # warm-up (one extra token)
    cache.decode(qb, scale)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cache.appendStep(kb, vb)
        cache.decode(qb, scale)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(args.warmup, args.warmup + steps):
        kb.copy_(kn[i])
        vb.copy_(vn[i])
        qb.copy_(qs[i])
        ev[i - args.warmup][0].record()
        graph.replay()
        ev[i - args.warmup][1].record()
    torch.cuda.synchronize()
    us_graph = (time.perf_counter() - t0) * 1e6 / steps
    reps = np.array([a.elapsed_time(b) * 1e3 for a, b in ev])
    p10, p50, p90 = np.percentile(reps, [10, 50, 90])
    dist = {"p10": round(float(p10), 3), "p50": round(float(p50), 3), "p90": round(float(p90), 3),
            "reps": steps, "what": "GPU time of one replayed step (input copies excluded)"}
    cache.sync()
    log(f"[bench] c4: {us_graph:.2f} us/step as a replayed HIP graph (inputs copied in per step)")
    result.update({
        "two_calls_us_per_step": round(us_two, 3),
        "graph_us_per_step": round(us_graph, 3),
        "graph_step_us_distribution": dist,
        "copy_bandwidth": copy_bandwidth(torch, dev),
        "gather_GBps_at_kernel_time": round(gather / (total * 1e-6) / 1e9, 1) if total else None,
    })
    return result


def bench_prefill(args, bits=0):
    """Dense causal prefill attention of a 512-token chunk at the end of a
    32768-token context (B=8, Hq=32, Hkv=8, Tb=64; bf16 caches,
    or with bits = 4 MLX-affine int4 caches, group 64, fp16), over 4 layer
    caches (beyond the 256 MB Infinity Cache).  MFMA-bound: algorithmic
    FLOPs = 4 * D * sum over queries of the tokens they see."""
    import torch
    import bsattn
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, HQ, HKV, TB, T, L, LAYERS = 8, 32, 8, 64, 32768, 512, 4
    dt = torch.float16 if bits else torch.bfloat16
    g = torch.Generator(device=dev)
    g.manual_seed(5005 + bits)
    caches = []
    for _ in range(LAYERS):
        c = bsattn.BlockSparseKVCache(max_seqs=B, num_q_heads=HQ, num_kv_heads=HKV, head_dim=D,
                                      block_size=TB, dtype=dt, kv_bits=bits, top_k=32,
                                      max_blocks_per_seq=T // TB + 2, device=0)
        for b in range(B):
            k = torch.randn(1, HKV, T, D, device=dev, generator=g).to(dt)
            v = torch.randn(1, HKV, T, D, device=dev, generator=g).to(dt)
            c.append(k, v, seq_ids=[b])
            del k, v
        caches.append(c)
    q = torch.randn(B, HQ, L, D, device=dev, generator=g).to(dt)
    scale = 1.0 / math.sqrt(D)
    for i in range(args.warmup):
        caches[i % LAYERS].prefill(q, scale)
    torch.cuda.synchronize()
    steps = args.steps
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        caches[i % LAYERS].prefill(q, scale)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    turn = iter(range(1 << 30))
    dist = replay_distribution(lambda: caches[next(turn) % LAYERS].prefill(q, scale), steps, 1)
    flops = 4.0 * D * B * HQ * sum(T - L + i + 1 for i in range(L))
    tf = flops / (us * 1e-6) / 1e12
    kind = f"int{bits} affine" if bits else "bf16"
    log(f"[bench] prefill chunk {L} at {T} ctx ({kind} cache): {us:.1f} us/layer, {tf:.1f} TFLOP/s "
        f"({100 * tf / 2500:.1f}% of 2.5 PFLOP/s dense 16-bit)")
    print(json.dumps({
        "metric": f"dense causal prefill attention µs per layer, 512-token chunk at 32k ctx, {kind} cache",
        "value": round(us, 2), "unit": "us/layer", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16 (int4 KV)" if bits else "bf16",
        "data": "synthetic: torch RNG on device, N(0,1)",
        "config": {"workload": "prefill chunk attention x4 distinct layer caches", "batch": B,
                   "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "context": T, "chunk": L,
                   "block_size": TB, "kv": kind},
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tf / 2500.0, 4), "traffic": None},
        "us_per_layer_distribution": dist,
    }), flush=True)


def bench_multi(args, cfg: Config, L: int = 4):
    """Speculative verify at B=8, Hq=32, Hkv=8, 32k tokens, Tb=64, bf16:
    decodeMulti of L query tokens per sequence (each selects its own blocks
    over its own prefix), over the workload's distinct layer caches, as a
    replayed HIP graph; against L single-token decodes of the same caches."""
    import torch
    import bsattn
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    NL = args.layers or cfg.layers
    layers = [make_layer(cfg, i, dev, torch, bsattn) for i in range(NL)]
    g = torch.Generator(device=dev)
    g.manual_seed(7007)
    qm = torch.randn(cfg.B, cfg.HQ, L, D, device=dev, generator=g).to(torch_dtype(torch, cfg))
    scale = 1.0 / math.sqrt(D)

    def timed(step):
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            step()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e6 / args.steps / NL, replay_distribution(
            graph.replay, max(args.steps, 50), NL)

    multi_us, dist = timed(lambda: [c.decodeMulti(qm, scale) for c, _ in layers])
    qs = [qm[:, :, i:i + 1].contiguous() for i in range(L)]
    single_us, _ = timed(lambda: [c.decode(qq, scale) for c, _ in layers for qq in qs])
    log(f"[bench] mq: {L} query tokens per sequence: {multi_us:.2f} us/layer-step "
        f"(L single decodes: {single_us:.2f})")
    print(json.dumps({
        "metric": f"block-sparse multi-token decode (speculative verify, L={L}) µs per layer-step",
        "value": round(multi_us, 3), "unit": "us/layer-step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(multi_us * NL / 1e3, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": cfg.dtype,
        "data": "synthetic: layer caches from the counter-based generator (as the decode benchmark), "
                "the L query tokens per sequence from torch's device RNG, N(0,1)",
        "config": {"workload": f"decodeMulti x{NL} distinct layer caches", "batch": cfg.B,
                   "q_heads": cfg.HQ, "kv_heads": cfg.HKV, "head_dim": D, "context": cfg.T,
                   "block_size": cfg.TB, "top_k": cfg.top_k, "query_tokens": L},
        "single_decodes_us_per_layer_step": round(single_us, 3),
        "us_per_layer_step_distribution": dist,
    }), flush=True)


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only: the block-sparse decode "
                                   "path is a single-GPU kernel set (it would shard by sequence, "
                                   "then by kv head, with no exchange on this path); run with "
                                   "--gpus 1"}))
        sys.exit(2)
    if args.config == "c4":
        print(json.dumps(bench_loop(args)), flush=True)
    elif args.config == "pf":
        bench_prefill(args)
    elif args.config == "pfq":
        bench_prefill(args, bits=4)
    elif args.config == "mq":
        bench_multi(args, CONFIGS["c2"])
    elif args.config == "c2" and not args.no_others and not args.counters:
        # the headline, then the other decode workloads (no CPU legs), all
        # in the one JSON line
        result = bench_layers(args, CONFIGS["c2"])
        others = {}
        for key in ("c3", "c5"):
            t0 = time.time()
            others[key] = other_summary(bench_layers(args, CONFIGS[key], light=True), "us_per_layer_step")
            log(f"[bench] other config {key}: {others[key]['us_per_layer_step']} us/layer-step "
                f"({time.time() - t0:.0f}s)")
        t0 = time.time()
        others["c4"] = other_summary(bench_loop(args, light=True), "us_per_step")
        log(f"[bench] other config c4: {others['c4']['us_per_step']} us/step ({time.time() - t0:.0f}s)")
        result["other_configs"] = others
        print(json.dumps(result), flush=True)
    else:
        r = bench_layers(args, CONFIGS[args.config])
        if r is not None:
            print(json.dumps(r), flush=True)


if __name__ == "__main__":
    main()
