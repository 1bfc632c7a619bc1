"""Block-sparse decode attention benchmark on one MI355X.

Workload (the headline configuration): B=8 sequences, Hq=32, Hkv=8, D=128,
32768 tokens each in 64-token blocks (512 blocks), bf16 K/V ~ N(0,1) with 1%
of key positions per (sequence, kv head) scaled x8, top-32 + sink + recent
(34 blocks selected), softmax scale 1/sqrt(128).  36 distinct layer caches
(one per layer, ~1.1 GB each) so the working set is far above the 256 MB
Infinity Cache.

A step = one decode step through all 36 layers: per layer, block scoring +
top-K select + gathered attention (bsattn_decode).  `value` = microseconds
per layer-step.  Steps are replayed from a HIP graph (captured once) so the
timing is the GPU's, not the Python launcher's; the eager (ctypes per call)
figure is reported alongside.

roofline: the gather + attention kernel (k_attend, via bsattn_attend on
precomputed indices), timed with HIP start/stop events attached to each of
its dispatches on the launch stream (the library's profiling hook);
algorithmic bytes per launch = selected K+V bytes + q + out + indices.
cpu_baseline: the CPU oracle (single thread) doing the same layer-step
(score given summaries, select, attend) on layer 0's data.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-swift-lm_amd"))

METRIC = "block-sparse decode attn µs/layer-step + achieved HBM GB/s (% of peak), 32k ctx"
HBM_PEAK_GBPS = 8000.0

B, HQ, HKV, D, T, TB = 8, 32, 8, 128, 32768, 64
TOP_K, NS, NR = 32, 1, 1
LAYERS = 36
SALIENT = 0.01


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one plain 256 MiB device copy (a known-traffic dispatch "
                         "for scaling hardware byte counters)")
    return ap.parse_args()


def make_layer(layer, dev, torch, bsattn):
    g = torch.Generator(device=dev)
    g.manual_seed(1001 * 1000 + layer)
    cache = bsattn.BlockSparseKVCache(max_seqs=B, num_q_heads=HQ, num_kv_heads=HKV, head_dim=D,
                                      block_size=TB, dtype=torch.bfloat16, top_k=TOP_K,
                                      sink_blocks=NS, recent_blocks=NR,
                                      max_blocks_per_seq=T // TB + 2, device=dev.index)
    n_sal = int(round(SALIENT * T))
    for b in range(B):  # one sequence at a time keeps the temporaries small
        mult = torch.ones(HKV, T, device=dev)
        pos = torch.rand(HKV, T, device=dev, generator=g).argsort(dim=1)[:, :n_sal]
        mult.scatter_(1, pos, 8.0)
        k = (torch.randn(HKV, T, D, device=dev, generator=g) * mult[..., None]).to(torch.bfloat16)
        v = torch.randn(HKV, T, D, device=dev, generator=g).to(torch.bfloat16)
        cache.append(k[None].contiguous(), v[None].contiguous(), seq_ids=[b])
        del k, v, mult, pos
    q = torch.randn(B, HQ, 1, D, device=dev, generator=g).to(torch.bfloat16)
    return cache, q


def algorithmic_bytes(nsel):
    bytes_tok = 2 * D * 2                      # K + V row, bf16
    gather = B * HKV * nsel * TB * bytes_tok
    qo = B * HQ * D * 2 * 2
    idx = B * HKV * nsel * 4
    summ = B * HKV * (T // TB) * D * 2
    return gather + qo + idx, summ


def recorded_traffic():
    """HBM bytes per k_attend launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (copy-calibrated); None when it is absent."""
    path = os.path.join(ROOT, "profiles", "k_attend_b8_ctx32k_bf16_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1]), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def cpu_baseline(cache, q, seconds):
    """Oracle layer-step on layer 0's data: per (sequence, kv head) score all
    candidate summaries, select, attend.  Single thread."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    k, v = cache.export(list(range(B)))
    kh = k.view(torch.int16).cpu().numpy().view(np.uint16)
    vh = v.view(torch.int16).cpu().numpy().view(np.uint16)
    qh = q.view(torch.int16).cpu().numpy().view(np.uint16).reshape(B, HQ, D)
    summ = [cache.exportSummaries(b).view(torch.int16).cpu().numpy().view(np.uint16) for b in range(B)]
    G = HQ // HKV
    scale = 1.0 / math.sqrt(D)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        for b in range(B):
            for h in range(HKV):
                qq = qh[b, h * G:(h + 1) * G]
                sc = O.score_blocks(qq, summ[b][h], "bf16")
                idx, n = O.select(sc, T, TB, NS, NR, TOP_K)
                O.attend(qq, kh[b, h], vh[b, h], TB, idx[:n], scale, "bf16")
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2] * 1e6, len(times)


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only: the block-sparse decode "
                                   "path is a single-GPU kernel set (see DESIGN.md for how it "
                                   "would shard); run with --gpus 1"}))
        sys.exit(2)
    import torch
    import bsattn
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = args.layers
    t0 = time.time()
    layers = [make_layer(i, dev, torch, bsattn) for i in range(L)]
    torch.cuda.synchronize()
    log(f"[bench] built {L} layer caches in {time.time() - t0:.1f}s "
        f"({layers[0][0].poolBytes / 2**30:.2f} GiB each)")
    scale = 1.0 / math.sqrt(D)
    outs = [torch.empty_like(q) for _, q in layers]

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

    if args.copy_calibration:
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log("[bench] calibration copy: 256 MiB read + 256 MiB written")
        del src, dst

    # roofline: the gather + attention kernel alone, on precomputed indices.
    # Eager bsattn_attend calls with the library's profiling on: each kernel
    # dispatch carries its own HIP start/stop events on the launch stream.
    idx = [cache.selectBlocks(q) for cache, q in layers]
    torch.cuda.synchronize()
    nsel = int((idx[0] >= 0).sum(dim=2).max().item())
    for (cache, q), ii in zip(layers, idx):  # warm
        cache.attend(q, ii, scale)
    torch.cuda.synchronize()
    for cache, _ in layers:
        cache.profile(True)
    reps = max(5, args.steps)
    for _ in range(reps):
        for (cache, q), ii in zip(layers, idx):
            cache.attend(q, ii, scale)
    torch.cuda.synchronize()
    tot_ms, launches, comb_ms = 0.0, 0, 0.0
    for cache, _ in layers:
        ms, n = cache.profileRead(bsattn._lib.KERNEL_ATTEND)
        cms, _ = cache.profileRead(bsattn._lib.KERNEL_COMBINE)
        tot_ms, launches, comb_ms = tot_ms + ms, launches + n, comb_ms + cms
        cache.profile(False)
    attend_us = tot_ms * 1e3 / launches
    combine_us = comb_ms * 1e3 / launches
    attn_bytes, summ_bytes = algorithmic_bytes(nsel)
    achieved = attn_bytes / (attend_us * 1e-6) / 1e9
    layer_bytes = attn_bytes + summ_bytes
    log(f"[bench] attend kernel: {attend_us:.2f} us, {achieved:.0f} GB/s "
        f"({100 * achieved / HBM_PEAK_GBPS:.1f}% of peak); combine {combine_us:.2f} us")

    cpu = None
    if not args.no_cpu and args.cpu_seconds > 0:
        cpu_us, n = cpu_baseline(layers[0][0], layers[0][1], args.cpu_seconds)
        cpu = {"value": round(cpu_us, 1), "unit": "us/layer-step", "cores": 1, "kind": "port",
               "sample": f"layer 0 of the same workload (8 seq x 8 kv heads x 32768 tokens), "
                         f"oracle score+select+attend per (seq, kv head) given summaries, "
                         f"median of {n} layer-steps, 1 thread"}
        log(f"[bench] cpu oracle: {cpu_us:.0f} us/layer-step")

    traffic, traffic_src = recorded_traffic()
    result = {
        "metric": METRIC,
        "value": round(us_per_layer, 3),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: torch RNG on device, bf16 K/V ~ N(0,1), 1% of key positions x8, random-init q",
        "config": {"workload": f"block-sparse decode layer-step x{L} distinct layer caches",
                   "batch": B, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "context": T,
                   "block_size": TB, "top_k": TOP_K, "sink_blocks": NS, "recent_blocks": NR,
                   "selected_blocks": nsel, "layers": L, "step": "score + top-K + attend"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": "k_attend (gather + attention)", "launch_us": round(attend_us, 3),
                     "bytes_per_launch": attn_bytes, "combine_us": round(combine_us, 3)},
        "layer_step_GBps": round(layer_bytes / (us_per_layer * 1e-6) / 1e9, 1),
        "eager_us_per_layer_step": round(eager_ms * 1e3 / L, 3),
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
