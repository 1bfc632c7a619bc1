"""Shared helpers for the tests: seeded workload generation with the oracle's
counter-based RNG, oracle evaluation per (sequence, kv head), and the GPU
upload / comparison plumbing."""
from __future__ import annotations

import math
import sys
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

import oracle as O

DT = {"f16": O.F16, "bf16": O.BF16}

# Streams of the counter-based RNG
S_Q, S_K, S_V, S_SALIENT, S_LEN, S_SHUFFLE = 0, 1, 2, 3, 4, 5


@dataclass
class Workload:
    """Seeded decode workload: sequences of (possibly different) lengths."""
    seed: int
    B: int
    Hq: int
    Hkv: int
    D: int
    Tb: int
    dtype: str
    lens: List[int]
    top_k: int
    ns: int = 1
    nr: int = 1
    salient_frac: float = 0.0
    salient_mult: float = 8.0
    q: np.ndarray = field(default=None, repr=False)       # [B, Hq, D]
    keys: List[np.ndarray] = field(default=None, repr=False)    # per seq [Hkv, T, D]
    values: List[np.ndarray] = field(default=None, repr=False)

    @property
    def G(self):
        return self.Hq // self.Hkv

    @property
    def scale(self):
        return 1.0 / math.sqrt(self.D)

    @property
    def nsel_max(self):
        return self.ns + self.nr + self.top_k


def make_workload(seed, B, Hq, Hkv, T, Tb, dtype, top_k, ns=1, nr=1, D=128,
                  salient_frac=0.0, lens=None, prefix=None) -> Workload:
    """Keys of sequence b, kv head h, token t, dim d use element index
    ((b*Hkv + h)*Tcap + t)*D + d of stream 1 (values: stream 2); q uses
    (b*Hq + hq)*D + d of stream 0.  salient_frac of each (b, h)'s token
    positions (chosen on stream 3) have their keys scaled by 8 before
    rounding.  With `prefix`, only each sequence's first `prefix` tokens are
    generated (the same values as in the full workload; `lens` stays full)."""
    lens = list(lens) if lens is not None else [T] * B
    Tcap = max(lens)
    w = Workload(seed, B, Hq, Hkv, D, Tb, dtype, lens, top_k, ns, nr, salient_frac)
    w.q = O.fill_normal(seed, S_Q, 0, (B, Hq, D), dtype)
    w.keys, w.values = [], []
    for b in range(B):
        Tl = lens[b]
        Tg = Tl if prefix is None else min(Tl, prefix)
        mult = None
        if salient_frac > 0:
            mult = np.ones((Hkv, Tl), np.float64)
            cnt = int(round(salient_frac * Tl))
            for h in range(Hkv):
                pos = O.choose_positions(seed, S_SALIENT, b * Hkv + h, Tl, cnt)
                mult[h, pos] = w.salient_mult
        k = np.empty((Hkv, Tg, D), np.uint16)
        v = np.empty((Hkv, Tg, D), np.uint16)
        for h in range(Hkv):
            start = ((b * Hkv + h) * Tcap) * D
            k[h] = O.fill_normal(seed, S_K, start, (Tg, D), dtype,
                                 row_mult=None if mult is None else np.ascontiguousarray(mult[h, :Tg]))
            v[h] = O.fill_normal(seed, S_V, start, (Tg, D), dtype)
        w.keys.append(k)
        w.values.append(v)
    return w


# The configurations' inputs (seed 1000 + config number).  C4's lengths are
# its initial lengths U[8192, 65536] (stream 4) plus its 256 appended tokens.
def config_args(name: str) -> dict:
    if name in ("C1_f16", "C1_bf16"):
        return dict(seed=1001, B=1, Hq=32, Hkv=8, T=4096, Tb=64, dtype=name[3:], top_k=8)
    if name == "C2":
        return dict(seed=1002, B=8, Hq=32, Hkv=8, T=32768, Tb=64, dtype="bf16", top_k=32,
                    salient_frac=0.01)
    if name == "C3":
        return dict(seed=1003, B=4, Hq=32, Hkv=8, T=131072, Tb=64, dtype="f16", top_k=64)
    if name == "C4":
        lens = [O.uniform_int(1004, S_LEN, b, 8192, 65536) + 256 for b in range(32)]
        return dict(seed=1004, B=32, Hq=32, Hkv=8, T=max(lens), Tb=64, dtype="f16", top_k=32, lens=lens)
    if name == "C5":
        return dict(seed=1005, B=8, Hq=64, Hkv=4, T=262144, Tb=32, dtype="f16", top_k=128, nr=4)
    raise KeyError(name)


CONFIGS = ("C1_f16", "C1_bf16", "C2", "C3", "C4", "C5")
DIGEST_PREFIX = 256


def workload_digest(w: Workload, prefix: Optional[int] = None) -> str:
    """SHA-256 over the lengths (int32), q, then every (sequence, kv head)'s
    keys and values (their first `prefix` tokens with `prefix`), as
    little-endian 16-bit storage words."""
    import hashlib
    h = hashlib.sha256()
    h.update(np.asarray(w.lens, "<i4").tobytes())
    h.update(np.ascontiguousarray(w.q, "<u2").tobytes())
    for b in range(w.B):
        for hh in range(w.Hkv):
            n = w.keys[b].shape[1] if prefix is None else min(prefix, w.lens[b])
            h.update(np.ascontiguousarray(w.keys[b][hh, :n], "<u2").tobytes())
            h.update(np.ascontiguousarray(w.values[b][hh, :n], "<u2").tobytes())
    return h.hexdigest()


def input_digests() -> dict:
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "input_digests.json")) as f:
        return json.load(f)


def check_config_inputs(w: Workload, name: str) -> None:
    """The generated inputs of configuration `name` hash to the committed
    digests (full and prefix)."""
    want = input_digests()[name]
    assert workload_digest(w, DIGEST_PREFIX) == want["prefix_sha256"], f"{name}: input prefix digest differs"
    assert workload_digest(w) == want["sha256"], f"{name}: input digest differs"


def oracle_decode(w: Workload):
    """-> idx [B, Hkv, nsel_max] int32, out [B, Hq, D] float64, summaries per seq."""
    idx = np.full((w.B, w.Hkv, w.nsel_max), -1, np.int32)
    out = np.zeros((w.B, w.Hq, w.D), np.float64)
    for b in range(w.B):
        for h in range(w.Hkv):
            i, n, o = O.decode_head(w.q[b, h * w.G:(h + 1) * w.G], w.keys[b][h], w.values[b][h],
                                    w.Tb, w.ns, w.nr, w.top_k, w.scale, w.dtype)
            idx[b, h] = i
            out[b, h * w.G:(h + 1) * w.G] = o
    return idx, out


def oracle_summaries(w: Workload, b: int) -> np.ndarray:
    return np.stack([O.summaries(w.keys[b][h], w.Tb, w.dtype) for h in range(w.Hkv)])


def ulp(x: np.ndarray, dtype: str) -> np.ndarray:
    """Spacing of the output dtype at |x|."""
    mant = 10 if dtype == "f16" else 7
    ax = np.maximum(np.abs(x), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(ax)) - mant)


def output_error(gpu_out: np.ndarray, ref: np.ndarray, dtype: str) -> float:
    """Error of a dtype-rounded output against the fp64 oracle, net of the
    final rounding to dtype: max(|gpu - ref| - ulp(ref)/2)."""
    return float(np.max(np.abs(gpu_out - ref) - 0.5 * ulp(ref, dtype)))


def check_literal_bar(gpu_out: np.ndarray, ref: np.ndarray, dtype: str, bar: float, what: str) -> float:
    """The raw max-abs error against the fp64 oracle, logged beside the bar.
    fp16 outputs are held to the bar itself (half an fp16 ulp is below 5e-4
    for |o| < 2); bf16 outputs only to the error net of their own final
    rounding (output_error), since half a bf16 ulp is 3.9e-3 at |o| >= 1."""
    raw = float(np.max(np.abs(gpu_out - ref)))
    log(f"[{what}] raw max-abs {raw:.3g} (|o| max {float(np.max(np.abs(ref))):.3g}), bar {bar:g}, {dtype}")
    if dtype == "f16":
        assert raw <= bar, f"{what}: raw max-abs error {raw:.3g} > {bar:g}"
    return raw


# ---------------------------------------------------------------------------
# torch plumbing (GPU tests only)
# ---------------------------------------------------------------------------

def to_dev(a: np.ndarray, dtype: str, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16))
    return t.to(device).view(torch.float16 if dtype == "f16" else torch.bfloat16)


def from_dev(t) -> np.ndarray:
    import torch
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def torch_dtype(dtype: str):
    import torch
    return torch.float16 if dtype == "f16" else torch.bfloat16


# ---------------------------------------------------------------------------
# cache plumbing (GPU tests only)
# ---------------------------------------------------------------------------

def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def new_cache(w: Workload, mbps=None, num_pages=0, kv_bits=0):
    from bsattn import BlockSparseKVCache
    mbps = mbps or (max(w.lens) + w.Tb - 1) // w.Tb + 2
    return BlockSparseKVCache(max_seqs=w.B, num_q_heads=w.Hq, num_kv_heads=w.Hkv, head_dim=w.D,
                              block_size=w.Tb, dtype=torch_dtype(w.dtype), top_k=w.top_k,
                              sink_blocks=w.ns, recent_blocks=w.nr, max_blocks_per_seq=mbps,
                              num_pages=num_pages, kv_bits=kv_bits, device=0)


def fill(cache, w: Workload, device, chunk=None, seed=7):
    """Append every sequence's tokens; with `chunk`, round-robin in random-size
    chunks so the sequences' pages interleave in the pool."""
    if chunk is None:
        for b in range(w.B):
            if w.lens[b]:
                cache.append(to_dev(w.keys[b][None], w.dtype, device),
                             to_dev(w.values[b][None], w.dtype, device), seq_ids=[b])
        return
    rng = np.random.default_rng(seed)
    pos = [0] * w.B
    while any(pos[b] < w.lens[b] for b in range(w.B)):
        for b in rng.permutation(w.B):
            if pos[b] >= w.lens[b]:
                continue
            n = int(min(w.lens[b] - pos[b], rng.integers(1, chunk + 1)))
            k = np.ascontiguousarray(w.keys[b][:, pos[b]:pos[b] + n][None])
            v = np.ascontiguousarray(w.values[b][:, pos[b]:pos[b] + n][None])
            cache.append(to_dev(k, w.dtype, device), to_dev(v, w.dtype, device), seq_ids=[int(b)])
            pos[b] += n
