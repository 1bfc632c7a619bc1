"""Affine-quantized KV caches (int4 / int8, group 64, fp16 scale and bias):
HIP path vs the CPU oracle, through the C ABI.

Bars:
  * quantize-on-append codes / scales / biases and the MLX-layout round trip:
    bit-exact with the oracle's affine codec;
  * block summaries (means of dequantized keys) and selected block indices:
    bit-exact;
  * attention outputs: max-abs error <= 1e-2 against the fp64 oracle over the
    dequantized keys / values, net of the final rounding to fp16.
The codec is mlx's published affine rule (signed scale, the larger-magnitude
extreme as bias, scale = edge / rint(edge / scale)), which the reference reaches
through quantized() (KVCache.swift:416-417, 856-857); the oracle's statement
of it is pinned by hand-derived cases in test_oracle.py.  The MLX-internal
rounding of the reference's quantizedMM / softmax is not available offline
(mlx is not vendored) and is covered by the 1e-2 bar.
"""
from __future__ import annotations

import numpy as np
import pytest

from common import (Workload, check_config_inputs, check_literal_bar, config_args, fill, from_dev, log,
                    make_workload, new_cache, output_error, to_dev)
import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-2
GS = 64


def quantize_all(w: Workload, bits: int):
    """Oracle codec of every (sequence, kv head): lists of (codes, scales, biases)."""
    kq = [[O.quantize(w.keys[b][h], bits, GS) for h in range(w.Hkv)] for b in range(w.B)]
    vq = [[O.quantize(w.values[b][h], bits, GS) for h in range(w.Hkv)] for b in range(w.B)]
    return kq, vq


def oracle_decode_q(w: Workload, bits: int, kq, vq):
    idx = np.full((w.B, w.Hkv, w.nsel_max), -1, np.int32)
    out = np.zeros((w.B, w.Hq, w.D), np.float64)
    for b in range(w.B):
        for h in range(w.Hkv):
            q = w.q[b, h * w.G:(h + 1) * w.G]
            summ = O.summaries_q(*kq[b][h], w.Tb, bits, GS)
            sc = O.score_blocks(q, summ, "f16")
            i, _ = O.select(sc, w.lens[b], w.Tb, w.ns, w.nr, w.top_k)
            idx[b, h] = i
            out[b, h * w.G:(h + 1) * w.G] = O.attend_q(q, kq[b][h], vq[b][h], w.Tb, bits, GS, i, w.scale)
    return idx, out


def _host(t) -> np.ndarray:
    """int32 code words -> uint32; fp16 scales / biases -> uint16 bits."""
    return from_dev(t) if t.dtype.is_floating_point else t.cpu().numpy().view(np.uint32)


def export_seq(cache, b):
    (kw, ks, kb), (vw, vs, vb) = cache.exportQuantized([b])
    return tuple(_host(t)[0] for t in (kw, ks, kb)), tuple(_host(t)[0] for t in (vw, vs, vb))


def check_storage(cache, w: Workload, bits: int, kq, vq):
    for b in range(w.B):
        if w.lens[b] == 0:
            continue
        gk, gv = export_seq(cache, b)
        for name, got, ref in (("keys", gk, kq[b]), ("values", gv, vq[b])):
            for part, g_, r_ in zip(("codes", "scales", "biases"), got, zip(*ref)):
                r_ = np.stack(r_)
                assert np.array_equal(g_, r_), f"seq {b} {name} {part} differ at {np.argwhere(g_ != r_)[:4]}"
        s = from_dev(cache.exportSummaries(b))
        ref = np.stack([O.summaries_q(*kq[b][h], w.Tb, bits, GS) for h in range(w.Hkv)])
        assert np.array_equal(s, ref), f"summaries differ for seq {b}"


def run_and_check_q(cache, w: Workload, device, bits: int, kq, vq):
    import torch
    q = to_dev(w.q[:, :, None, :], "f16", device)
    idx_ref, out_ref = oracle_decode_q(w, bits, kq, vq)
    idx = cache.selectBlocks(q)
    out = cache.attend(q, idx, w.scale)
    out2 = cache.decode(q, w.scale)
    torch.cuda.synchronize()
    idx = idx.cpu().numpy()
    assert np.array_equal(idx, idx_ref), f"selected blocks differ: {np.argwhere(idx != idx_ref)[:5]}"
    a, a2 = from_dev(out).reshape(w.B, w.Hq, w.D), from_dev(out2).reshape(w.B, w.Hq, w.D)
    assert np.array_equal(a, a2), "decode != select + attend"
    got = O.to_f32(a, "f16").astype(np.float64)
    err = output_error(got, out_ref, "f16")
    assert err <= TOL, f"output error {err:.3g} > {TOL}"
    check_literal_bar(got, out_ref, "f16", TOL, f"int{bits} B{w.B} Hq{w.Hq} T{max(w.lens)}")
    return err


def with_constant_rows(w: Workload):
    """Groups that reach the codec's special cases: constant rows (scale
    1e-7 -> fp16 0x8002 / 0x0002, bias = the value), all-zero groups (q0 = 0,
    bias 0), |min| == |max| (the max side wins), repeated extremes."""
    for b in range(w.B):
        T = w.lens[b]
        for h in range(w.Hkv):
            if T > 5:
                w.keys[b][h, 1, :] = 0x3C00          # all 1.0
                w.values[b][h, 2, :64] = 0xBC00      # group of -1.0
                w.keys[b][h, 3, ::7] = 0x4400        # repeated maximum 4.0
                w.keys[b][h, 4, 64:] = 0x0000        # all-zero group
                w.values[b][h, 4, :] = 0x8000        # -0.0 row
                w.keys[b][h, 5, 0] = 0x4200          # 3.0 and -3.0: equal magnitudes
                w.keys[b][h, 5, 1:64] = np.clip(w.keys[b][h, 5, 1:64], 0, 0x3BFF)
                w.keys[b][h, 5, 9] = 0xC200
    return w


@pytest.mark.parametrize("bits,Tb", [(4, 64), (8, 32), (4, 32), (8, 64)])
def test_quantize_on_append_bit_exact(gpu, bits, Tb):
    """fp16 appends in ragged chunks (partly filled code words, interleaved
    pages) quantize exactly as the codec; summaries of dequantized keys."""
    lens = [1, 5, Tb - 1, Tb, Tb + 9, 6 * Tb + 3, 17 * Tb]
    log(f"[q-append] bits={bits} Tb={Tb}")
    w = with_constant_rows(make_workload(3000 + bits + Tb, B=len(lens), Hq=32, Hkv=8, T=max(lens),
                                         Tb=Tb, dtype="f16", top_k=4, lens=lens))
    cache = new_cache(w, kv_bits=bits)
    fill(cache, w, gpu, chunk=Tb + 11)
    kq, vq = quantize_all(w, bits)
    check_storage(cache, w, bits, kq, vq)


@pytest.mark.parametrize("bits", [4, 8])
def test_append_quantized_round_trip(gpu, bits):
    """MLX-layout appends (bsattn_append_quantized) in ragged chunks export
    bit-identically; state round trip through a second cache."""
    import torch
    Tb = 64
    lens = [3, 2 * Tb + 1, 9 * Tb + 30]
    log(f"[q-mlx] bits={bits}")
    w = make_workload(3100 + bits, B=len(lens), Hq=16, Hkv=4, T=max(lens), Tb=Tb, dtype="f16",
                      top_k=3, lens=lens)
    kq, vq = quantize_all(w, bits)
    cache = new_cache(w, kv_bits=bits)
    rng = np.random.default_rng(1)

    def dev(a, floating):
        t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16 if floating else np.int32)).to(gpu)
        return t.view(torch.float16) if floating else t

    pos = [0] * w.B
    while any(pos[b] < lens[b] for b in range(w.B)):
        for b in rng.permutation(w.B):
            if pos[b] >= lens[b]:
                continue
            n = int(min(lens[b] - pos[b], rng.integers(1, 40)))
            sl = slice(pos[b], pos[b] + n)
            kt = tuple(dev(np.stack([kq[b][h][i][sl] for h in range(w.Hkv)])[None], i > 0) for i in range(3))
            vt = tuple(dev(np.stack([vq[b][h][i][sl] for h in range(w.Hkv)])[None], i > 0) for i in range(3))
            cache.appendQuantized(kt, vt, seq_ids=[int(b)])
            pos[b] += n
    check_storage(cache, w, bits, kq, vq)
    # state of a single full-length batch row, restored into a fresh cache
    c1 = new_cache(make_workload(1, B=1, Hq=16, Hkv=4, T=1, Tb=Tb, dtype="f16", top_k=3), mbps=16,
                   kv_bits=bits)
    (kw, ks, kb), (vw, vs, vb) = cache.exportQuantized([2])
    c1.state = [kw, ks, kb, vw, vs, vb]
    assert c1.offset == lens[2]
    (kw2, ks2, kb2), (vw2, vs2, vb2) = c1.exportQuantized([0])
    for a, b_ in ((kw, kw2), (ks, ks2), (kb, kb2), (vw, vw2), (vs, vs2), (vb, vb2)):
        assert torch.equal(a, b_)
    with pytest.raises(RuntimeError):
        c1.update(torch.zeros((1, 4, 1, 128), dtype=torch.float16, device=gpu),
                  torch.zeros((1, 4, 1, 128), dtype=torch.float16, device=gpu))


@pytest.mark.parametrize("bits,Tb,Hq,Hkv", [
    (4, 64, 32, 8), (8, 32, 64, 4), (4, 32, 16, 16), (8, 64, 32, 8), (4, 64, 16, 8), (8, 32, 16, 2),
])
def test_quantized_decode_ragged(gpu, bits, Tb, Hq, Hkv):
    """Selection bit-exact and outputs within 1e-2 over ragged, paged,
    quantize-on-append caches (fused-selection and select + attend paths)."""
    lens = [1, Tb - 1, Tb + 1, 7 * Tb + 5, 40 * Tb + 17, 23 * Tb]
    log(f"[q-decode] bits={bits} Tb={Tb} Hq={Hq} Hkv={Hkv}")
    w = make_workload(3200 + bits + Tb + Hq, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb,
                      dtype="f16", top_k=6, ns=2, nr=2, lens=lens, salient_frac=0.01)
    cache = new_cache(w, kv_bits=bits)
    fill(cache, w, gpu, chunk=2 * Tb + 3)
    kq, vq = quantize_all(w, bits)
    err = run_and_check_q(cache, w, gpu, bits, kq, vq)
    log(f"[q-decode] bits={bits} Tb={Tb} err={err:.3g}")


@pytest.mark.parametrize("bits,Hq,Hkv,qscale", [
    (4, 32, 8, 1e-4), (4, 32, 8, 300.0), (4, 64, 4, 1e-4), (8, 32, 8, 1e-4), (8, 64, 4, 300.0),
])
def test_quantized_decode_query_magnitudes(gpu, bits, Hq, Hkv, qscale):
    """Queries scaled by 1e-4 (the int4 kernel's query operand, scaled by 1/16
    at half of the dims, then falls below fp16's normal range) and by 300 (a
    softmax that one token dominates): selection bit-exact, outputs within
    1e-2 of the oracle over the same fp16 queries."""
    Tb = 64
    lens = [30 * Tb + 5, 12 * Tb, 45 * Tb + 63]
    log(f"[q-mag] bits={bits} Hq={Hq} Hkv={Hkv} q x {qscale:g}")
    w = make_workload(3250 + bits + Hq, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype="f16",
                      top_k=8, ns=1, nr=1, lens=lens, salient_frac=0.01)
    w.q = (O.to_f32(w.q, "f16").astype(np.float64) * qscale).astype(np.float16).view(np.uint16)
    cache = new_cache(w, kv_bits=bits)
    fill(cache, w, gpu)
    kq, vq = quantize_all(w, bits)
    err = run_and_check_q(cache, w, gpu, bits, kq, vq)
    log(f"[q-mag] err={err:.3g}")


def test_quantized_many_candidates(gpu):
    """int8, 32-token blocks, GQA 16, 1500+ candidate blocks (radix
    selection path), top-128 + sink + 4 recent."""
    log("[q-many] generating")
    lens = [50000, 49000]
    w = make_workload(3300, B=2, Hq=64, Hkv=4, T=max(lens), Tb=32, dtype="f16", top_k=128, ns=1,
                      nr=4, lens=lens, salient_frac=0.01)
    cache = new_cache(w, kv_bits=8)
    fill(cache, w, gpu)
    kq, vq = quantize_all(w, 8)
    err = run_and_check_q(cache, w, gpu, 8, kq, vq)
    log(f"[q-many] err={err:.3g}")


def test_config3_int4_full(gpu):
    """B=4, Hq=32, Hkv=8, 131072 tokens in 64-token blocks, int4 group 64,
    top-64 + sink + recent: every head against the oracle."""
    log("[config3] generating")
    w = make_workload(**config_args("C3"))
    check_config_inputs(w, "C3")
    cache = new_cache(w, kv_bits=4)
    fill(cache, w, gpu)
    log("[config3] oracle")
    kq, vq = quantize_all(w, 4)
    err = run_and_check_q(cache, w, gpu, 4, kq, vq)
    log(f"[config3] err={err:.3g}")


def test_config5_int8_wide_group_full(gpu):
    """B=8, Hq=64, Hkv=4 (GQA 16), 262144 tokens in 32-token blocks (8192
    blocks per head), int8 group 64, top-128 + sink + 4 recent: every head
    against the oracle (the MFMA-band scoring and the workgroup selection at
    full size)."""
    log("[config5] generating")
    w = make_workload(**config_args("C5"))
    check_config_inputs(w, "C5")
    cache = new_cache(w, kv_bits=8)
    fill(cache, w, gpu)
    log("[config5] oracle")
    kq, vq = quantize_all(w, 8)
    err = run_and_check_q(cache, w, gpu, 8, kq, vq)
    log(f"[config5] err={err:.3g}")


def test_quantized_decode_loop_with_appends(gpu):
    """Decode steps that append one token per sequence (crossing block
    boundaries, so summaries refresh) on an int4 cache."""
    import torch
    Tb, steps = 32, 40
    lens0 = [Tb * 5 - 3, Tb * 9 - 20, 2]
    log("[q-loop]")
    w = make_workload(3500, B=3, Hq=32, Hkv=8, T=max(lens0) + steps, Tb=Tb, dtype="f16", top_k=3,
                      lens=[l + steps for l in lens0])
    full_k, full_v, full_lens = w.keys, w.values, list(w.lens)
    cache = new_cache(w, kv_bits=4)
    for b in range(w.B):
        cache.append(to_dev(full_k[b][:, :lens0[b]][None], "f16", gpu),
                     to_dev(full_v[b][:, :lens0[b]][None], "f16", gpu), seq_ids=[b])
    for step in range(steps):
        k = np.stack([full_k[b][:, lens0[b] + step] for b in range(w.B)])[:, :, None]
        v = np.stack([full_v[b][:, lens0[b] + step] for b in range(w.B)])[:, :, None]
        cache.append(to_dev(k, "f16", gpu), to_dev(v, "f16", gpu))
        if step % 13 == 12 or step == steps - 1:
            w.lens = [l + step + 1 for l in lens0]
            w.keys = [full_k[b][:, :w.lens[b]] for b in range(w.B)]
            w.values = [full_v[b][:, :w.lens[b]] for b in range(w.B)]
            kq, vq = quantize_all(w, 4)
            check_storage(cache, w, 4, kq, vq)
            run_and_check_q(cache, w, gpu, 4, kq, vq)
    torch.cuda.synchronize()
    assert [cache.seqLen(b) for b in range(w.B)] == full_lens


@pytest.mark.parametrize("bits,Tb,dtype", [(4, 64, "f16"), (8, 32, "f16"), (4, 64, "bf16")])
def test_to_quantized(gpu, bits, Tb, dtype):
    """toQuantized (KVCacheSimple.toQuantized): a 16-bit cache (ragged
    lengths, interleaved pages, one empty sequence) becomes a quantized cache
    holding the same tokens: codes / scales / biases bit-exact against the
    codec on the fp16 tokens (bf16 tokens rounded to fp16 first), lengths
    kept, selection and outputs as the oracle's over the quantized tokens."""
    import torch
    lens = [Tb * 40 + 3, Tb * 9, Tb * 23 + 17, 0]
    log(f"[to-quantized] bits={bits} Tb={Tb} {dtype}")
    w = make_workload(3600 + bits + Tb, B=len(lens), Hq=32, Hkv=8, T=max(lens), Tb=Tb, dtype=dtype,
                      top_k=5, ns=1, nr=2, lens=lens, salient_frac=0.01)
    src = new_cache(w)
    fill(src, w, gpu, chunk=3 * Tb + 1)
    qc = src.toQuantized(groupSize=64, bits=bits)
    assert qc.bits == bits and qc.dtype == torch.float16
    assert [qc.seqLen(b) for b in range(w.B)] == lens
    # the fp16 tokens the quantized cache holds
    w16 = Workload(w.seed, w.B, w.Hq, w.Hkv, w.D, Tb, "f16", lens, w.top_k, w.ns, w.nr)
    w16.q = w.q if dtype == "f16" else O.from_f32(O.to_f32(w.q, dtype), "f16")
    conv = (lambda a: a) if dtype == "f16" else (lambda a: O.from_f32(O.to_f32(a, dtype), "f16"))
    w16.keys = [conv(k) for k in w.keys]
    w16.values = [conv(v) for v in w.values]
    kq, vq = quantize_all(w16, bits)
    check_storage(qc, w16, bits, kq, vq)
    wd = Workload(w.seed, 3, w.Hq, w.Hkv, w.D, Tb, "f16", lens[:3], w.top_k, w.ns, w.nr)
    wd.q, wd.keys, wd.values = w16.q[:3], w16.keys[:3], w16.values[:3]
    err = run_and_check_q(qc, wd, gpu, bits, kq[:3], vq[:3])
    log(f"[to-quantized] err={err:.3g}")


def test_maybe_quantize_kv_cache(gpu):
    """maybeQuantizeKVCache: nothing for kvBits None or offset <= start;
    past the start every 16-bit cache of the list is replaced by its
    quantized form (same tokens); an already quantized list is left alone."""
    from bsattn import maybeQuantizeKVCache
    lens = [300, 200]
    w = make_workload(3700, B=2, Hq=32, Hkv=8, T=max(lens), Tb=64, dtype="f16", top_k=2, lens=lens)
    caches = [new_cache(w) for _ in range(3)]
    for c in caches:
        fill(c, w, gpu)
    before = list(caches)
    maybeQuantizeKVCache(caches, None)
    maybeQuantizeKVCache(caches, 4, quantizedKVStart=300)      # offset 300 is not > 300
    assert all(a is b for a, b in zip(caches, before))
    maybeQuantizeKVCache(caches, 4, kvGroupSize=64, quantizedKVStart=299)
    assert all(c.bits == 4 and c is not b for c, b in zip(caches, before))
    assert [caches[0].seqLen(b) for b in range(2)] == lens
    again = list(caches)
    maybeQuantizeKVCache(caches, 8, quantizedKVStart=0)
    assert all(a is b for a, b in zip(caches, again))
    kq, vq = quantize_all(w, 4)
    check_storage(caches[2], w, 4, kq, vq)
