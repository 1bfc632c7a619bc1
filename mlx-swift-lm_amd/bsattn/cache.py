"""BlockSparseKVCache: the host-side mirror of the reference's KVCache
protocol (Libraries/MLXLMCommon/KVCache.swift:38-77) for the block-sparse
cache, over the C ABI of libbsattn.so.

Member names follow the Swift protocol (offset, maxSize, update, state,
metaState, isTrimmable, trim, makeMask, copy) plus the additive
selector-index API (blockSize, topK, sinkBlocks, recentBlocks,
selectBlocks).  Misuse raises (the Swift code traps with fatalError /
precondition, e.g. KVCache.swift:386-388); library failures raise
BsattnError carrying the C status code.

torch tensors are used only as device memory and streams; every
computation runs in the HIP kernels of libbsattn.so.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence

import torch

from . import _lib
from ._lib import BsattnError, check, i32_array, lib

_DTYPES = {torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr())


class BlockSparseKVCache:
    """One layer's paged KV cache for up to `max_seqs` sequences."""

    def __init__(self, *, max_seqs: int, num_q_heads: int, num_kv_heads: int,
                 head_dim: int = 128, block_size: int = 64,
                 dtype: torch.dtype = torch.bfloat16, kv_bits: int = 0,
                 group_size: int = 64, top_k: int = 32, sink_blocks: int = 1,
                 recent_blocks: int = 1, max_blocks_per_seq: int = 512,
                 num_pages: int = 0, device: int | torch.device = 0,
                 _handle: Optional[ctypes.c_void_p] = None):
        if dtype not in _DTYPES:
            raise TypeError(f"dtype {dtype} unsupported (float16 or bfloat16)")
        self.device = torch.device("cuda", device if isinstance(device, int) else device.index or 0)
        self.dtype = dtype
        self.desc = _lib.Desc(
            max_seqs=max_seqs, num_q_heads=num_q_heads, num_kv_heads=num_kv_heads,
            head_dim=head_dim, block_size=block_size, dtype=_DTYPES[dtype], kv_bits=kv_bits,
            group_size=group_size, top_k=top_k, sink_blocks=sink_blocks,
            recent_blocks=recent_blocks, max_blocks_per_seq=max_blocks_per_seq,
            num_pages=num_pages, device=self.device.index)
        if _handle is None:
            h = ctypes.c_void_p()
            check(lib().bsattn_cache_create(ctypes.byref(self.desc), ctypes.byref(h)))
            self._h = h
        else:
            self._h = _handle
        info = _lib.Info()
        check(lib().bsattn_cache_info(self._h, ctypes.byref(info)))
        self.nselMax = info.nsel_max
        self.numSplits = info.num_splits
        self.poolBytes = info.pool_bytes

    # -- lifetime ----------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().bsattn_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- geometry ------------------------------------------------------------
    @property
    def blockSize(self) -> int:
        return self.desc.block_size

    @property
    def topK(self) -> int:
        return self.desc.top_k

    @property
    def sinkBlocks(self) -> int:
        return self.desc.sink_blocks

    @property
    def recentBlocks(self) -> int:
        return self.desc.recent_blocks

    @property
    def bits(self) -> int:
        return self.desc.kv_bits

    @property
    def groupSize(self) -> int:
        return self.desc.group_size

    @property
    def maxSize(self):
        return None

    @property
    def freePages(self) -> int:
        info = _lib.Info()
        check(lib().bsattn_cache_info(self._h, ctypes.byref(info)))
        return int(info.free_pages)

    def shuffleFreePages(self, seed: int) -> None:
        """Permutes the free pages (seeded): later appends take pages in a
        shuffled physical order.  Results do not depend on it."""
        check(lib().bsattn_shuffle_free_pages(self._h, seed))

    def seqPages(self, seq: int) -> List[int]:
        """Physical page ids of sequence `seq` in logical order."""
        n = ctypes.c_int32()
        rc = lib().bsattn_seq_pages(self._h, seq, None, 0, ctypes.byref(n))
        if n.value == 0:
            check(rc)
            return []
        buf = (ctypes.c_int32 * n.value)()
        check(lib().bsattn_seq_pages(self._h, seq, buf, n.value, ctypes.byref(n)))
        return list(buf)

    def seqLen(self, seq: int) -> int:
        out = ctypes.c_int32()
        check(lib().bsattn_seq_len(self._h, seq, ctypes.byref(out)))
        return out.value

    @property
    def offset(self) -> int:
        """Tokens held by sequence 0 (the reference keeps one offset for the
        whole batch, KVCache.swift:40)."""
        return self.seqLen(0)

    # -- KV writes -----------------------------------------------------------
    def _check_kv(self, t: torch.Tensor, name: str) -> None:
        if t.device != self.device or t.dtype != self.dtype or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {self.dtype} tensor on {self.device}")
        if t.dim() != 4 or t.shape[1] != self.desc.num_kv_heads or t.shape[3] != self.desc.head_dim:
            raise ValueError(f"{name} must be [B, {self.desc.num_kv_heads}, L, {self.desc.head_dim}], got {tuple(t.shape)}")

    def append(self, keys: torch.Tensor, values: torch.Tensor,
               seq_ids: Optional[Sequence[int]] = None) -> None:
        """Appends keys/values [B, Hkv, L, D] to sequences seq_ids (default
        0..B-1)."""
        self._check_kv(keys, "keys")
        self._check_kv(values, "values")
        if keys.shape != values.shape:
            raise ValueError("keys and values shapes differ")
        B, _, L, _ = keys.shape
        ids = i32_array(seq_ids)
        check(lib().bsattn_append(self._h, _ptr(keys), _ptr(values), ids, B, L,
                                  _stream(self.device)))

    # -- graph-capturable decode loop ------------------------------------------
    def reserve(self, n_tokens: int, seq_ids: Optional[Sequence[int]] = None) -> None:
        """Takes the pages for n_tokens more tokens of each sequence now, so
        that appendStep needs no host work."""
        ids = list(seq_ids) if seq_ids is not None else list(range(max(self.batchSize(), 1)))
        check(lib().bsattn_reserve(self._h, i32_array(ids), len(ids), n_tokens, _stream(self.device)))

    def appendStep(self, keys: torch.Tensor, values: torch.Tensor,
                   seq_ids: Optional[Sequence[int]] = None) -> None:
        """One token per sequence ([B, Hkv, 1, D]) at the device-side length,
        which it advances: capturable in a CUDA/HIP graph and replayed once
        per step (reserve first).  Until sync(), calls that need exact token
        counts raise; decode runs."""
        self._check_kv(keys, "keys")
        self._check_kv(values, "values")
        if keys.shape != values.shape or keys.shape[2] != 1:
            raise ValueError("keys / values must both be [B, Hkv, 1, D]")
        check(lib().bsattn_append_step(self._h, _ptr(keys), _ptr(values), i32_array(seq_ids), keys.shape[0],
                                       _stream(self.device)))

    def sync(self) -> None:
        """Copies the device-side lengths back to the host view (waits for the stream)."""
        check(lib().bsattn_sync(self._h, _stream(self.device)))

    def update(self, keys: torch.Tensor, values: torch.Tensor):
        """KVCache.update (KVCache.swift:328-371): append, then return all
        cached keys/values [B, Hkv, offset, D].  A quantized cache traps like
        QuantizedKVCache.update (KVCache.swift:891-896): use updateQuantized."""
        if self.bits:
            raise RuntimeError("`update` was called on a quantized BlockSparseKVCache. "
                               "Use `updateQuantized` instead.")
        self.append(keys, values)
        return self.export(list(range(keys.shape[0])))

    # -- quantized caches (QuantizedKVCache, KVCache.swift:728-988) -----------
    def _require_quantized(self) -> None:
        if not self.bits:
            raise RuntimeError("not a quantized cache (bits 0)")

    def quantizedShapes(self, B: int, L: int):
        """Shapes of (weights, scales, biases) in the MLX layout for B
        sequences of L tokens: [B, Hkv, L, D*bits/32] uint32 (stored as
        int32) and [B, Hkv, L, D/groupSize] fp16."""
        d = self.desc
        return ((B, d.num_kv_heads, L, d.head_dim * d.kv_bits // 32),
                (B, d.num_kv_heads, L, d.head_dim // d.group_size))

    def appendQuantized(self, keys, values, seq_ids: Optional[Sequence[int]] = None) -> None:
        """Appends already-quantized tokens: keys / values are (weights,
        scales, biases) tuples in the MLX layout (quantizedShapes)."""
        self._require_quantized()
        (kw, ks, kb), (vw, vs, vb) = keys, values
        B, L = kw.shape[0], kw.shape[2]
        wshape, sshape = self.quantizedShapes(B, L)
        for name, t, shape, dt in (("keys.weights", kw, wshape, torch.int32), ("keys.scales", ks, sshape, torch.float16),
                                   ("keys.biases", kb, sshape, torch.float16), ("values.weights", vw, wshape, torch.int32),
                                   ("values.scales", vs, sshape, torch.float16), ("values.biases", vb, sshape, torch.float16)):
            if tuple(t.shape) != shape or t.dtype != dt or t.device != self.device or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous {dt} tensor {shape} on {self.device}, "
                                 f"got {t.dtype} {tuple(t.shape)}")
        check(lib().bsattn_append_quantized(self._h, _ptr(kw), _ptr(ks), _ptr(kb), _ptr(vw), _ptr(vs),
                                            _ptr(vb), i32_array(seq_ids), B, L, _stream(self.device)))

    def exportQuantized(self, seq_ids: Sequence[int]):
        """((kw, ks, kb), (vw, vs, vb)) of the listed sequences, MLX layout."""
        self._require_quantized()
        B = len(seq_ids)
        T = self.seqLen(seq_ids[0])
        wshape, sshape = self.quantizedShapes(B, T)
        kw, ks, kb, vw, vs, vb = (
            torch.empty(shape, dtype=dt, device=self.device)
            for shape, dt in [(wshape, torch.int32), (sshape, torch.float16), (sshape, torch.float16)] * 2)
        if T > 0:
            check(lib().bsattn_export_quantized(self._h, i32_array(seq_ids), B, _ptr(kw), _ptr(ks), _ptr(kb),
                                                _ptr(vw), _ptr(vs), _ptr(vb), _stream(self.device)))
        return (kw, ks, kb), (vw, vs, vb)

    def updateQuantized(self, keys: torch.Tensor, values: torch.Tensor):
        """QuantizedKVCache.updateQuantized (KVCache.swift:816-889): quantize
        and append fp16 keys / values [B, Hkv, L, D], then return the
        quantized tuples of all cached tokens."""
        self._require_quantized()
        self.append(keys, values)
        return self.exportQuantized(list(range(keys.shape[0])))

    def getQuantizedState(self):
        """QuantizedKVCache.getQuantizedState (KVCache.swift:797-806)."""
        self._require_quantized()
        n = self.batchSize()
        return self.exportQuantized(list(range(n))) if n else None

    def export(self, seq_ids: Sequence[int]):
        B = len(seq_ids)
        T = self.seqLen(seq_ids[0])
        shape = (B, self.desc.num_kv_heads, T, self.desc.head_dim)
        k = torch.empty(shape, dtype=self.dtype, device=self.device)
        v = torch.empty(shape, dtype=self.dtype, device=self.device)
        check(lib().bsattn_export(self._h, i32_array(seq_ids), B, _ptr(k), _ptr(v),
                                  _stream(self.device)))
        return k, v

    def exportSummaries(self, seq: int) -> torch.Tensor:
        n = self.seqLen(seq) // self.blockSize
        out = torch.empty((self.desc.num_kv_heads, n, self.desc.head_dim), dtype=self.dtype,
                          device=self.device)
        if n:
            check(lib().bsattn_export_summaries(self._h, seq, _ptr(out), _stream(self.device)))
        return out

    # -- selector-index API and attention -----------------------------------
    def _check_q(self, q: torch.Tensor, multi: bool = False) -> int:
        if q.device != self.device or q.dtype != self.dtype or not q.is_contiguous():
            raise ValueError(f"queries must be a contiguous {self.dtype} tensor on {self.device}")
        L = "L" if multi else 1
        if q.dim() != 4 or q.shape[1] != self.desc.num_q_heads or (not multi and q.shape[2] != 1) \
                or q.shape[3] != self.desc.head_dim:
            raise ValueError(f"queries must be [B, {self.desc.num_q_heads}, {L}, {self.desc.head_dim}], "
                             f"got {tuple(q.shape)}")
        return q.shape[0]

    def selectBlocks(self, queries: torch.Tensor,
                     seq_ids: Optional[Sequence[int]] = None) -> torch.Tensor:
        """Selected block indices [B, Hkv, nselMax] int32, ascending, -1 padded."""
        B = self._check_q(queries)
        idx = torch.empty((B, self.desc.num_kv_heads, self.nselMax), dtype=torch.int32,
                          device=self.device)
        check(lib().bsattn_select(self._h, _ptr(queries), i32_array(seq_ids), B, _ptr(idx),
                                  _stream(self.device)))
        return idx

    def attend(self, queries: torch.Tensor, idx: torch.Tensor, scale: float,
               seq_ids: Optional[Sequence[int]] = None) -> torch.Tensor:
        B = self._check_q(queries)
        if idx.dtype != torch.int32 or idx.device != self.device or not idx.is_contiguous() \
                or tuple(idx.shape) != (B, self.desc.num_kv_heads, self.nselMax):
            raise ValueError("idx must be a contiguous int32 [B, Hkv, nselMax] tensor on the cache device")
        out = torch.empty_like(queries)
        check(lib().bsattn_attend(self._h, _ptr(queries), i32_array(seq_ids), B, _ptr(idx),
                                  ctypes.c_float(scale), _ptr(out), _stream(self.device)))
        return out

    def decode(self, queries: torch.Tensor, scale: float,
               seq_ids: Optional[Sequence[int]] = None,
               idx_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        B = self._check_q(queries)
        out = torch.empty_like(queries)
        idx_p = None
        if idx_out is not None:
            if idx_out.dtype != torch.int32 or tuple(idx_out.shape) != (B, self.desc.num_kv_heads, self.nselMax):
                raise ValueError("idx_out must be int32 [B, Hkv, nselMax]")
            idx_p = _ptr(idx_out)
        check(lib().bsattn_decode(self._h, _ptr(queries), i32_array(seq_ids), B,
                                  ctypes.c_float(scale), _ptr(out), idx_p, _stream(self.device)))
        return out

    def decodeNoAlloc(self, queries: torch.Tensor, scale: float, out: torch.Tensor,
                      seq_ids: Optional[Sequence[int]] = None,
                      idx_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """decode() through bsattn_decode_noalloc: the same results, with the
        workspaces in the library's fixed per-GPU scratch and nothing
        allocated (the caller brings `out`, [B, Hq, 1, D]); at most 64
        sequences; calls that overlap on one GPU race."""
        B = self._check_q(queries)
        if out.shape != queries.shape or out.dtype != queries.dtype or not out.is_contiguous():
            raise ValueError("out must be a contiguous tensor shaped and typed like queries")
        idx_p = None
        if idx_out is not None:
            if idx_out.dtype != torch.int32 or tuple(idx_out.shape) != (B, self.desc.num_kv_heads, self.nselMax):
                raise ValueError("idx_out must be int32 [B, Hkv, nselMax]")
            idx_p = _ptr(idx_out)
        check(lib().bsattn_decode_noalloc(self._h, _ptr(queries), i32_array(seq_ids), B,
                                          ctypes.c_float(scale), _ptr(out), idx_p, _stream(self.device)))
        return out

    def appendDecode(self, keys: torch.Tensor, values: torch.Tensor, queries: torch.Tensor,
                     scale: float, seq_ids: Optional[Sequence[int]] = None,
                     idx_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One decode step (attentionWithCacheUpdate with L = 1): appends
        keys / values [B, Hkv, 1, D] and decodes queries [B, Hq, 1, D] over
        the caches that now hold them; the same results as append() then
        decode(), in one launch (the append inside the fused decode) or with
        the append and the block scoring in one launch where the cache allows
        it."""
        self._check_kv(keys, "keys")
        self._check_kv(values, "values")
        if keys.shape != values.shape or keys.shape[2] != 1:
            raise ValueError("keys and values must both be [B, Hkv, 1, D]")
        B = self._check_q(queries)
        if keys.shape[0] != B:
            raise ValueError("keys / values and queries disagree on B")
        out = torch.empty_like(queries)
        idx_p = None
        if idx_out is not None:
            if idx_out.dtype != torch.int32 or tuple(idx_out.shape) != (B, self.desc.num_kv_heads, self.nselMax):
                raise ValueError("idx_out must be int32 [B, Hkv, nselMax]")
            idx_p = _ptr(idx_out)
        check(lib().bsattn_append_decode(self._h, _ptr(keys), _ptr(values), _ptr(queries),
                                         i32_array(seq_ids), B, ctypes.c_float(scale), _ptr(out),
                                         idx_p, _stream(self.device)))
        return out

    def decodeMulti(self, queries: torch.Tensor, scale: float,
                    seq_ids: Optional[Sequence[int]] = None,
                    idx_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Decode of L = queries.shape[2] (1..16) query tokens per sequence
        whose keys / values were appended last (speculative verify,
        Evaluate.swift:862-870): query i of a sequence holding T tokens sees
        its first T - L + 1 + i tokens and selects its own blocks there, as L
        single-token decodes would.  queries / result [B, Hq, L, D];
        idx_out [B, L, Hkv, nselMax] int32."""
        B = self._check_q(queries, multi=True)
        L = queries.shape[2]
        out = torch.empty_like(queries)
        idx_p = None
        if idx_out is not None:
            if idx_out.dtype != torch.int32 or not idx_out.is_contiguous() \
                    or tuple(idx_out.shape) != (B, L, self.desc.num_kv_heads, self.nselMax):
                raise ValueError("idx_out must be a contiguous int32 [B, L, Hkv, nselMax] tensor")
            idx_p = _ptr(idx_out)
        check(lib().bsattn_decode_multi(self._h, _ptr(queries), i32_array(seq_ids), B, L,
                                        ctypes.c_float(scale), _ptr(out), idx_p, _stream(self.device)))
        return out

    def prefill(self, queries: torch.Tensor, scale: float,
                seq_ids: Optional[Sequence[int]] = None) -> torch.Tensor:
        """Dense causal attention of the last L = queries.shape[2] tokens of
        each sequence (a prefill chunk appended just before): query i of a
        sequence holding T tokens attends to tokens [0, T - L + i], as the
        reference's attentionWithCacheUpdate does for L > 1 with the causal
        mask.  queries / result [B, Hq, L, D] (fp16 on a quantized cache)."""
        B = self._check_q(queries, multi=True)
        out = torch.empty_like(queries)
        check(lib().bsattn_prefill(self._h, _ptr(queries), i32_array(seq_ids), B, queries.shape[2],
                                   ctypes.c_float(scale), _ptr(out), _stream(self.device)))
        return out

    # -- kernel timing -------------------------------------------------------
    def profile(self, enable: bool = True) -> None:
        """Start (or stop) timing this cache's eager kernel launches; resets sums."""
        check(lib().bsattn_profile_enable(self._h, 1 if enable else 0))

    def profileRead(self, kernel: int):
        """(total milliseconds, launches) of one kernel kind (bsattn KERNEL_*)."""
        ms, n = ctypes.c_double(), ctypes.c_int64()
        check(lib().bsattn_profile_read(self._h, kernel, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    # -- KVCache protocol: state, trim, mask, copy -----------------------------
    @property
    def state(self) -> List[torch.Tensor]:
        """[keys, values] (KVCacheSimple, KVCache.swift:373-384) or, for a
        quantized cache, [kw, ks, kb, vw, vs, vb] (QuantizedKVCache,
        KVCache.swift:906-925)."""
        n = self.batchSize()
        if n == 0:
            return []
        if self.bits:
            (kw, ks, kb), (vw, vs, vb) = self.exportQuantized(list(range(n)))
            return [kw, ks, kb, vw, vs, vb]
        return list(self.export(list(range(n))))

    @state.setter
    def state(self, arrays: List[torch.Tensor]) -> None:
        want = 6 if self.bits else 2
        if len(arrays) != want:
            raise ValueError(f"BlockSparseKVCache state must have exactly {want} arrays")
        self.reset(list(range(self.desc.max_seqs)))
        if arrays[0].shape[2] == 0:
            return
        if self.bits:
            a = [t.contiguous() for t in arrays]
            self.appendQuantized((a[0], a[1], a[2]), (a[3], a[4], a[5]))
        else:
            k, v = arrays
            self.append(k.contiguous(), v.contiguous())

    @property
    def metaState(self) -> List[str]:
        d = self.desc
        return [str(d.block_size), str(d.top_k), str(d.sink_blocks), str(d.recent_blocks),
                str(self.offset), str(d.kv_bits), str(d.group_size)]

    @metaState.setter
    def metaState(self, values: List[str]) -> None:
        if len(values) != 7:
            raise ValueError("BlockSparseKVCache metaState must have exactly 7 values")
        want = [int(x) for x in values]
        d = self.desc
        have = [d.block_size, d.top_k, d.sink_blocks, d.recent_blocks, want[4], d.kv_bits, d.group_size]
        if want != have:
            raise ValueError(f"metaState {values} does not match this cache's geometry")
        if self.offset != want[4]:
            raise ValueError(f"metaState offset {want[4]} != cached tokens {self.offset}")

    def batchSize(self) -> int:
        """Number of leading sequences that hold tokens."""
        n = 0
        while n < self.desc.max_seqs and self.seqLen(n) > 0:
            n += 1
        return n

    @property
    def isTrimmable(self) -> bool:
        return True

    def trim(self, n: int, seq_ids: Optional[Sequence[int]] = None) -> int:
        ids = list(seq_ids) if seq_ids is not None else list(range(max(self.batchSize(), 1)))
        out = (ctypes.c_int32 * len(ids))()
        check(lib().bsattn_trim(self._h, i32_array(ids), len(ids), n, out, _stream(self.device)))
        return int(out[0])

    def reset(self, seq_ids: Sequence[int]) -> None:
        check(lib().bsattn_reset(self._h, i32_array(seq_ids), len(seq_ids), _stream(self.device)))

    def makeMask(self, n: int, windowSize=None, returnArray: bool = False):
        """BaseKVCache.makeMask (KVCache.swift:160-174): decode needs none."""
        if n == 1:
            return "none"
        if returnArray or (windowSize is not None and n > windowSize):
            return "array"
        return "causal"

    def toQuantized(self, groupSize: int = 64, bits: int = 4) -> "BlockSparseKVCache":
        """KVCacheSimple.toQuantized (KVCache.swift:407-427): a new cache of
        the same geometry holding every sequence's tokens as MLX-affine
        `bits`-bit codes with fp16 scales / biases (exported and quantized on
        append, on the device), with the summaries of the dequantized keys.
        Quantized caches hold fp16, so a bf16 cache's tokens are rounded to
        fp16 first."""
        if self.bits:
            raise ValueError("toQuantized: the cache is already quantized")
        d = self.desc
        qc = BlockSparseKVCache(
            max_seqs=d.max_seqs, num_q_heads=d.num_q_heads, num_kv_heads=d.num_kv_heads,
            head_dim=d.head_dim, block_size=d.block_size, dtype=torch.float16, kv_bits=bits,
            group_size=groupSize, top_k=d.top_k, sink_blocks=d.sink_blocks,
            recent_blocks=d.recent_blocks, max_blocks_per_seq=d.max_blocks_per_seq,
            num_pages=d.num_pages, device=self.device.index)
        for s in range(d.max_seqs):
            if self.seqLen(s) == 0:
                continue
            k, v = self.export([s])
            if self.dtype != torch.float16:
                k, v = k.half(), v.half()
            qc.append(k, v, seq_ids=[s])
            del k, v
        return qc

    def copy(self) -> "BlockSparseKVCache":
        h = ctypes.c_void_p()
        check(lib().bsattn_copy(self._h, ctypes.byref(h), _stream(self.device)))
        d = self.desc
        return BlockSparseKVCache(
            max_seqs=d.max_seqs, num_q_heads=d.num_q_heads, num_kv_heads=d.num_kv_heads,
            head_dim=d.head_dim, block_size=d.block_size, dtype=self.dtype, kv_bits=d.kv_bits,
            group_size=d.group_size, top_k=d.top_k, sink_blocks=d.sink_blocks,
            recent_blocks=d.recent_blocks, max_blocks_per_seq=d.max_blocks_per_seq,
            num_pages=d.num_pages, device=self.device.index, _handle=h)


def maybeQuantizeKVCache(cache: list, kvBits: Optional[int], kvGroupSize: int = 64,
                         quantizedKVStart: int = 0) -> None:
    """maybeQuantizeKVCache (KVCache.swift:1637-1660), in place: once
    cache[0] holds more than quantizedKVStart tokens, every 16-bit
    BlockSparseKVCache in the list is replaced by its toQuantized(kvGroupSize,
    kvBits); nothing happens when kvBits is None, the list is empty or
    cache[0] is already quantized."""
    if kvBits is None or not cache:
        return
    first = cache[0]
    if not isinstance(first, BlockSparseKVCache) or first.bits != 0 or first.offset <= quantizedKVStart:
        return
    for i, c in enumerate(cache):
        if isinstance(c, BlockSparseKVCache) and c.bits == 0:
            cache[i] = c.toQuantized(groupSize=kvGroupSize, bits=kvBits)


@dataclass
class GenerateParameters:
    """The cache fields of GenerateParameters (Evaluate.swift:64-73)."""
    maxKVSize: Optional[int] = None
    kvBits: Optional[int] = None
    kvGroupSize: int = 64
    quantizedKVStart: int = 0


def newCache(kvHeads: Sequence[int], parameters: Optional[GenerateParameters] = None, *,
             num_q_heads: int, max_seqs: int, max_tokens: int, dtype: torch.dtype = torch.bfloat16,
             block_size: int = 64, top_k: int = 32, sink_blocks: int = 1, recent_blocks: int = 1,
             device: int | torch.device = 0) -> List["BlockSparseKVCache"]:
    """The block-sparse form of LanguageModel.newCache(parameters:)
    (LanguageModel.swift:215-230): one cache per layer, layer i with
    kvHeads[i] kv heads (the reference's KVCacheSimple ignores the head
    count; a paged cache needs it), for up to max_seqs sequences of
    max_tokens tokens.  As in the reference the caches start 16-bit even when
    parameters.kvBits is set: maybeQuantizeKVCache converts them once
    quantizedKVStart is passed.  A maxKVSize asks for the reference's
    RotatingKVCache (a bounded window), which this cache does not replace."""
    if parameters is not None and parameters.maxKVSize is not None:
        raise ValueError("maxKVSize selects RotatingKVCache (KVCache.swift:445-578), which stays on "
                         "the reference's dense path")
    mbps = -(-max_tokens // block_size)
    return [BlockSparseKVCache(max_seqs=max_seqs, num_q_heads=num_q_heads, num_kv_heads=h,
                               block_size=block_size, dtype=dtype, top_k=top_k,
                               sink_blocks=sink_blocks, recent_blocks=recent_blocks,
                               max_blocks_per_seq=mbps, device=device) for h in kvHeads]


__all__ = ["BlockSparseKVCache", "BsattnError", "GenerateParameters", "maybeQuantizeKVCache",
           "newCache"]
