// bsattn_prefill.hip -- gfx950 (CDNA4) dense causal attention of a prefill
// chunk over a 16-bit block-sparse cache (the quantized caches' version is
// in bsattn_quant.hip).
//
// Built with -fno-honor-nans -mno-amdgpu-ieee: the scores are MFMA results
// (never signalling NaNs), so max trees compile to v_max3_f32 without the
// operand quieting IEEE mode asks for.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

// (the shared header's NaN-aware helpers are not used here)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wnan-infinity-disabled"
#include "bsattn_device.h"
#pragma clang diagnostic pop

namespace bsattn {

// ---------------------------------------------------------------------------
// dense causal attention for the last L tokens of each sequence (a prefill
// chunk whose keys / values were appended): query token i of a sequence
// holding T tokens sits at position T - L + i and attends to tokens
// [0, T - L + i] (the causal mask BaseKVCache.makeMask gives for n > 1).
// A wave owns R column sets of 16 MFMA columns, each column a (query token,
// q head) pair (16 / G tokens x the G heads of kv head h); the workgroup's
// W waves take consecutive tokens of one (sequence, kv head) and stream its
// K / V blocks from block 0 to the last one any of them sees, with an online
// softmax per column:
//   S^T[token][col] = K[token] . Q[col]        (A = K rows, B = Q^T)
//   O^T[dim][col]  += V^T[dim] . P^T[col]      (A = V^T, B = P^T)
// An MFMA's A and B operands take the same lane layout, so the
// fragment-major K / V tiles and the P registers of the decode kernel serve
// both products unchanged, and each lane holds the running max, sum and
// O^T entries of its own column.
// The K / V blocks are streamed in units of 32 tokens (a block of 32, or
// half of a block of 64: 8 K and 8 V fragments of 1 KiB), each loaded from
// memory once per workgroup into one of two 16 KiB LDS buffers (every wave
// fetches 16 / W fragments): the loads of unit u + 1 are in flight while the
// workgroup computes unit u from the other buffer.  A wave reads each
// fragment from LDS once and applies it to all R column sets.
// Affine-quantized caches (KB = 4 / 8 bits, fp16 q / out): a unit's codes
// and scales / biases are loaded raw into LDS (4.5 / 8.5 KiB) and
// dequantized once per workgroup into the 16-bit fragment layout above, as
// fp16 values fl16(scale * code + bias) (one packed fused multiply-add per
// pair, so each is the correctly rounded dequantized value); the rest runs
// as for an fp16 cache.  The raw loads run two units ahead: in step u the
// workgroup loads unit u + 2, dequantizes unit u + 1 and computes unit u.
// The workgroups of one (sequence, kv head) read the same blocks, so the
// flat workgroup index is remapped to give them consecutive indices within
// one XCD (workgroups are dealt to the 8 XCDs in turn): they then share that
// XCD's L2 instead of fetching every block into all eight.
// grid (ceil(L / (W * R * 16 / G)), Hkv, n)
// ---------------------------------------------------------------------------
template <int DT, int TB, int G, int R, int W, int OCC, int KB>
__global__ __launch_bounds__(64 * W, OCC) void k_prefill(Geometry geo, SeqBatch sb, int L,
                                                   const uint16_t* __restrict__ q, float sl2,
                                                   uint16_t* __restrict__ out) {
  constexpr int QPS = 16 / G;   // query tokens per column set
  constexpr int KS2 = TB / 32;  // 32-token units (PV k-steps) of a block
  constexpr int FPW = 16 / W;   // fragments of a unit each wave fetches
  static_assert(16 % W == 0 && (W == 1 || 8 % W == 0), "fragments split evenly over the waves");
  static_assert(KB == 0 || (DT == 0 && W == 4), "quantized caches: fp16, four waves");
  // raw quantized unit: K code fragments (2 tiles x KB / 4), V code fragments
  // (8 dim tiles / (16 / KB) per fragment), then 32 scale / bias entries
  constexpr int RKF = KB / 2, RVF = KB / 2, RAWF = RKF + RVF;
  // the running maximum a column's weights are taken against is raised only
  // when a block's maximum exceeds it by more than 2^kLazy: the weights then
  // stay below 2^kLazy, and the rescaling of O^T (a pass over its registers)
  // is skipped for most blocks; O^T / l is unchanged by the choice
  constexpr float kLazy = 8.f;
  __shared__ __align__(16) u32x4 s_kv0[16 * 64], s_kv1[16 * 64];
  __shared__ __align__(16) u32x4 s_raw0[KB ? RAWF * 64 + 32 : 1], s_raw1[KB ? RAWF * 64 + 32 : 1];
  // bf16 caches: the unit's V as fp16 (exact for |v| < 65520 down to the
  // fp16 normal range) for an fp16 PV product without the hi / lo split of
  // P; s_big[u & 1] flags a unit holding a value fp16 cannot take (its PV
  // then runs in bf16 with P as hi + lo)
  constexpr bool CV = KB == 0 && DT == 1;
  __shared__ __align__(16) u32x4 s_v16[CV ? 8 * 64 : 1];
  __shared__ int s_big[2];
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  // XCD-grouped workgroup order (a bijection on [0, total))
  const int gx = gridDim.x, gy = gridDim.y;
  const int total = gx * gy * gridDim.z;
  const int flat = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const int even = total & ~7;
  const int lid = flat < even ? (flat & 7) * (even >> 3) + (flat >> 3) : flat;
  const int bx = lid % gx, h = (lid / gx) % gy, bi = lid / (gx * gy);
  const int twg = bx * W * R * QPS;     // the workgroup's first query token
  const int t0 = twg + wave * R * QPS;  // this wave's
  const bool active = t0 < L;
  const int seq = sb.ids[bi];
  const int T = uniform(geo.meta[seq]);
  const int head = h * G + n % G;
  // scores are taken as (K . Q') * |sl2| with Q' = Q * sign(sl2): the sign
  // flip is exact, and a positive factor lets the block maximum be found on
  // the raw products
  const uint32_t qflip = sl2 < 0.f ? 0x80008000u : 0u;
  const float sc = fabsf(sl2);
  // column n of set r: query token t0 + r * QPS + n / G, at position pos[r];
  // a padding column (no query token) has Q = 0, sees every token and is not
  // stored
  int pos[R];
  u32x4 qf[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int tq = t0 + r * QPS + n / G;
    pos[r] = tq < L ? T - L + tq : T;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[r][s] = u32x4{0u, 0u, 0u, 0u};
    if (tq < L) {
      const uint16_t* src = q + q_row(sb, bi, head) + (size_t)tq * kHeadDim + 8 * g;
#pragma unroll
      for (int s = 0; s < 4; ++s) qf[r][s] = *(const u32x4*)(src + 32 * s) ^ qflip;
    }
  }
  const int last = T - L + min(L - 1, twg + W * R * QPS - 1);  // the workgroup's last position
  const int nunit = last / 32 + 1;
  // units below nfull are whole and visible to every column of the wave
  const int nfull = (T - L + t0 + 1) / 32;
  const int32_t* bt = block_table(geo, seq);
  // this wave's fragments of unit u go straight from memory into LDS
  // (global_load_lds: lane i's 16 bytes land at dst + 16 i).  Buffer slot
  // f = wave + i * W: K fragment 8 hh + f of the block for f < 8 (QK tiles
  // 2 hh, 2 hh + 1), V fragment (f - 8) * KS2 + hh (dims 16 (f - 8) ..,
  // PV k-step hh) for f >= 8, where hh = u % KS2
  auto fetch = [&](int u, u32x4* buf) __attribute__((always_inline)) {
    const int page = uniform(bt[u / KS2]), hh = u % KS2;
    const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
    const u32x4* Kf = (const u32x4*)(slab + geo.k_off) + (8 * hh + wave) * 64 + lane;
    const u32x4* Vf = (const u32x4*)(slab + geo.v_off) + (wave * KS2 + hh) * 64 + lane;
#pragma unroll
    for (int i = 0; i < FPW; ++i)
      __builtin_amdgcn_global_load_lds(
          (const void*)(i < 8 / W ? Kf + i * W * 64 : Vf + (i - 8 / W) * W * KS2 * 64),
          (__attribute__((address_space(3))) void*)(buf + (wave + i * W) * 64), 16, 0, 0);
  };
  // raw quantized unit u: slots f = wave + i * W; K fragment hh * RKF + f of
  // the block for f < RKF (QK tiles 2 hh, 2 hh + 1), V fragment
  // (f - RKF) * KS2 + hh for f >= RKF; the unit's scale / bias entries for
  // tokens 8 g' + e (g' = 0..3, e = 0..7) go to entries 8 g' + e, loaded by
  // lanes 0..31 of the last wave
  auto fetch_raw = [&](int u, u32x4* buf) __attribute__((always_inline)) {
    const int page = uniform(bt[u / KS2]), hh = u % KS2;
    const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
    const u32x4* Kf = (const u32x4*)(slab + geo.k_off) + lane;
    const u32x4* Vf = (const u32x4*)(slab + geo.v_off) + lane;
#pragma unroll
    for (int i = 0; i < RAWF / W; ++i) {
      const int f = wave + i * W;
      __builtin_amdgcn_global_load_lds(
          (const void*)(f < RKF ? Kf + (hh * RKF + f) * 64 : Vf + ((f - RKF) * KS2 + hh) * 64),
          (__attribute__((address_space(3))) void*)(buf + f * 64), 16, 0, 0);
    }
    if (wave == W - 1 && lane < 32) {
      const u32x4* Sf = (const u32x4*)(slab + geo.sb_off) + (lane >> 3) * (TB / 4) + 8 * hh + (lane & 7);
      __builtin_amdgcn_global_load_lds((const void*)Sf,
                                       (__attribute__((address_space(3))) void*)(buf + RAWF * 64), 16, 0, 0);
    }
  };
  // dequantize a raw unit into the fp16 fragment layout: wave 0 / 1 writes
  // the 4 K fragments of QK tile 0 / 1 (one token per lane), wave 2 / 3 the
  // V fragments of dim tiles 0..3 / 4..7 (8 tokens per lane)
  auto dequant = [&](const u32x4* raw, u32x4* kv) __attribute__((always_inline)) {
    using QC = QCode<KB>;
    const u32x4* ent = raw + RAWF * 64;  // scale / bias entry of token x of the unit
    // f16 pairs (s * c + b): c from the f16 values OFF + c / INV_UNIT exactly
    auto deq = [&](u32x4 hv, const uint32_t* sp, const uint32_t* bp) __attribute__((always_inline)) {
      const f16x2 unit2 = {(_Float16)QC::INV_UNIT, (_Float16)QC::INV_UNIT};
      const f16x2 off2 = {(_Float16)(-QC::OFF * QC::INV_UNIT), (_Float16)(-QC::OFF * QC::INV_UNIT)};
      u32x4 r;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        // (a vector element is copied out first: __builtin_bit_cast of
        // hv[k] itself reads element 0 with this compiler)
        const uint32_t w = hv[k];
        const f16x2 c = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, w), unit2, off2);
        r[k] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, sp[k]), c,
                                                                       __builtin_bit_cast(f16x2, bp[k])));
      }
      return r;
    };
    if (wave < 2) {
      // row m of QK tile t is token 8 (m / 4) + 4 t + m % 4 of the unit (the
      // tile's MFMA output rows then land on tok_of(g, 4 t + i))
      const int t = wave, m = lane & 15;
      const u32x4 e = ent[8 * (m >> 2) + 4 * t + (m & 3)];
      // (k scale, k bias) of dim group 0 / 1 in both halves
      const uint32_t s0 = __builtin_amdgcn_perm(e[0], e[0], 0x01000100u), s1 = __builtin_amdgcn_perm(e[0], e[0], 0x03020302u);
      const uint32_t b0 = __builtin_amdgcn_perm(e[1], e[1], 0x01000100u), b1 = __builtin_amdgcn_perm(e[1], e[1], 0x03020302u);
      u32x4 rw[2];
#pragma unroll
      for (int f = 0; f < RKF / 2; ++f) rw[f] = raw[(t * (RKF / 2) + f) * 64 + lane];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        u32x4 hv;
        if constexpr (KB == 4) hv = nib_to_f16(rw[0][s]);
        else hv = byte_to_f16(rw[s >> 1][2 * (s & 1)], rw[s >> 1][2 * (s & 1) + 1]);
        const uint32_t sp[4] = {s < 2 ? s0 : s1, s < 2 ? s0 : s1, s < 2 ? s0 : s1, s < 2 ? s0 : s1};
        const uint32_t bp[4] = {s < 2 ? b0 : b1, s < 2 ? b0 : b1, s < 2 ? b0 : b1, s < 2 ? b0 : b1};
        kv[(t * 4 + s) * 64 + lane] = deq(hv, sp, bp);
      }
    } else {
      const int half = wave - 2;  // dim group of dim tiles 4 half .. 4 half + 3
      // (v scale, v bias) of tokens 8 g + 2 k, 8 g + 2 k + 1 as f16 pairs
      uint32_t sp[4], bp[4];
      const uint32_t sel = half ? 0x07060302u : 0x05040100u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const u32x4 e0 = ent[8 * g + 2 * k], e1 = ent[8 * g + 2 * k + 1];
        sp[k] = __builtin_amdgcn_perm(e1[2], e0[2], sel);
        bp[k] = __builtin_amdgcn_perm(e1[3], e0[3], sel);
      }
      u32x4 rw[2];
#pragma unroll
      for (int f = 0; f < RVF / 2; ++f) rw[f] = raw[(RKF + half * (RVF / 2) + f) * 64 + lane];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        u32x4 hv;
        if constexpr (KB == 4) hv = nib_to_f16(rw[0][d]);
        else hv = byte_to_f16(rw[d >> 1][2 * (d & 1)], rw[d >> 1][2 * (d & 1) + 1]);
        kv[(8 + 4 * half + d) * 64 + lane] = deq(hv, sp, bp);
      }
    }
  };
  float m[R], l[R], thr[R];
  f32x4 o[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    thr[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[r][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // unit u from LDS (tokens 32 u .. 32 u + 31 of the sequence); MASK: the
  // causal limit and the sequence end apply.  PDT: type of the PV product
  // (P and V); when it differs from DT, V comes from the fp16 copy vkv.
  auto unit = [&](int u, const u32x4* kv, const u32x4* vkv, auto mask_tag, auto pdt_tag)
      __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_tag)::value;
    constexpr int PDT = decltype(pdt_tag)::value;
    f32x4 acc[R][2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      u32x4 kf[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[s] = kv[(t * 4 + s) * 64];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[r][t] = mfma16x16x32<DT>(kf[s], qf[r][s], acc[r][t]);
      }
    }
    // P^T operand: lane (column n, group g) -> tokens 32 u + tok_of(g,
    // 2 jj (+1)); bf16 P is split into hi + lo
    u32x4 pf[R], pl[R];
    (void)pl;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float x[8];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * t + i] = acc[r][t][i];
      if constexpr (MASK) {
        // causal: token 32 u + tok_of(g, e) <= pos (which is below T)
        const int lim = pos[r] - 32 * u;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = tok_of(g, e) <= lim ? x[e] : -INFINITY;
      }
      // the column's maximum is needed only when some lane's scores pass
      // the raising threshold thr = (m + kLazy) / sc
      const float lm = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
      if (__builtin_amdgcn_ballot_w64(lm > thr[r])) {
        // every column sees token 0 in block 0, so bm is finite there
        const float bm = max_over_groups(lm) * sc;
        const bool raise = bm > m[r] + kLazy;
        const float mn = raise ? bm : m[r];
        const float alpha = __builtin_amdgcn_exp2f(m[r] - mn);  // 0 from -inf
        l[r] *= alpha;
        m[r] = mn;
        thr[r] = (mn + kLazy) / sc;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[r][dt][i] *= alpha;
      }
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = __builtin_amdgcn_exp2f(fmaf(x[e], sc, -m[r]));
        ps += x[e];
      }
      l[r] += ps;  // this lane's tokens; the column's groups are summed at the end
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float p0 = x[2 * jj], p1 = x[2 * jj + 1];
        const uint32_t hi = cvt_pk<PDT>(p0, p1);
        pf[r][jj] = hi;
        if constexpr (PDT == 1)
          pl[r][jj] = cvt_pk<1>(p0 - __uint_as_float(hi << 16), p1 - __uint_as_float(hi & 0xFFFF0000u));
      }
    }
    const int valid = min(32, T - 32 * u);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      u32x4 vf = PDT == DT ? kv[(8 + dt) * 64] : vkv[dt * 64];
      if constexpr (MASK) {
        // V of tokens past the sequence end (stale page data) is zeroed
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int tk = 8 * g + 2 * jj;
          vf[jj] &= (tk < valid ? 0x0000FFFFu : 0u) | (tk + 1 < valid ? 0xFFFF0000u : 0u);
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        o[r][dt] = mfma16x16x32<PDT>(vf, pf[r], o[r][dt]);
        if constexpr (PDT == 1) o[r][dt] = mfma16x16x32<PDT>(vf, pl[r], o[r][dt]);
      }
    }
  };
  // 16-bit: unit u is read from buffer u & 1 while unit u + 1 is loaded
  // into the other one, which held unit u - 1: every wave finished that
  // before the barrier ending the previous step.  Quantized: raw buffer
  // u & 1 (unit u, dequantized in the previous step) takes the loads of unit
  // u + 2 while raw buffer (u + 1) & 1 is dequantized into fp16 buffer
  // (u + 1) & 1 (which held unit u - 1).  Every wave takes nunit steps (one
  // barrier each); a wave past the last query token only loads (and
  // dequantizes).
  auto step = [&](int u, const u32x4* cur, u32x4* nxt, u32x4* raw_ld, const u32x4* raw_dq, auto act,
                  auto mask_tag) __attribute__((always_inline)) {
    if constexpr (KB == 0) {
      if (u + 1 < nunit) fetch(u + 1, nxt);
    } else {
      if (u + 2 < nunit) fetch_raw(u + 2, raw_ld);
      if (u + 1 < nunit) dequant(raw_dq, nxt);
    }
    if constexpr (CV) {
      // V of unit u to fp16 (two fragment lanes per thread); a bf16 value of
      // magnitude >= 65536 (or inf / NaN) flags the unit
      bool big = false;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int it = threadIdx.x + 256 * i;
        const u32x4 w = cur[(8 + (it >> 6)) * 64 + (it & 63)];
        u32x4 h;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t x = w[k];
          big |= (x & 0x7FFFu) >= 0x4780u || ((x >> 16) & 0x7FFFu) >= 0x4780u;
          h[k] = cvt_pk<0>(__uint_as_float(x << 16), __uint_as_float(x & 0xFFFF0000u));
        }
        s_v16[it] = h;
      }
      if (__builtin_amdgcn_ballot_w64(big) != 0 && lane == 0) s_big[u & 1] = 1;
      if (threadIdx.x == 0) s_big[(u + 1) & 1] = 0;  // last read in step u - 1
      __syncthreads();
      if constexpr (decltype(act)::value) {
        if (s_big[u & 1]) unit(u, cur + lane, s_v16 + lane, mask_tag, std::integral_constant<int, 1>{});
        else unit(u, cur + lane, s_v16 + lane, mask_tag, std::integral_constant<int, 0>{});
      }
    } else if constexpr (decltype(act)::value) {
      unit(u, cur + lane, nullptr, mask_tag, std::integral_constant<int, DT>{});
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's LDS loads have landed
    __syncthreads();
  };
  // the mask-free units in pairs (fixed buffers, no branch between the
  // products of consecutive units), then the rest one by one
  auto run = [&](auto act) __attribute__((always_inline)) {
    const int npair = min(nfull, nunit) & ~1;
    int u = 0;
#pragma unroll 1
    for (; u < npair; u += 2) {
      step(u, s_kv0, s_kv1, s_raw0, s_raw1, act, std::false_type{});
      step(u + 1, s_kv1, s_kv0, s_raw1, s_raw0, act, std::false_type{});
    }
#pragma unroll 1
    for (; u < nunit; ++u) {
      const bool odd = u & 1;
      const u32x4* cur = odd ? s_kv1 : s_kv0;
      u32x4* nxt = odd ? s_kv0 : s_kv1;
      u32x4* raw_ld = odd ? s_raw1 : s_raw0;
      const u32x4* raw_dq = odd ? s_raw0 : s_raw1;
      if (u < nfull) step(u, cur, nxt, raw_ld, raw_dq, act, std::false_type{});
      else step(u, cur, nxt, raw_ld, raw_dq, act, std::true_type{});
    }
  };
  if constexpr (KB == 0) {
    if (threadIdx.x == 0) s_big[0] = 0;
    fetch(0, s_kv0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
  } else {
    fetch_raw(0, s_raw0);
    if (nunit > 1) fetch_raw(1, s_raw1);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    dequant(s_raw0, s_kv0);
    __syncthreads();
  }
  if (active) run(std::true_type{});
  else run(std::false_type{});
  if (!active) return;
  // O^T: lane (column n, group g) holds dims 16 dt + 4 g + i of its column
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float lt = sum_over_groups(l[r]);
    const int tq = t0 + r * QPS + n / G;
    if (tq >= L) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t* dst = out + q_row(sb, bi, head) + (size_t)tq * kHeadDim + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint32_t lo = (uint32_t)from_f32<DT>(o[r][dt][0] * inv) | ((uint32_t)from_f32<DT>(o[r][dt][1] * inv) << 16);
      const uint32_t hi = (uint32_t)from_f32<DT>(o[r][dt][2] * inv) | ((uint32_t)from_f32<DT>(o[r][dt][3] * inv) << 16);
      *(uint2*)(dst + 16 * dt) = make_uint2(lo, hi);
    }
  }
}

template <int DT, int TB, int KB>
static void prefill_dispatch(const Geometry& g, const SeqBatch& b, int L, const uint16_t* q, float sl2,
                             uint16_t* out, hipStream_t s, Timing* prof) {
  constexpr int W = 4, R = 2, OCC = 2;
  const int per_wg = W * R * (16 / g.group);
  const dim3 grid((L + per_wg - 1) / per_wg, g.hkv, b.n), blk(64 * W);
  const int kd = kProfPrefill;
  switch (g.group) {
    case 1: launch(k_prefill<DT, TB, 1, R, W, OCC, KB>, grid, blk, 0, s, prof, kd, g, b, L, q, sl2, out); break;
    case 2: launch(k_prefill<DT, TB, 2, R, W, OCC, KB>, grid, blk, 0, s, prof, kd, g, b, L, q, sl2, out); break;
    case 4: launch(k_prefill<DT, TB, 4, R, W, OCC, KB>, grid, blk, 0, s, prof, kd, g, b, L, q, sl2, out); break;
    case 8: launch(k_prefill<DT, TB, 8, R, W, OCC, KB>, grid, blk, 0, s, prof, kd, g, b, L, q, sl2, out); break;
    default: launch(k_prefill<DT, TB, 16, R, W, OCC, KB>, grid, blk, 0, s, prof, kd, g, b, L, q, sl2, out); break;
  }
}

hipError_t launch_prefill(const Geometry& g, const SeqBatch& b, int L, const void* q, float scale,
                          void* out, hipStream_t s, Timing* prof) {
  const float sl2 = scale * 1.4426950408889634f;
  const uint16_t* qq = (const uint16_t*)q;
  uint16_t* oo = (uint16_t*)out;
  if (g.kv_bits == 4) {
    if (g.tb == 64) prefill_dispatch<0, 64, 4>(g, b, L, qq, sl2, oo, s, prof);
    else prefill_dispatch<0, 32, 4>(g, b, L, qq, sl2, oo, s, prof);
  } else if (g.kv_bits == 8) {
    if (g.tb == 64) prefill_dispatch<0, 64, 8>(g, b, L, qq, sl2, oo, s, prof);
    else prefill_dispatch<0, 32, 8>(g, b, L, qq, sl2, oo, s, prof);
  } else if (g.dtype == 0) {
    if (g.tb == 64) prefill_dispatch<0, 64, 0>(g, b, L, qq, sl2, oo, s, prof);
    else prefill_dispatch<0, 32, 0>(g, b, L, qq, sl2, oo, s, prof);
  } else {
    if (g.tb == 64) prefill_dispatch<1, 64, 0>(g, b, L, qq, sl2, oo, s, prof);
    else prefill_dispatch<1, 32, 0>(g, b, L, qq, sl2, oo, s, prof);
  }
  return hipGetLastError();
}

}  // namespace bsattn
