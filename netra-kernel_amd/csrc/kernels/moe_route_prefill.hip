// Routing front end for large token counts (prefill, T > 256), three kernels:
//   route_screen  bf16-MFMA screen of the router logits, certified candidate
//                 sets, exact contract logits for the candidates, top-k +
//                 weights + shared-expert append, input quant, and per-
//                 workgroup expert histograms and in-workgroup ranks
//   sort_scan     per-expert totals, 64-row block layout, padding, and the
//                 absolute row base of every (workgroup, expert) pair
//   sort_scatter  sorted ids = base + in-workgroup rank
// The results equal those of the exact front end (moe_router.hip): top-k ids,
// weights, counts and the sorted layout are the same bits. Logits of the
// experts that were not candidates are the screen's values rounded to bf16.
#pragma once
#include "moe_numerics.h"

#define NK_KERNEL extern "C" __global__

namespace nkroute {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr uint32_t kTok = 16;       // tokens per route_screen workgroup (one MFMA row tile)
constexpr uint32_t kThreads = 512;  // 8 waves
constexpr uint32_t kWaves = kThreads / 64u;
constexpr uint32_t kMaxSlots = 64;  // K + S <= 64
// Screen margin: |L - a| <= 2^-10 * sum |x_i w_i| covers the contract's fp32
// chains (< 140 roundings of relative size 2^-24) plus the MFMA's fp32
// accumulation of exact bf16 products (< 2^11 roundings of at most 2^-23 even
// if truncating), with a factor > 3 to spare.
constexpr float kScreenMargin = 0.0009765625f;
// Exact logits in the per-token scratch are tagged with this prefix; the
// screen's sum |x w| values stored in the same words are non-negative floats,
// whose top half is never 0xFFFF.
constexpr uint32_t kExactTag = 0xFFFF0000u;

__device__ __forceinline__ nk::v4f mfma_bf16(uint4 a, uint4 b, nk::v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ uint4 abs8(uint4 v) {
  return make_uint4(v.x & 0x7fff7fffu, v.y & 0x7fff7fffu, v.z & 0x7fff7fffu, v.w & 0x7fff7fffu);
}
__device__ __forceinline__ uint32_t lane_rank(unsigned long long bal) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
}

__device__ __forceinline__ void quant8(uint4 v, uint8_t* __restrict__ q_dst, float* __restrict__ s_dst,
                                       bool first_lane) {
  float f[8] = {nk::bf16_lo(v.x), nk::bf16_hi(v.x), nk::bf16_lo(v.y), nk::bf16_hi(v.y),
                nk::bf16_lo(v.z), nk::bf16_hi(v.z), nk::bf16_lo(v.w), nk::bf16_hi(v.w)};
  float amax = nk::kAmaxFloor;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
  amax = fmaxf(amax, __shfl_xor(amax, 1u));
  amax = fmaxf(amax, __shfl_xor(amax, 2u));
  amax = fmaxf(amax, __shfl_xor(amax, 4u));
  amax = fmaxf(amax, __shfl_xor(amax, 8u));
  const float scale = amax * nk::inv_e4m3_max();
  const float inv = 1.0f / scale;
  uint2 q;
  q.x = nk::e4m3x4(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv);
  q.y = nk::e4m3x4(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv);
  *reinterpret_cast<uint2*>(q_dst) = q;
  if (first_lane) *s_dst = scale;
}

// Exact contract logit of one (token, router row) pair by a 16-lane group:
// lane s runs the sequential fmaf chain over elements 128 j + 8 s + i from +0,
// then the +8/+4/+2/+1 tree (the same order as netra_moe_router_h<H>).
template <uint32_t NJ>
__device__ __forceinline__ float exact_dot(const uint4* __restrict__ xrow, const uint4 (&wv)[NJ], uint32_t s) {
  float a = 0.0f;
#pragma unroll
  for (uint32_t j = 0; j < NJ; ++j) {
    const uint4 x = xrow[16u * j + s];
    const uint4 w = wv[j];
    a = fmaf(nk::bf16_lo(x.x), nk::bf16_lo(w.x), a);
    a = fmaf(nk::bf16_hi(x.x), nk::bf16_hi(w.x), a);
    a = fmaf(nk::bf16_lo(x.y), nk::bf16_lo(w.y), a);
    a = fmaf(nk::bf16_hi(x.y), nk::bf16_hi(w.y), a);
    a = fmaf(nk::bf16_lo(x.z), nk::bf16_lo(w.z), a);
    a = fmaf(nk::bf16_hi(x.z), nk::bf16_hi(w.z), a);
    a = fmaf(nk::bf16_lo(x.w), nk::bf16_lo(w.w), a);
    a = fmaf(nk::bf16_hi(x.w), nk::bf16_hi(w.w), a);
  }
  a = a + __shfl_down(a, 8u, 16);
  a = a + __shfl_down(a, 4u, 16);
  a = a + __shfl_down(a, 2u, 16);
  a = a + __shfl_down(a, 1u, 16);
  return a;
}

// route_screen: one workgroup per 16 tokens, 512 threads.
//  1. stage the 16 token rows in LDS (bf16, natural order) and quantise them
//     (1x128 groups, the same rule as the exact router);
//  2. bf16 MFMA over all router rows: a = x . w and b = |x| . |w| (wave w owns
//     column tiles w, w + 8, ...; the K order inside a 128-wide block is a
//     permutation shared by both operands);
//  3. per token (one wave): bounds zlo/zhi of z = f32(bf16(L)) + bias from
//     L in [a - m, a + m], m = 2^-10 b (bf16 rounding and the bias add are
//     monotone); theta = K-th largest zlo; candidates = {e : zhi_e >= theta}
//     contain the true top-K, since every other expert lies strictly below K
//     experts;
//  4. exact logits of every candidate and of the shared-gate row (16-lane
//     groups, two dot products at a time);
//  5. per token: top-K over the candidates' exact z (descending, ties to the
//     lower expert index), weights, shared expert append (as the exact top-k
//     kernel);
//  6. logits out, in-workgroup rank of every route among the workgroup's
//     routes to the same expert (token order), per-expert histogram.
template <uint32_t NJ, uint32_t RP, uint32_t EMAX>
__device__ __forceinline__ void route_screen(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ bias,
    uint16_t* __restrict__ logits, int32_t* __restrict__ ids, float* __restrict__ weights,
    uint8_t* __restrict__ xq, float* __restrict__ xs, int32_t* __restrict__ hist,
    int32_t* __restrict__ lrank, uint32_t T, uint32_t E, uint32_t K, uint32_t S) {
  constexpr uint32_t H = 128u * NJ;
  constexpr uint32_t kRow16 = 16u * NJ;                    // uint4 per token row
  constexpr uint32_t kMaxTiles = (RP / 16u + kWaves - 1u) / kWaves;
  constexpr uint32_t P = EMAX / 64u;                       // experts per lane
  static_assert(RP % 16u == 0 && EMAX % 64u == 0 && P <= 8u, "shape");
  __shared__ uint4 s_x[kTok * kRow16];
  __shared__ float s_a[kTok * RP];
  __shared__ uint32_t s_b[kTok * RP];
  __shared__ uint16_t s_cand[kTok * EMAX];
  __shared__ uint32_t s_n[kTok];
  __shared__ int32_t s_ids[kTok * kMaxSlots];
  __shared__ uint32_t s_hist[RP];

  const uint32_t rows = E + S, Ktot = K + S;
  if (rows > RP || E > EMAX || K == 0 || K > E || Ktot > kMaxSlots || S > 1u) return;  // uniform
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t t0 = blockIdx.x * kTok;
  for (uint32_t e = tid; e < RP; e += kThreads) s_hist[e] = 0u;

  // 1. staging + input quant
  constexpr uint32_t kPass = kTok * kRow16 / kThreads;
  static_assert(kTok * kRow16 % kThreads == 0, "staging passes");
  {
    uint4 v[kPass];
#pragma unroll
    for (uint32_t p = 0; p < kPass; ++p) {
      const uint32_t idx = p * kThreads + tid;
      const uint32_t tt = idx / kRow16, c16 = idx - tt * kRow16;
      const uint32_t t = t0 + tt < T ? t0 + tt : T - 1u;
      v[p] = *reinterpret_cast<const uint4*>(x + (size_t)t * H + 8u * c16);
    }
#pragma unroll
    for (uint32_t p = 0; p < kPass; ++p) {
      const uint32_t idx = p * kThreads + tid;
      const uint32_t tt = idx / kRow16, c16 = idx - tt * kRow16;
      s_x[idx] = v[p];
      if (t0 + tt < T)  // uniform per wave: a row is >= 64 uint4
        quant8(v[p], xq + (size_t)(t0 + tt) * H + 8u * c16, xs + (size_t)(t0 + tt) * NJ + (c16 >> 4),
               (tid & 15u) == 0);
    }
  }
  __syncthreads();

  // 2. screen: a = x . w, b = |x| . |w|
  {
    const uint32_t g = lane >> 4, rl = lane & 15u;
    const uint32_t ntiles = (rows + 15u) / 16u;
    nk::v4f acc[kMaxTiles], aab[kMaxTiles];
    const uint16_t* wrow[kMaxTiles];
#pragma unroll
    for (uint32_t m = 0; m < kMaxTiles; ++m) {
      acc[m] = nk::v4f{0.0f, 0.0f, 0.0f, 0.0f};
      aab[m] = acc[m];
      const uint32_t r = (wave + kWaves * m) * 16u + rl;
      wrow[m] = w + (size_t)(r < rows ? r : rows - 1u) * H + 32u * g;
    }
    const uint4* arow = s_x + rl * kRow16 + 4u * g;
    uint4 bb[2][kMaxTiles][4];
    auto load_b = [&](uint32_t kb, uint32_t buf) {
#pragma unroll
      for (uint32_t m = 0; m < kMaxTiles; ++m)
        if (wave + kWaves * m < ntiles)
#pragma unroll
          for (uint32_t q = 0; q < 4; ++q)
            bb[buf][m][q] = *reinterpret_cast<const uint4*>(wrow[m] + 128u * kb + 8u * q);
    };
    auto compute = [&](uint32_t kb, uint32_t buf) {
      uint4 a[4];
#pragma unroll
      for (uint32_t q = 0; q < 4; ++q) a[q] = arow[16u * kb + q];
#pragma unroll
      for (uint32_t m = 0; m < kMaxTiles; ++m)
        if (wave + kWaves * m < ntiles)
#pragma unroll
          for (uint32_t q = 0; q < 4; ++q) {
            acc[m] = mfma_bf16(a[q], bb[buf][m][q], acc[m]);
            aab[m] = mfma_bf16(abs8(a[q]), abs8(bb[buf][m][q]), aab[m]);
          }
    };
    load_b(0, 0);
    for (uint32_t kb = 0; kb < NJ; kb += 2u) {
      load_b(kb + 1u, 1);  // NJ is even
      compute(kb, 0);
      if (kb + 2u < NJ) load_b(kb + 2u, 0);
      compute(kb + 1u, 1);
    }
#pragma unroll
    for (uint32_t m = 0; m < kMaxTiles; ++m) {
      const uint32_t c = wave + kWaves * m;
      if (c < ntiles) {
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
          const uint32_t at = (g * 4u + i) * RP + c * 16u + rl;
          s_a[at] = acc[m][i];
          s_b[at] = __float_as_uint(aab[m][i]);
        }
      }
    }
  }
  __syncthreads();

  // 3. certified candidate sets, one wave per token
  for (uint32_t tt = wave; tt < kTok; tt += kWaves) {
    if (t0 + tt >= T) {
      if (lane == 0) s_n[tt] = 0u;
      continue;
    }
    uint32_t clo[P], chi[P];
#pragma unroll
    for (uint32_t j = 0; j < P; ++j) {
      const uint32_t e = lane + 64u * j;
      clo[j] = 0u;
      chi[j] = 0u;
      if (e < E) {
        const float a = s_a[tt * RP + e];
        const float m = __uint_as_float(s_b[tt * RP + e]) * kScreenMargin;
        const float b = bias[e];
        clo[j] = nk::order_bits(nk::bf16_f32(nk::bf16_rne(a - m)) + b);
        chi[j] = nk::order_bits(nk::bf16_f32(nk::bf16_rne(a + m)) + b);
      }
    }
    uint32_t theta = 0u;
    for (uint32_t r = 0; r < K; ++r) {
      uint32_t best = 0u, bj = 0u;
#pragma unroll
      for (uint32_t j = 0; j < P; ++j)
        if (clo[j] > best) { best = clo[j]; bj = j; }
      theta = nk::wave_reduce_u32<true>(best);
      const int wl = __ffsll(__ballot(best == theta)) - 1;
      if ((int)lane == wl) {
#pragma unroll
        for (uint32_t j = 0; j < P; ++j)
          if (j == bj) clo[j] = 0u;
      }
    }
    uint32_t n = 0u;
#pragma unroll
    for (uint32_t j = 0; j < P; ++j) {
      const uint32_t e = lane + 64u * j;
      const bool pred = e < E && chi[j] >= theta;
      const unsigned long long bal = __ballot(pred);
      if (pred) s_cand[tt * EMAX + n + lane_rank(bal)] = (uint16_t)e;
      n += (uint32_t)__popcll(bal);
    }
    if (lane == 0) s_n[tt] = n;
  }
  __syncthreads();

  // 4. exact logits of the candidates (+ the shared-gate row), two per group
  {
    const uint32_t grp = tid >> 4, s = tid & 15u;
    uint32_t pref[kTok + 1];
    pref[0] = 0u;
#pragma unroll
    for (uint32_t i = 0; i < kTok; ++i)
      pref[i + 1] = pref[i] + s_n[i] + ((S != 0u && t0 + i < T) ? 1u : 0u);
    const uint32_t jobs = pref[kTok];
    auto decode = [&](uint32_t q, uint32_t& tt, uint32_t& e) {
      tt = 0u;
#pragma unroll
      for (uint32_t i = 1; i < kTok; ++i) tt += q >= pref[i] ? 1u : 0u;
      const uint32_t idx = q - pref[tt];
      e = idx < s_n[tt] ? (uint32_t)s_cand[tt * EMAX + idx] : E;
    };
    for (uint32_t q0 = grp; q0 < jobs; q0 += 2u * (kThreads / 16u)) {
      const uint32_t q1 = q0 + kThreads / 16u;
      const bool has1 = q1 < jobs;
      uint32_t tt0, e0, tt1, e1;
      decode(q0, tt0, e0);
      decode(has1 ? q1 : q0, tt1, e1);
      uint4 w0[NJ], w1[NJ];
#pragma unroll
      for (uint32_t j = 0; j < NJ; ++j) {
        w0[j] = *reinterpret_cast<const uint4*>(w + (size_t)e0 * H + 128u * j + 8u * s);
        w1[j] = *reinterpret_cast<const uint4*>(w + (size_t)e1 * H + 128u * j + 8u * s);
      }
      const float l0 = exact_dot<NJ>(s_x + tt0 * kRow16, w0, s);
      const float l1 = exact_dot<NJ>(s_x + tt1 * kRow16, w1, s);
      if (s == 0) {
        s_b[tt0 * RP + e0] = kExactTag | nk::bf16_rne(l0);
        if (has1) s_b[tt1 * RP + e1] = kExactTag | nk::bf16_rne(l1);
      }
    }
  }
  __syncthreads();

  // 5. top-K over the candidates' exact z, weights, shared append
  for (uint32_t tt = wave; tt < kTok; tt += kWaves) {
    const uint32_t t = t0 + tt;
    if (t >= T) continue;
    const uint32_t n = s_n[tt];
    uint32_t code[P], eid[P];
#pragma unroll
    for (uint32_t j = 0; j < P; ++j) {
      const uint32_t i = lane + 64u * j;
      code[j] = 0u;
      eid[j] = 0u;
      if (i < n) {
        const uint32_t e = s_cand[tt * EMAX + i];
        eid[j] = e;
        code[j] = nk::order_bits(nk::bf16_f32(s_b[tt * RP + e] & 0xffffu) + bias[e]);
      }
    }
    uint32_t my_id = 0u, my_code = 0u;
    for (uint32_t r = 0; r < K; ++r) {
      uint32_t best = 0u, bj = 0u;
#pragma unroll
      for (uint32_t j = 0; j < P; ++j)
        if (code[j] > best) { best = code[j]; bj = j; }
      const uint32_t m = nk::wave_reduce_u32<true>(best);
      const unsigned long long tied = __ballot(best == m);
      uint32_t wl, wj;
      if (__popcll(tied) == 1) {
        wl = (uint32_t)(__ffsll(tied) - 1);
        wj = (uint32_t)__builtin_amdgcn_readlane((int)bj, (int)wl);
      } else {  // candidates are in ascending expert order along (j, lane)
        const uint32_t k = nk::wave_reduce_u32<false>(best == m ? (bj << 6) | lane : 0xffffffffu);
        wl = k & 63u;
        wj = k >> 6;
      }
      uint32_t ej = eid[0];
#pragma unroll
      for (uint32_t j = 1; j < P; ++j)
        if (j == wj) ej = eid[j];
      const uint32_t win = (uint32_t)__builtin_amdgcn_readlane((int)ej, (int)wl);
      if (lane == wl) {
#pragma unroll
        for (uint32_t j = 0; j < P; ++j)
          if (j == wj) code[j] = 0u;
      }
      if (lane == r) { my_id = win; my_code = m; }
    }
    const float z = nk::from_order_bits(my_code);
    const float z0 = __shfl(z, 0);
    const float ex = lane < K ? nk::nexp(z - z0) : 0.0f;
    float sum = 0.0f;
    for (uint32_t r = 0; r < K; ++r)
      sum = sum + __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(ex), (int)r));
    if (lane < K) {
      ids[(size_t)t * Ktot + lane] = (int32_t)my_id;
      weights[(size_t)t * Ktot + lane] = ex / sum;
    }
    if (S != 0u && lane == K) {
      my_id = E;
      const uint32_t lb = s_b[tt * RP + E] & 0xffffu;
      ids[(size_t)t * Ktot + K] = (int32_t)E;
      weights[(size_t)t * Ktot + K] = nk::bf16_f32(nk::bf16_rne(nk::sigmoid(nk::bf16_f32(lb))));
    }
    if (lane < Ktot) {
      s_ids[tt * kMaxSlots + lane] = (int32_t)my_id;
      atomicAdd(&s_hist[my_id], 1u);
    }
  }
  __syncthreads();

  // 6. logits, in-workgroup ranks, histogram
  for (uint32_t idx = tid; idx < kTok * rows; idx += kThreads) {
    const uint32_t tt = idx / rows, e = idx - tt * rows;
    if (t0 + tt >= T) break;  // later idx belong to later tokens
    const uint32_t b = s_b[tt * RP + e];
    const uint16_t bits = (b & kExactTag) == kExactTag ? (uint16_t)(b & 0xffffu) : nk::bf16_rne(s_a[tt * RP + e]);
    logits[(size_t)(t0 + tt) * rows + e] = bits;
  }
  for (uint32_t r = tid; r < kTok * Ktot; r += kThreads) {
    const uint32_t tt = r / Ktot, s = r - tt * Ktot;
    if (t0 + tt >= T) break;
    const int32_t e = s_ids[tt * kMaxSlots + s];
    uint32_t rank = 0u;
    for (uint32_t u = 0; u < tt; ++u)
      for (uint32_t v = 0; v < Ktot; ++v) rank += s_ids[u * kMaxSlots + v] == e ? 1u : 0u;
    lrank[(size_t)(t0 + tt) * Ktot + s] = (int32_t)rank;
  }
  for (uint32_t e = tid; e < rows; e += kThreads) hist[(size_t)blockIdx.x * rows + e] = (int32_t)s_hist[e];
}

}  // namespace nkroute

#define NK_ROUTE_SCREEN(HV, RPV, EMAXV)                                                           \
  NK_KERNEL __launch_bounds__(512) void netra_moe_route_screen_h##HV##_r##RPV##_gfx950(           \
      const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,                             \
      const float* __restrict__ bias, uint16_t* __restrict__ logits, int32_t* __restrict__ ids,   \
      float* __restrict__ weights, uint8_t* __restrict__ xq, float* __restrict__ xs,              \
      int32_t* __restrict__ hist, int32_t* __restrict__ lrank, uint32_t T, uint32_t H,            \
      uint32_t E, uint32_t K, uint32_t S) {                                                       \
    (void)H;                                                                                      \
    nkroute::route_screen<HV / 128, RPV, EMAXV>(x, w, bias, logits, ids, weights, xq, xs, hist,   \
                                                lrank, T, E, K, S);                               \
  }
NK_ROUTE_SCREEN(512, 384, 384)
NK_ROUTE_SCREEN(1024, 384, 384)
NK_ROUTE_SCREEN(2048, 384, 384)
NK_ROUTE_SCREEN(512, 528, 512)
NK_ROUTE_SCREEN(1024, 528, 512)
NK_ROUTE_SCREEN(2048, 528, 512)

// ---------------------------------------------------------------------------
// sort_scan (one 1024-thread workgroup): hist[g][e] holds the routes of
// route_screen workgroup g to expert e. Teams of Q = min(4, 1024 / Etot)
// threads own one expert each and split the G workgroups; counts[e] is the
// total, experts get ceil(count / 64) blocks in expert order (wave scans of
// 64 experts, then the wave totals), tiles of 16 rows likewise. hist is then
// overwritten in place with the absolute sorted row of the first route of
// (g, e): block_off[e] * 64 + routes of e in workgroups before g. Also writes
// sorted_expert, tile_map, num_valid = {padded rows, routes, tiles, 0} and
// the padding rows (Ktot << 24) | T of sorted_ids (the scatter fills the rest).
// Dynamic LDS: 4 * (1024 + 3 * Etot + 34 + CAP) bytes.
NK_KERNEL __launch_bounds__(1024) void netra_moe_sort_scan_gfx950(
    int32_t* __restrict__ hist, int32_t* __restrict__ sorted_ids, int32_t* __restrict__ sorted_expert,
    int32_t* __restrict__ tile_map, int32_t* __restrict__ num_valid, int32_t* __restrict__ counts,
    uint32_t T, uint32_t Ktot, uint32_t Etot, uint32_t G, uint32_t cap_blocks) {
  extern __shared__ uint32_t lds[];
  uint32_t* part = lds;                      // [1024]
  uint32_t* cnt = part + 1024;               // [Etot]
  uint32_t* block_off = cnt + Etot;          // [Etot + 1]
  uint32_t* tile_off = block_off + Etot + 1; // [Etot + 1]
  uint32_t* chunk = tile_off + Etot + 1;     // [32]
  int32_t* owner = reinterpret_cast<int32_t*>(chunk + 32);  // [cap_blocks]
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  if (Etot == 0u || Etot > 1024u) return;
  const uint32_t Q = 1024u / Etot >= 4u ? 4u : 1024u / Etot;
  const uint32_t e = tid / Q, q = tid - e * Q;
  const bool member = e < Etot;
  const uint32_t g0 = (G * q) / Q, g1 = (G * (q + 1u)) / Q;
  uint32_t sum = 0u;
  if (member)
    for (uint32_t g = g0; g < g1; ++g) sum += (uint32_t)hist[(size_t)g * Etot + e];
  part[tid] = sum;
  for (uint32_t b = tid; b < cap_blocks; b += 1024u) owner[b] = -1;
  __syncthreads();
  uint32_t before = 0u, total_e = 0u;
  if (member) {
    for (uint32_t u = 0; u < Q; ++u) {
      const uint32_t v = part[e * Q + u];
      before += u < q ? v : 0u;
      total_e += v;
    }
    if (q == 0) { cnt[e] = total_e; counts[e] = (int32_t)total_e; }
  }
  __syncthreads();
  const uint32_t run = tid < Etot ? cnt[tid] : 0u;
  const uint32_t vb = (run + 63u) >> 6, vt = (run + 15u) >> 4;
  uint32_t ib = vb, it = vt;
#pragma unroll
  for (uint32_t off = 1; off < 64; off <<= 1) {
    const uint32_t ob = __shfl_up(ib, off);
    const uint32_t ot = __shfl_up(it, off);
    if (lane >= off) { ib += ob; it += ot; }
  }
  if (lane == 63u) { chunk[wave] = ib; chunk[16u + wave] = it; }
  __syncthreads();
  uint32_t cb = 0, ct = 0, total = 0, total_t = 0;
#pragma unroll
  for (uint32_t c = 0; c < 16u; ++c) {
    const uint32_t b = chunk[c], t = chunk[16u + c];
    if (c < wave) { cb += b; ct += t; }
    total += b;
    total_t += t;
  }
  if (tid < Etot) { block_off[tid] = cb + ib - vb; tile_off[tid] = ct + it - vt; }
  if (tid == 0) { block_off[Etot] = total; tile_off[Etot] = total_t; }
  const uint32_t cap_tiles = (T * Ktot + 15u) / 16u + Etot;
  if (total > cap_blocks || total_t > cap_tiles) {  // impossible for route_screen histograms; write nothing
    if (tid == 0) { num_valid[0] = 0; num_valid[1] = -1; num_valid[2] = 0; num_valid[3] = 0; }
    return;
  }
  __syncthreads();
  if (member) {  // absolute base rows, in place
    uint32_t pos = block_off[e] * 64u + before;
    for (uint32_t g = g0; g < g1; ++g) {
      const uint32_t v = (uint32_t)hist[(size_t)g * Etot + e];
      hist[(size_t)g * Etot + e] = (int32_t)pos;
      pos += v;
    }
  }
  if (tid < Etot) {
    const uint32_t b0 = block_off[tid], b1 = block_off[tid + 1u];
    for (uint32_t b = b0; b < b1; ++b) owner[b] = (int32_t)tid;
    const uint32_t i0 = tile_off[tid], i1 = tile_off[tid + 1u];
    for (uint32_t i = i0; i < i1; ++i) tile_map[i] = (int32_t)(b0 * 4u + (i - i0));
  }
  if (tid == 0) {
    num_valid[0] = (int32_t)(total * 64u);
    num_valid[1] = (int32_t)(T * Ktot);
    num_valid[2] = (int32_t)total_t;
    num_valid[3] = 0;
  }
  __syncthreads();
  for (uint32_t b = tid; b < cap_blocks; b += 1024u) sorted_expert[b] = owner[b];
  const int32_t pad = (int32_t)((Ktot << 24) | T);
  for (uint32_t p = tid; p < cap_blocks * 64u; p += 1024u) {
    const int32_t o = owner[p >> 6];
    if (o < 0 || p >= block_off[o] * 64u + cnt[o]) sorted_ids[p] = pad;
  }
}

// sort_scatter: route r = (t, s) to expert e lands at base[t / 16][e] +
// lrank[r], written as (s << 24) | t. Grid ceil(T * Ktot / 256), block 256.
NK_KERNEL __launch_bounds__(256) void netra_moe_sort_scatter_gfx950(
    const int32_t* __restrict__ ids, const int32_t* __restrict__ base, const int32_t* __restrict__ lrank,
    int32_t* __restrict__ sorted_ids, uint32_t T, uint32_t Ktot, uint32_t Etot, uint32_t cap_blocks) {
  const uint32_t r = blockIdx.x * 256u + threadIdx.x;
  if (r >= T * Ktot) return;
  const uint32_t e = (uint32_t)ids[r];
  if (e >= Etot) return;
  const uint32_t t = r / Ktot, s = r - t * Ktot;
  const uint32_t pos = (uint32_t)base[(size_t)(t / nkroute::kTok) * Etot + e] + (uint32_t)lrank[r];
  if (pos < cap_blocks * 64u) sorted_ids[pos] = (int32_t)((s << 24) | t);
}
