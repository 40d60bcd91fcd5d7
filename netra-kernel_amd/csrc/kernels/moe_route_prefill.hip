// Routing front end for large token counts (prefill, T > 256), three kernels:
//   route_screen  bf16-MFMA router GEMM over all tokens and router rows, K
//                 split for small T: partial sums of the approximate logit a,
//                 and partial squared norms of the router rows
//   route_select  one to four waves per token: certified candidate set from a and
//                 the bound m = 2^-10 ||x|| ||w|| on |L - a| (Cauchy-Schwarz),
//                 exact contract logits of the candidates and the shared-gate
//                 row, top-k + weights + shared-expert append, input quant,
//                 logits out; per workgroup: its routes' sorted-id entries
//                 grouped by expert with the groups' offsets, and the expert
//                 totals added into slice counters
//   sort_route    one workgroup per expert: the expert layout (64-row blocks,
//                 padding, tile and pair lists) from the totals, the expert's
//                 prefix over the route_select workgroups, and its routes
//                 copied from the workgroups' lists into their sorted rows
// The results equal those of the exact front end (moe_router.hip): top-k ids,
// weights, counts and the sorted layout are the same bits. Logits of the
// experts that were not candidates are the screen's values rounded to bf16.
#pragma once
#include "moe_gemm_lds.hip"
#include "moe_numerics.h"

#define NK_KERNEL extern "C" __global__

namespace nkroute {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr uint32_t kMaxSlots = 64;  // K + S <= 64 (and the K selected slots fit in a candidate list)
// Screen margin: |L - a| <= 2^-10 * ||x|| ||w||. Both the contract's fp32
// chains (< 140 roundings of relative size 2^-24) and the MFMA's fp32
// accumulation of exact bf16 products (< 2^11 roundings of at most 2^-23 even
// if truncating) stay within 2.5e-4 * sum |x_i w_i| <= 2.5e-4 * ||x|| ||w||;
// 2^-10 leaves a factor > 3, and the norms are rounded up by (1 + 2^-9).
constexpr float kScreenMargin = 0.0009765625f;
constexpr float kNormSlack = 1.001953125f;
// route_select adds each expert's per-workgroup count into one of kSlices
// counters of that expert (slice = workgroup index mod kSlices), which spreads
// the atomic adds of many workgroups over more addresses; sort_route sums the
// slices. route_screen clears them (route_select runs after it).
constexpr uint32_t kSlices = 8;

__device__ __forceinline__ nk::v4f mfma_bf16(uint4 a, uint4 b, nk::v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t lane_rank(unsigned long long bal) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
}
__device__ __forceinline__ float sumsq8(uint4 v) {
  float s = 0.0f;
  s = fmaf(nk::bf16_lo(v.x), nk::bf16_lo(v.x), s);
  s = fmaf(nk::bf16_hi(v.x), nk::bf16_hi(v.x), s);
  s = fmaf(nk::bf16_lo(v.y), nk::bf16_lo(v.y), s);
  s = fmaf(nk::bf16_hi(v.y), nk::bf16_hi(v.y), s);
  s = fmaf(nk::bf16_lo(v.z), nk::bf16_lo(v.z), s);
  s = fmaf(nk::bf16_hi(v.z), nk::bf16_hi(v.z), s);
  s = fmaf(nk::bf16_lo(v.w), nk::bf16_lo(v.w), s);
  s = fmaf(nk::bf16_hi(v.w), nk::bf16_hi(v.w), s);
  return s;
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
  const nk::u32x2 q = {nk::e4m3x4(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv),
                       nk::e4m3x4(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv)};
  // non-temporal: written here, read by the gate/up GEMM two kernels later
  __builtin_nontemporal_store(q, reinterpret_cast<nk::u32x2*>(q_dst));
  if (first_lane) __builtin_nontemporal_store(scale, s_dst);
}

// Exact contract logit of one (token, router row) pair by a 16-lane group:
// lane s runs the sequential fmaf chain over elements 128 j + 8 s + i from +0,
// then the +8/+4/+2/+1 tree (the same order as netra_moe_router_h<H>). The
// token row comes from LDS, widened to fp32 and stored so that the 16 lanes'
// elements 128 j + 8 s .. + 3 are 16 consecutive float4 (32 j + s), then their
// elements + 4 .. + 7 (32 j + 16 + s): each 16-lane read is 256 contiguous
// bytes (the natural order, 32 bytes a lane, read two lanes per bank group);
// the router row comes from wv.
template <uint32_t NJ>
__device__ __forceinline__ float exact_dot(const float4* __restrict__ xrow, const uint4 (&wv)[NJ], uint32_t s) {
  float a = 0.0f;
#pragma unroll
  for (uint32_t j = 0; j < NJ; ++j) {
    const float4 xl = xrow[32u * j + s], xh = xrow[32u * j + 16u + s];
    const uint4 w = wv[j];
    a = fmaf(xl.x, nk::bf16_lo(w.x), a);
    a = fmaf(xl.y, nk::bf16_hi(w.x), a);
    a = fmaf(xl.z, nk::bf16_lo(w.y), a);
    a = fmaf(xl.w, nk::bf16_hi(w.y), a);
    a = fmaf(xh.x, nk::bf16_lo(w.z), a);
    a = fmaf(xh.y, nk::bf16_hi(w.z), a);
    a = fmaf(xh.z, nk::bf16_lo(w.w), a);
    a = fmaf(xh.w, nk::bf16_hi(w.w), a);
  }
  a = a + __shfl_down(a, 8u, 16);
  a = a + __shfl_down(a, 4u, 16);
  a = a + __shfl_down(a, 2u, 16);
  a = a + __shfl_down(a, 1u, 16);
  return a;
}

// ---------------------------------------------------------------------------
// route_screen: workgroup (tm, tn, z), 256 threads (4 waves): tokens
// 128 tm .. +127 x rows 128 tn .. +127 over K blocks [z KBS, (z + 1) KBS)
// (split K, so that a few hundred workgroups cover the token count). The K
// range is walked in 64-element half blocks: both 128 x 64 bf16 tiles (16 KiB
// each) of a half block are copied global -> LDS by buffer loads with the
// LDS-destination bit into a ring of four stages, three half blocks ahead of
// the multiplies (one workgroup per CU: its copies in flight are what hides
// the memory latency). A tile is row-major, 128 bytes a row, with the 16-byte
// chunk c of row r at position c ^ ((r >> 1) & 7): one wave copy moves eight
// whole rows (lane l: row l >> 3, position l & 7), and an operand read (one
// chunk of 16 rows per 16 lanes) hits 16 distinct (row parity, position)
// pairs, i.e. all 64 banks. Wave w multiplies rows 64 (w & 1) .. +63 by
// tokens 64 (w >> 1) .. +63 with v_mfma_f32_16x16x32_bf16, the router rows as
// the A operand, so a lane's four results are four consecutive rows of one
// token: one 16-byte store. Each tile element is read from LDS by two waves
// (the 64 x 64 wave tile keeps LDS reads at 32 flops a byte, the matrix
// cores' bf16 rate against the LDS bandwidth). Output screen[z][t][e] = the
// split's partial sum for t < T, e < RP (rows past `rows` read as zeros), row
// stride RP; the select kernel adds the splits in z order. The engine screens
// the E expert rows only (rows = E): the shared-gate row's logit is always
// computed exactly by route_select. The workgroups of the first token tile
// also write the rows' partial squared norms wsq[z][e]. Workgroup (0, 0, 0)
// clears route_select's slice counters cslice[0 .. nslice). Needs T H < 2^30
// (the buffer offsets are 32-bit).
template <uint32_t NJ, uint32_t KBS>  // H / 128, K blocks per split
__device__ __forceinline__ void route_screen(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                             float* __restrict__ screen, float* __restrict__ wsq,
                                             int32_t* __restrict__ cslice, uint32_t nslice,
                                             uint32_t T, uint32_t rows, uint32_t RP) {
  constexpr uint32_t H = 128u * NJ;
  constexpr uint32_t kTile = 128u * 128u;  // bytes of one 128 x 64 bf16 tile
  constexpr uint32_t kStages = 4u;
  constexpr uint32_t kAhead = kStages - 1u;  // half blocks in flight ahead of the one multiplied
  constexpr uint32_t kCopies = 8u;           // copies per wave per half block: 4 of x rows, 4 of router rows
  constexpr uint32_t NS = 2u * KBS;          // half blocks of the split
  static_assert(KBS <= NJ && NJ % KBS == 0, "splits cover K");
  __shared__ __align__(16) uint8_t s_tile[kStages][2][kTile];  // [stage][x, w]
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const bool norms = blockIdx.x == 0;  // uniform
  const uint32_t t0 = blockIdx.x * 128u, r0 = blockIdx.y * 128u, z = blockIdx.z, kb0 = z * KBS;
  if (norms && blockIdx.y == 0 && z == 0)
    for (uint32_t i = tid; i < nslice; i += 256u) cslice[i] = 0;
  auto swz = [](uint32_t r) { return (r >> 1) & 7u; };
  // copy c of this wave moves tile rows 32 wave + 8 c .. + 7; lane l fetches
  // the chunk that position l & 7 of row 32 wave + 8 c + (l >> 3) holds
  const nk::u32x4 rx = nklds::rsrc(x, T * H * 2u), rw = nklds::rsrc(w, rows * H * 2u);
  uint32_t xoff[4], woff[4];
#pragma unroll
  for (uint32_t c = 0; c < 4u; ++c) {
    const uint32_t row = 32u * wave + 8u * c + (lane >> 3), chunk = (lane & 7u) ^ swz(row);
    const uint32_t t = t0 + row, r = r0 + row;
    xoff[c] = t < T ? t * H * 2u + chunk * 16u : nklds::kFar;
    woff[c] = r < rows ? r * H * 2u + chunk * 16u : nklds::kFar;
  }
  const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)nklds::lds_offset(&s_tile[0][0][0]));
  auto issue = [&](uint32_t hs) __attribute__((always_inline)) {  // half block hs of the split
    const uint32_t st = lds0 + (hs % kStages) * 2u * kTile + (32u * wave) * 128u;
    const uint32_t koff = kb0 * 256u + hs * 128u;  // bytes into each row
#pragma unroll
    for (uint32_t c = 0; c < 4u; ++c) nklds::copy16(st + 8u * c * 128u, rx, xoff[c], koff);
#pragma unroll
    for (uint32_t c = 0; c < 4u; ++c) nklds::copy16(st + kTile + 8u * c * 128u, rw, woff[c], koff);
  };
#pragma unroll
  for (uint32_t hs = 0; hs < kAhead; ++hs)
    if (hs < NS) issue(hs);
  nk::v4f acc[4][4];
#pragma unroll
  for (uint32_t i = 0; i < 4; ++i)
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) acc[i][j] = nk::v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t g = lane >> 4, rl = lane & 15u;
  const uint32_t mrow = 64u * (wave & 1u), ntok = 64u * (wave >> 1);
  float nsum = 0.0f;
#pragma unroll
  for (uint32_t hs = 0; hs < NS; ++hs) {
    // copies issued after half block hs's: those of the next ones up to kAhead - 1
    if (hs + 2u < NS) nklds::wait_copies<2u * kCopies>();
    else if (hs + 1u < NS) nklds::wait_copies<kCopies>();
    else nklds::wait_copies<0>();
    nklds::barrier();  // every wave's copies of half block hs have landed, and every wave is past hs - 1
    if (hs + kAhead < NS) issue(hs + kAhead);  // into the stage half block hs - 1 used
    const uint8_t* sx = s_tile[hs % kStages][0];
    const uint8_t* sw = s_tile[hs % kStages][1];
#pragma unroll
    for (uint32_t q = 0; q < 2; ++q) {
      uint4 a[4], b[4];
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t r = mrow + 16u * i + rl;
        a[i] = *reinterpret_cast<const uint4*>(sw + r * 128u + ((4u * q + g) ^ swz(r)) * 16u);
      }
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t r = ntok + 16u * j + rl;
        b[j] = *reinterpret_cast<const uint4*>(sx + r * 128u + ((4u * q + g) ^ swz(r)) * 16u);
      }
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i)
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) acc[i][j] = mfma_bf16(a[i], b[j], acc[i][j]);
    }
    if (norms) {  // thread: half (tid & 1) of row tid >> 1 of the router tile
      const uint32_t row = tid >> 1;
#pragma unroll
      for (uint32_t c = 0; c < 4u; ++c) {
        const uint32_t chunk = 4u * (tid & 1u) + c;
        nsum += sumsq8(*reinterpret_cast<const uint4*>(sw + row * 128u + ((chunk ^ swz(row)) * 16u)));
      }
    }
  }
  if (norms) {
    nsum += __shfl_xor(nsum, 1u);
    const uint32_t r = r0 + (tid >> 1);
    if ((tid & 1u) == 0 && r < rows) wsq[(size_t)z * RP + r] = nsum;
  }
#pragma unroll
  for (uint32_t i = 0; i < 4; ++i) {
    const uint32_t e0 = r0 + mrow + 16u * i + 4u * g;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint32_t t = t0 + ntok + 16u * j + rl;
      if (t < T && e0 < RP)  // non-temporal: read once, by route_select
        __builtin_nontemporal_store(acc[i][j], reinterpret_cast<nk::v4f*>(screen + ((size_t)z * T + t) * RP + e0));
    }
  }
}

// ---------------------------------------------------------------------------
// route_select: workgroup of W waves, WPT of them per token (a token's group),
// so TW = W / WPT tokens per workgroup. The engine picks WPT so that small T
// still gives the chip a few thousand waves: a token's exact dot products,
// row staging and quant are then shared by its group's waves.
//  0. wave v of a group stages its share of the token row (512-element
//     chunks v, v + WPT, ...) in LDS widened to fp32, quantises it (1x128),
//     sums its squares, and reads the screen sums of its share of the experts
//     (lane l: experts l + 64 j for j = v, v + WPT, ...);
//  1. bounds zlo/zhi of z = f32(bf16(L)) + bias from L in [a - m, a + m],
//     m = 2^-10 ||x|| ||w_e|| (norms rounded up; bf16 rounding and the bias
//     add are monotone); theta <= K-th largest zlo; candidates =
//     {e : zhi_e >= theta} contain the true top-K, since every other expert
//     lies strictly below K experts. With WPT > 1 the codes meet in LDS and
//     every wave of the group runs the same search and candidate list;
//  2. exact logits of the candidates and of the shared-gate row, job q by
//     16-lane group q mod 4 WPT of the group (the token row staged in LDS);
//  3. the group's first wave: top-K over the candidates' exact z
//     (descending, ties to the lower expert index), weights, shared expert
//     append (as the exact top-k kernel);
//  4. logits row, each wave its share of the experts;
//  5. per workgroup g: its routes' sorted-id entries (slot << 24) | token
//     as one list bucket[g][..] grouped by expert (token order within an
//     expert), the list's expert offsets hist[g][0 .. E + S] (an exclusive
//     scan of the per-expert counts, last entry the total), and the routed
//     experts' nonzero counts added into cslice[e][g mod kSlices].
template <uint32_t NJ, uint32_t EMAX, uint32_t W, uint32_t WPT>
__device__ __forceinline__ void route_select(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ bias,
    const float* __restrict__ screen, const float* __restrict__ wsq, uint16_t* __restrict__ logits,
    int32_t* __restrict__ ids,
    float* __restrict__ weights, uint8_t* __restrict__ xq, float* __restrict__ xs,
    int32_t* __restrict__ hist, int32_t* __restrict__ bucket, int32_t* __restrict__ cslice, uint32_t T,
    uint32_t E, uint32_t K, uint32_t S, uint32_t RP, uint32_t Z, uint32_t G) {
  constexpr uint32_t H = 128u * NJ;
  constexpr uint32_t P = EMAX / 64u;         // experts per lane over the whole row
  constexpr uint32_t PW = P / WPT;           // experts per lane of one wave's share
  constexpr uint32_t TW = W / WPT;           // tokens per workgroup
  constexpr uint32_t NX = NJ / (4u * WPT);   // 512-element chunks of the row per wave
  constexpr bool kShared = WPT > 1u;         // several waves per token
  static_assert(EMAX % 64u == 0 && P <= 8u && W <= 32u && W % WPT == 0 && P % WPT == 0 &&
                NJ % (4u * WPT) == 0, "shape");
  __shared__ float4 s_x[TW][32u * NJ];        // the tokens' rows, widened to fp32
  __shared__ __align__(16) uint16_t s_cand[TW][EMAX];  // also the selected slots (K * 8 <= 2 * EMAX bytes)
  __shared__ uint16_t s_exact[TW][EMAX + 1];  // exact logit bits, candidate order; shared row last
  __shared__ int32_t s_ids[TW][kMaxSlots];
  __shared__ uint32_t s_hist[EMAX + 1];  // bit u: token u of the workgroup routes to the expert
  __shared__ float s_wn[EMAX];  // router-row norms, ||w_e|| (1 + 2^-9), from the screen's Z partial sums
  // several waves per token: the codes of every expert, and the row's partial squared norms
  __shared__ uint32_t s_lo[kShared ? TW : 1u][kShared ? EMAX : 1u];
  __shared__ uint32_t s_hi[kShared ? TW : 1u][kShared ? EMAX : 1u];
  __shared__ float s_xx[TW][WPT];
  const uint32_t rows = E + S, Ktot = K + S;
  if (E > EMAX || K == 0 || K > E || Ktot > kMaxSlots || S > 1u) return;  // uniform
  constexpr uint32_t kThreads = 64u * W;
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const uint32_t tt = wave / WPT, v = wave % WPT;  // the wave's token in the workgroup, its place in the group
  const uint32_t t = blockIdx.x * TW + tt;
  const bool active = t < T;  // uniform per group; inactive waves still take every barrier
  // This wave's row chunks, screen sums and biases are requested before the
  // workgroup's norm set-up below, so the dependent round trips overlap. The
  // split partial sums come kZBatch splits at a time (all of them, Z <= 8,
  // when a wave reads one or two experts a lane), every load of a batch
  // issued before the first add (indices clamped into range, so no load sits
  // under a condition, which would make each one its own round trip); the
  // adds run in split order from the first split's value.
  constexpr uint32_t kZBatch = PW <= 2u ? 8u : 4u;
  uint4 xv[NX];
  float aval[PW], bv[PW];
  if (active) {
#pragma unroll
    for (uint32_t p = 0; p < NX; ++p)
      xv[p] = *reinterpret_cast<const uint4*>(x + (size_t)t * H + 512u * (v + WPT * p) + 8u * lane);
    const float* srow = screen + (size_t)t * RP;  // split z at srow + z * T * RP
#pragma unroll
    for (uint32_t jj = 0; jj < PW; ++jj) bv[jj] = bias[min(lane + 64u * (v + WPT * jj), E - 1u)];
    for (uint32_t z0 = 0; z0 < Z; z0 += kZBatch) {  // uniform; one trip for Z <= kZBatch
      float part[kZBatch][PW];
#pragma unroll
      for (uint32_t zz = 0; zz < kZBatch; ++zz) {
        const float* sz = srow + (size_t)min(z0 + zz, Z - 1u) * T * RP;
#pragma unroll
        for (uint32_t jj = 0; jj < PW; ++jj) part[zz][jj] = sz[min(lane + 64u * (v + WPT * jj), E - 1u)];
      }
#pragma unroll
      for (uint32_t zz = 0; zz < kZBatch; ++zz)
        if (z0 + zz < Z) {
#pragma unroll
          for (uint32_t jj = 0; jj < PW; ++jj) aval[jj] = z0 + zz == 0u ? part[zz][jj] : aval[jj] + part[zz][jj];
        }
    }
#pragma unroll
    for (uint32_t jj = 0; jj < PW; ++jj)
      if (lane + 64u * (v + WPT * jj) >= E) aval[jj] = bv[jj] = 0.0f;
  }
  for (uint32_t e = tid; e <= EMAX; e += kThreads) {
    s_hist[e] = 0u;
    float wz[8];  // every split's partial norm at once (Z <= 8 for H <= 2048; more run a second batch)
    const uint32_t ec = min(e, E - 1u);
    float q = 0.0f;
    for (uint32_t z0 = 0; z0 < Z; z0 += 8u) {
#pragma unroll
      for (uint32_t zz = 0; zz < 8u; ++zz) wz[zz] = wsq[(size_t)min(z0 + zz, Z - 1u) * RP + ec];
#pragma unroll
      for (uint32_t zz = 0; zz < 8u; ++zz)
        if (z0 + zz < Z) q += wz[zz];
    }
    if (e < E) s_wn[e] = sqrtf(q) * kNormSlack;
  }
  const uint32_t s = lane & 15u, g = lane >> 4;

  // 0. this wave's chunks of the token row -> LDS, their 1x128 quant and squares
  float xx = 0.0f;
  if (active) {
#pragma unroll
    for (uint32_t p = 0; p < NX; ++p) {
      const uint32_t i0 = 512u * (v + WPT * p) + 8u * lane;
      const uint4 u = xv[p];
      const uint32_t jx = i0 >> 7, sx = (i0 >> 3) & 15u;  // exact_dot's order: 32 j + s, then 32 j + 16 + s
      s_x[tt][32u * jx + sx] = make_float4(nk::bf16_lo(u.x), nk::bf16_hi(u.x), nk::bf16_lo(u.y), nk::bf16_hi(u.y));
      s_x[tt][32u * jx + 16u + sx] = make_float4(nk::bf16_lo(u.z), nk::bf16_hi(u.z), nk::bf16_lo(u.w), nk::bf16_hi(u.w));
      quant8(u, xq + (size_t)t * H + i0, xs + (size_t)t * NJ + (i0 >> 7), s == 0);
      xx += sumsq8(u);
    }
#pragma unroll
    for (uint32_t off = 1; off < 64u; off <<= 1) xx += __shfl_xor(xx, off);
    if (kShared && lane == 0) s_xx[tt][v] = xx;
  }
  __syncthreads();  // s_wn, s_hist, every chunk of the rows and their squares

  // 1. certified candidates
  uint32_t clo[P], chi[P], pos[P], n = 0u;
  if (active) {
    if constexpr (kShared) {
      xx = s_xx[tt][0];
#pragma unroll
      for (uint32_t u = 1; u < WPT; ++u) xx += s_xx[tt][u];
    }
    const float mx = kScreenMargin * sqrtf(xx) * kNormSlack;
#pragma unroll
    for (uint32_t jj = 0; jj < PW; ++jj) {
      const uint32_t j = v + WPT * jj, e = lane + 64u * j;
      uint32_t lo = 0u, hi = 0u;
      if (e < E) {
        const float a = aval[jj], m = mx * s_wn[e], b = bv[jj];
        lo = nk::order_bits(nk::bf16_round_hw(a - m) + b);  // bf16 RNE (hardware; a is finite)
        hi = nk::order_bits(nk::bf16_round_hw(a + m) + b);
      }
      if constexpr (kShared) {
        s_lo[tt][e] = lo;
        s_hi[tt][e] = hi;
      } else {
        clo[j] = lo;
        chi[j] = hi;
      }
    }
  }
  if constexpr (kShared) __syncthreads();  // every expert's codes
  if (active) {
    if constexpr (kShared) {
#pragma unroll
      for (uint32_t j = 0; j < P; ++j) {
        clo[j] = s_lo[tt][lane + 64u * j];
        chi[j] = s_hi[tt][lane + 64u * j];
      }
    }
    // theta <= the K-th largest zlo: the largest code with its low 16 bits
    // clear that has at least K codes >= it, found bit by bit from the top
    // (absent experts have code 0). Any theta at or below the K-th largest
    // zlo certifies (every expert outside {zhi >= theta} lies below K
    // experts); stopping at 16 bits lowers it by less than one bf16 step of
    // z and halves the search.
    uint32_t theta = 0u;
#pragma unroll 1
    for (int bit = 31; bit >= 16; --bit) {
      const uint32_t cand = theta | (1u << bit);
      uint32_t cnt = 0u;
#pragma unroll
      for (uint32_t j = 0; j < P; ++j) cnt += (uint32_t)__popcll(__ballot(clo[j] >= cand));
      if (cnt >= K) theta = cand;
    }
#pragma unroll
    for (uint32_t j = 0; j < P; ++j) {
      const uint32_t e = lane + 64u * j;
      const bool pred = e < E && chi[j] >= theta;
      const unsigned long long bal = __ballot(pred);
      pos[j] = pred ? n + lane_rank(bal) : 0xffffffffu;
      // each wave writes the list entries of its own share of the experts
      if (pred && (!kShared || j % WPT == v)) s_cand[tt][pos[j]] = (uint16_t)e;
      n += (uint32_t)__popcll(bal);
    }
  }

  // 2. exact logits: jobs 0..n-1 are the candidates, job n the shared-gate row
  if constexpr (kShared) {
    __syncthreads();  // the whole candidate list
  } else {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's row and list are in LDS
    __builtin_amdgcn_wave_barrier();
  }
  if (active) {
    const uint32_t jobs = n + S;
#pragma unroll 1
    for (uint32_t q = 4u * v + g; q < jobs; q += 4u * WPT) {
      // Re-read the token row from LDS for every job: kept in registers
      // across jobs it costs 128 VGPRs and halves the resident waves.
      asm volatile("" ::: "memory");
      const uint32_t e = q < n ? (uint32_t)s_cand[tt][q] : E;
      uint4 wv[NJ];
#pragma unroll
      for (uint32_t j = 0; j < NJ; ++j) wv[j] = *reinterpret_cast<const uint4*>(w + (size_t)e * H + 128u * j + 8u * s);
      const float l = exact_dot<NJ>(s_x[tt], wv, s);
      if (s == 0) s_exact[tt][q] = nk::bf16_rne(l);
    }
  }
  if constexpr (kShared) {
    __syncthreads();  // every exact logit of the group
  } else {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the exact values are read back by this wave only
    __builtin_amdgcn_wave_barrier();
  }

  if (active && v == 0u) {
    // 3. top-K over the candidates' exact z (descending, ties to the lower id)
    uint32_t my_id = 0u, my_code = 0u;
    if (n <= 64u) {  // one candidate per lane: slot = rank among the candidates
      uint32_t ei = 0xffffu, ci = 0u;
      if (lane < n) {
        ei = s_cand[tt][lane];
        ci = nk::order_bits(nk::bf16_f32(s_exact[tt][lane]) + bias[ei]);
      }
      uint32_t rank = 0u;
      for (uint32_t i = 0; i < n; ++i) {
        const uint32_t c2 = (uint32_t)__builtin_amdgcn_readlane((int)ci, (int)i);
        const uint32_t e2 = (uint32_t)__builtin_amdgcn_readlane((int)ei, (int)i);
        rank += (c2 > ci || (c2 == ci && e2 < ei)) ? 1u : 0u;
      }
      // (expert, code) by slot, over the candidate list: this wave read its
      // entries into ei above, and a wave's LDS accesses complete in order
      uint2* sel_slots = reinterpret_cast<uint2*>(s_cand[tt]);
      if (lane < n && rank < K) sel_slots[rank] = make_uint2(ei, ci);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_wave_barrier();
      if (lane < K) {
        const uint2 sel = sel_slots[lane];
        my_id = sel.x;
        my_code = sel.y;
      }
    } else {  // more candidates than lanes: K selection rounds over (j, lane)
      const uint32_t Pc = (n + 63u) / 64u;
      uint32_t code[P], eid[P];
#pragma unroll
      for (uint32_t j = 0; j < P; ++j) {
        const uint32_t i = lane + 64u * j;
        code[j] = 0u;
        eid[j] = 0u;
        if (j < Pc && i < n) {
          const uint32_t e = s_cand[tt][i];
          eid[j] = e;
          code[j] = nk::order_bits(nk::bf16_f32(s_exact[tt][i]) + bias[e]);
        }
      }
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
      ids[(size_t)t * Ktot + K] = (int32_t)E;
      weights[(size_t)t * Ktot + K] = nk::bf16_f32(nk::bf16_rne(nk::sigmoid(nk::bf16_f32(s_exact[tt][n]))));
    }
    if (lane < Ktot) {
      s_ids[tt][lane] = (int32_t)my_id;
      atomicOr(&s_hist[my_id], 1u << tt);
    }
  }
  if (active) {
    // 4. logits row, this wave's share of the experts (non-temporal: no later
    // kernel of the layer reads the logits)
    uint16_t* lrow = logits + (size_t)t * rows;
#pragma unroll
    for (uint32_t jj = 0; jj < PW; ++jj) {
      const uint32_t j = v + WPT * jj, e = lane + 64u * j;
      if (e < E)
        __builtin_nontemporal_store(pos[j] != 0xffffffffu ? s_exact[tt][pos[j]] : nk::bf16_rne(aval[jj]), lrow + e);
    }
    if (S != 0u && v == 0u && lane == 0) __builtin_nontemporal_store(s_exact[tt][n], lrow + E);
  }
  __syncthreads();

  // 5. the workgroup's routes as one list grouped by expert, in token order
  // within an expert: route (tk, sl) to e lands at pre[e] + rank, pre[e] =
  // the workgroup's routes to experts below e (an exclusive scan of the
  // per-expert counts, each thread a contiguous run of experts), rank = the
  // earlier tokens in e's mask (a token routes to an expert at most once).
  // hist[g][0 .. rows] = pre (pre[rows] = the workgroup's route count), so
  // workgroup g's entries of expert e are bucket[g][pre[e] .. pre[e + 1]):
  // every store of this step goes to the workgroup's own rows.
  constexpr uint32_t kPer = (EMAX + 1u + kThreads - 1u) / kThreads;
  __shared__ uint32_t s_pre[EMAX + 2];
  __shared__ uint32_t s_wsum[W];
  uint32_t cnt[kPer], sum = 0u;
#pragma unroll
  for (uint32_t i = 0; i < kPer; ++i) {
    const uint32_t e = tid * kPer + i;
    cnt[i] = e < rows ? (uint32_t)__popc(s_hist[e]) : 0u;
    sum += cnt[i];
  }
  uint32_t inc = sum;
#pragma unroll
  for (uint32_t off = 1; off < 64u; off <<= 1) {
    const uint32_t o = __shfl_up(inc, off);
    if (lane >= off) inc += o;
  }
  if (lane == 63u) s_wsum[wave] = inc;
  __syncthreads();
  uint32_t run = inc - sum;
  for (uint32_t u = 0; u < wave; ++u) run += s_wsum[u];
  int32_t* hrow = hist + (size_t)blockIdx.x * (rows + 1u);
#pragma unroll
  for (uint32_t i = 0; i < kPer; ++i) {
    const uint32_t e = tid * kPer + i;
    if (e <= rows) {
      s_pre[e] = run;
      hrow[e] = (int32_t)run;
    }
    // a routed expert's count into its slice g mod kSlices (the shared
    // expert's total is T, which sort_route knows)
    if (e < E && cnt[i] != 0u)
      __hip_atomic_fetch_add(&cslice[e * kSlices + (blockIdx.x & (kSlices - 1u))], (int32_t)cnt[i],
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    run += cnt[i];
  }
  __syncthreads();
  const uint32_t t0 = blockIdx.x * TW;
  int32_t* brow = bucket + (size_t)blockIdx.x * (TW * Ktot);
  for (uint32_t r = tid; r < TW * Ktot; r += kThreads) {
    const uint32_t tk = r / Ktot, sl = r - tk * Ktot;
    if (t0 + tk >= T) break;
    const uint32_t e = (uint32_t)s_ids[tk][sl];
    const uint32_t rank = __popc(s_hist[e] & ((1u << tk) - 1u));
    brow[s_pre[e] + rank] = (int32_t)((sl << 24) | (t0 + tk));
  }
  (void)G;
}

}  // namespace nkroute

#define NK_ROUTE_SCREEN(HV, KBS)                                                                  \
  NK_KERNEL __launch_bounds__(256) void netra_moe_route_screen_h##HV##_k##KBS##_gfx950(           \
      const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, float* __restrict__ screen,  \
      float* __restrict__ wsq, int32_t* __restrict__ cslice, uint32_t nslice, uint32_t T,         \
      uint32_t H, uint32_t rows, uint32_t RP) {                                                   \
    (void)H;                                                                                      \
    nkroute::route_screen<HV / 128, KBS>(x, w, screen, wsq, cslice, nslice, T, rows, RP);         \
  }
NK_ROUTE_SCREEN(512, 2)
NK_ROUTE_SCREEN(512, 4)
NK_ROUTE_SCREEN(1024, 2)
NK_ROUTE_SCREEN(1024, 4)
NK_ROUTE_SCREEN(1024, 8)
NK_ROUTE_SCREEN(2048, 2)
NK_ROUTE_SCREEN(2048, 4)
NK_ROUTE_SCREEN(2048, 8)
NK_ROUTE_SCREEN(2048, 16)

#define NK_ROUTE_SELECT(HV, EMAXV, WV, PV)                                                        \
  NK_KERNEL __launch_bounds__(64 * WV) __attribute__((amdgpu_waves_per_eu(4)))                     \
  void netra_moe_route_select_h##HV##_e##EMAXV##_w##WV##x##PV##_gfx950(                           \
      const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,                             \
      const float* __restrict__ bias, const float* __restrict__ screen,                           \
      const float* __restrict__ wsq, uint16_t* __restrict__ logits, int32_t* __restrict__ ids,    \
      float* __restrict__ weights, uint8_t* __restrict__ xq, float* __restrict__ xs,              \
      int32_t* __restrict__ hist, int32_t* __restrict__ bucket, int32_t* __restrict__ cslice,     \
      uint32_t T, uint32_t H, uint32_t E, uint32_t K, uint32_t S, uint32_t RP, uint32_t Z,        \
      uint32_t G) {                                                                               \
    (void)H;                                                                                      \
    nkroute::route_select<HV / 128, EMAXV, WV, PV>(x, w, bias, screen, wsq, logits, ids, weights, \
                                                   xq, xs, hist, bucket, cslice, T, E, K, S, RP, Z, G); \
  }
// w<W>x<WPT>: W waves a workgroup, WPT of them per token (WPT <= H / 512)
#define NK_ROUTE_SELECT_1(HV, EMAXV) NK_ROUTE_SELECT(HV, EMAXV, 4, 1) NK_ROUTE_SELECT(HV, EMAXV, 8, 1)
NK_ROUTE_SELECT_1(512, 256)
NK_ROUTE_SELECT_1(1024, 256)
NK_ROUTE_SELECT_1(2048, 256)
NK_ROUTE_SELECT_1(512, 512)
NK_ROUTE_SELECT_1(1024, 512)
NK_ROUTE_SELECT_1(2048, 512)
NK_ROUTE_SELECT(1024, 256, 8, 2)
NK_ROUTE_SELECT(1024, 512, 8, 2)
NK_ROUTE_SELECT(2048, 256, 8, 2)
NK_ROUTE_SELECT(2048, 512, 8, 2)
NK_ROUTE_SELECT(2048, 256, 8, 4)
NK_ROUTE_SELECT(2048, 512, 8, 4)

// ---------------------------------------------------------------------------
// sort_route: workgroup me (256 threads) of a grid of exactly Etot, one per
// expert:
//  a. every routed expert's total = the sum of its kSlices slice counters
//     (the shared expert's: T), and the
//     expert layout from the totals (every workgroup computes the same one):
//     experts in order get ceil(count / 64) 64-row blocks, ceil(count / 16)
//     16-row tiles and ceil(blocks / 2) block pairs, an exclusive scan over
//     the experts with each thread summing a contiguous run of them;
//  b. (the shared expert: every token in order) expert me's count in each
//     route_select workgroup g (of G, W tokens
//     each, W <= 8), v_g = hist[g][me + 1] - hist[g][me], as an exclusive
//     scan over g, 256 workgroups a round: workgroup g's entries
//     bucket[g][hist[g][me] ..][0 .. v_g) are copied to rows
//     block_off[me] * 64 + prefix(g) + 0, 1, ...; counts[me] = the total;
//  c. expert me's sorted_expert blocks, tile_map and pair_map entries, and
//     its padding rows (Ktot << 24) | T after its routes;
//  d. a grid-stride share of the unused blocks: sorted_expert -1, every row
//     padding; workgroup 0 writes num_valid = {padded rows, routes, tiles,
//     pairs}.
// Dynamic LDS 4 * (4 * Etot + 3) bytes.
NK_KERNEL __launch_bounds__(256) void netra_moe_sort_route_gfx950(
    const int32_t* __restrict__ hist, const int32_t* __restrict__ bucket, const int32_t* __restrict__ cslice,
    int32_t* __restrict__ counts, int32_t* __restrict__ sorted_ids, int32_t* __restrict__ sorted_expert,
    int32_t* __restrict__ tile_map, int32_t* __restrict__ pair_map, int32_t* __restrict__ num_valid,
    uint32_t T, uint32_t Ktot, uint32_t Etot, uint32_t S, uint32_t G, uint32_t W, uint32_t cap_blocks) {
  extern __shared__ uint32_t lds[];
  uint32_t* cnt = lds;                        // [Etot]
  uint32_t* block_off = cnt + Etot;           // [Etot + 1]
  uint32_t* tile_off = block_off + Etot + 1;  // [Etot + 1]
  uint32_t* pair_off = tile_off + Etot + 1;   // [Etot + 1]
  __shared__ uint32_t s_wave[3][4];
  __shared__ uint32_t s_row[2][4];
  using nkroute::kSlices;
  static_assert(kSlices == 8u, "two 16-byte loads per expert");
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, me = blockIdx.x;
  if (Etot == 0u || Etot > 1024u || me >= Etot || W == 0u || W > 8u) return;
  // the first kRounds rounds of expert me's list offsets and the slice
  // counters of experts tid, tid + 256, ..., all requested before the first
  // wait
  constexpr uint32_t kRounds = 4;
  const uint32_t hstride = Etot + 1u, dc = W * Ktot;  // a workgroup's offsets row, its list length
  const int32_t* hcol = hist + me;                     // hist[g][me] at hcol + g * hstride
  uint32_t plo[kRounds], phi[kRounds];
#pragma unroll
  for (uint32_t i = 0; i < kRounds; ++i) {
    const uint32_t g = tid + 256u * i;
    plo[i] = phi[i] = 0u;
    if (g < G) {
      plo[i] = (uint32_t)hcol[(size_t)g * hstride];
      phi[i] = (uint32_t)hcol[(size_t)g * hstride + 1u];
    }
  }
  uint32_t cv[4];
#pragma unroll
  for (uint32_t i = 0; i < 4u; ++i) {
    const uint32_t e = tid + 256u * i;
    cv[i] = 0u;
    if (e < Etot) {
      const int4 a = *reinterpret_cast<const int4*>(cslice + e * kSlices);
      const int4 b = *reinterpret_cast<const int4*>(cslice + e * kSlices + 4u);
      cv[i] = (uint32_t)(a.x + a.y + a.z + a.w + b.x + b.y + b.z + b.w);
    }
  }
#pragma unroll
  for (uint32_t i = 0; i < 4u; ++i) {
    const uint32_t e = tid + 256u * i;
    if (e < Etot) cnt[e] = S != 0u && e == Etot - 1u ? T : cv[i];  // the shared expert: every token
  }
  __syncthreads();
  // a. layout
  const uint32_t ept = (Etot + 255u) / 256u, e0 = tid * ept;
  uint32_t sb = 0u, st = 0u, sp = 0u;
  for (uint32_t i = 0; i < ept; ++i) {
    const uint32_t e = e0 + i;
    const uint32_t c = e < Etot ? cnt[e] : 0u;
    const uint32_t vb = (c + 63u) >> 6;
    sb += vb;
    st += (c + 15u) >> 4;
    sp += (vb + 1u) >> 1;
  }
  uint32_t ib = sb, it = st, ip = sp;
#pragma unroll
  for (uint32_t off = 1; off < 64u; off <<= 1) {
    const uint32_t ob = __shfl_up(ib, off), ot = __shfl_up(it, off), op = __shfl_up(ip, off);
    if (lane >= off) { ib += ob; it += ot; ip += op; }
  }
  if (lane == 63u) { s_wave[0][wave] = ib; s_wave[1][wave] = it; s_wave[2][wave] = ip; }
  __syncthreads();
  uint32_t ob = ib - sb, ot = it - st, op = ip - sp, tb = 0u, tt = 0u, tp = 0u;
#pragma unroll
  for (uint32_t w = 0; w < 4u; ++w) {
    if (w < wave) { ob += s_wave[0][w]; ot += s_wave[1][w]; op += s_wave[2][w]; }
    tb += s_wave[0][w];
    tt += s_wave[1][w];
    tp += s_wave[2][w];
  }
  for (uint32_t i = 0; i < ept; ++i) {
    const uint32_t e = e0 + i;
    if (e < Etot) {
      block_off[e] = ob;
      tile_off[e] = ot;
      pair_off[e] = op;
      const uint32_t c = cnt[e], vb = (c + 63u) >> 6;
      ob += vb;
      ot += (c + 15u) >> 4;
      op += (vb + 1u) >> 1;
    }
  }
  if (tid == 0) { block_off[Etot] = tb; tile_off[Etot] = tt; pair_off[Etot] = tp; }
  __syncthreads();
  const uint32_t routes = T * Ktot, cap_rows = cap_blocks * 64u;
  const uint32_t cap_tiles = (routes + 15u) / 16u + Etot;
  if (tb > cap_blocks || tt > cap_tiles) {  // impossible for route_select's counts; write nothing
    if (me == 0 && tid == 0) { num_valid[0] = 0; num_valid[1] = -1; num_valid[2] = 0; num_valid[3] = 0; }
    return;
  }
  // b. expert me's routes, in route_select workgroup order (= token order).
  // The shared expert (S = 1, the last one) has every token once, in slot
  // Ktot - 1: its rows are the tokens in order, written without the lists.
  const uint32_t rbase = block_off[me] * 64u;
  uint32_t carry = 0u;
  const bool shared = S != 0u && me == Etot - 1u;
  if (shared) {
    const uint32_t slot = (Ktot - 1u) << 24;
    for (uint32_t t = tid; t < T; t += 256u)
      if (rbase + t < cap_rows) sorted_ids[rbase + t] = (int32_t)(slot | t);
    carry = T;
  }
  for (uint32_t g0 = 0; g0 < (shared ? 0u : G); g0 += 256u) {  // uniform trip count
    const uint32_t g = g0 + tid;
    uint32_t lo = 0u, hi = 0u;
    if (g0 < 256u * kRounds) {
#pragma unroll
      for (uint32_t i = 0; i < kRounds; ++i)
        if (g0 == 256u * i) { lo = plo[i]; hi = phi[i]; }
    } else if (g < G) {
      lo = (uint32_t)hcol[(size_t)g * hstride];
      hi = (uint32_t)hcol[(size_t)g * hstride + 1u];
    }
    const uint32_t v = min(hi - lo, W);  // (hi >= lo for route_select's offsets)
    // the round's list entries, requested before the scan's barrier
    const int32_t* src = bucket + (size_t)g * dc + lo;
    int32_t ent[8];
#pragma unroll
    for (uint32_t i = 0; i < 8u; ++i) ent[i] = i < v ? src[i] : 0;
    uint32_t inc = v;
#pragma unroll
    for (uint32_t off = 1; off < 64u; off <<= 1) {
      const uint32_t o = __shfl_up(inc, off);
      if (lane >= off) inc += o;
    }
    // alternate buffers: a round's reads of s_row[par] finish before the
    // barrier of the next round, ahead of the writes of the round after it
    const uint32_t par = (g0 >> 8) & 1u;
    if (lane == 63u) s_row[par][wave] = inc;
    __syncthreads();
    uint32_t before = carry, total = 0u;
#pragma unroll
    for (uint32_t w = 0; w < 4u; ++w) {
      const uint32_t x = s_row[par][w];
      before += w < wave ? x : 0u;
      total += x;
    }
    if (v != 0u) {
      const uint32_t dst = rbase + before + inc - v;
#pragma unroll
      for (uint32_t i = 0; i < 8u; ++i)
        if (i < v && dst + i < cap_rows) sorted_ids[dst + i] = ent[i];
    }
    carry += total;
  }
  if (tid == 0) counts[me] = (int32_t)carry;
  // c. expert me's blocks, tiles, pairs and padding rows
  const int32_t pad = (int32_t)((Ktot << 24) | T);
  const uint32_t b0 = block_off[me], b1 = block_off[me + 1u];
  for (uint32_t b = b0 + tid; b < b1; b += 256u) sorted_expert[b] = (int32_t)me;
  const uint32_t i0 = tile_off[me], i1 = tile_off[me + 1u];
  for (uint32_t i = i0 + tid; i < i1; i += 256u) tile_map[i] = (int32_t)(b0 * 4u + (i - i0));
  const uint32_t p0 = pair_off[me], p1 = pair_off[me + 1u];
  for (uint32_t i = p0 + tid; i < p1; i += 256u) pair_map[i] = (int32_t)(b0 + 2u * (i - p0));
  const uint32_t prow = b0 * 64u + cnt[me] + tid;  // at most 63 rows after the expert's routes
  if (tid < 64u && prow < b1 * 64u) sorted_ids[prow] = pad;
  // d. unused blocks
  const uint32_t stride = Etot * 256u;
  for (uint32_t p = tb * 64u + me * 256u + tid; p < cap_rows; p += stride) sorted_ids[p] = pad;
  for (uint32_t b = tb + me * 256u + tid; b < cap_blocks; b += stride) sorted_expert[b] = -1;
  if (me == 0 && tid == 0) {
    num_valid[0] = (int32_t)(tb * 64u);
    num_valid[1] = (int32_t)routes;
    num_valid[2] = (int32_t)tt;
    num_valid[3] = (int32_t)tp;
  }
}
