// Routing front end, three kernels per layer call:
//   router  bf16 router logits (+ shared-gate logit) and the 1x128 input quant
//   topk    top-k + renormalised softmax + shared-expert append per token
//   sort    count / scan / pad / scatter into 64-row expert blocks
#pragma once
#include "moe_numerics.h"

#define NK_KERNEL extern "C" __global__

// ---------------------------------------------------------------------------
// Router logits and input quantisation.
// (a1: kernels/gfx950/templates/routing/bf16_gemv.inc:16-150, semantics
// tools/benchmark/export_qwen36_router_bf16_capture.py:78; a5: the AITER 1x128
// input quant, same rule as harness/gfx950/fp8/moe/decode/
// qwen36_moe_silu_mul_quant_fp8_gfx950.hip:57-94.)
//
// logits[t, r] = bf16_rne(dot(x[t], w[r])) for r < rows = E + S (row E is the
// shared-expert gate). fp32 order (the layer's contract): 16 slices per dot
// product, slice s owning elements 128 j + 8 s + i, each a sequential fmaf
// chain from +0 in (j, i) order, folded by the tree (+8, +4, +2, +1).
// Workgroup (g, tt): 16 router rows x kRouterTokens tokens. One 16-lane group
// owns one row, keeps its slice of the row in registers and walks the tokens
// with the next token's activations already in flight, so each router weight
// byte is read once per token tile. Workgroups of column 0 also quantise their
// tokens: each 16-lane group owns one 128-element group, scale = max(amax,
// 1e-10) * 0x3b124925, q = e4m3(x * (1 / scale)). Every workgroup zeroes a
// slice of the routing bitmask that topk fills later on the same stream.
constexpr uint32_t kRouterTokens = 4;

template <uint32_t NJ>
__device__ __forceinline__ void load_slice(uint4 (&v)[NJ], const uint16_t* p) {
#pragma unroll
  for (uint32_t j = 0; j < NJ; ++j) v[j] = *reinterpret_cast<const uint4*>(p + 128u * j);
}

template <uint32_t NJ>  // NJ = H / 128
__device__ __forceinline__ void router(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                       uint16_t* __restrict__ logits, uint8_t* __restrict__ xq,
                                       float* __restrict__ xs, unsigned long long* __restrict__ mask,
                                       uint32_t T, uint32_t rows, uint32_t mask_words) {
  constexpr uint32_t H = 128 * NJ;
  const uint32_t tid = threadIdx.x;
  const uint32_t wg = blockIdx.y * gridDim.x + blockIdx.x;
  if (wg * 256u + tid < mask_words) mask[wg * 256u + tid] = 0ull;
  const uint32_t t0 = blockIdx.y * kRouterTokens;
  const uint32_t t1 = t0 + kRouterTokens < T ? t0 + kRouterTokens : T;

  const uint32_t r = blockIdx.x * 16u + (tid >> 4);
  const uint32_t s = tid & 15u;
  const bool row_ok = r < rows;
  uint4 wv[NJ], xv[NJ], xn[NJ];
  load_slice<NJ>(wv, w + (size_t)(row_ok ? r : 0u) * H + 8u * s);
  load_slice<NJ>(xv, x + (size_t)t0 * H + 8u * s);

  if (blockIdx.x == 0) {
    for (uint32_t t = t0; t < t1; ++t) {
#pragma unroll
      for (uint32_t base = 0; base < H; base += 2048u) {
        const uint32_t i0 = base + tid * 8u;
        const bool active = i0 < H;  // uniform per 16-lane group
        uint4 v = {0u, 0u, 0u, 0u};
        if (active) v = *reinterpret_cast<const uint4*>(x + (size_t)t * H + i0);
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
        if (active) {
          uint2 q;
          q.x = nk::e4m3x4(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv);
          q.y = nk::e4m3x4(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv);
          *reinterpret_cast<uint2*>(xq + (size_t)t * H + i0) = q;
          if ((tid & 15u) == 0) xs[(size_t)t * NJ + (i0 >> 7)] = scale;
        }
      }
    }
  }

  for (uint32_t t = t0; t < t1; ++t) {
    if (t + 1u < t1) load_slice<NJ>(xn, x + (size_t)(t + 1u) * H + 8u * s);
    float acc = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < NJ; ++j) {
      acc = fmaf(nk::bf16_lo(xv[j].x), nk::bf16_lo(wv[j].x), acc);
      acc = fmaf(nk::bf16_hi(xv[j].x), nk::bf16_hi(wv[j].x), acc);
      acc = fmaf(nk::bf16_lo(xv[j].y), nk::bf16_lo(wv[j].y), acc);
      acc = fmaf(nk::bf16_hi(xv[j].y), nk::bf16_hi(wv[j].y), acc);
      acc = fmaf(nk::bf16_lo(xv[j].z), nk::bf16_lo(wv[j].z), acc);
      acc = fmaf(nk::bf16_hi(xv[j].z), nk::bf16_hi(wv[j].z), acc);
      acc = fmaf(nk::bf16_lo(xv[j].w), nk::bf16_lo(wv[j].w), acc);
      acc = fmaf(nk::bf16_hi(xv[j].w), nk::bf16_hi(wv[j].w), acc);
    }
    acc = acc + __shfl_down(acc, 8u, 16);
    acc = acc + __shfl_down(acc, 4u, 16);
    acc = acc + __shfl_down(acc, 2u, 16);
    acc = acc + __shfl_down(acc, 1u, 16);
    if (s == 0 && row_ok) logits[(size_t)t * rows + r] = nk::bf16_rne(acc);
#pragma unroll
    for (uint32_t j = 0; j < NJ; ++j) xv[j] = xn[j];
  }
}

#define NK_ROUTER(HV)                                                                          \
  NK_KERNEL __launch_bounds__(256) void netra_moe_router_h##HV##_gfx950(                       \
      const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,                          \
      uint16_t* __restrict__ logits, uint8_t* __restrict__ xq, float* __restrict__ xs,         \
      unsigned long long* __restrict__ mask, uint32_t T, uint32_t H, uint32_t rows,            \
      uint32_t mask_words) {                                                                   \
    (void)H;                                                                                   \
    router<HV / 128>(x, w, logits, xq, xs, mask, T, rows, mask_words);                         \
  }
NK_ROUTER(512)
NK_ROUTER(1024)
NK_ROUTER(2048)
NK_ROUTER(4096)

// ---------------------------------------------------------------------------
// Top-k + renormalised softmax + shared-expert append.
// (a2: SGLang fused_topk, external to the reference; a3:
// runtime/gfx950/routing/decode/qwen36_shared_gate_append_bridge.hip:76-112,
// semantics tools/benchmark/export_qwen36_shared_gate_append_capture.py:97-107,134-139.)
//
// One wave per token: z_e = f32(logit_e) + bias_e; each candidate's key is
// (order-preserving bits of z) << 32 | (2^32 - 1 - e), so keys are distinct,
// larger z ranks first and equal z goes to the lower expert index. Every lane
// counts, for its candidates, how many of the E keys are larger (keys read
// from LDS eight at a time); rank r < K takes slot r. Weights: the contract
// exp of (z_slot - z_0), summed in slot order in fp32, each divided by the
// sum. With S = 1 the shared expert (id E) is appended at slot K with weight
// f32(bf16(sigmoid(f32(logit_E)))). Each (token, expert) pair sets bit t % 64
// of mask[e][t / 64]; the sort ranks tokens inside an expert from these bits.
constexpr uint32_t kTopkMaxPerLane = 8;  // E <= 512

__device__ __forceinline__ uint64_t rank_key(float z, uint32_t e) {
  uint32_t u = __float_as_uint(z);
  if (z == 0.0f) u = 0u;  // -0 and +0 compare equal
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - e);
}

NK_KERNEL __launch_bounds__(256) void netra_moe_topk_gfx950(
    const uint16_t* __restrict__ logits, const float* __restrict__ bias,
    int32_t* __restrict__ ids, float* __restrict__ weights,
    unsigned long long* __restrict__ mask, uint32_t T, uint32_t E, uint32_t K, uint32_t S,
    uint32_t W) {
  __shared__ uint64_t s_keys[4][512 + 8];
  __shared__ float s_zsel[4][64];
  __shared__ uint32_t s_idsel[4][64];
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  const uint32_t t = blockIdx.x * 4u + wave;
  const bool active = t < T;  // uniform per wave; every wave reaches the barriers
  const uint32_t rows = E + S, Ktot = K + S;
  const uint32_t per_lane = (E + 63u) >> 6;
  const uint32_t Epad = (E + 7u) & ~7u;
  uint64_t* keys = s_keys[wave];
  const uint16_t* lrow = logits + (size_t)(active ? t : 0u) * rows;

  float z[kTopkMaxPerLane];
  uint64_t key[kTopkMaxPerLane];
#pragma unroll
  for (uint32_t j = 0; j < kTopkMaxPerLane; ++j) {
    const uint32_t e = lane + 64u * j;
    z[j] = 0.0f;
    key[j] = 0ull;
    if (j < per_lane && e < Epad) {
      if (e < E) {
        z[j] = nk::bf16_f32(lrow[e]) + bias[e];
        key[j] = rank_key(z[j], e);
      }
      keys[e] = key[j];  // padding keys are 0 and never outrank a candidate
    }
  }
  __syncthreads();
  uint32_t rank[kTopkMaxPerLane];
#pragma unroll
  for (uint32_t j = 0; j < kTopkMaxPerLane; ++j) rank[j] = 0u;
  for (uint32_t u = 0; u < Epad; u += 8u) {
    uint64_t ku[8];
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) ku[q] = keys[u + q];
#pragma unroll
    for (uint32_t j = 0; j < kTopkMaxPerLane; ++j)
      if (j < per_lane)
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) rank[j] += ku[q] > key[j] ? 1u : 0u;
  }
#pragma unroll
  for (uint32_t j = 0; j < kTopkMaxPerLane; ++j) {
    const uint32_t e = lane + 64u * j;
    if (j < per_lane && e < E && rank[j] < K) {
      s_zsel[wave][rank[j]] = z[j];
      s_idsel[wave][rank[j]] = e;
    }
  }
  __syncthreads();
  if (!active) return;
  const float z0 = s_zsel[wave][0];
  float sum = 0.0f, my_ex = 0.0f;
  for (uint32_t s = 0; s < K; ++s) {
    const float ex = nk::nexp(s_zsel[wave][s] - z0);
    sum = sum + ex;
    if (lane == s) my_ex = ex;
  }
  uint32_t my_id = 0;
  if (lane < K) {
    my_id = s_idsel[wave][lane];
    ids[(size_t)t * Ktot + lane] = (int32_t)my_id;
    weights[(size_t)t * Ktot + lane] = my_ex / sum;
  }
  if (S != 0 && lane == K) {
    my_id = E;
    ids[(size_t)t * Ktot + K] = (int32_t)E;
    weights[(size_t)t * Ktot + K] = nk::bf16_f32(nk::bf16_rne(nk::sigmoid(nk::bf16_f32(lrow[E]))));
  }
  if (lane < Ktot && my_id < rows)
    atomicOr(&mask[(size_t)my_id * W + (t >> 6)], 1ull << (t & 63u));
}

// ---------------------------------------------------------------------------
// Count / scan / pad / scatter into 64-row expert blocks (a4: AITER
// moe_sorting, external to the reference; output format consumed by
// kernels/gfx950/templates/moe/prefill/fused_splitk2/entry_routing.inc:27-112,
// capacity manifests/gfx950/models/qwen36-35b-c64-fp8.json:43-49).
//
// One 1024-thread workgroup. counts[e] = popcount over mask[e][*]; expert e
// gets ceil(counts / 64) blocks laid out in expert order by an exclusive scan
// (one wave); pair (t, slot) -> e lands at block_off[e] * 64 + (rank of t among
// e's tokens, a popcount of lower mask bits), written as (slot << 24) | t.
// Rows after an expert's tokens hold (Ktot << 24) | T; unused block entries
// hold -1. Also lists the non-empty 16-row tiles, expert by expert:
// tile_map[i] = block * 4 + tile-in-block for i < num_valid[2] (the decode
// GEMMs take one tile per work item). num_valid = {padded rows, routes, tiles,
// 0}. The routing ids of the first kSortPrefetch rounds are loaded before the
// count so their latency overlaps.
// Dynamic LDS: 4 * (Etot * W + 3 * Etot + 2 + CAP) bytes.
constexpr uint32_t kSortPrefetch = 4;

NK_KERNEL __launch_bounds__(1024) void netra_moe_sort_gfx950(
    const int32_t* __restrict__ ids, const unsigned long long* __restrict__ mask,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ sorted_expert,
    int32_t* __restrict__ tile_map, int32_t* __restrict__ num_valid,
    int32_t* __restrict__ counts, uint32_t T, uint32_t Ktot, uint32_t Etot, uint32_t W,
    uint32_t cap_blocks) {
  extern __shared__ uint32_t lds[];
  uint32_t* prefix = lds;                                  // [Etot * W]
  uint32_t* block_off = prefix + Etot * W;                 // [Etot + 1]
  uint32_t* cnt = block_off + Etot + 1;                    // [Etot]
  uint32_t* tile_off = cnt + Etot;                         // [Etot + 1]
  int32_t* owner = reinterpret_cast<int32_t*>(tile_off + Etot + 1); // [cap_blocks]
  const uint32_t tid = threadIdx.x;
  const uint32_t routes = T * Ktot;

  int32_t pre[kSortPrefetch];
#pragma unroll
  for (uint32_t i = 0; i < kSortPrefetch; ++i) {
    const uint32_t r = tid + 1024u * i;
    pre[i] = r < routes ? ids[r] : -1;
  }
  for (uint32_t e = tid; e < Etot; e += 1024u) {
    uint32_t run = 0;
    for (uint32_t w = 0; w < W; ++w) {
      prefix[e * W + w] = run;
      run += (uint32_t)__popcll(mask[(size_t)e * W + w]);
    }
    cnt[e] = run;
    counts[e] = (int32_t)run;
    block_off[e] = (run + 63u) >> 6;
    tile_off[e] = (run + 15u) >> 4;
  }
  for (uint32_t b = tid; b < cap_blocks; b += 1024u) owner[b] = -1;
  __syncthreads();
  if (tid < 64u) {  // exclusive scans of blocks and tiles per expert
    uint32_t carry_b = 0, carry_t = 0;
    for (uint32_t base = 0; base < Etot; base += 64u) {
      const uint32_t e = base + tid;
      const uint32_t vb = e < Etot ? block_off[e] : 0u;
      const uint32_t vt = e < Etot ? tile_off[e] : 0u;
      uint32_t ib = vb, it = vt;
#pragma unroll
      for (uint32_t off = 1; off < 64; off <<= 1) {
        const uint32_t ob = __shfl_up(ib, off);
        const uint32_t ot = __shfl_up(it, off);
        if (tid >= off) { ib += ob; it += ot; }
      }
      if (e < Etot) { block_off[e] = carry_b + ib - vb; tile_off[e] = carry_t + it - vt; }
      carry_b += __shfl(ib, 63);
      carry_t += __shfl(it, 63);
    }
    if (tid == 0) { block_off[Etot] = carry_b; tile_off[Etot] = carry_t; }
  }
  __syncthreads();
  const uint32_t total = block_off[Etot];
  if (total > cap_blocks) {  // impossible for ids from the top-k kernel; write nothing
    if (tid == 0) { num_valid[0] = 0; num_valid[1] = -1; num_valid[2] = 0; num_valid[3] = 0; }
    return;
  }
  for (uint32_t e = tid; e < Etot; e += 1024u) {
    for (uint32_t b = block_off[e]; b < block_off[e + 1]; ++b) owner[b] = (int32_t)e;
    for (uint32_t i = tile_off[e]; i < tile_off[e + 1]; ++i)
      tile_map[i] = (int32_t)(block_off[e] * 4u + (i - tile_off[e]));
  }
  if (tid == 0) {
    num_valid[0] = (int32_t)(total * 64u);
    num_valid[1] = (int32_t)routes;
    num_valid[2] = (int32_t)tile_off[Etot];
    num_valid[3] = 0;
  }
  __syncthreads();

  for (uint32_t b = tid; b < cap_blocks; b += 1024u) sorted_expert[b] = owner[b];
  const int32_t pad = (int32_t)((Ktot << 24) | T);
  for (uint32_t p = tid; p < cap_blocks * 64u; p += 1024u) {
    const int32_t e = owner[p >> 6];
    if (e < 0 || p >= block_off[e] * 64u + cnt[e]) sorted_ids[p] = pad;
  }
  auto scatter = [&](uint32_t r, int32_t eid) {
    const uint32_t e = (uint32_t)eid;
    if (e >= Etot) return;
    const uint32_t t = r / Ktot, s = r - t * Ktot;
    const uint32_t w = t >> 6, bit = t & 63u;
    const unsigned long long word = mask[(size_t)e * W + w];
    const uint32_t pos = block_off[e] * 64u + prefix[e * W + w] +
                         (uint32_t)__popcll(word & ((1ull << bit) - 1ull));
    if (pos < cap_blocks * 64u) sorted_ids[pos] = (int32_t)((s << 24) | t);
  };
#pragma unroll
  for (uint32_t i = 0; i < kSortPrefetch; ++i)
    if (tid + 1024u * i < routes) scatter(tid + 1024u * i, pre[i]);
  for (uint32_t r = tid + 1024u * kSortPrefetch; r < routes; r += 1024u) scatter(r, ids[r]);
}
