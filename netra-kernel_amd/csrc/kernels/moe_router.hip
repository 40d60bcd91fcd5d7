// Routing front end:
//   route          bf16 router logits (+ shared-gate logit), the 1x128 input
//                  quant, and top-k + renormalised softmax + shared-expert
//                  append per token (by each token group's last workgroup)
//   router_logits  the logits and the quant only (the narrow decode FFN runs
//                  the top-k in its prologue); router: the same with the
//                  routing bitmask cleared (the router bridge)
//   sort           count / scan / pad / scatter into 64-row expert blocks
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
// Workgroup (g, tt): 16 router rows x NT tokens. One 16-lane group owns one
// row and keeps its slice of the row in registers (lane s: elements
// 128 j + 8 s .. +7). The NT tokens are staged once per workgroup in LDS as
// fp32 (coalesced loads, eight consecutive values per lane), so the 16 row
// groups read them from LDS instead of each refetching them through L1; the
// row slice loads are issued first and overlap the staging. Workgroups of
// column 0 also quantise their tokens from the staging registers: each 16-lane
// group holds one 128-element block, scale = max(amax, 1e-10) * 0x3b124925,
// q = e4m3(x * (1 / scale)). With mask non-null every workgroup zeroes a
// slice of the routing bitmask (mask_words words in all); with xq and mask
// null (the router bridge) only the logits are written.
template <uint32_t NJ>
__device__ __forceinline__ void load_slice(uint4 (&v)[NJ], const uint16_t* p) {
#pragma unroll
  for (uint32_t j = 0; j < NJ; ++j) v[j] = *reinterpret_cast<const uint4*>(p + 128u * j);
}

// 1x128 quantisation of eight consecutive activations per lane; the 16 lanes
// of a group hold one 128-element block.
__device__ __forceinline__ void quant8(const float (&f)[8], uint8_t* __restrict__ q_dst,
                                       float* __restrict__ s_dst, bool first_lane) {
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

// kCoherent: logits are stored at agent scope (write-through, sc1), so a
// workgroup of the same launch on another XCD can read them once this
// workgroup's stores have completed (the route kernel's top-k hand-off).
template <uint32_t NJ, uint32_t NT, bool kCoherent = false>  // NJ = H / 128, NT tokens per workgroup
__device__ __forceinline__ void router(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                       uint16_t* __restrict__ logits, uint8_t* __restrict__ xq,
                                       float* __restrict__ xs, unsigned long long* __restrict__ mask,
                                       uint32_t T, uint32_t rows, uint32_t mask_words) {
  constexpr uint32_t H = 128 * NJ;
  constexpr uint32_t kPasses = NT * H / 2048u;  // staging: 256 lanes x 8 values per pass
  static_assert(NT * H % 2048u == 0, "staging covers whole passes");
  __shared__ float4 s_x[NT * H / 4];
  const uint32_t tid = threadIdx.x;
  const uint32_t wg = blockIdx.y * gridDim.x + blockIdx.x;
  if (mask != nullptr && wg * 256u + tid < mask_words) mask[wg * 256u + tid] = 0ull;
  const uint32_t t0 = blockIdx.y * NT;
  const uint32_t r = blockIdx.x * 16u + (tid >> 4);
  const uint32_t s = tid & 15u;
  const bool row_ok = r < rows;

  uint4 wv[NJ];
  load_slice<NJ>(wv, w + (size_t)(row_ok ? r : 0u) * H + 8u * s);
  uint4 sv[kPasses];
#pragma unroll
  for (uint32_t p = 0; p < kPasses; ++p) {
    const uint32_t e = (p * 256u + tid) * 8u;  // flat element of the NT x H tile
    const uint32_t k = e / H;
    const uint32_t t = t0 + k < T ? t0 + k : T - 1u;  // missing tokens repeat a valid row
    sv[p] = *reinterpret_cast<const uint4*>(x + (size_t)t * H + (e - k * H));
  }
  const bool quant = blockIdx.x == 0 && xq != nullptr;  // logits only when xq is null
#pragma unroll
  for (uint32_t p = 0; p < kPasses; ++p) {
    const uint32_t e = (p * 256u + tid) * 8u;
    const uint4 v = sv[p];
    float f[8] = {nk::bf16_lo(v.x), nk::bf16_hi(v.x), nk::bf16_lo(v.y), nk::bf16_hi(v.y),
                  nk::bf16_lo(v.z), nk::bf16_hi(v.z), nk::bf16_lo(v.w), nk::bf16_hi(v.w)};
    // element 128 j + 8 s + i of a token row sits at float4 32 j + s (i < 4)
    // or 32 j + 16 + s (i >= 4): the chain's 16-lane reads are contiguous
    const uint32_t eb = e - (e / H) * H, fx = (e / H) * (H / 4u) + 32u * (eb >> 7) + ((eb >> 3) & 15u);
    s_x[fx] = make_float4(f[0], f[1], f[2], f[3]);
    s_x[fx + 16u] = make_float4(f[4], f[5], f[6], f[7]);
    const uint32_t k = e / H, i0 = e - k * H;  // uniform per 16-lane group
    if (quant && t0 + k < T)
      quant8(f, xq + (size_t)(t0 + k) * H + i0, xs + (size_t)(t0 + k) * NJ + (i0 >> 7), s == 0);
  }
  __syncthreads();

  // Each token is one sequential fmaf chain over LDS reads; the NT tokens'
  // chains run interleaved (independent accumulators), and each weight is
  // widened from bf16 where the chains read it, once for all NT tokens (the
  // slice stays packed: 64 VGPRs at H = 2048). The x values of block j + 1
  // are read while block j's fmas run. With several tokens, empty asm
  // statements pin the order: one claims to rewrite block j's packed weights
  // (with a memory clobber, so no later block's reads or widenings move up),
  // the others claim to rewrite every accumulator after block j (so the
  // compiler cannot run the chains one after another, holding 128 widened
  // weights: that spilled at NT = 4).
  float acc[NT];
  float4 lo[NT], hi[NT];
#pragma unroll
  for (uint32_t k = 0; k < NT; ++k) {
    acc[k] = 0.0f;
    lo[k] = s_x[k * (H / 4u) + s];  // lo at 32 j, hi at 32 j + 16 (the staging order)
    hi[k] = s_x[k * (H / 4u) + s + 16u];
  }
#pragma unroll
  for (uint32_t j = 0; j < NJ; ++j) {
    float4 nlo[NT], nhi[NT];
    if (j + 1u < NJ) {
#pragma unroll
      for (uint32_t k = 0; k < NT; ++k) {
        nlo[k] = s_x[k * (H / 4u) + s + 32u * (j + 1u)];
        nhi[k] = s_x[k * (H / 4u) + s + 32u * (j + 1u) + 16u];
      }
    }
    uint4 wj = wv[j];
    if constexpr (NT > 1) asm volatile("" : "+v"(wj.x), "+v"(wj.y), "+v"(wj.z), "+v"(wj.w) : : "memory");
    const float w8[8] = {nk::bf16_lo(wj.x), nk::bf16_hi(wj.x), nk::bf16_lo(wj.y), nk::bf16_hi(wj.y),
                         nk::bf16_lo(wj.z), nk::bf16_hi(wj.z), nk::bf16_lo(wj.w), nk::bf16_hi(wj.w)};
#pragma unroll
    for (uint32_t k = 0; k < NT; ++k) {
      float a = acc[k];
      a = fmaf(lo[k].x, w8[0], a);
      a = fmaf(lo[k].y, w8[1], a);
      a = fmaf(lo[k].z, w8[2], a);
      a = fmaf(lo[k].w, w8[3], a);
      a = fmaf(hi[k].x, w8[4], a);
      a = fmaf(hi[k].y, w8[5], a);
      a = fmaf(hi[k].z, w8[6], a);
      a = fmaf(hi[k].w, w8[7], a);
      acc[k] = a;
    }
    if (j + 1u < NJ) {
#pragma unroll
      for (uint32_t k = 0; k < NT; ++k) {
        lo[k] = nlo[k];
        hi[k] = nhi[k];
      }
    }
    // every chain has taken block j here: the tokens stay interleaved
    if constexpr (NT > 1)
#pragma unroll
      for (uint32_t k = 0; k < NT; ++k) asm volatile("" : "+v"(acc[k]));
  }
#pragma unroll
  for (uint32_t k = 0; k < NT; ++k) {
    float a = acc[k];
    a = a + __shfl_down(a, 8u, 16);
    a = a + __shfl_down(a, 4u, 16);
    a = a + __shfl_down(a, 2u, 16);
    a = a + __shfl_down(a, 1u, 16);
    if (s == 0 && row_ok && t0 + k < T) {
      uint16_t* dst = logits + (size_t)(t0 + k) * rows + r;
      if constexpr (kCoherent) __hip_atomic_store(dst, nk::bf16_rne(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else *dst = nk::bf16_rne(a);
    }
  }
}

#define NK_ROUTER(HV, NT)                                                                      \
  NK_KERNEL __launch_bounds__(256)                                                         \
  void netra_moe_router_h##HV##_t##NT##_gfx950(                                                \
      const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,                          \
      uint16_t* __restrict__ logits, uint8_t* __restrict__ xq, float* __restrict__ xs,         \
      unsigned long long* __restrict__ mask, uint32_t T, uint32_t H, uint32_t rows,            \
      uint32_t mask_words) {                                                                   \
    (void)H;                                                                                   \
    router<HV / 128, NT>(x, w, logits, xq, xs, mask, T, rows, mask_words);                     \
  }
// Logits and the input quant only (no bitmask): the router in front of the
// fused decode FFN, which runs top-k and the sort itself.
#define NK_ROUTER_LOGITS(HV, NT)                                                                   \
  NK_KERNEL __launch_bounds__(256) void netra_moe_router_logits_h##HV##_t##NT##_gfx950(              \
      const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint16_t* __restrict__ logits, \
      uint8_t* __restrict__ xq, float* __restrict__ xs, uint32_t T, uint32_t H, uint32_t rows) {     \
    (void)H;                                                                                       \
    router<HV / 128, NT>(x, w, logits, xq, xs, nullptr, T, rows, 0u);                              \
  }
NK_ROUTER_LOGITS(512, 4)
NK_ROUTER_LOGITS(1024, 2)
NK_ROUTER_LOGITS(2048, 1)
NK_ROUTER_LOGITS(4096, 2)

// Symbol netra_moe_router_h2048_t1_gfx950: the router bridge's kernel. (NT
// tokens per workgroup elsewhere: for small T the fewest the staging allows,
// NT * H a multiple of 2048, so each wave's fmaf chains run fewer tokens and
// more workgroups share the weight rows; 7.9 -> 6.0 us at T = 64, H = 2048.)
NK_ROUTER(2048, 1)
NK_ROUTER(4096, 2)

// ---------------------------------------------------------------------------
// Top-k + renormalised softmax + shared-expert append.
// (a2: SGLang fused_topk, external to the reference; a3:
// runtime/gfx950/routing/decode/qwen36_shared_gate_append_bridge.hip:76-112,
// semantics tools/benchmark/export_qwen36_shared_gate_append_capture.py:97-107,134-139.)
//
// One wave per token: z_e = f32(logit_e) + bias_e; lane l holds experts
// l + 64 j as order-preserving codes of z. K selection rounds: every lane
// offers its largest remaining code (the lowest j on equal codes), a wave max
// finds the round's code, and among lanes offering it the lowest expert index
// wins (a ballot, or a second wave reduction when several lanes tie); the
// winner is removed. Round r fills slot r, so slots hold descending z with ties
// to the lower expert index. Weights: the contract exp of (z_slot - z_0),
// summed in slot order in fp32, each divided by the sum. With S = 1 the shared
// expert (id E) is appended at slot K with weight
// f32(bf16(sigmoid(f32(logit_E)))). Each (token, expert) pair sets bit t % 64
// of mask[e][t / 64]; the sort ranks tokens inside an expert from these bits.
// A logit as fp32; kCoherent reads at agent scope (the logits of the same
// launch, written by other workgroups with agent-scope stores).
template <bool kCoherent>
__device__ __forceinline__ float logit_f32(const uint16_t* p) {
  if constexpr (kCoherent) return nk::bf16_f32(__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  else return nk::bf16_f32(*p);
}

// The selection of one token (one wave): lane r < K gets slot r's expert and
// weight, lane K (S = 1) the shared expert's; other lanes' values are unused.
template <uint32_t P, bool kCoherent = false>  // experts per lane, P * 64 >= E
__device__ __forceinline__ void topk_select(const uint16_t* __restrict__ lrow, const float* __restrict__ bias,
                                            uint32_t E, uint32_t K, uint32_t S, uint32_t lane, uint32_t& id,
                                            float& weight) {
  // loads at clamped indices, all issued before the first use (a conditional
  // load per j would wait for each in turn)
  float lg[P], bs[P];
#pragma unroll
  for (uint32_t j = 0; j < P; ++j) {
    const uint32_t e = min(lane + 64u * j, E - 1u);
    lg[j] = logit_f32<kCoherent>(lrow + e);
    bs[j] = bias[e];
  }
  // the shared gate's logit (column E, present when S = 1) joins the same
  // batch; with S = 0 the load reads column E - 1 and is not used
  const float sg = logit_f32<kCoherent>(lrow + (E - 1u + (S != 0 ? 1u : 0u)));
  // Key of expert e = lane + 64 j: its code in the high word, ~e in the low
  // word (larger key: larger z, then lower expert index; 0: absent). Each
  // lane sorts its P keys once (descending; networks checked by the 0-1
  // principle), so a round offers every lane's head: the wave max of the
  // heads' codes, the lowest expert among lanes offering it, and the winning
  // lane moves to its next key.
  uint64_t key[P];
#pragma unroll
  for (uint32_t j = 0; j < P; ++j) {
    const uint32_t e = lane + 64u * j;
    key[j] = e < E ? ((uint64_t)nk::order_bits(lg[j] + bs[j]) << 32) | (0xffffffffu - e) : 0ull;
  }
  auto cx = [&](uint32_t i, uint32_t j) __attribute__((always_inline)) {  // key[i] >= key[j] after
    const uint64_t a = key[i], b = key[j];
    const bool sw = b > a;
    key[i] = sw ? b : a;
    key[j] = sw ? a : b;
  };
  if constexpr (P == 2) {
    cx(0, 1);
  } else if constexpr (P == 4) {
    cx(0, 1); cx(2, 3); cx(0, 2); cx(1, 3); cx(1, 2);
  } else if constexpr (P == 8) {
    cx(0, 1); cx(2, 3); cx(4, 5); cx(6, 7); cx(0, 2); cx(1, 3); cx(4, 6); cx(5, 7); cx(1, 2); cx(5, 6);
    cx(0, 4); cx(1, 5); cx(2, 6); cx(3, 7); cx(2, 4); cx(3, 5); cx(1, 2); cx(3, 4); cx(5, 6);
  } else {
    static_assert(P == 1, "P in {1, 2, 4, 8}");
  }
  uint32_t my_id = 0, my_code = 0;
  for (uint32_t r = 0; r < K; ++r) {
    const uint32_t hc = (uint32_t)(key[0] >> 32), hl = (uint32_t)key[0];
    const uint32_t m = nk::wave_max_u32_all(hc);  // in every lane
    const unsigned long long tied = __ballot(hc == m);
    uint32_t wl = (uint32_t)(__ffsll((long long)tied) - 1);  // the winning lane (uniform)
    if (__popcll(tied) != 1)  // several lanes offer the code: the lowest expert wins
      wl = (0xffffffffu - (uint32_t)__builtin_amdgcn_readfirstlane((int)nk::wave_max_u32_all(hc == m ? hl : 0u))) &
           63u;
    const uint32_t win = 0xffffffffu - (uint32_t)__builtin_amdgcn_readlane((int)hl, (int)wl);
    const bool shift = lane == wl;
#pragma unroll
    for (uint32_t j = 0; j + 1 < P; ++j) key[j] = shift ? key[j + 1] : key[j];
    key[P - 1] = shift ? 0ull : key[P - 1];
    if (lane == r) { my_id = win; my_code = m; }
  }
  const float z = nk::from_order_bits(my_code);
  const float z0 = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(z), 0));
  const float ex = lane < K ? nk::nexp(z - z0) : 0.0f;
  float sum = 0.0f;
  for (uint32_t r = 0; r < K; ++r) sum = sum + __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(ex), (int)r));
  id = my_id;
  weight = ex / sum;
  if (S != 0 && lane == K) {
    id = E;
    weight = nk::bf16_f32(nk::bf16_rne(nk::sigmoid(sg)));
  }
}

// topk_select by the expert count (E <= 512), a wave-uniform dispatch.
template <bool kCoherent = false>
__device__ __forceinline__ void topk_select_any(const uint16_t* __restrict__ lrow, const float* __restrict__ bias,
                                                uint32_t E, uint32_t K, uint32_t S, uint32_t lane, uint32_t& id,
                                                float& weight) {
  if (E <= 64u) topk_select<1, kCoherent>(lrow, bias, E, K, S, lane, id, weight);
  else if (E <= 128u) topk_select<2, kCoherent>(lrow, bias, E, K, S, lane, id, weight);
  else if (E <= 256u) topk_select<4, kCoherent>(lrow, bias, E, K, S, lane, id, weight);
  else topk_select<8, kCoherent>(lrow, bias, E, K, S, lane, id, weight);
}

// One token's selection stored as its topk_ids / topk_weights rows.
template <bool kCoherent = false>
__device__ __forceinline__ void topk_token(const uint16_t* __restrict__ lrow, const float* __restrict__ bias,
                                           int32_t* __restrict__ ids, float* __restrict__ weights, uint32_t t,
                                           uint32_t E, uint32_t K, uint32_t S, uint32_t lane) {
  const uint32_t Ktot = K + S;
  uint32_t id = 0;
  float weight = 0.0f;
  topk_select_any<kCoherent>(lrow, bias, E, K, S, lane, id, weight);
  if (lane < Ktot) {
    ids[(size_t)t * Ktot + lane] = (int32_t)id;
    weights[(size_t)t * Ktot + lane] = weight;
  }
}

// ---------------------------------------------------------------------------
// Router + top-k in one launch (the exact front end): the router above, with
// the logits stored at agent scope; the last of the gridDim.x row-group
// workgroups of a token group to finish runs top-k for those NT tokens (one
// wave each, the top-k below). Workgroups of a token group count their
// arrivals on counters[kCounterStride * blockIdx.y] (an atomic per workgroup,
// after its logit stores have completed; one counter per 256-byte line, as
// atomics on one line serialise); the last arriver reads the logits at agent
// scope. The arrival is a wrapping increment (old >= gridDim.x - 1 ? 0 :
// old + 1, one atomic), so the last arrival itself puts the counter back to
// zero for the next launch and no separate reset can be lost between two
// launches (counters start at zero: the engine zeroes its workspace when it
// is created). No workgroup waits on another, so the launch cannot deadlock
// whatever the residency.
constexpr uint32_t kCounterStride = 64;  // u32 words between hand-off counters
template <uint32_t NJ, uint32_t NT>
__device__ __forceinline__ void route(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                      const float* __restrict__ bias, uint16_t* __restrict__ logits,
                                      uint8_t* __restrict__ xq, float* __restrict__ xs, int32_t* __restrict__ ids,
                                      float* __restrict__ weights, uint32_t* __restrict__ counters, uint32_t T,
                                      uint32_t rows, uint32_t E, uint32_t K, uint32_t S) {
  static_assert(NT <= 4, "one top-k wave per token of the group");
  __shared__ uint32_t s_arrival;
  router<NJ, NT, true>(x, w, logits, xq, xs, nullptr, T, rows, 0u);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this workgroup's logit stores have completed
  __syncthreads();
  if (threadIdx.x == 0)
    s_arrival = __builtin_amdgcn_atomic_inc32(&counters[kCounterStride * blockIdx.y], gridDim.x - 1u,
                                              __ATOMIC_RELAXED, "agent");
  __syncthreads();
  if (s_arrival != gridDim.x - 1u) return;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  const uint32_t t = blockIdx.y * NT + wave;
  if (wave < NT && t < T && E <= 512u && K <= E && K + S <= 64u) {  // wave-uniform
    const uint16_t* lrow = logits + (size_t)t * rows;
    topk_token<true>(lrow, bias, ids, weights, t, E, K, S, lane);
  }
}

#define NK_ROUTE(HV, NT)                                                                          \
  NK_KERNEL __launch_bounds__(256) void netra_moe_route_h##HV##_t##NT##_gfx950(                     \
      const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ bias, \
      uint16_t* __restrict__ logits, uint8_t* __restrict__ xq, float* __restrict__ xs,            \
      int32_t* __restrict__ ids, float* __restrict__ weights, uint32_t* __restrict__ counters,     \
      uint32_t T, uint32_t H, uint32_t rows, uint32_t E, uint32_t K, uint32_t S) {                 \
    (void)H;                                                                                      \
    route<HV / 128, NT>(x, w, bias, logits, xq, xs, ids, weights, counters, T, rows, E, K, S);     \
  }
// Symbol netra_moe_route_h<H>_t<NT>_gfx950: the tokens-per-workgroup choices of the router.
NK_ROUTE(512, 4)
NK_ROUTE(1024, 2)
NK_ROUTE(1024, 4)
NK_ROUTE(2048, 1)
NK_ROUTE(2048, 4)
NK_ROUTE(4096, 2)

// ---------------------------------------------------------------------------
// Count / scan / pad / scatter into 64-row expert blocks (a4: AITER
// moe_sorting, external to the reference; output format consumed by
// kernels/gfx950/templates/moe/prefill/fused_splitk2/entry_routing.inc:27-112,
// capacity manifests/gfx950/models/qwen36-35b-c64-fp8.json:43-49).
//
// One 1024-thread workgroup. counts[e] = popcount over mask[e][*]; expert e
// gets ceil(counts / 64) blocks laid out in expert order by an exclusive scan
// (wave scans of 64 experts in parallel, then the wave totals); pair
// (t, slot) -> e lands at block_off[e] * 64 + (rank of t among e's tokens, a
// popcount of lower mask bits), written as (slot << 24) | t. Rows after an
// expert's tokens hold (Ktot << 24) | T; unused block entries hold -1. Also
// lists the non-empty 16-row tiles, expert by expert: tile_map[i] = block * 4 +
// tile-in-block for i < num_valid[2] (the decode GEMMs take one tile per work
// item), and the 128-row chunks: pair_map[i] = first block of the i-th pair
// of consecutive blocks of one expert (an expert's last block may stand
// alone), i < num_valid[3]. num_valid = {padded rows, routes, tiles, pairs}.
// The routing ids of the
// first kSortPrefetch rounds are loaded before the count so their latency
// overlaps, and when it fits (sort_mask_in_lds) the bitmask is kept in LDS for
// the scatter. Dynamic LDS: sort_lds_words(...) * 4 bytes.
constexpr uint32_t kSortPrefetch = 4;
constexpr uint32_t kSortLdsLimit = 160u * 1024u;

__host__ __device__ constexpr uint32_t sort_base_words(uint32_t Etot, uint32_t W, uint32_t cap) {
  return (Etot * W + 4u * Etot + 3u + 48u + cap + 1u) & ~1u;  // even: the mask copy is 8-byte aligned
}
__host__ __device__ constexpr bool sort_mask_in_lds(uint32_t Etot, uint32_t W, uint32_t cap) {
  return 4u * (sort_base_words(Etot, W, cap) + 2u * Etot * W) <= kSortLdsLimit;
}

NK_KERNEL __launch_bounds__(1024) void netra_moe_sort_gfx950(
    const int32_t* __restrict__ ids, unsigned long long* __restrict__ mask,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ sorted_expert,
    int32_t* __restrict__ tile_map, int32_t* __restrict__ pair_map, int32_t* __restrict__ num_valid,
    int32_t* __restrict__ counts, uint32_t T, uint32_t Ktot, uint32_t Etot, uint32_t W,
    uint32_t cap_blocks) {
  extern __shared__ uint32_t lds[];
  uint32_t* prefix = lds;                                  // [Etot * W]
  uint32_t* block_off = prefix + Etot * W;                 // [Etot + 1]
  uint32_t* cnt = block_off + Etot + 1;                    // [Etot]
  uint32_t* tile_off = cnt + Etot;                         // [Etot + 1]
  uint32_t* pair_off = tile_off + Etot + 1;                // [Etot + 1]
  uint32_t* chunk = pair_off + Etot + 1;                   // [48]: wave totals (blocks, tiles, pairs)
  int32_t* owner = reinterpret_cast<int32_t*>(chunk + 48); // [cap_blocks]
  unsigned long long* mcopy =
      reinterpret_cast<unsigned long long*>(lds + sort_base_words(Etot, W, cap_blocks));  // [Etot * W]
  const bool mlds = sort_mask_in_lds(Etot, W, cap_blocks);
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t routes = T * Ktot;
  if (Etot > 1024u) return;  // one expert per thread below

  int32_t pre[kSortPrefetch];
#pragma unroll
  for (uint32_t i = 0; i < kSortPrefetch; ++i) {
    const uint32_t r = tid + 1024u * i;
    pre[i] = r < routes ? ids[r] : -1;
  }
  // The routing bitmask (bit t % 64 of word [e][t / 64]: token t routes to
  // expert e), built here from the ids: in LDS when it fits, else in the
  // global workspace, whose words are then written and read at agent scope
  // (so no stale L1 copy is read back).
  for (uint32_t i = tid; i < Etot * W; i += 1024u) {
    if (mlds) mcopy[i] = 0ull;
    else __hip_atomic_store(&mask[i], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  auto mark = [&](uint32_t r, int32_t eid) {
    const uint32_t e = (uint32_t)eid, t = r / Ktot;
    if (e >= Etot) return;
    const unsigned long long bit = 1ull << (t & 63u);
    if (mlds) atomicOr(&mcopy[e * W + (t >> 6)], bit);
    else __hip_atomic_fetch_or(&mask[(size_t)e * W + (t >> 6)], bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
#pragma unroll
  for (uint32_t i = 0; i < kSortPrefetch; ++i)
    if (tid + 1024u * i < routes) mark(tid + 1024u * i, pre[i]);
  for (uint32_t r = tid + 1024u * kSortPrefetch; r < routes; r += 1024u) mark(r, ids[r]);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  auto mword = [&](uint32_t i) -> unsigned long long {
    return mlds ? mcopy[i] : __hip_atomic_load(&mask[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  uint32_t run = 0;
  if (tid < Etot) {
    for (uint32_t w = 0; w < W; ++w) {
      const unsigned long long m = mword(tid * W + w);
      prefix[tid * W + w] = run;
      run += (uint32_t)__popcll(m);
    }
    cnt[tid] = run;
    counts[tid] = (int32_t)run;
  }
  const uint32_t vb = (run + 63u) >> 6, vt = (run + 15u) >> 4, vp = (vb + 1u) >> 1;
  uint32_t ib = vb, it = vt, ip = vp;
#pragma unroll
  for (uint32_t off = 1; off < 64; off <<= 1) {
    const uint32_t ob = __shfl_up(ib, off);
    const uint32_t ot = __shfl_up(it, off);
    const uint32_t op = __shfl_up(ip, off);
    if (lane >= off) { ib += ob; it += ot; ip += op; }
  }
  if (lane == 63u) { chunk[wave] = ib; chunk[16u + wave] = it; chunk[32u + wave] = ip; }
  for (uint32_t b = tid; b < cap_blocks; b += 1024u) owner[b] = -1;
  __syncthreads();
  uint32_t cb = 0, ct = 0, cp = 0, total = 0, total_t = 0, total_p = 0;
#pragma unroll
  for (uint32_t c = 0; c < 16u; ++c) {
    const uint32_t b = chunk[c], t = chunk[16u + c], q = chunk[32u + c];
    if (c < wave) { cb += b; ct += t; cp += q; }
    total += b;
    total_t += t;
    total_p += q;
  }
  if (tid < Etot) { block_off[tid] = cb + ib - vb; tile_off[tid] = ct + it - vt; pair_off[tid] = cp + ip - vp; }
  if (tid == 0) { block_off[Etot] = total; tile_off[Etot] = total_t; pair_off[Etot] = total_p; }
  const uint32_t cap_tiles = (T * Ktot + 15u) / 16u + Etot;
  if (total > cap_blocks || total_t > cap_tiles) {  // impossible for ids from the top-k kernel; write nothing
    if (tid == 0) { num_valid[0] = 0; num_valid[1] = -1; num_valid[2] = 0; num_valid[3] = 0; }
    return;
  }
  __syncthreads();
  if (tid < Etot) {
    const uint32_t b0 = block_off[tid], b1 = block_off[tid + 1u];
    for (uint32_t b = b0; b < b1; ++b) owner[b] = (int32_t)tid;
    const uint32_t i0 = tile_off[tid], i1 = tile_off[tid + 1u];
    for (uint32_t i = i0; i < i1; ++i) tile_map[i] = (int32_t)(b0 * 4u + (i - i0));
    const uint32_t p0 = pair_off[tid], p1 = pair_off[tid + 1u];
    for (uint32_t i = p0; i < p1; ++i) pair_map[i] = (int32_t)(b0 + 2u * (i - p0));
  }
  if (tid == 0) {
    num_valid[0] = (int32_t)(total * 64u);
    num_valid[1] = (int32_t)routes;
    num_valid[2] = (int32_t)total_t;
    num_valid[3] = (int32_t)total_p;
  }
  __syncthreads();

  for (uint32_t b = tid; b < cap_blocks; b += 1024u) sorted_expert[b] = owner[b];
  // padding rows: each expert's rows after its routes, then the unused blocks
  const int32_t pad = (int32_t)((Ktot << 24) | T);
  for (uint32_t idx = tid; idx < Etot * 64u; idx += 1024u) {
    const uint32_t x = idx >> 6, row = block_off[x] * 64u + cnt[x] + (idx & 63u);
    if (row < block_off[x + 1u] * 64u) sorted_ids[row] = pad;
  }
  for (uint32_t p = total * 64u + tid; p < cap_blocks * 64u; p += 1024u) sorted_ids[p] = pad;
  auto scatter = [&](uint32_t r, int32_t eid) {
    const uint32_t e = (uint32_t)eid;
    if (e >= Etot) return;
    const uint32_t t = r / Ktot, s = r - t * Ktot;
    const uint32_t w = t >> 6, bit = t & 63u;
    const unsigned long long word = mword(e * W + w);
    const uint32_t pos = block_off[e] * 64u + prefix[e * W + w] +
                         (uint32_t)__popcll(word & ((1ull << bit) - 1ull));
    if (pos < cap_blocks * 64u) sorted_ids[pos] = (int32_t)((s << 24) | t);
  };
#pragma unroll
  for (uint32_t i = 0; i < kSortPrefetch; ++i)
    if (tid + 1024u * i < routes) scatter(tid + 1024u * i, pre[i]);
  for (uint32_t r = tid + 1024u * kSortPrefetch; r < routes; r += 1024u) scatter(r, ids[r]);
}
