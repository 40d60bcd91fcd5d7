// FP8 E4M3 block-scaled routed-MoE kernels for gfx950 (CDNA4, wave64).
//
// Pipeline (one engine operation per kernel, fixed grids, device-side early
// exit so the whole layer is graph-capturable):
//   router_logits -> topk_quant -> sort -> gate_up -> down -> combine
//
// Every kernel takes plain pointers followed by u32 shape constants, the
// argument order declared in include/netra_moe.h. Host code validates shapes
// before a launch; kernels additionally bound-check every data-dependent index
// (expert ids, sorted positions) so that malformed routing cannot address
// memory outside the buffers the shapes describe.
#include "moe_numerics.h"

using nk::v4f;
using nk::v8i;

#define NK_KERNEL extern "C" __global__

// ---------------------------------------------------------------------------
// Router logits (reference: kernels/gfx950/templates/routing/bf16_gemv.inc:16-150,
// semantics tools/benchmark/export_qwen36_router_bf16_capture.py:78).
//
// logits[t, r] = bf16_rne(dot(x[t], w[r])) for r < rows, where rows = E + S and
// row E (when S = 1) is the shared-expert gate. The fp32 order is the layer's
// contract: 16 slices per dot product (slice s owns elements 128j + 8s + i),
// each a sequential fmaf chain from +0 in (j, i) order, folded by the tree
// (+8, +4, +2, +1). One 16-lane group computes one dot product; a 256-thread
// workgroup covers 16 rows of one token. Side job: zero the routing bitmask
// that topk_quant fills in the same call (it runs later on the same stream).
NK_KERNEL __launch_bounds__(256) void netra_moe_router_logits_gfx950(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ logits, unsigned long long* __restrict__ mask,
    uint32_t T, uint32_t H, uint32_t rows, uint32_t mask_words) {
  const uint32_t tid = threadIdx.x;
  const uint32_t wg = blockIdx.y * gridDim.x + blockIdx.x;
  if (wg * 256u + tid < mask_words) mask[wg * 256u + tid] = 0ull;

  const uint32_t t = blockIdx.y;
  const uint32_t r = blockIdx.x * 16u + (tid >> 4);
  const uint32_t s = tid & 15u;
  if (t >= T) return;  // uniform across the workgroup
  float acc = 0.0f;
  if (r < rows) {
    const uint16_t* xr = x + (size_t)t * H + 8u * s;
    const uint16_t* wr = w + (size_t)r * H + 8u * s;
    for (uint32_t j = 0; j < H / 128u; ++j) {
      const uint4 xv = *reinterpret_cast<const uint4*>(xr + 128u * j);
      const uint4 wv = *reinterpret_cast<const uint4*>(wr + 128u * j);
      acc = fmaf(nk::bf16_lo(xv.x), nk::bf16_lo(wv.x), acc);
      acc = fmaf(nk::bf16_hi(xv.x), nk::bf16_hi(wv.x), acc);
      acc = fmaf(nk::bf16_lo(xv.y), nk::bf16_lo(wv.y), acc);
      acc = fmaf(nk::bf16_hi(xv.y), nk::bf16_hi(wv.y), acc);
      acc = fmaf(nk::bf16_lo(xv.z), nk::bf16_lo(wv.z), acc);
      acc = fmaf(nk::bf16_hi(xv.z), nk::bf16_hi(wv.z), acc);
      acc = fmaf(nk::bf16_lo(xv.w), nk::bf16_lo(wv.w), acc);
      acc = fmaf(nk::bf16_hi(xv.w), nk::bf16_hi(wv.w), acc);
    }
  }
  acc = acc + __shfl_down(acc, 8u, 16);
  acc = acc + __shfl_down(acc, 4u, 16);
  acc = acc + __shfl_down(acc, 2u, 16);
  acc = acc + __shfl_down(acc, 1u, 16);
  if (s == 0 && r < rows) logits[(size_t)t * rows + r] = nk::bf16_rne(acc);
}

// ---------------------------------------------------------------------------
// Top-k + renormalised softmax + shared-expert append + 1x128 input quant.
// (a2: SGLang fused_topk, external; a3: runtime/gfx950/routing/decode/
// qwen36_shared_gate_append_bridge.hip:76-112 with semantics
// tools/benchmark/export_qwen36_shared_gate_append_capture.py:97-107,134-139;
// a5: AITER 1x128 input quant, same rule as the SiLU requant.)
//
// One wave per token. z_e = f32(logit_e) + bias_e; K rounds of a wave-wide
// arg-max (ties -> lower expert index) give slots in descending z; weights are
// the contract exp of (z - z_max) over a slot-ordered fp32 sum. The shared
// expert (id E) is appended at slot K with weight f32(bf16(sigmoid(logit_E))).
// Each routed (token, expert) pair sets bit t%64 of mask[e][t/64]; sort ranks
// tokens inside an expert from these bits.
constexpr uint32_t kMaxExpertsPerLane = 8;  // E <= 512

__device__ __forceinline__ bool better(float za, uint32_t ia, float zb, uint32_t ib) {
  // true when (za, ia) ranks before (zb, ib); ib == ~0u marks "no candidate".
  if (ib == 0xffffffffu) return ia != 0xffffffffu;
  if (ia == 0xffffffffu) return false;
  return za > zb || (za == zb && ia < ib);
}

NK_KERNEL __launch_bounds__(256) void netra_moe_topk_quant_gfx950(
    const uint16_t* __restrict__ logits, const float* __restrict__ bias,
    const uint16_t* __restrict__ x, int32_t* __restrict__ ids,
    float* __restrict__ weights, uint8_t* __restrict__ xq, float* __restrict__ xs,
    unsigned long long* __restrict__ mask, uint32_t T, uint32_t H, uint32_t E,
    uint32_t K, uint32_t S, uint32_t mask_words_per_expert) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t t = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (t >= T) return;  // uniform across the wave
  const uint32_t rows = E + S, Ktot = K + S;
  const uint16_t* lrow = logits + (size_t)t * rows;

  float z[kMaxExpertsPerLane];
  uint32_t live = 0;  // bit j: expert lane + 64 j is a remaining candidate
#pragma unroll
  for (uint32_t j = 0; j < kMaxExpertsPerLane; ++j) {
    const uint32_t e = lane + 64u * j;
    z[j] = 0.0f;
    if (e < E) {
      z[j] = nk::bf16_f32(lrow[e]) + bias[e];
      live |= 1u << j;
    }
  }
  uint32_t my_id = 0;
  float my_z = 0.0f;
  float zsel0 = 0.0f;
  for (uint32_t s = 0; s < K; ++s) {
    float bz = 0.0f;
    uint32_t bi = 0xffffffffu;
#pragma unroll
    for (uint32_t j = 0; j < kMaxExpertsPerLane; ++j)
      if ((live >> j) & 1u) {
        const uint32_t e = lane + 64u * j;
        if (better(z[j], e, bz, bi)) { bz = z[j]; bi = e; }
      }
#pragma unroll
    for (uint32_t off = 1; off < 64; off <<= 1) {
      const float oz = __shfl_xor(bz, off);
      const uint32_t oi = __shfl_xor(bi, off);
      if (better(oz, oi, bz, bi)) { bz = oz; bi = oi; }
    }
    if ((bi & 63u) == lane) live &= ~(1u << (bi >> 6));
    if (lane == s) { my_id = bi; my_z = bz; }
    if (s == 0) zsel0 = bz;
  }
  // Slot-ordered sum of exp(z_s - z_0), evaluated identically on every lane.
  float sum = 0.0f, my_ex = 0.0f;
  for (uint32_t s = 0; s < K; ++s) {
    const float zs = __shfl(my_z, s);
    const float ex = nk::nexp(zs - zsel0);
    sum = sum + ex;
    if (lane == s) my_ex = ex;
  }
  if (lane < K) {
    ids[(size_t)t * Ktot + lane] = (int32_t)my_id;
    weights[(size_t)t * Ktot + lane] = my_ex / sum;
  }
  if (S != 0 && lane == K) {
    const float sig = nk::sigmoid(nk::bf16_f32(lrow[E]));
    my_id = E;
    ids[(size_t)t * Ktot + K] = (int32_t)E;
    weights[(size_t)t * Ktot + K] = nk::bf16_f32(nk::bf16_rne(sig));
  }
  if (lane < Ktot && my_id < E + S)
    atomicOr(&mask[(size_t)my_id * mask_words_per_expert + (t >> 6)], 1ull << (t & 63u));

  // 1x128 group quantisation of the token row: each lane owns 2 of 128.
  const uint16_t* xr = x + (size_t)t * H;
  for (uint32_t g = 0; g < H / 128u; ++g) {
    const uint32_t pair = *reinterpret_cast<const uint32_t*>(xr + g * 128u + 2u * lane);
    const float v0 = nk::bf16_lo(pair), v1 = nk::bf16_hi(pair);
    float amax = fmaxf(nk::kAmaxFloor, fmaxf(fabsf(v0), fabsf(v1)));
#pragma unroll
    for (uint32_t off = 1; off < 64; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float scale = amax * nk::inv_e4m3_max();
    const float inv = 1.0f / scale;
    const uint32_t q = nk::e4m3_rne(v0 * inv) | (nk::e4m3_rne(v1 * inv) << 8);
    *reinterpret_cast<uint16_t*>(xq + (size_t)t * H + g * 128u + 2u * lane) = (uint16_t)q;
    if (lane == 0) xs[(size_t)t * (H / 128u) + g] = scale;
  }
}

// ---------------------------------------------------------------------------
// Count / scan / pad / scatter (reference consumer format:
// kernels/gfx950/templates/moe/prefill/fused_splitk2/entry_routing.inc:27-112;
// AITER moe_sorting itself is external).
//
// One 1024-thread workgroup. counts[e] = popcount over mask[e][*]; each
// expert gets ceil(counts / 64) blocks of 64 rows, blocks laid out in expert
// order (exclusive scan by one wave); every routed pair (t, slot) -> e lands
// at block_off[e]*64 + rank of t among e's tokens (popcount of the lower mask
// bits), written as (slot << 24) | t. Rows after an expert's tokens hold
// (Ktot << 24) | T. Unused block entries hold -1. num_valid = {rows, routes}.
// Dynamic LDS: (Etot * W + 2 * Etot + 1) u32.
NK_KERNEL __launch_bounds__(1024) void netra_moe_sort_gfx950(
    const int32_t* __restrict__ ids, const unsigned long long* __restrict__ mask,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ sorted_expert,
    int32_t* __restrict__ num_valid, int32_t* __restrict__ counts, uint32_t T,
    uint32_t Ktot, uint32_t Etot, uint32_t W, uint32_t cap_blocks) {
  extern __shared__ uint32_t lds[];
  uint32_t* prefix = lds;                  // [Etot * W]
  uint32_t* block_off = lds + Etot * W;    // [Etot + 1]
  uint32_t* cnt = block_off + Etot + 1;    // [Etot]
  const uint32_t tid = threadIdx.x;

  for (uint32_t e = tid; e < Etot; e += 1024u) {
    uint32_t run = 0;
    for (uint32_t w = 0; w < W; ++w) {
      prefix[e * W + w] = run;
      run += (uint32_t)__popcll(mask[(size_t)e * W + w]);
    }
    cnt[e] = run;
    counts[e] = (int32_t)run;
    block_off[e] = (run + 63u) >> 6;
  }
  __syncthreads();
  if (tid < 64u) {
    uint32_t carry = 0;
    for (uint32_t base = 0; base < Etot; base += 64u) {
      const uint32_t e = base + tid;
      const uint32_t v = e < Etot ? block_off[e] : 0u;
      uint32_t incl = v;
#pragma unroll
      for (uint32_t off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off);
        if (tid >= off) incl += o;
      }
      if (e < Etot) block_off[e] = carry + incl - v;
      carry += __shfl(incl, 63);
    }
    if (tid == 0) block_off[Etot] = carry;
  }
  __syncthreads();
  const uint32_t total = block_off[Etot];
  if (total > cap_blocks) {  // cannot happen for valid ids; refuse to write
    if (tid == 0) { num_valid[0] = 0; num_valid[1] = -1; }
    return;
  }
  if (tid == 0) { num_valid[0] = (int32_t)(total * 64u); num_valid[1] = (int32_t)(T * Ktot); }

  const int32_t pad = (int32_t)((Ktot << 24) | T);
  for (uint32_t b = tid; b < cap_blocks; b += 1024u) {
    int32_t owner = -1;
    uint32_t valid_end = 0;
    if (b < total) {
      uint32_t lo = 0, hi = Etot;  // last e with block_off[e] <= b
      while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (block_off[mid] <= b) lo = mid; else hi = mid;
      }
      owner = (int32_t)lo;
      valid_end = block_off[lo] * 64u + cnt[lo];
    }
    sorted_expert[b] = owner;
    for (uint32_t i = 0; i < 64u; ++i) {
      const uint32_t p = b * 64u + i;
      if (owner < 0 || p >= valid_end) sorted_ids[p] = pad;
    }
  }
  for (uint32_t r = tid; r < T * Ktot; r += 1024u) {
    const uint32_t t = r / Ktot, s = r - t * Ktot;
    const uint32_t e = (uint32_t)ids[r];
    if (e >= Etot) continue;
    const uint32_t w = t >> 6, bit = t & 63u;
    const unsigned long long word = mask[(size_t)e * W + w];
    const uint32_t pos = block_off[e] * 64u + prefix[e * W + w] +
                         (uint32_t)__popcll(word & ((1ull << bit) - 1ull));
    if (pos < cap_blocks * 64u) sorted_ids[pos] = (int32_t)((s << 24) | t);
  }
}

// ---------------------------------------------------------------------------
// Grouped gate/up GEMM + SiLU.mul + 1x128 FP8 requant
// (reference: kernels/gfx950/templates/moe/decode/gate_up_mfma.inc:12-161 and
// silu_quant.inc:16-236; oracle tools/benchmark/export_qwen36_moe_stage1_capture.py:80-97).
//
// Workgroup (b, ng): expert block b (64 sorted rows of one expert), h columns
// [128 ng, 128 ng + 128). Wave w owns h columns 32w..32w+31: W13 rows for gate
// (n) and up (I + n), four 16-column MFMA tiles, looped over the block's
// non-empty 16-row tiles. Per 128-K block the partial product is scaled as
// acc += w_s * (a_s * mfma) (mfma.inc:20-24). Epilogue: h = bf16(silu(g) * u),
// amax over the 128-column group (lanes, then waves through LDS), scale =
// max(amax, 1e-10) * 0x3b124925, q = e4m3(h * (1 / scale)).
NK_KERNEL __launch_bounds__(256) void netra_moe_gate_up_gfx950(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs,
    const uint8_t* __restrict__ w13, const float* __restrict__ w13s,
    const int32_t* __restrict__ sorted_ids, const int32_t* __restrict__ sorted_expert,
    const int32_t* __restrict__ num_valid, uint8_t* __restrict__ hq,
    float* __restrict__ hs, uint32_t T, uint32_t H, uint32_t I, uint32_t Ktot,
    uint32_t Etot) {
  __shared__ int32_t s_tok[64];
  __shared__ float s_amax[4][64];
  __shared__ float s_scale[64];
  const uint32_t b = blockIdx.x, ng = blockIdx.y;
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
  if (b * 64u >= (uint32_t)num_valid[0]) return;
  const int32_t e = sorted_expert[b];
  if (e < 0 || (uint32_t)e >= Etot) return;
  if (tid < 64u) {
    const int32_t id = sorted_ids[b * 64u + tid];
    const uint32_t t = (uint32_t)id & 0xffffffu, slot = (uint32_t)id >> 24;
    s_tok[tid] = (t < T && slot < Ktot) ? (int32_t)t : -1;
  }
  __syncthreads();
  const uint32_t nvalid = (uint32_t)__popcll(__ballot(s_tok[lane] >= 0));
  const uint32_t ntiles = (nvalid + 15u) >> 4;
  const uint32_t KB = H / 128u;
  const uint8_t* we = w13 + (size_t)e * 2u * I * H;
  const float* wse = w13s + (size_t)e * (2u * I / 128u) * KB;
  const uint32_t kofs = (lane >> 4) * 32u;
  const uint32_t ncol = ng * 128u + wave * 32u + (lane & 15u);
  uint32_t nrow[4] = {ncol, ncol + 16u, I + ncol, I + ncol + 16u};

  int32_t arow_tok[4];
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt) {
    const int32_t tk = s_tok[rt * 16u + (lane & 15u)];
    arow_tok[rt] = tk < 0 ? 0 : tk;
  }
  int32_t srow_tok[4][4];
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt)
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const int32_t tk = s_tok[rt * 16u + (lane >> 4) * 4u + j];
      srow_tok[rt][j] = tk < 0 ? 0 : tk;
    }

  v4f acc[4][4];
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt)
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) acc[rt][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  for (uint32_t kb = 0; kb < KB; ++kb) {
    v8i bf[4];
    float wsc[4];
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
      bf[c] = nk::load_fp8x32(we + (size_t)nrow[c] * H + kb * 128u + kofs);
      wsc[c] = wse[(nrow[c] >> 7) * KB + kb];
    }
#pragma unroll
    for (uint32_t rt = 0; rt < 4; ++rt) {
      if (rt < ntiles) {
        const v8i af = nk::load_fp8x32(xq + (size_t)arow_tok[rt] * H + kb * 128u + kofs);
        float asc[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) asc[j] = xs[(size_t)srow_tok[rt][j] * KB + kb];
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
          const v4f d = nk::mfma_e4m3_16x16x128(af, bf[c]);
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) acc[rt][c][j] = acc[rt][c][j] + wsc[c] * (asc[j] * d[j]);
        }
      }
    }
  }

  // Epilogue: h = bf16(silu(g) * u); per-row amax over this wave's 32 columns.
  float h[4][2][4];
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt) {
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      float m = 0.0f;
#pragma unroll
      for (uint32_t c = 0; c < 2; ++c) {
        const float v = nk::bf16_f32(nk::bf16_rne(nk::silu(acc[rt][c][j]) * acc[rt][c + 2][j]));
        h[rt][c][j] = v;
        m = fmaxf(m, fabsf(v));
      }
      m = fmaxf(m, __shfl_xor(m, 1u));
      m = fmaxf(m, __shfl_xor(m, 2u));
      m = fmaxf(m, __shfl_xor(m, 4u));
      m = fmaxf(m, __shfl_xor(m, 8u));
      if ((lane & 15u) == 0) s_amax[wave][rt * 16u + (lane >> 4) * 4u + j] = m;
    }
  }
  __syncthreads();
  if (tid < 64u) {
    float m = nk::kAmaxFloor;
#pragma unroll
    for (uint32_t w = 0; w < 4; ++w) m = fmaxf(m, s_amax[w][tid]);
    const float scale = m * nk::inv_e4m3_max();
    s_scale[tid] = scale;
    if (tid < nvalid) hs[(size_t)(b * 64u + tid) * (I / 128u) + ng] = scale;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt) {
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint32_t row = rt * 16u + (lane >> 4) * 4u + j;
      if (row < nvalid) {
        const float inv = 1.0f / s_scale[row];
        uint8_t* dst = hq + (size_t)(b * 64u + row) * I + ng * 128u + wave * 32u + (lane & 15u);
        dst[0] = (uint8_t)nk::e4m3_rne(h[rt][0][j] * inv);
        dst[16] = (uint8_t)nk::e4m3_rne(h[rt][1][j] * inv);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Grouped down GEMM (reference: kernels/gfx950/templates/moe/decode/
// down_reduce_mfma_2wave.inc:14-291; oracle
// tools/benchmark/export_qwen36_moe_stage2_capture.py:90-110).
//
// Workgroup (b, nb): expert block b, output columns [256 nb, 256 nb + 256).
// Wave w owns 64 columns (four 16-column tiles); rows are the block's
// non-empty 16-row tiles of h (already in sorted order, so A loads are
// contiguous). Each valid row writes its fp32 result to partial[route], route
// = token * Ktot + slot; combine applies the top-k weights in slot order.
NK_KERNEL __launch_bounds__(256) void netra_moe_down_gfx950(
    const uint8_t* __restrict__ hq, const float* __restrict__ hs,
    const uint8_t* __restrict__ w2, const float* __restrict__ w2s,
    const int32_t* __restrict__ sorted_ids, const int32_t* __restrict__ sorted_expert,
    const int32_t* __restrict__ num_valid, float* __restrict__ partial, uint32_t T,
    uint32_t H, uint32_t I, uint32_t Ktot, uint32_t Etot) {
  __shared__ int32_t s_route[64];
  const uint32_t b = blockIdx.x, nb = blockIdx.y;
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
  if (b * 64u >= (uint32_t)num_valid[0]) return;
  const int32_t e = sorted_expert[b];
  if (e < 0 || (uint32_t)e >= Etot) return;
  if (tid < 64u) {
    const int32_t id = sorted_ids[b * 64u + tid];
    const uint32_t t = (uint32_t)id & 0xffffffu, slot = (uint32_t)id >> 24;
    s_route[tid] = (t < T && slot < Ktot) ? (int32_t)(t * Ktot + slot) : -1;
  }
  __syncthreads();
  const uint32_t nvalid = (uint32_t)__popcll(__ballot(s_route[lane] >= 0));
  const uint32_t ntiles = (nvalid + 15u) >> 4;
  const uint32_t KB = I / 128u;
  const uint8_t* we = w2 + (size_t)e * H * I;
  const float* wse = w2s + (size_t)e * (H / 128u) * KB;
  const uint32_t kofs = (lane >> 4) * 32u;
  const uint32_t ncol0 = nb * 256u + wave * 64u + (lane & 15u);

  v4f acc[4][4];
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt)
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) acc[rt][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  for (uint32_t kb = 0; kb < KB; ++kb) {
    v8i bf[4];
    float wsc[4];
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
      const uint32_t n = ncol0 + 16u * c;
      bf[c] = nk::load_fp8x32(we + (size_t)n * I + kb * 128u + kofs);
      wsc[c] = wse[(n >> 7) * KB + kb];
    }
#pragma unroll
    for (uint32_t rt = 0; rt < 4; ++rt) {
      if (rt < ntiles) {
        const size_t arow = (size_t)b * 64u + rt * 16u + (lane & 15u);
        const v8i af = nk::load_fp8x32(hq + arow * I + kb * 128u + kofs);
        float asc[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j)
          asc[j] = hs[((size_t)b * 64u + rt * 16u + (lane >> 4) * 4u + j) * KB + kb];
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
          const v4f d = nk::mfma_e4m3_16x16x128(af, bf[c]);
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) acc[rt][c][j] = acc[rt][c][j] + wsc[c] * (asc[j] * d[j]);
        }
      }
    }
  }
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt) {
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint32_t row = rt * 16u + (lane >> 4) * 4u + j;
      if (row < nvalid) {
        float* dst = partial + (size_t)s_route[row] * H + ncol0;
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) dst[16u * c] = acc[rt][c][j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Top-k weighted combine (reference: kernels/gfx950/templates/moe/prefill/
// route_reduce_splitk2_f16.inc:6-117 and down_reduce_mfma_2wave.inc:202-213:
// slot-ordered weighted sum, then bf16). out[t, n] = bf16(sum over slots in
// order of fmaf(w[t, s], partial[t * Ktot + s, n], acc)).
NK_KERNEL __launch_bounds__(256) void netra_moe_combine_gfx950(
    const float* __restrict__ partial, const float* __restrict__ weights,
    uint16_t* __restrict__ out, uint32_t T, uint32_t H, uint32_t Ktot) {
  const uint32_t t = blockIdx.y;
  const uint32_t n = (blockIdx.x * 256u + threadIdx.x) * 4u;
  if (t >= T || n >= H) return;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  for (uint32_t s = 0; s < Ktot; ++s) {
    const float w = weights[(size_t)t * Ktot + s];
    const float4 p = *reinterpret_cast<const float4*>(partial + ((size_t)t * Ktot + s) * H + n);
    a0 = fmaf(w, p.x, a0);
    a1 = fmaf(w, p.y, a1);
    a2 = fmaf(w, p.z, a2);
    a3 = fmaf(w, p.w, a3);
  }
  uint2 o;
  o.x = (uint32_t)nk::bf16_rne(a0) | ((uint32_t)nk::bf16_rne(a1) << 16);
  o.y = (uint32_t)nk::bf16_rne(a2) | ((uint32_t)nk::bf16_rne(a3) << 16);
  *reinterpret_cast<uint2*>(out + (size_t)t * H + n) = o;
}

// ---------------------------------------------------------------------------
// Weight preparation: fp32 [groups, n, k] -> e4m3 + fp32 128x128 block scales
// (scale = max(amax, 1e-10) * 0x3b124925, q = e4m3(w * (1 / scale))); one
// workgroup per 128x128 block (reference recipe: compiler/netra_compiler/
// layouts.py:175-206 plans the scale layout [groups, n/128, k/128]).
NK_KERNEL __launch_bounds__(256) void netra_moe_quant_blocks_gfx950(
    const float* __restrict__ w, uint8_t* __restrict__ q, float* __restrict__ s,
    uint32_t groups, uint32_t n, uint32_t k) {
  __shared__ float s_max[4];
  const uint32_t nb = n / 128u, kb = k / 128u;
  const uint32_t blk = blockIdx.x;
  if (blk >= groups * nb * kb) return;
  const uint32_t g = blk / (nb * kb), bn = (blk / kb) % nb, bk = blk % kb;
  const size_t base = ((size_t)g * n + bn * 128u) * k + bk * 128u;
  const uint32_t tid = threadIdx.x;
  // thread owns column 4*(tid&31)..+3 of rows (tid>>5) + 8 i, i = 0..15
  const uint32_t col = (tid & 31u) * 4u, row0 = tid >> 5;
  float amax = nk::kAmaxFloor;
  for (uint32_t i = 0; i < 16u; ++i) {
    const float4 v = *reinterpret_cast<const float4*>(w + base + (size_t)(row0 + 8u * i) * k + col);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
#pragma unroll
  for (uint32_t off = 1; off < 64; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if ((tid & 63u) == 0) s_max[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
  const float scale = amax * nk::inv_e4m3_max();
  const float inv = 1.0f / scale;
  if (tid == 0) s[blk] = scale;
  for (uint32_t i = 0; i < 16u; ++i) {
    const size_t off = base + (size_t)(row0 + 8u * i) * k + col;
    const float4 v = *reinterpret_cast<const float4*>(w + off);
    const uint32_t packed = nk::e4m3_rne(v.x * inv) | (nk::e4m3_rne(v.y * inv) << 8) |
                            (nk::e4m3_rne(v.z * inv) << 16) | (nk::e4m3_rne(v.w * inv) << 24);
    *reinterpret_cast<uint32_t*>(q + off) = packed;
  }
}
