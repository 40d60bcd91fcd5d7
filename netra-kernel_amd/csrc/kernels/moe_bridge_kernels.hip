// Kernels behind the reference's per-operation bridge ABIs (the decode trio,
// the shared-gate append and the M768 prefill producer/reducer pair), in the
// argument formats those bridges exchange with their callers:
//
//   netra_moe_shared_gate_append_h<H>_gfx950   routed top-k + sigmoid shared gate -> K + 1 slots
//   netra_moe_gate_up_route_h<H>_gfx950        per-route gate/up, fp32 [routes, 2I] out, AITER W13
//   netra_moe_silu_mul_quant_gfx950            fp32 [rows, 2I] -> h e4m3 [rows, I] + 1x128 scales
//   netra_moe_down_reduce_route_i<I>_gfx950    per-token down + slot-ordered reduce, AITER W2, bf16 out
//   netra_moe_block_pairs_gfx950               AITER sorted expert blocks -> block pairs + counts
//   netra_moe_route_reduce_f16x2_gfx950        split-K2 fp16 route partials -> bf16 out
//
// (The router bridge uses netra_moe_router_h<H>_t<NT>_gfx950 with null
// quantisation outputs; the M768 producer uses netra_moe_gate_up_lds_aiter_h<H>
// and netra_moe_down_rows_aiter_f16x2_i<I>.)
//
// The decode kernels are the M = 1 shape of the reference's decode bridges:
// one route (gate/up) or one token (down) per workgroup, every weight tile
// streamed once per route, no sort. Their GEMM outputs are fp32/bf16 and
// checked against the oracle within a tolerance; the shared-gate append and
// the SiLU-quant follow the layer's exact numeric contract (bit-exact).
#pragma once
#include "moe_numerics.h"

#define NK_KERNEL extern "C" __global__

namespace nkbridge {

using nk::v4f;
using nk::v8i;

// Row 0 of an MFMA A operand from one FP8 row (32 bytes per lane of rows
// 0..15 at K bytes (lane >> 4) * 32); the other 15 rows are zero.
__device__ __forceinline__ v8i single_row_operand(const uint8_t* row_kb, uint32_t lane) {
  if ((lane & 15u) != 0u) return v8i{0, 0, 0, 0, 0, 0, 0, 0};
  return nk::load_fp8x32(row_kb + (lane >> 4) * 32u);
}

// ---------------------------------------------------------------------------
// Shared-expert gate + append (reference: runtime/gfx950/routing/decode/
// qwen36_shared_gate_append_bridge.hip:76-112; semantics tools/benchmark/
// export_qwen36_shared_gate_append_capture.py:97-107,134-139).
//
// One wave per token. The gate logit is the layer's router contract dot
// product (16 slices, slice s owning elements 128 j + 8 s + i, each a
// sequential fmaf chain from +0 in (j, i) order, folded +8, +4, +2, +1,
// bf16 RNE), the weight f32(bf16(sigmoid(f32(logit)))). Output slots 0..K-1
// copy the routed ids and weights, slot K holds expert id E and the gate
// weight.
template <uint32_t NJ>  // H / 128
__device__ __forceinline__ void shared_gate_append(int32_t* __restrict__ out_ids, float* __restrict__ out_w,
                                                   const uint16_t* __restrict__ x,
                                                   const uint16_t* __restrict__ wsg,
                                                   const int32_t* __restrict__ ids,
                                                   const float* __restrict__ w, uint32_t T, uint32_t E,
                                                   uint32_t K) {
  constexpr uint32_t H = 128u * NJ;
  const uint32_t t = blockIdx.x, lane = threadIdx.x;
  if (t >= T) return;
  if (lane < K) {
    out_ids[(size_t)t * (K + 1u) + lane] = ids[(size_t)t * K + lane];
    out_w[(size_t)t * (K + 1u) + lane] = w[(size_t)t * K + lane];
  }
  const uint32_t s = lane & 15u;
  float a = 0.0f;
  if (lane < 16u) {
    const uint16_t* xr = x + (size_t)t * H + 8u * s;
    const uint16_t* wr = wsg + 8u * s;
#pragma unroll
    for (uint32_t j = 0; j < NJ; ++j) {
      const uint4 xv = *reinterpret_cast<const uint4*>(xr + 128u * j);
      const uint4 wv = *reinterpret_cast<const uint4*>(wr + 128u * j);
      a = fmaf(nk::bf16_lo(xv.x), nk::bf16_lo(wv.x), a);
      a = fmaf(nk::bf16_hi(xv.x), nk::bf16_hi(wv.x), a);
      a = fmaf(nk::bf16_lo(xv.y), nk::bf16_lo(wv.y), a);
      a = fmaf(nk::bf16_hi(xv.y), nk::bf16_hi(wv.y), a);
      a = fmaf(nk::bf16_lo(xv.z), nk::bf16_lo(wv.z), a);
      a = fmaf(nk::bf16_hi(xv.z), nk::bf16_hi(wv.z), a);
      a = fmaf(nk::bf16_lo(xv.w), nk::bf16_lo(wv.w), a);
      a = fmaf(nk::bf16_hi(xv.w), nk::bf16_hi(wv.w), a);
    }
  }
  a = a + __shfl_down(a, 8u, 16);
  a = a + __shfl_down(a, 4u, 16);
  a = a + __shfl_down(a, 2u, 16);
  a = a + __shfl_down(a, 1u, 16);
  if (lane == 0u) {
    const float logit = nk::bf16_f32(nk::bf16_rne(a));
    out_ids[(size_t)t * (K + 1u) + K] = (int32_t)E;
    out_w[(size_t)t * (K + 1u) + K] = nk::bf16_f32(nk::bf16_rne(nk::sigmoid(logit)));
  }
}

// ---------------------------------------------------------------------------
// Per-route gate/up, fp32 out (reference: kernels/gfx950/templates/moe/decode/
// gate_up_mfma.inc:12-161 behind qwen36_moe_silu_mul_quant_bridge.h:50-60;
// oracle tools/benchmark/export_qwen36_moe_stage1_capture.py:80-97).
//
// Workgroup (c, r): route r = t * Ktot + slot, h columns 16 c .. 16 c + 15 of
// gate (W13 rows 16 c..) and up (rows I + 16 c..). W13 is in the AITER layout
// the reference consumes, gate row tiles 0..I/16-1 then up row tiles. The four
// waves split K into quarters and issue every weight load of their quarter at
// once; row 0 of the MFMA A operand is the route's token row. Per 128-K block
// acc += w_s * (a_s * mfma); the quarters are added in order through LDS.
// out[r, n] = g (n < I), out[r, I + n] = u.
template <uint32_t KB>  // H / 128
__device__ __forceinline__ void gate_up_route(const uint8_t* __restrict__ xq, const float* __restrict__ xs,
                                              const uint8_t* __restrict__ w13, const float* __restrict__ w13s,
                                              const int32_t* __restrict__ ids, float* __restrict__ out,
                                              uint32_t I, uint32_t Ktot, uint32_t Etot) {
  constexpr uint32_t H = 128u * KB;
  constexpr uint32_t kWaves = 4, KPW = KB / kWaves;
  static_assert(KB % kWaves == 0, "K quarters");
  __shared__ float s_p[kWaves][2][16];
  const uint32_t c = blockIdx.x, r = blockIdx.y, t = r / Ktot;
  const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int32_t e = ids[r];
  const bool ok = e >= 0 && (uint32_t)e < Etot;
  float pg = 0.0f, pu = 0.0f;
  if (ok) {  // uniform
    const uint8_t* w13e = w13 + (size_t)e * 2u * I * H;
    const float* wse = w13s + (size_t)e * (2u * I / 128u) * KB;
    const uint8_t* xrow = xq + (size_t)t * H;
    v8i g[KPW], u[KPW], a[KPW];
#pragma unroll
    for (uint32_t i = 0; i < KPW; ++i) {
      const uint32_t kb = wave * KPW + i;
      g[i] = nk::load_block_operand<true>(nk::tile_base(w13e, c, kb, KB), lane);
      u[i] = nk::load_block_operand<true>(nk::tile_base(w13e, I / 16u + c, kb, KB), lane);
      a[i] = single_row_operand(xrow + kb * 128u, lane);
    }
#pragma unroll
    for (uint32_t i = 0; i < KPW; ++i) {
      const uint32_t kb = wave * KPW + i;
      const float as = xs[(size_t)t * KB + kb];
      const float sg = wse[(c >> 3) * KB + kb], su = wse[(I / 128u + (c >> 3)) * KB + kb];
      const v4f dg = nk::mfma_e4m3_16x16x128(a[i], g[i]);
      const v4f du = nk::mfma_e4m3_16x16x128(a[i], u[i]);
      pg = pg + sg * (as * dg[0]);
      pu = pu + su * (as * du[0]);
    }
  }
  if (lane < 16u) {
    s_p[wave][0][lane] = pg;
    s_p[wave][1][lane] = pu;
  }
  __syncthreads();
  if (wave == 0u && lane < 16u) {
    float gs = s_p[0][0][lane], us = s_p[0][1][lane];
#pragma unroll
    for (uint32_t q = 1; q < kWaves; ++q) {
      gs = gs + s_p[q][0][lane];
      us = us + s_p[q][1][lane];
    }
    out[(size_t)r * 2u * I + 16u * c + lane] = gs;
    out[(size_t)r * 2u * I + I + 16u * c + lane] = us;
  }
}

// ---------------------------------------------------------------------------
// SiLU.mul + 1x128 FP8 requant of fp32 gate/up rows (reference: kernels/
// gfx950/templates/moe/decode/silu_quant.inc:16-236 behind
// qwen36_moe_silu_mul_quant_bridge.h:14-29; rule harness/gfx950/fp8/moe/
// decode/qwen36_moe_silu_mul_quant_fp8_gfx950.hip:41-94).
//
// Four waves per row of [g (I values) | u (I values)]: h = bf16(silu(g) * u)
// with the contract exp, amax per 128 columns (floor 1e-10), scale = amax *
// 0x3b124925, q = e4m3(h * (1 / scale)). Wave w takes 128-column blocks w,
// w + 4, ..; lane l two consecutive columns of a block, so a block's amax is
// one wave reduction and each lane evaluates two SiLUs (the per-value
// arithmetic does not depend on the mapping).
constexpr uint32_t kSiluWaves = 4;
__device__ __forceinline__ void silu_mul_quant(const float* __restrict__ in, uint8_t* __restrict__ q,
                                               float* __restrict__ s, uint32_t rows, uint32_t I) {
  const uint32_t row = blockIdx.x, lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  if (row >= rows) return;
  const float* g = in + (size_t)row * 2u * I;
  const float* u = g + I;
  for (uint32_t blk = wave; blk < I / 128u; blk += kSiluWaves) {
    const uint32_t n0 = blk * 128u + lane * 2u;
    const float2 gv = *reinterpret_cast<const float2*>(g + n0), uv = *reinterpret_cast<const float2*>(u + n0);
    const float h0 = nk::bf16_f32(nk::bf16_rne(nk::silu(gv.x) * uv.x));
    const float h1 = nk::bf16_f32(nk::bf16_rne(nk::silu(gv.y) * uv.y));
    float amax = fmaxf(nk::kAmaxFloor, fmaxf(fabsf(h0), fabsf(h1)));
#pragma unroll
    for (uint32_t m = 1; m < 64u; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
    const float scale = amax * nk::inv_e4m3_max();
    const float inv = 1.0f / scale;
    const uint32_t qq = nk::e4m3x4(h0 * inv, h1 * inv, 0.0f, 0.0f);
    *reinterpret_cast<uint16_t*>(q + (size_t)row * I + n0) = (uint16_t)(qq & 0xffffu);
    if (lane == 0u) s[(size_t)row * (I / 128u) + blk] = scale;
  }
}

// ---------------------------------------------------------------------------
// Per-token down + top-k weighted reduce (reference: kernels/gfx950/templates/
// moe/decode/down_reduce_mfma_2wave.inc:14-291 behind
// qwen36_moe_silu_mul_quant_bridge.h:31-48; oracle tools/benchmark/
// export_qwen36_moe_stage2_capture.py:90-110,151-155).
//
// Workgroup (c, t): output columns 16 c .. 16 c + 15 of token t, one wave per
// slot s (Ktot waves): route r = t * Ktot + s against W2 row tile c of expert
// ids[r] (AITER layout), every K block's weight load issued at once; per
// 128-K block acc += w_s * (a_s * mfma). The slots' partials meet in LDS and
// are summed in slot order, out = bf16(fmaf(w_s, p_s, acc)) from acc = 0 (the
// order of netra_moe_combine_gfx950). A slot whose expert id is out of range
// contributes zero.
template <uint32_t KB>  // I / 128
__device__ __forceinline__ void down_reduce_route(const uint8_t* __restrict__ hq, const float* __restrict__ hs,
                                                  const uint8_t* __restrict__ w2, const float* __restrict__ w2s,
                                                  const float* __restrict__ weights,
                                                  const int32_t* __restrict__ ids, uint16_t* __restrict__ out,
                                                  uint32_t H, uint32_t Ktot, uint32_t Etot) {
  constexpr uint32_t I = 128u * KB;
  __shared__ float s_p[16][16];
  const uint32_t c = blockIdx.x, t = blockIdx.y;
  const uint32_t lane = threadIdx.x & 63u, s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t r = t * Ktot + s;
  const int32_t e = ids[r];
  float acc = 0.0f;
  if (e >= 0 && (uint32_t)e < Etot) {  // uniform
    const uint8_t* w2e = w2 + (size_t)e * H * I;
    const float* wse = w2s + (size_t)e * (H / 128u) * KB;
    const uint8_t* hrow = hq + (size_t)r * I;
    v8i b[KB], a[KB];
#pragma unroll
    for (uint32_t kb = 0; kb < KB; ++kb) {
      b[kb] = nk::load_block_operand<true>(nk::tile_base(w2e, c, kb, KB), lane);
      a[kb] = single_row_operand(hrow + kb * 128u, lane);
    }
#pragma unroll
    for (uint32_t kb = 0; kb < KB; ++kb) {
      const v4f d = nk::mfma_e4m3_16x16x128(a[kb], b[kb]);
      acc = acc + wse[(c >> 3) * KB + kb] * (hs[(size_t)r * KB + kb] * d[0]);
    }
  }
  if (lane < 16u) s_p[s][lane] = acc;
  __syncthreads();
  if (s == 0u && lane < 16u) {
    float y = 0.0f;
    for (uint32_t q = 0; q < Ktot; ++q) y = fmaf(weights[(size_t)t * Ktot + q], s_p[q][lane], y);
    out[(size_t)t * H + 16u * c + lane] = nk::bf16_rne(y);
  }
}

}  // namespace nkbridge

// ---------------------------------------------------------------------------
// Block pairs of an AITER-sorted routing (the format of entry_routing.inc:
// 27-112: 64-row blocks, an expert's blocks consecutive, sorted_expert_ids per
// block, num_valid_ids[0] = padded rows). pair_map[i] = first block of the
// i-th pair of consecutive blocks of one expert (an expert's last block may
// stand alone); counts = {padded rows, 0, 0, pairs}. One workgroup, one
// thread per block; blocks beyond the capacity are ignored.
NK_KERNEL __launch_bounds__(1024) void netra_moe_block_pairs_gfx950(
    const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid_ids,
    int32_t* __restrict__ pair_map, int32_t* __restrict__ counts, uint32_t cap_blocks) {
  __shared__ uint32_t s_sum[1024];
  const uint32_t b = threadIdx.x;
  const int32_t rows_in = num_valid_ids[0];
  const uint32_t nb_in = rows_in > 0 ? (uint32_t)rows_in / 64u : 0u;
  const uint32_t nblocks = nb_in < cap_blocks ? nb_in : cap_blocks;
  bool start = false;
  if (b < nblocks) {
    const int32_t e = sorted_expert[b];
    uint32_t run0 = b;  // first block of this expert's run
    while (run0 > 0u && sorted_expert[run0 - 1u] == e) --run0;
    start = ((b - run0) & 1u) == 0u;
  }
  s_sum[b] = start ? 1u : 0u;
  __syncthreads();
  for (uint32_t d = 1; d < 1024u; d <<= 1) {  // inclusive scan (Hillis-Steele)
    const uint32_t v = b >= d ? s_sum[b - d] : 0u;
    __syncthreads();
    s_sum[b] += v;
    __syncthreads();
  }
  if (start) pair_map[s_sum[b] - 1u] = (int32_t)b;
  if (b == 0u) {
    counts[0] = (int32_t)(nblocks * 64u);
    counts[1] = 0;
    counts[2] = 0;
    counts[3] = (int32_t)s_sum[1023];
  }
}

// ---------------------------------------------------------------------------
// Split-K2 fp16 route reducer (reference: kernels/gfx950/templates/moe/
// prefill/route_reduce_splitk2_f16.inc:6-117, semantics
// "sum_halves_then_weight_topk_slot_ascending_fp32_rne_bf16",
// manifests/gfx950/models/qwen36-35b-c64-fp8.json:97).
// out[t, n] = bf16(sum over slots in order of w[t, s] * (p0 + p1)), with
// p_h = f32(partial_h[t * Ktot + s, n]), the product and the sum rounded
// separately (multiply, then add; the first slot starts the sum). Eight
// columns per thread.
NK_KERNEL __launch_bounds__(256) void netra_moe_route_reduce_f16x2_gfx950(
    const uint16_t* __restrict__ partials, const float* __restrict__ weights, uint16_t* __restrict__ out,
    uint32_t T, uint32_t H, uint32_t Ktot, uint32_t half_rows) {
  const uint32_t t = blockIdx.y, n = (blockIdx.x * 256u + threadIdx.x) * 8u;
  if (t >= T || n >= H) return;
  const uint16_t* p0 = partials + (size_t)t * Ktot * H + n;
  const uint16_t* p1 = p0 + (size_t)half_rows * H;
  float acc[8];
  for (uint32_t s = 0; s < Ktot; ++s) {
    const uint4 a = *reinterpret_cast<const uint4*>(p0 + (size_t)s * H);
    const uint4 b = *reinterpret_cast<const uint4*>(p1 + (size_t)s * H);
    const float w = weights[(size_t)t * Ktot + s];
    const uint32_t av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      const uint16_t ha = (uint16_t)(av[i >> 1] >> (16u * (i & 1u)));
      const uint16_t hb = (uint16_t)(bv[i >> 1] >> (16u * (i & 1u)));
      const float v = (float)__builtin_bit_cast(_Float16, ha) + (float)__builtin_bit_cast(_Float16, hb);
      const float term = w * v;
      acc[i] = s == 0u ? term : acc[i] + term;
    }
  }
  uint4 o;
  o.x = (uint32_t)nk::bf16_rne(acc[0]) | ((uint32_t)nk::bf16_rne(acc[1]) << 16);
  o.y = (uint32_t)nk::bf16_rne(acc[2]) | ((uint32_t)nk::bf16_rne(acc[3]) << 16);
  o.z = (uint32_t)nk::bf16_rne(acc[4]) | ((uint32_t)nk::bf16_rne(acc[5]) << 16);
  o.w = (uint32_t)nk::bf16_rne(acc[6]) | ((uint32_t)nk::bf16_rne(acc[7]) << 16);
  *reinterpret_cast<uint4*>(out + (size_t)t * H + n) = o;
}

#define NK_SHARED_GATE_APPEND(HV)                                                                  \
  NK_KERNEL __launch_bounds__(64) void netra_moe_shared_gate_append_h##HV##_gfx950(                \
      int32_t* __restrict__ out_ids, float* __restrict__ out_w, const uint16_t* __restrict__ x,    \
      const uint16_t* __restrict__ wsg, const int32_t* __restrict__ ids, const float* __restrict__ w, \
      uint32_t T, uint32_t H, uint32_t E, uint32_t K) {                                            \
    (void)H;                                                                                       \
    nkbridge::shared_gate_append<HV / 128>(out_ids, out_w, x, wsg, ids, w, T, E, K);               \
  }
NK_SHARED_GATE_APPEND(2048)

#define NK_GATE_UP_ROUTE(HV)                                                                       \
  NK_KERNEL __launch_bounds__(256) void netra_moe_gate_up_route_h##HV##_gfx950(                    \
      const uint8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ w13, \
      const float* __restrict__ w13s, const int32_t* __restrict__ ids, float* __restrict__ out,    \
      uint32_t T, uint32_t H, uint32_t I, uint32_t Ktot, uint32_t Etot) {                          \
    (void)T;                                                                                       \
    (void)H;                                                                                       \
    nkbridge::gate_up_route<HV / 128>(xq, xs, w13, w13s, ids, out, I, Ktot, Etot);                 \
  }
NK_GATE_UP_ROUTE(2048)

NK_KERNEL __launch_bounds__(256) void netra_moe_silu_mul_quant_gfx950(const float* __restrict__ in,
                                                                     uint8_t* __restrict__ q,
                                                                     float* __restrict__ s, uint32_t rows,
                                                                     uint32_t I) {
  nkbridge::silu_mul_quant(in, q, s, rows, I);
}

#define NK_DOWN_REDUCE_ROUTE(IV)                                                                   \
  NK_KERNEL __launch_bounds__(1024) void netra_moe_down_reduce_route_i##IV##_gfx950(               \
      const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2, \
      const float* __restrict__ w2s, const float* __restrict__ weights,                            \
      const int32_t* __restrict__ ids, uint16_t* __restrict__ out, uint32_t T, uint32_t H,         \
      uint32_t I, uint32_t Ktot, uint32_t Etot) {                                                  \
    (void)T;                                                                                       \
    (void)I;                                                                                       \
    nkbridge::down_reduce_route<IV / 128>(hq, hs, w2, w2s, weights, ids, out, H, Ktot, Etot);      \
  }
NK_DOWN_REDUCE_ROUTE(512)
