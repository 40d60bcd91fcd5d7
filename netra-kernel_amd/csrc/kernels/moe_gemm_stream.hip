// Decode-regime grouped GEMMs: wave-level persistent HBM weight streaming.
//
// A work item is one 16-row tile of an expert block (from the sort's tile
// list) times one column tile, over the full K extent. Items are numbered
// tile * col_tiles + col and every wave of a fixed-size grid takes a
// contiguous run of them. An item is streamed in K steps; the routing
// metadata of the next item and the activations and weights of the next step
// are issued before the current step's MFMAs wait, in the order they will be
// consumed, so the in-order load counter never drains the prefetched data.
// Waves never synchronise with each other; per-item values that every lane
// needs (activation scales) go through the wave's own LDS slot.
//
// gate/up writes h = bf16(silu(g) * u) in sorted-row order; a requant kernel
// turns each (16-row tile, 128-column block) into the FP8 operand plus row
// scales once (the SiLU-quant step of the reference's decode trio); down
// streams W2 against it and writes fp32 route partials.
// Symbols: netra_moe_gate_up_stream_h<H>_gfx950, netra_moe_requant_h_gfx950,
// netra_moe_down_stream_i<I>_gfx950.
#pragma once
#include "moe_numerics.h"

#define NK_KERNEL extern "C" __global__

// Resident waves per SIMD the stream kernels are register-budgeted for (the
// engine sizes their grids to match: 256 CUs x 4 SIMDs x this / 4 waves).
#ifndef NK_GATE_UP_WAVES_PER_EU
#define NK_GATE_UP_WAVES_PER_EU 2
#endif
#ifndef NK_DOWN_WAVES_PER_EU
#define NK_DOWN_WAVES_PER_EU 4
#endif

namespace nkstream {

struct Range {
  uint32_t beg, end;
};

__device__ __forceinline__ uint32_t wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// Contiguous run of items owned by the calling wave (uniform values).
__device__ __forceinline__ Range wave_range(uint32_t items) {
  const uint32_t waves = gridDim.x * (blockDim.x >> 6);
  const uint32_t gw = blockIdx.x * (blockDim.x >> 6) + wave_id();
  const uint32_t per = (items + waves - 1u) / waves;
  const uint32_t beg = gw * per;
  const uint32_t end = beg + per < items ? beg + per : items;
  return {beg, beg < items ? end : beg};
}

// Routing metadata of one 16-row tile. row0 and expert are uniform; lane l
// holds row (l & 15): its token (gate/up) or route t * Ktot + slot (down),
// -1 for padding rows.
struct TileRows {
  uint32_t row0 = 0;
  int32_t expert = 0;
  int32_t row = -1;
};

__device__ __forceinline__ void load_tile(TileRows& tr, const int32_t* __restrict__ tile_map,
                                          const int32_t* __restrict__ sorted_ids,
                                          const int32_t* __restrict__ sorted_expert, uint32_t tile,
                                          uint32_t T, uint32_t Ktot, uint32_t Etot, bool as_route) {
  const uint32_t m = (uint32_t)tile_map[tile];
  const uint32_t b = m >> 2;
  tr.row0 = b * 64u + (m & 3u) * 16u;
  const int32_t e = sorted_expert[b];
  tr.expert = (e < 0 || (uint32_t)e >= Etot) ? 0 : e;  // out of range only for malformed routing
  const int32_t id = sorted_ids[tr.row0 + (threadIdx.x & 15u)];
  const uint32_t t = (uint32_t)id & 0xffffffu, slot = (uint32_t)id >> 24;
  tr.row = (t < T && slot < Ktot) ? (int32_t)(as_route ? t * Ktot + slot : t) : -1;
}

}  // namespace nkstream

// ---------------------------------------------------------------------------
// (reference: kernels/gfx950/templates/moe/decode/gate_up_mfma.inc:12-161;
// oracle tools/benchmark/export_qwen36_moe_stage1_capture.py:80-97)
//
// Item (tile, c): h columns [16 c, 16 c + 16) of one 16-row tile, i.e. W13
// rows n (gate) and I + n (up). Steps of kGuChunk 128-wide K blocks; per block
// acc += w_s * (a_s * mfma) (mfma.inc:20-24) in ascending K order. After the
// last step h = bf16_rne(silu(g) * u) for every valid row.
constexpr uint32_t kGuChunk = 2;

struct GateUpStep {
  nk::v8i g[kGuChunk], u[kGuChunk], a[kGuChunk];
  float sg[kGuChunk], su[kGuChunk];
};

template <uint32_t KB>
__device__ __forceinline__ void gate_up_stream(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs,
    const uint8_t* __restrict__ w13, const float* __restrict__ w13s,
    const int32_t* __restrict__ sorted_ids, const int32_t* __restrict__ sorted_expert,
    const int32_t* __restrict__ tile_map, const int32_t* __restrict__ num_valid,
    uint16_t* __restrict__ h, uint32_t T, uint32_t I, uint32_t Ktot, uint32_t Etot) {
  using namespace nkstream;
  constexpr uint32_t H = 128 * KB;
  constexpr uint32_t NCH = KB / kGuChunk;
  constexpr uint32_t SPL = (KB + 3) / 4;  // activation scales per lane per item
  static_assert(KB % (2 * kGuChunk) == 0, "H must be a multiple of 512");
  // Activation scales of the current and next item: [wave][slot][row * KB + kb].
  __shared__ float s_xs[4][2][16 * KB];
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = wave_id();
  const uint32_t kofs = (lane >> 4) * 32u;
  const uint32_t cols = I / 16u;
  const Range r = wave_range((uint32_t)num_valid[2] * cols);
  const uint32_t steps = (r.end - r.beg) * NCH;
  if (steps == 0) return;

  // Lane l fetches row l & 15's scales for K blocks [(l >> 4) * SPL, +SPL).
  auto fetch_meta = [&](TileRows& m, float (&xsv)[SPL], uint32_t item) {
    load_tile(m, tile_map, sorted_ids, sorted_expert, item / cols, T, Ktot, Etot, false);
    const int32_t t = m.row < 0 ? 0 : m.row;
    const uint32_t k0 = (lane >> 4) * SPL;
#pragma unroll
    for (uint32_t i = 0; i < SPL; ++i) xsv[i] = (k0 + i < KB) ? xs[(size_t)t * KB + k0 + i] : 0.0f;
  };
  auto store_scales = [&](const float (&xsv)[SPL], uint32_t slot) {
    const uint32_t k0 = (lane >> 4) * SPL;
#pragma unroll
    for (uint32_t i = 0; i < SPL; ++i)
      if (k0 + i < KB) s_xs[wave][slot][(lane & 15u) * KB + k0 + i] = xsv[i];
  };
  auto issue = [&](GateUpStep& st, const TileRows& m, uint32_t s) {
    const uint32_t item = r.beg + s / NCH, ch = s % NCH;
    const uint32_t c = item % cols;
    const int32_t ta = __shfl(m.row, lane & 15u);
    const uint8_t* arow = xq + (size_t)(ta < 0 ? 0 : ta) * H + kofs;
#pragma unroll
    for (uint32_t i = 0; i < kGuChunk; ++i) st.a[i] = nk::load_fp8x32(arow + (ch * kGuChunk + i) * 128u);
    const uint8_t* we = w13 + (size_t)m.expert * 2u * I * H;
    const float* wse = w13s + (size_t)m.expert * (2u * I / 128u) * KB;
#pragma unroll
    for (uint32_t i = 0; i < kGuChunk; ++i) {
      const uint32_t kb = ch * kGuChunk + i;
      st.g[i] = nk::load_tile_operand(nk::tile_base(we, c, kb, KB), lane);
      st.u[i] = nk::load_tile_operand(nk::tile_base(we, I / 16u + c, kb, KB), lane);
      st.sg[i] = wse[(c >> 3) * KB + kb];                 // 128-row scale block of rows 16c..
      st.su[i] = wse[((I / 16u + c) >> 3) * KB + kb];
    }
  };
  nk::v4f ag = {0.0f, 0.0f, 0.0f, 0.0f}, au = {0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](const GateUpStep& st, const TileRows& m, uint32_t slot, uint32_t s) {
    const uint32_t ch = s % NCH;
#pragma unroll
    for (uint32_t i = 0; i < kGuChunk; ++i) {
      const uint32_t kb = ch * kGuChunk + i;
      const nk::v4f dg = nk::mfma_e4m3_16x16x128(st.a[i], st.g[i]);
      const nk::v4f du = nk::mfma_e4m3_16x16x128(st.a[i], st.u[i]);
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const float as = s_xs[wave][slot][((lane >> 4) * 4u + j) * KB + kb];
        ag[j] = ag[j] + st.sg[i] * (as * dg[j]);
        au[j] = au[j] + st.su[i] * (as * du[j]);
      }
    }
    if (ch == NCH - 1u) {
      const uint32_t c = (r.beg + s / NCH) % cols;
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t row = (lane >> 4) * 4u + j;
        if (__shfl(m.row, row) >= 0)
          h[nk::h_tile_index(m.row0 + row, c * 16u + (lane & 15u), I / 128u)] =
              nk::bf16_rne(nk::silu(ag[j]) * au[j]);
      }
      ag = nk::v4f{0.0f, 0.0f, 0.0f, 0.0f};
      au = nk::v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };

  // Item k (slot k & 1): its metadata and scales were fetched at the start of
  // item k - 1, its scales stored and its first step issued during the last
  // step of item k - 1; inside the item step ch + 1 is issued before step ch
  // computes.
  GateUpStep sx, sy;
  TileRows ma, mb;
  float xa[SPL], xb[SPL];
  auto item_body = [&](uint32_t k, const TileRows& cur, uint32_t slot, TileRows& nxt,
                       float (&xnxt)[SPL]) {
    const bool more = k + 1u < r.end;
    if (more) fetch_meta(nxt, xnxt, k + 1u);
#pragma unroll 1
    for (uint32_t ch = 0; ch < NCH; ch += 2u) {
      const uint32_t s = (k - r.beg) * NCH + ch;
      issue(sy, cur, s + 1u);
      compute(sx, cur, slot, s);
      if (ch + 2u < NCH) {
        issue(sx, cur, s + 2u);
      } else if (more) {
        store_scales(xnxt, slot ^ 1u);
        issue(sx, nxt, s + 2u);
      }
      compute(sy, cur, slot, s + 1u);
    }
  };
  fetch_meta(ma, xa, r.beg);
  store_scales(xa, 0u);
  issue(sx, ma, 0);
  for (uint32_t k = r.beg; k < r.end; k += 2u) {
    item_body(k, ma, 0u, mb, xb);
    if (k + 1u < r.end) item_body(k + 1u, mb, 1u, ma, xa);
  }
}

#define NK_GATE_UP_STREAM_V(NAME, HV, WPE)                                                       \
  NK_KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE)))                     \
  void NAME(                                                                                     \
      const uint8_t* __restrict__ xq, const float* __restrict__ xs,                              \
      const uint8_t* __restrict__ w13, const float* __restrict__ w13s,                           \
      const int32_t* __restrict__ sorted_ids, const int32_t* __restrict__ sorted_expert,         \
      const int32_t* __restrict__ tile_map, const int32_t* __restrict__ num_valid,               \
      uint16_t* __restrict__ h, uint32_t T, uint32_t H, uint32_t I, uint32_t Ktot,               \
      uint32_t Etot) {                                                                           \
    (void)H;                                                                                     \
    gate_up_stream<HV / 128>(xq, xs, w13, w13s, sorted_ids, sorted_expert, tile_map, num_valid, \
                             h, T, I, Ktot, Etot);                                               \
  }
#define NK_GATE_UP_STREAM(HV) \
  NK_GATE_UP_STREAM_V(netra_moe_gate_up_stream_h##HV##_gfx950, HV, NK_GATE_UP_WAVES_PER_EU)
NK_GATE_UP_STREAM(512)
NK_GATE_UP_STREAM(1024)
NK_GATE_UP_STREAM(2048)
NK_GATE_UP_STREAM(4096)
// occupancy alternatives kept for tuning runs
NK_GATE_UP_STREAM_V(netra_moe_gate_up_stream_h2048_o3_gfx950, 2048, 3)
NK_GATE_UP_STREAM_V(netra_moe_gate_up_stream_h2048_o4_gfx950, 2048, 4)

// ---------------------------------------------------------------------------
// 1x128 FP8 requant of h between the decode GEMMs (reference: kernels/gfx950/
// templates/moe/decode/silu_quant.inc:16-236; rule of harness/gfx950/fp8/moe/
// decode/qwen36_moe_silu_mul_quant_fp8_gfx950.hip:57-94).
//
// One wave per (16-row tile, 128-column block), persistent over the sort's
// tile list: lane l holds 32 bf16 of row l & 15 (columns (l >> 4) * 32 .. +31
// of the block); the four lanes of a row combine their maxima, scale =
// max(amax, 1e-10) * 0x3b124925, q = e4m3(h * (1 / scale)). The FP8 tile is
// written in the tile16x128 operand layout (lo half at l * 16, hi half at
// 1024 + l * 16) and the 16 row scales of the (tile, block) contiguously, so
// the down GEMM loads its A operand and scales without further arithmetic.
NK_KERNEL __launch_bounds__(256) void netra_moe_requant_h_gfx950(
    const uint16_t* __restrict__ h, uint8_t* __restrict__ hq, float* __restrict__ hs,
    const int32_t* __restrict__ tile_map, const int32_t* __restrict__ num_valid, uint32_t I) {
  using namespace nkstream;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t KB = I / 128u;
  const Range r = wave_range((uint32_t)num_valid[2] * KB);
  for (uint32_t item = r.beg; item < r.end; ++item) {
    const uint32_t ti = item / KB, kb = item - ti * KB;
    const uint32_t m = (uint32_t)tile_map[ti];
    const uint32_t tile = (m >> 2) * 4u + (m & 3u);  // 16-row tile index in sorted order
    const size_t blk = (size_t)tile * KB + kb;
    const uint4* src = reinterpret_cast<const uint4*>(h + blk * 2048u) + lane;
    uint4 raw[4];
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) raw[q] = src[q * 64u];
    float f[32];
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
      f[8 * q + 0] = nk::bf16_lo(raw[q].x); f[8 * q + 1] = nk::bf16_hi(raw[q].x);
      f[8 * q + 2] = nk::bf16_lo(raw[q].y); f[8 * q + 3] = nk::bf16_hi(raw[q].y);
      f[8 * q + 4] = nk::bf16_lo(raw[q].z); f[8 * q + 5] = nk::bf16_hi(raw[q].z);
      f[8 * q + 6] = nk::bf16_lo(raw[q].w); f[8 * q + 7] = nk::bf16_hi(raw[q].w);
    }
    float amax = nk::kAmaxFloor;
#pragma unroll
    for (uint32_t q = 0; q < 32; ++q) amax = fmaxf(amax, fabsf(f[q]));
    amax = fmaxf(amax, __shfl_xor(amax, 16u));
    amax = fmaxf(amax, __shfl_xor(amax, 32u));
    const float scale = amax * nk::inv_e4m3_max();
    const float inv = 1.0f / scale;
    uint4 lo, hi;
    lo.x = nk::e4m3x4(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv);
    lo.y = nk::e4m3x4(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv);
    lo.z = nk::e4m3x4(f[8] * inv, f[9] * inv, f[10] * inv, f[11] * inv);
    lo.w = nk::e4m3x4(f[12] * inv, f[13] * inv, f[14] * inv, f[15] * inv);
    hi.x = nk::e4m3x4(f[16] * inv, f[17] * inv, f[18] * inv, f[19] * inv);
    hi.y = nk::e4m3x4(f[20] * inv, f[21] * inv, f[22] * inv, f[23] * inv);
    hi.z = nk::e4m3x4(f[24] * inv, f[25] * inv, f[26] * inv, f[27] * inv);
    hi.w = nk::e4m3x4(f[28] * inv, f[29] * inv, f[30] * inv, f[31] * inv);
    uint8_t* dst = hq + blk * 2048u;
    *reinterpret_cast<uint4*>(dst + lane * 16u) = lo;
    *reinterpret_cast<uint4*>(dst + 1024u + lane * 16u) = hi;
    if (lane < 16u) hs[blk * 16u + lane] = scale;
  }
}

// ---------------------------------------------------------------------------
// (reference: kernels/gfx950/templates/moe/decode/down_reduce_mfma_2wave.inc:
// 14-291; oracle tools/benchmark/export_qwen36_moe_stage2_capture.py:90-110)
//
// Item (tile, c): output columns [32 c, 32 c + 32) (two 16-column tiles) of one
// 16-row tile; one 128-wide K block per step. The A operand is the requantised
// FP8 tile and its row scales (netra_moe_requant_h_gfx950); per block
// acc += w_s * (a_s * mfma). After the last step each valid row's fp32 result
// goes to partial[route].
struct DownStep {
  nk::v8i a;
  float4 as;
  nk::v8i w[2];
  float s[2];
};

template <uint32_t KB>
__device__ __forceinline__ void down_stream(
    const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2,
    const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ tile_map,
    const int32_t* __restrict__ num_valid, float* __restrict__ partial, uint32_t T, uint32_t H,
    uint32_t Ktot, uint32_t Etot) {
  using namespace nkstream;
  constexpr uint32_t I = 128 * KB;
  constexpr uint32_t NCH = KB;
  static_assert(NCH % 2 == 0, "I must be a multiple of 256");
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t cols = H / 32u;
  const Range r = wave_range((uint32_t)num_valid[2] * cols);
  const uint32_t steps = (r.end - r.beg) * NCH;
  if (steps == 0) return;

  auto fetch_meta = [&](TileRows& m, uint32_t item) {
    load_tile(m, tile_map, sorted_ids, sorted_expert, item / cols, T, Ktot, Etot, true);
  };
  auto issue = [&](DownStep& st, const TileRows& m, uint32_t s) {
    const uint32_t item = r.beg + s / NCH, kb = s % NCH;
    const uint32_t c = item % cols;
    const size_t blk = (size_t)(m.row0 >> 4) * KB + kb;
    st.a = nk::load_tile_operand(hq + blk * 2048u, lane);
    st.as = *reinterpret_cast<const float4*>(hs + blk * 16u + (lane >> 4) * 4u);
    const uint8_t* we = w2 + (size_t)m.expert * H * I;
    const float* wse = w2s + (size_t)m.expert * (H / 128u) * KB;
#pragma unroll
    for (uint32_t t2 = 0; t2 < 2; ++t2) {
      st.w[t2] = nk::load_tile_operand(nk::tile_base(we, c * 2u + t2, kb, KB), lane);
      st.s[t2] = wse[((c * 2u + t2) >> 3) * KB + kb];   // 128-row scale block of the tile
    }
  };
  nk::v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](const DownStep& st, const TileRows& m, uint32_t s) {
    const float as[4] = {st.as.x, st.as.y, st.as.z, st.as.w};
    const nk::v4f d0 = nk::mfma_e4m3_16x16x128(st.a, st.w[0]);
    const nk::v4f d1 = nk::mfma_e4m3_16x16x128(st.a, st.w[1]);
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      acc0[j] = acc0[j] + st.s[0] * (as[j] * d0[j]);
      acc1[j] = acc1[j] + st.s[1] * (as[j] * d1[j]);
    }
    if (s % NCH == NCH - 1u) {
      const uint32_t c = (r.beg + s / NCH) % cols;
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const int32_t route = __shfl(m.row, (lane >> 4) * 4u + j);
        if (route >= 0) {
          float* dst = partial + (size_t)route * H + c * 32u + (lane & 15u);
          dst[0] = acc0[j];
          dst[16] = acc1[j];
        }
      }
      acc0 = nk::v4f{0.0f, 0.0f, 0.0f, 0.0f};
      acc1 = nk::v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };

  DownStep sx, sy;
  TileRows ma, mb;
  auto item_body = [&](uint32_t k, const TileRows& cur, TileRows& nxt) {
    if (k + 1u < r.end) fetch_meta(nxt, k + 1u);
#pragma unroll 1
    for (uint32_t ch = 0; ch < NCH; ch += 2u) {
      const uint32_t s = (k - r.beg) * NCH + ch;
      issue(sy, cur, s + 1u);
      compute(sx, cur, s);
      if (ch + 2u < NCH) issue(sx, cur, s + 2u);
      else if (k + 1u < r.end) issue(sx, nxt, s + 2u);
      compute(sy, cur, s + 1u);
    }
  };
  fetch_meta(ma, r.beg);
  issue(sx, ma, 0);
  for (uint32_t k = r.beg; k < r.end; k += 2u) {
    item_body(k, ma, mb);
    if (k + 1u < r.end) item_body(k + 1u, mb, ma);
  }
}

#define NK_DOWN_STREAM_V(NAME, IV, WPE)                                                         \
  NK_KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE)))                     \
  void NAME(                                                                                    \
      const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2, \
      const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,                    \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ tile_map,          \
      const int32_t* __restrict__ num_valid, float* __restrict__ partial, uint32_t T,           \
      uint32_t H, uint32_t I, uint32_t Ktot, uint32_t Etot) {                                   \
    (void)I;                                                                                    \
    down_stream<IV / 128>(hq, hs, w2, w2s, sorted_ids, sorted_expert, tile_map, num_valid,      \
                          partial, T, H, Ktot, Etot);                                           \
  }
#define NK_DOWN_STREAM(IV) NK_DOWN_STREAM_V(netra_moe_down_stream_i##IV##_gfx950, IV, NK_DOWN_WAVES_PER_EU)
NK_DOWN_STREAM(256)
NK_DOWN_STREAM(512)
NK_DOWN_STREAM(1024)
NK_DOWN_STREAM(2048)
// occupancy alternatives kept for tuning runs
NK_DOWN_STREAM_V(netra_moe_down_stream_i512_o6_gfx950, 512, 6)
NK_DOWN_STREAM_V(netra_moe_down_stream_i512_o8_gfx950, 512, 8)
