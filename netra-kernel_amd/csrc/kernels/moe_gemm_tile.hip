// Tile-regime grouped GEMMs (prefill-sized T): one workgroup per (64-row
// expert block, column group), SiLU.mul + 1x128 FP8 requant fused into the
// gate/up epilogue, bf16 route partials out of the down GEMM.
//
// Both kernels stage the block's activation rows in LDS once per workgroup
// (the four waves share them), prefetch the next 128-K block of weight
// operands while the current one is multiplied, and synchronise through LDS-only barriers so the weight
// prefetch is never drained. Work items are assigned XCD-major: the hardware
// hands consecutive workgroup ids to the eight XCDs in turn, so workgroup i
// takes item (i % 8) * per + i / 8 and each XCD walks a contiguous range of
// (block, column group) items; the blocks of one expert then read its weights
// through the same L2.
#pragma once
#include <type_traits>

#include "moe_numerics.h"

#define NK_KERNEL extern "C" __global__

namespace nktile {

using nk::v4f;
using nk::v8i;

constexpr uint32_t kRows = 64;  // rows per expert block

// Barrier for LDS hand-off only: waits for this wave's LDS traffic, not for
// its outstanding global loads (a full __syncthreads also waits for those).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Item of workgroup i among n items, XCD-major; false when i has none.
__device__ __forceinline__ bool xcd_item(uint32_t i, uint32_t n, uint32_t& item) {
  const uint32_t per = (n + 7u) / 8u;
  item = (i % 8u) * per + i / 8u;
  return i / 8u < per && item < n;
}

__device__ __forceinline__ v8i lds_fp8x32(const uint8_t* p) {
  const uint4 lo = *reinterpret_cast<const uint4*>(p);
  const uint4 hi = *reinterpret_cast<const uint4*>(p + 16);
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}

// ---------------------------------------------------------------------------
// Grouped gate/up GEMM + SiLU.mul + 1x128 FP8 requant
// (reference: kernels/gfx950/templates/moe/decode/gate_up_mfma.inc:12-161 and
// silu_quant.inc:16-236; oracle tools/benchmark/export_qwen36_moe_stage1_capture.py:80-97).
//
// Item (b, ng): expert block b, h columns [128 ng, 128 ng + 128). Wave w owns
// h columns 32 w .. 32 w + 31: W13 rows n and n + 16 (gate) and I + n,
// I + n + 16 (up), against the block's non-empty 16-row tiles. Per 128-K
// block: acc += (w_s * a_s) * mfma. Epilogue: h = bf16(silu(g) * u), amax over
// the 128-column group (lanes, then waves through LDS), scale = max(amax,
// 1e-10) * 0x3b124925, q = e4m3(h * (1 / scale)).
template <uint32_t KB>  // H / 128
__device__ __forceinline__ void gate_up_tile(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ w13,
    const float* __restrict__ w13s, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,
    uint8_t* __restrict__ hq, float* __restrict__ hs, uint32_t T, uint32_t I, uint32_t Ktot,
    uint32_t Etot) {
  constexpr uint32_t H = 128u * KB;
  constexpr uint32_t kStride = 144;  // LDS bytes per A row (128 + 16: rotates banks across rows)
  __shared__ __align__(16) uint8_t s_a[2][kRows * kStride];
  __shared__ float s_as[kRows * KB];
  __shared__ int32_t s_tok[kRows];
  __shared__ float s_amax[4][kRows];
  __shared__ float s_scale[kRows];
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
  const uint32_t NG = I / 128u;
  uint32_t item;
  if (!xcd_item(blockIdx.x, ((uint32_t)num_valid[0] / kRows) * NG, item)) return;
  const uint32_t b = item / NG, ng = item - b * NG;
  const int32_t e = sorted_expert[b];
  if (e < 0 || (uint32_t)e >= Etot) return;
  if (tid < kRows) {
    const int32_t id = sorted_ids[b * kRows + tid];
    const uint32_t t = (uint32_t)id & 0xffffffu, slot = (uint32_t)id >> 24;
    s_tok[tid] = (t < T && slot < Ktot) ? (int32_t)t : -1;
  }
  __syncthreads();
  const uint32_t nvalid = (uint32_t)__popcll(__ballot(s_tok[lane] >= 0));
  const uint32_t ntiles = (nvalid + 15u) >> 4;
  for (uint32_t i = tid; i < kRows * KB; i += 256u) {
    const int32_t tk = s_tok[i / KB];
    s_as[i] = tk >= 0 ? xs[(size_t)tk * KB + (i % KB)] : 0.0f;
  }
  // A loader: thread moves 16 bytes of rows (tid >> 3) and 32 + (tid >> 3)
  const uint32_t ar0 = tid >> 3, ac = (tid & 7u) * 16u;
  const int32_t tk0 = s_tok[ar0], tk1 = s_tok[ar0 + 32u];
  const uint8_t* asrc0 = xq + (size_t)(tk0 < 0 ? 0 : tk0) * H + ac;
  const uint8_t* asrc1 = xq + (size_t)(tk1 < 0 ? 0 : tk1) * H + ac;
  uint8_t* adst0 = &s_a[0][ar0 * kStride + ac];
  uint8_t* adst1 = &s_a[0][(ar0 + 32u) * kStride + ac];

  const uint8_t* we = w13 + (size_t)e * 2u * I * H;
  const float* wse = w13s + (size_t)e * (2u * I / 128u) * KB;
  const uint32_t n0 = ng * 128u + wave * 32u;
  const uint32_t ntile[4] = {n0 >> 4, (n0 >> 4) + 1u, (I + n0) >> 4, ((I + n0) >> 4) + 1u};
  const float* wsg = wse + (size_t)ng * KB;           // gate rows' 128-row block
  const float* wsu = wse + (size_t)(I / 128u + ng) * KB;  // up rows' block
  v8i bq[2][4];
  auto load_b = [&](uint32_t kb, v8i (&dst)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) dst[c] = nk::load_tile_operand(nk::tile_base(we, ntile[c], kb, KB), lane);
  };

  v4f acc[4][4];
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt)
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) acc[rt][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t g = lane >> 4;

  // The K loop is instantiated per number of non-empty row tiles so it has no
  // branches: the compiler then keeps every load where it is issued (it sinks
  // loads into the branch that uses them otherwise).
  auto kloop = [&](auto ntc) __attribute__((always_inline)) {
    constexpr uint32_t NT = decltype(ntc)::value;
    uint4 a0 = *reinterpret_cast<const uint4*>(asrc0);
    uint4 a1 = *reinterpret_cast<const uint4*>(asrc1);
    load_b(0, bq[0]);
    *reinterpret_cast<uint4*>(adst0) = a0;
    *reinterpret_cast<uint4*>(adst1) = a1;
    if (KB > 1) {
      a0 = *reinterpret_cast<const uint4*>(asrc0 + 128u);
      a1 = *reinterpret_cast<const uint4*>(asrc1 + 128u);
    }
    lds_barrier();
#pragma unroll
    for (uint32_t kb = 0; kb < KB; ++kb) {
      if (kb + 1u < KB) load_b(kb + 1u, bq[(kb + 1u) & 1u]);
      const float sg = wsg[kb], su = wsu[kb];
      const uint8_t* abuf = s_a[kb & 1u];
#pragma unroll
      for (uint32_t rt = 0; rt < NT; ++rt) {
        const v8i af = lds_fp8x32(abuf + (rt * 16u + (lane & 15u)) * kStride + g * 32u);
        float scg[4], scu[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          const float as = s_as[(rt * 16u + g * 4u + j) * KB + kb];
          scg[j] = sg * as;
          scu[j] = su * as;
        }
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
          const v4f d = nk::mfma_e4m3_16x16x128(af, bq[kb & 1u][c]);
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) acc[rt][c][j] = fmaf(c < 2 ? scg[j] : scu[j], d[j], acc[rt][c][j]);
        }
      }
      if (kb + 1u < KB) {
        constexpr uint32_t kBuf = sizeof(s_a[0]);
        *reinterpret_cast<uint4*>(adst0 + ((kb + 1u) & 1u) * kBuf) = a0;
        *reinterpret_cast<uint4*>(adst1 + ((kb + 1u) & 1u) * kBuf) = a1;
        if (kb + 2u < KB) {
          a0 = *reinterpret_cast<const uint4*>(asrc0 + (kb + 2u) * 128u);
          a1 = *reinterpret_cast<const uint4*>(asrc1 + (kb + 2u) * 128u);
        }
      }
      lds_barrier();
    }
  };
  switch (ntiles) {
    case 1: kloop(std::integral_constant<uint32_t, 1>{}); break;
    case 2: kloop(std::integral_constant<uint32_t, 2>{}); break;
    case 3: kloop(std::integral_constant<uint32_t, 3>{}); break;
    default: kloop(std::integral_constant<uint32_t, 4>{}); break;
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
      if ((lane & 15u) == 0) s_amax[wave][rt * 16u + g * 4u + j] = m;
    }
  }
  __syncthreads();
  if (tid < kRows) {
    float m = nk::kAmaxFloor;
#pragma unroll
    for (uint32_t w = 0; w < 4; ++w) m = fmaxf(m, s_amax[w][tid]);
    const float scale = m * nk::inv_e4m3_max();
    s_scale[tid] = scale;
    if (tid < nvalid) hs[(size_t)(b * kRows + tid) * (I / 128u) + ng] = scale;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt) {
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint32_t row = rt * 16u + g * 4u + j;
      if (row < nvalid) {
        const float inv = 1.0f / s_scale[row];
        const uint32_t q = nk::e4m3x4(h[rt][0][j] * inv, h[rt][1][j] * inv, 0.0f, 0.0f);
        uint8_t* dst = hq + (size_t)(b * kRows + row) * I + n0 + (lane & 15u);
        dst[0] = (uint8_t)q;
        dst[16] = (uint8_t)(q >> 8);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Grouped down GEMM (reference: kernels/gfx950/templates/moe/decode/
// down_reduce_mfma_2wave.inc:14-291, prefill route partials
// moe/prefill/route_reduce_splitk2_f16.inc:6-117; oracle
// tools/benchmark/export_qwen36_moe_stage2_capture.py:90-110).
//
// Item (b, nb): expert block b, output columns [256 nb, 256 nb + 256). The
// block's 64 h rows (contiguous in sorted order, all of K) are staged in LDS
// once; wave w owns 64 columns (four 16-column tiles). Each valid row's
// result, rounded to bf16, goes to partial[route], route = token * Ktot +
// slot, through an LDS transpose so each row is written as 512 contiguous
// bytes; combine applies the top-k weights in slot order.
template <uint32_t KB>  // I / 128
__device__ __forceinline__ void down_tile(
    const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2,
    const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,
    uint16_t* __restrict__ partial, uint32_t T, uint32_t H, uint32_t Ktot, uint32_t Etot) {
  constexpr uint32_t I = 128u * KB;
  constexpr uint32_t kStride = I + 16u;   // LDS bytes per A row
  constexpr uint32_t kOut = 512u + 16u;   // LDS bytes per output row (256 bf16 + pad)
  constexpr uint32_t kLds = (kRows * kStride > kRows * kOut) ? kRows * kStride : kRows * kOut;
  __shared__ __align__(16) uint8_t s_buf[kLds];
  __shared__ float s_as[kRows * KB];
  __shared__ int32_t s_route[kRows];
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
  const uint32_t NB = H / 256u;
  uint32_t item;
  if (!xcd_item(blockIdx.x, ((uint32_t)num_valid[0] / kRows) * NB, item)) return;
  const uint32_t b = item / NB, nb = item - b * NB;
  const int32_t e = sorted_expert[b];
  if (e < 0 || (uint32_t)e >= Etot) return;
  if (tid < kRows) {
    const int32_t id = sorted_ids[b * kRows + tid];
    const uint32_t t = (uint32_t)id & 0xffffffu, slot = (uint32_t)id >> 24;
    s_route[tid] = (t < T && slot < Ktot) ? (int32_t)(t * Ktot + slot) : -1;
  }
  // all of A (64 rows x I bytes, contiguous) and its scales
  constexpr uint32_t kA16 = kRows * I / 16u / 256u;  // uint4 per thread
  uint4 areg[kA16];
  const uint8_t* ablk = hq + (size_t)b * kRows * I;
#pragma unroll
  for (uint32_t p = 0; p < kA16; ++p) areg[p] = reinterpret_cast<const uint4*>(ablk)[p * 256u + tid];
  for (uint32_t i = tid; i < kRows * KB; i += 256u) s_as[i] = hs[(size_t)b * kRows * KB + i];

  const uint8_t* we = w2 + (size_t)e * H * I;
  const float* wse = w2s + (size_t)e * (H / 128u) * KB;
  const uint32_t n0 = nb * 256u + wave * 64u;
  const float* wsn = wse + (size_t)(n0 >> 7) * KB;  // the wave's 64 columns lie in one 128-row block
  v8i bq[2][4];
  auto load_b = [&](uint32_t kb, v8i (&dst)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) dst[c] = nk::load_tile_operand(nk::tile_base(we, (n0 >> 4) + c, kb, KB), lane);
  };
  load_b(0, bq[0]);
  if (KB > 1) load_b(1, bq[1]);
#pragma unroll
  for (uint32_t p = 0; p < kA16; ++p) {
    const uint32_t idx = p * 256u + tid;            // uint4 index in the block
    const uint32_t row = idx / (I / 16u), c16 = idx - row * (I / 16u);
    *reinterpret_cast<uint4*>(&s_buf[row * kStride + c16 * 16u]) = areg[p];
  }
  __syncthreads();
  const uint32_t nvalid = (uint32_t)__popcll(__ballot(s_route[lane] >= 0));
  const uint32_t ntiles = (nvalid + 15u) >> 4;
  const uint32_t g = lane >> 4;

  v4f acc[4][4];
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt)
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) acc[rt][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  auto kloop = [&](auto ntc) __attribute__((always_inline)) {  // per tile count, branch-free (see gate_up_tile)
    constexpr uint32_t NT = decltype(ntc)::value;
#pragma unroll
    for (uint32_t kb = 0; kb < KB; ++kb) {
      const float sw = wsn[kb];
#pragma unroll
      for (uint32_t rt = 0; rt < NT; ++rt) {
        const v8i af = lds_fp8x32(&s_buf[(rt * 16u + (lane & 15u)) * kStride + kb * 128u + g * 32u]);
        float sc[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) sc[j] = sw * s_as[(rt * 16u + g * 4u + j) * KB + kb];
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
          const v4f d = nk::mfma_e4m3_16x16x128(af, bq[kb & 1u][c]);
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) acc[rt][c][j] = fmaf(sc[j], d[j], acc[rt][c][j]);
        }
      }
      if (kb + 2u < KB) load_b(kb + 2u, bq[kb & 1u]);
    }
  };
  switch (ntiles) {
    case 1: kloop(std::integral_constant<uint32_t, 1>{}); break;
    case 2: kloop(std::integral_constant<uint32_t, 2>{}); break;
    case 3: kloop(std::integral_constant<uint32_t, 3>{}); break;
    default: kloop(std::integral_constant<uint32_t, 4>{}); break;
  }
  __syncthreads();  // A no longer needed: the buffer becomes the output tile
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt)
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint32_t row = rt * 16u + g * 4u + j;
#pragma unroll
      for (uint32_t c = 0; c < 4; ++c)
        *reinterpret_cast<uint16_t*>(&s_buf[row * kOut + (wave * 64u + c * 16u + (lane & 15u)) * 2u]) =
            nk::bf16_rne(acc[rt][c][j]);
    }
  __syncthreads();
  // 64 rows x 512 bytes: 32 uint4 per row, 8 per thread
#pragma unroll
  for (uint32_t p = 0; p < 8u; ++p) {
    const uint32_t idx = p * 256u + tid;
    const uint32_t row = idx >> 5, c16 = idx & 31u;
    const int32_t route = s_route[row];
    if (row < nvalid && route >= 0)
      *reinterpret_cast<uint4*>(partial + (size_t)route * H + nb * 256u + c16 * 8u) =
          *reinterpret_cast<const uint4*>(&s_buf[row * kOut + c16 * 16u]);
  }
}

}  // namespace nktile

#define NK_GATE_UP_TILE(HV)                                                                        \
  NK_KERNEL __launch_bounds__(256) void netra_moe_gate_up_tile_h##HV##_gfx950(                     \
      const uint8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ w13, \
      const float* __restrict__ w13s, const int32_t* __restrict__ sorted_ids,                      \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,            \
      uint8_t* __restrict__ hq, float* __restrict__ hs, uint32_t T, uint32_t H, uint32_t I,        \
      uint32_t Ktot, uint32_t Etot) {                                                              \
    (void)H;                                                                                       \
    nktile::gate_up_tile<HV / 128>(xq, xs, w13, w13s, sorted_ids, sorted_expert, num_valid, hq,    \
                                   hs, T, I, Ktot, Etot);                                          \
  }
NK_GATE_UP_TILE(512)
NK_GATE_UP_TILE(1024)
NK_GATE_UP_TILE(2048)
NK_GATE_UP_TILE(4096)

#define NK_DOWN_TILE(IV)                                                                           \
  NK_KERNEL __launch_bounds__(256)                                                                \
  void netra_moe_down_tile_i##IV##_gfx950(                                                        \
      const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2, \
      const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,                       \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,            \
      uint16_t* __restrict__ partial, uint32_t T, uint32_t H, uint32_t I, uint32_t Ktot,           \
      uint32_t Etot) {                                                                             \
    (void)I;                                                                                       \
    nktile::down_tile<IV / 128>(hq, hs, w2, w2s, sorted_ids, sorted_expert, num_valid, partial, T, \
                                H, Ktot, Etot);                                                    \
  }
NK_DOWN_TILE(256)
NK_DOWN_TILE(512)
NK_DOWN_TILE(1024)
