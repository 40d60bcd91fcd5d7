// Tile-regime grouped GEMMs (prefill-sized T): one workgroup per (64-row
// expert block, column group), SiLU.mul + 1x128 FP8 requant fused into the
// gate/up epilogue, bf16 route partials out of the down GEMM.
//
// Both kernels stage the block's activation rows in LDS once per workgroup
// (the waves share them), keep several 128-K blocks of weight operands in
// flight per wave, and synchronise through LDS-only barriers so the weight
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
// Item (b, ng): expert block b, h columns [128 ng, 128 ng + 128), WAVES waves.
// Wave w owns the CPW = 128 / WAVES h columns n = 128 ng + CPW w .. +CPW-1:
// CPW / 16 W13 tiles of gate rows and as many of up rows (I + n; stored
// gate/up-interleaved, so a wave's tiles are one contiguous range), against the
// block's non-empty 16-row tiles. Weight operands are prefetched AHEAD 128-K
// blocks ahead (a ring in registers, raw buffer loads with scalar offsets),
// activation rows two blocks ahead of their LDS store. Per 128-K block:
// acc += (w_s * a_s) * mfma. Epilogue: h = bf16(silu(g) * u), amax over the
// 128-column group (lanes, then the waves through LDS), scale = max(amax,
// 1e-10) * 0x3b124925, q = e4m3(h * (1 / scale)).
template <uint32_t KB, uint32_t WAVES, uint32_t AHEAD>  // KB = H / 128
__device__ __forceinline__ void gate_up_tile(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ w13,
    const float* __restrict__ w13s, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,
    uint8_t* __restrict__ hq, float* __restrict__ hs, uint32_t T, uint32_t I, uint32_t Ktot,
    uint32_t Etot) {
  constexpr uint32_t H = 128u * KB;
  constexpr uint32_t kThreads = 64u * WAVES;
  constexpr uint32_t CPW = 128u / WAVES;  // h columns per wave
  constexpr uint32_t CT = CPW / 16u;      // 16-column tiles per wave (gate; up likewise)
  constexpr uint32_t APT = 8u / WAVES;    // A uint4 per thread per 128-K block
  constexpr uint32_t kStride = 144;       // LDS bytes per A row (128 + 16: rotates banks across rows)
  constexpr uint32_t kRing = AHEAD + 1u;
  static_assert(WAVES == 4 || WAVES == 8, "128 columns over 4 or 8 waves");
  __shared__ __align__(16) uint8_t s_a[2][kRows * kStride];
  __shared__ float s_sg[kRows * KB];  // w_s(gate block, kb) * a_s(row, kb)
  __shared__ float s_su[kRows * KB];  // w_s(up block, kb) * a_s(row, kb)
  __shared__ int32_t s_tok[kRows];
  __shared__ float s_amax[WAVES][kRows];
  __shared__ float s_scale[kRows];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));  // uniform: scalar addressing
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
  // A loader: thread moves APT x 16 bytes of the 64 x 128 block per step
  // (pieces tid and, with 4 waves, tid + 256; explicit variables, not arrays,
  // so they stay in registers)
  const uint32_t ar0 = tid >> 3, ar1 = (tid + kThreads) >> 3, ac = (tid & 7u) * 16u;
  const int32_t tka0 = s_tok[ar0], tka1 = APT > 1 ? s_tok[ar1 & 63u] : 0;
  const uint8_t* asrc0 = xq + (size_t)(tka0 < 0 ? 0 : tka0) * H + ac;
  const uint8_t* asrc1 = xq + (size_t)(tka1 < 0 ? 0 : tka1) * H + ac;
  uint8_t* adst0 = &s_a[0][ar0 * kStride + ac];
  uint8_t* adst1 = &s_a[0][(ar1 & 63u) * kStride + ac];

  const uint32_t n0 = ng * 128u + wave * CPW;
  // gate / up tile strips: CT row tiles x KB tiles of 2 KiB, contiguous in the tile16x128 layout
  const uint8_t* w13e = w13 + (size_t)e * 2u * I * H;
  // gate/up-interleaved W13: gate tile t at 2 t, up tile t at 2 t + 1; the
  // wave's CT pairs are one contiguous range
  const __amdgpu_buffer_rsrc_t wgu = nk::buffer_rsrc(nk::tile_base(w13e, 2u * (n0 >> 4), 0, KB), 2u * CT * KB * 2048u);
  const float* wse = w13s + (size_t)e * (2u * I / 128u) * KB;
  const float* wsg = wse + (size_t)ng * KB;               // gate rows' 128-row block
  const float* wsu = wse + (size_t)(I / 128u + ng) * KB;  // up rows' block
  for (uint32_t i = tid; i < kRows * KB; i += kThreads) {
    const int32_t tk = s_tok[i / KB];
    const float as = tk >= 0 ? xs[(size_t)tk * KB + (i % KB)] : 0.0f;
    s_sg[i] = wsg[i % KB] * as;
    s_su[i] = wsu[i % KB] * as;
  }
  const uint32_t g = lane >> 4;

  v4f acc[4][2 * CT];
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt)
#pragma unroll
    for (uint32_t c = 0; c < 2 * CT; ++c) acc[rt][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  // K loop, instantiated per number of non-empty row tiles so it has no
  // branches (the compiler sinks loads into the branch that uses them
  // otherwise, which would serialise them with their use).
  auto kloop = [&](auto ntc) __attribute__((always_inline)) {
    constexpr uint32_t NT = decltype(ntc)::value;
    v8i bq[kRing][2 * CT];
    uint4 e0, e1, o0, o1;  // A pieces (0 / 1) of the even / odd 128-K block in flight
    auto load_b = [&](uint32_t kb, v8i (&dst)[2 * CT]) __attribute__((always_inline)) {
#pragma unroll
      for (uint32_t c = 0; c < CT; ++c) {
        dst[c] = nk::load_tile_operand(wgu, (2u * c * KB + kb) * 2048u, lane);
        dst[CT + c] = nk::load_tile_operand(wgu, ((2u * c + 1u) * KB + kb) * 2048u, lane);
      }
    };
#pragma unroll
    for (uint32_t k = 0; k < AHEAD && k < KB; ++k) load_b(k, bq[k]);
    e0 = *reinterpret_cast<const uint4*>(asrc0);
    if (APT > 1) e1 = *reinterpret_cast<const uint4*>(asrc1);
    if (KB > 1) {
      o0 = *reinterpret_cast<const uint4*>(asrc0 + 128u);
      if (APT > 1) o1 = *reinterpret_cast<const uint4*>(asrc1 + 128u);
    }
    *reinterpret_cast<uint4*>(adst0) = e0;
    if (APT > 1) *reinterpret_cast<uint4*>(adst1) = e1;
    if (KB > 2) {
      e0 = *reinterpret_cast<const uint4*>(asrc0 + 256u);
      if (APT > 1) e1 = *reinterpret_cast<const uint4*>(asrc1 + 256u);
    }
    lds_barrier();
#pragma unroll
    for (uint32_t kb = 0; kb < KB; ++kb) {
      if (kb + AHEAD < KB) load_b(kb + AHEAD, bq[(kb + AHEAD) % kRing]);
      const uint8_t* abuf = s_a[kb & 1u];
#pragma unroll
      for (uint32_t rt = 0; rt < NT; ++rt) {
        const v8i af = lds_fp8x32(abuf + (rt * 16u + (lane & 15u)) * kStride + g * 32u);
        float scg[4], scu[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          scg[j] = s_sg[(rt * 16u + g * 4u + j) * KB + kb];
          scu[j] = s_su[(rt * 16u + g * 4u + j) * KB + kb];
        }
#pragma unroll
        for (uint32_t c = 0; c < 2 * CT; ++c) {
          const v4f d = nk::mfma_e4m3_16x16x128(af, bq[kb % kRing][c]);
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) acc[rt][c][j] = fmaf(c < CT ? scg[j] : scu[j], d[j], acc[rt][c][j]);
        }
      }
      if (kb + 1u < KB) {  // A(kb + 1) -> LDS, A(kb + 3) requested
        constexpr uint32_t kBuf = sizeof(s_a[0]);
        uint4& q0 = ((kb + 1u) & 1u) ? o0 : e0;
        uint4& q1 = ((kb + 1u) & 1u) ? o1 : e1;
        *reinterpret_cast<uint4*>(adst0 + ((kb + 1u) & 1u) * kBuf) = q0;
        if (APT > 1) *reinterpret_cast<uint4*>(adst1 + ((kb + 1u) & 1u) * kBuf) = q1;
        if (kb + 3u < KB) {
          q0 = *reinterpret_cast<const uint4*>(asrc0 + (kb + 3u) * 128u);
          if (APT > 1) q1 = *reinterpret_cast<const uint4*>(asrc1 + (kb + 3u) * 128u);
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

  // Epilogue: h = bf16(silu(g) * u); per-row amax over this wave's columns.
  float h[4][CT][4];
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt) {
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      float m = 0.0f;
#pragma unroll
      for (uint32_t c = 0; c < CT; ++c) {
        const float v = nk::bf16_f32(nk::bf16_rne(nk::silu(acc[rt][c][j]) * acc[rt][CT + c][j]));
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
    for (uint32_t w = 0; w < WAVES; ++w) m = fmaxf(m, s_amax[w][tid]);
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
        uint8_t* dst = hq + (size_t)(b * kRows + row) * I + n0 + (lane & 15u);
#pragma unroll
        for (uint32_t c = 0; c < CT; ++c) dst[16u * c] = (uint8_t)nk::e4m3x4(h[rt][c][j] * inv, 0.0f, 0.0f, 0.0f);
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
// Item (b, nb), 256 threads: expert block b, output columns [128 nb, 128 nb
// + 128). The block's 64 h rows (contiguous in sorted order, all of K) are
// staged in LDS once; wave w owns 32 columns (two 16-column tiles), all of
// whose weight operands are requested before the first multiply. Each valid
// row's result, rounded to bf16, goes to partial[route], route = token * Ktot
// + slot, through an LDS transpose so each row is written as 256 contiguous
// bytes; combine applies the top-k weights in slot order.
template <uint32_t KB>  // I / 128
__device__ __forceinline__ void down_tile(
    const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2,
    const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,
    uint16_t* __restrict__ partial, uint32_t T, uint32_t H, uint32_t Ktot, uint32_t Etot) {
  constexpr uint32_t I = 128u * KB;
  constexpr uint32_t kStride = I + 16u;   // LDS bytes per A row
  constexpr uint32_t kOut = 256u + 16u;   // LDS bytes per output row (128 bf16 + pad)
  constexpr uint32_t kLds = (kRows * kStride > kRows * kOut) ? kRows * kStride : kRows * kOut;
  __shared__ __align__(16) uint8_t s_buf[kLds];
  __shared__ float s_as[kRows * KB];  // w_s(kb) * h_s(row, kb)
  __shared__ int32_t s_route[kRows];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));  // uniform: scalar addressing
  const uint32_t NB = H / 128u;
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
  const uint32_t n0 = nb * 128u + wave * 32u;
  // row tiles n0 / 16 and n0 / 16 + 1: 2 KB tiles of 2 KiB, contiguous
  const __amdgpu_buffer_rsrc_t wt =
      nk::buffer_rsrc(nk::tile_base(w2 + (size_t)e * H * I, n0 >> 4, 0, KB), 2u * KB * 2048u);
  v8i bq[KB][2];
#pragma unroll
  for (uint32_t kb = 0; kb < KB; ++kb) {
    bq[kb][0] = nk::load_tile_operand(wt, kb * 2048u, lane);
    bq[kb][1] = nk::load_tile_operand(wt, (KB + kb) * 2048u, lane);
  }
  // all of A (64 rows x I bytes, contiguous) and its scales
  constexpr uint32_t kA16 = kRows * I / 16u / 256u;  // uint4 per thread
  uint4 areg[kA16];
  const uint8_t* ablk = hq + (size_t)b * kRows * I;
#pragma unroll
  for (uint32_t p = 0; p < kA16; ++p) areg[p] = reinterpret_cast<const uint4*>(ablk)[p * 256u + tid];
  const float* wsn = w2s + ((size_t)e * (H / 128u) + (nb * 128u >> 7)) * KB;  // the item's 128-row block
  for (uint32_t i = tid; i < kRows * KB; i += 256u) s_as[i] = wsn[i % KB] * hs[(size_t)b * kRows * KB + i];
#pragma unroll
  for (uint32_t p = 0; p < kA16; ++p) {
    const uint32_t idx = p * 256u + tid;  // uint4 index in the block
    const uint32_t row = idx / (I / 16u), c16 = idx - row * (I / 16u);
    *reinterpret_cast<uint4*>(&s_buf[row * kStride + c16 * 16u]) = areg[p];
  }
  __syncthreads();
  const uint32_t nvalid = (uint32_t)__popcll(__ballot(s_route[lane] >= 0));
  const uint32_t ntiles = (nvalid + 15u) >> 4;
  const uint32_t g = lane >> 4;

  v4f acc[4][2];
#pragma unroll
  for (uint32_t rt = 0; rt < 4; ++rt) acc[rt][0] = acc[rt][1] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  auto kloop = [&](auto ntc) __attribute__((always_inline)) {  // branch-free per tile count
    constexpr uint32_t NT = decltype(ntc)::value;
#pragma unroll
    for (uint32_t kb = 0; kb < KB; ++kb) {
      v4f d[NT][2];  // the block's MFMAs first, into separate results
#pragma unroll
      for (uint32_t rt = 0; rt < NT; ++rt) {
        const v8i af = lds_fp8x32(&s_buf[(rt * 16u + (lane & 15u)) * kStride + kb * 128u + g * 32u]);
        d[rt][0] = nk::mfma_e4m3_16x16x128(af, bq[kb][0]);
        d[rt][1] = nk::mfma_e4m3_16x16x128(af, bq[kb][1]);
      }
#pragma unroll
      for (uint32_t rt = 0; rt < NT; ++rt) {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          const float sc = s_as[(rt * 16u + g * 4u + j) * KB + kb];
          acc[rt][0][j] = fmaf(sc, d[rt][0][j], acc[rt][0][j]);
          acc[rt][1][j] = fmaf(sc, d[rt][1][j], acc[rt][1][j]);
        }
      }
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
      for (uint32_t c = 0; c < 2; ++c)
        *reinterpret_cast<uint16_t*>(&s_buf[row * kOut + (wave * 32u + c * 16u + (lane & 15u)) * 2u]) =
            nk::bf16_rne(acc[rt][c][j]);
    }
  __syncthreads();
  // 64 rows x 256 bytes: 16 uint4 per row, 4 per thread
#pragma unroll
  for (uint32_t p = 0; p < 4u; ++p) {
    const uint32_t idx = p * 256u + tid;
    const uint32_t row = idx >> 4, c16 = idx & 15u;
    const int32_t route = s_route[row];
    if (row < nvalid && route >= 0)
      *reinterpret_cast<uint4*>(partial + (size_t)route * H + nb * 128u + c16 * 8u) =
          *reinterpret_cast<const uint4*>(&s_buf[row * kOut + c16 * 16u]);
  }
}

// ---------------------------------------------------------------------------
// Grouped down GEMM over row blocks (reference: kernels/gfx950/templates/moe/
// prefill/fused_splitk2/down_partial.inc and route_reduce_splitk2_f16.inc:6-117;
// oracle tools/benchmark/export_qwen36_moe_stage2_capture.py:90-110).
//
// Item (b, c): expert block b against NBC consecutive 128-column groups
// nb = c NBC .. (c + 1) NBC - 1 of H, 8 waves. The block's FP8 rows (64 x I)
// and their 1x128 scales are staged in LDS once per item; wave w owns columns
// 128 nb + 16 w .. +15 of every group (one 16-row W2 tile, K contiguous) and
// refills each K block's weight registers with the next group's tile right
// after using them (a one-group register ring, so a group of loads is always
// in flight). Per 128-K block acc += (w_s(nb, kb) * h_s(row, kb)) * mfma,
// the MFMA taking the weight tile as A and the h rows as B so each lane ends
// with four consecutive columns of one route row; each group's result,
// rounded to bf16, goes through an LDS transpose (8-byte writes, two buffers,
// one barrier per group) so each route row leaves as 256 contiguous bytes
// (2-byte transposes of the other orientation cost 37% of LDS cycles in
// bank conflicts; 8-byte stores straight to memory ran 30% slower than whole
// rows); rows past the block's valid count take an offset past the buffer
// and the hardware drops their stores.
//
// kAiter: W2 in the reference's AITER 16x16 shuffle. kSplitF16: the output
// format of the reference's prefill producer (moe_prefill_m768_bridge.hip:
// 144-147, route_reduce_splitk2_f16.inc:44-61): two fp16 partial tensors,
// half h holding the sum over K blocks [h KB/2, (h + 1) KB/2) of each route
// row, the second one half_rows rows after the first.
constexpr uint32_t kDownWaves = 8;

__device__ __forceinline__ uint16_t f16_bits(float x) {
  const _Float16 h = (_Float16)x;  // v_cvt_f16_f32, round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

template <uint32_t KB, bool kAiter = false, bool kSplitF16 = false>  // I / 128
__device__ __forceinline__ void down_rows(
    const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2,
    const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,
    uint16_t* __restrict__ partial, uint32_t T, uint32_t H, uint32_t Ktot, uint32_t Etot, uint32_t NBC,
    uint32_t half_rows = 0) {
  static_assert(!kSplitF16 || KB % 2 == 0, "split-K halves need an even K block count");
  constexpr uint32_t I = 128u * KB;
  constexpr uint32_t kThreads = 64u * kDownWaves;
  static_assert((KB & (KB - 1u)) == 0 && KB <= 64u, "one scale lane per K block");
  // the block's rows in the MFMA operand layout: 2 KiB per (16-row tile rt,
  // K block kb), lane l's 32 bytes (row l & 15, K bytes 32 (l >> 4) ..) as a
  // low half at 16 l and a high half at 1024 + 16 l, so each operand read is
  // 64 lanes x 16 contiguous bytes (a row-major copy with any row padding
  // had the four K groups of a row tile fight over the same banks: 43% of
  // LDS cycles in conflicts)
  __shared__ __align__(16) uint8_t s_a[kRows * I];
  constexpr uint32_t kOut = 256u + 16u;  // LDS bytes per output row (128 bf16 + pad)
  __shared__ __align__(16) uint8_t s_out[2][kRows * kOut];
  __shared__ __align__(16) float s_hs[KB * kRows];  // h_s(row, kb) at [kb][row]
  __shared__ int32_t s_route[kRows];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const uint32_t NB = H / 128u, NCH = NB / NBC;
  if (NBC == 0u || NCH * NBC != NB) return;  // the engine passes a divisor of H / 128
  uint32_t item;
  if (!xcd_item(blockIdx.x, ((uint32_t)num_valid[0] / kRows) * NCH, item)) return;
  const uint32_t b = item / NCH, nb0 = (item - b * NCH) * NBC;
  const int32_t e = sorted_expert[b];
  if (e < 0 || (uint32_t)e >= Etot) return;
  if (tid < kRows) {
    const int32_t id = sorted_ids[b * kRows + tid];
    const uint32_t t = (uint32_t)id & 0xffffffu, slot = (uint32_t)id >> 24;
    s_route[tid] = (t < T && slot < Ktot) ? (int32_t)(t * Ktot + slot) : -1;
  }
  // The expert's W2 in tile16x128 (row tile rt's K blocks contiguous); wave
  // w's tile of group nb is row tile 8 nb + w. Its weight scales come one per
  // lane (lane kb holds w_s(nb, kb)) by a vector load: a scalar load would
  // share the LDS counter and make the next LDS wait a full drain.
  const __amdgpu_buffer_rsrc_t wt = nk::buffer_rsrc(w2 + (size_t)e * H * I, H * I);
  const float* wse = w2s + (size_t)e * NB * KB;
  v8i bq[KB];
#pragma unroll
  for (uint32_t kb = 0; kb < KB; ++kb)
    bq[kb] = nk::load_tile_operand<kAiter>(wt, ((nb0 * 8u + wave) * KB + kb) * 2048u, lane);
  float wsv = wse[nb0 * KB + (lane & (KB - 1u))];
  // the block's A rows (64 x I bytes, contiguous) and scales; thread slot s
  // of the operand layout fetches the 16 bytes that belong there
  constexpr uint32_t kA16 = kRows * I / 16u / kThreads;  // uint4 per thread
  static_assert(kA16 >= 1u, "A staging");
  uint4 areg[kA16];
  const uint8_t* ablk = hq + (size_t)b * kRows * I;
#pragma unroll
  for (uint32_t p = 0; p < kA16; ++p) {
    const uint32_t slot = p * kThreads + tid, t = slot >> 7, half = (slot >> 6) & 1u, l = slot & 63u;
    const uint32_t row = (t / KB) * 16u + (l & 15u), col = (t % KB) * 128u + (l >> 4) * 32u + half * 16u;
    areg[p] = *reinterpret_cast<const uint4*>(ablk + row * I + col);
  }
  // thread i: row i % 64 of K block i / 64, so a wave's stores are 64
  // consecutive floats (the global gather is 1 KiB per item)
  for (uint32_t i = tid; i < kRows * KB; i += kThreads) {
    const uint32_t row = i & (kRows - 1u), kb = i / kRows;
    s_hs[i] = hs[(size_t)b * kRows * KB + row * KB + kb];
  }
#pragma unroll
  for (uint32_t p = 0; p < kA16; ++p) *reinterpret_cast<uint4*>(&s_a[(p * kThreads + tid) * 16u]) = areg[p];
  lds_barrier();
  const uint32_t nvalid = (uint32_t)__popcll(__ballot(s_route[lane] >= 0));
  const uint32_t ntiles = (nvalid + 15u) >> 4;
  const uint32_t g = lane >> 4;
  // The MFMA takes the weight tile as its A operand and the h rows as B, so
  // lane l holds output columns 4 (l >> 4) .. + 3 of route row l & 15 of each
  // 16-row tile: four consecutive outputs, one 8-byte LDS write into the
  // group's 64 x 256-byte output rows (row stride 272: the 32 lanes of a
  // write pass cover 64 distinct banks), then each route row leaves as 256
  // contiguous bytes (2 x 16 per thread). Rows past nvalid (or padding) take
  // offset 2^31, past the buffer's range (the engine keeps the partial
  // buffer below 2^31 bytes), so their stores are dropped.
  const uint32_t half_bytes = half_rows * H * 2u;
  const __amdgpu_buffer_rsrc_t pr = nk::buffer_rsrc(partial, kSplitF16 ? 2u * half_bytes : T * Ktot * H * 2u);
  uint32_t soff[2];
  bool live[2];
#pragma unroll
  for (uint32_t p = 0; p < 2u; ++p) {
    const uint32_t idx = p * kThreads + tid, row = idx >> 4, c16 = idx & 15u;
    const int32_t route = s_route[row];
    live[p] = row < nvalid && route >= 0;
    soff[p] = live[p] ? ((uint32_t)route * H + c16 * 8u) * 2u : 0x80000000u;
  }
  auto pack2 = [&](float lo, float hi) __attribute__((always_inline)) {
    return kSplitF16 ? ((uint32_t)f16_bits(lo) | ((uint32_t)f16_bits(hi) << 16)) : nk::bf16x2_hw(lo, hi);
  };
  // One output group through the LDS transpose: buffer v & 1, one barrier (the
  // other buffer was read before the previous barrier); `extra` moves live
  // rows to the second split-K half.
  auto emit = [&](auto ntc, const v4f* acc, uint32_t v, uint32_t nb, uint32_t extra) __attribute__((always_inline)) {
    constexpr uint32_t NT = decltype(ntc)::value;
    // rows r and r + 8 of a 16-lane write pass would share banks (row stride
    // 68 dwords): odd row octets swap the two 8-byte halves of every 16-byte
    // chunk, and the 16-byte reads swap them back
    uint8_t* so = s_out[v & 1u];
#pragma unroll
    for (uint32_t rt = 0; rt < NT; ++rt) {
      const uint32_t row = rt * 16u + (lane & 15u);
      *reinterpret_cast<uint2*>(&so[row * kOut + (((wave * 16u + g * 4u) * 2u) ^ (((row >> 3) & 1u) << 3))]) =
          make_uint2(pack2(acc[rt][0], acc[rt][1]), pack2(acc[rt][2], acc[rt][3]));
    }
    lds_barrier();
#pragma unroll
    for (uint32_t p = 0; p < 2u; ++p) {
      const uint32_t idx = p * kThreads + tid, row = idx >> 4, c16 = idx & 15u;
      uint4 val = *reinterpret_cast<const uint4*>(&so[row * kOut + c16 * 16u]);
      if ((row >> 3) & 1u) val = make_uint4(val.z, val.w, val.x, val.y);
      __builtin_amdgcn_raw_buffer_store_b128(nk::u32x4{val.x, val.y, val.z, val.w}, pr,
                                             (int)(soff[p] + (live[p] ? extra : 0u)), (int)(nb * 256u), 0);
    }
  };

  // One output group; kRefill: the next group's weight tiles and scales load
  // under this one's MFMAs (the last group of the item, peeled, loads none:
  // no load under a branch, whose join would make the compiler's wait counts
  // drain the group in flight). kSplitF16 keeps one loop whose last refill
  // repeats its group: peeled, it needs more than the 128 VGPRs of two
  // workgroups per CU.
  auto group = [&](auto ntc, auto refc, uint32_t q) __attribute__((always_inline)) {
    constexpr uint32_t NT = decltype(ntc)::value;
    constexpr bool kRefill = decltype(refc)::value;
    {
      const uint32_t nb = nb0 + q, nbn = nb0 + (kRefill && q + 1u < NBC ? q + 1u : q);
      const float wsn = kRefill ? wse[nbn * KB + (lane & (KB - 1u))] : 0.0f;
      v4f acc[NT];
#pragma unroll
      for (uint32_t rt = 0; rt < NT; ++rt) acc[rt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (uint32_t kb = 0; kb < KB; ++kb) {
        const float ws = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(wsv), (int)kb));
        v4f d[NT];
#pragma unroll
        for (uint32_t rt = 0; rt < NT; ++rt)
          d[rt] = nk::mfma_e4m3_16x16x128(bq[kb], nk::load_tile_operand(&s_a[(rt * KB + kb) * 2048u], lane));
        if constexpr (kRefill)  // the next group's tile
          bq[kb] = nk::load_tile_operand<kAiter>(wt, ((nbn * 8u + wave) * KB + kb) * 2048u, lane);
#pragma unroll
        for (uint32_t rt = 0; rt < NT; ++rt) {
          const float sc = ws * s_hs[kb * kRows + rt * 16u + (lane & 15u)];  // this lane's route row
          acc[rt][0] = fmaf(sc, d[rt][0], acc[rt][0]);
          acc[rt][1] = fmaf(sc, d[rt][1], acc[rt][1]);
          acc[rt][2] = fmaf(sc, d[rt][2], acc[rt][2]);
          acc[rt][3] = fmaf(sc, d[rt][3], acc[rt][3]);
        }
        // This block's accumulation completes here (the accumulators are
        // operands of the asm) and the next block's LDS reads stay below it
        // (memory clobber): otherwise the compiler issues every block's MFMAs
        // first and holds all their results, which costs ~128 VGPRs.
#pragma unroll
        for (uint32_t rt = 0; rt < NT; ++rt) asm volatile("" : "+v"(acc[rt]) : : "memory");
        if constexpr (kSplitF16) {
          if (kb == KB / 2u - 1u) {  // first split-K half complete
            emit(ntc, acc, 2u * q, nb, 0u);
#pragma unroll
            for (uint32_t rt = 0; rt < NT; ++rt) acc[rt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
          }
        }
      }
      if constexpr (kRefill) wsv = wsn;
      if constexpr (kSplitF16) emit(ntc, acc, 2u * q + 1u, nb, half_bytes);
      else emit(ntc, acc, q, nb, 0u);
    }
  };
  auto run = [&](auto ntc) __attribute__((always_inline)) {
    if constexpr (kSplitF16) {
#pragma unroll 1
      for (uint32_t q = 0; q < NBC; ++q) group(ntc, std::true_type{}, q);
    } else {
#pragma unroll 1
      for (uint32_t q = 0; q + 1u < NBC; ++q) group(ntc, std::true_type{}, q);
      group(ntc, std::false_type{}, NBC - 1u);
    }
  };
  switch (ntiles) {
    case 1: run(std::integral_constant<uint32_t, 1>{}); break;
    case 2: run(std::integral_constant<uint32_t, 2>{}); break;
    case 3: run(std::integral_constant<uint32_t, 3>{}); break;
    default: run(std::integral_constant<uint32_t, 4>{}); break;
  }
}

}  // namespace nktile

// Gate/up tile kernels: 4 waves x 32 columns, one weight block in flight
// ahead. The engine uses them for H = 4096, where the block-pair LDS ring
// does not fit; the other widths are instantiated for tests and comparison.
#define NK_GATE_UP_TILE_V(NAME, HV, WAVES, AHEAD)                                                 \
  NK_KERNEL __launch_bounds__(64 * WAVES) void NAME(                                               \
      const uint8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ w13, \
      const float* __restrict__ w13s, const int32_t* __restrict__ sorted_ids,                      \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,            \
      uint8_t* __restrict__ hq, float* __restrict__ hs, uint32_t T, uint32_t H, uint32_t I,        \
      uint32_t Ktot, uint32_t Etot) {                                                              \
    (void)H;                                                                                       \
    nktile::gate_up_tile<HV / 128, WAVES, AHEAD>(xq, xs, w13, w13s, sorted_ids, sorted_expert,     \
                                                 num_valid, hq, hs, T, I, Ktot, Etot);             \
  }
NK_GATE_UP_TILE_V(netra_moe_gate_up_tile_h512_gfx950, 512, 4, 1)
NK_GATE_UP_TILE_V(netra_moe_gate_up_tile_h1024_gfx950, 1024, 4, 1)
NK_GATE_UP_TILE_V(netra_moe_gate_up_tile_h2048_gfx950, 2048, 4, 1)
NK_GATE_UP_TILE_V(netra_moe_gate_up_tile_h4096_gfx950, 4096, 4, 1)

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

#define NK_DOWN_ROWS(IV)                                                                           \
  NK_KERNEL __launch_bounds__(512)                                                                \
  void netra_moe_down_rows_i##IV##_gfx950(                                                        \
      const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2, \
      const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,                       \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,            \
      uint16_t* __restrict__ partial, uint32_t T, uint32_t H, uint32_t I, uint32_t Ktot,           \
      uint32_t Etot, uint32_t NBC) {                                                               \
    (void)I;                                                                                       \
    nktile::down_rows<IV / 128>(hq, hs, w2, w2s, sorted_ids, sorted_expert, num_valid, partial, T, \
                                H, Ktot, Etot, NBC);                                               \
  }
NK_DOWN_ROWS(256)
NK_DOWN_ROWS(512)

// The M768 prefill bridge's producer format: W2 in the AITER layout, fp16
// split-K2 route partials (half 1 starts half_rows rows after half 0).
#define NK_DOWN_ROWS_AITER_F16X2(IV)                                                               \
  NK_KERNEL __launch_bounds__(512)                                                                \
  void netra_moe_down_rows_aiter_f16x2_i##IV##_gfx950(                                            \
      const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2, \
      const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,                       \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,            \
      uint16_t* __restrict__ partial, uint32_t T, uint32_t H, uint32_t I, uint32_t Ktot,           \
      uint32_t Etot, uint32_t NBC, uint32_t half_rows) {                                           \
    (void)I;                                                                                       \
    nktile::down_rows<IV / 128, true, true>(hq, hs, w2, w2s, sorted_ids, sorted_expert, num_valid, \
                                            partial, T, H, Ktot, Etot, NBC, half_rows);            \
  }
NK_DOWN_ROWS_AITER_F16X2(512)
