// Tile-regime grouped GEMMs: one workgroup per (64-row expert block, column
// group) with the SiLU.mul + 1x128 FP8 requant fused into the gate/up epilogue.
// Used where expert blocks are full (prefill-sized T).
#pragma once
#include "moe_numerics.h"

#define NK_KERNEL extern "C" __global__

using nk::v4f;
using nk::v8i;

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
NK_KERNEL __launch_bounds__(256) void netra_moe_gate_up_tile_gfx950(
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
      bf[c] = nk::load_tile_operand(nk::tile_base(we, nrow[c] >> 4, kb, KB), lane);
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
NK_KERNEL __launch_bounds__(256) void netra_moe_down_tile_gfx950(
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
      bf[c] = nk::load_tile_operand(nk::tile_base(we, n >> 4, kb, KB), lane);
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

