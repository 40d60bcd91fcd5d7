// Top-k weighted combine and the weight-preparation quantiser.
#pragma once
#include "moe_numerics.h"

#define NK_KERNEL extern "C" __global__

// ---------------------------------------------------------------------------
// Top-k weighted combine (reference: kernels/gfx950/templates/moe/prefill/
// route_reduce_splitk2_f16.inc:6-117 and down_reduce_mfma_2wave.inc:202-213:
// slot-ordered weighted sum, then bf16). out[t, n] = bf16(sum over slots in
// order of fmaf(w[t, s], partial[t * Ktot + s, n], acc)).
// Up to kCombineBatch slots' partial rows are requested before the first fmaf,
// so a token waits on memory once per batch rather than once per slot.
constexpr uint32_t kCombineBatch = 16;

NK_KERNEL __launch_bounds__(256) void netra_moe_combine_gfx950(
    const float* __restrict__ partial, const float* __restrict__ weights,
    uint16_t* __restrict__ out, uint32_t T, uint32_t H, uint32_t Ktot) {
  const uint32_t t = blockIdx.y;
  const uint32_t n = (blockIdx.x * 256u + threadIdx.x) * 4u;
  if (t >= T || n >= H) return;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  const float* prow = partial + (size_t)t * Ktot * H + n;
  for (uint32_t s0 = 0; s0 < Ktot; s0 += kCombineBatch) {
    float4 p[kCombineBatch];
    float w[kCombineBatch];
#pragma unroll
    for (uint32_t i = 0; i < kCombineBatch; ++i) {
      if (s0 + i < Ktot) {
        p[i] = *reinterpret_cast<const float4*>(prow + (size_t)(s0 + i) * H);
        w[i] = weights[(size_t)t * Ktot + s0 + i];
      }
    }
#pragma unroll
    for (uint32_t i = 0; i < kCombineBatch; ++i) {
      if (s0 + i < Ktot) {
        a0 = fmaf(w[i], p[i].x, a0);
        a1 = fmaf(w[i], p[i].y, a1);
        a2 = fmaf(w[i], p[i].z, a2);
        a3 = fmaf(w[i], p[i].w, a3);
      }
    }
  }
  uint2 o;
  o.x = (uint32_t)nk::bf16_rne(a0) | ((uint32_t)nk::bf16_rne(a1) << 16);
  o.y = (uint32_t)nk::bf16_rne(a2) | ((uint32_t)nk::bf16_rne(a3) << 16);
  *reinterpret_cast<uint2*>(out + (size_t)t * H + n) = o;
}

// The same combine over bf16 route partials (the tile-path down GEMM's output,
// as the reference's prefill route reducer reads 16-bit partials): eight
// columns per lane, fp32 accumulation in slot order, bf16 out.
NK_KERNEL __launch_bounds__(256) void netra_moe_combine_bf16_gfx950(
    const uint16_t* __restrict__ partial, const float* __restrict__ weights,
    uint16_t* __restrict__ out, uint32_t T, uint32_t H, uint32_t Ktot) {
  const uint32_t t = blockIdx.y;
  const uint32_t n = (blockIdx.x * 256u + threadIdx.x) * 8u;
  if (t >= T || n >= H) return;
  float a[8];
#pragma unroll
  for (uint32_t i = 0; i < 8; ++i) a[i] = 0.0f;
  const uint16_t* prow = partial + (size_t)t * Ktot * H + n;
  for (uint32_t s0 = 0; s0 < Ktot; s0 += kCombineBatch) {
    uint4 p[kCombineBatch];
    float w[kCombineBatch];
#pragma unroll
    for (uint32_t i = 0; i < kCombineBatch; ++i) {
      if (s0 + i < Ktot) {
        p[i] = *reinterpret_cast<const uint4*>(prow + (size_t)(s0 + i) * H);
        w[i] = weights[(size_t)t * Ktot + s0 + i];
      }
    }
#pragma unroll
    for (uint32_t i = 0; i < kCombineBatch; ++i) {
      if (s0 + i < Ktot) {
        a[0] = fmaf(w[i], nk::bf16_lo(p[i].x), a[0]);
        a[1] = fmaf(w[i], nk::bf16_hi(p[i].x), a[1]);
        a[2] = fmaf(w[i], nk::bf16_lo(p[i].y), a[2]);
        a[3] = fmaf(w[i], nk::bf16_hi(p[i].y), a[3]);
        a[4] = fmaf(w[i], nk::bf16_lo(p[i].z), a[4]);
        a[5] = fmaf(w[i], nk::bf16_hi(p[i].z), a[5]);
        a[6] = fmaf(w[i], nk::bf16_lo(p[i].w), a[6]);
        a[7] = fmaf(w[i], nk::bf16_hi(p[i].w), a[7]);
      }
    }
  }
  uint4 o;
  o.x = (uint32_t)nk::bf16_rne(a[0]) | ((uint32_t)nk::bf16_rne(a[1]) << 16);
  o.y = (uint32_t)nk::bf16_rne(a[2]) | ((uint32_t)nk::bf16_rne(a[3]) << 16);
  o.z = (uint32_t)nk::bf16_rne(a[4]) | ((uint32_t)nk::bf16_rne(a[5]) << 16);
  o.w = (uint32_t)nk::bf16_rne(a[6]) | ((uint32_t)nk::bf16_rne(a[7]) << 16);
  *reinterpret_cast<uint4*>(out + (size_t)t * H + n) = o;
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

// ---------------------------------------------------------------------------
// Conversion self-check: the integer E4M3 encoder (the contract, shared with
// the CPU oracle) next to the hardware conversion the hot kernels use.
NK_KERNEL __launch_bounds__(256) void netra_moe_e4m3_check_gfx950(
    const float* __restrict__ in, uint8_t* __restrict__ sw, uint8_t* __restrict__ hw, uint32_t n) {
  const uint32_t i = (blockIdx.x * 256u + threadIdx.x) * 4u;
  if (i >= n) return;
  float v[4];
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) v[k] = (i + k < n) ? in[i + k] : 0.0f;
  const uint32_t h = nk::e4m3x4(v[0], v[1], v[2], v[3]);
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    if (i + k < n) {
      sw[i + k] = (uint8_t)nk::e4m3_rne(v[k]);
      hw[i + k] = (uint8_t)(h >> (8u * k));
    }
  }
}

// ---------------------------------------------------------------------------
// Weight layout change: row-major e4m3 [groups, n, k] -> tile16x128 (see
// nk::tile_base). One wave per 16 x 128 tile; lane l moves row l & 15,
// columns (l >> 4) * 32 .. +15 to tile offset l * 16 and columns +16 .. +31
// to 1024 + l * 16. With gate_up != 0 (W13: gate rows, then as many up rows)
// the row tiles are stored interleaved, gate tile t at 2 t and up tile t at
// 2 t + 1 (nk::gu_tile), so a gate/up tile pair is 2 x k/128 tiles contiguous.
NK_KERNEL __launch_bounds__(256) void netra_moe_pack_tiles_gfx950(
    const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t groups, uint32_t n,
    uint32_t k, uint32_t gate_up) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t tile = blockIdx.x * 4u + (threadIdx.x >> 6);
  const uint32_t nt = n / 16u, kb = k / 128u;
  if (tile >= groups * nt * kb) return;
  const uint32_t g = tile / (nt * kb), rt = (tile / kb) % nt, cb = tile % kb;
  const uint8_t* s = src + ((size_t)g * n + rt * 16u + (lane & 15u)) * k + cb * 128u + (lane >> 4) * 32u;
  const uint4 lo = *reinterpret_cast<const uint4*>(s);
  const uint4 hi = *reinterpret_cast<const uint4*>(s + 16);
  const uint32_t prt = gate_up ? nk::gu_tile(rt, n) : rt;
  uint8_t* d = dst + (((size_t)g * nt + prt) * kb + cb) * 2048u + lane * 16u;
  *reinterpret_cast<uint4*>(d) = lo;
  *reinterpret_cast<uint4*>(d + 1024) = hi;
}

// ---------------------------------------------------------------------------
// Weight layout change from the AITER 16x16 shuffle the reference's kernels
// consume (checkpoint layout "aiter_shuffle_16x16_fp8_block128",
// compiler/netra_compiler/layouts.py:90-106; its inverse is
// tools/benchmark/export_qwen36_dense_m1_capture.py:55-63): bytes of a
// [groups, n, k] e4m3 matrix stored as [n/16][k/32][2][16][16], i.e. row tile,
// 32-column group, 16-column half, row, byte. A 16 x 128 block of either
// layout is 2 KiB at the same place (row tiles outermost, k contiguous per row
// tile) made of eight 256-byte chunks (16 rows x 16 bytes); AITER orders the
// chunks (group, half), tile16x128 orders them (half, group). One wave per
// block moves 128 16-byte pieces; with gate_up != 0 the row tiles are stored
// gate/up-interleaved as by netra_moe_pack_tiles_gfx950.
NK_KERNEL __launch_bounds__(256) void netra_moe_pack_tiles_aiter_gfx950(
    const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t groups, uint32_t n,
    uint32_t k, uint32_t gate_up) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t tile = blockIdx.x * 4u + (threadIdx.x >> 6);
  const uint32_t nt = n / 16u, kb = k / 128u;
  if (tile >= groups * nt * kb) return;
  const uint32_t g = tile / (nt * kb), rt = (tile / kb) % nt, cb = tile % kb;
  const uint32_t prt = gate_up ? nk::gu_tile(rt, n) : rt;
  const uint8_t* s = src + (((size_t)g * nt + rt) * kb + cb) * 2048u;
  uint8_t* d = dst + (((size_t)g * nt + prt) * kb + cb) * 2048u;
#pragma unroll
  for (uint32_t q = 0; q < 2u; ++q) {
    const uint32_t piece = q * 64u + lane;        // destination order: chunk (half, group), row
    const uint32_t chunk = piece >> 4, row = piece & 15u;
    const uint32_t half = chunk >> 2, grp = chunk & 3u;
    const uint4 v = *reinterpret_cast<const uint4*>(s + (grp * 2u + half) * 256u + row * 16u);
    *reinterpret_cast<uint4*>(d + chunk * 256u + row * 16u) = v;
  }
}

// ---------------------------------------------------------------------------
// Plain 16-byte-per-lane copy of known size. Counter calibration: its
// FETCH_SIZE / WRITE_SIZE readings over a copy of B bytes convert the same
// counters' readings on the MoE kernels into HBM bytes, and its duration gives
// the achievable copy bandwidth of the box.
NK_KERNEL __launch_bounds__(256) void netra_moe_copy_gfx950(
    const uint4* __restrict__ src, uint4* __restrict__ dst, uint64_t n16) {
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}
