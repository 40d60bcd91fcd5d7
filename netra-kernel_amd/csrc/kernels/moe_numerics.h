// Device numerics shared by the MoE kernels (gfx950, wave64).
//
// Every helper here is part of the layer's numeric contract: the same
// operation sequence is evaluated on the CPU by the test oracle, so the results
// are bit-identical. The kernels are compiled with -ffp-contract=off; every
// fused multiply-add below is an explicit fmaf().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nk {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// 1/448 rounded to fp32 (0x3b124925): the FP8 scale constant of the
// reference's quantisers (harness/gfx950/fp8/moe/decode/
// qwen36_moe_silu_mul_quant_fp8_gfx950.hip:35, silu_quant.inc:40).
__device__ __forceinline__ float inv_e4m3_max() { return __uint_as_float(0x3b124925u); }
constexpr float kAmaxFloor = 1.0e-10f;

__device__ __forceinline__ uint16_t bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

// OCP E4M3 (e4m3fn), round to nearest even, magnitudes >= 448 saturate,
// NaN -> 0x7f. Integer re-rounding of the fp32 mantissa; no table.
__device__ __forceinline__ uint32_t e4m3_rne(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  const float fa = __uint_as_float(a);
  if (fa >= 448.0f) return sign | 0x7eu;
  if (fa < 0.015625f) return sign | (uint32_t)rintf(fa * 512.0f);
  const uint32_t e = (a >> 23) - 127u + 7u;
  const uint32_t mant = a & 0x7fffffu;
  const uint32_t rounded = mant + 0x7ffffu + ((mant >> 20) & 1u);
  uint32_t code = (e << 3) + (rounded >> 20);
  code = code > 0x7eu ? 0x7eu : code;
  return sign | code;
}

// Four E4M3 encodings through the gfx950 conversion instruction
// (v_cvt_pk_fp8_f32: OCP e4m3fn, round to nearest even). Inputs are clamped to
// +-448 first, which reproduces the saturating rule of e4m3_rne for every
// finite input (netra_moe_e4m3_check compares the two on the device); NaN
// inputs, which the layer never produces from finite data, are outside the
// contract. Byte i of the result encodes argument i.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  a = fminf(fmaxf(a, -448.0f), 448.0f);
  b = fminf(fmaxf(b, -448.0f), 448.0f);
  c = fminf(fmaxf(c, -448.0f), 448.0f);
  d = fminf(fmaxf(d, -448.0f), 448.0f);
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// Contract exp: Cody-Waite reduction with n = rint(x log2 e), ln2 split into
// 0x3f317200 + 0x35bfbe8e (the hi/lo split of fdlibm's single-precision
// expf), degree-7 Taylor polynomial of e^r in Horner form,
// scaled by 2^n through the exponent field; x < -87 -> 0, x > 88 -> +inf.
__device__ __forceinline__ float nexp(float x) {
  if (x != x) return x;
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) return __uint_as_float(0x7f800000u);
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187045037746429443359375e-06f, r);
  float p = 1.98412701138295233249664306640625e-04f;
  p = fmaf(p, r, 1.388888922519981861114501953125e-03f);
  p = fmaf(p, r, 8.333333767950534820556640625e-03f);
  p = fmaf(p, r, 4.1666667163372039794921875e-02f);
  p = fmaf(p, r, 1.6666667163372039794921875e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  return p * __uint_as_float((uint32_t)(ni + 127) << 23);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + nexp(-g)); }

// Epilogue forms for the GEMMs, whose outputs are checked against the oracle
// within a tolerance (their fp32 accumulation order differs from it anyway):
// SiLU through the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32, about
// 1 ulp each), and bf16 rounding through the gfx950 conversion
// (v_cvt_pk_bf16_f32, round to nearest even, the same value as bf16_rne for
// every non-NaN input).
__device__ __forceinline__ float silu_hw(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
}
__device__ __forceinline__ float bf16_round_hw(float x) { return (float)(__bf16)x; }
// Two floats to packed bf16 (low half first) by one v_cvt_pk_bf16_f32: the
// bits of bf16_rne for every non-NaN input, without its NaN branch.
__device__ __forceinline__ uint32_t bf16x2_hw(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float sigmoid(float z) { return 1.0f / (1.0f + nexp(-z)); }

// 32 contiguous FP8 bytes as one MFMA operand (two 16-byte loads).
__device__ __forceinline__ v8i load_fp8x32(const uint8_t* p) {
  const uint4 lo = *reinterpret_cast<const uint4*>(p);
  const uint4 hi = *reinterpret_cast<const uint4*>(p + 16);
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}

// Packed expert-weight layout ("tile16x128"): a [N, K] e4m3 matrix is stored
// as N/16 x K/128 tiles of 2 KiB, row tiles outermost, so a 16-row tile's full
// K extent is contiguous. Lane l's MFMA operand (row l & 15, columns
// (l >> 4) * 32 .. +31) is split in two 16-byte halves stored at l * 16 and
// 1024 + l * 16: each of the wave's two 16-byte loads reads 1 KiB contiguous.
// W13 stores its row tiles gate/up interleaved: logical row tile t of a
// [2I, K] matrix (gate rows 0 .. I-1, up rows I .. 2I-1) is stored at
// 2 t (gate) or 2 (t - I/16) + 1 (up), n2i = 2I rows.
__host__ __device__ __forceinline__ uint32_t gu_tile(uint32_t t, uint32_t n2i) {
  const uint32_t half = n2i / 32u;  // gate row tiles
  return t < half ? 2u * t : 2u * (t - half) + 1u;
}

__device__ __forceinline__ const uint8_t* tile_base(const uint8_t* matrix, uint32_t row_tile,
                                                    uint32_t kb, uint32_t kblocks) {
  return matrix + ((size_t)row_tile * kblocks + kb) * 2048u;
}

__device__ __forceinline__ v8i load_tile_operand(const uint8_t* tile, uint32_t lane) {
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + lane * 16u);
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + 1024u + lane * 16u);
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}

// The same operand with non-temporal loads, for weights a launch reads once:
// streaming a 480 MB weight set this way runs at 6.8 TB/s on one MI355X
// against 6.3 TB/s with ordinary loads (the decode GEMMs, where every expert
// tile is read by one workgroup).
__device__ __forceinline__ v8i load_tile_operand_once(const uint8_t* tile, uint32_t lane) {
  const u32x4 lo = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + lane * 16u));
  const u32x4 hi = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + 1024u + lane * 16u));
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}

// The reference's weight layout ("aiter_shuffle_16x16_fp8_block128",
// compiler/netra_compiler/layouts.py:90-106): [N, K] bytes stored as
// [N/16][K/32][2][16][16], i.e. element (n, k) at
// [n/16][k/32][(k%32)/16][n%16][k%16]. Like tile16x128 it keeps a 16-row
// tile's K extent contiguous and one (16-row, 128-K) block in 2 KiB, so row
// tiles and K blocks are addressed the same way (tile_base); only the place of
// a lane's two 16-byte operand halves inside the block differs: the 32-K chunk
// (l >> 4) is 512 bytes, its low K half of rows 0..15 first, then the high
// half. Each half-operand wave load reads four 256-byte runs.
template <bool kAiter>
__host__ __device__ __forceinline__ uint32_t operand_lo(uint32_t lane) {
  return kAiter ? lane * 16u + (lane >> 4) * 256u : lane * 16u;
}
template <bool kAiter>
__host__ __device__ __forceinline__ uint32_t operand_hi(uint32_t lane) {
  return kAiter ? lane * 16u + (lane >> 4) * 256u + 256u : 1024u + lane * 16u;
}

template <bool kAiter>
__device__ __forceinline__ v8i load_block_operand(const uint8_t* tile, uint32_t lane) {
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + operand_lo<kAiter>(lane));
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + operand_hi<kAiter>(lane));
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}

// The same operand through a raw buffer resource (SGPR base, per-lane offset
// lane * 16 and a uniform scalar offset per tile): a run of tiles costs one
// address VGPR instead of a 64-bit address per load. Loads past `bytes`
// return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
template <bool kAiter = false>
__device__ __forceinline__ v8i load_tile_operand(__amdgpu_buffer_rsrc_t r, uint32_t tile_offset,
                                                 uint32_t lane) {
  const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(r, (int)operand_lo<kAiter>(lane), (int)tile_offset, 0);
  const u32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(r, (int)operand_hi<kAiter>(lane), (int)tile_offset, 0);
  v8i v;
  v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
  v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
  return v;
}

// D = A(16x128 e4m3) * B(128x16 e4m3), fp32 accumulate. Lane l supplies row
// (l & 15) of A / column (l & 15) of B over K bytes [(l >> 4) * 32, +32); it
// receives D rows (l >> 4) * 4 + j, column (l & 15), j = 0..3.
__device__ __forceinline__ v4f mfma_e4m3_16x16x128(v8i a, v8i b) {
  v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
}

// Wave-wide unsigned max / min (every lane active): DPP inside each 16-lane
// row (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror), then the four row results combined from scalar readlanes.
template <bool kMax>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v) {
  auto pick = [](uint32_t a, uint32_t b) { return kMax ? (a > b ? a : b) : (a < b ? a : b); };
  v = pick(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = pick(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = pick(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = pick(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return pick(pick(a, b), pick(c, d));
}

// Wave-wide unsigned max with the result in every lane (every lane active):
// the same DPP row steps, then v_permlane16_swap (rows 0 <-> 1, 2 <-> 3) and
// v_permlane32_swap (the two halves), each followed by a max of the lane's
// own and swapped values: no scalar round trip.
__device__ __forceinline__ uint32_t wave_max_u32_all(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max((uint32_t)r16[0], (uint32_t)r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max((uint32_t)r32[0], (uint32_t)r32[1]);
}

// Order-preserving map of fp32 onto uint32 (larger float -> larger code);
// -0 is first folded onto +0 so the two compare equal. Finite and infinite
// inputs map to codes >= 0x007fffff, so 0 is free as an "absent" marker.
__device__ __forceinline__ uint32_t order_bits(float z) {
  uint32_t u = __float_as_uint(z);
  if (z == 0.0f) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_order_bits(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

}  // namespace nk
