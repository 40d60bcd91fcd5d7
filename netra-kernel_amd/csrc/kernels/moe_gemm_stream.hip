// Decode-regime grouped GEMMs: persistent HBM weight streaming.
//
// A work item is one 16-row tile of an expert block (from the sort's tile
// list) times one column tile, over the full K extent. Items of one tile are
// dealt to workgroups in groups of consecutive columns: the workgroup copies
// the tile's FP8 activation operand and scales into LDS once, and each wave
// streams the weight tiles of its own columns in K steps. The weights of the
// next step are issued before the current step's MFMAs wait, so the in-order
// load counter never drains the prefetched data, and waves synchronise only
// at group boundaries.
//
// gate/up computes h = bf16(silu(g) * u) and requantises every (16-row tile,
// 128-column block) of it to the FP8 operand plus row scales before it leaves
// the workgroup (the SiLU-quant step of the reference's decode trio); down
// streams W2 against it and writes fp32 route partials.
// Symbols: netra_moe_gate_up_stream_h<H>_gfx950, netra_moe_down_stream_i<I>_gfx950.
#pragma once
#include "moe_numerics.h"

#define NK_KERNEL extern "C" __global__

// Resident waves per SIMD the stream kernels are register-budgeted for
// (gate/up's grid fills the chip once at this occupancy).
#ifndef NK_GATE_UP_WAVES_PER_EU
#define NK_GATE_UP_WAVES_PER_EU 2
#endif
#ifndef NK_DOWN_WAVES_PER_EU
#define NK_DOWN_WAVES_PER_EU 4
#endif

namespace nkstream {

// Barrier for LDS hand-off only: waits for this wave's LDS traffic, not for its
// outstanding global loads (__syncthreads would wait for those too).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// Routing metadata of one 16-row tile. row0 and expert are uniform; lane l
// holds row (l & 15): its token (gate/up) or route t * Ktot + slot (down),
// -1 for padding rows.
struct TileRows {
  uint32_t row0 = 0;
  int32_t expert = 0;
  int32_t row = -1;
};

// The tile of rows row0 .. row0 + 15 of block b.
__device__ __forceinline__ void load_rows(TileRows& tr, const int32_t* __restrict__ sorted_ids,
                                          const int32_t* __restrict__ sorted_expert, uint32_t b, uint32_t row0,
                                          uint32_t T, uint32_t Ktot, uint32_t Etot, bool as_route) {
  tr.row0 = row0;
  const int32_t e = sorted_expert[b];
  tr.expert = (e < 0 || (uint32_t)e >= Etot) ? 0 : e;  // out of range only for malformed routing
  const int32_t id = sorted_ids[tr.row0 + (threadIdx.x & 15u)];
  const uint32_t t = (uint32_t)id & 0xffffffu, slot = (uint32_t)id >> 24;
  tr.row = (t < T && slot < Ktot) ? (int32_t)(as_route ? t * Ktot + slot : t) : -1;
}

// max_block bounds the block a tile_map entry names (an entry past the tile
// count, read ahead of it, may hold stale bytes).
__device__ __forceinline__ void load_tile(TileRows& tr, const int32_t* __restrict__ tile_map,
                                          const int32_t* __restrict__ sorted_ids,
                                          const int32_t* __restrict__ sorted_expert, uint32_t tile,
                                          uint32_t T, uint32_t Ktot, uint32_t Etot, bool as_route,
                                          uint32_t max_block = 0xffffffffu) {
  const uint32_t m = (uint32_t)tile_map[tile];
  const uint32_t b = min(m >> 2, max_block);
  load_rows(tr, sorted_ids, sorted_expert, b, b * 64u + (m & 3u) * 16u, T, Ktot, Etot, as_route);
}

}  // namespace nkstream

// ---------------------------------------------------------------------------
// (reference: kernels/gfx950/templates/moe/decode/gate_up_mfma.inc:12-161 and
// silu_quant.inc:16-236; oracle tools/benchmark/export_qwen36_moe_stage1_capture.py:80-97,
// quant rule harness/gfx950/fp8/moe/decode/qwen36_moe_silu_mul_quant_fp8_gfx950.hip:57-94)
//
// Item (tile, c): h columns [16 c, 16 c + 16) of one 16-row tile, i.e. W13
// rows n (gate) and I + n (up), over the full K extent; per 128-wide K block
// acc += w_s * (a_s * mfma) (mfma.inc:20-24) in ascending K order, and after
// the last block h = bf16_rne(silu(g) * u).
//
// Work is dealt in groups of Q = 8 P consecutive columns of one tile (P, the
// items per wave, a power of two <= 4 with Q dividing the tile's I / 16
// columns), so a group covers P whole 128-column blocks of h. Workgroup w
// (8 waves) takes groups w, w + gridDim.x, ... For a group it stages the
// tile's FP8 activation rows (16 x H, in the MFMA operand layout) and their
// scales in LDS once, and each wave then streams only the W13 tiles of its P
// columns, in steps of CH K blocks, one step ahead. (Loading the 16
// gathered activation rows from L2 at every step as well doubled the
// cache-line requests per step and held the weight stream at ~5.1 TB/s.)
// Each item's 16 x 16 bf16 h block goes to LDS; when the group is done, waves
// 0 .. P-1 requantise one 128-column block each by the 1x128 rule
// (scale = max(amax, 1e-10) * 0x3b124925, q = e4m3(h * (1 / scale))) and
// write it in the tile16x128 operand layout with its 16 row scales, which is
// what the down GEMM loads.
constexpr uint32_t kGuWaves = 8;
constexpr uint32_t kGuMaxP = 4;

template <uint32_t CH>
struct GateUpStep {
  nk::v8i g[CH], u[CH];
  float ws;  // lane i < KB: gate block scale of K block i; KB <= i < 2 KB: up block scale of K block i - KB
};

template <uint32_t KB, uint32_t CH>  // H / 128, K blocks per step
__device__ __forceinline__ void gate_up_stream(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs,
    const uint8_t* __restrict__ w13, const float* __restrict__ w13s,
    const int32_t* __restrict__ sorted_ids, const int32_t* __restrict__ sorted_expert,
    const int32_t* __restrict__ tile_map, const int32_t* __restrict__ num_valid,
    uint8_t* __restrict__ hq, float* __restrict__ hs, uint32_t T, uint32_t I, uint32_t Ktot,
    uint32_t Etot) {
  using namespace nkstream;
  constexpr uint32_t H = 128 * KB;
  constexpr uint32_t NCH = KB / CH;
  constexpr uint32_t kThreads = 64u * kGuWaves;
  constexpr uint32_t kHbStride = 128u * kGuMaxP + 8u;  // bf16 per LDS h row (+16 bytes rotates banks)
  static_assert(KB % (2 * CH) == 0, "an even step count per item");
  static_assert(H % kThreads == 0, "staging moves H / 512 pieces per thread");
  __shared__ __align__(16) uint8_t s_a[KB * 2048u];  // the tile's activations, operand layout per K block
  __shared__ float s_xs[16 * KB];                    // their scales, [row][kb]
  __shared__ __align__(16) uint16_t s_hb[16 * kHbStride];  // the group's h rows (bf16)
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = wave_id();
  const uint32_t cols = I / 16u, KBI = I / 128u;
  // tiles as the sort counted them, never past the capacity (T Ktot / 16 + Etot):
  // an operation launched out of order may find another tensor's bytes here
  const uint32_t ntiles = min((uint32_t)num_valid[2], (T * Ktot + 15u) / 16u + Etot);
  const uint32_t items = ntiles * cols;
  const uint32_t waves_total = gridDim.x * kGuWaves;
  uint32_t P = 1u;  // items per wave
  while (P < kGuMaxP && P * waves_total < items && cols % (16u * P) == 0u) P <<= 1;
  const uint32_t Q = kGuWaves * P, groups = items / Q;
  const uint32_t nsteps = P * NCH;

  nk::v4f ag = {0.0f, 0.0f, 0.0f, 0.0f}, au = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
  for (uint32_t grp = blockIdx.x; grp < groups; grp += gridDim.x) {
    const uint32_t item0 = grp * Q, tile = item0 / cols;
    const uint32_t cg = item0 - tile * cols;  // the group's first column
    const uint32_t c0 = cg + wave * P;        // this wave's first column
    TileRows m;
    load_tile(m, tile_map, sorted_ids, sorted_expert, tile, T, Ktot, Etot, false);
    const uint8_t* we = w13 + (size_t)m.expert * 2u * I * H;
    const float* wse = w13s + (size_t)m.expert * (2u * I / 128u) * KB;
    // Weight scales come in with a vector load (in order with the weights on
    // the vector-memory counter): scalar loads would share the LDS counter,
    // and their out-of-order returns make every LDS wait a full drain.
    auto issue = [&](GateUpStep<CH>& st, uint32_t s) __attribute__((always_inline)) {
      const uint32_t c = c0 + s / NCH, ch = s % NCH;
#pragma unroll
      for (uint32_t i = 0; i < CH; ++i) {
        const uint32_t kb = ch * CH + i;
        st.g[i] = nk::load_tile_operand(nk::tile_base(we, 2u * c, kb, KB), lane);        // gate tile c
        st.u[i] = nk::load_tile_operand(nk::tile_base(we, 2u * c + 1u, kb, KB), lane);   // up tile c
      }
      // 128-row scale blocks of gate rows 16c.. and up rows I + 16c..
      const uint32_t sl = lane < 2u * KB ? lane : 0u;
      st.ws = wse[((sl < KB ? c : I / 16u + c) >> 3) * KB + (sl < KB ? sl : sl - KB)];
    };
    // Stage the tile: 16 rows x H bytes in 16-byte pieces; lane l of K block
    // kb's operand holds row l & 15, bytes (l >> 4) * 32 .. +31 (lo half at
    // l * 16, hi half at 1024 + l * 16). The pieces are loaded before the
    // first weight step is issued, so waiting for them does not drain the
    // weight stream. (s_a and s_hb are free: the previous group ended with a
    // barrier after its last MFMA, and its requant reads finish before the
    // requant waves reach the barrier below.)
    constexpr uint32_t kPieces = H / kThreads, kScales = (16u * KB + kThreads - 1u) / kThreads;
    uint4 av[kPieces];
#pragma unroll
    for (uint32_t q = 0; q < kPieces; ++q) {
      const uint32_t p = tid + q * kThreads, row = p / (H / 16u), k = (p % (H / 16u)) * 16u;
      const int32_t t = __shfl(m.row, row);
      av[q] = *reinterpret_cast<const uint4*>(xq + (size_t)(t < 0 ? 0 : t) * H + k);
    }
    float xv[kScales];
#pragma unroll
    for (uint32_t q = 0; q < kScales; ++q) {
      const uint32_t i = tid + q * kThreads;
      const int32_t t = __shfl(m.row, (i / KB) & 15u);
      xv[q] = i < 16u * KB ? xs[(size_t)(t < 0 ? 0 : t) * KB + i % KB] : 0.0f;
    }
    GateUpStep<CH> b0, b1;
    issue(b0, 0u);
#pragma unroll
    for (uint32_t q = 0; q < kPieces; ++q) {
      const uint32_t p = tid + q * kThreads, row = p / (H / 16u), k = (p % (H / 16u)) * 16u;
      const uint32_t kb = k >> 7, kk = k & 127u;
      *reinterpret_cast<uint4*>(&s_a[kb * 2048u + ((kk >> 4) & 1u) * 1024u + ((kk >> 5) * 16u + row) * 16u]) = av[q];
    }
#pragma unroll
    for (uint32_t q = 0; q < kScales; ++q)
      if (tid + q * kThreads < 16u * KB) s_xs[tid + q * kThreads] = xv[q];
    lds_barrier();

    auto compute = [&](const GateUpStep<CH>& st, uint32_t s) __attribute__((always_inline)) {
      const uint32_t ch = s % NCH;
#pragma unroll
      for (uint32_t i = 0; i < CH; ++i) {
        const uint32_t kb = ch * CH + i;
        const nk::v8i a = nk::load_tile_operand(s_a + kb * 2048u, lane);
        const nk::v4f dg = nk::mfma_e4m3_16x16x128(a, st.g[i]);
        const nk::v4f du = nk::mfma_e4m3_16x16x128(a, st.u[i]);
        const float sg = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(st.ws), (int)kb));
        const float su = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(st.ws), (int)(KB + kb)));
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          const float as = s_xs[((lane >> 4) * 4u + j) * KB + kb];
          ag[j] = ag[j] + sg * (as * dg[j]);
          au[j] = au[j] + su * (as * du[j]);
        }
      }
      if (ch == NCH - 1u) {  // the item's 16 x 16 h block -> the group's LDS rows
        const uint32_t col = (c0 + s / NCH - cg) * 16u + (lane & 15u);
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j)
          s_hb[((lane >> 4) * 4u + j) * kHbStride + col] = nk::bf16_rne(nk::silu(ag[j]) * au[j]);
        ag = nk::v4f{0.0f, 0.0f, 0.0f, 0.0f};
        au = nk::v4f{0.0f, 0.0f, 0.0f, 0.0f};
      }
    };
    // Two step buffers, two steps per iteration (nsteps is even): step s + 1
    // is in flight while step s computes. No load is issued under a branch:
    // the compiler's load-counter bookkeeping merges branch paths
    // conservatively and would drain the prefetch at the join, so the last
    // prefetch reloads the final step instead of being skipped.
#pragma unroll 1
    for (uint32_t s = 0; s < nsteps; s += 2u) {
      issue(b1, s + 1u);
      __builtin_amdgcn_sched_barrier(0);  // keep step s + 1's loads ahead of step s's MFMAs
      compute(b0, s);
      issue(b0, s + 2u < nsteps ? s + 2u : nsteps - 1u);
      __builtin_amdgcn_sched_barrier(0);
      compute(b1, s + 1u);
    }
    lds_barrier();  // every wave's h blocks are in LDS, and s_a is no longer read

    // 1x128 requant: wave w < P takes the group's 128-column block w; lane l
    // holds row l & 15, columns (l >> 4) * 32 .. +31 of it, and the four lanes
    // of a row combine their maxima.
    if (wave < P) {
      const uint16_t* src = &s_hb[(lane & 15u) * kHbStride + wave * 128u + (lane >> 4) * 32u];
      uint4 raw[4];
#pragma unroll
      for (uint32_t q = 0; q < 4; ++q) raw[q] = *reinterpret_cast<const uint4*>(src + 8u * q);
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
      const size_t blk = (size_t)(m.row0 >> 4) * KBI + (cg >> 3) + wave;  // (16-row tile, 128-column block)
      uint8_t* dst = hq + blk * 2048u;
      *reinterpret_cast<uint4*>(dst + lane * 16u) = lo;
      *reinterpret_cast<uint4*>(dst + 1024u + lane * 16u) = hi;
      if (lane < 16u) hs[blk * 16u + lane] = scale;
    }
  }
}

#define NK_GATE_UP_STREAM_V(NAME, HV, CH, WPE)                                                   \
  NK_KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(WPE)))                     \
  void NAME(                                                                                     \
      const uint8_t* __restrict__ xq, const float* __restrict__ xs,                              \
      const uint8_t* __restrict__ w13, const float* __restrict__ w13s,                           \
      const int32_t* __restrict__ sorted_ids, const int32_t* __restrict__ sorted_expert,         \
      const int32_t* __restrict__ tile_map, const int32_t* __restrict__ num_valid,               \
      uint8_t* __restrict__ hq, float* __restrict__ hs, uint32_t T, uint32_t H, uint32_t I,      \
      uint32_t Ktot, uint32_t Etot) {                                                            \
    (void)H;                                                                                     \
    gate_up_stream<HV / 128, CH>(xq, xs, w13, w13s, sorted_ids, sorted_expert, tile_map, num_valid, \
                             hq, hs, T, I, Ktot, Etot);                                          \
  }
// Symbol netra_moe_gate_up_stream_h<H>_c<CH>_gfx950: CH K blocks per step.
#define NK_GATE_UP_STREAM(HV, CH) \
  NK_GATE_UP_STREAM_V(netra_moe_gate_up_stream_h##HV##_c##CH##_gfx950, HV, CH, NK_GATE_UP_WAVES_PER_EU)
NK_GATE_UP_STREAM(512, 2)
NK_GATE_UP_STREAM(1024, 2)
NK_GATE_UP_STREAM(1024, 4)
NK_GATE_UP_STREAM(2048, 2)
NK_GATE_UP_STREAM(2048, 4)
NK_GATE_UP_STREAM(4096, 2)
NK_GATE_UP_STREAM(4096, 4)

// ---------------------------------------------------------------------------
// (reference: kernels/gfx950/templates/moe/decode/down_reduce_mfma_2wave.inc:
// 14-291; oracle tools/benchmark/export_qwen36_moe_stage2_capture.py:90-110)
//
// Item (tile, c): output columns [32 c, 32 c + 32) (two 16-row W2 tiles) of
// one 16-row tile; DC 128-wide K blocks per step; per block
// acc += w_s * (a_s * mfma). After the last step each valid row's fp32 result
// goes to partial[route].
//
// As in gate/up, work is dealt in groups of Q = 4 P consecutive columns of one
// tile (P, the items per wave, a power of two with Q dividing H / 32):
// workgroup w (4 waves) takes groups w, w + gridDim.x, ... and copies the
// tile's FP8 A operand (the gate/up epilogue's output: KB contiguous 2 KiB
// operand tiles) and its row scales into LDS once; each wave then streams
// only the W2 tiles of its P columns, one step ahead.
constexpr uint32_t kDnWaves = 4;
constexpr uint32_t kDnMaxP = 16;

template <uint32_t DC>
struct DownStep {
  nk::v8i w[DC][2];
  float ws;  // lane 2 i + t: w_s of 16-row tile t's block at the step's K block i (vector load)
};

template <uint32_t KB, uint32_t DC>  // I / 128, K blocks per step
__device__ __forceinline__ void down_stream(
    const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2,
    const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ tile_map,
    const int32_t* __restrict__ num_valid, float* __restrict__ partial, uint32_t T, uint32_t H,
    uint32_t Ktot, uint32_t Etot) {
  using namespace nkstream;
  constexpr uint32_t I = 128 * KB;
  constexpr uint32_t NCH = KB / DC;
  constexpr uint32_t kThreads = 64u * kDnWaves;
  constexpr uint32_t kPieces = KB * 128u / kThreads;  // 16-byte pieces of the A operand per thread
  static_assert(KB % (2 * DC) == 0, "an even step count per item");
  static_assert(KB * 128u % kThreads == 0, "A operand copy");
  __shared__ __align__(16) uint8_t s_a[KB * 2048u];  // the tile's A operand, KB operand tiles
  __shared__ __align__(16) float s_as[KB * 16u];     // its row scales, [kb][row]
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = wave_id();
  const uint32_t cols = H / 32u;
  // tiles as the sort counted them, never past the capacity (T Ktot / 16 + Etot):
  // an operation launched out of order may find another tensor's bytes here
  const uint32_t ntiles = min((uint32_t)num_valid[2], (T * Ktot + 15u) / 16u + Etot);
  const uint32_t items = ntiles * cols;
  const uint32_t waves_total = gridDim.x * kDnWaves;
  uint32_t P = 1u;  // items per wave
  while (P < kDnMaxP && P * waves_total < items && cols % (8u * P) == 0u) P <<= 1;
  const uint32_t Q = kDnWaves * P, groups = items / Q;
  const uint32_t nsteps = P * NCH;

  nk::v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
  for (uint32_t grp = blockIdx.x; grp < groups; grp += gridDim.x) {
    const uint32_t item0 = grp * Q, tile = item0 / cols;
    const uint32_t c0 = item0 - tile * cols + wave * P;  // this wave's first column
    TileRows m;
    load_tile(m, tile_map, sorted_ids, sorted_expert, tile, T, Ktot, Etot, true);
    const uint8_t* we = w2 + (size_t)m.expert * H * I;
    const float* wse = w2s + (size_t)m.expert * (H / 128u) * KB;
    // weight scales by a vector load (scalar loads would share the LDS
    // counter, and their out-of-order returns make every LDS wait a full drain)
    auto issue = [&](DownStep<DC>& st, uint32_t s) __attribute__((always_inline)) {
      const uint32_t c = c0 + s / NCH, kb0 = (s % NCH) * DC;
#pragma unroll
      for (uint32_t i = 0; i < DC; ++i)
#pragma unroll
        for (uint32_t t2 = 0; t2 < 2; ++t2)
          st.w[i][t2] = nk::load_tile_operand(nk::tile_base(we, c * 2u + t2, kb0 + i, KB), lane);
      const uint32_t li = (lane >> 1) < DC ? lane >> 1 : 0u;
      st.ws = wse[((c * 2u + (lane & 1u)) >> 3) * KB + kb0 + li];
    };
    // the tile's operand and scales, loaded before the first weight step is
    // issued so that waiting for them does not drain the weight stream
    const size_t tile16 = m.row0 >> 4;
    const uint4* asrc = reinterpret_cast<const uint4*>(hq + tile16 * KB * 2048u);
    uint4 av[kPieces];
#pragma unroll
    for (uint32_t q = 0; q < kPieces; ++q) av[q] = asrc[tid + q * kThreads];
    float4 sv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (tid < KB * 4u) sv = reinterpret_cast<const float4*>(hs + tile16 * KB * 16u)[tid];
    DownStep<DC> b0, b1;
    issue(b0, 0u);
#pragma unroll
    for (uint32_t q = 0; q < kPieces; ++q) reinterpret_cast<uint4*>(s_a)[tid + q * kThreads] = av[q];
    if (tid < KB * 4u) reinterpret_cast<float4*>(s_as)[tid] = sv;
    lds_barrier();

    auto compute = [&](const DownStep<DC>& st, uint32_t s) __attribute__((always_inline)) {
      const uint32_t ch = s % NCH;
#pragma unroll
      for (uint32_t i = 0; i < DC; ++i) {
        const uint32_t kb = ch * DC + i;
        const nk::v8i a = nk::load_tile_operand(s_a + kb * 2048u, lane);
        const float4 as4 = *reinterpret_cast<const float4*>(&s_as[kb * 16u + (lane >> 4) * 4u]);
        const float as[4] = {as4.x, as4.y, as4.z, as4.w};
        const nk::v4f d0 = nk::mfma_e4m3_16x16x128(a, st.w[i][0]);
        const nk::v4f d1 = nk::mfma_e4m3_16x16x128(a, st.w[i][1]);
        const float s0 = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(st.ws), (int)(2u * i)));
        const float s1 = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(st.ws), (int)(2u * i + 1u)));
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          acc0[j] = acc0[j] + s0 * (as[j] * d0[j]);
          acc1[j] = acc1[j] + s1 * (as[j] * d1[j]);
        }
      }
      if (ch == NCH - 1u) {
        const uint32_t c = c0 + s / NCH;
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
    // Two step buffers, two steps per iteration (nsteps is even): step s + 1
    // is in flight while step s computes; no load is issued under a branch
    // (the last prefetch reloads the final step).
#pragma unroll 1
    for (uint32_t s = 0; s < nsteps; s += 2u) {
      issue(b1, s + 1u);
      __builtin_amdgcn_sched_barrier(0);  // keep step s + 1's loads ahead of step s's MFMAs
      compute(b0, s);
      issue(b0, s + 2u < nsteps ? s + 2u : nsteps - 1u);
      __builtin_amdgcn_sched_barrier(0);
      compute(b1, s + 1u);
    }
    lds_barrier();  // s_a and s_as are free for the next group
  }
}

#define NK_DOWN_STREAM_V(NAME, IV, DC, WPE)                                                     \
  NK_KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE)))                     \
  void NAME(                                                                                    \
      const uint8_t* __restrict__ hq, const float* __restrict__ hs, const uint8_t* __restrict__ w2, \
      const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,                    \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ tile_map,          \
      const int32_t* __restrict__ num_valid, float* __restrict__ partial, uint32_t T,           \
      uint32_t H, uint32_t I, uint32_t Ktot, uint32_t Etot) {                                   \
    (void)I;                                                                                    \
    down_stream<IV / 128, DC>(hq, hs, w2, w2s, sorted_ids, sorted_expert, tile_map, num_valid,  \
                          partial, T, H, Ktot, Etot);                                           \
  }
// Symbol netra_moe_down_stream_i<I>_c<DC>_gfx950: DC K blocks per step.
#define NK_DOWN_STREAM(IV, DC) \
  NK_DOWN_STREAM_V(netra_moe_down_stream_i##IV##_c##DC##_gfx950, IV, DC, NK_DOWN_WAVES_PER_EU)
NK_DOWN_STREAM(256, 1)
NK_DOWN_STREAM(512, 1)
NK_DOWN_STREAM(512, 2)
NK_DOWN_STREAM(1024, 1)
NK_DOWN_STREAM(1024, 2)
NK_DOWN_STREAM(2048, 1)
NK_DOWN_STREAM(2048, 2)
