// Prefill gate/up GEMM with both operands staged through an LDS ring.
//
// A work item is (pair p, column group ng): the up to two 64-row blocks
// pair_map[p], pair_map[p] + 1 of one expert (128 routes) against that
// expert's 128 h columns [128 ng, 128 ng + 128) of gate and of up (256 W13
// rows), so each weight tile read serves 128 routes. Per 128-K block (a
// "step") the workgroup needs 16 KiB of activation rows and 32 KiB of weight
// tiles; both are copied global -> LDS by buffer loads with the
// LDS-destination bit (each wave instruction moves 1 KiB: lane l's 16 bytes
// land at M0 + 16 l), two steps ahead of use, into a ring of three stages, so
// no VGPRs hold operands in flight. Each step's copies for the next-but-one
// step are spread over its row tiles, so the load path works while the
// matrix core does. (A persistent variant that also ran the ring across work
// items measured slower: its step loop could not be unrolled without spills.)
//
// The copies are inline assembly waited for by explicit vmcnt counts: every
// wave issues the same six copies per step (seven in the tail variant below)
// and nothing else in the K loop touches vector memory, so "this wave's
// copies for step kb are done" is vmcnt <= 6 (7): the next step's copies. A
// barrier then makes every wave's
// copies visible to all, and (being after every read of the stage about to be
// refilled) keeps refills behind reads.
//
// The 8 waves split the 128 x 256 tile as 2 (row blocks) x 4 (32 h columns:
// 16 gate rows twice, 16 up rows twice); each holds 4 x 4 accumulators. Per
// step: acc += (w_s * a_s) * mfma. Epilogue: h = bf16(silu(g) * u) with the
// hardware exp2 / reciprocal / bf16 conversion (the GEMM outputs are checked
// within a tolerance), 1x128 FP8 requant, bytes through LDS to 16-byte stores.
// Weight tiles sit in LDS in the tile16x128 operand layout (every ds_read_b128
// 1 KiB contiguous across the wave); activation rows arrive as whole 128-byte
// lines, 8 lanes per row, into a row-major tile with swizzled 16-byte chunks
// (row_swizzle), whose operand reads are conflict-free as well. (Fetching
// them straight in the operand layout read every activation line half.)
//
// (reference: kernels/gfx950/templates/moe/decode/gate_up_mfma.inc:12-161,
// silu_quant.inc:16-236; oracle tools/benchmark/export_qwen36_moe_stage1_capture.py:80-97)
#pragma once
#include <type_traits>

#include "moe_numerics.h"

#define NK_KERNEL extern "C" __global__

namespace nklds {

using nk::u32x4;
using nk::v4f;
using nk::v8i;

constexpr uint32_t kThreads = 512;
constexpr uint32_t kStages = 3;
constexpr uint32_t kRowsPerBlock = 64;
constexpr uint32_t kRows = 128;                   // two blocks
constexpr uint32_t kTailTile = 8;                 // row tile of an absorbed tail (rows 128 .. 143)
constexpr uint32_t kAllRows = kRows + 16u;
constexpr uint32_t kABytes = 9u * 2048u;          // 8 row tiles + the tail tile
constexpr uint32_t kBBytes = 16u * 2048u;         // 8 gate + 8 up weight tiles
constexpr uint32_t kStageBytes = kABytes + kBBytes;
constexpr uint32_t kCopiesPerWave = 7;            // per step: A tile (2) + gate tile (2) + up tile (2) [+ tail share (1)]
constexpr uint32_t kFar = 0x80000000u;            // an offset past the activation range (T * H < 2^31): zeros

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)p;
}

// Raw buffer descriptor (base, num_records bytes, raw dword format) in SGPRs.
__device__ __forceinline__ u32x4 rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  u32x4 r;
  r.x = (uint32_t)a;
  r.y = (uint32_t)(a >> 32) & 0xffffu;
  r.z = bytes;
  r.w = 0x00020000u;
  return r;
}

// 16 bytes per lane, global (rsrc + voff + soff) -> LDS (m0 + 16 * lane).
// Offsets at or past num_records read as zeros without a memory access.
// The compiler's hazard recognizer does not look inside inline assembly, so
// the s_nop 4 supplies the five wait states a vector-memory instruction needs
// after a VALU write (v_readfirstlane, v_readlane, carry outputs) of an SGPR
// it reads (resource, offset), which also covers the M0 write before an
// LDS-destination load. The compiler treats m0 as a reserved register and
// does not honour it in a clobber list, so the copy saves m0 and puts it back
// (the LDS address is taken from m0 when the load issues): any value the
// compiler keeps in m0 survives the copy.
__device__ __forceinline__ void copy16(uint32_t m0, u32x4 r, uint32_t voff, uint32_t soff) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 4\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
               "s_mov_b32 m0, %0"
               : "=&s"(saved)
               : "s"(m0), "v"(voff), "s"(r), "s"(soff)
               : "memory");
}

// 4 bytes per lane, global (rsrc + voff + soff) -> LDS (m0 + 4 * lane); as copy16.
__device__ __forceinline__ void copy4(uint32_t m0, u32x4 r, uint32_t voff, uint32_t soff) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 4\n\tbuffer_load_dword %2, %3, %4 offen lds\n\t"
               "s_mov_b32 m0, %0"
               : "=&s"(saved)
               : "s"(m0), "v"(voff), "s"(r), "s"(soff)
               : "memory");
}

template <uint32_t N>
__device__ __forceinline__ void wait_copies() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Barrier for LDS hand-off: waits for this wave's LDS traffic, not for its
// copies in flight (a full __syncthreads would drain those).
__device__ __forceinline__ void barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Swizzle of the activation rows in LDS: a 16-row x 128-byte tile is stored
// row-major with the 16-byte chunk c of row r at position c ^ row_swizzle(r),
// so that each copy can fetch whole 128-byte lines (8 lanes per row) while the
// operand reads stay conflict-free: the 16 rows of one read land on 16
// distinct chunk positions within each 64-bank (or each 8-lane, 32-bank)
// pass.
__device__ __forceinline__ uint32_t row_swizzle(uint32_t r) { return (r ^ (r >> 3)) & 7u; }

// MFMA operand of a swizzled activation tile: lane l gets row l & 15, bytes
// 32 (l >> 4) .. + 31 (chunks 2 (l >> 4) and 2 (l >> 4) + 1).
__device__ __forceinline__ v8i lds_operand_rows(const uint8_t* tile, uint32_t lane) {
  const uint32_t r = lane & 15u, c = 2u * (lane >> 4), f = row_swizzle(r);
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + r * 128u + (c ^ f) * 16u);
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + r * 128u + ((c + 1u) ^ f) * 16u);
  v8i v;
  v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
  v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
  return v;
}

template <bool kAiter = false>
__device__ __forceinline__ v8i lds_operand(const uint8_t* tile, uint32_t lane) {
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + nk::operand_lo<kAiter>(lane));
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + nk::operand_hi<kAiter>(lane));
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}

// Item of workgroup i among n items, XCD-major (the hardware deals workgroup
// ids to the eight XCDs in turn); false when i has none.
__device__ __forceinline__ bool xcd_item(uint32_t i, uint32_t n, uint32_t& item) {
  const uint32_t per = (n + 7u) / 8u;
  item = (i % 8u) * per + i / 8u;
  return i / 8u < per && item < n;
}

// kAiter: W13 in the reference's AITER 16x16 shuffle (gate rows 0..I-1, up
// rows I..2I-1 as plain row tiles) instead of the gate/up-interleaved
// tile16x128 layout; the copies move the same 2 KiB blocks, only the up tile's
// place and the operand reads out of LDS differ.
template <uint32_t KB, bool kAiter = false>  // H / 128
__device__ __forceinline__ void gate_up_lds(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ w13,
    const float* __restrict__ w13s, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,
    const int32_t* __restrict__ pair_map, uint8_t* __restrict__ hq, float* __restrict__ hs, uint32_t T,
    uint32_t I, uint32_t Ktot, uint32_t Etot) {
  constexpr uint32_t H = 128u * KB;
  static_assert(2u * KB <= 64u && KB % 4u == 0, "scale copies");
  constexpr uint32_t kAsLanesPerRow = KB / 4u, kAsRowsPerCopy = 64u / kAsLanesPerRow;
  constexpr uint32_t kAsCopies = (kAllRows + kAsRowsPerCopy - 1u) / kAsRowsPerCopy;  // 1 KiB each
  static_assert(kAsCopies <= 9u, "scale copies: one per wave, plus one by wave 0");
  auto as_swizzle = [](uint32_t r) { return (r >> 2) & (kAsLanesPerRow - 1u); };
  __shared__ __align__(16) uint8_t s_stage[kStages][kStageBytes];
  __shared__ __align__(16) float s_as[kAsCopies * 256u];  // a_s(row, kb) at row * KB + kb (swizzled chunks)
  // a_s(row, kb): 16 consecutive rows of one kb fall in 16 distinct banks
  auto s_as_at = [&](uint32_t r, uint32_t kb) __attribute__((always_inline)) {
    return s_as[r * KB + (((kb >> 2) ^ as_swizzle(r)) << 2) + (kb & 3u)];
  };
  __shared__ __align__(16) float s_wsv[64];               // weight block scales: lane kb gate, KB + kb up
  __shared__ int32_t s_tok[kAllRows + 1u];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const uint32_t NG = I / 128u;
  uint32_t item;
  if (!xcd_item(blockIdx.x, (uint32_t)num_valid[3] * NG, item)) return;
  const uint32_t p = item / NG, ng = item - p * NG;
  const uint32_t nblocks = (uint32_t)num_valid[0] / kRowsPerBlock;
  const uint32_t b0 = (uint32_t)pair_map[p];
  if (b0 >= nblocks) return;
  // The rows' sorted ids, the first 17 of the next block, and the experts of
  // the blocks around the pair, in one round trip (the prologue's dependent
  // loads are the item's fixed cost). An expert whose rows end in a last
  // block of at most 16 rows (after an even number of full blocks) has that
  // tail computed by the item of the pair before it, as row tile 8: the
  // tail's own item would stream the expert's whole W13 slice again for a
  // few rows.
  const bool has2 = b0 + 1u < nblocks, has3 = b0 + 2u < nblocks;
  int32_t id = -1;
  if (tid < kRows) {
    if (tid < kRowsPerBlock || has2) id = sorted_ids[b0 * kRowsPerBlock + tid];
  } else if (tid <= kAllRows) {
    if (has3) id = sorted_ids[(b0 + 2u) * kRowsPerBlock + (tid - kRows)];
  }
  const int32_t e = sorted_expert[b0];
  const int32_t e2 = has2 ? sorted_expert[b0 + 1u] : -1;
  const int32_t e3 = has3 ? sorted_expert[b0 + 2u] : -1;
  const int32_t e4 = b0 + 3u < nblocks ? sorted_expert[b0 + 3u] : -1;
  const int32_t ep = b0 >= 1u ? sorted_expert[b0 - 1u] : -1;
  if (e < 0 || (uint32_t)e >= Etot) return;
  const bool two = e2 == e;
  if (tid <= kAllRows) {
    const uint32_t t = (uint32_t)id & 0xffffffu, slot = (uint32_t)id >> 24;
    s_tok[tid] = (id >= 0 && (tid < kRowsPerBlock || tid >= kRows || two) && t < T && slot < Ktot) ? (int32_t)t : -1;
  }
  __syncthreads();
  // absorb: the pair's expert continues in block b0 + 2 and ends there with
  // row 16 of it padding; skip: this single block is such a tail (the pair
  // before it takes it), so that item and this one agree
  const bool absorb = two && e3 == e && e4 != e && s_tok[kAllRows] < 0;
  if (!two && ep == e && s_tok[16] < 0) return;
  if (!absorb && tid >= kRows && tid < kAllRows) s_tok[tid] = -1;
  __syncthreads();
  const uint32_t m = wave >> 2, n = wave & 3u;  // row block, 32-column quarter
  const uint32_t nvalid = (uint32_t)__popcll(__ballot(s_tok[m * kRowsPerBlock + lane] >= 0));
  const uint32_t ntiles = (nvalid + 15u) >> 4;
  // copy sources: wave w moves A row tile w and weight tiles w of gate and of up.
  // A copy h fetches rows 8 h .. 8 h + 7 of the tile as whole 128-byte lines:
  // lane l takes row 8 h + (l >> 3), the chunk its swizzled slot l & 7 holds
  uint32_t avoff[2];
#pragma unroll
  for (uint32_t h = 0; h < 2u; ++h) {
    const uint32_t r = 8u * h + (lane >> 3);
    const int32_t atok = s_tok[wave * 16u + r];
    avoff[h] = atok >= 0 ? (uint32_t)atok * H + (((lane & 7u) ^ row_swizzle(r)) * 16u) : kFar;
  }
  // the tail tile's half w & 1 (rows 8 (w & 1) .. + 7, as an A copy): every
  // wave copies one half, so four waves write the same bytes to the same
  // place and each wave still issues seven copies per step with no branch in
  // the K loop (a lane-masked copy there costs the loop its registers)
  uint32_t tvoff;
  {
    const uint32_t r = 8u * (wave & 1u) + (lane >> 3);
    const int32_t ttok = s_tok[kRows + r];
    tvoff = ttok >= 0 ? (uint32_t)ttok * H + (((lane & 7u) ^ row_swizzle(r)) * 16u) : kFar;
  }
  const u32x4 ra = rsrc(xq, T * H);
  const uint8_t* w13e = w13 + (size_t)e * 2u * I * H;
  // gate tile t and up tile t are adjacent (gate/up-interleaved W13), or I/16
  // row tiles apart (AITER): one range from the gate tile through the up tile
  const uint32_t up_tiles = kAiter ? I / 16u : 1u;  // row tiles from gate tile t to up tile t
  const u32x4 rg = rsrc(nk::tile_base(w13e, kAiter ? ng * 8u + wave : 2u * (ng * 8u + wave), 0, KB),
                        (up_tiles + 1u) * KB * 2048u);
  const uint32_t bvoff = lane * 16u;
  const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_offset(&s_stage[0][0]));
  // copy q = 0..6 of step kb (A halves, gate halves, up halves, tail share) into its stage
  auto issue_part = [&](uint32_t kb, uint32_t q) __attribute__((always_inline)) {
    const uint32_t st = lds0 + (kb % kStages) * kStageBytes;
    const uint32_t half = (q & 1u) * 1024u;
    if (q < 2u) copy16(st + wave * 2048u + half, ra, avoff[q], kb * 128u);
    else if (q < 4u) copy16(st + kABytes + wave * 2048u + half, rg, bvoff + half, kb * 2048u);
    else if (q < 6u) copy16(st + kABytes + (8u + wave) * 2048u + half, rg, bvoff + half, (up_tiles * KB + kb) * 2048u);
    else copy16(st + kTailTile * 2048u + (wave & 1u) * 1024u, ra, tvoff, kb * 128u);
  };
  // The scales travel with the first step's copies (so no further round trip
  // precedes the ring): copy c (wave c, and wave 0 for copy 8) moves the
  // activation scales of rows (256 / KB) c .. + 256 / KB - 1 (KB / 4 lanes a
  // row, zeros for padding rows), and wave 0 copies the item's weight block
  // scales (lane kb: gate, lane KB + kb: up). Row r's 16-byte chunk c sits at
  // slot c ^ as_swizzle(r), so the four rows 4 g + j (g = 0..3) a K step
  // reads at once fall in four different banks.
  {
    const u32x4 rxs = rsrc(xs, T * KB * 4u);
    auto scale_copy = [&](uint32_t c) __attribute__((always_inline)) {
      const uint32_t row = c * kAsRowsPerCopy + lane / kAsLanesPerRow;
      const int32_t stok = row < kAllRows ? s_tok[row] : -1;
      const uint32_t chunk = (lane % kAsLanesPerRow) ^ as_swizzle(row);
      const uint32_t xsoff = stok >= 0 ? (uint32_t)stok * KB * 4u + chunk * 16u : kFar;
      copy16((uint32_t)__builtin_amdgcn_readfirstlane((int)lds_offset(&s_as[c * 256u])), rxs, xsoff, 0u);
    };
    if (wave < kAsCopies) scale_copy(wave);
    if (kAsCopies > 8u && wave == 0u) scale_copy(8u);
    if (wave == 0u) {
      const float* wse = w13s + (size_t)e * (2u * I / 128u) * KB;
      const uint32_t wsoff = lane < 2u * KB ? ((lane < KB ? ng : I / 128u + ng) * KB + lane % KB) * 4u : kFar;
      copy4((uint32_t)__builtin_amdgcn_readfirstlane((int)lds_offset(&s_wsv[0])),
            rsrc(wse, (2u * I / 128u) * KB * 4u), wsoff, 0u);
    }
  }
  float wsv = 0.0f;
  v4f acc[4][4];
#pragma unroll
  for (uint32_t i = 0; i < 4; ++i)
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) acc[i][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // the tail tile against this wave's gate and up tiles 2 n + m (16 h columns)
  v4f acc_t[2] = {v4f{0.0f, 0.0f, 0.0f, 0.0f}, v4f{0.0f, 0.0f, 0.0f, 0.0f}};
  auto kloop = [&](auto ntc, auto tailc) __attribute__((always_inline)) {
    constexpr uint32_t NT = decltype(ntc)::value;
    constexpr bool kTail = decltype(tailc)::value;
    // copies per step: the tail share only in the tail variant
    constexpr uint32_t kCopies = kTail ? kCopiesPerWave : kCopiesPerWave - 1u;
#pragma unroll
    for (uint32_t q = 0; q < kCopies; ++q) issue_part(0, q);
    if (KB > 1)
#pragma unroll
      for (uint32_t q = 0; q < kCopies; ++q) issue_part(1, q);
#pragma unroll
    for (uint32_t kb = 0; kb < KB; ++kb) {
      if (kb + 1u < KB) wait_copies<kCopies>(); else wait_copies<0>();
      barrier();
      // the next-but-one step's copies: two before each of the first row
      // tiles, the rest before the last
      constexpr uint32_t kPer = NT > 1 ? 2u : kCopies;
      uint32_t q = 0;
      auto some_copies = [&](uint32_t count) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t u = 0; u < kCopies; ++u)
          if (u < count && q < kCopies && kb + 2u < KB) { issue_part(kb + 2u, q); ++q; }
      };
      if (kb == 0) wsv = s_wsv[lane];  // the scale copy landed with step 0's copies
      if (NT > 0) {
        const uint8_t* st = s_stage[kb % kStages];
        v8i bw[4];
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c)  // gate tiles 2n, 2n + 1, up tiles 8 + 2n, 8 + 2n + 1
          bw[c] = lds_operand<kAiter>(st + kABytes + ((c >> 1) * 8u + 2u * n + (c & 1u)) * 2048u, lane);
        const float sg = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(wsv), (int)kb));
        const float su = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(wsv), (int)(KB + kb)));
#pragma unroll
        for (uint32_t i = 0; i < NT; ++i) {
          const uint32_t rt = 4u * m + i;
          const v8i af = lds_operand_rows(st + rt * 2048u, lane);
          const float as = s_as_at(rt * 16u + (lane & 15u), kb);  // this lane's token row
          const float sgi = sg * as, sui = su * as;
          some_copies(i + 1u < NT ? kPer : kCopies);
          v4f d[4];
#pragma unroll
          for (uint32_t c = 0; c < 4; ++c) d[c] = nk::mfma_e4m3_16x16x128(bw[c], af);
#pragma unroll
          for (uint32_t c = 0; c < 4; ++c)
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) acc[i][c][j] = fmaf(c < 2 ? sgi : sui, d[c][j], acc[i][c][j]);
        }
        // The tail tile: a variant of its own (a branch inside the unrolled
        // loop costs it its registers); an absorbing item's blocks are full.
        if constexpr (kTail) {
          const v8i af = lds_operand_rows(st + kTailTile * 2048u, lane);
          const float as = s_as_at(kTailTile * 16u + (lane & 15u), kb);
          const float sgi = sg * as, sui = su * as;
          const v4f dg = nk::mfma_e4m3_16x16x128(m == 0u ? bw[0] : bw[1], af);
          const v4f du = nk::mfma_e4m3_16x16x128(m == 0u ? bw[2] : bw[3], af);
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) {
            acc_t[0][j] = fmaf(sgi, dg[j], acc_t[0][j]);
            acc_t[1][j] = fmaf(sui, du[j], acc_t[1][j]);
          }
        }
      } else {
        some_copies(kCopies);
      }
    }
  };
  using no_tail = std::false_type;
  if (absorb) {
    kloop(std::integral_constant<uint32_t, 4>{}, std::true_type{});
  } else {
    switch (ntiles) {
      case 0: kloop(std::integral_constant<uint32_t, 0>{}, no_tail{}); break;
      case 1: kloop(std::integral_constant<uint32_t, 1>{}, no_tail{}); break;
      case 2: kloop(std::integral_constant<uint32_t, 2>{}, no_tail{}); break;
      case 3: kloop(std::integral_constant<uint32_t, 3>{}, no_tail{}); break;
      default: kloop(std::integral_constant<uint32_t, 4>{}, no_tail{}); break;
    }
  }
  // Epilogue: h = bf16(silu(g) * u); amax per row over the 128-column group
  // (in stage KB % 3, which no wave reads after the K loop); FP8 bytes
  // through LDS (stage 0, free once every wave is past the K loop). The tail
  // rows' amax comes from all eight waves (16 columns each).
  float* s_amax = reinterpret_cast<float*>(s_stage[KB % kStages]);  // [2][4][64]: row block, quarter, row
  float* s_amax_t = s_amax + 2u * 4u * kRowsPerBlock;                // [8][16]: wave, tail row
  float* s_scale = s_amax_t + 8u * 16u;                              // [kAllRows]
  // The MFMAs take the weight tile as A: lane l holds channels 4 (l >> 4) ..
  // + 3 of each 16-row weight tile for token row l & 15 of each row tile, so
  // a lane's four h values of a tile are consecutive columns of one row.
  float h[4][2][4];
#pragma unroll
  for (uint32_t i = 0; i < 4; ++i) {
    float mx = 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < 2; ++c)
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const float v = nk::bf16_round_hw(nk::silu_hw(acc[i][c][j]) * acc[i][2u + c][j]);
        h[i][c][j] = v;
        mx = fmaxf(mx, fabsf(v));
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16u));
    mx = fmaxf(mx, __shfl_xor(mx, 32u));
    if (lane < 16u) s_amax[(m * 4u + n) * kRowsPerBlock + i * 16u + lane] = mx;
  }
  float ht[4];
  if (absorb) {
    float mx = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      ht[j] = nk::bf16_round_hw(nk::silu_hw(acc_t[0][j]) * acc_t[1][j]);
      mx = fmaxf(mx, fabsf(ht[j]));
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16u));
    mx = fmaxf(mx, __shfl_xor(mx, 32u));
    if (lane < 16u) s_amax_t[wave * 16u + lane] = mx;
  }
  __syncthreads();
  if (tid < kAllRows) {
    const uint32_t r = tid & 63u;
    float mx = nk::kAmaxFloor;
    if (tid < kRows) {
#pragma unroll
      for (uint32_t q = 0; q < 4; ++q) mx = fmaxf(mx, s_amax[((tid >> 6) * 4u + q) * kRowsPerBlock + r]);
    } else {
#pragma unroll
      for (uint32_t w = 0; w < 8; ++w) mx = fmaxf(mx, s_amax_t[w * 16u + r]);
    }
    const float scale = mx * nk::inv_e4m3_max();
    s_scale[tid] = scale;
    // rows 128 .. 143 are rows 0 .. 15 of block b0 + 2: the sorted rows are contiguous
    if (s_tok[tid] >= 0) hs[(size_t)(b0 * kRowsPerBlock + tid) * (I / 128u) + ng] = scale;
  }
  __syncthreads();
  constexpr uint32_t kOut = 144;  // LDS bytes per output row (128 + 16)
  uint8_t* s_out = s_stage[0];
  const uint32_t ocol = 4u * (lane >> 4);  // this lane's four columns within a 16-column tile
#pragma unroll
  for (uint32_t i = 0; i < 4; ++i) {
    const uint32_t row = m * kRowsPerBlock + i * 16u + (lane & 15u);
    const float inv = 1.0f / s_scale[row];
#pragma unroll
    for (uint32_t c = 0; c < 2; ++c)
      *reinterpret_cast<uint32_t*>(&s_out[row * kOut + (2u * n + c) * 16u + ocol]) =
          nk::e4m3x4(h[i][c][0] * inv, h[i][c][1] * inv, h[i][c][2] * inv, h[i][c][3] * inv);
  }
  if (absorb) {
    const uint32_t row = kRows + (lane & 15u);
    const float inv = 1.0f / s_scale[row];
    *reinterpret_cast<uint32_t*>(&s_out[row * kOut + (2u * n + m) * 16u + ocol]) =
        nk::e4m3x4(ht[0] * inv, ht[1] * inv, ht[2] * inv, ht[3] * inv);
  }
  __syncthreads();
  // 144 rows x 128 bytes: 4 threads per row, two 16-byte pieces each
  for (uint32_t row = tid >> 2; row < kAllRows; row += kThreads / 4u) {
    const uint32_t c0 = (tid & 3u) * 32u;
    if (s_tok[row] >= 0) {
      uint8_t* dst = hq + (size_t)(b0 * kRowsPerBlock + row) * I + ng * 128u + c0;
      *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(&s_out[row * kOut + c0]);
      *reinterpret_cast<uint4*>(dst + 16) = *reinterpret_cast<const uint4*>(&s_out[row * kOut + c0 + 16u]);
    }
  }
}
}  // namespace nklds

#define NK_GATE_UP_LDS(HV)                                                                         \
  NK_KERNEL __launch_bounds__(512) void netra_moe_gate_up_lds_h##HV##_gfx950(                      \
      const uint8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ w13, \
      const float* __restrict__ w13s, const int32_t* __restrict__ sorted_ids,                      \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,            \
      const int32_t* __restrict__ pair_map, uint8_t* __restrict__ hq, float* __restrict__ hs,      \
      uint32_t T, uint32_t H, uint32_t I, uint32_t Ktot, uint32_t Etot) {                          \
    (void)H;                                                                                       \
    nklds::gate_up_lds<HV / 128>(xq, xs, w13, w13s, sorted_ids, sorted_expert, num_valid,          \
                                 pair_map, hq, hs, T, I, Ktot, Etot);                              \
  }
NK_GATE_UP_LDS(512)
NK_GATE_UP_LDS(1024)
NK_GATE_UP_LDS(2048)

// W13 in the reference's AITER layout (the M768 prefill bridge): same ABI.
#define NK_GATE_UP_LDS_AITER(HV)                                                                   \
  NK_KERNEL __launch_bounds__(512) void netra_moe_gate_up_lds_aiter_h##HV##_gfx950(                \
      const uint8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ w13, \
      const float* __restrict__ w13s, const int32_t* __restrict__ sorted_ids,                      \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ num_valid,            \
      const int32_t* __restrict__ pair_map, uint8_t* __restrict__ hq, float* __restrict__ hs,      \
      uint32_t T, uint32_t H, uint32_t I, uint32_t Ktot, uint32_t Etot) {                          \
    (void)H;                                                                                       \
    nklds::gate_up_lds<HV / 128, true>(xq, xs, w13, w13s, sorted_ids, sorted_expert, num_valid,    \
                                       pair_map, hq, hs, T, I, Ktot, Etot);                        \
  }
NK_GATE_UP_LDS_AITER(2048)
