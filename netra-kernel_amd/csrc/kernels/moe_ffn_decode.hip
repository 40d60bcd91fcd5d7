// Decode FFN for T <= 64 tokens after the route kernel (wide) or the router
// logits kernel (narrow, T <= 16): the sort rebuilt in the gate/up prologue,
// and (narrow) the top-k too, and the top-k weighted combine folded into down
// through a hand-off between workgroups.
//
//   netra_moe_ffn_gate_up_h<H>_i<I>_<wide|narrow>_gfx950(logits, bias,
//       topk_ids, topk_weights, xq, xs, w13, w13s, sorted_ids, sorted_expert,
//       tile_map, pair_map, num_valid, counts, hrows, hq, hs; T, E, K, S, CAP)
//     wide reads topk_ids (logits, bias and topk_weights unused); narrow
//     selects from logits + bias and writes topk_ids / topk_weights
//   netra_moe_ffn_down_h<H>_i<I>_<wide|narrow|rows>_gfx950(topk_weights, w2, w2s,
//       sorted_ids, sorted_expert, tile_map, num_valid, hrows, hq, hs, partial,
//       counters, out; T, E, K, S)
// The narrow down combines in the kernel (the hand-off below); the wide one
// leaves the fp32 route partials to netra_moe_combine_gfx950: with tens of
// tokens the hand-off's combine work lands in the kernel's tail (57.9 us
// against 46.2 us without it at T = 64 on one MI355X, more than the separate
// combine launch costs). The rows down takes the narrow gate/up's bf16 rows
// through the wide down's items and leaves the combine to the same kernel;
// from five tokens it is the faster of the two after the narrow gate/up.
//   netra_moe_ffn_gate_up_down_h<H>_i<I>[_ksplit]_gfx950(the gate/up arguments
//       with w2, w2s and partial after hs)
//     the wide gate/up with each tile's down run by the same workgroup from the
//     requantised h in its LDS (fp32 partials to the combine kernel); _ksplit
//     splits gate/up's K over the waves. Chosen when a call has enough tiles
//     to keep the chip streaming.
//   block 512 (8 waves), any grid
// Weights are read with non-temporal loads: every tile is read by one
// workgroup per launch (the tiles of an expert with more than 16 routes by
// one per 16 of them); 83.1 -> 80 us for gate/up and 49.1 -> 46.3 us for down
// at T = 64 against ordinary loads.
//
// gate/up prologue (every workgroup, redundantly; the inputs are a few KB in
// L2): the route kernel's ids go to LDS (narrow: wave w runs the top-k of tokens
// w and w + 8 on the logits, the route kernel's selection, and puts its ids there, and
// workgroup 0 writes topk_ids / topk_weights); the routing bitmask (bit t of word e:
// token t routes to expert e) gives each expert's count and each route's rank
// among its expert's tokens; a scan over experts gives block, tile and pair
// offsets in the AITER sorted format. Workgroup 0 writes the counts, the tile
// and pair lists and num_valid; all workgroups write a grid-stride share of
// sorted_ids and sorted_expert. These are the outputs of the separate sort
// kernel, bit for bit, and what down reads.
//
// Tile g (expert e, sub-tile k of e's rows): the 16 routes of e with ranks
// 16k..16k+15 (token order).
//   gate/up item (g, a), a < GA = I / (16 CA): h columns [16 CA a, 16 CA (a + 1))
//     of the tile. Wave w takes 16-column item w % CA over the K blocks of
//     split w / CA (SA = 8 / CA splits), streaming W13 in steps of up to CHM
//     K blocks, one step ahead, against the tile's x rows staged in LDS. Split
//     sums are added in LDS in split order and h = bf16(silu(g) * u). wide
//     (CA = 8: the item is one 128-column block) requantises it in the
//     workgroup (1x128 rule) to hq/hs in the stream path's tile16x128 layout;
//     narrow writes the bf16 rows to hrows and leaves the requant to down.
//   down item (g, b), b < GB = H / (32 CB): output columns [32 CB b, 32 CB (b + 1)).
//     The first W2 step is issued, the tile's h operand is staged in LDS
//     (wide: hq/hs as they are; narrow: hrows requantised, item b == 0 also
//     writing hq/hs for inspection), and wave w takes 32-column item w % CB
//     over K split w / CB (SB = 8 / CB). Each valid row's fp32 result goes to
//     partial[route] (agent-scope stores where the hand-off reads it back).
// Items are dealt round-robin (item = workgroup, + grid, ...). Nothing waits
// for another workgroup.
//
// Combine hand-off: when a down item's partial stores have completed, each
// valid row counts an arrival on the (token, column group b) counter (a
// workgroup does this for up to 32 of its items at once, after its last one
// or when 32 are held, so it waits for its stores once); the
// arrival that brings it to Ktot is the last of the token's routes for that
// group, and its workgroup reads the Ktot partial rows back at agent scope and
// writes out[t, group] = bf16(sum over slots in order of fmaf(w_s, p_s, acc))
// from acc = 0 (the order of netra_moe_combine_gfx950). The arrival is one
// wrapping atomic increment (old >= Ktot - 1 ? 0 : old + 1), so the last
// arrival leaves the counter at zero for the next launch with no separate
// reset that could be lost. Agent-scope (sc1) stores and loads carry
// the hand-off: the per-XCD L2s are not coherent with each other for plain
// accesses.
//
// (reference: the decode trio kernels/gfx950/templates/moe/decode/
// gate_up_mfma.inc:12-161, silu_quant.inc:16-236, down_reduce_mfma_2wave.inc:
// 14-291; sorted format entry_routing.inc:27-112)
#pragma once
#include "moe_gemm_lds.hip"
#include "moe_gemm_stream.hip"
#include "moe_numerics.h"

namespace nkffn {

using nk::v4f;
using nk::v8i;

constexpr uint32_t kWaves = 8, kThreads = 64u * kWaves;
constexpr uint32_t kMaxT = 64;       // one bitmask word per expert
constexpr uint32_t kMaxKtot = 16;    // routes per token
constexpr uint32_t kMaxE = 512;      // experts incl. shared, one per thread in the scan
constexpr uint32_t kMaxCap = 1024;   // capacity blocks
constexpr uint32_t kMaxGroups = 64;  // down column groups per token (H / 64 at most)
constexpr uint32_t kCounters = kMaxT * kMaxGroups;  // combine counters [token][group]
constexpr uint32_t kNarrowT = 16;    // tokens the narrow variant serves (their x rows: one 16-row A tile)

// Position of the j-th set bit (0-based) of m; 64 if there is none.
__device__ __forceinline__ uint32_t nth_bit(unsigned long long m, uint32_t j) {
  for (uint32_t i = 0; i < j && m; ++i) m &= m - 1ull;
  return m ? (uint32_t)__ffsll((long long)m) - 1u : 64u;
}

// nth_bit for a wave-uniform m and j, every lane active: lane l holds bit l
// and counts the set bits below it, so one ballot finds the position.
__device__ __forceinline__ uint32_t nth_bit_wave(unsigned long long m, uint32_t j, uint32_t lane) {
  const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
  const unsigned long long hit = __ballot(((m >> lane) & 1ull) != 0ull && below == j);
  return hit ? (uint32_t)__ffsll((long long)hit) - 1u : 64u;
}

// Slot of expert e in token t's route list, or Ktot.
__device__ __forceinline__ uint32_t slot_of(const int32_t* s_ids, uint32_t t, uint32_t Ktot, uint32_t e) {
  for (uint32_t s = 0; s < Ktot; ++s)
    if ((uint32_t)s_ids[t * Ktot + s] == e) return s;
  return Ktot;
}

// Barrier after this wave's global stores have completed (vmcnt) and its LDS
// traffic is done.
__device__ __forceinline__ void store_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 1x128 requant of one (row, 128-column block): lane l holds row l & 15,
// columns 32 (l >> 4) .. + 31 as 16 packed bf16 pairs; the four lanes of a row
// share the amax. scale = max(amax, floor) * (1 / 448), q = e4m3(h * (1 / scale)).
__device__ __forceinline__ void quant_block(const uint32_t (&raw)[16], uint4& qlo, uint4& qhi, float& scale) {
  float amax = nk::kAmaxFloor;
#pragma unroll
  for (uint32_t q = 0; q < 16; ++q) amax = fmaxf(amax, fmaxf(fabsf(nk::bf16_lo(raw[q])), fabsf(nk::bf16_hi(raw[q]))));
  amax = fmaxf(amax, __shfl_xor(amax, 16u));
  amax = fmaxf(amax, __shfl_xor(amax, 32u));
  scale = amax * nk::inv_e4m3_max();
  const float inv = 1.0f / scale;
  auto q4 = [&](uint32_t q) __attribute__((always_inline)) {  // columns 4q .. 4q + 3
    return nk::e4m3x4(nk::bf16_lo(raw[2 * q]) * inv, nk::bf16_hi(raw[2 * q]) * inv,
                      nk::bf16_lo(raw[2 * q + 1]) * inv, nk::bf16_hi(raw[2 * q + 1]) * inv);
  };
  qlo = make_uint4(q4(0), q4(1), q4(2), q4(3));
  qhi = make_uint4(q4(4), q4(5), q4(6), q4(7));
}

// ---------------------------------------------------------------------------
// gate/up with the sort as its prologue
template <uint32_t KB, uint32_t KBI, uint32_t SA, uint32_t CHM, uint32_t P,  // H / 128, I / 128, K splits,
          bool kDown = false, bool kKSplit = false>  // K blocks per step, items per wave; kDown: the
                                                     // tile's down too; kKSplit: gate/up K over the waves
__device__ __forceinline__ void ffn_gate_up(
    const uint16_t* __restrict__ logits, const float* __restrict__ bias, int32_t* __restrict__ topk_ids,
    float* __restrict__ topk_weights, const uint8_t* __restrict__ xq, const float* __restrict__ xs,
    const uint8_t* __restrict__ w13, const float* __restrict__ w13s, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ sorted_expert, int32_t* __restrict__ tile_map, int32_t* __restrict__ pair_map,
    int32_t* __restrict__ num_valid, int32_t* __restrict__ counts, uint16_t* __restrict__ hrows,
    uint8_t* __restrict__ hq, float* __restrict__ hs, uint32_t T, uint32_t E, uint32_t K, uint32_t S,
    uint32_t cap_blocks, const uint8_t* __restrict__ w2 = nullptr, const float* __restrict__ w2s = nullptr,
    float* __restrict__ partial = nullptr) {
  using nkstream::lds_barrier;
  constexpr uint32_t H = 128u * KB, I = 128u * KBI;
  constexpr uint32_t CA = kWaves / SA;                 // column items per gate/up item
  constexpr uint32_t KBA = KB / SA;                    // K blocks per wave
  constexpr uint32_t kCH = KBA >= CHM ? CHM : 1u;      // K blocks per step
  constexpr uint32_t NA = KBA / kCH;                   // steps per wave
  constexpr uint32_t GA = I / (16u * CA * P);          // items per tile
  constexpr uint32_t NS = P * NA;                      // steps per wave and item
  constexpr bool kQuant = CA == kWaves;                // the item is P whole 128-column blocks
  constexpr uint32_t kHb = 128u * P + 8u;              // bf16 per LDS h row (+16 bytes rotates banks)
  static_assert(CA * SA == kWaves && KB % SA == 0 && KBA % kCH == 0, "K splits");
  static_assert(I % (16u * CA * P) == 0 && H % kThreads == 0 && (P == 1 || SA == 1) && P <= kWaves, "shares");
  constexpr uint32_t kRed = SA > 1 ? kWaves * 8u * 64u * 4u : 0u;  // split sums
  constexpr bool kStageAll = SA > 1;  // narrow: one A operand (every token's row) for all items
  // kDown: after its gate/up steps the workgroup runs the tile's down over all
  // H output columns (wave w: 32-column items w, w + 8, ..), its A operand the
  // requantised h in LDS (s_big, scales in s_xs), and leaves fp32 route
  // partials to the combine kernel
  constexpr uint32_t PDN = H / (32u * kWaves);         // 32-column down items per wave
  constexpr uint32_t kDCN = KBI >= 2u ? 2u : 1u;       // down K blocks per step
  constexpr uint32_t NBN = KBI / kDCN;                 // down steps per 32-column item
  constexpr uint32_t NSN = PDN * NBN;                  // down steps per wave
  static_assert(!kDown || (SA == 1 && P == KBI && I == 128u * P && KBI <= KB && NSN >= 2u),
                "kDown: one item per tile, the requantised h fits the x rows' LDS");
  // kKS (kDown, H = 2048): gate/up step s is 16-column item s for every wave,
  // wave w taking K blocks kCH w .. (the workgroup reads the item's 64 KiB of
  // W13 together); the waves' split sums are added in wave order in LDS
  constexpr bool kKS = kKSplit;
  static_assert(!kKS || (kDown && KB == kWaves * kCH && NS == I / 16u && kQuant), "kKS: one step per 16-column item");
  constexpr uint32_t kBig = KB * 2048u > kRed || kStageAll ? KB * 2048u : kRed;
  // s_big: the tile's x rows | split sums
  __shared__ __align__(16) uint8_t s_big[kBig];
  __shared__ __align__(16) float s_xs[16 * KB];                   // x row scales [kb][row] | kDown: h scales
  __shared__ __align__(16) uint16_t s_hb[kQuant ? 16u * kHb : 8u];  // the item's h rows (bf16)
  __shared__ float s_ksred[kKS ? 2u * kWaves * 8u * 64u : 1u];     // kKS: split sums, two steps
  __shared__ int32_t s_ids[kMaxT * kMaxKtot];
  __shared__ unsigned long long s_mask[kMaxE];
  __shared__ uint32_t s_boff[kMaxE + 1], s_toff[kMaxE + 1];
  __shared__ uint32_t s_chunk[48];
  __shared__ float s_rsum[kStageAll ? kRed / 4u : 1u];  // narrow: split sums (s_big holds the A operand)
  uint8_t* const s_a = s_big;
  float* const s_red = kStageAll ? s_rsum : reinterpret_cast<float*>(s_big);
  // wide prologue tables (block owner, pair offsets) and the first item's expert
  __shared__ int32_t s_owner[kStageAll ? 1u : kMaxCap];
  __shared__ uint32_t s_poff[kStageAll ? 1u : kMaxE + 1u];
  __shared__ uint32_t s_e0;
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = nkstream::wave_id();
  const uint32_t Ktot = K + S, Etot = E + S, routes = T * Ktot;
  if (T == 0u || T > (kStageAll ? kNarrowT : kMaxT) || Ktot > kMaxKtot || Etot > kMaxE || cap_blocks > kMaxCap ||
      K > E)
    return;  // host-checked

  // Step s of item `item` (tile expert e): 16-column item c0 + s / NA, K blocks
  // kbw + ((s + rot) % NA) * kCH ..  Rotating the K order by the item spreads
  // the workgroups running together over different offsets of their experts'
  // weights (same-offset streams of 2 MiB-strided experts share HBM channels).
  const uint32_t ca = wave % CA, sa = wave / CA;
  const uint32_t kbw = sa * KBA;  // this wave's first K block
  auto issue_at = [&](GateUpStep<kCH>& st, uint32_t e, uint32_t item, uint32_t s) __attribute__((always_inline)) {
    const uint8_t* w13e = w13 + (size_t)e * 2u * I * H;
    const float* w13se = w13s + (size_t)e * (2u * I / 128u) * KB;
    const uint32_t c = kKS ? s : ((item % GA) * CA + ca) * P + s / NA, rot = item % NA;
#pragma unroll
    for (uint32_t i = 0; i < kCH; ++i) {
      const uint32_t kb = kKS ? wave * kCH + i : kbw + ((s + rot) % NA) * kCH + i;
      st.g[i] = nk::load_tile_operand_once(nk::tile_base(w13e, 2u * c, kb, KB), lane);
      st.u[i] = nk::load_tile_operand_once(nk::tile_base(w13e, 2u * c + 1u, kb, KB), lane);
    }
    const uint32_t sl = lane < 2u * KB ? lane : 0u;
    st.ws = w13se[((sl < KB ? c : I / 16u + c) >> 3) * KB + (sl < KB ? sl : sl - KB)];
  };
  GateUpStep<kCH> b0, b1;
  uint32_t e_pre = 0xffffffffu;  // the expert of the steps issued in the prologue

  // ---- routes into LDS, routing bitmask ------------------------------------------------------
  // (every entry cleared: the narrow presence ballots read all of them
  // unconditionally, entries past Etot as zero)
  static_assert(kMaxE == kThreads, "one mask entry per thread");
  s_mask[tid] = 0ull;
  constexpr uint32_t kTokW = kNarrowT / kWaves;  // narrow: tokens per wave
  uint32_t topk_id[kTokW] = {};  // narrow: wave w lane s < Ktot, token w + 8 j's slot s
  float topk_wt[kTokW] = {};
  if constexpr (kStageAll) {
    // narrow: the A operand of every item is the T token rows themselves
    // (row t = token t, rows T .. 15 zero), copied by DMA into the tile layout
    // of s_a (K block kb, half h: the 16-byte piece of row r at columns
    // 128 kb + 32 c + 16 h .. + 15 sits at 2048 kb + 1024 h + 16 (16 c + r))
    // with the scales s_xs[kb][r]; pieces past the T rows read as zeros. The
    // copies use no registers and are in flight under the top-k; wave w
    // selects the experts of tokens w and w + 8 from the logits (the route
    // kernel's top-k, one wave per token and round)
    static_assert(KB % 4u == 0u, "scale copies of 64 floats");
    const nk::u32x4 rx = nklds::rsrc(xq, T * H), rxs = nklds::rsrc(xs, T * KB * 4u);
    for (uint32_t c = wave; c < 2u * KB; c += kWaves)  // copy c: K block c / 2, half c % 2
      nklds::copy16((uint32_t)__builtin_amdgcn_readfirstlane((int)nklds::lds_offset(s_a + c * 1024u)), rx,
                    (lane & 15u) * H + (c >> 1) * 128u + (lane >> 4) * 32u + (c & 1u) * 16u, 0u);
    for (uint32_t c = wave; c < KB / 4u; c += kWaves) {  // s_xs[64 c + l]: K block (64 c + l) / 16, row l % 16
      const uint32_t i = 64u * c + lane;
      nklds::copy4((uint32_t)__builtin_amdgcn_readfirstlane((int)nklds::lds_offset(&s_xs[64u * c])), rxs,
                   ((i & 15u) * KB + (i >> 4)) * 4u, 0u);
    }
    // With a shared expert, items 0 .. GA - 1 are the shared expert's tile
    // (narrow_tile below), whose expert E is known before the selection: its
    // first item steps go out now, under the logits loads (the waits below
    // cover them too)
    if (S != 0u && blockIdx.x < GA) {  // uniform
      e_pre = E;
      issue_at(b0, E, blockIdx.x, 0u);
      if constexpr (NS == 2) issue_at(b1, E, blockIdx.x, 1u);
    }
#pragma unroll
    for (uint32_t j = 0; j < kTokW; ++j) {
      const uint32_t tk = wave + kWaves * j;
      if (tk < T) {  // uniform
        topk_select_any(logits + (size_t)tk * Etot, bias, E, K, S, lane, topk_id[j], topk_wt[j]);
        if (lane < Ktot) s_ids[tk * Ktot + lane] = (int32_t)topk_id[j];
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the copies have landed
    lds_barrier();
    // workgroup 0 publishes the selection (after the barrier: no store is in
    // the wait above)
#pragma unroll
    for (uint32_t j = 0; j < kTokW; ++j) {
      const uint32_t tk = wave + kWaves * j;
      if (blockIdx.x == 0 && tk < T && lane < Ktot) {
        topk_ids[tk * Ktot + lane] = (int32_t)topk_id[j];
        topk_weights[tk * Ktot + lane] = topk_wt[j];
      }
    }
  } else {
    for (uint32_t r = tid; r < routes; r += kThreads) s_ids[r] = topk_ids[r];
    lds_barrier();
  }
  for (uint32_t r = tid; r < routes; r += kThreads) {
    const uint32_t e = (uint32_t)s_ids[r];
    if (e < Etot) atomicOr(&s_mask[e], 1ull << (r / Ktot));
  }
  lds_barrier();

  // wide: the x rows of sub-tile k of expert e, loaded into registers
  // (stage_load: rows past e's routes zero) and then stored into s_a in the
  // MFMA operand layout with their scales in s_xs (stage_store; the caller
  // puts a barrier behind it). Lane l's row l & 15 is token
  // nth_bit(mask, 16 k + (l & 15)).
  constexpr uint32_t kPieces = kStageAll ? 1u : H / kThreads, kScales = (16u * KB + kThreads - 1u) / kThreads;
  uint4 av[kPieces];
  float xv[kScales];
  auto stage_load = [&](uint32_t e, uint32_t k) __attribute__((always_inline)) {
    if constexpr (!kStageAll) {
      int32_t tok = -1;
      {
        const unsigned long long emask = s_mask[e];
        const uint32_t j = 16u * k + (lane & 15u);
        if (j < (uint32_t)__popcll(emask)) tok = (int32_t)nth_bit(emask, j);
      }
#pragma unroll
      for (uint32_t q = 0; q < kPieces; ++q) {
        const uint32_t pc = tid + q * kThreads, row = pc / (H / 16u), kk = (pc % (H / 16u)) * 16u;
        const int32_t t = __shfl(tok, row);
        av[q] = t >= 0 ? *reinterpret_cast<const uint4*>(xq + (size_t)t * H + kk) : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (uint32_t q = 0; q < kScales; ++q) {
        const uint32_t i = tid + q * kThreads;
        const int32_t t = __shfl(tok, (i / KB) & 15u);
        xv[q] = (i < 16u * KB && t >= 0) ? xs[(size_t)t * KB + i % KB] : 0.0f;
      }
    }
  };
  auto stage_store = [&]() __attribute__((always_inline)) {
    if constexpr (!kStageAll) {
#pragma unroll
      for (uint32_t q = 0; q < kPieces; ++q) {
        const uint32_t pc = tid + q * kThreads, row = pc / (H / 16u), kk = (pc % (H / 16u)) * 16u;
        const uint32_t kb = kk >> 7, k7 = kk & 127u;
        *reinterpret_cast<uint4*>(&s_a[kb * 2048u + ((k7 >> 4) & 1u) * 1024u + ((k7 >> 5) * 16u + row) * 16u]) = av[q];
      }
#pragma unroll
      for (uint32_t q = 0; q < kScales; ++q)
        if (tid + q * kThreads < 16u * KB) {  // element i = row * KB + kb of the gather
          const uint32_t i = tid + q * kThreads;
          s_xs[(i % KB) * 16u + i / KB] = xv[q];
        }
    }
  };
  const int32_t pad = (int32_t)((Ktot << 24) | T);
  // narrow: an expert holds at most T <= kNarrowT <= 16 routes, so it has one
  // block, one tile and one pair, all numbered g for the g-th expert with a
  // route. Every wave holds the experts' presence as ballots (bit l of
  // used[c]: expert 64 c + l has a route), from which the sorted format
  // follows without a scan; the first item's steps are issued before the
  // sorted format is written, their weight loads in flight under it.
  static_assert(kNarrowT <= 16u && (!kStageAll || NS <= 2u), "one tile per expert; an item's steps issued at once");
  constexpr uint32_t kChunks = kStageAll ? kMaxE / 64u : 1u;
  unsigned long long used[kChunks];
  uint32_t before[kChunks + 1];
  // the b-th expert with a route (b < the count, uniform, every lane active):
  // the last chunk c with before[c] <= b (before[] does not decrease, so the
  // test holds for a prefix of the chunks) by a chain of scalar selects (the
  // empty asm keeps it a chain rather than an indexed register read), then
  // its bit by one ballot
  auto used_expert = [&](uint32_t b) __attribute__((always_inline)) {
    unsigned long long m = used[0];
    uint32_t c0 = 0, b0 = 0;
#pragma unroll
    for (uint32_t c = 1; c < kChunks; ++c) {
      const bool in = b >= before[c];
      m = in ? used[c] : m;
      c0 = in ? 64u * c : c0;
      b0 = in ? before[c] : b0;
      asm volatile("" : "+s"(m), "+s"(c0), "+s"(b0));
    }
    return c0 + nth_bit_wave(m, b - b0, lane);
  };
  uint32_t ntile = 0;
  // narrow: the tile of item q. The shared expert's tile is the last one (E
  // is the largest used id); with S = 1 it takes items 0 .. GA - 1 and the
  // routed tiles follow in order, so its weights can be requested before the
  // selection whatever T is. (Positions in the outputs use the tile itself.)
  auto narrow_tile = [&](uint32_t q) __attribute__((always_inline)) {
    return S == 0u ? q / GA : (q < GA ? ntile - 1u : q / GA - 1u);
  };
  if constexpr (kStageAll) {
    // all chunks' mask entries read before the first ballot: one LDS wait
    unsigned long long mv[kChunks];
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) mv[c] = s_mask[64u * c + lane];
    before[0] = 0;
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
      used[c] = __ballot(mv[c] != 0ull);
      before[c + 1] = before[c] + (uint32_t)__popcll(used[c]);
    }
    ntile = before[kChunks];
    if (e_pre == 0xffffffffu && blockIdx.x < ntile * GA) {
      e_pre = used_expert(narrow_tile(blockIdx.x));
      issue_at(b0, e_pre, blockIdx.x, 0u);
      if constexpr (NS == 2) issue_at(b1, e_pre, blockIdx.x, 1u);
    }
    if (blockIdx.x == 0) {
      if (tid < Etot) counts[tid] = (int32_t)__popcll(s_mask[tid]);
      if (tid < ntile) {
        tile_map[tid] = (int32_t)(4u * tid);
        pair_map[tid] = (int32_t)tid;
      }
      if (tid == 0) {
        num_valid[0] = (int32_t)(ntile * 64u);
        num_valid[1] = (int32_t)routes;
        num_valid[2] = (int32_t)ntile;
        num_valid[3] = (int32_t)ntile;
      }
    }
    // sorted ids and the block table, a grid-stride share per workgroup (a
    // wave's 64 entries are one block)
    for (uint32_t p = blockIdx.x * kThreads + tid; p < cap_blocks * 64u; p += gridDim.x * kThreads) {
      const uint32_t b = __builtin_amdgcn_readfirstlane(p >> 6);
      int32_t v = pad, e = -1;
      if (b < ntile) {
        e = (int32_t)used_expert(b);
        const unsigned long long m = s_mask[e];
        const uint32_t j = p & 63u;  // rank among expert e's tokens
        if (j < (uint32_t)__popcll(m)) {
          const uint32_t t = nth_bit(m, j);
          v = (int32_t)((slot_of(s_ids, t, Ktot, (uint32_t)e) << 24) | t);
        }
      }
      sorted_ids[p] = v;
      if ((p & 63u) == 0u) sorted_expert[b] = e;
    }
  } else {
    // ---- counts and block / tile / pair offsets (one expert per thread) -----------------------
    const uint32_t cnt = tid < Etot ? (uint32_t)__popcll(s_mask[tid]) : 0u;
    const uint32_t vb = (cnt + 63u) >> 6, vt = (cnt + 15u) >> 4, vp = (vb + 1u) >> 1;
    uint32_t ib = vb, it = vt, ip = vp;
#pragma unroll
    for (uint32_t off = 1; off < 64; off <<= 1) {
      const uint32_t ob = __shfl_up(ib, off), ot = __shfl_up(it, off), op = __shfl_up(ip, off);
      if (lane >= off) { ib += ob; it += ot; ip += op; }
    }
    if (lane == 63u) { s_chunk[wave] = ib; s_chunk[16u + wave] = it; s_chunk[32u + wave] = ip; }
    lds_barrier();
    uint32_t cb = 0, ct = 0, cp = 0, nblk = 0, npair = 0;
#pragma unroll
    for (uint32_t c = 0; c < kWaves; ++c) {
      if (c < wave) { cb += s_chunk[c]; ct += s_chunk[16u + c]; cp += s_chunk[32u + c]; }
      nblk += s_chunk[c];
      ntile += s_chunk[16u + c];
      npair += s_chunk[32u + c];
    }
    if (tid < Etot) { s_boff[tid] = cb + ib - vb; s_toff[tid] = ct + it - vt; s_poff[tid] = cp + ip - vp; }
    if (tid == 0) { s_boff[Etot] = nblk; s_toff[Etot] = ntile; s_poff[Etot] = npair; }
    if (nblk > cap_blocks) return;  // impossible for T <= 64 with the engine's capacity; uniform
    // This workgroup's round-0 item (the item loop's dealing) and its expert,
    // read off the scan by the thread whose tile range holds it, so the item's
    // first weight steps and x rows go out before the sorted outputs below.
    uint32_t item0 = blockIdx.x;
    bool has0 = item0 < ntile * GA;
    if (gridDim.x % 8u == 0u) has0 = nklds::xcd_item(blockIdx.x, min(gridDim.x, ntile * GA), item0);
    if (has0 && tid < Etot && item0 / GA - (ct + it - vt) < vt) s_e0 = tid;
    for (uint32_t b = tid; b < cap_blocks; b += kThreads) s_owner[b] = -1;
    lds_barrier();
    if (has0) {  // uniform
      // x row loads, then the weight steps, then the rows' LDS stores: the
      // stores wait only for the (older) row loads
      const uint32_t e = __builtin_amdgcn_readfirstlane((int)s_e0);
      stage_load(e, item0 / GA - s_toff[e]);
      issue_at(b0, e, item0, 0u);
      if constexpr (NS == 2) issue_at(b1, e, item0, 1u);
      stage_store();
    }
    if (tid < Etot) {
      for (uint32_t b = s_boff[tid]; b < s_boff[tid + 1u]; ++b) s_owner[b] = (int32_t)tid;
      if (blockIdx.x == 0) {
        counts[tid] = (int32_t)cnt;
        for (uint32_t i = s_toff[tid]; i < s_toff[tid + 1u]; ++i) tile_map[i] = (int32_t)(s_boff[tid] * 4u + (i - s_toff[tid]));
        for (uint32_t i = s_poff[tid]; i < s_poff[tid + 1u]; ++i) pair_map[i] = (int32_t)(s_boff[tid] + 2u * (i - s_poff[tid]));
      }
    }
    if (blockIdx.x == 0 && tid == 0) {
      num_valid[0] = (int32_t)(nblk * 64u);
      num_valid[1] = (int32_t)routes;
      num_valid[2] = (int32_t)ntile;
      num_valid[3] = (int32_t)npair;
    }
    lds_barrier();
    // sorted ids and the block table, a grid-stride share per workgroup
    for (uint32_t p = blockIdx.x * kThreads + tid; p < cap_blocks * 64u; p += gridDim.x * kThreads) {
      const uint32_t b = p >> 6;
      const int32_t e = s_owner[b];
      int32_t v = pad;
      if (e >= 0) {
        const uint32_t j = (b - s_boff[e]) * 64u + (p & 63u);  // rank among expert e's tokens
        const unsigned long long m = s_mask[e];
        if (j < (uint32_t)__popcll(m)) {
          const uint32_t t = nth_bit(m, j);
          v = (int32_t)((slot_of(s_ids, t, Ktot, (uint32_t)e) << 24) | t);
        }
      }
      sorted_ids[p] = v;
      if ((p & 63u) == 0u) sorted_expert[b] = e;
    }
    lds_barrier();  // the staged x rows and scales are visible to every wave
  }

  // ---- items --------------------------------------------------------------------------------
#pragma unroll 1
  for (uint32_t base = 0; base < ntile * GA; base += gridDim.x) {
    // round base: items base .. base + grid - 1. Wide: dealt XCD-major over
    // the round's items (workgroup i runs on XCD i % 8), so an expert's
    // consecutive tiles (the shared expert's four at T = 64) stream its
    // weights concurrently through one L2; narrow: item = base + workgroup
    uint32_t item = base + blockIdx.x;
    if (!kStageAll && gridDim.x % 8u == 0u) {
      if (!nklds::xcd_item(blockIdx.x, min(gridDim.x, ntile * GA - base), item)) break;
      item += base;
    } else if (item >= ntile * GA) {
      break;
    }
    const uint32_t g = kStageAll ? narrow_tile(item) : item / GA, grp = item % GA;
    uint32_t e, k, row0;  // the tile's expert, its sub-tile among e's rows and its sorted position
    if constexpr (kStageAll) {
      e = used_expert(g);
      k = 0;
      row0 = 64u * g;
    } else {  // the last e with s_toff[e] <= g (uniform binary search)
      uint32_t lo = 0, hi = Etot;  // s_toff[lo] <= g < s_toff[hi]
      while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (s_toff[mid] <= g) lo = mid; else hi = mid;
      }
      e = lo;
      k = g - s_toff[e];
      row0 = (s_boff[e] + (k >> 2)) * 64u + (k & 3u) * 16u;
    }
    const uint32_t c0 = (grp * CA + ca) * P;  // this wave's first 16-column item within the tile's I / 16
    const uint32_t rot = item % NA;
    auto issue = [&](GateUpStep<kCH>& st, uint32_t s) __attribute__((always_inline)) { issue_at(st, e, item, s); };
    // steps 0 and (NS > 1) 1 issued: in the prologue (narrow: the first
    // item; wide: round 0, x rows staged too) or now
    const bool pre = kStageAll ? item == blockIdx.x && e == e_pre : base == 0u;
    if (!pre) {
      issue(b0, 0u);
      if constexpr (NS == 2) issue(b1, 1u);
    }
    if (!kStageAll && !pre) {  // wide: stage the tile's x rows and scales
      stage_load(e, k);
      stage_store();
      lds_barrier();
    }

    v4f ag = {0.0f, 0.0f, 0.0f, 0.0f}, au = {0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](const GateUpStep<kCH>& st, uint32_t s) __attribute__((always_inline)) {
#pragma unroll
      for (uint32_t i = 0; i < kCH; ++i) {
        const uint32_t kb = kKS ? wave * kCH + i : kbw + ((s + rot) % NA) * kCH + i;
        const v8i a = nk::load_tile_operand(s_a + kb * 2048u, lane);
        const v4f dg = nk::mfma_e4m3_16x16x128(a, st.g[i]);
        const v4f du = nk::mfma_e4m3_16x16x128(a, st.u[i]);
        const float sg = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(st.ws), (int)kb));
        const float su = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(st.ws), (int)(KB + kb)));
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          const float as = s_xs[kb * 16u + (lane >> 4) * 4u + j];
          ag[j] = ag[j] + sg * (as * dg[j]);
          au[j] = au[j] + su * (as * du[j]);
        }
      }
      if constexpr (kKS) {  // item s's split sums -> LDS; wave s % 8 adds them in wave order
        float* const red = s_ksred + (s & 1u) * (kWaves * 8u * 64u);
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          red[(wave * 8u + j) * 64u + lane] = ag[j];
          red[(wave * 8u + 4u + j) * 64u + lane] = au[j];
        }
        ag = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        au = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        lds_barrier();  // (the buffer of step s - 2 was read before step s - 1's barrier)
        if (wave == s % kWaves) {
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) {
            float gs = 0.0f, us = 0.0f;
#pragma unroll
            for (uint32_t w = 0; w < kWaves; ++w) {
              gs += red[(w * 8u + j) * 64u + lane];
              us += red[(w * 8u + 4u + j) * 64u + lane];
            }
            s_hb[((lane >> 4) * 4u + j) * kHb + s * 16u + (lane & 15u)] = nk::bf16_rne(nk::silu(gs) * us);
          }
        }
      } else if constexpr (kQuant) {
        if (s % NA == NA - 1u) {  // item c0 + s / NA done: its 16 x 16 h block -> LDS
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j)
            s_hb[((lane >> 4) * 4u + j) * kHb + (ca * P + s / NA) * 16u + (lane & 15u)] =
                nk::bf16_rne(nk::silu(ag[j]) * au[j]);
          ag = v4f{0.0f, 0.0f, 0.0f, 0.0f};
          au = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
    };
    if constexpr (NS == 1) {
      compute(b0, 0u);
    } else if constexpr (NS == 2) {  // both steps in flight since the item's start
      compute(b0, 0u);
      compute(b1, 1u);
    } else {
      // the last one or two steps peeled: no load is issued under a branch
      // (the wait counts at a join would drain the step in flight) and none
      // past the last step
      uint32_t s = 0;
#pragma unroll 1
      for (; s + 2u < NS; s += 2u) {
        issue(b1, s + 1u);
        __builtin_amdgcn_sched_barrier(0);
        compute(b0, s);
        issue(b0, s + 2u);
        __builtin_amdgcn_sched_barrier(0);
        compute(b1, s + 1u);
      }
      if constexpr (NS % 2u == 0u) {
        issue(b1, s + 1u);
        __builtin_amdgcn_sched_barrier(0);
        compute(b0, s);
        __builtin_amdgcn_sched_barrier(0);
        compute(b1, s + 1u);
      } else {
        compute(b0, s);
      }
    }
    if constexpr (SA > 1) {  // add the K splits in split order (s_red has LDS of its own)
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        s_red[(wave * 8u + j) * 64u + lane] = ag[j];
        s_red[(wave * 8u + 4u + j) * 64u + lane] = au[j];
      }
      lds_barrier();
      if (sa == 0) {
#pragma unroll
        for (uint32_t s2 = 1; s2 < SA; ++s2)
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) {
            ag[j] = ag[j] + s_red[((s2 * CA + ca) * 8u + j) * 64u + lane];
            au[j] = au[j] + s_red[((s2 * CA + ca) * 8u + 4u + j) * 64u + lane];
          }
      }
    }
    if constexpr (kQuant) {
      // kDown: W2 step s of wave w covers 32-column item 8 (s / NBN) + w, K
      // blocks ((s + g) % NBN) kDCN .. (rotated by the tile, as above): the 8
      // waves read neighbouring items, so the workgroup's reads advance through
      // the expert's W2 as one front (items PDN w .. per wave, 8 fronts 128 KiB
      // apart: 1.7 us slower at T=64)
      const uint8_t* w2e = w2 + (size_t)e * H * I;
      const float* w2se = w2s + (size_t)e * (H / 128u) * KBI;
      const uint32_t rotn = g % NBN;
      auto issue_dn = [&](DownStep<kDCN>& st, uint32_t s) __attribute__((always_inline)) {
        const uint32_t d = (s / NBN) * kWaves + wave, kb0 = ((s + rotn) % NBN) * kDCN;
#pragma unroll
        for (uint32_t i = 0; i < kDCN; ++i)
#pragma unroll
          for (uint32_t t2 = 0; t2 < 2; ++t2)
            st.w[i][t2] = nk::load_tile_operand_once(nk::tile_base(w2e, d * 2u + t2, kb0 + i, KBI), lane);
        const uint32_t li = (lane >> 1) < kDCN ? lane >> 1 : 0u;
        st.ws = w2se[((d * 2u + (lane & 1u)) >> 3) * KBI + kb0 + li];
      };
      DownStep<kDCN> f0, f1;
      if constexpr (kDown) issue_dn(f0, 0u);  // the weight stream goes on under the requant
      // the item's h rows are in LDS; waves 0 .. P - 1 requantise one 128-column block each
      lds_barrier();
      if (wave < P) {
        const uint4* src = reinterpret_cast<const uint4*>(&s_hb[(lane & 15u) * kHb + wave * 128u + (lane >> 4) * 32u]);
        uint32_t raw[16];
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
          const uint4 v = src[q];
          raw[4 * q] = v.x; raw[4 * q + 1] = v.y; raw[4 * q + 2] = v.z; raw[4 * q + 3] = v.w;
        }
        uint4 qlo, qhi;
        float scale;
        quant_block(raw, qlo, qhi, scale);
        const size_t blk = (size_t)(row0 >> 4) * KBI + grp * P + wave;  // the stream path's h layout
        *reinterpret_cast<uint4*>(hq + blk * 2048u + lane * 16u) = qlo;
        *reinterpret_cast<uint4*>(hq + blk * 2048u + 1024u + lane * 16u) = qhi;
        if (lane < 16u) hs[blk * 16u + lane] = scale;
        if constexpr (kDown) {  // and the down's A operand: K block `wave` (s_a is free)
          *reinterpret_cast<uint4*>(&s_big[wave * 2048u + lane * 16u]) = qlo;
          *reinterpret_cast<uint4*>(&s_big[wave * 2048u + 1024u + lane * 16u]) = qhi;
          if (lane < 16u) s_xs[wave * 16u + lane] = scale;
        }
      }
      if constexpr (kDown) {
        // lane l: the route of the tile's row l & 15 (the rank among e's
        // tokens, as staged), -1 for padding
        int32_t route = -1;
        {
          const unsigned long long emask = s_mask[e];
          const uint32_t j = 16u * k + (lane & 15u);
          if (j < (uint32_t)__popcll(emask)) {
            const uint32_t t = nth_bit(emask, j), sl = slot_of(s_ids, t, Ktot, e);
            if (sl < Ktot) route = (int32_t)(t * Ktot + sl);  // (always: the mask comes from the ids)
          }
        }
        lds_barrier();  // the h operand is in LDS
        v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
        auto compute_dn = [&](const DownStep<kDCN>& st, uint32_t s) __attribute__((always_inline)) {
#pragma unroll
          for (uint32_t i = 0; i < kDCN; ++i) {
            const uint32_t kb = ((s + rotn) % NBN) * kDCN + i;
            const v8i a = nk::load_tile_operand(s_big + kb * 2048u, lane);
            const float4 as4 = *reinterpret_cast<const float4*>(&s_xs[kb * 16u + (lane >> 4) * 4u]);
            const float as[4] = {as4.x, as4.y, as4.z, as4.w};
            const v4f d0v = nk::mfma_e4m3_16x16x128(a, st.w[i][0]);
            const v4f d1v = nk::mfma_e4m3_16x16x128(a, st.w[i][1]);
            const float s0 = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(st.ws), (int)(2u * i)));
            const float s1 = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(st.ws), (int)(2u * i + 1u)));
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
              acc0[j] = acc0[j] + s0 * (as[j] * d0v[j]);
              acc1[j] = acc1[j] + s1 * (as[j] * d1v[j]);
            }
          }
          if (s % NBN == NBN - 1u) {  // 32-column item PDN w + s / NBN done: its route partials
            const uint32_t d = (s / NBN) * kWaves + wave;
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
              const int32_t r = __shfl(route, (lane >> 4) * 4u + j);
              if (r >= 0) {
                float* dst = partial + (size_t)r * H + d * 32u + (lane & 15u);
                dst[0] = acc0[j];
                dst[16] = acc1[j];
              }
            }
            acc0 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            acc1 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
          }
        };
        // two step buffers, the last one or two steps peeled (no load under a branch)
        uint32_t s = 0;
#pragma unroll 1
        for (; s + 2u < NSN; s += 2u) {
          issue_dn(f1, s + 1u);
          __builtin_amdgcn_sched_barrier(0);
          compute_dn(f0, s);
          issue_dn(f0, s + 2u);
          __builtin_amdgcn_sched_barrier(0);
          compute_dn(f1, s + 1u);
        }
        if constexpr (NSN % 2u == 0u) {
          issue_dn(f1, s + 1u);
          __builtin_amdgcn_sched_barrier(0);
          compute_dn(f0, s);
          __builtin_amdgcn_sched_barrier(0);
          compute_dn(f1, s + 1u);
        } else {
          compute_dn(f0, s);
        }
      }
    } else if (sa == 0) {  // bf16 h of tile g, column 16 c0 + (l & 15) (P = 1)
      // lane l, j: MFMA row q = (l >> 4) * 4 + j is token q; the tile's row of
      // a token routed to e is its rank among e's tokens, and the rows past
      // e's count take zeros from the other rows q in order (a bijection)
      uint16_t* const hg = hrows + (size_t)g * 16u * I;
      const unsigned long long emask = s_mask[e];
      const uint32_t cnt = (uint32_t)__popcll(emask);
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t q = (lane >> 4) * 4u + j;
        const uint32_t below = (uint32_t)__popcll(emask & ((1ull << q) - 1ull));
        const bool routed = (emask >> q) & 1ull;  // q < T <= 16 for a set bit
        const uint32_t r = routed ? below : cnt + q - below;
        hg[r * I + c0 * 16u + (lane & 15u)] = routed ? nk::bf16_rne(nk::silu(ag[j]) * au[j]) : (uint16_t)0u;
      }
    }
    lds_barrier();  // every wave is done with s_a / s_hb before the next item
  }
}

// ---------------------------------------------------------------------------
// down with the combine folded in
// kFromRows: h from hrows (bf16); PD: items per wave; kHandoff: combine in
// the kernel (else the partials are left to the combine kernel)
template <uint32_t KB, uint32_t KBI, uint32_t SB, uint32_t CHM, bool kFromRows, uint32_t PD, bool kHandoff>
__device__ __forceinline__ void ffn_down(
    const float* __restrict__ topk_weights, const uint8_t* __restrict__ w2, const float* __restrict__ w2s,
    const int32_t* __restrict__ sorted_ids, const int32_t* __restrict__ sorted_expert,
    const int32_t* __restrict__ tile_map, const int32_t* __restrict__ num_valid,
    const uint16_t* __restrict__ hrows, uint8_t* __restrict__ hq, float* __restrict__ hs,
    float* __restrict__ partial, uint32_t* __restrict__ counters, uint16_t* __restrict__ out, uint32_t T,
    uint32_t E, uint32_t K, uint32_t S) {
  using nkstream::lds_barrier;
  constexpr uint32_t H = 128u * KB, I = 128u * KBI;
  constexpr uint32_t CB = kWaves / SB;                 // 32-column items per down item
  constexpr uint32_t KBB = KBI / SB;                   // K blocks per wave
  constexpr uint32_t kDC = KBB >= CHM ? CHM : 1u;      // K blocks per step
  constexpr uint32_t NB = KBB / kDC;                   // steps per wave
  constexpr uint32_t GB = H / (32u * CB * PD);         // items per tile
  constexpr uint32_t NS = PD * NB;                     // steps per wave and item
  constexpr uint32_t kCols = 32u * CB * PD;            // output columns of an item
  static_assert(CB * SB == kWaves && KBI % SB == 0 && KBB % kDC == 0, "K splits");
  static_assert(H % kCols == 0 && GB <= kMaxGroups && KBI <= kWaves && (PD == 1 || SB == 1), "shares");
  static_assert(CB >= 2u && (kCols % kThreads == 0 || kThreads % kCols == 0), "combine columns");
  constexpr uint32_t kRed = SB > 1 ? kWaves * 8u * 64u * 4u : 0u;
  constexpr uint32_t kBig = KBI * 2048u > kRed ? KBI * 2048u : kRed;
  __shared__ __align__(16) uint8_t s_big[kBig];      // h operand | split sums
  __shared__ __align__(16) float s_hsc[KBI * 16u];   // h row scales [kb][row]
  constexpr uint32_t kHeld = kHandoff ? 4u * kWaves : 1u;  // items whose hand-off is made together
  __shared__ int32_t s_itok[kHeld * 16u];                  // held items' row tokens, -1 for padding
  __shared__ uint32_t s_igrp[kHeld], s_ilast[kHeld];       // their column groups, completed-row masks
  uint8_t* const s_h = s_big;
  float* const s_red = reinterpret_cast<float*>(s_big);
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = nkstream::wave_id();
  const uint32_t Ktot = K + S, Etot = E + S;
  if (T > kMaxT || Ktot > kMaxKtot || Etot > kMaxE) return;  // host-checked
  // tiles as the sort counted them, never past the capacity (T Ktot / 16 + Etot):
  // an operation launched out of order may find another tensor's bytes here
  // narrow: an expert holds at most kNarrowT <= 16 rows, so tile g is the first
  // 16 rows of block g (no tile_map hop); the first item's rows and bf16 h
  // rows (wave w < KBI: 128-column block w, lane l row l & 15, columns
  // 32 (l >> 4) .. + 31) load together with the tile count
  const uint32_t cap_blocks = (T * Ktot + 63u) / 64u + Etot;
  // Items, XCD-aware: workgroups are dealt round-robin over the 8 XCDs, so
  // workgroup i (XCD i % 8, j = i / 8) takes column group j % GB of tile slot
  // j / GB of its XCD (tiles round-robin over the XCDs): a tile's GB items
  // share one L2 and fetch its h operand once. Round r adds r * grid. (A grid
  // that is not a multiple of 8 GB keeps item = workgroup.)
  const uint32_t off = gridDim.x % (8u * GB) == 0u
                           ? ((blockIdx.x / 8u / GB) * 8u + blockIdx.x % 8u) * GB + (blockIdx.x / 8u) % GB
                           : blockIdx.x;
  const uint32_t g_first = off / GB;
  nkstream::TileRows tr_first;
  uint4 h_first[kFromRows ? 4 : 1];
  auto load_hrows = [&](uint4 (&v)[kFromRows ? 4 : 1], uint32_t g) __attribute__((always_inline)) {
    const uint4* src = reinterpret_cast<const uint4*>(hrows + ((size_t)g * 16u + (lane & 15u)) * I + wave * 128u +
                                                      (lane >> 4) * 32u);
#pragma unroll
    for (uint32_t q = 0; q < (kFromRows ? 4u : 1u); ++q) v[q] = src[q];
  };
  // wide: the first item's tile_map entry loads with the tile count (its
  // block clamped: past the count the entry may hold stale bytes), its rows
  // and h operand (fp8 block and scales) right after
  const uint32_t cap_tiles = (T * Ktot + 15u) / 16u + Etot;
  uint4 q_first[2];
  float s_first = 0.0f;
  if constexpr (kFromRows) {
    const uint32_t b = min(g_first, cap_blocks - 1u);
    nkstream::load_rows(tr_first, sorted_ids, sorted_expert, b, b * 64u, T, Ktot, Etot, true);
    if (wave < KBI) load_hrows(h_first, b);
  } else {
    nkstream::load_tile(tr_first, tile_map, sorted_ids, sorted_expert, min(g_first, cap_tiles - 1u), T, Ktot, Etot,
                        true, cap_blocks - 1u);
    if (wave < KBI) {
      const size_t blk = (size_t)(tr_first.row0 >> 4) * KBI + wave;
      q_first[0] = *reinterpret_cast<const uint4*>(hq + blk * 2048u + lane * 16u);
      q_first[1] = *reinterpret_cast<const uint4*>(hq + blk * 2048u + 1024u + lane * 16u);
      if (lane < 16u) s_first = hs[blk * 16u + lane];
    }
  }
  const uint32_t ntile = min((uint32_t)num_valid[2], kFromRows ? cap_blocks : cap_tiles);

  // Combine hand-off of the held items: once every wave's partial stores have
  // completed, wave w lane l counts the arrival of held item 4w + (l >> 4),
  // row l & 15; the arrivals that complete a (token, group) are then combined.
  uint32_t nheld = 0;
  auto handoff = [&](uint32_t n) __attribute__((always_inline)) {
    store_barrier();
    {
      const uint32_t i = wave * 4u + (lane >> 4);
      uint32_t last = 0;
      if (i < n) {
        const int32_t t = s_itok[i * 16u + (lane & 15u)];
        if (t >= 0) {
          uint32_t* ctr = &counters[(uint32_t)t * kMaxGroups + s_igrp[i]];
          // wrapping increment: the Ktot-th arrival leaves the counter at zero
          last = __builtin_amdgcn_atomic_inc32(ctr, Ktot - 1u, __ATOMIC_RELAXED, "agent") == Ktot - 1u;
        }
      }
      const unsigned long long m = __ballot(last);
      if (lane < 4u && wave * 4u + lane < n) s_ilast[wave * 4u + lane] = (uint32_t)(m >> (16u * lane)) & 0xffffu;
    }
    lds_barrier();
    // the completed rows' tokens: kRows at once, kCpt columns of the group per thread
    constexpr uint32_t kRows = kCols >= kThreads ? 1u : kThreads / kCols;
    constexpr uint32_t kCpt = kCols >= kThreads ? kCols / kThreads : 1u;
    const uint32_t slot_r = tid / (kThreads / kRows);
#pragma unroll 1
    for (uint32_t i = 0; i < n; ++i) {
      uint32_t todo = __builtin_amdgcn_readfirstlane(s_ilast[i]);
      const uint32_t gi = __builtin_amdgcn_readfirstlane(s_igrp[i]);
      while (todo) {  // uniform
        uint32_t pick = todo, rowsel = 16u;
        for (uint32_t r = 0; r < kRows && pick; ++r) {
          const uint32_t row = (uint32_t)__ffs((int)pick) - 1u;
          pick &= pick - 1u;
          if (r == slot_r) rowsel = row;
        }
        todo = pick;
        if (rowsel < 16u) {
          const int32_t t = s_itok[i * 16u + rowsel];
          const float* wrow = topk_weights + (size_t)t * Ktot;
#pragma unroll
          for (uint32_t q = 0; q < kCpt; ++q) {
            const uint32_t nc = gi * kCols + (tid % (kThreads / kRows)) + q * kThreads;
            const float* prow = partial + (size_t)t * Ktot * H + nc;
            float pv[kMaxKtot];
#pragma unroll
            for (uint32_t s = 0; s < kMaxKtot; ++s)
              if (s < Ktot) pv[s] = __hip_atomic_load(prow + (size_t)s * H, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float y = 0.0f;
#pragma unroll
            for (uint32_t s = 0; s < kMaxKtot; ++s)
              if (s < Ktot) y = fmaf(wrow[s], pv[s], y);
            out[(size_t)t * H + nc] = nk::bf16_rne(y);
          }
        }
      }
    }
  };

#pragma unroll 1
  for (uint32_t item = off; item < ntile * GB; item += gridDim.x) {
    const uint32_t g = item / GB, grp = item % GB;
    nkstream::TileRows tr;
    // rows (and h) loaded at the start
    const bool first = item == off && g_first < (kFromRows ? cap_blocks : cap_tiles);
    if (first) {
      tr = tr_first;
    } else if constexpr (kFromRows) {
      nkstream::load_rows(tr, sorted_ids, sorted_expert, g, g * 64u, T, Ktot, Etot, true);
    } else {
      nkstream::load_tile(tr, tile_map, sorted_ids, sorted_expert, g, T, Ktot, Etot, true, cap_blocks - 1u);
    }
    const uint32_t e = (uint32_t)tr.expert, row0 = tr.row0;
    const int32_t route = tr.row;  // lane l: the route of row l & 15, -1 for padding
    const int32_t tok = route >= 0 ? route / (int32_t)Ktot : -1;
    const uint8_t* w2e = w2 + (size_t)e * H * I;
    const float* w2se = w2s + (size_t)e * (H / 128u) * KBI;
    const uint32_t cbw = wave % CB, sb = wave / CB;
    const uint32_t d0 = (grp * CB + cbw) * PD;  // this wave's first 32-column item within H / 32
    const uint32_t kbw = sb * KBB;
    // step s: 32-column item d0 + s / NB, K blocks kbw + ((s + rot) % NB) * kDC .. (rotated as above)
    const uint32_t rot = item % NB;
    auto issue = [&](DownStep<kDC>& st, uint32_t s) __attribute__((always_inline)) {
      const uint32_t d = d0 + s / NB, kb0 = kbw + ((s + rot) % NB) * kDC;
#pragma unroll
      for (uint32_t i = 0; i < kDC; ++i)
#pragma unroll
        for (uint32_t t2 = 0; t2 < 2; ++t2)
          st.w[i][t2] = nk::load_tile_operand_once(nk::tile_base(w2e, d * 2u + t2, kb0 + i, KBI), lane);
      const uint32_t li = (lane >> 1) < kDC ? lane >> 1 : 0u;
      st.ws = w2se[((d * 2u + (lane & 1u)) >> 3) * KBI + kb0 + li];
    };
    DownStep<kDC> e0, e1;
    issue(e0, 0u);
    // the tile's h operand: wave w < KBI stages 128-column block w
    if (wave < KBI) {
      const size_t blk = (size_t)(row0 >> 4) * KBI + wave;
      uint4 qlo, qhi;
      float scale = 0.0f;
      if constexpr (kFromRows) {  // requantise bf16 rows: lane l row l & 15, columns 32 (l >> 4) .. + 31
        uint4 hv[4];
        if (first) {
#pragma unroll
          for (uint32_t q = 0; q < 4; ++q) hv[q] = h_first[q];
        } else {
          load_hrows(hv, g);
        }
        uint32_t raw[16];
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
          const uint4 v = hv[q];
          raw[4 * q] = v.x; raw[4 * q + 1] = v.y; raw[4 * q + 2] = v.z; raw[4 * q + 3] = v.w;
        }
        quant_block(raw, qlo, qhi, scale);
        if (grp == 0) {  // for inspection: the stream path's h layout
          *reinterpret_cast<uint4*>(hq + blk * 2048u + lane * 16u) = qlo;
          *reinterpret_cast<uint4*>(hq + blk * 2048u + 1024u + lane * 16u) = qhi;
          if (lane < 16u) hs[blk * 16u + lane] = scale;
        }
      } else if (first) {
        qlo = q_first[0];
        qhi = q_first[1];
        scale = s_first;
      } else {
        qlo = *reinterpret_cast<const uint4*>(hq + blk * 2048u + lane * 16u);
        qhi = *reinterpret_cast<const uint4*>(hq + blk * 2048u + 1024u + lane * 16u);
        if (lane < 16u) scale = hs[blk * 16u + lane];
      }
      *reinterpret_cast<uint4*>(&s_h[wave * 2048u + lane * 16u]) = qlo;
      *reinterpret_cast<uint4*>(&s_h[wave * 2048u + 1024u + lane * 16u]) = qhi;
      if (lane < 16u) s_hsc[wave * 16u + lane] = scale;
    }
    lds_barrier();

    v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    auto store_partials = [&](uint32_t d) __attribute__((always_inline)) {
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const int32_t r = __shfl(route, (lane >> 4) * 4u + j);
        if (r >= 0) {
          float* dst = partial + (size_t)r * H + d * 32u + (lane & 15u);
          if constexpr (kHandoff) {  // read back by another workgroup of this launch
            __hip_atomic_store(dst, acc0[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(dst + 16, acc1[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          } else {  // read by the combine kernel after this launch
            dst[0] = acc0[j];
            dst[16] = acc1[j];
          }
        }
      }
    };
    auto compute = [&](const DownStep<kDC>& st, uint32_t s) __attribute__((always_inline)) {
#pragma unroll
      for (uint32_t i = 0; i < kDC; ++i) {
        const uint32_t kb = kbw + ((s + rot) % NB) * kDC + i;
        const v8i a = nk::load_tile_operand(s_h + kb * 2048u, lane);
        const float4 as4 = *reinterpret_cast<const float4*>(&s_hsc[kb * 16u + (lane >> 4) * 4u]);
        const float as[4] = {as4.x, as4.y, as4.z, as4.w};
        const v4f d0v = nk::mfma_e4m3_16x16x128(a, st.w[i][0]);
        const v4f d1v = nk::mfma_e4m3_16x16x128(a, st.w[i][1]);
        const float s0 = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(st.ws), (int)(2u * i)));
        const float s1 = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(st.ws), (int)(2u * i + 1u)));
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          acc0[j] = acc0[j] + s0 * (as[j] * d0v[j]);
          acc1[j] = acc1[j] + s1 * (as[j] * d1v[j]);
        }
      }
      if constexpr (SB == 1) {
        if (s % NB == NB - 1u) {  // item d0 + s / NB done
          store_partials(d0 + s / NB);
          acc0 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
          acc1 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
    };
    if constexpr (NS == 1) {
      compute(e0, 0u);
    } else {
      // the last one or two steps peeled: no load is issued under a branch
      // (the wait counts at a join would drain the step in flight) and none
      // past the last step
      uint32_t s = 0;
#pragma unroll 1
      for (; s + 2u < NS; s += 2u) {
        issue(e1, s + 1u);
        __builtin_amdgcn_sched_barrier(0);
        compute(e0, s);
        issue(e0, s + 2u);
        __builtin_amdgcn_sched_barrier(0);
        compute(e1, s + 1u);
      }
      if constexpr (NS % 2u == 0u) {
        issue(e1, s + 1u);
        __builtin_amdgcn_sched_barrier(0);
        compute(e0, s);
        if constexpr (!kFromRows) __builtin_amdgcn_sched_barrier(0);  // (rows: spills at 128 VGPRs)
        compute(e1, s + 1u);
      } else {
        compute(e0, s);
      }
    }
    if constexpr (SB > 1) {
      lds_barrier();  // every wave is done with s_h
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        s_red[(wave * 8u + j) * 64u + lane] = acc0[j];
        s_red[(wave * 8u + 4u + j) * 64u + lane] = acc1[j];
      }
      lds_barrier();
      if (sb == 0) {
#pragma unroll
        for (uint32_t s2 = 1; s2 < SB; ++s2)
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) {
            acc0[j] = acc0[j] + s_red[((s2 * CB + cbw) * 8u + j) * 64u + lane];
            acc1[j] = acc1[j] + s_red[((s2 * CB + cbw) * 8u + 4u + j) * 64u + lane];
          }
        store_partials(d0);  // PD = 1
      }
    }
    // note the item's rows for the combine hand-off, made for up to kHeld
    // items at once: one wait for the partial stores instead of one per item
    if constexpr (kHandoff) {
      if (wave == 0 && lane < 16u) s_itok[nheld * 16u + lane] = tok;
      if (tid == 0) s_igrp[nheld] = grp;
      ++nheld;
      if (nheld == kHeld || item + gridDim.x >= ntile * GB) {  // uniform
        handoff(nheld);
        nheld = 0;
      }
    }
    lds_barrier();  // every wave is done with s_h before the next item
  }
}

// ---------------------------------------------------------------------------
// down for a single token (T = 1), the combine in the workgroup
// (reference: kernels/gfx950/templates/moe/decode/down_reduce_mfma_2wave.inc:14-291)
//
// With one token every tile g < Ktot holds one row, the token's route of slot
// s_g to expert e_g, so a workgroup can own output columns across all the
// routes: workgroup b computes columns [16 b, 16 b + 16) of every route's fp32
// partial and adds them in slot order itself, with no hand-off between
// workgroups. Wave w takes tiles w and w + 8: lane l loads h columns
// 8 l .. 8 l + 7 of the tile's row (K block l / 16 is a 16-lane row), which is
// requantised under the 1x128 rule of the narrow down (row max by DPP) into a
// per-wave LDS row; the MFMA A operand is that row with rows 1 .. 15 zero.
// Per tile p = sum over K blocks in order of w_s * (a_s * mfma) from 0 (the
// narrow down's split order), written to partial[route] and to LDS by slot;
// out = bf16(sum over slots in order of fmaf(weight, p, acc)) from 0.
// Workgroup 0 also writes the tiles' requantised h (hq / hs, tile layout) for
// inspection, as the narrow down's first column group does.
template <uint32_t KB, uint32_t KBI>
__device__ __forceinline__ void ffn_down_single(
    const float* __restrict__ topk_weights, const uint8_t* __restrict__ w2, const float* __restrict__ w2s,
    const int32_t* __restrict__ sorted_ids, const int32_t* __restrict__ sorted_expert,
    const uint16_t* __restrict__ hrows, uint8_t* __restrict__ hq, float* __restrict__ hs,
    float* __restrict__ partial, uint16_t* __restrict__ out, uint32_t T, uint32_t E, uint32_t K, uint32_t S) {
  constexpr uint32_t H = 128u * KB, I = 128u * KBI;
  static_assert(I == 512u, "lane l holds h columns 8 l .. 8 l + 7: one 512-column row per wave");
  constexpr uint32_t kTilesPerWave = kMaxKtot / kWaves;  // 2
  __shared__ __align__(16) uint8_t s_q[kWaves][kTilesPerWave][I];  // requantised h rows
  __shared__ float s_p[kMaxKtot * 16u];                             // partials [slot][column]
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = nkstream::wave_id();
  const uint32_t Ktot = K + S, Etot = E + S;
  if (T != 1u || Ktot > kMaxKtot || Etot > kMaxE) return;  // host-checked
  const uint32_t c16 = blockIdx.x;  // 16-column group
  if (c16 >= H / 16u) return;

  // everything a tile needs that does not depend on its expert, loaded first
  uint32_t eg[kTilesPerWave], slot[kTilesPerWave];
  uint4 hv[kTilesPerWave];
#pragma unroll
  for (uint32_t i = 0; i < kTilesPerWave; ++i) {
    const uint32_t g = min(wave + kWaves * i, Ktot - 1u);
    const int32_t e = sorted_expert[g];
    eg[i] = (e < 0 || (uint32_t)e >= Etot) ? 0u : (uint32_t)e;  // out of range only for malformed routing
    slot[i] = (uint32_t)sorted_ids[64u * g] >> 24;
    hv[i] = *reinterpret_cast<const uint4*>(hrows + (size_t)g * 16u * I + lane * 8u);
  }
  // the tiles' W2 blocks (16 output columns x 128 K) and block scales
  v8i wb[kTilesPerWave][KBI];
  float ws[kTilesPerWave][KBI];
#pragma unroll
  for (uint32_t i = 0; i < kTilesPerWave; ++i) {
    const uint8_t* w2e = w2 + (size_t)eg[i] * H * I;
    const float* w2se = w2s + (size_t)eg[i] * (H / 128u) * KBI;
#pragma unroll
    for (uint32_t kb = 0; kb < KBI; ++kb) {
      wb[i][kb] = nk::load_tile_operand_once(nk::tile_base(w2e, c16, kb, KBI), lane);
      ws[i][kb] = w2se[(c16 >> 3) * KBI + kb];
    }
  }
  // requantise the rows: amax over the 16 lanes of a K block
  float scale[kTilesPerWave];
#pragma unroll
  for (uint32_t i = 0; i < kTilesPerWave; ++i) {
    const uint4 v = hv[i];
    const float f[8] = {nk::bf16_lo(v.x), nk::bf16_hi(v.x), nk::bf16_lo(v.y), nk::bf16_hi(v.y),
                        nk::bf16_lo(v.z), nk::bf16_hi(v.z), nk::bf16_lo(v.w), nk::bf16_hi(v.w)};
    float amax = nk::kAmaxFloor;
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) amax = fmaxf(amax, fabsf(f[q]));
    uint32_t ab = __float_as_uint(amax);  // non-negative: the bit patterns order as the values
    ab = max(ab, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)ab, 0xB1, 0xF, 0xF, false));
    ab = max(ab, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)ab, 0x4E, 0xF, 0xF, false));
    ab = max(ab, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)ab, 0x141, 0xF, 0xF, false));
    ab = max(ab, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)ab, 0x140, 0xF, 0xF, false));
    scale[i] = __uint_as_float(ab) * nk::inv_e4m3_max();
    const float inv = 1.0f / scale[i];
    *reinterpret_cast<uint2*>(&s_q[wave][i][lane * 8u]) =
        make_uint2(nk::e4m3x4(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv),
                   nk::e4m3x4(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv));
  }
  // p of each tile: lanes 0 .. 15 hold row 0 (the route), column l
  const bool row0 = (lane & 15u) == 0u;
  const float floor_scale = nk::kAmaxFloor * nk::inv_e4m3_max();  // an all-zero row's scale
#pragma unroll
  for (uint32_t i = 0; i < kTilesPerWave; ++i) {
    const uint32_t g = wave + kWaves * i;
    if (g >= Ktot) break;  // uniform
    float p = 0.0f;
#pragma unroll
    for (uint32_t kb = 0; kb < KBI; ++kb) {
      // A operand: lane 16 c holds row 0's columns 128 kb + 32 c .. + 31, other rows zero
      const uint4* src = reinterpret_cast<const uint4*>(&s_q[wave][i][kb * 128u + 32u * (lane >> 4)]);
      const uint4 lo = row0 ? src[0] : make_uint4(0u, 0u, 0u, 0u);
      const uint4 hi = row0 ? src[1] : make_uint4(0u, 0u, 0u, 0u);
      v8i a;
      a[0] = (int)lo.x; a[1] = (int)lo.y; a[2] = (int)lo.z; a[3] = (int)lo.w;
      a[4] = (int)hi.x; a[5] = (int)hi.y; a[6] = (int)hi.z; a[7] = (int)hi.w;
      const v4f d = nk::mfma_e4m3_16x16x128(a, wb[i][kb]);
      const float as = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(scale[i]), (int)(16u * kb)));
      p = p + ws[i][kb] * (as * d[0]);
      if (blockIdx.x == 0) {  // for inspection: the tile's requantised h in the stream path's layout
        const size_t blk = (size_t)(4u * g) * KBI + kb;
        *reinterpret_cast<uint4*>(hq + blk * 2048u + lane * 16u) = lo;
        *reinterpret_cast<uint4*>(hq + blk * 2048u + 1024u + lane * 16u) = hi;
        if (lane < 16u) hs[blk * 16u + lane] = lane == 0u ? as : floor_scale;
      }
    }
    if (lane < 16u) {
      s_p[slot[i] * 16u + lane] = p;
      partial[(size_t)slot[i] * H + c16 * 16u + lane] = p;
    }
  }
  nkstream::lds_barrier();
  if (wave == 0 && lane < 16u) {
    float y = 0.0f;
    for (uint32_t s = 0; s < Ktot; ++s) y = fmaf(topk_weights[s], s_p[s * 16u + lane], y);
    out[c16 * 16u + lane] = nk::bf16_rne(y);
  }
}

}  // namespace nkffn

#define NK_FFN_DOWN_SINGLE(HV, IV)                                                                 \
  NK_KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))                        \
  void netra_moe_ffn_down_h##HV##_i##IV##_single_gfx950(                                          \
      const float* __restrict__ topk_weights, const uint8_t* __restrict__ w2,                      \
      const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,                       \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ tile_map,             \
      const int32_t* __restrict__ num_valid, const uint16_t* __restrict__ hrows,                   \
      uint8_t* __restrict__ hq, float* __restrict__ hs, float* __restrict__ partial,               \
      uint32_t* __restrict__ counters, uint16_t* __restrict__ out, uint32_t T, uint32_t E,         \
      uint32_t K, uint32_t S) {                                                                    \
    (void)tile_map; (void)num_valid; (void)counters;                                               \
    nkffn::ffn_down_single<HV / 128, IV / 128>(topk_weights, w2, w2s, sorted_ids, sorted_expert,   \
                                               hrows, hq, hs, partial, out, T, E, K, S);           \
  }
// Symbol netra_moe_ffn_down_h<H>_i512_single_gfx950: the T = 1 down (H / 16 workgroups).
NK_FFN_DOWN_SINGLE(2048, 512)

#define NK_FFN_PAIR(HV, IV, NAME, SAV, SBV, CHG, WPEG, PG, CHD, WPED, PDV)                                               \
  NK_KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(WPEG)))                      \
  void netra_moe_ffn_gate_up_h##HV##_i##IV##_##NAME##_gfx950(                                      \
      const uint16_t* __restrict__ logits, const float* __restrict__ bias,                         \
      int32_t* __restrict__ topk_ids, float* __restrict__ topk_weights, const uint8_t* __restrict__ xq, \
      const float* __restrict__ xs, const uint8_t* __restrict__ w13, const float* __restrict__ w13s, \
      int32_t* __restrict__ sorted_ids, int32_t* __restrict__ sorted_expert,                       \
      int32_t* __restrict__ tile_map, int32_t* __restrict__ pair_map, int32_t* __restrict__ num_valid, \
      int32_t* __restrict__ counts, uint16_t* __restrict__ hrows, uint8_t* __restrict__ hq,        \
      float* __restrict__ hs, uint32_t T, uint32_t E, uint32_t K, uint32_t S, uint32_t cap_blocks) { \
    nkffn::ffn_gate_up<HV / 128, IV / 128, SAV, CHG, PG>(logits, bias, topk_ids, topk_weights, xq, xs, w13,  \
                                                     w13s, sorted_ids,                              \
                                                     sorted_expert, tile_map, pair_map, num_valid,  \
                                                     counts, hrows, hq, hs, T, E, K, S, cap_blocks); \
  }                                                                                                \
  NK_KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(WPED)))                      \
  void netra_moe_ffn_down_h##HV##_i##IV##_##NAME##_gfx950(                                         \
      const float* __restrict__ topk_weights, const uint8_t* __restrict__ w2,                      \
      const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,                       \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ tile_map,             \
      const int32_t* __restrict__ num_valid, const uint16_t* __restrict__ hrows,                   \
      uint8_t* __restrict__ hq, float* __restrict__ hs, float* __restrict__ partial,               \
      uint32_t* __restrict__ counters, uint16_t* __restrict__ out, uint32_t T, uint32_t E,         \
      uint32_t K, uint32_t S) {                                                                    \
    nkffn::ffn_down<HV / 128, IV / 128, SBV, CHD, (SAV > 1), PDV, (SAV > 1)>(topk_weights, w2, w2s, sorted_ids,     \
                                                             sorted_expert, tile_map, num_valid,   \
                                                             hrows, hq, hs, partial, counters, out, \
                                                             T, E, K, S);                          \
  }
// Symbols netra_moe_ffn_{gate_up,down}_h<H>_i<I>_{wide,narrow}_gfx950: wide has
// no K split (gate/up requantises in the workgroup); narrow splits gate/up K
// over SA and down K over SB waves and requantises in down. CHG / CHD: K
// blocks per step; WPEG / WPED: resident waves per SIMD each is budgeted for;
// PG / PDV: consecutive column items per wave (wide gate/up at P = I / 128
// streams a whole tile per workgroup).
NK_FFN_PAIR(512, 256, wide, 1, 1, 2, 2, 2, 2, 4, 1)
NK_FFN_PAIR(512, 256, narrow, 4, 2, 1, 4, 1, 1, 4, 1)
NK_FFN_PAIR(1024, 1024, wide, 1, 1, 2, 2, 4, 1, 4, 1)
NK_FFN_PAIR(1024, 1024, narrow, 8, 4, 1, 4, 1, 1, 4, 1)
NK_FFN_PAIR(2048, 512, wide, 1, 1, 2, 2, 4, 2, 4, 1)
NK_FFN_PAIR(2048, 512, narrow, 8, 4, 1, 4, 1, 1, 4, 1)
NK_FFN_PAIR(4096, 256, wide, 1, 1, 2, 2, 2, 2, 4, 1)
NK_FFN_PAIR(4096, 256, narrow, 8, 2, 2, 2, 1, 1, 4, 1)

// Symbols netra_moe_ffn_gate_up_down_h<H>_i<I>[_ksplit]_gfx950: the wide gate/up
// with each tile's down in the same workgroup (the tile's h requantised into
// LDS, the expert's W2 streamed right behind its W13, fp32 route partials left
// to the combine kernel): one launch and one weight stream per tile instead of
// two. _ksplit: gate/up K split over the waves, one 16-column item per step.
#define NK_FFN_MERGED(HV, IV, CHG, PG, KSV, SFX)                                                    \
  NK_KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))                         \
  void netra_moe_ffn_gate_up_down_h##HV##_i##IV##SFX##_gfx950(                                     \
      const uint16_t* __restrict__ logits, const float* __restrict__ bias,                         \
      int32_t* __restrict__ topk_ids, float* __restrict__ topk_weights, const uint8_t* __restrict__ xq, \
      const float* __restrict__ xs, const uint8_t* __restrict__ w13, const float* __restrict__ w13s, \
      int32_t* __restrict__ sorted_ids, int32_t* __restrict__ sorted_expert,                       \
      int32_t* __restrict__ tile_map, int32_t* __restrict__ pair_map, int32_t* __restrict__ num_valid, \
      int32_t* __restrict__ counts, uint16_t* __restrict__ hrows, uint8_t* __restrict__ hq,        \
      float* __restrict__ hs, const uint8_t* __restrict__ w2, const float* __restrict__ w2s,       \
      float* __restrict__ partial, uint32_t T, uint32_t E, uint32_t K, uint32_t S, uint32_t cap_blocks) { \
    nkffn::ffn_gate_up<HV / 128, IV / 128, 1, CHG, PG, true, KSV>(logits, bias, topk_ids, topk_weights, xq, xs, \
                                                          w13, w13s, sorted_ids, sorted_expert,   \
                                                          tile_map, pair_map, num_valid, counts,  \
                                                          hrows, hq, hs, T, E, K, S, cap_blocks,  \
                                                          w2, w2s, partial);                      \
  }
NK_FFN_MERGED(512, 256, 2, 2, false, )
NK_FFN_MERGED(2048, 512, 2, 4, false, )
NK_FFN_MERGED(2048, 512, 2, 4, true, _ksplit)

// Symbols netra_moe_ffn_down_h<H>_i<I>_rows_gfx950: the down for the narrow
// gate/up's bf16 h rows (requantised per tile, as the narrow down does) with
// the wide down's item shape and no hand-off, leaving fp32 route partials to
// the combine kernel: from 5 tokens on the hand-off's K-split sums, counters
// and last-arriver combines cost more than a separate combine launch.
#define NK_FFN_DOWN_ROWS(HV, IV, SBV, CHD, WPED, PDV)                                                \
  NK_KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(WPED)))                      \
  void netra_moe_ffn_down_h##HV##_i##IV##_rows_gfx950(                                             \
      const float* __restrict__ topk_weights, const uint8_t* __restrict__ w2,                      \
      const float* __restrict__ w2s, const int32_t* __restrict__ sorted_ids,                       \
      const int32_t* __restrict__ sorted_expert, const int32_t* __restrict__ tile_map,             \
      const int32_t* __restrict__ num_valid, const uint16_t* __restrict__ hrows,                   \
      uint8_t* __restrict__ hq, float* __restrict__ hs, float* __restrict__ partial,               \
      uint32_t* __restrict__ counters, uint16_t* __restrict__ out, uint32_t T, uint32_t E,         \
      uint32_t K, uint32_t S) {                                                                    \
    nkffn::ffn_down<HV / 128, IV / 128, SBV, CHD, true, PDV, false>(topk_weights, w2, w2s, sorted_ids, \
                                                                 sorted_expert, tile_map, num_valid, \
                                                                 hrows, hq, hs, partial, counters, out, \
                                                                 T, E, K, S);                    \
  }
// (the wide pairs' down parameters above)
NK_FFN_DOWN_ROWS(512, 256, 1, 2, 4, 1)
NK_FFN_DOWN_ROWS(1024, 1024, 1, 1, 4, 1)
NK_FFN_DOWN_ROWS(2048, 512, 1, 2, 4, 1)
NK_FFN_DOWN_ROWS(4096, 256, 1, 2, 4, 1)
