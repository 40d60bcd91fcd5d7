// Launch plan of the M768 prefill producer/reducer pair on this build's
// kernels, shared by the module-loaded bridge (netra_moe_prefill_m768_launch)
// and the allocation-free entry point (netra_moe_prefill_launch_noalloc).
//
// The reference runs one fused producer (gate/up + SiLU + requant + split-K2
// down, fp16 partials) and one reducer (runtime/gfx950/fp8/moe/
// moe_prefill_m768_bridge.hip:134-154). This build runs four kernels with the
// same inputs, outputs and partial format:
//   1 netra_moe_block_pairs_gfx950             sorted expert blocks -> block pairs
//   2 netra_moe_gate_up_lds_aiter_h2048_gfx950 h (e4m3, scratch) + 1x128 scales
//                                              (route_scale_workspace_f32)
//   3 netra_moe_down_rows_aiter_f16x2_i512_gfx950  fp16 split-K2 partials
//   4 netra_moe_route_reduce_f16x2_gfx950      slot-ordered reduce -> bf16
// The shape is the reference's (hidden 2048, intermediate 512, 257 experts,
// 9 routes per token, 64-row blocks); rows is 768 for the bridge and at most
// 768 for the allocation-free entry point, with capacity
// ceil(rows * 9 / 64) + 257 blocks (365 at 768,
// manifests/gfx950/models/qwen36-35b-c64-fp8.json:43-49) and the split-K2
// halves rows * 9 + capacity rows apart (7277 at 768, the reference's
// kHalfElements / 2048).
//
// Scratch (device memory beyond the caller's buffers): h e4m3 [capacity * 64,
// 512], the block-pair list [capacity] and four counts.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace netra_prefill {

constexpr uint32_t kHidden = 2048;
constexpr uint32_t kInter = 512;
constexpr uint32_t kExperts = 257;
constexpr uint32_t kTopk = 9;
constexpr uint32_t kBlockRows = 64;
constexpr uint32_t kMaxRows = 768;
constexpr uint32_t kDownGroups = 2;  // 128-column groups per down item (about 1024 items at 768 rows)

constexpr uint32_t capacity_blocks(uint32_t rows) { return (rows * kTopk + kBlockRows - 1) / kBlockRows + kExperts; }
constexpr uint32_t half_rows(uint32_t rows) { return rows * kTopk + capacity_blocks(rows); }
constexpr size_t align256(size_t n) { return (n + 255) / 256 * 256; }
constexpr size_t h_bytes(uint32_t rows) { return static_cast<size_t>(capacity_blocks(rows)) * kBlockRows * kInter; }
constexpr size_t pairs_offset(uint32_t rows) { return align256(h_bytes(rows)); }
constexpr size_t counts_offset(uint32_t rows) { return pairs_offset(rows) + align256(capacity_blocks(rows) * 4u); }
constexpr size_t scratch_bytes(uint32_t rows) { return counts_offset(rows) + 256; }

static_assert(capacity_blocks(kMaxRows) == 365 && half_rows(kMaxRows) == 7277, "the reference's M768 shape");
static_assert(capacity_blocks(kMaxRows) <= 1024, "netra_moe_block_pairs_gfx950 takes one block per thread");

enum Kernel : uint32_t { kPairs = 0, kGateUp = 1, kDown = 2, kReduce = 3, kKernels = 4 };

inline const char* symbol(Kernel k) {
  static const char* const names[kKernels] = {
      "netra_moe_block_pairs_gfx950", "netra_moe_gate_up_lds_aiter_h2048_gfx950",
      "netra_moe_down_rows_aiter_f16x2_i512_gfx950", "netra_moe_route_reduce_f16x2_gfx950"};
  return names[k];
}

struct Buffers {
  const void* hidden_fp8;
  const float* hidden_scale;
  const void* w13;
  const float* w13_scale;
  const void* w2;
  const float* w2_scale;
  const int32_t* sorted_ids;
  const int32_t* sorted_expert;
  const int32_t* num_valid;
  const float* topk_weights;
  float* route_scale;  // h 1x128 scales [capacity * 64, 4]
  void* partials;      // fp16 [2, half_rows, 2048]
  void* output;        // bf16 [rows, 2048]
  void* scratch;       // scratch_bytes(rows)
};

// Kernel argument values of the four launches and the pointer arrays that
// hipModuleLaunchKernel / hipLaunchKernel read them through. Lives on the
// caller's stack for the duration of the launches.
struct Args {
  // pairs
  const void* p_sorted_expert;
  const void* p_num_valid;
  void* p_pair_map;
  void* p_counts;
  uint32_t p_cap;
  // gate/up
  const void* g_xq;
  const void* g_xs;
  const void* g_w13;
  const void* g_w13s;
  const void* g_sorted_ids;
  const void* g_sorted_expert;
  const void* g_counts;
  const void* g_pair_map;
  void* g_hq;
  void* g_hs;
  uint32_t g_T, g_H, g_I, g_Ktot, g_Etot;
  // down
  const void* d_hq;
  const void* d_hs;
  const void* d_w2;
  const void* d_w2s;
  const void* d_sorted_ids;
  const void* d_sorted_expert;
  const void* d_counts;
  void* d_partials;
  uint32_t d_T, d_H, d_I, d_Ktot, d_Etot, d_nbc, d_half;
  // reduce
  const void* r_partials;
  const void* r_weights;
  void* r_out;
  uint32_t r_T, r_H, r_Ktot, r_half;

  void* params[kKernels][16];
  dim3 grid[kKernels];
  dim3 block[kKernels];
};

inline uint32_t xcd_grid(uint32_t items) { return (items + 7u) / 8u * 8u; }

inline void build(Args& a, const Buffers& b, uint32_t rows) {
  const uint32_t cap = capacity_blocks(rows), half = half_rows(rows);
  uint8_t* scratch = static_cast<uint8_t*>(b.scratch);
  void* hq = scratch;
  void* pair_map = scratch + pairs_offset(rows);
  void* counts = scratch + counts_offset(rows);

  a.p_sorted_expert = b.sorted_expert;
  a.p_num_valid = b.num_valid;
  a.p_pair_map = pair_map;
  a.p_counts = counts;
  a.p_cap = cap;
  void* pp[] = {&a.p_sorted_expert, &a.p_num_valid, &a.p_pair_map, &a.p_counts, &a.p_cap};
  for (size_t i = 0; i < sizeof(pp) / sizeof(pp[0]); ++i) a.params[kPairs][i] = pp[i];
  a.grid[kPairs] = dim3(1);
  a.block[kPairs] = dim3(1024);

  a.g_xq = b.hidden_fp8;
  a.g_xs = b.hidden_scale;
  a.g_w13 = b.w13;
  a.g_w13s = b.w13_scale;
  a.g_sorted_ids = b.sorted_ids;
  a.g_sorted_expert = b.sorted_expert;
  a.g_counts = counts;
  a.g_pair_map = pair_map;
  a.g_hq = hq;
  a.g_hs = b.route_scale;
  a.g_T = rows;
  a.g_H = kHidden;
  a.g_I = kInter;
  a.g_Ktot = kTopk;
  a.g_Etot = kExperts;
  void* gp[] = {&a.g_xq, &a.g_xs, &a.g_w13, &a.g_w13s, &a.g_sorted_ids, &a.g_sorted_expert, &a.g_counts,
                &a.g_pair_map, &a.g_hq, &a.g_hs, &a.g_T, &a.g_H, &a.g_I, &a.g_Ktot, &a.g_Etot};
  for (size_t i = 0; i < sizeof(gp) / sizeof(gp[0]); ++i) a.params[kGateUp][i] = gp[i];
  a.grid[kGateUp] = dim3(xcd_grid(cap * (kInter / 128u)));
  a.block[kGateUp] = dim3(512);

  a.d_hq = hq;
  a.d_hs = b.route_scale;
  a.d_w2 = b.w2;
  a.d_w2s = b.w2_scale;
  a.d_sorted_ids = b.sorted_ids;
  a.d_sorted_expert = b.sorted_expert;
  a.d_counts = counts;
  a.d_partials = b.partials;
  a.d_T = rows;
  a.d_H = kHidden;
  a.d_I = kInter;
  a.d_Ktot = kTopk;
  a.d_Etot = kExperts;
  a.d_nbc = kDownGroups;
  a.d_half = half;
  void* dp[] = {&a.d_hq, &a.d_hs, &a.d_w2, &a.d_w2s, &a.d_sorted_ids, &a.d_sorted_expert, &a.d_counts,
                &a.d_partials, &a.d_T, &a.d_H, &a.d_I, &a.d_Ktot, &a.d_Etot, &a.d_nbc, &a.d_half};
  for (size_t i = 0; i < sizeof(dp) / sizeof(dp[0]); ++i) a.params[kDown][i] = dp[i];
  a.grid[kDown] = dim3(xcd_grid(cap * (kHidden / 128u / kDownGroups)));
  a.block[kDown] = dim3(512);

  a.r_partials = b.partials;
  a.r_weights = b.topk_weights;
  a.r_out = b.output;
  a.r_T = rows;
  a.r_H = kHidden;
  a.r_Ktot = kTopk;
  a.r_half = half;
  void* rp[] = {&a.r_partials, &a.r_weights, &a.r_out, &a.r_T, &a.r_H, &a.r_Ktot, &a.r_half};
  for (size_t i = 0; i < sizeof(rp) / sizeof(rp[0]); ++i) a.params[kReduce][i] = rp[i];
  a.grid[kReduce] = dim3((kHidden + 2047u) / 2048u, rows);
  a.block[kReduce] = dim3(256);
}

}  // namespace netra_prefill
