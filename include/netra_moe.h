// FP8 E4M3 block-scaled routed-MoE for gfx950: kernel ABI of the engine
// operations and the direct C entry points of libnetra_moe.so.
//
// Engine operations (code object netra_moe_gfx950.hsaco, launched through
// netra_engine_* from include/netra_engine.h). Each kernel takes pointers
// first, then u32 shape constants, in the order listed. They replace, in
// order, the reference's router GEMV (kernels/gfx950/templates/routing/
// bf16_gemv.inc:16-150), the external SGLang top-k + the shared-gate append
// (runtime/gfx950/routing/decode/qwen36_shared_gate_append_bridge.hip:76-112),
// the external AITER moe_sorting whose output format the reference consumes
// (kernels/gfx950/templates/moe/prefill/fused_splitk2/entry_routing.inc:27-112),
// the decode gate/up + SiLU-quant pair (moe/decode/gate_up_mfma.inc:12-161,
// moe/decode/silu_quant.inc:16-236), the down GEMM (moe/decode/
// down_reduce_mfma_2wave.inc:14-291) and the route reducer
// (moe/prefill/route_reduce_splitk2_f16.inc:6-117):
//
//   exact front end, H in {512,1024,2048,4096}:
//   netra_moe_route_h<H>_t<NT>_gfx950(x bf16[T,H], w bf16[E+S,H], bias f32[E],
//       logits bf16[T,E+S], xq e4m3[T,H], xs f32[T,H/128], ids i32[T,Ktot],
//       weights f32[T,Ktot], counters u32[64*ceil(T/NT)] (zero before the first
//       launch, zero again after each); T, H, rows=E+S, E, K, S)
//       grid (ceil(rows/16), ceil(T/NT)), block 256, NT = max(1, 2048/H) for T <= 128
//       else 4 (NT = 2 for H = 4096); router logits and input quant, then top-k by
//       each token group's last workgroup to finish
//   netra_moe_router_logits_h<H>_t<NT>_gfx950(x, w, logits, xq, xs; T, H, rows)
//       the same grid without the top-k (in front of the narrow decode FFN)
//   netra_moe_router_h2048_t1_gfx950(x, w, logits, xq, xs, mask; T, H, rows,
//       mask_words)   the router bridge's kernel (xq and mask may be null)
//   netra_moe_sort_gfx950(ids, mask, sorted_ids i32[CAP*64], sorted_expert i32[CAP],
//       tile_map i32[CAPT], pair_map i32[CAP], num_valid i32[4], counts i32[E+S];
//       T, Ktot, Etot, W, CAP)
//       grid 1, block 1024, dynamic LDS 4*B + (8*Etot*W if that stays <= 160 KiB),
//       B = Etot*W + 4*Etot + 51 + CAP rounded up to even
//   prefill ("screen") front end, H in {512,1024,2048}, EMAX in {256,512}:
//   netra_moe_route_screen_h<H>_k<KBS>_gfx950(x, w, screen f32[Z,T,RP],
//       wsq f32[Z,RP], slices i32[Etot*8]; Etot*8, T, H, E, RP)
//       grid (ceil(T/128), ceil(RP/128), Z), block 256,
//       RP = E rounded up to 64 (the shared-gate row is not screened), Z = H/128/KBS
//       K splits (KBS in {2,4,8,16}, at most H/128); workgroups with
//       blockIdx.x == 0 write the partial squared router-row norms wsq, and
//       workgroup (0,0,0) clears slices
//   netra_moe_route_select_h<H>_e<EMAX>_w<W>x<V>_gfx950(x, w, bias, screen, wsq, logits,
//       ids, weights, xq, xs, hist i32[G,Etot+1], bucket i32[G,(W/V)*Ktot], slices i32[Etot,8];
//       T, H, E, K, S, RP, Z, G)   grid G = ceil(T/(W/V)), block 64*W,
//       (W, V) in {(4,1), (8,1), (8,2), (8,4)}, V <= H/512 waves per token;
//       slices must hold zeros (route_screen clears them)
//   netra_moe_sort_route_gfx950(hist, bucket, slices, counts, sorted_ids,
//       sorted_expert, tile_map, pair_map, num_valid; T, Ktot, Etot, S, G, W/V, CAP)
//       grid exactly Etot, block 256, dynamic LDS 4*(4*Etot+3)
//   fused decode FFN (T <= 64), (H, I) in {(512,256), (1024,1024), (2048,512), (4096,256)}:
//   netra_moe_ffn_gate_up_h<H>_i<I>_<wide|narrow>_gfx950(logits, bias, ids, weights,
//       xq, xs, w13, w13s, sorted_ids, sorted_expert, tile_map, pair_map, num_valid,
//       counts, hrows bf16[CAPT*16,I], hq, hs; T, E, K, S, CAP)
//       block 512, grid 256 (wide, or H = 4096) / 512 (narrow); the sort rebuilt in
//       the prologue (its outputs as netra_moe_sort_gfx950's); wide (16 < T) reads
//       ids and requantises h to hq / hs; narrow (T <= 16) runs the top-k from
//       logits + bias itself (writing ids / weights) and writes bf16 h rows
//   netra_moe_ffn_down_h<H>_i<I>_<wide|narrow>_gfx950(weights, w2, w2s, sorted_ids,
//       sorted_expert, tile_map, num_valid, hrows, hq, hs, partial f32[T*Ktot,H],
//       counters u32[64*64], out bf16[T,H]; T, E, K, S)   block 512, grid 2048 (wide)
//       / 1024 (narrow); wide leaves the partials to netra_moe_combine_gfx950,
//       narrow combines through the counters (zero before and after each launch)
//   netra_moe_ffn_down_h2048_i512_single_gfx950(the same arguments)   T = 1,
//       grid H/16, block 512: a workgroup owns 16 output columns across all
//       routes and writes out itself (partial for inspection; counters unused)
//   netra_moe_ffn_gate_up_down_h<H>_i<I>[_ksplit]_gfx950(the gate/up arguments, with w2,
//       w2s and partial f32[T*Ktot,H] after hs)   (H, I) in {(512,256), (2048,512)}
//       (_ksplit: (2048,512) only), grid 256, block 512: the wide gate/up (_ksplit: K
//       split over the waves), each workgroup then running its tile's down over all H
//       columns from the requantised h in its LDS; the partials go to
//       netra_moe_combine_gfx950 (used at H = 2048 from 128 expected tiles, _ksplit from
//       150; at H = 512 for every T > 16)
//   netra_moe_ffn_down_h<H>_i<I>_rows_gfx950(the same arguments)   grid 2048,
//       block 512: the narrow gate/up's bf16 rows (requantised per tile, hq / hs
//       written for inspection) through the wide down's items; the partials go
//       to netra_moe_combine_gfx950 (counters and out unused); used for 5 <= T <= 16
//   decode ("stream") GEMMs, H in {512,1024,2048,4096}, I in {256,512,1024,2048}:
//   (every w13 below is in the gate/up-interleaved tile16x128 layout of
//   netra_moe_pack_tiles_gate_up)
//   netra_moe_gate_up_stream_h<H>_c<CH>_gfx950(xq, xs, w13 e4m3[Etot,2I,H],
//       w13s f32[Etot,2I/128,H/128], sorted_ids, sorted_expert, tile_map, num_valid,
//       hq e4m3[CAP*64,I] (tile16x128), hs f32[CAP*4,I/128,16]; T, H, I, Ktot, Etot)
//       grid 256, block 512 (persistent; CH K blocks per prefetch step, 2 or 4;
//       h = bf16(silu(g)*u) is requantised 1x128 in the epilogue)
//   netra_moe_down_stream_i<I>_c<DC>_gfx950(hq, hs, w2 e4m3[Etot,H,I],
//       w2s f32[Etot,H/128,I/128], sorted_ids, sorted_expert, tile_map, num_valid,
//       partial f32[T*Ktot,H]; T, H, I, Ktot, Etot)   grid 2048, block 256
//       (DC K blocks per step, 1 or 2)
//   prefill ("tile") GEMMs, H in {512,1024,2048,4096}, I in {256,512,1024}:
//   netra_moe_gate_up_tile_h<H>_gfx950(xq, xs, w13, w13s, sorted_ids, sorted_expert,
//       num_valid, hq e4m3[CAP*64,I], hs f32[CAP*64,I/128]; T, H, I, Ktot, Etot)
//       grid 8*ceil(CAP*I/128/8), block 256 (items assigned XCD-major); used for H = 4096
//   netra_moe_gate_up_lds_h<H>_gfx950(xq, xs, w13, w13s, sorted_ids, sorted_expert,
//       num_valid, pair_map, hq, hs; T, H, I, Ktot, Etot)   H in {512,1024,2048},
//       grid 8*ceil(CAP*I/128/8), block 512, static LDS <= 155 KiB, T*H < 2^31;
//       one item per (block pair, 128 h columns), assigned XCD-major
//   netra_moe_down_rows_i<I>_gfx950(hq, hs, w2, w2s, sorted_ids, sorted_expert, num_valid,
//       partial bf16[T*Ktot,H]; T, H, I, Ktot, Etot, NBC)   I in {256,512},
//       grid 8*ceil(CAP*(H/128/NBC)/8), block 512, T*Ktot*H*2 < 2^31; one item per
//       (64-row block, NBC consecutive 128-column groups), NBC divides H/128
//   netra_moe_down_tile_i<I>_gfx950(hq, hs, w2, w2s, sorted_ids, sorted_expert, num_valid,
//       partial bf16[T*Ktot,H]; T, H, I, Ktot, Etot)   grid 8*ceil(CAP*H/128/8), block 256;
//       used for I = 1024
//   netra_moe_combine_gfx950(partial f32, weights, out bf16[T,H]; T, H, Ktot)
//       grid (ceil(H/1024), T), block 256
//   netra_moe_combine_bf16_gfx950(partial bf16, weights, out; T, H, Ktot)
//       grid (ceil(H/2048), T), block 256
//
// with Ktot = K + S, Etot = E + S (the shared expert is expert E), W =
// ceil(T/64) mask words per expert, CAP = ceil(T*Ktot/64) + Etot blocks,
// CAPT = ceil(T*Ktot/16) + Etot row tiles.
// Sorted ids are (slot << 24) | token; padding rows hold (Ktot << 24) | T.
#pragma once

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

// Weight preparation: fp32 w[groups, n, k] -> e4m3 q[groups, n, k] plus fp32
// 128x128 block scales s[groups, n/128, k/128] (scale = max(amax, 1e-10) *
// 0x3b124925, q = e4m3_rne(w * (1/scale))). n and k must be multiples of 128.
// Replaces the checkpoint re-quantisation recipe the reference plans in
// compiler/netra_compiler/layouts.py:175-206 and delegates to its loader.
// Returns 0 or a hipError_t value (-1 for invalid shapes); the message is
// available from netra_moe_last_error() on the calling thread, following the
// reference bridges (runtime/gfx950/fp8/moe/qwen36_moe_silu_mul_quant_bridge.h:18-59).
int netra_moe_quant_blocks(const float* w, uint8_t* q, float* s, uint32_t groups, uint32_t n,
                           uint32_t k, hipStream_t stream);

// Weight layout change for the GEMM kernels: row-major e4m3 src[groups, n, k]
// -> dst in the tile16x128 layout (n/16 x k/128 tiles, row tiles outermost;
// each tile is 2 KiB; lane l's 32-byte MFMA operand, row l % 16, columns
// (l / 16) * 32 .. +31, is split into its low half at byte l * 16 and its high
// half at byte 1024 + l * 16, so each half-operand wave load reads 1 KiB
// contiguous). n % 16 == 0, k % 128 == 0, src and dst distinct. The
// reference consumes AITER's own shuffled layout
// (kernels/gfx950/templates/common/addressing.inc:22-27); this is the
// layout of this build's kernels. Same error convention as above.
int netra_moe_pack_tiles(const uint8_t* src, uint8_t* dst, uint32_t groups, uint32_t n,
                         uint32_t k, hipStream_t stream);

// The same for W13 (n = 2I: gate rows, then up rows; n % 32 == 0), with the
// row tiles interleaved: gate tile t at 2 t, up tile t at 2 t + 1, so each
// gate/up pair the gate/up kernels stream together is contiguous. The gate/up
// kernels read W13 only in this layout. Same error convention as above.
int netra_moe_pack_tiles_gate_up(const uint8_t* src, uint8_t* dst, uint32_t groups, uint32_t n,
                                 uint32_t k, hipStream_t stream);

// The same two layout changes from weights already in the AITER 16x16 shuffle
// the reference's kernels consume (layout "aiter_shuffle_16x16_fp8_block128",
// compiler/netra_compiler/layouts.py:90-106; bytes of [groups, n, k] stored as
// [n/16][k/32][2][16][16], the inverse of
// tools/benchmark/export_qwen36_dense_m1_capture.py:55-63), so a checkpoint
// prepared for the reference loads without a round trip through row-major.
// src is the shuffled tensor; same shape rules and error convention as above.
int netra_moe_pack_tiles_from_aiter(const uint8_t* src, uint8_t* dst, uint32_t groups, uint32_t n,
                                    uint32_t k, hipStream_t stream);
int netra_moe_pack_tiles_gate_up_from_aiter(const uint8_t* src, uint8_t* dst, uint32_t groups,
                                            uint32_t n, uint32_t k, hipStream_t stream);

// Conversion self-check: writes the contract's integer E4M3 encoding (sw) and
// the hardware conversion used by the hot kernels (hw) of n fp32 inputs.
// No counterpart in the reference; tests use it to prove the two agree.
int netra_moe_e4m3_check(const float* in, uint8_t* sw, uint8_t* hw, uint32_t n,
                         hipStream_t stream);

// Device-to-device copy of `bytes` (a multiple of 16, both pointers 16-byte
// aligned) by a plain streaming kernel. No counterpart in the reference: the
// benchmark uses it to calibrate the HBM byte counters and to measure the
// achievable copy bandwidth.
int netra_moe_copy(const void* src, void* dst, uint64_t bytes, hipStream_t stream);

// Allocation-free prefill producer/reducer. No counterpart in the reference:
// it is for callers that cannot allocate device memory (code under HIP stream
// capture, tight serving loops, harnesses that forbid hipMalloc). It computes
// what netra_moe_prefill_m768_launch (include/netra_qwen36_bridges.h)
// computes, with the same arguments and formats, for `rows` tokens in
// 1..768 (capacity ceil(rows * 9 / 64) + 257 sorted blocks; partials_f16 is
// [2, rows * 9 + capacity, 2048]; route_scale_workspace_f32 [capacity * 64,
// 4]; output_bf16 [rows, 2048]), needs no load call, and allocates nothing:
// its 11.7 MiB of scratch is a static device array of this library, resolved
// once per device. Calls that overlap on one GPU share that array and race.
// rows outside 1..768 are refused (-1). Same error convention as above.
int netra_moe_prefill_launch_noalloc(const void* hidden_fp8, const float* hidden_scale_f32, const void* w13_fp8,
                                     const float* w13_scale_f32, const void* w2_fp8, const float* w2_scale_f32,
                                     const int32_t* sorted_token_ids_i32, const float* sorted_weights_f32,
                                     const int32_t* sorted_expert_ids_i32, const int32_t* num_valid_ids_i32,
                                     const float* topk_weights_f32, float* route_scale_workspace_f32,
                                     void* partials_f16, void* output_bf16, uint32_t rows, hipStream_t stream);

const char* netra_moe_last_error(void);

#ifdef __cplusplus
}
#endif
