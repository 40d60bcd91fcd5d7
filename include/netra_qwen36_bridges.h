// Per-operation bridges at the reference's own C ABIs, implemented by
// libnetra_bridges.so over this build's code object (netra_moe_gfx950.hsaco).
//
// Each family replaces the same-named entry points of the reference; names,
// argument order and meaning, return convention and lifecycle are the
// reference's:
//   * *_load(path) loads the code object at `path` (pass this build's
//     netra_moe_gfx950.hsaco) and resolves its kernels. Loading the same path
//     again is a no-op; a different path needs *_unload first. gfx950 only.
//   * *_launch(...) dispatches on the caller's stream. It allocates nothing,
//     synchronises nothing and is safe under stream capture.
//   * *_unload() releases the module (and the family's scratch) after every
//     launch and graph replay has completed.
//   * Returns 0 on success, the hipError_t value of a failed HIP call, or -1
//     for a refused argument or state; *_last_error() returns a thread-local
//     description of the most recent nonzero return of that family.
//
// Tensor formats (the reference's): FP8 is OCP e4m3fn, weights in the AITER
// 16x16 shuffle ("aiter_shuffle_16x16_fp8_block128",
// compiler/netra_compiler/layouts.py:90-106) with fp32 128x128 block scales,
// activations with fp32 1x128 scales, the shared expert stored as expert 256
// of 257. Numerics follow this build's layer contract: the router and
// shared-gate logits use its fixed fp32 dot-product order, the SiLU its
// contract exp, so those outputs are bit-exact against the CPU oracle; the
// GEMM outputs are checked against it within a tolerance.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ---- router logits (replaces runtime/gfx950/routing/verify/qwen36_router_bf16_bridge.h:10-21)
// output_logits_bf16 [rows, 256] = bf16(hidden_bf16 [rows, 2048] . router_weight_bf16 [256, 2048]^T).
// rows must be 1 or 16, as in the reference.
int netra_qwen36_router_bf16_load(const char* hsaco_path);
int netra_qwen36_router_bf16_launch(void* output_logits_bf16, const void* hidden_bf16,
                                    const void* router_weight_bf16, uint32_t rows, hipStream_t stream);
int netra_qwen36_router_bf16_unload(void);
const char* netra_qwen36_router_bf16_last_error(void);

// ---- shared-expert gate + append (replaces runtime/gfx950/routing/decode/
// qwen36_shared_gate_append_bridge.h:10-24). Slots 0..7 copy routed_ids_i32 /
// routed_weights_f32 [rows, 8]; slot 8 holds expert 256 with weight
// f32(bf16(sigmoid(bf16(hidden . shared_gate_weight)))). Outputs [rows, 9].
// rows must be 1 or 16, as in the reference.
int netra_qwen36_shared_gate_append_load(const char* hsaco_path);
int netra_qwen36_shared_gate_append_launch(void* output_ids_i32, void* output_weights_f32,
                                           const void* hidden_bf16, const void* shared_gate_weight_bf16,
                                           const void* routed_ids_i32, const void* routed_weights_f32,
                                           uint32_t rows, hipStream_t stream);
int netra_qwen36_shared_gate_append_unload(void);
const char* netra_qwen36_shared_gate_append_last_error(void);

// ---- decode trio (replaces runtime/gfx950/fp8/moe/qwen36_moe_silu_mul_quant_bridge.h:14-64).
// Routes are token-major, r = t * 9 + slot, experts from topk_ids_i32 [rows, 9].
//
// SiLU.mul + 1x128 FP8 quant: input_f32 [rows, 1024] (gate 0..511, up
// 512..1023) -> output_fp8 [rows, 512] + output_scale_f32 [rows, 4]; here
// `rows` counts route rows.
int netra_qwen36_moe_silu_mul_quant_load(const char* hsaco_path);
int netra_qwen36_moe_silu_mul_quant_launch(const float* input_f32, void* output_fp8, float* output_scale_f32,
                                           int rows, hipStream_t stream);
int netra_qwen36_moe_silu_mul_quant_unload(void);
const char* netra_qwen36_moe_silu_mul_quant_last_error(void);

// Down projection + top-9 weighted reduce: activation_fp8 [rows * 9, 512] +
// activation_scale_f32 [rows * 9, 4], w2_fp8 [257, 2048, 512] (AITER) +
// w2_scale_f32 [257, 16, 4], topk_weights_f32 / topk_ids_i32 [rows, 9] ->
// output_bf16 [rows, 2048]. Any rows >= 1.
int netra_qwen36_moe_down_reduce_load(const char* hsaco_path);
int netra_qwen36_moe_down_reduce_launch(const void* activation_fp8, const float* activation_scale_f32,
                                        const void* w2_fp8, const float* w2_scale_f32,
                                        const float* topk_weights_f32, const int32_t* topk_ids_i32,
                                        void* output_bf16, int rows, hipStream_t stream);
int netra_qwen36_moe_down_reduce_unload(void);
const char* netra_qwen36_moe_down_reduce_last_error(void);

// Gate/up: hidden_fp8 [rows, 2048] + hidden_scale_f32 [rows, 16], w13_fp8
// [257, 1024, 2048] (AITER; rows 0..511 gate, 512..1023 up) + w13_scale_f32
// [257, 8, 16], topk_ids_i32 [rows, 9] -> output_f32 [rows * 9, 1024]
// (gate then up, before SiLU). Any rows >= 1.
int netra_qwen36_moe_gate_up_load(const char* hsaco_path);
int netra_qwen36_moe_gate_up_launch(const void* hidden_fp8, const float* hidden_scale_f32, const void* w13_fp8,
                                    const float* w13_scale_f32, const int32_t* topk_ids_i32, float* output_f32,
                                    int rows, hipStream_t stream);
int netra_qwen36_moe_gate_up_unload(void);
const char* netra_qwen36_moe_gate_up_last_error(void);

// ---- M768 prefill producer/reducer (replaces runtime/gfx950/fp8/moe/moe_prefill_m768_bridge.h:10-23).
// 768 tokens x 9 routes in the AITER sorted format: sorted_token_ids_i32
// [23360] ((slot << 24) | token, 64-row expert blocks, an expert's blocks
// consecutive with its valid rows before its padding), sorted_expert_ids_i32
// [365], num_valid_ids_i32 [1] (padded rows); sorted_weights_f32 is unused
// (as in the reference). Writes route_scale_workspace_f32 [23360, 4] (the h
// scales), partials_f16 [2, 7277, 2048] (split-K2 halves, route rows
// t * 9 + slot) and output_bf16 [768, 2048] = bf16(sum over slots in order of
// topk_weights_f32 [768, 9] * (half 0 + half 1)). Both paths may name the
// same code object. load() also allocates the launch's 12 MB of scratch.
int netra_moe_prefill_m768_load(const char* producer_hsaco, const char* reducer_hsaco);
int netra_moe_prefill_m768_launch(const void* hidden_fp8, const float* hidden_scale_f32, const void* w13_fp8,
                                  const float* w13_scale_f32, const void* w2_fp8, const float* w2_scale_f32,
                                  const int32_t* sorted_token_ids_i32, const float* sorted_weights_f32,
                                  const int32_t* sorted_expert_ids_i32, const int32_t* num_valid_ids_i32,
                                  const float* topk_weights_f32, float* route_scale_workspace_f32,
                                  void* partials_f16, void* output_bf16, hipStream_t stream);
int netra_moe_prefill_m768_unload(void);
const char* netra_moe_prefill_m768_last_error(void);

#ifdef __cplusplus
}
#endif
