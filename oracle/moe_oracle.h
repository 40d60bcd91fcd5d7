/*
 * CPU oracle for the FP8 E4M3 block-scaled routed-MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is
 * compared against; only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may load it. The product path never calls into it.
 *
 * Every function restates the reference's algorithm for one step of the path.
 * Reference files are cited relative to the reference repository root.
 */
#ifndef NETRA_MOE_ORACLE_H
#define NETRA_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar numerics -------------------------------------------------- */
uint16_t orc_bf16_from_f32(float x);             /* round-to-nearest-even */
float orc_f32_from_bf16(uint16_t b);
uint8_t orc_e4m3_from_f32(float x);              /* OCP e4m3fn, RNE, saturating */
float orc_f32_from_e4m3(uint8_t q);
float orc_exp(float x);                          /* contract exp (see .c) */
float orc_silu(float g);
float orc_sigmoid(float z);

/* ---- quantisation (a5, a7, weight prep) -------------------------------- */
/* x bf16 [rows, cols] -> q e4m3 [rows, cols] + s f32 [rows, cols/128]. */
void orc_quant_rows_bf16(const uint16_t* x, int64_t rows, int64_t cols,
                         uint8_t* q, float* s);
/* w f32 [groups, n, k] -> q e4m3 [groups, n, k] + s f32 [groups, n/128, k/128]. */
void orc_quant_blocks_f32(const float* w, int64_t groups, int64_t n, int64_t k,
                          uint8_t* q, float* s, int threads);

/* ---- router (a1) ------------------------------------------------------- */
/* logits bf16 [T, rows] = x bf16 [T, H] . w bf16 [rows, H]^T in the contract order. */
void orc_router_logits(const uint16_t* x, const uint16_t* w, int64_t T, int64_t H,
                       int64_t rows, uint16_t* logits, int threads);

/* ---- top-k, renormalised softmax, shared-expert append (a2, a3) --------- */
/* logits bf16 [T, E + S] (column E holds the shared-gate logit when S == 1);
 * bias f32 [E] or NULL.  ids int32 [T, K + S], weights f32 [T, K + S]. */
void orc_topk(const uint16_t* logits, const float* bias, int64_t T, int64_t E,
              int64_t K, int64_t S, int32_t* ids, float* weights);

/* ---- count / sort / pad (a4) ------------------------------------------- */
int64_t orc_capacity_blocks(int64_t T, int64_t Ktot, int64_t Etot, int64_t BM);
/* Returns the number of padded rows (num_valid_ids[0]) or -1 on bad input.
 * tile_map (may be NULL) lists non-empty 16-row tiles as block * 4 + tile;
 * pair_map (may be NULL) lists each expert's blocks two at a time by the
 * first block of the two; num_valid = {padded rows, routes, tiles, pairs}. */
int64_t orc_sort(const int32_t* ids, int64_t T, int64_t Ktot, int64_t Etot,
                 int64_t BM, int64_t cap_blocks, int32_t* sorted_ids,
                 int32_t* sorted_expert, int32_t* tile_map, int32_t* pair_map,
                 int32_t* num_valid, int32_t* counts);

/* ---- grouped GEMMs (a6 + a7, a8) ---------------------------------------- */
/* Gate/up + SiLU.mul + 1x128 requant over sorted rows.
 * h_q e4m3 [cap_blocks*BM, I], h_s f32 [cap_blocks*BM, I/128]; pad rows are zero.
 * Optionally returns h bf16 [cap_blocks*BM, I] (NULL to skip). */
void orc_gate_up(const uint8_t* x_q, const float* x_s, const uint8_t* w13,
                 const float* w13_s, const int32_t* sorted_ids,
                 const int32_t* sorted_expert, int64_t num_valid_rows,
                 int64_t T, int64_t H, int64_t I, int64_t BM, uint8_t* h_q,
                 float* h_s, uint16_t* h_bf16, int threads);
/* Down GEMM per route, then top-k weighted combine.
 * partial f32 [T*Ktot, H] (may be NULL), out_f32 [T, H] (may be NULL), out bf16 [T, H]. */
void orc_down_combine(const uint8_t* h_q, const float* h_s, const uint8_t* w2,
                      const float* w2_s, const int32_t* sorted_ids,
                      const int32_t* sorted_expert, int64_t num_valid_rows,
                      const float* weights, int64_t T, int64_t H, int64_t I,
                      int64_t Ktot, int64_t BM, float* partial, float* out_f32,
                      uint16_t* out, int threads);

/* Token-major whole expert path for a token list (sampled checks, CPU baseline).
 * ids/weights [T, Ktot]; tokens int64 [n]; out_f32/out [n, H]. */
void orc_moe_tokens(const uint8_t* x_q, const float* x_s, const uint8_t* w13,
                    const float* w13_s, const uint8_t* w2, const float* w2_s,
                    const int32_t* ids, const float* weights, const int64_t* tokens,
                    int64_t n_tokens, int64_t H, int64_t I, int64_t Ktot,
                    float* out_f32, uint16_t* out, int threads);

/* ---- per-operation bridge contracts ------------------------------------ */
/* Stage 1 per route, before SiLU (export_qwen36_moe_stage1_capture.py:80-97):
 * out f32 [T*Ktot, 2I], route r = t*Ktot + s with expert ids[r]; rows with an
 * expert id outside [0, Etot) are zero. */
void orc_stage1_routes(const uint8_t* x_q, const float* x_s, const uint8_t* w13,
                       const float* w13_s, const int32_t* ids, int64_t T, int64_t Ktot,
                       int64_t Etot, int64_t H, int64_t I, float* out, int threads);
/* SiLU.mul + 1x128 quant of fp32 rows [g | u] (qwen36_moe_silu_mul_quant_fp8_gfx950.hip:41-94):
 * q e4m3 [rows, I], s f32 [rows, I/128]. */
void orc_silu_mul_quant(const float* in, int64_t rows, int64_t I, uint8_t* q, float* s);
/* Down per route + slot-ordered weighted reduce per token
 * (export_qwen36_moe_stage2_capture.py:90-110,151-155): h rows are route-major
 * [T*Ktot, I]; out_f32 [T, H] (may be NULL), out bf16 [T, H]. */
void orc_down_reduce_routes(const uint8_t* h_q, const float* h_s, const uint8_t* w2,
                            const float* w2_s, const int32_t* ids, const float* weights,
                            int64_t T, int64_t Ktot, int64_t Etot, int64_t H, int64_t I,
                            float* out_f32, uint16_t* out, int threads);

#ifdef __cplusplus
}
#endif
#endif
