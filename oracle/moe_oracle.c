/*
 * CPU oracle for the FP8 E4M3 block-scaled routed-MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path. Only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py load it.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off). Contraction is
 * off so that every fused multiply-add below is an explicit fmaf() and every
 * other product/sum rounds on its own, exactly as the HIP kernels do.
 *
 * Sources restated (paths relative to the reference repository root):
 *   - GEMM stage 1 (gate/up), per-128-K dequantised accumulation:
 *       tools/benchmark/export_qwen36_moe_stage1_capture.py:80-97
 *   - GEMM stage 2 (down) and the top-k-slot-ordered weighted combine:
 *       tools/benchmark/export_qwen36_moe_stage2_capture.py:90-110,151-155
 *   - SiLU.mul + 1x128 FP8 requant (amax floor 1e-10, scale = amax * 0x3b124925,
 *       q = e4m3(v * (1/scale))):
 *       harness/gfx950/fp8/moe/decode/qwen36_moe_silu_mul_quant_fp8_gfx950.hip:35-94
 *   - scale application order (mfma * a_s) * w_s, added per K block:
 *       kernels/gfx950/templates/common/mfma.inc:20-24
 *   - router logits = bf16(linear(x_bf16, W_bf16)) with fp32 accumulation:
 *       tools/benchmark/export_qwen36_router_bf16_capture.py:78
 *   - shared expert weight = bf16(sigmoid(bf16(x . w_sg))), id 256 appended:
 *       tools/benchmark/export_qwen36_shared_gate_append_capture.py:97-107,134-139
 *   - sorted-id wire format (slot << 24) | token, 64-row expert blocks, padding
 *       entries have token >= T or slot >= Ktot:
 *       kernels/gfx950/templates/moe/prefill/fused_splitk2/entry_routing.inc:27-112
 *   - capacity = ceil(routes / 64) + experts blocks (365 blocks for 768 x 9 routes
 *       over 257 experts): manifests/gfx950/models/qwen36-35b-c64-fp8.json:43-49
 *
 * Where the reference leaves the arithmetic to an external library (SGLang
 * fused_topk, AITER moe_sorting and input quant) this file states the build's
 * own contract; the comments at each function say which parts that covers.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* 1/448 rounded to fp32 (bit pattern 0x3b124925), the reference's quant constant. */
#define ORC_INV_E4M3_MAX u2f(0x3b124925u)
#define ORC_AMAX_FLOOR 1.0e-10f

/* ---------------------------------------------------------------------- */
uint16_t orc_bf16_from_f32(float x) {
  uint32_t u = f2u(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_f32_from_bf16(uint16_t b) { return u2f((uint32_t)b << 16); }

/* OCP E4M3 (e4m3fn): bias 7, 3 mantissa bits, max finite 448 (0x7e), 0x7f NaN,
 * subnormals m * 2^-9.  Round to nearest even; magnitudes >= 448 saturate. */
uint8_t orc_e4m3_from_f32(float x) {
  const uint32_t u = f2u(x);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);
  const float fa = u2f(a);
  if (fa >= 448.0f) return (uint8_t)(sign | 0x7eu);
  if (fa < 0.015625f) {                       /* below 2^-6: subnormal grid 2^-9 */
    const float m = rintf(fa * 512.0f);       /* exact scaling, RNE to integer */
    return (uint8_t)(sign | (uint8_t)m);      /* m == 8 encodes the min normal */
  }
  const uint32_t e = (a >> 23) - 127u + 7u;   /* biased e4m3 exponent, 1..15 */
  const uint32_t mant = a & 0x7fffffu;
  const uint32_t rounded = mant + 0x7ffffu + ((mant >> 20) & 1u);
  uint32_t code = (e << 3) + (rounded >> 20); /* mantissa carry bumps exponent */
  if (code > 0x7eu) code = 0x7eu;
  return (uint8_t)(sign | code);
}

float orc_f32_from_e4m3(uint8_t q) {
  const uint32_t e = (q >> 3) & 15u, m = q & 7u;
  float v;
  if (e == 15u && m == 7u) return u2f(0x7fc00000u);
  if (e == 0u) v = (float)m * (1.0f / 512.0f);
  else v = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
  return (q & 0x80u) ? -v : v;
}

/* Contract exp: Cody-Waite reduction x = n ln2 + r with n = rint(x log2 e),
 * ln2 split hi/lo as fdlibm's single-precision expf splits it (0x3f317200 +
 * 0x35bfbe8e), then the degree-7 Taylor polynomial of e^r in Horner form
 * with explicit fmaf, scaled by 2^n through the exponent field. x < -87 -> 0,
 * x > 88 -> +inf (no subnormal results). The HIP kernels evaluate the same
 * operation sequence, so both sides produce identical bits. */
float orc_exp(float x) {
  if (x != x) return x;
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) return u2f(0x7f800000u);
  const float n = rintf(x * 1.44269502162933349609375f);      /* 0x3fb8aa3b */
  float r = fmaf(-n, 0.693145751953125f, x);                   /* 0x3f317200 */
  r = fmaf(-n, 1.428606765330187045037746429443359375e-06f, r); /* 0x35bfbe8e */
  float p = 1.98412701138295233249664306640625e-04f;           /* 1/5040 */
  p = fmaf(p, r, 1.388888922519981861114501953125e-03f);        /* 1/720 */
  p = fmaf(p, r, 8.333333767950534820556640625e-03f);           /* 1/120 */
  p = fmaf(p, r, 4.1666667163372039794921875e-02f);             /* 1/24 */
  p = fmaf(p, r, 1.6666667163372039794921875e-01f);             /* 1/6 */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  return p * u2f((uint32_t)(ni + 127) << 23);
}

float orc_silu(float g) { return g / (1.0f + orc_exp(-g)); }
float orc_sigmoid(float z) { return 1.0f / (1.0f + orc_exp(-z)); }

/* ---------------------------------------------------------------------- */
/* 1x128 group quantisation of one row of fp32 values (already bf16-exact). */
static void quant_row_f32(const float* v, int64_t cols, uint8_t* q, float* s) {
  for (int64_t g = 0; g < cols / 128; ++g) {
    float amax = ORC_AMAX_FLOOR;
    for (int64_t i = 0; i < 128; ++i) amax = fmaxf(amax, fabsf(v[g * 128 + i]));
    const float scale = amax * ORC_INV_E4M3_MAX;
    const float inv = 1.0f / scale;
    s[g] = scale;
    for (int64_t i = 0; i < 128; ++i) q[g * 128 + i] = orc_e4m3_from_f32(v[g * 128 + i] * inv);
  }
}

void orc_quant_rows_bf16(const uint16_t* x, int64_t rows, int64_t cols, uint8_t* q,
                         float* s) {
  float* tmp = (float*)malloc(sizeof(float) * (size_t)cols);
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) tmp[c] = orc_f32_from_bf16(x[r * cols + c]);
    quant_row_f32(tmp, cols, q + r * cols, s + r * (cols / 128));
  }
  free(tmp);
}

/* 128x128 block quantisation of fp32 weights [groups, n, k]; same scale rule. */
void orc_quant_blocks_f32(const float* w, int64_t groups, int64_t n, int64_t k,
                          uint8_t* q, float* s, int threads) {
  const int64_t nb = n / 128, kb = k / 128, blocks = groups * nb * kb;
  (void)threads;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t b = 0; b < blocks; ++b) {
    const int64_t gi = b / (nb * kb), bn = (b / kb) % nb, bk = b % kb;
    const float* base = w + (gi * n + bn * 128) * k + bk * 128;
    uint8_t* qb = q + (gi * n + bn * 128) * k + bk * 128;
    float amax = ORC_AMAX_FLOOR;
    for (int64_t i = 0; i < 128; ++i)
      for (int64_t j = 0; j < 128; ++j) amax = fmaxf(amax, fabsf(base[i * k + j]));
    const float scale = amax * ORC_INV_E4M3_MAX;
    const float inv = 1.0f / scale;
    s[b] = scale;
    for (int64_t i = 0; i < 128; ++i)
      for (int64_t j = 0; j < 128; ++j) qb[i * k + j] = orc_e4m3_from_f32(base[i * k + j] * inv);
  }
}

/* ---------------------------------------------------------------------- */
/* Router dot product in the build's fixed order (the reference fixes its own
 * order in kernels/gfx950/templates/routing/bf16_gemv.inc:45-79: per-lane
 * strided partial sums then a DPP tree).  Here: 16 slices; slice s holds the
 * elements 128*j + 8*s + i (j over K blocks, i in 0..7), accumulated with fmaf
 * from +0 in (j, i) order; the 16 partials are folded by the tree
 * p[s] += p[s+8], p[s] += p[s+4], p[s] += p[s+2], p[0] += p[1]. */
static float router_dot(const uint16_t* x, const uint16_t* w, int64_t H) {
  float p[16];
  for (int s = 0; s < 16; ++s) {
    float acc = 0.0f;
    for (int64_t j = 0; j < H / 128; ++j)
      for (int i = 0; i < 8; ++i) {
        const int64_t k = 128 * j + 8 * s + i;
        acc = fmaf(orc_f32_from_bf16(x[k]), orc_f32_from_bf16(w[k]), acc);
      }
    p[s] = acc;
  }
  for (int s = 0; s < 8; ++s) p[s] = p[s] + p[s + 8];
  for (int s = 0; s < 4; ++s) p[s] = p[s] + p[s + 4];
  for (int s = 0; s < 2; ++s) p[s] = p[s] + p[s + 2];
  return p[0] + p[1];
}

void orc_router_logits(const uint16_t* x, const uint16_t* w, int64_t T, int64_t H,
                       int64_t rows, uint16_t* logits, int threads) {
  (void)threads;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t t = 0; t < T; ++t)
    for (int64_t r = 0; r < rows; ++r)
      logits[t * rows + r] = orc_bf16_from_f32(router_dot(x + t * H, w + r * H, H));
}

/* ---------------------------------------------------------------------- */
/* Top-k on z_e = f32(logit_e) (+ bias_e), ties to the lower expert index,
 * slots in descending z; weights = softmax over the k selected z (the same as
 * softmax-then-renormalise of SGLang fused_topk, computed with the contract
 * exp and a slot-ordered fp32 sum).  With S == 1 the shared expert (id E) is
 * appended at slot K with weight f32(bf16(sigmoid(f32(logit_E)))). */
void orc_topk(const uint16_t* logits, const float* bias, int64_t T, int64_t E,
              int64_t K, int64_t S, int32_t* ids, float* weights) {
  const int64_t rows = E + S, Ktot = K + S;
  float* z = (float*)malloc(sizeof(float) * (size_t)E);
  unsigned char* taken = (unsigned char*)malloc((size_t)E);
  for (int64_t t = 0; t < T; ++t) {
    const uint16_t* l = logits + t * rows;
    for (int64_t e = 0; e < E; ++e) {
      z[e] = orc_f32_from_bf16(l[e]);
      if (bias) z[e] = z[e] + bias[e];
      taken[e] = 0;
    }
    int32_t sel[64];
    for (int64_t s = 0; s < K; ++s) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || z[e] > z[best]) best = e;
      }
      taken[best] = 1;
      sel[s] = (int32_t)best;
    }
    float ex[64], sum = 0.0f;
    const float m = z[sel[0]];
    for (int64_t s = 0; s < K; ++s) { ex[s] = orc_exp(z[sel[s]] - m); sum = sum + ex[s]; }
    for (int64_t s = 0; s < K; ++s) {
      ids[t * Ktot + s] = sel[s];
      weights[t * Ktot + s] = ex[s] / sum;
    }
    if (S) {
      const float sig = orc_sigmoid(orc_f32_from_bf16(l[E]));
      ids[t * Ktot + K] = (int32_t)E;
      weights[t * Ktot + K] = orc_f32_from_bf16(orc_bf16_from_f32(sig));
    }
  }
  free(z);
  free(taken);
}

/* ---------------------------------------------------------------------- */
int64_t orc_capacity_blocks(int64_t T, int64_t Ktot, int64_t Etot, int64_t BM) {
  return (T * Ktot + BM - 1) / BM + Etot;
}

/* Count -> exclusive scan of per-expert padded block counts -> scatter in
 * (expert, token) order.  Pads fill every unused row with (Ktot << 24) | T;
 * unused expert-block entries are -1.  The non-empty 16-row tiles are listed
 * expert by expert as block * 4 + tile-in-block (tile_map, capacity
 * ceil(routes / 16) + Etot, may be NULL), and each expert's blocks two at a
 * time by the first of the two (pair_map, capacity cap_blocks, may be NULL;
 * an expert's last block stands alone when its block count is odd).
 * num_valid = {padded rows, routes, tiles, pairs}. */
int64_t orc_sort(const int32_t* ids, int64_t T, int64_t Ktot, int64_t Etot, int64_t BM,
                 int64_t cap_blocks, int32_t* sorted_ids, int32_t* sorted_expert,
                 int32_t* tile_map, int32_t* pair_map, int32_t* num_valid, int32_t* counts) {
  int64_t* off = (int64_t*)calloc((size_t)Etot, sizeof(int64_t));
  int64_t* cur = (int64_t*)calloc((size_t)Etot, sizeof(int64_t));
  for (int64_t e = 0; e < Etot; ++e) counts[e] = 0;
  for (int64_t r = 0; r < T * Ktot; ++r) {
    if (ids[r] < 0 || ids[r] >= Etot) { free(off); free(cur); return -1; }
    counts[ids[r]]++;
  }
  int64_t blocks = 0;
  for (int64_t e = 0; e < Etot; ++e) { off[e] = blocks; blocks += (counts[e] + BM - 1) / BM; }
  if (blocks > cap_blocks) { free(off); free(cur); return -1; }
  const int32_t pad = (int32_t)((Ktot << 24) | T);
  for (int64_t p = 0; p < cap_blocks * BM; ++p) sorted_ids[p] = pad;
  for (int64_t b = 0; b < cap_blocks; ++b) sorted_expert[b] = -1;
  for (int64_t e = 0; e < Etot; ++e)
    for (int64_t j = 0; j < (counts[e] + BM - 1) / BM; ++j) sorted_expert[off[e] + j] = (int32_t)e;
  for (int64_t t = 0; t < T; ++t)
    for (int64_t s = 0; s < Ktot; ++s) {
      const int32_t e = ids[t * Ktot + s];
      sorted_ids[off[e] * BM + cur[e]++] = (int32_t)((s << 24) | t);
    }
  int64_t tiles = 0;
  for (int64_t e = 0; e < Etot; ++e)
    for (int64_t j = 0; j < (counts[e] + 15) / 16; ++j) {
      if (tile_map) tile_map[tiles] = (int32_t)(off[e] * (BM / 16) + j);
      ++tiles;
    }
  int64_t pairs = 0;
  for (int64_t e = 0; e < Etot; ++e)
    for (int64_t j = 0; j < (counts[e] + BM - 1) / BM; j += 2) {
      if (pair_map) pair_map[pairs] = (int32_t)(off[e] + j);
      ++pairs;
    }
  num_valid[0] = (int32_t)(blocks * BM);
  num_valid[1] = (int32_t)(T * Ktot);
  num_valid[2] = (int32_t)tiles;
  num_valid[3] = (int32_t)pairs;
  free(off);
  free(cur);
  return blocks * BM;
}

/* ---------------------------------------------------------------------- */
static float g_e4m3_table[256];
static int g_table_ready = 0;
static void ensure_table(void) {
  if (g_table_ready) return;
  for (int i = 0; i < 256; ++i) g_e4m3_table[i] = orc_f32_from_e4m3((uint8_t)i);
  g_table_ready = 1;
}

/* One output element of a block-scaled FP8 GEMM row:
 * sum over K blocks of ((sum_k a8*w8) * a_s) * w_s. The inner 128-term sum of
 * e4m3 products is exact in double; the scale products follow mfma.inc:20-24. */
static double fp8_row_dot(const uint8_t* a, const float* a_s, const uint8_t* w,
                          const float* w_s_row, int64_t K) {
  double acc = 0.0;
  for (int64_t kb = 0; kb < K / 128; ++kb) {
    double dot = 0.0;
    for (int64_t i = 0; i < 128; ++i)
      dot += (double)g_e4m3_table[a[kb * 128 + i]] * (double)g_e4m3_table[w[kb * 128 + i]];
    acc += (dot * (double)a_s[kb]) * (double)w_s_row[kb];
  }
  return acc;
}

/* Stage 1 for one route: gate/up (rows 0..I-1 gate, I..2I-1 up of W13[e]),
 * then h = bf16(silu(g) * u) and 1x128 requant of h. */
static void route_stage1(const uint8_t* xq, const float* xs, const uint8_t* w13e,
                         const float* w13se, int64_t H, int64_t I, uint8_t* hq,
                         float* hs, uint16_t* hb, float* scratch) {
  const int64_t kb = H / 128;
  for (int64_t n = 0; n < I; ++n) {
    const float g = (float)fp8_row_dot(xq, xs, w13e + n * H, w13se + (n / 128) * kb, H);
    const float u = (float)fp8_row_dot(xq, xs, w13e + (I + n) * H,
                                       w13se + ((I + n) / 128) * kb, H);
    const uint16_t h = orc_bf16_from_f32(orc_silu(g) * u);
    if (hb) hb[n] = h;
    scratch[n] = orc_f32_from_bf16(h);
  }
  quant_row_f32(scratch, I, hq, hs);
}

void orc_gate_up(const uint8_t* x_q, const float* x_s, const uint8_t* w13,
                 const float* w13_s, const int32_t* sorted_ids,
                 const int32_t* sorted_expert, int64_t num_valid_rows, int64_t T,
                 int64_t H, int64_t I, int64_t BM, uint8_t* h_q, float* h_s,
                 uint16_t* h_bf16, int threads) {
  ensure_table();
  (void)threads;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    float* scratch = (float*)malloc(sizeof(float) * (size_t)I);
#pragma omp for schedule(dynamic, 4)
    for (int64_t p = 0; p < num_valid_rows; ++p) {
      const int32_t id = sorted_ids[p];
      const int64_t t = id & 0xffffff, s = (uint32_t)id >> 24;
      uint8_t* hq = h_q + p * I;
      float* hs = h_s + p * (I / 128);
      uint16_t* hb = h_bf16 ? h_bf16 + p * I : NULL;
      (void)s;
      if (t >= T) {
        memset(hq, 0, (size_t)I);
        memset(hs, 0, sizeof(float) * (size_t)(I / 128));
        if (hb) memset(hb, 0, 2 * (size_t)I);
        continue;
      }
      const int64_t e = sorted_expert[p / BM];
      route_stage1(x_q + t * H, x_s + t * (H / 128), w13 + e * 2 * I * H,
                   w13_s + e * (2 * I / 128) * (H / 128), H, I, hq, hs, hb, scratch);
    }
    free(scratch);
  }
}

/* Stage 2 for one route row: partial[n] = sum_kb ((sum_k h8*w8) * h_s) * w_s. */
static void route_stage2(const uint8_t* hq, const float* hs, const uint8_t* w2e,
                         const float* w2se, int64_t H, int64_t I, double* out) {
  for (int64_t n = 0; n < H; ++n)
    out[n] = fp8_row_dot(hq, hs, w2e + n * I, w2se + (n / 128) * (I / 128), I);
}

void orc_down_combine(const uint8_t* h_q, const float* h_s, const uint8_t* w2,
                      const float* w2_s, const int32_t* sorted_ids,
                      const int32_t* sorted_expert, int64_t num_valid_rows,
                      const float* weights, int64_t T, int64_t H, int64_t I,
                      int64_t Ktot, int64_t BM, float* partial, float* out_f32,
                      uint16_t* out, int threads) {
  ensure_table();
  double* part = (double*)calloc((size_t)(T * Ktot * H), sizeof(double));
  (void)threads;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(dynamic, 4)
  for (int64_t p = 0; p < num_valid_rows; ++p) {
    const int32_t id = sorted_ids[p];
    const int64_t t = id & 0xffffff, s = (uint32_t)id >> 24;
    if (t >= T || s >= Ktot) continue;
    const int64_t e = sorted_expert[p / BM];
    route_stage2(h_q + p * I, h_s + p * (I / 128), w2 + e * H * I,
                 w2_s + e * (H / 128) * (I / 128), H, I, part + (t * Ktot + s) * H);
  }
  if (partial)
    for (int64_t i = 0; i < T * Ktot * H; ++i) partial[i] = (float)part[i];
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t t = 0; t < T; ++t)
    for (int64_t n = 0; n < H; ++n) {
      double acc = 0.0;
      for (int64_t s = 0; s < Ktot; ++s)
        acc += part[(t * Ktot + s) * H + n] * (double)weights[t * Ktot + s];
      if (out_f32) out_f32[t * H + n] = (float)acc;
      out[t * H + n] = orc_bf16_from_f32((float)acc);
    }
  free(part);
}

/* Token-major restatement of the whole expert path for a list of tokens (the
 * shape of the reference's stage1/stage2 oracles, which iterate slots of one
 * token): for each slot, stage 1, requant, stage 2, then the slot-ordered
 * weighted sum.  Used for sampled checks at large T and as the CPU baseline. */
void orc_moe_tokens(const uint8_t* x_q, const float* x_s, const uint8_t* w13,
                    const float* w13_s, const uint8_t* w2, const float* w2_s,
                    const int32_t* ids, const float* weights, const int64_t* tokens,
                    int64_t n_tokens, int64_t H, int64_t I, int64_t Ktot,
                    float* out_f32, uint16_t* out, int threads) {
  ensure_table();
  (void)threads;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    uint8_t* hq = (uint8_t*)malloc((size_t)I);
    float* hs = (float*)malloc(sizeof(float) * (size_t)(I / 128));
    float* scratch = (float*)malloc(sizeof(float) * (size_t)I);
    double* part = (double*)malloc(sizeof(double) * (size_t)H);
    double* acc = (double*)malloc(sizeof(double) * (size_t)H);
#pragma omp for schedule(dynamic, 1)
    for (int64_t j = 0; j < n_tokens; ++j) {
      const int64_t t = tokens[j];
      for (int64_t n = 0; n < H; ++n) acc[n] = 0.0;
      for (int64_t s = 0; s < Ktot; ++s) {
        const int64_t e = ids[t * Ktot + s];
        route_stage1(x_q + t * H, x_s + t * (H / 128), w13 + e * 2 * I * H,
                     w13_s + e * (2 * I / 128) * (H / 128), H, I, hq, hs, NULL, scratch);
        route_stage2(hq, hs, w2 + e * H * I, w2_s + e * (H / 128) * (I / 128), H, I, part);
        for (int64_t n = 0; n < H; ++n) acc[n] += part[n] * (double)weights[t * Ktot + s];
      }
      for (int64_t n = 0; n < H; ++n) {
        if (out_f32) out_f32[j * H + n] = (float)acc[n];
        out[j * H + n] = orc_bf16_from_f32((float)acc[n]);
      }
    }
    free(hq); free(hs); free(scratch); free(part); free(acc);
  }
}

/* ---------------------------------------------------------------------- */
/* Per-operation bridge contracts (runtime/gfx950/fp8/moe/
 * qwen36_moe_silu_mul_quant_bridge.h:14-64). */

void orc_stage1_routes(const uint8_t* x_q, const float* x_s, const uint8_t* w13,
                       const float* w13_s, const int32_t* ids, int64_t T, int64_t Ktot,
                       int64_t Etot, int64_t H, int64_t I, float* out, int threads) {
  ensure_table();
  (void)threads;
  const int64_t kb = H / 128;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(dynamic, 1)
  for (int64_t r = 0; r < T * Ktot; ++r) {
    const int64_t t = r / Ktot, e = ids[r];
    float* o = out + r * 2 * I;
    if (e < 0 || e >= Etot) {
      memset(o, 0, sizeof(float) * (size_t)(2 * I));
      continue;
    }
    const uint8_t* w13e = w13 + e * 2 * I * H;
    const float* w13se = w13_s + e * (2 * I / 128) * kb;
    for (int64_t n = 0; n < 2 * I; ++n)
      o[n] = (float)fp8_row_dot(x_q + t * H, x_s + t * kb, w13e + n * H, w13se + (n / 128) * kb, H);
  }
}

void orc_silu_mul_quant(const float* in, int64_t rows, int64_t I, uint8_t* q, float* s) {
  float* h = (float*)malloc(sizeof(float) * (size_t)I);
  for (int64_t r = 0; r < rows; ++r) {
    const float* g = in + r * 2 * I;
    const float* u = g + I;
    for (int64_t n = 0; n < I; ++n) h[n] = orc_f32_from_bf16(orc_bf16_from_f32(orc_silu(g[n]) * u[n]));
    quant_row_f32(h, I, q + r * I, s + r * (I / 128));
  }
  free(h);
}

void orc_down_reduce_routes(const uint8_t* h_q, const float* h_s, const uint8_t* w2,
                            const float* w2_s, const int32_t* ids, const float* weights,
                            int64_t T, int64_t Ktot, int64_t Etot, int64_t H, int64_t I,
                            float* out_f32, uint16_t* out, int threads) {
  ensure_table();
  (void)threads;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    double* part = (double*)malloc(sizeof(double) * (size_t)H);
    double* acc = (double*)malloc(sizeof(double) * (size_t)H);
#pragma omp for schedule(dynamic, 1)
    for (int64_t t = 0; t < T; ++t) {
      for (int64_t n = 0; n < H; ++n) acc[n] = 0.0;
      for (int64_t s = 0; s < Ktot; ++s) {
        const int64_t r = t * Ktot + s, e = ids[r];
        if (e < 0 || e >= Etot) continue;
        route_stage2(h_q + r * I, h_s + r * (I / 128), w2 + e * H * I,
                     w2_s + e * (H / 128) * (I / 128), H, I, part);
        for (int64_t n = 0; n < H; ++n) acc[n] += part[n] * (double)weights[r];
      }
      for (int64_t n = 0; n < H; ++n) {
        if (out_f32) out_f32[t * H + n] = (float)acc[n];
        out[t * H + n] = orc_bf16_from_f32((float)acc[n]);
      }
    }
    free(part);
    free(acc);
  }
}
