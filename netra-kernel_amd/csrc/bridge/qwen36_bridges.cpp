// libnetra_bridges.so: the reference's per-operation bridge ABIs
// (include/netra_qwen36_bridges.h) over this build's code object. Host code
// only: module management and dispatch on the caller's stream, as in the
// reference's bridges (runtime/gfx950/fp8/moe/*_bridge.hip,
// runtime/gfx950/routing/*/*_bridge.hip).
//
// Every family is one `Family` record: its kernel symbols, the code object(s)
// it loaded, the resolved functions and (for the prefill pair) its scratch.
// load/unload serialise on the family's mutex; launches read the resolved
// functions without locking, so (as in the reference) a family must not be
// unloaded while launches or graph replays that use it are outstanding.
#include "../../../include/netra_qwen36_bridges.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "prefill_plan.h"

namespace {

constexpr uint32_t kHidden = 2048, kInter = 512, kRouted = 256, kExperts = 257, kRoutedTopk = 8,
                   kTopk = 9;

struct Family {
  const char* what;                  // prefix of this family's messages
  std::vector<const char*> symbols;  // kernels, in launch order
  std::vector<int> module_of;        // index into modules[] for each symbol
  std::mutex mutex;
  hipModule_t modules[2] = {nullptr, nullptr};
  std::string paths[2];
  std::vector<hipFunction_t> functions;
  size_t scratch_bytes = 0;
  void* scratch = nullptr;
};

Family g_router{"router", {"netra_moe_router_h2048_t1_gfx950"}, {0}};
Family g_shared{"shared-gate/append", {"netra_moe_shared_gate_append_h2048_gfx950"}, {0}};
Family g_silu{"silu-mul-quant", {"netra_moe_silu_mul_quant_gfx950"}, {0}};
Family g_down{"down-reduce", {"netra_moe_down_reduce_route_i512_gfx950"}, {0}};
Family g_gate_up{"gate/up", {"netra_moe_gate_up_route_h2048_gfx950"}, {0}};
Family g_prefill{"prefill M768",
                 {netra_prefill::symbol(netra_prefill::kPairs), netra_prefill::symbol(netra_prefill::kGateUp),
                  netra_prefill::symbol(netra_prefill::kDown), netra_prefill::symbol(netra_prefill::kReduce)},
                 {0, 0, 0, 1},
                 {},
                 {nullptr, nullptr},
                 {},
                 {},
                 netra_prefill::scratch_bytes(netra_prefill::kMaxRows)};

// One diagnostic per family and thread (the reference keeps one thread-local
// string per bridge source file).
std::string& error_of(const Family& f) {
  thread_local std::string router, shared, silu, down, gate_up, prefill;
  if (&f == &g_router) return router;
  if (&f == &g_shared) return shared;
  if (&f == &g_silu) return silu;
  if (&f == &g_down) return down;
  if (&f == &g_gate_up) return gate_up;
  return prefill;
}

int refuse(Family& f, const std::string& why) {
  error_of(f) = std::string(f.what) + ": " + why;
  return -1;
}

int hip_error(Family& f, const char* call, hipError_t err) {
  error_of(f) = std::string(f.what) + ": " + call + " failed: " + hipGetErrorString(err);
  return static_cast<int>(err);
}

int ok(Family& f) {
  error_of(f).clear();
  return 0;
}

bool loaded(const Family& f) { return !f.functions.empty() && f.functions.back() != nullptr; }

// Frees the scratch and unloads each distinct module once (both paths may
// name one module); returns the first HIP error.
hipError_t release(Family& f) {
  hipError_t first = hipSuccess;
  if (f.scratch) first = hipFree(f.scratch);
  f.scratch = nullptr;
  const hipModule_t shared = f.modules[1] == f.modules[0] ? f.modules[0] : nullptr;
  for (int m = 0; m < 2; ++m) {
    if (f.modules[m] && !(m == 1 && f.modules[1] == shared)) {
      const hipError_t err = hipModuleUnload(f.modules[m]);
      if (first == hipSuccess) first = err;
    }
    f.modules[m] = nullptr;
    f.paths[m].clear();
  }
  f.functions.clear();
  return first;
}

// Loads the family's code object(s); paths[1] may repeat paths[0] (one module).
int load(Family& f, const char* path0, const char* path1) {
  const char* paths[2] = {path0, path1};
  const int n = path1 ? 2 : 1;
  for (int m = 0; m < n; ++m)
    if (paths[m] == nullptr || paths[m][0] == '\0') return refuse(f, "code-object path must be nonempty");
  std::lock_guard<std::mutex> lock(f.mutex);
  if (loaded(f)) {
    for (int m = 0; m < n; ++m)
      if (f.paths[m] != paths[m]) return refuse(f, "a different code object is loaded; unload it first");
    return ok(f);
  }
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_error(f, "hipGetDevice", err);
  hipDeviceProp_t prop{};
  err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) return hip_error(f, "hipGetDeviceProperties", err);
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return refuse(f, std::string("this code object needs gfx950, the device is ") + prop.gcnArchName);
  for (int m = 0; m < n; ++m) {
    if (m == 1 && std::strcmp(paths[1], paths[0]) == 0) {
      f.modules[1] = f.modules[0];
    } else {
      err = hipModuleLoad(&f.modules[m], paths[m]);
      if (err != hipSuccess) {
        f.modules[m] = nullptr;
        (void)release(f);
        return hip_error(f, "hipModuleLoad", err);
      }
    }
    f.paths[m] = paths[m];
  }
  std::vector<hipFunction_t> functions(f.symbols.size(), nullptr);
  for (size_t i = 0; i < f.symbols.size(); ++i) {
    err = hipModuleGetFunction(&functions[i], f.modules[f.module_of[i]], f.symbols[i]);
    if (err != hipSuccess) {
      (void)release(f);
      return hip_error(f, "hipModuleGetFunction", err);
    }
  }
  if (f.scratch_bytes) {
    err = hipMalloc(&f.scratch, f.scratch_bytes);
    if (err != hipSuccess) {
      f.scratch = nullptr;
      (void)release(f);
      return hip_error(f, "hipMalloc(scratch)", err);
    }
  }
  f.functions = std::move(functions);
  return ok(f);
}

int unload(Family& f) {
  std::lock_guard<std::mutex> lock(f.mutex);
  const hipError_t err = release(f);
  return err == hipSuccess ? ok(f) : hip_error(f, "hipModuleUnload", err);
}

int dispatch(Family& f, size_t kernel, dim3 grid, dim3 block, void** args, hipStream_t stream) {
  const hipError_t err =
      hipModuleLaunchKernel(f.functions[kernel], grid.x, grid.y, grid.z, block.x, block.y, block.z, 0, stream,
                            args, nullptr);
  return err == hipSuccess ? 0 : hip_error(f, "hipModuleLaunchKernel", err);
}

template <size_t N>
bool all_set(const void* const (&pointers)[N]) {
  for (const void* p : pointers)
    if (p == nullptr) return false;
  return true;
}

}  // namespace

// ---- router ------------------------------------------------------------------------------

extern "C" int netra_qwen36_router_bf16_load(const char* hsaco_path) { return load(g_router, hsaco_path, nullptr); }

extern "C" int netra_qwen36_router_bf16_launch(void* output_logits_bf16, const void* hidden_bf16,
                                               const void* router_weight_bf16, uint32_t rows,
                                               hipStream_t stream) {
  Family& f = g_router;
  if (!loaded(f)) return refuse(f, "module is not loaded");
  const void* const ptrs[] = {output_logits_bf16, hidden_bf16, router_weight_bf16};
  if (!all_set(ptrs)) return refuse(f, "launch pointers must be nonnull");
  if (rows != 1 && rows != 16) return refuse(f, "rows must be 1 or 16");
  // netra_moe_router_h2048_t1_gfx950(x, w, logits, xq, xs, mask; T, H, rows, mask_words):
  // null quantisation outputs, no mask
  const void* x = hidden_bf16;
  const void* w = router_weight_bf16;
  void* logits = output_logits_bf16;
  void* none = nullptr;
  uint32_t T = rows, H = kHidden, nrows = kRouted, mask_words = 0;
  void* args[] = {&x, &w, &logits, &none, &none, &none, &T, &H, &nrows, &mask_words};
  const int rc = dispatch(f, 0, dim3((kRouted + 15) / 16, rows), dim3(256), args, stream);
  return rc ? rc : ok(f);
}

extern "C" int netra_qwen36_router_bf16_unload(void) { return unload(g_router); }
extern "C" const char* netra_qwen36_router_bf16_last_error(void) { return error_of(g_router).c_str(); }

// ---- shared-expert gate + append ----------------------------------------------------------

extern "C" int netra_qwen36_shared_gate_append_load(const char* hsaco_path) {
  return load(g_shared, hsaco_path, nullptr);
}

extern "C" int netra_qwen36_shared_gate_append_launch(void* output_ids_i32, void* output_weights_f32,
                                                      const void* hidden_bf16, const void* shared_gate_weight_bf16,
                                                      const void* routed_ids_i32, const void* routed_weights_f32,
                                                      uint32_t rows, hipStream_t stream) {
  Family& f = g_shared;
  if (!loaded(f)) return refuse(f, "module is not loaded");
  const void* const ptrs[] = {output_ids_i32, output_weights_f32, hidden_bf16, shared_gate_weight_bf16,
                              routed_ids_i32, routed_weights_f32};
  if (!all_set(ptrs)) return refuse(f, "launch pointers must be nonnull");
  if (rows != 1 && rows != 16) return refuse(f, "rows must be 1 or 16");
  const void* x = hidden_bf16;
  const void* wsg = shared_gate_weight_bf16;
  const void* ids = routed_ids_i32;
  const void* w = routed_weights_f32;
  uint32_t T = rows, H = kHidden, E = kRouted, K = kRoutedTopk;
  void* args[] = {&output_ids_i32, &output_weights_f32, &x, &wsg, &ids, &w, &T, &H, &E, &K};
  const int rc = dispatch(f, 0, dim3(rows), dim3(64), args, stream);
  return rc ? rc : ok(f);
}

extern "C" int netra_qwen36_shared_gate_append_unload(void) { return unload(g_shared); }
extern "C" const char* netra_qwen36_shared_gate_append_last_error(void) { return error_of(g_shared).c_str(); }

// ---- SiLU.mul + quant ------------------------------------------------------------------------

extern "C" int netra_qwen36_moe_silu_mul_quant_load(const char* hsaco_path) {
  return load(g_silu, hsaco_path, nullptr);
}

extern "C" int netra_qwen36_moe_silu_mul_quant_launch(const float* input_f32, void* output_fp8,
                                                      float* output_scale_f32, int rows, hipStream_t stream) {
  Family& f = g_silu;
  if (!loaded(f)) return refuse(f, "module is not loaded");
  const void* const ptrs[] = {input_f32, output_fp8, output_scale_f32};
  if (!all_set(ptrs)) return refuse(f, "launch pointers must be nonnull");
  if (rows <= 0) return refuse(f, "rows must be positive");
  const float* in = input_f32;
  uint32_t n = static_cast<uint32_t>(rows), I = kInter;
  void* args[] = {&in, &output_fp8, &output_scale_f32, &n, &I};
  const int rc = dispatch(f, 0, dim3(n), dim3(256), args, stream);  // four waves per row
  return rc ? rc : ok(f);
}

extern "C" int netra_qwen36_moe_silu_mul_quant_unload(void) { return unload(g_silu); }
extern "C" const char* netra_qwen36_moe_silu_mul_quant_last_error(void) { return error_of(g_silu).c_str(); }

// ---- down + reduce ---------------------------------------------------------------------------

extern "C" int netra_qwen36_moe_down_reduce_load(const char* hsaco_path) { return load(g_down, hsaco_path, nullptr); }

extern "C" int netra_qwen36_moe_down_reduce_launch(const void* activation_fp8, const float* activation_scale_f32,
                                                   const void* w2_fp8, const float* w2_scale_f32,
                                                   const float* topk_weights_f32, const int32_t* topk_ids_i32,
                                                   void* output_bf16, int rows, hipStream_t stream) {
  Family& f = g_down;
  if (!loaded(f)) return refuse(f, "module is not loaded");
  const void* const ptrs[] = {activation_fp8, activation_scale_f32, w2_fp8, w2_scale_f32,
                              topk_weights_f32, topk_ids_i32, output_bf16};
  if (!all_set(ptrs)) return refuse(f, "launch pointers must be nonnull");
  if (rows <= 0) return refuse(f, "rows must be positive");
  const void* hq = activation_fp8;
  const void* hs = activation_scale_f32;
  const void* w2 = w2_fp8;
  const void* w2s = w2_scale_f32;
  const void* weights = topk_weights_f32;
  const void* ids = topk_ids_i32;
  uint32_t T = static_cast<uint32_t>(rows), H = kHidden, I = kInter, Ktot = kTopk, Etot = kExperts;
  void* args[] = {&hq, &hs, &w2, &w2s, &weights, &ids, &output_bf16, &T, &H, &I, &Ktot, &Etot};
  const int rc = dispatch(f, 0, dim3(kHidden / 16, T), dim3(64 * kTopk), args, stream);
  return rc ? rc : ok(f);
}

extern "C" int netra_qwen36_moe_down_reduce_unload(void) { return unload(g_down); }
extern "C" const char* netra_qwen36_moe_down_reduce_last_error(void) { return error_of(g_down).c_str(); }

// ---- gate/up -----------------------------------------------------------------------------

extern "C" int netra_qwen36_moe_gate_up_load(const char* hsaco_path) { return load(g_gate_up, hsaco_path, nullptr); }

extern "C" int netra_qwen36_moe_gate_up_launch(const void* hidden_fp8, const float* hidden_scale_f32,
                                               const void* w13_fp8, const float* w13_scale_f32,
                                               const int32_t* topk_ids_i32, float* output_f32, int rows,
                                               hipStream_t stream) {
  Family& f = g_gate_up;
  if (!loaded(f)) return refuse(f, "module is not loaded");
  const void* const ptrs[] = {hidden_fp8, hidden_scale_f32, w13_fp8, w13_scale_f32, topk_ids_i32, output_f32};
  if (!all_set(ptrs)) return refuse(f, "launch pointers must be nonnull");
  if (rows <= 0) return refuse(f, "rows must be positive");
  const void* xq = hidden_fp8;
  const void* xs = hidden_scale_f32;
  const void* w13 = w13_fp8;
  const void* w13s = w13_scale_f32;
  const void* ids = topk_ids_i32;
  uint32_t T = static_cast<uint32_t>(rows), H = kHidden, I = kInter, Ktot = kTopk, Etot = kExperts;
  void* args[] = {&xq, &xs, &w13, &w13s, &ids, &output_f32, &T, &H, &I, &Ktot, &Etot};
  const int rc = dispatch(f, 0, dim3(kInter / 16, T * kTopk), dim3(256), args, stream);
  return rc ? rc : ok(f);
}

extern "C" int netra_qwen36_moe_gate_up_unload(void) { return unload(g_gate_up); }
extern "C" const char* netra_qwen36_moe_gate_up_last_error(void) { return error_of(g_gate_up).c_str(); }

// ---- M768 prefill producer/reducer -------------------------------------------------------

extern "C" int netra_moe_prefill_m768_load(const char* producer_hsaco, const char* reducer_hsaco) {
  if (producer_hsaco == nullptr || producer_hsaco[0] == '\0' || reducer_hsaco == nullptr ||
      reducer_hsaco[0] == '\0')
    return refuse(g_prefill, "both code-object paths must be nonempty");
  return load(g_prefill, producer_hsaco, reducer_hsaco);
}

extern "C" int netra_moe_prefill_m768_launch(const void* hidden_fp8, const float* hidden_scale_f32,
                                             const void* w13_fp8, const float* w13_scale_f32, const void* w2_fp8,
                                             const float* w2_scale_f32, const int32_t* sorted_token_ids_i32,
                                             const float* sorted_weights_f32,
                                             const int32_t* sorted_expert_ids_i32,
                                             const int32_t* num_valid_ids_i32, const float* topk_weights_f32,
                                             float* route_scale_workspace_f32, void* partials_f16,
                                             void* output_bf16, hipStream_t stream) {
  Family& f = g_prefill;
  if (!loaded(f)) return refuse(f, "modules are not loaded");
  const void* const ptrs[] = {hidden_fp8, hidden_scale_f32, w13_fp8, w13_scale_f32, w2_fp8,
                              w2_scale_f32, sorted_token_ids_i32, sorted_weights_f32, sorted_expert_ids_i32,
                              num_valid_ids_i32, topk_weights_f32, route_scale_workspace_f32, partials_f16,
                              output_bf16};
  if (!all_set(ptrs)) return refuse(f, "launch pointers must be nonnull");
  netra_prefill::Buffers b{hidden_fp8, hidden_scale_f32, w13_fp8, w13_scale_f32, w2_fp8, w2_scale_f32,
                           sorted_token_ids_i32, sorted_expert_ids_i32, num_valid_ids_i32, topk_weights_f32,
                           route_scale_workspace_f32, partials_f16, output_bf16, f.scratch};
  netra_prefill::Args a;
  netra_prefill::build(a, b, netra_prefill::kMaxRows);
  for (uint32_t k = 0; k < netra_prefill::kKernels; ++k) {
    const int rc = dispatch(f, k, a.grid[k], a.block[k], a.params[k], stream);
    if (rc) return rc;
  }
  return ok(f);
}

extern "C" int netra_moe_prefill_m768_unload(void) { return unload(g_prefill); }
extern "C" const char* netra_moe_prefill_m768_last_error(void) { return error_of(g_prefill).c_str(); }
