// Direct C entry points of libnetra_moe.so: weight preparation, and the
// allocation-free prefill entry point. The MoE layer itself runs through the
// engine ABI; this library carries its own copy of the kernels (compiled in,
// launched without a code-object load).
#include "../../../include/netra_moe.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../kernels/moe_kernels.hip"
#include "prefill_plan.h"

namespace {
thread_local std::string g_last_error;

int fail(int code, const std::string& message) {
  g_last_error = message;
  return code;
}
}  // namespace

extern "C" int netra_moe_quant_blocks(const float* w, uint8_t* q, float* s, uint32_t groups,
                                      uint32_t n, uint32_t k, hipStream_t stream) {
  if (!w || !q || !s || groups == 0 || n == 0 || k == 0 || n % 128u || k % 128u)
    return fail(-1, "netra_moe_quant_blocks: null pointer or n/k not a positive multiple of 128");
  const uint64_t blocks = static_cast<uint64_t>(groups) * (n / 128u) * (k / 128u);
  if (blocks > 0x7fffffffull) return fail(-1, "netra_moe_quant_blocks: too many blocks");
  hipLaunchKernelGGL(netra_moe_quant_blocks_gfx950, dim3(static_cast<uint32_t>(blocks)), dim3(256),
                     0, stream, w, q, s, groups, n, k);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(static_cast<int>(err), hipGetErrorString(err));
  g_last_error.clear();
  return 0;
}

extern "C" int netra_moe_pack_tiles(const uint8_t* src, uint8_t* dst, uint32_t groups, uint32_t n,
                                    uint32_t k, hipStream_t stream) {
  if (!src || !dst || src == dst || groups == 0 || n == 0 || k == 0 || n % 16u || k % 128u)
    return fail(-1, "netra_moe_pack_tiles: null/aliased pointers or n % 16, k % 128 != 0");
  const uint64_t tiles = static_cast<uint64_t>(groups) * (n / 16u) * (k / 128u);
  if (tiles > 0xfffffffcull) return fail(-1, "netra_moe_pack_tiles: too many tiles");
  hipLaunchKernelGGL(netra_moe_pack_tiles_gfx950, dim3(static_cast<uint32_t>((tiles + 3u) / 4u)),
                     dim3(256), 0, stream, src, dst, groups, n, k, 0u);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(static_cast<int>(err), hipGetErrorString(err));
  g_last_error.clear();
  return 0;
}

extern "C" int netra_moe_pack_tiles_gate_up(const uint8_t* src, uint8_t* dst, uint32_t groups,
                                            uint32_t n, uint32_t k, hipStream_t stream) {
  if (!src || !dst || src == dst || groups == 0 || n == 0 || k == 0 || n % 32u || k % 128u)
    return fail(-1, "netra_moe_pack_tiles_gate_up: null/aliased pointers or n % 32, k % 128 != 0");
  const uint64_t tiles = static_cast<uint64_t>(groups) * (n / 16u) * (k / 128u);
  if (tiles > 0xfffffffcull) return fail(-1, "netra_moe_pack_tiles_gate_up: too many tiles");
  hipLaunchKernelGGL(netra_moe_pack_tiles_gfx950, dim3(static_cast<uint32_t>((tiles + 3u) / 4u)),
                     dim3(256), 0, stream, src, dst, groups, n, k, 1u);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(static_cast<int>(err), hipGetErrorString(err));
  g_last_error.clear();
  return 0;
}

static int pack_from_aiter(const char* name, const uint8_t* src, uint8_t* dst, uint32_t groups,
                           uint32_t n, uint32_t k, uint32_t gate_up, hipStream_t stream) {
  if (!src || !dst || src == dst || groups == 0 || n == 0 || k == 0 || n % (gate_up ? 32u : 16u) ||
      k % 128u)
    return fail(-1, std::string(name) + ": null/aliased pointers or n % " + (gate_up ? "32" : "16") +
                        ", k % 128 != 0");
  const uint64_t tiles = static_cast<uint64_t>(groups) * (n / 16u) * (k / 128u);
  if (tiles > 0xfffffffcull) return fail(-1, std::string(name) + ": too many tiles");
  hipLaunchKernelGGL(netra_moe_pack_tiles_aiter_gfx950, dim3(static_cast<uint32_t>((tiles + 3u) / 4u)),
                     dim3(256), 0, stream, src, dst, groups, n, k, gate_up);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(static_cast<int>(err), hipGetErrorString(err));
  g_last_error.clear();
  return 0;
}

extern "C" int netra_moe_pack_tiles_from_aiter(const uint8_t* src, uint8_t* dst, uint32_t groups,
                                               uint32_t n, uint32_t k, hipStream_t stream) {
  return pack_from_aiter("netra_moe_pack_tiles_from_aiter", src, dst, groups, n, k, 0u, stream);
}

extern "C" int netra_moe_pack_tiles_gate_up_from_aiter(const uint8_t* src, uint8_t* dst, uint32_t groups,
                                                       uint32_t n, uint32_t k, hipStream_t stream) {
  return pack_from_aiter("netra_moe_pack_tiles_gate_up_from_aiter", src, dst, groups, n, k, 1u, stream);
}

extern "C" int netra_moe_e4m3_check(const float* in, uint8_t* sw, uint8_t* hw, uint32_t n,
                                    hipStream_t stream) {
  if (!in || !sw || !hw || n == 0) return fail(-1, "netra_moe_e4m3_check: null pointer or n == 0");
  const uint32_t grid = (n + 1023u) / 1024u;
  hipLaunchKernelGGL(netra_moe_e4m3_check_gfx950, dim3(grid), dim3(256), 0, stream, in, sw, hw, n);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(static_cast<int>(err), hipGetErrorString(err));
  g_last_error.clear();
  return 0;
}

extern "C" int netra_moe_copy(const void* src, void* dst, uint64_t bytes, hipStream_t stream) {
  if (!src || !dst || bytes == 0 || bytes % 16u || (reinterpret_cast<uintptr_t>(src) & 15u) ||
      (reinterpret_cast<uintptr_t>(dst) & 15u))
    return fail(-1, "netra_moe_copy: null pointer, or size/alignment not a multiple of 16 bytes");
  hipLaunchKernelGGL(netra_moe_copy_gfx950, dim3(2048), dim3(256), 0, stream,
                     static_cast<const uint4*>(src), static_cast<uint4*>(dst), bytes / 16u);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(static_cast<int>(err), hipGetErrorString(err));
  g_last_error.clear();
  return 0;
}

extern "C" const char* netra_moe_last_error(void) { return g_last_error.c_str(); }

// ---------------------------------------------------------------------------
// Allocation-free prefill producer/reducer (no counterpart in the reference;
// the variant of netra_moe_prefill_m768_launch for callers that cannot
// allocate: code under stream capture, serving loops, harnesses).
//
// The launch's scratch (h e4m3 for 365 x 64 rows of 512, the block-pair list
// and four counts; 11.7 MiB) lives in `scratch`, a file-scope device array
// that every GPU the library runs on holds until the process ends. Host code
// never passes the array's name to a kernel: the name is a host-side stand-in.
// The first call on a device, with that device current, resolves the
// device's own copy with hipGetSymbolAddress, once; every later call uses that
// address. Calls on one GPU share its array, so calls that overlap on one GPU
// (two streams, or two threads) race; nothing in the array has to start at
// zero (the block-pair kernel rewrites the list and counts, gate/up writes h
// for every valid row before down reads it, and padding rows' garbage only
// reaches outputs that are never stored).
constexpr size_t kScratchBytes = netra_prefill::scratch_bytes(netra_prefill::kMaxRows);
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_on_device[kMaxDevices];
std::mutex g_scratch_mutex;

// This device's address of `scratch` (resolved once per device).
int device_scratch(void** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(static_cast<int>(err), std::string("hipGetDevice: ") + hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices) return fail(-1, "netra_moe_prefill_launch_noalloc: device index out of range");
  void* p = g_scratch_on_device[device].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_on_device[device].load(std::memory_order_relaxed);
    if (p == nullptr) {
      err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (err != hipSuccess || p == nullptr)
        return fail(err != hipSuccess ? static_cast<int>(err) : -1,
                    std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(err));
      g_scratch_on_device[device].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}
}  // namespace

extern "C" int netra_moe_prefill_launch_noalloc(
    const void* hidden_fp8, const float* hidden_scale_f32, const void* w13_fp8, const float* w13_scale_f32,
    const void* w2_fp8, const float* w2_scale_f32, const int32_t* sorted_token_ids_i32,
    const float* sorted_weights_f32, const int32_t* sorted_expert_ids_i32, const int32_t* num_valid_ids_i32,
    const float* topk_weights_f32, float* route_scale_workspace_f32, void* partials_f16, void* output_bf16,
    uint32_t rows, hipStream_t stream) {
  if (rows == 0 || rows > netra_prefill::kMaxRows)
    return fail(-1, "netra_moe_prefill_launch_noalloc: rows must be 1.." + std::to_string(netra_prefill::kMaxRows) +
                        " (the static scratch holds the 768-row shape), got " + std::to_string(rows));
  const void* const ptrs[] = {hidden_fp8, hidden_scale_f32, w13_fp8, w13_scale_f32, w2_fp8,
                              w2_scale_f32, sorted_token_ids_i32, sorted_weights_f32, sorted_expert_ids_i32,
                              num_valid_ids_i32, topk_weights_f32, route_scale_workspace_f32, partials_f16,
                              output_bf16};
  for (const void* p : ptrs)
    if (p == nullptr) return fail(-1, "netra_moe_prefill_launch_noalloc: launch pointers must be nonnull");
  void* dev_scratch = nullptr;
  const int rc = device_scratch(&dev_scratch);
  if (rc != 0) return rc;
  const netra_prefill::Buffers b{hidden_fp8, hidden_scale_f32, w13_fp8, w13_scale_f32, w2_fp8, w2_scale_f32,
                                 sorted_token_ids_i32, sorted_expert_ids_i32, num_valid_ids_i32, topk_weights_f32,
                                 route_scale_workspace_f32, partials_f16, output_bf16, dev_scratch};
  netra_prefill::Args a;
  netra_prefill::build(a, b, rows);
  const void* const kernels[netra_prefill::kKernels] = {
      reinterpret_cast<const void*>(&netra_moe_block_pairs_gfx950),
      reinterpret_cast<const void*>(&netra_moe_gate_up_lds_aiter_h2048_gfx950),
      reinterpret_cast<const void*>(&netra_moe_down_rows_aiter_f16x2_i512_gfx950),
      reinterpret_cast<const void*>(&netra_moe_route_reduce_f16x2_gfx950)};
  for (uint32_t k = 0; k < netra_prefill::kKernels; ++k) {
    const hipError_t err = hipLaunchKernel(kernels[k], a.grid[k], a.block[k], a.params[k], 0, stream);
    if (err != hipSuccess)
      return fail(static_cast<int>(err), std::string("netra_moe_prefill_launch_noalloc: ") + hipGetErrorString(err));
  }
  g_last_error.clear();
  return 0;
}
