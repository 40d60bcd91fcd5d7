// Direct C entry points of libnetra_moe.so (weight preparation). The MoE
// layer itself runs through the engine ABI; this library carries the kernels
// that run once at weight-load time.
#include "../../../include/netra_moe.h"

#include <hip/hip_runtime.h>

#include <string>

#include "../kernels/moe_kernels.hip"

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
