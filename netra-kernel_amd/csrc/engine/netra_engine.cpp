// Netra engine C-ABI runtime for gfx950: engine directory -> loaded code
// objects, bound pointers, fixed launches on the caller's stream.
//
// Behaviour mirrors the reference runtime (runtime/gfx950/engine/
// netra_engine.hip): create 249-395, query 400-405, bind 406-420, finalize
// 421-434, prepare (graph capture) 435-449, launch 450-466, launch_operation
// 467-497, launch_operation_bound 498-558, last_error 559, destroy 562-566.
// The launch paths allocate nothing, parse nothing, never synchronise and
// touch no files or environment.
#include "../../../include/netra_engine.h"

#include <hip/hip_runtime.h>

#include <array>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <map>
#include <new>
#include <string>
#include <vector>

#include "manifest.h"

namespace {

struct OpRecord {
  bool fallback = true;
  hipFunction_t function = nullptr;
  std::array<uint32_t, 3> grid{1, 1, 1};
  std::array<uint32_t, 3> block{1, 1, 1};
  uint32_t dynamic_lds_bytes = 0;
  uint32_t argument_count = 0;
  // Argument storage: kernelParams entries point into these arrays, so a
  // record is never moved after create (profiles reserve their vectors).
  std::array<void*, netra::kMaxArguments> pointers{};
  std::array<uint32_t, netra::kMaxArguments> scalars{};
  std::array<void*, netra::kMaxArguments> params{};
  std::array<bool, netra::kMaxArguments> bindable{};
  std::array<bool, netra::kMaxArguments> is_scalar{};
};

struct ProfileRecord {
  netra_profile_info_t info{};
  std::vector<OpRecord> ops;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  bool graph_ready = false;
};

}  // namespace

struct netra_engine {
  int device = -1;
  bool graph_capture = false;
  void* workspace = nullptr;
  uint64_t workspace_bytes = 0;
  std::map<std::string, hipModule_t> modules;
  std::vector<ProfileRecord> profiles;
  std::atomic<bool> finalized{false};
  std::atomic<uint32_t> in_flight{0};
  char last_error[512] = {0};
};

namespace {

netra_status_t fail(netra_engine* e, netra_status_t status, const char* message) {
  if (e) std::snprintf(e->last_error, sizeof(e->last_error), "%s", message);
  return status;
}

netra_status_t hip_fail(netra_engine* e, const char* what, hipError_t err) {
  if (e) std::snprintf(e->last_error, sizeof(e->last_error), "%s: %s", what, hipGetErrorString(err));
  return NETRA_STATUS_HIP;
}

void clear_error(netra_engine* e) { e->last_error[0] = '\0'; }

bool guard_ok(const netra_profile_info_t& p, const netra_launch_shape_t& s) {
  return s.m >= p.min_m && s.m <= p.max_m && s.batch >= p.min_batch && s.batch <= p.max_batch &&
         s.sequence >= p.min_sequence && s.sequence <= p.max_sequence &&
         s.tensor_parallel == p.tensor_parallel;
}

bool all_bound(const OpRecord& op) {
  for (uint32_t i = 0; i < op.argument_count; ++i)
    if (op.bindable[i] && op.pointers[i] == nullptr) return false;
  return true;
}

hipError_t submit(const OpRecord& op, void** params, hipStream_t stream) {
  return hipModuleLaunchKernel(op.function, op.grid[0], op.grid[1], op.grid[2], op.block[0],
                               op.block[1], op.block[2], op.dynamic_lds_bytes, stream, params,
                               nullptr);
}

netra_status_t launch_all(netra_engine* e, ProfileRecord& p, hipStream_t stream) {
  for (OpRecord& op : p.ops) {
    if (op.fallback)
      return fail(e, NETRA_STATUS_FALLBACK_REQUIRED, "profile contains a framework fallback operation");
    if (!all_bound(op)) return fail(e, NETRA_STATUS_BINDING, "kernel pointer argument is unbound");
    const hipError_t err = submit(op, op.params.data(), stream);
    if (err != hipSuccess) return hip_fail(e, "hipModuleLaunchKernel", err);
  }
  return NETRA_STATUS_OK;
}

void release(netra_engine* e) {
  for (ProfileRecord& p : e->profiles) {
    if (p.graph_exec) (void)hipGraphExecDestroy(p.graph_exec);
    if (p.graph) (void)hipGraphDestroy(p.graph);
  }
  for (auto& kv : e->modules)
    if (kv.second) (void)hipModuleUnload(kv.second);
  if (e->workspace) (void)hipFree(e->workspace);
}

netra_status_t check_device(netra_engine* e) {
  int device = -1;
  const hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_fail(e, "hipGetDevice", err);
  if (device != e->device)
    return fail(e, NETRA_STATUS_UNSUPPORTED_TARGET,
                "caller stream/device does not belong to engine device");
  return NETRA_STATUS_OK;
}

// Restores the caller's current device when create returns.
struct DeviceScope {
  int previous = -1;
  ~DeviceScope() {
    if (previous >= 0) (void)hipSetDevice(previous);
  }
};

}  // namespace

extern "C" netra_status_t netra_engine_manifest_check(const char* directory, char* error,
                                                      size_t error_size) {
  if (!directory || !*directory) return NETRA_STATUS_INVALID_ARGUMENT;
  try {
    (void)netra::load_manifest(directory);
    if (error && error_size) error[0] = '\0';
    return NETRA_STATUS_OK;
  } catch (const std::exception& ex) {
    if (error && error_size) std::snprintf(error, error_size, "%s", ex.what());
    return std::strncmp(ex.what(), "cannot open", 11) == 0 ? NETRA_STATUS_IO : NETRA_STATUS_MANIFEST;
  }
}

extern "C" netra_status_t netra_engine_create(const char* directory,
                                              const netra_engine_options_t* options,
                                              netra_engine_t** output) {
  if (!directory || !*directory || !options || !output ||
      options->struct_size != sizeof(netra_engine_options_t))
    return NETRA_STATUS_INVALID_ARGUMENT;
  *output = nullptr;
  netra_engine* e = new (std::nothrow) netra_engine;
  if (!e) return NETRA_STATUS_IO;
  e->device = options->device_id;
  e->graph_capture = options->enable_graph_capture != 0;

  DeviceScope scope;
  hipError_t err = hipGetDevice(&scope.previous);
  if (err != hipSuccess) { delete e; return NETRA_STATUS_HIP; }
  err = hipSetDevice(e->device);
  if (err != hipSuccess) { delete e; return NETRA_STATUS_HIP; }
  hipDeviceProp_t prop{};
  err = hipGetDeviceProperties(&prop, e->device);
  if (err != hipSuccess) { delete e; return NETRA_STATUS_HIP; }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0 || prop.warpSize != 64) {
    delete e;
    return NETRA_STATUS_UNSUPPORTED_TARGET;
  }

  netra::EngineManifest manifest;
  try {
    manifest = netra::load_manifest(directory);
  } catch (const std::exception&) {
    delete e;
    return NETRA_STATUS_MANIFEST;
  }
  int runtime_version = 0;
  err = hipRuntimeGetVersion(&runtime_version);
  if (err != hipSuccess) { delete e; return NETRA_STATUS_HIP; }
  const uint32_t major = static_cast<uint32_t>(runtime_version / 10000000);
  const uint32_t minor = static_cast<uint32_t>((runtime_version / 100000) % 100);
  if (major < manifest.rocm_major || (major == manifest.rocm_major && minor < manifest.rocm_minor)) {
    delete e;
    return NETRA_STATUS_MANIFEST;
  }

  e->workspace_bytes = manifest.workspace_bytes;
  if (e->workspace_bytes) {
    err = hipMalloc(&e->workspace, static_cast<size_t>(e->workspace_bytes));
    if (err != hipSuccess) { release(e); delete e; return NETRA_STATUS_HIP; }
  }

  // Load each distinct code object once and resolve every kernel symbol.
  std::vector<hipFunction_t> functions(manifest.operations.size(), nullptr);
  for (size_t i = 0; i < manifest.operations.size(); ++i) {
    const netra::OperationSpec& spec = manifest.operations[i];
    if (spec.fallback) continue;
    auto it = e->modules.find(spec.hsaco);
    if (it == e->modules.end()) {
      hipModule_t module = nullptr;
      err = hipModuleLoad(&module, (std::string(directory) + "/" + spec.hsaco).c_str());
      if (err != hipSuccess) { release(e); delete e; return NETRA_STATUS_MANIFEST; }
      it = e->modules.emplace(spec.hsaco, module).first;
    }
    err = hipModuleGetFunction(&functions[i], it->second, spec.kernel_symbol.c_str());
    if (err != hipSuccess) { release(e); delete e; return NETRA_STATUS_MANIFEST; }
    // The launch must fit what the code object was compiled for: a block
    // beyond the kernel's flat work-group bound, or static + dynamic LDS beyond
    // the CU's 160 KiB, is a manifest error here rather than a failed launch.
    int max_threads = 0, static_lds = 0;
    if (hipFuncGetAttribute(&max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, functions[i]) != hipSuccess ||
        hipFuncGetAttribute(&static_lds, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, functions[i]) != hipSuccess) {
      release(e);
      delete e;
      return NETRA_STATUS_HIP;
    }
    const uint64_t threads = static_cast<uint64_t>(spec.block[0]) * spec.block[1] * spec.block[2];
    if (threads > static_cast<uint64_t>(max_threads) ||
        static_cast<uint64_t>(static_lds) + spec.dynamic_lds_bytes > 160u * 1024u) {
      release(e);
      delete e;
      return NETRA_STATUS_MANIFEST;
    }
  }

  e->profiles.resize(manifest.profiles.size());
  for (size_t pi = 0; pi < manifest.profiles.size(); ++pi) {
    const netra::ProfileSpec& ps = manifest.profiles[pi];
    ProfileRecord& pr = e->profiles[pi];
    pr.info.struct_size = sizeof(netra_profile_info_t);
    pr.info.profile_id = static_cast<uint32_t>(pi);
    pr.info.min_m = ps.min_m;
    pr.info.max_m = ps.max_m;
    pr.info.min_batch = ps.min_batch;
    pr.info.max_batch = ps.max_batch;
    pr.info.min_sequence = ps.min_sequence;
    pr.info.max_sequence = ps.max_sequence;
    pr.info.tensor_parallel = ps.tensor_parallel;
    pr.info.workspace_bytes = manifest.workspace_bytes;
    pr.ops.resize(manifest.operations.size());  // never resized again
    for (size_t oi = 0; oi < manifest.operations.size(); ++oi) {
      const netra::OperationSpec& spec = manifest.operations[oi];
      OpRecord& op = pr.ops[oi];
      op.fallback = spec.fallback;
      if (op.fallback) { pr.info.requires_fallback = 1; continue; }
      op.function = functions[oi];
      op.grid = spec.grid;
      op.block = spec.block;
      op.dynamic_lds_bytes = spec.dynamic_lds_bytes;
      op.argument_count = static_cast<uint32_t>(spec.arguments.size());
      for (uint32_t a = 0; a < op.argument_count; ++a) {
        const netra::ArgumentSpec& as = spec.arguments[a];
        switch (as.kind) {
          case netra::ArgumentSpec::Kind::Binding:
            op.bindable[a] = true;
            break;
          case netra::ArgumentSpec::Kind::Workspace:
            op.pointers[a] = static_cast<unsigned char*>(e->workspace) + as.workspace_offset;
            break;
          case netra::ArgumentSpec::Kind::U32:
            op.is_scalar[a] = true;
            op.scalars[a] = as.value;
            break;
        }
        op.params[a] = op.is_scalar[a] ? static_cast<void*>(&op.scalars[a])
                                       : static_cast<void*>(&op.pointers[a]);
      }
    }
  }
  *output = e;
  return NETRA_STATUS_OK;
}

extern "C" size_t netra_engine_profile_count(const netra_engine_t* e) {
  return e ? e->profiles.size() : 0;
}

extern "C" netra_status_t netra_engine_query_profile(const netra_engine_t* e, uint32_t profile_id,
                                                     netra_profile_info_t* out) {
  if (!e || !out || out->struct_size != sizeof(netra_profile_info_t))
    return NETRA_STATUS_INVALID_ARGUMENT;
  if (profile_id >= e->profiles.size()) return NETRA_STATUS_UNSUPPORTED_PROFILE;
  *out = e->profiles[profile_id].info;
  return NETRA_STATUS_OK;
}

extern "C" netra_status_t netra_engine_bind(netra_engine_t* e, uint32_t profile_id,
                                            uint32_t op_index, uint32_t arg_index, void* ptr) {
  if (!e || !ptr) return NETRA_STATUS_INVALID_ARGUMENT;
  if (e->finalized.load(std::memory_order_acquire))
    return fail(e, NETRA_STATUS_BUSY, "bindings are finalized and immutable");
  if (e->in_flight.load(std::memory_order_acquire))
    return fail(e, NETRA_STATUS_BUSY, "cannot bind during launch");
  if (profile_id >= e->profiles.size() || op_index >= e->profiles[profile_id].ops.size())
    return fail(e, NETRA_STATUS_BINDING, "binding index out of range");
  ProfileRecord& p = e->profiles[profile_id];
  if (p.graph_ready) return fail(e, NETRA_STATUS_BUSY, "bindings are immutable after graph preparation");
  OpRecord& op = p.ops[op_index];
  if (arg_index >= op.argument_count) return fail(e, NETRA_STATUS_BINDING, "argument index out of range");
  if (!op.bindable[arg_index])
    return fail(e, NETRA_STATUS_BINDING, "constant kernel arguments cannot be rebound");
  op.pointers[arg_index] = ptr;
  clear_error(e);
  return NETRA_STATUS_OK;
}

extern "C" netra_status_t netra_engine_finalize_bindings(netra_engine_t* e) {
  if (!e) return NETRA_STATUS_INVALID_ARGUMENT;
  if (e->in_flight.load(std::memory_order_acquire))
    return fail(e, NETRA_STATUS_BUSY, "cannot finalize bindings during launch");
  for (const ProfileRecord& p : e->profiles)
    for (const OpRecord& op : p.ops)
      if (!op.fallback && !all_bound(op))
        return fail(e, NETRA_STATUS_BINDING,
                    "all direct-launch pointers must be bound before finalization");
  e->finalized.store(true, std::memory_order_release);
  clear_error(e);
  return NETRA_STATUS_OK;
}

extern "C" netra_status_t netra_engine_prepare_profile(netra_engine_t* e, uint32_t profile_id,
                                                       hipStream_t stream) {
  if (!e || profile_id >= e->profiles.size()) return NETRA_STATUS_INVALID_ARGUMENT;
  ProfileRecord& p = e->profiles[profile_id];
  if (!e->graph_capture || p.graph_ready) return NETRA_STATUS_OK;
  if (p.info.requires_fallback)
    return fail(e, NETRA_STATUS_FALLBACK_REQUIRED, "fallback profile cannot be captured");
  const netra_status_t fin = netra_engine_finalize_bindings(e);
  if (fin != NETRA_STATUS_OK) return fin;
  hipError_t err = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
  if (err != hipSuccess) return hip_fail(e, "hipStreamBeginCapture", err);
  const netra_status_t st = launch_all(e, p, stream);
  hipGraph_t graph = nullptr;
  err = hipStreamEndCapture(stream, &graph);
  if (st != NETRA_STATUS_OK) {
    if (graph) (void)hipGraphDestroy(graph);
    return st;
  }
  if (err != hipSuccess) return hip_fail(e, "hipStreamEndCapture", err);
  err = hipGraphInstantiate(&p.graph_exec, graph, nullptr, nullptr, 0);
  if (err != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return hip_fail(e, "hipGraphInstantiate", err);
  }
  p.graph = graph;
  p.graph_ready = true;
  return NETRA_STATUS_OK;
}

extern "C" netra_status_t netra_engine_launch(netra_engine_t* e, uint32_t profile_id,
                                              const netra_launch_shape_t* shape,
                                              hipStream_t stream) {
  if (!e || !shape || profile_id >= e->profiles.size()) return NETRA_STATUS_INVALID_ARGUMENT;
  netra_status_t st = check_device(e);
  if (st != NETRA_STATUS_OK) return st;
  ProfileRecord& p = e->profiles[profile_id];
  if (!guard_ok(p.info, *shape))
    return fail(e, NETRA_STATUS_UNSUPPORTED_PROFILE,
                "exact/bounded profile guard failed; framework fallback required");
  if (p.info.requires_fallback)
    return fail(e, NETRA_STATUS_FALLBACK_REQUIRED, "profile contains a framework fallback operation");
  if (!p.graph_ready && !e->finalized.load(std::memory_order_acquire))
    return fail(e, NETRA_STATUS_BINDING, "direct-launch bindings were not finalized");
  e->in_flight.fetch_add(1, std::memory_order_acq_rel);
  if (p.graph_ready) {
    const hipError_t err = hipGraphLaunch(p.graph_exec, stream);
    st = err == hipSuccess ? NETRA_STATUS_OK : hip_fail(e, "hipGraphLaunch", err);
  } else {
    st = launch_all(e, p, stream);
  }
  e->in_flight.fetch_sub(1, std::memory_order_acq_rel);
  return st;
}

extern "C" netra_status_t netra_engine_launch_operation(netra_engine_t* e, uint32_t profile_id,
                                                        uint32_t op_index,
                                                        const netra_launch_shape_t* shape,
                                                        hipStream_t stream) {
  if (!e || !shape || profile_id >= e->profiles.size() ||
      op_index >= e->profiles[profile_id].ops.size())
    return NETRA_STATUS_INVALID_ARGUMENT;
  netra_status_t st = check_device(e);
  if (st != NETRA_STATUS_OK) return st;
  ProfileRecord& p = e->profiles[profile_id];
  if (!guard_ok(p.info, *shape))
    return fail(e, NETRA_STATUS_UNSUPPORTED_PROFILE,
                "exact/bounded profile guard failed; framework fallback required");
  if (p.graph_ready)
    return fail(e, NETRA_STATUS_BUSY, "individual operations cannot launch after graph preparation");
  OpRecord& op = p.ops[op_index];
  if (op.fallback) return fail(e, NETRA_STATUS_FALLBACK_REQUIRED, "operation requires framework fallback");
  if (!e->finalized.load(std::memory_order_acquire))
    return fail(e, NETRA_STATUS_BINDING, "direct-launch bindings were not finalized");
  if (!all_bound(op)) return fail(e, NETRA_STATUS_BINDING, "kernel pointer argument is unbound");
  e->in_flight.fetch_add(1, std::memory_order_acq_rel);
  const hipError_t err = submit(op, op.params.data(), stream);
  st = err == hipSuccess ? NETRA_STATUS_OK : hip_fail(e, "hipModuleLaunchKernel", err);
  e->in_flight.fetch_sub(1, std::memory_order_acq_rel);
  return st;
}

extern "C" netra_status_t netra_engine_launch_operation_bound(
    netra_engine_t* e, uint32_t profile_id, uint32_t op_index, const netra_launch_shape_t* shape,
    const netra_pointer_binding_t* bindings, uint32_t count, hipStream_t stream) {
  if (!e || !shape || profile_id >= e->profiles.size() ||
      op_index >= e->profiles[profile_id].ops.size() || (count && !bindings) || count > 16)
    return NETRA_STATUS_INVALID_ARGUMENT;
  netra_status_t st = check_device(e);
  if (st != NETRA_STATUS_OK) return st;
  ProfileRecord& p = e->profiles[profile_id];
  if (!guard_ok(p.info, *shape))
    return fail(e, NETRA_STATUS_UNSUPPORTED_PROFILE,
                "exact/bounded profile guard failed; framework fallback required");
  if (p.graph_ready)
    return fail(e, NETRA_STATUS_BUSY, "operation bindings are immutable after graph preparation");
  const OpRecord& op = p.ops[op_index];
  if (op.fallback) return fail(e, NETRA_STATUS_FALLBACK_REQUIRED, "operation requires framework fallback");
  uint32_t slots = 0;
  for (uint32_t a = 0; a < op.argument_count; ++a) slots += op.bindable[a] ? 1u : 0u;
  if (count != slots)
    return fail(e, NETRA_STATUS_BINDING, "bound operation must provide every declared pointer slot");
  std::array<void*, netra::kMaxArguments> values{};
  std::array<void*, netra::kMaxArguments> params{};
  std::array<bool, netra::kMaxArguments> seen{};
  for (uint32_t a = 0; a < op.argument_count; ++a) values[a] = op.bindable[a] ? nullptr : op.pointers[a];
  for (uint32_t i = 0; i < count; ++i) {
    const uint32_t a = bindings[i].argument_index;
    if (bindings[i].reserved || !bindings[i].pointer || a >= op.argument_count || !op.bindable[a])
      return fail(e, NETRA_STATUS_BINDING, "bound operation contains an invalid pointer slot");
    if (seen[a]) return fail(e, NETRA_STATUS_BINDING, "bound operation contains a duplicate pointer slot");
    seen[a] = true;
    values[a] = bindings[i].pointer;
  }
  for (uint32_t a = 0; a < op.argument_count; ++a)
    params[a] = op.is_scalar[a] ? const_cast<uint32_t*>(&op.scalars[a]) : static_cast<void*>(&values[a]);
  e->in_flight.fetch_add(1, std::memory_order_acq_rel);
  const hipError_t err = submit(op, params.data(), stream);
  st = err == hipSuccess ? NETRA_STATUS_OK : hip_fail(e, "hipModuleLaunchKernel", err);
  e->in_flight.fetch_sub(1, std::memory_order_acq_rel);
  return st;
}

extern "C" const char* netra_engine_last_error(const netra_engine_t* e) {
  return e ? e->last_error : "netra_engine is null";
}

extern "C" netra_status_t netra_engine_destroy(netra_engine_t* e) {
  if (!e) return NETRA_STATUS_OK;
  if (e->in_flight.load(std::memory_order_acquire))
    return fail(e, NETRA_STATUS_BUSY, "launches remain in flight");
  release(e);
  delete e;
  return NETRA_STATUS_OK;
}
