// Netra engine C-ABI runtime for gfx950: engine directory -> loaded code
// objects, bound pointers, fixed launches on the caller's stream.
//
// The entry points are those of the reference runtime
// (runtime/gfx950/engine/netra_engine.h:60-108). Which status a given misuse
// returns, and which check wins when several apply, is interface a caller of
// the reference depends on; those precedences are kept and listed, entry by
// entry, above each function below. The bodies, the engine's state model and
// the error texts are this runtime's own (one text, "bindings are finalized
// and immutable", is kept word for word because a reference test looks for
// it: tests/compiler/test_runtime_hotpath.py:68).
//
// State: bindings are open until netra_engine_finalize_bindings (engine-wide,
// one way); a profile captured by netra_engine_prepare_profile is immutable
// and launches only as its graph. `in_flight` counts launch calls between
// admission and return, so bind / finalize / destroy can refuse during one.
// The launch paths allocate nothing, parse nothing, never synchronise and
// touch no files or environment.
#include "../../../include/netra_engine.h"

#include <hip/hip_runtime.h>

#include <array>
#include <atomic>
#include <cstdarg>
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
  uint32_t slot_count = 0;  // pointer arguments the caller binds
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
  bool captured = false;
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

// Records a refusal (formatted into the engine's last_error) and returns its status.
__attribute__((format(printf, 3, 4))) netra_status_t refuse(netra_engine* e, netra_status_t status,
                                                           const char* format, ...) {
  if (e) {
    va_list args;
    va_start(args, format);
    std::vsnprintf(e->last_error, sizeof(e->last_error), format, args);
    va_end(args);
  }
  return status;
}

netra_status_t hip_refusal(netra_engine* e, const char* call, hipError_t err) {
  return refuse(e, NETRA_STATUS_HIP, "%s failed: %s", call, hipGetErrorString(err));
}

netra_status_t accept(netra_engine* e) {
  e->last_error[0] = '\0';
  return NETRA_STATUS_OK;
}

bool busy(const netra_engine* e) { return e->in_flight.load(std::memory_order_acquire) != 0; }
bool finalized(const netra_engine* e) { return e->finalized.load(std::memory_order_acquire); }

// First pointer slot of an operation with nothing bound, or -1.
int first_unbound(const OpRecord& op) {
  for (uint32_t a = 0; a < op.argument_count; ++a)
    if (op.bindable[a] && op.pointers[a] == nullptr) return static_cast<int>(a);
  return -1;
}

bool within_guards(const netra_profile_info_t& p, const netra_launch_shape_t& s) {
  return p.min_m <= s.m && s.m <= p.max_m && p.min_batch <= s.batch && s.batch <= p.max_batch &&
         p.min_sequence <= s.sequence && s.sequence <= p.max_sequence &&
         s.tensor_parallel == p.tensor_parallel;
}

// Shared first checks of the three launch entry points, after argument
// validation: the current device is the engine's (UNSUPPORTED_TARGET), then
// the shape is inside the profile's guards (UNSUPPORTED_PROFILE).
netra_status_t admit(netra_engine* e, const ProfileRecord& p, const netra_launch_shape_t& shape) {
  int device = -1;
  const hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_refusal(e, "hipGetDevice", err);
  if (device != e->device)
    return refuse(e, NETRA_STATUS_UNSUPPORTED_TARGET,
                  "launch refused: current device %d is not the engine's device %d", device, e->device);
  if (!within_guards(p.info, shape))
    return refuse(e, NETRA_STATUS_UNSUPPORTED_PROFILE,
                  "launch refused: shape (m=%u, batch=%u, sequence=%llu, tp=%u) is outside profile %u's "
                  "guards; the caller takes its framework path",
                  shape.m, shape.batch, static_cast<unsigned long long>(shape.sequence),
                  shape.tensor_parallel, p.info.profile_id);
  return NETRA_STATUS_OK;
}

// Marks one launch call in flight for its lifetime.
struct LaunchScope {
  netra_engine* e;
  explicit LaunchScope(netra_engine* engine) : e(engine) { e->in_flight.fetch_add(1, std::memory_order_acq_rel); }
  ~LaunchScope() { e->in_flight.fetch_sub(1, std::memory_order_acq_rel); }
};

hipError_t dispatch(const OpRecord& op, void** params, hipStream_t stream) {
  return hipModuleLaunchKernel(op.function, op.grid[0], op.grid[1], op.grid[2], op.block[0],
                               op.block[1], op.block[2], op.dynamic_lds_bytes, stream, params,
                               nullptr);
}

// Every operation of a profile in order, from the bound records.
netra_status_t dispatch_profile(netra_engine* e, const ProfileRecord& p, hipStream_t stream) {
  for (size_t i = 0; i < p.ops.size(); ++i) {
    const OpRecord& op = p.ops[i];
    if (op.fallback)
      return refuse(e, NETRA_STATUS_FALLBACK_REQUIRED,
                    "profile %u operation %zu is a framework-fallback operation", p.info.profile_id, i);
    const int hole = first_unbound(op);
    if (hole >= 0)
      return refuse(e, NETRA_STATUS_BINDING, "operation %zu argument %d has no pointer bound", i, hole);
    void** params = const_cast<void**>(op.params.data());
    const hipError_t err = dispatch(op, params, stream);
    if (err != hipSuccess) return hip_refusal(e, "hipModuleLaunchKernel", err);
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

  // The workspace starts zeroed (kernels that hand work between workgroups
  // keep counters there that every launch leaves at zero again).
  e->workspace_bytes = manifest.workspace_bytes;
  if (e->workspace_bytes) {
    err = hipMalloc(&e->workspace, static_cast<size_t>(e->workspace_bytes));
    if (err == hipSuccess) err = hipMemset(e->workspace, 0, static_cast<size_t>(e->workspace_bytes));
    if (err == hipSuccess) err = hipDeviceSynchronize();
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
            ++op.slot_count;
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

// bind, checks in order:
//   null engine or pointer                          INVALID_ARGUMENT
//   bindings finalized                              BUSY
//   a launch in flight                              BUSY
//   profile or operation index out of range         BINDING
//   profile already captured                        BUSY
//   argument index out of range                     BINDING
//   argument is not a caller pointer slot           BINDING
extern "C" netra_status_t netra_engine_bind(netra_engine_t* e, uint32_t profile_id,
                                            uint32_t op_index, uint32_t arg_index, void* ptr) {
  if (!e || !ptr) return NETRA_STATUS_INVALID_ARGUMENT;
  if (finalized(e)) return refuse(e, NETRA_STATUS_BUSY, "bindings are finalized and immutable");
  if (busy(e)) return refuse(e, NETRA_STATUS_BUSY, "bind refused: a launch is in progress");
  const bool indexed = profile_id < e->profiles.size() && op_index < e->profiles[profile_id].ops.size();
  if (!indexed)
    return refuse(e, NETRA_STATUS_BINDING, "bind refused: no operation %u in profile %u", op_index, profile_id);
  ProfileRecord& p = e->profiles[profile_id];
  if (p.captured)
    return refuse(e, NETRA_STATUS_BUSY, "bind refused: profile %u is captured into a graph", profile_id);
  OpRecord& op = p.ops[op_index];
  if (arg_index >= op.argument_count)
    return refuse(e, NETRA_STATUS_BINDING, "bind refused: operation %u has %u arguments, not %u", op_index,
                  op.argument_count, arg_index + 1);
  if (!op.bindable[arg_index])
    return refuse(e, NETRA_STATUS_BINDING,
                  "bind refused: argument %u of operation %u is fixed by the manifest", arg_index, op_index);
  op.pointers[arg_index] = ptr;
  return accept(e);
}

// finalize_bindings (idempotent), checks in order:
//   null engine                                     INVALID_ARGUMENT
//   a launch in flight                              BUSY
//   a kernel operation with an unbound pointer slot BINDING
extern "C" netra_status_t netra_engine_finalize_bindings(netra_engine_t* e) {
  if (!e) return NETRA_STATUS_INVALID_ARGUMENT;
  if (busy(e)) return refuse(e, NETRA_STATUS_BUSY, "finalize refused: a launch is in progress");
  for (const ProfileRecord& p : e->profiles) {
    for (size_t i = 0; i < p.ops.size(); ++i) {
      if (p.ops[i].fallback) continue;
      const int hole = first_unbound(p.ops[i]);
      if (hole >= 0)
        return refuse(e, NETRA_STATUS_BINDING,
                      "finalize refused: profile %u operation %zu argument %d has no pointer bound",
                      p.info.profile_id, i, hole);
    }
  }
  e->finalized.store(true, std::memory_order_release);
  return accept(e);
}

// prepare_profile, checks in order:
//   null engine or profile out of range             INVALID_ARGUMENT
//   capture disabled, or profile already captured   OK (nothing to do)
//   profile has a framework-fallback operation      FALLBACK_REQUIRED
//   finalize_bindings                               its status
//   capture / instantiate                           HIP, or the dispatch status
extern "C" netra_status_t netra_engine_prepare_profile(netra_engine_t* e, uint32_t profile_id,
                                                       hipStream_t stream) {
  if (!e || profile_id >= e->profiles.size()) return NETRA_STATUS_INVALID_ARGUMENT;
  ProfileRecord& p = e->profiles[profile_id];
  if (!e->graph_capture || p.captured) return NETRA_STATUS_OK;
  if (p.info.requires_fallback)
    return refuse(e, NETRA_STATUS_FALLBACK_REQUIRED,
                  "capture refused: profile %u contains a framework-fallback operation", profile_id);
  const netra_status_t bound = netra_engine_finalize_bindings(e);
  if (bound != NETRA_STATUS_OK) return bound;
  hipError_t err = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
  if (err != hipSuccess) return hip_refusal(e, "hipStreamBeginCapture", err);
  const netra_status_t recorded = dispatch_profile(e, p, stream);
  hipGraph_t graph = nullptr;
  err = hipStreamEndCapture(stream, &graph);
  if (recorded != NETRA_STATUS_OK || err != hipSuccess) {
    if (graph) (void)hipGraphDestroy(graph);
    return recorded != NETRA_STATUS_OK ? recorded : hip_refusal(e, "hipStreamEndCapture", err);
  }
  hipGraphExec_t exec = nullptr;
  err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (err != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return hip_refusal(e, "hipGraphInstantiate", err);
  }
  p.graph = graph;
  p.graph_exec = exec;
  p.captured = true;
  return accept(e);
}

// launch, checks in order:
//   null engine or shape, profile out of range      INVALID_ARGUMENT
//   current device is not the engine's              UNSUPPORTED_TARGET
//   shape outside the profile's guards              UNSUPPORTED_PROFILE
//   profile has a framework-fallback operation      FALLBACK_REQUIRED
//   not captured and bindings not finalized         BINDING
//   graph launch / kernel launch                    HIP
extern "C" netra_status_t netra_engine_launch(netra_engine_t* e, uint32_t profile_id,
                                              const netra_launch_shape_t* shape,
                                              hipStream_t stream) {
  if (!e || !shape || profile_id >= e->profiles.size()) return NETRA_STATUS_INVALID_ARGUMENT;
  const ProfileRecord& p = e->profiles[profile_id];
  const netra_status_t admitted = admit(e, p, *shape);
  if (admitted != NETRA_STATUS_OK) return admitted;
  if (p.info.requires_fallback)
    return refuse(e, NETRA_STATUS_FALLBACK_REQUIRED,
                  "launch refused: profile %u contains a framework-fallback operation", profile_id);
  if (!p.captured && !finalized(e))
    return refuse(e, NETRA_STATUS_BINDING, "launch refused: bindings are not finalized");
  LaunchScope scope(e);
  if (p.captured) {
    const hipError_t err = hipGraphLaunch(p.graph_exec, stream);
    return err == hipSuccess ? NETRA_STATUS_OK : hip_refusal(e, "hipGraphLaunch", err);
  }
  return dispatch_profile(e, p, stream);
}

// launch_operation, checks in order:
//   null engine or shape, profile/operation out of range   INVALID_ARGUMENT
//   current device is not the engine's                      UNSUPPORTED_TARGET
//   shape outside the profile's guards                      UNSUPPORTED_PROFILE
//   profile captured (single operations are closed)         BUSY
//   operation is a framework-fallback operation             FALLBACK_REQUIRED
//   bindings not finalized                                  BINDING
//   an unbound pointer slot                                 BINDING
//   kernel launch                                           HIP
extern "C" netra_status_t netra_engine_launch_operation(netra_engine_t* e, uint32_t profile_id,
                                                        uint32_t op_index,
                                                        const netra_launch_shape_t* shape,
                                                        hipStream_t stream) {
  if (!e || !shape || profile_id >= e->profiles.size() || op_index >= e->profiles[profile_id].ops.size())
    return NETRA_STATUS_INVALID_ARGUMENT;
  const ProfileRecord& p = e->profiles[profile_id];
  const netra_status_t admitted = admit(e, p, *shape);
  if (admitted != NETRA_STATUS_OK) return admitted;
  if (p.captured)
    return refuse(e, NETRA_STATUS_BUSY,
                  "launch refused: profile %u is captured; it launches only as its graph", profile_id);
  const OpRecord& op = p.ops[op_index];
  if (op.fallback)
    return refuse(e, NETRA_STATUS_FALLBACK_REQUIRED,
                  "launch refused: operation %u is a framework-fallback operation", op_index);
  if (!finalized(e)) return refuse(e, NETRA_STATUS_BINDING, "launch refused: bindings are not finalized");
  const int hole = first_unbound(op);
  if (hole >= 0)
    return refuse(e, NETRA_STATUS_BINDING, "launch refused: operation %u argument %d has no pointer bound",
                  op_index, hole);
  LaunchScope scope(e);
  const hipError_t err = dispatch(op, const_cast<void**>(op.params.data()), stream);
  return err == hipSuccess ? NETRA_STATUS_OK : hip_refusal(e, "hipModuleLaunchKernel", err);
}

// launch_operation_bound (caller-local pointers; the engine's records are not
// touched, so concurrent calls need no lock), checks in order:
//   null engine or shape, profile/operation out of range,
//   more than 16 entries, entries without an array          INVALID_ARGUMENT
//   current device is not the engine's                      UNSUPPORTED_TARGET
//   shape outside the profile's guards                      UNSUPPORTED_PROFILE
//   profile captured                                        BUSY
//   operation is a framework-fallback operation             FALLBACK_REQUIRED
//   entry count differs from the operation's pointer slots  BINDING
//   an entry with reserved != 0, a null pointer, or an
//   index that is not a pointer slot                        BINDING
//   the same slot twice                                     BINDING
//   kernel launch                                           HIP
extern "C" netra_status_t netra_engine_launch_operation_bound(
    netra_engine_t* e, uint32_t profile_id, uint32_t op_index, const netra_launch_shape_t* shape,
    const netra_pointer_binding_t* bindings, uint32_t count, hipStream_t stream) {
  constexpr uint32_t kMaxEntries = 16;
  if (!e || !shape || profile_id >= e->profiles.size() || op_index >= e->profiles[profile_id].ops.size() ||
      count > kMaxEntries || (count != 0 && bindings == nullptr))
    return NETRA_STATUS_INVALID_ARGUMENT;
  const ProfileRecord& p = e->profiles[profile_id];
  const netra_status_t admitted = admit(e, p, *shape);
  if (admitted != NETRA_STATUS_OK) return admitted;
  if (p.captured)
    return refuse(e, NETRA_STATUS_BUSY,
                  "bound launch refused: profile %u is captured; it launches only as its graph", profile_id);
  const OpRecord& op = p.ops[op_index];
  if (op.fallback)
    return refuse(e, NETRA_STATUS_FALLBACK_REQUIRED,
                  "bound launch refused: operation %u is a framework-fallback operation", op_index);
  if (count != op.slot_count)
    return refuse(e, NETRA_STATUS_BINDING, "bound launch refused: operation %u has %u pointer slots, got %u",
                  op_index, op.slot_count, count);
  // Kernel arguments on this call's stack: manifest constants and workspace
  // pointers from the record, pointer slots from the caller's entries.
  std::array<void*, netra::kMaxArguments> values{};
  std::array<void*, netra::kMaxArguments> params{};
  uint64_t supplied = 0;  // bit a: slot a has an entry (kMaxArguments <= 64)
  static_assert(netra::kMaxArguments <= 64, "slot bitmap");
  for (uint32_t i = 0; i < count; ++i) {
    const netra_pointer_binding_t& b = bindings[i];
    const uint32_t a = b.argument_index;
    if (b.reserved != 0 || b.pointer == nullptr || a >= op.argument_count || !op.bindable[a])
      return refuse(e, NETRA_STATUS_BINDING,
                    "bound launch refused: entry %u (argument %u) is not a usable pointer slot", i, a);
    if (supplied >> a & 1u)
      return refuse(e, NETRA_STATUS_BINDING, "bound launch refused: argument %u is supplied twice", a);
    supplied |= uint64_t{1} << a;
    values[a] = b.pointer;
  }
  for (uint32_t a = 0; a < op.argument_count; ++a) {
    if (op.is_scalar[a]) {
      params[a] = const_cast<uint32_t*>(&op.scalars[a]);
    } else {
      if (!op.bindable[a]) values[a] = op.pointers[a];
      params[a] = &values[a];
    }
  }
  LaunchScope scope(e);
  const hipError_t err = dispatch(op, params.data(), stream);
  return err == hipSuccess ? NETRA_STATUS_OK : hip_refusal(e, "hipModuleLaunchKernel", err);
}

extern "C" const char* netra_engine_last_error(const netra_engine_t* e) {
  return e ? e->last_error : "no engine handle";
}

// destroy: null engine is OK; a launch in flight is BUSY; otherwise every
// graph, module and the workspace are released.
extern "C" netra_status_t netra_engine_destroy(netra_engine_t* e) {
  if (!e) return NETRA_STATUS_OK;
  if (busy(e)) return refuse(e, NETRA_STATUS_BUSY, "destroy refused: a launch is in progress");
  release(e);
  delete e;
  return NETRA_STATUS_OK;
}
