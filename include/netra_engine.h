// Netra engine C ABI for gfx950 (MI355X): load an engine directory, bind
// caller-owned device pointers, launch fixed kernels on the caller's stream.
//
// Drop-in replacement for the reference runtime header
// runtime/gfx950/engine/netra_engine.h (status codes :14-25, option/profile/
// shape/binding structs :27-58, entry points :60-108). Struct layouts, enum
// values and entry-point signatures are identical so that an existing ctypes
// or C caller binds this library unchanged. One entry point is added:
// netra_engine_manifest_check (host-only manifest validation, no counterpart
// in the reference).
#pragma once

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct netra_engine netra_engine_t;

// reference: runtime/gfx950/engine/netra_engine.h:14-25
typedef enum netra_status {
  NETRA_STATUS_OK = 0,
  NETRA_STATUS_INVALID_ARGUMENT = 1,
  NETRA_STATUS_IO = 2,
  NETRA_STATUS_MANIFEST = 3,
  NETRA_STATUS_UNSUPPORTED_TARGET = 4,
  NETRA_STATUS_UNSUPPORTED_PROFILE = 5,
  NETRA_STATUS_BINDING = 6,
  NETRA_STATUS_HIP = 7,
  NETRA_STATUS_BUSY = 8,
  NETRA_STATUS_FALLBACK_REQUIRED = 9
} netra_status_t;

// reference: netra_engine.h:27-31
typedef struct netra_engine_options {
  uint32_t struct_size;
  int32_t device_id;
  uint32_t enable_graph_capture;
} netra_engine_options_t;

// reference: netra_engine.h:33-45
typedef struct netra_profile_info {
  uint32_t struct_size;
  uint32_t profile_id;
  uint32_t min_m;
  uint32_t max_m;
  uint32_t min_batch;
  uint32_t max_batch;
  uint64_t min_sequence;
  uint64_t max_sequence;
  uint32_t tensor_parallel;
  uint64_t workspace_bytes;
  uint32_t requires_fallback;
} netra_profile_info_t;

// reference: netra_engine.h:47-52
typedef struct netra_launch_shape {
  uint32_t m;
  uint32_t batch;
  uint64_t sequence;
  uint32_t tensor_parallel;
} netra_launch_shape_t;

// reference: netra_engine.h:54-58
typedef struct netra_pointer_binding {
  uint32_t argument_index;
  uint32_t reserved;
  void* pointer;
} netra_pointer_binding_t;

// Parse <dir>/engine.json, check the device (gfx950, wave64) and the HIP
// runtime version, allocate the engine workspace and load every kernel's code
// object. Replaces netra_engine_create (reference netra_engine.h:60-62).
netra_status_t netra_engine_create(const char* engine_directory,
                                   const netra_engine_options_t* options,
                                   netra_engine_t** output);
// reference: netra_engine.h:63
size_t netra_engine_profile_count(const netra_engine_t* engine);
// reference: netra_engine.h:64-66
netra_status_t netra_engine_query_profile(const netra_engine_t* engine,
                                          uint32_t profile_id,
                                          netra_profile_info_t* output);
// Bind one pointer slot (profile, operation, argument). Initialisation-phase
// only; not thread-safe with launch. reference: netra_engine.h:68-72
netra_status_t netra_engine_bind(netra_engine_t* engine, uint32_t profile_id,
                                 uint32_t operation_index,
                                 uint32_t argument_index, void* pointer);
// End of the binding phase; every pointer slot must be bound.
// reference: netra_engine.h:74-76
netra_status_t netra_engine_finalize_bindings(netra_engine_t* engine);
// Capture the profile's launches into a HIP graph (when graph capture is
// enabled). reference: netra_engine.h:78-82
netra_status_t netra_engine_prepare_profile(netra_engine_t* engine,
                                            uint32_t profile_id,
                                            hipStream_t stream);
// Guard check, then graph replay or direct launches on caller_stream.
// No allocation, parsing, synchronisation or file access. reference: :84-87
netra_status_t netra_engine_launch(netra_engine_t* engine,
                                   uint32_t profile_id,
                                   const netra_launch_shape_t* shape,
                                   hipStream_t caller_stream);
// Launch one operation of a profile. reference: netra_engine.h:89-93
netra_status_t netra_engine_launch_operation(
    netra_engine_t* engine, uint32_t profile_id, uint32_t operation_index,
    const netra_launch_shape_t* shape, hipStream_t caller_stream);
// Launch one operation with caller-local pointers for every pointer slot
// (at most 16). reference: netra_engine.h:95-103
netra_status_t netra_engine_launch_operation_bound(
    netra_engine_t* engine, uint32_t profile_id, uint32_t operation_index,
    const netra_launch_shape_t* shape,
    const netra_pointer_binding_t* bindings, uint32_t binding_count,
    hipStream_t caller_stream);
// reference: netra_engine.h:104
const char* netra_engine_last_error(const netra_engine_t* engine);
// Returns BUSY while a launch call is in progress. reference: :106-108
netra_status_t netra_engine_destroy(netra_engine_t* engine);

// Host-only validation of <dir>/engine.json: the same parsing and checks as
// netra_engine_create up to (excluding) device, workspace and module work.
// Writes a message into error (if non-null) on failure. No counterpart in the
// reference; it lets the manifest contract be tested on machines without a GPU.
netra_status_t netra_engine_manifest_check(const char* engine_directory,
                                           char* error, size_t error_size);

#ifdef __cplusplus
}
#endif
