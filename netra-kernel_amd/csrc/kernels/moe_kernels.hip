// FP8 E4M3 block-scaled routed-MoE kernels for gfx950 (CDNA4, wave64), built
// into one code object (netra_moe_gfx950.hsaco) that the engine loads.
//
// Layer pipeline, one engine operation per kernel, fixed grids with
// device-side early exit so a whole layer call is one capturable HIP graph:
//   front end, exact:  router (logits + input quant) -> topk -> sort
//   front end, screen: route_screen -> route_select -> sort_route
//   then gate_up_{stream|lds|tile} -> down_{stream|tile} -> combine
// Every kernel takes plain pointers followed by u32 shape constants, in the
// order documented in include/netra_moe.h. moe_bridge_kernels.hip adds the
// kernels behind the reference's per-operation bridge ABIs
// (include/netra_qwen36_bridges.h). Host code validates shapes before
// a launch; kernels also bound-check data-dependent indices (expert ids,
// sorted positions) so malformed routing cannot address memory outside the
// buffers the shapes describe.
#include "moe_router.hip"
#include "moe_route_prefill.hip"
#include "moe_gemm_stream.hip"
#include "moe_ffn_decode.hip"
#include "moe_gemm_tile.hip"
#include "moe_gemm_lds.hip"
#include "moe_misc.hip"
#include "moe_bridge_kernels.hip"
