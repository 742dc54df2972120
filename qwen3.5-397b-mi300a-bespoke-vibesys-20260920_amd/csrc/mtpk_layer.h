// Launch helpers of the fused MoE layer (`mtpk_moe_layer`), shared between the translation units
// that own the kernels: the router + shared gate_up GEMM tiles (mtpk_gemm.hip), the routing from
// split-K partials with the shared expert's SiLU product (mtpk_router.hip), and the routed expert
// launches that also run the shared down GEMM's tiles (mtpk_moe.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mtpk {

struct GemmArgs;

struct RouteActArgs {
  const float* rpart;  // router partials [rks, rows, rcols] (rcols = E + 1: the experts, then the shared gate)
  int rks, rows, rcols, E, top_k;
  float* top_w;    // [rows, top_k]
  void* top_i;     // [rows, top_k], dtype idt
  int idt;
  uint16_t* sgate;     // bf16 [rows]: column E of the router output, or null
  const float* spart;  // shared gate_up partials [sks, rows, 2 scols]
  int sks, scols;
  uint16_t* act;  // bf16 [rows, scols]
  int route_blocks;  // set by the launcher
};

// One launch of two GEMMs over the same token rows, both leaving fp32 partials (`part` set): the
// tiles of `first`, then those of `second`. Both take the same token rows (M), hence the same
// token tiles and row groups; `first` has no SiLU epilogue, `second` has it.
int launch_gemm_pair(const GemmArgs& first, const GemmArgs& second, hipStream_t st);

int launch_route_act(const RouteActArgs& a, hipStream_t st);

}  // namespace mtpk
