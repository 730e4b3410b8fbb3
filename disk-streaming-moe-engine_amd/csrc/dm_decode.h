// dm_decode.h -- the fused single-launch decode kernel (dm_decode.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dm_layout.h"

namespace dm {

// Launch geometry and LDS carve-up, computed once per layer on the host.
struct DecodePlan {
  int grid;         // persistent workgroups (one per CU, at least 2*H/16)
  int lds_bytes;
  int off_xs, off_xb, off_pv, off_sel, off_red, off_hb, off_redd;
  int n_router_wg;  // ceil((E+1)/16) router workgroups
  int s0;           // down halves: slots [0, s0) and [s0, K+1)
  int ldh;          // row stride of h (max(I, Ish))
};

// Cross-workgroup state of one context; counters only grow (launch n waits
// for n times the arrivals of one launch).
struct DecodeSync {
  unsigned* cnt_router;  // [1]
  unsigned* cnt_h;       // [K+1]
  unsigned* cnt_y;       // [H/16]
  float* z;              // [E+1] logits
  float* h;              // [K+1][ldh]
  float* ypart;          // [2][H]
  unsigned n;            // launch index, >= 1
};

DecodePlan make_decode_plan(const LayerDev& L, int num_cus);
hipError_t decode_occupancy(const LayerDev& L, const DecodePlan& P, int* blocks_per_cu);
hipError_t launch_moe_decode(const LayerDev& L, const DecodePlan& P, const float* x,
                             const float* residual, float* y, int32_t* ids, float* probs,
                             float* shg, const DecodeSync& S, unsigned long long* status, int token,
                             hipStream_t st);

}  // namespace dm
