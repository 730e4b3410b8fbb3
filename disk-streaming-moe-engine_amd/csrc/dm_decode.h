// dm_decode.h -- the fused single-launch decode kernel (dm_decode.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dm_layout.h"

namespace dm {

// Launch geometry and LDS carve-up, computed once per layer on the host.
struct DecodePlan {
  int grid;         // persistent workgroups (one per CU, at least H/16)
  int threads;      // workgroup size
  int lds_bytes;
  int off_xt, off_xb, off_zv, off_ev, off_sel, off_red, off_hb, off_yred;
  int n_router_wg;  // router workgroups (4 rows each)
  int ldh_log2;     // row stride of h: the power of two >= max(I, Ish)
};

// Cross-workgroup state of one layer: tagged words carry the launch index in
// their high half, so a consumer polls the data itself.
struct DecodeSync {
  uint64_t* zt;  // [256*ceil(E/256) + 64] (tag, logit); entry E = shared-expert gate
  uint64_t* ht;  // [K+1][ldh] (tag, h), ldh = 2^ldh_log2 >= max(I, Ish)
  unsigned n;    // launch index, >= 1 (the tag of this launch)
};
size_t decode_sync_bytes(const LayerDev& L);
DecodeSync decode_sync_carve(const LayerDev& L, void* base);

DecodePlan make_decode_plan(const LayerDev& L, int num_cus);
hipError_t decode_occupancy(const LayerDev& L, const DecodePlan& P, int* blocks_per_cu);
// nm.eps > 0: the router and experts see rmsnorm(x, nm.gamma, nm.eps) in the
// order nm.seq selects (NormSpec).  cooperative: launch with
// hipLaunchCooperativeKernel, which guarantees that every workgroup is
// resident (slower; for devices shared by several contexts).  status_out
// (may be NULL): P.grid words; each workgroup stores the status key there
// as it ends, and the launch's key is their minimum, so a caller waiting for
// the launch needs no separate read-back.
hipError_t launch_moe_decode(const LayerDev& L, const DecodePlan& P, const float* x,
                             const float* residual, float* y, int32_t* ids, float* probs,
                             float* shg, const DecodeSync& S, unsigned long long* status, int token,
                             hipStream_t st, const NormSpec& nm, bool cooperative,
                             unsigned long long* status_out);

}  // namespace dm
