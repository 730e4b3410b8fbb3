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
  // XCD-sliced form (xs != 0): the grid is spread over xs_nx XCDs in
  // rotation, num_cus / xs_nx workgroups on each.  The
  // expert work is cut into pairs (slot, 128-row slice of I); XCD x owns the
  // pairs p = x, x + nx, ...: their gate/up tiles and the matching 128
  // columns of their down matrices, so h never leaves the XCD.  Each XCD
  // publishes one partial output vector; the partials are summed at the end.
  int xs;
  int xs_nx;    // XCDs
  int xs_rpw;   // 16-row output tiles of the down partial per workgroup (1, 2, 4 or 8)
  int xs_rpf;   // output rows per workgroup in the final sum
  int xs_npx;   // most pairs on one XCD
  int xs_nrw;   // waves per workgroup holding router rows (each XCD forms all logits)
  int off_fin;  // LDS: the final sum's gathered partials
  // Several tokens in one launch (tok != 0, on top of the XCD-sliced form):
  // token t on XCD t % nx, its whole block on that XCD's workgroups
  // (launch_moe_tokens).  LDS: the sliced form's carve-up up to off_hb, then
  // every pair's h (bf16 hi / lo) and the down tile's reduction.
  int tok;
  int tok_off_hb, tok_off_yred, tok_off_ring, tok_lds_bytes;
};

// Most tokens of one launch_moe_tokens launch (and at most the XCD count),
// and the most LDS it may take (one workgroup per CU).
constexpr int kTokMaxT = 8;
constexpr int kTokMaxLds = 150 * 1024;

// Cross-workgroup state of one layer: tagged words carry the launch index in
// their high half, so a consumer polls the data itself.
struct DecodeSync {
  uint64_t* zt;  // [256*ceil(E/256) + 64] (tag, logit); entry E = shared-expert gate
                 // (XCD-sliced form: one such vector per XCD)
  uint64_t* ht;  // [K+1][ldh] (tag, h), ldh = 2^ldh_log2 >= max(I, Ish)
  uint64_t* hl;  // XCD-sliced form: [pairs][64] packed h words (pack_h2), XCD-local
  uint64_t* pt;  // XCD-sliced form: [nx][H] (tag, partial output)
  uint64_t* htk; // several-token form: [kTokMaxT][pairs][128] (tag, h), XCD-local
  unsigned n;    // launch index, >= 1 (the tag of this launch)
  long spin;     // polls of a wait before it gives up with a sync error
  int trace;     // phase-trace slot of the launch (the layer), -1: none; read only by
                 // a tracing build (DM_PHASE_TRACE, `make trace`)
};
// Tracing build: phase timestamps of k_moe_decode_xs, kTraceSlots slots
// (layers) x 256 workgroups x 8 points (wall_clock64, 100 MHz), fetched by
// the extern "C" dmh_phase_trace_fetch of libdismoen_hip_trace.so.
constexpr int kTraceSlots = 64;
constexpr int kTracePoints = 8;
size_t decode_sync_bytes(const LayerDev& L, const DecodePlan& P);
DecodeSync decode_sync_carve(const LayerDev& L, const DecodePlan& P, void* base);

// nx > 0: the XCD count, when the workgroups b of a num_cus grid were seen
// on XCD (b + r) % nx for one r (probed on the device); then the XCD-sliced
// form is planned
// where the layer's shape allows it.  nx = 0: the original form only.
DecodePlan make_decode_plan(const LayerDev& L, int num_cus, int nx = 0);
// Launches one workgroup per CU that records the XCD it runs on; *nx = the
// XCD count when the workgroups were placed on the XCDs in rotation, else 0.
hipError_t probe_xcd_map(int num_cus, int* nx);
// The decision of probe_xcd_map on a recorded placement (xcd[b] = the XCD
// workgroup b ran on): the XCD count n when xcd[b] = (b + r) % n for
// one r and n divides nwg, else 0.
int xcd_rotation(const unsigned* xcd, int nwg);
hipError_t decode_occupancy(const LayerDev& L, const DecodePlan& P, int* blocks_per_cu);
// T tokens (2 <= T <= min(kTokMaxT, P.xs_nx), P.tok) in one launch of the
// XCD-sliced grid: token t's routing, experts and combine on XCD t % nx
// (every hand-off stays in that XCD's L2, nothing is summed across XCDs).
// x, residual, y: [T][H]; ids, probs: [T][K]; shg: [T].  No norm.
hipError_t launch_moe_tokens(const LayerDev& L, const DecodePlan& P, const float* x, int T,
                             const float* residual, float* y, int32_t* ids, float* probs,
                             float* shg, const DecodeSync& S, unsigned long long* status,
                             hipStream_t st, bool cooperative);
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
