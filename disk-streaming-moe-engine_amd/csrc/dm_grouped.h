// dm_grouped.h -- the MoE block for several tokens at once (dm_grouped.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dm_layout.h"

namespace dm {

// Upper bound of the work units for T tokens (size of the units buffer).
int group_units_max(int T, int K, int E);

// Tokens per work unit of launch_group_build: units[0 .. meta[1]) hold up to
// kUnitBig of their expert's positions, units[meta[1] .. meta[0]) up to
// kUnitSmall.  A unit is (expert, first position within the expert); the
// expert E is the shared one, whose positions are the tokens.
constexpr int kUnitBig = 128;
constexpr int kUnitSmall = 16;

// Group the T*K assignments by expert: off [E+1], perm [T*K], units, meta[0].
hipError_t launch_group_build(const int32_t* ids, int T, int K, int E, int32_t* off,
                              int32_t* perm, int2* units, int32_t* meta, hipStream_t st);

// The front end of a small batch in one launch: x -> bf16 hi / lo rows and
// need-lo (flags[0]), router logits z [T][E+1] in the layer order, softmax /
// top-k / shared gate (ids, probs, shg) and the grouping (off, perm, units,
// meta) -- the work of launch_split_rows, launch_router_dec,
// launch_router_select and launch_group_build.  flags[1 .. 2 + T) are
// arrival counters that must be zero on entry and are zero again on exit.
constexpr int kFrontMaxT = 63;
constexpr int kFrontMaxE = 512;
bool front_supported(const LayerDev& L, int T);
hipError_t launch_front(const LayerDev& L, const float* x, int T, float* z, uint16_t* xhi,
                        uint16_t* xlo, int* flags, int32_t* ids, float* probs, float* shg,
                        int32_t* off, int32_t* perm, int2* units, int32_t* meta,
                        unsigned long long* status, hipStream_t st);

// n fp32 values (n % 8 == 0) -> bf16 hi / lo; *need_lo |= 1 if a lo part is nonzero
// (the caller zeroes *need_lo first).
hipError_t launch_split_rows(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, int* need_lo,
                             hipStream_t st);

// Routed and shared experts of all units: h as bf16 hi / lo parts (hrh, hrl
// [T*K][I] by position in expert order; hsh, hsl [T][Ish]), then the down
// projections r [T*K][H] (by assignment t*K + k) and rs [T][H].
hipError_t launch_experts_grouped(const LayerDev& L, const uint16_t* xhi, const uint16_t* xlo,
                                  const int* need_lo, const int32_t* off, const int32_t* perm,
                                  const int2* units, const int32_t* meta, int T, uint16_t* hrh,
                                  uint16_t* hrl, uint16_t* hsh, uint16_t* hsl, float* r,
                                  float* rs, unsigned long long* status, hipStream_t st);

// y = sum_k p_k r_k + g rs (+ residual), per token in the reference order.
hipError_t launch_combine(const float* r, const float* rs, const float* probs, const float* shg,
                          const float* residual, int T, int H, int K, float* y,
                          unsigned long long* status, hipStream_t st, int* clear_flag = nullptr);

}  // namespace dm
