// dm_kernels.h -- host-side launchers for the kernels in dm_kernels.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dm_layout.h"

namespace dm {

// ---- upload-time re-tiling and validation ----
// nmat matrices [R][C] in the reference 4-bit layout with source group size
// gsrc (32, 64, 128 or 256) -> A16 with one scale per 32 columns.  Invalid
// scales or reserved codes record (tensor << 34 | sub) into *vkey (atomicMin).
hipError_t launch_repack_a16(const uint8_t* src_nib, const uint16_t* src_sc, uint8_t* dst_nib,
                             uint16_t* dst_sc, int R, int C, int nmat, int tensor_base, int gsrc,
                             unsigned long long* vkey, hipStream_t st);
// router [E][H] bf16 + shared gate [H] bf16 -> R16 (E+1 rows).  Non-finite
// router weights set bit 0 of *flags.
hipError_t launch_repack_router(const uint16_t* router, const uint16_t* shgate, uint16_t* dst,
                                int E, int H, unsigned* flags, hipStream_t st);

// ---- unit entry points ----
hipError_t launch_dequant_ref(const uint16_t* scales, const uint8_t* packed, int64_t n,
                              int group, uint16_t* out, unsigned long long* vkey,
                              hipStream_t st);
// z[T][E] (z[T][E + 1] with the shared-expert gate row w_sh as column E)
hipError_t launch_router_generic(const float* x, const float* w, int T, int H, int E, float* z,
                                 unsigned long long* status, hipStream_t st,
                                 const float* w_sh = nullptr);

// The same logits (z[T][E + 1], column E the shared gate) for T >= 8 tokens
// from the chain-ordered fp32 copy of a GGUF layer's router and shared gate
// (rows of rs floats, launch_chain_router), four tokens per pass over each
// lane's chain held in registers; H / 64 in {8, 16, 32}.
bool router_rows_f32_ok(int T, int H, int E, int rs);
hipError_t launch_router_rows_f32(const float* x, const float* rchain, int rs, int T, int H, int E,
                                  float* z, unsigned long long* status, hipStream_t st);

// ---- decode path (one token per launch set) ----
hipError_t launch_router_dec(const LayerDev& L, const float* x, int T, float* z,
                             unsigned long long* status, hipStream_t st,
                             const int* gate = nullptr);
// Many tokens whose activations are bf16 values (*need_lo == 0): logits of
// all E experts and the shared gate, z [T][E+1], on the matrix cores.
hipError_t launch_router_mfma(const LayerDev& L, const uint16_t* xhi, const int* need_lo, int T,
                              float* z, hipStream_t st);
hipError_t launch_router_select(const float* z, int ldz, int T, int E, int K, int has_sh,
                                int32_t* ids, float* probs, float* shg,
                                unsigned long long* status, hipStream_t st);
hipError_t launch_gateup_dec(const LayerDev& L, const float* x, const int32_t* ids, float* h,
                             int ldh, int token, unsigned long long* status, hipStream_t st);
hipError_t launch_down_dec(const LayerDev& L, const float* h, int ldh, const int32_t* ids,
                           const float* probs, const float* shg, const float* residual,
                           float* y, int token, unsigned long long* status, hipStream_t st);

// Shared-expert gate scores from gate logits z[t] (ldz apart):
// sigmoid(z) with the checks of shared_gate_forward (src/layers/moe.mojo:83-100).
hipError_t launch_shared_gate_scores(const float* z, int ldz, int T, float* scores,
                                     unsigned long long* status, hipStream_t st);
// Expert ids [T][K] checked against [0, E): out-of-range entries are recorded
// (kPhExpert, kEkBadId, the id's low 28 bits as the position) and replaced by
// expert 0 in the copy out.
hipError_t launch_check_ids(const int32_t* ids, int T, int K, int E, int32_t* out,
                            unsigned long long* status, hipStream_t st);

// ---- glue ----
// p[0..n) = v (a kernel, so that it can be captured into a graph).
hipError_t launch_fill_i32(int32_t* p, int n, int32_t v, hipStream_t st);
// rmsnorm of T rows [T][H] (H <= 8192) into out, in the order nm.seq selects.
hipError_t launch_rmsnorm_rows(const float* x, int T, int H, const NormSpec& nm, float* out,
                               hipStream_t st);

}  // namespace dm
