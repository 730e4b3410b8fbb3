// dm_device.h -- gfx950 device helpers shared by the MoE kernels.
//
// The library is compiled with -ffp-contract=off: every multiply and add in
// this file rounds on its own unless written as an explicit fused
// multiply-add, which keeps the router, softmax and gate arithmetic
// bit-identical to the CPU restatement of the reference.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dm_layout.h"

namespace dm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ bool finite_f(float v) { return (f2u(v) & 0x7F800000u) != 0x7F800000u; }
__device__ __forceinline__ float bf16lo(uint32_t w) { return u2f(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return u2f(w & 0xFFFF0000u); }

// exp(x): Cody & Waite reduction x = k*ln2 + r with a 15-bit ln2 head, the
// degree-7 Taylor polynomial of exp(r) in Horner form with fused
// multiply-adds, and scaling by 2^k through the exponent field.  The CPU
// oracle evaluates the same operation sequence.
__device__ __forceinline__ float dm_expf(float x) {
  // branch-free form of the same operation sequence: the polynomial path is
  // evaluated on a clamped argument and the out-of-range cases are selected
  const bool nan = x != x, over = x > 0x1.62e43p+6f, under = x < -0x1.9fe36ap+6f;
  const float xc = (nan || over || under) ? 0.0f : x;
  const float kf = __builtin_rintf(xc * 0x1.715476p+0f);
  float r = __builtin_fmaf(kf, -0x1.62e4p-1f, xc);
  r = __builtin_fmaf(kf, -0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0x1p-1f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int k = (int)kf;
  const bool hi = k > 127;
  p = hi ? p * 0x1p127f : p;
  k = hi ? k - 127 : k;
  const bool sub = k < -126;
  const float s1 = u2f((uint32_t)((sub ? k + 227 : k + 127) & 0xFF) << 23);
  float res = p * s1;
  res = sub ? res * 0x1p-100f : res;
  res = over ? __builtin_inff() : res;
  res = under ? 0.0f : res;
  return nan ? x : res;
}

// sigmoid_f32 / silu_f32 of src/layers/swiglu.mojo:11-38.  Both branches of
// the reference share e = exp(-|z|): for z < 0 it is exp(z) and the result
// e / (1 + e), otherwise exp(-z) and 1 / (1 + e).  One exponential and one
// division per value, the special cases selected, so that lanes of a wave on
// different branches do not each run both.
__device__ __forceinline__ float dm_sigmoid(float z) {
  const float e = dm_expf(-__builtin_fabsf(z));
  const float r = (z < 0.0f ? e : 1.0f) / (1.0f + e);
  return z != z ? z : z < -88.0f ? 0.0f : z > 88.0f ? 1.0f : r;
}
__device__ __forceinline__ float dm_silu(float z) {
  const float s = z * dm_sigmoid(z);
  return z != z ? z : !finite_f(z) ? (z > 0.0f ? z : 0.0f) : s;
}

// Wavefront-wide maxima from the ROCm device library (ockl).
extern "C" __device__ __attribute__((const)) unsigned int __ockl_wfred_max_u32(unsigned int);
extern "C" __device__ __attribute__((const)) float __ockl_wfred_max_f32(float);

// Round-to-nearest-even fp32 -> bf16 pair packed as (lo, hi).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Split eight fp32 activations into bf16 hi and lo parts (x ~= hi + lo with
// a relative error below 2^-17), packed as MFMA B-operand lanes.
__device__ __forceinline__ void split8(const float* v, uint4& hi, uint4& lo) {
  float h[8], l[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t hb = pack_bf16x2(v[i], 0.0f) & 0xFFFFu;
    h[i] = u2f(hb << 16);
    l[i] = v[i] - h[i];
  }
  hi = make_uint4(pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3]), pack_bf16x2(h[4], h[5]),
                  pack_bf16x2(h[6], h[7]));
  lo = make_uint4(pack_bf16x2(l[0], l[1]), pack_bf16x2(l[2], l[3]), pack_bf16x2(l[4], l[5]),
                  pack_bf16x2(l[6], l[7]));
}

// Dequantise one A16 word (8 codes of one group, one lane) to the bf16
// A-operand: w = bf16_rne(fp32(s) * q), as src/quant/dequant_kernel.mojo:110-115.
// The half 0x6400|u is 1024+u exactly, and fma(1024+u, s, -1032*s) equals
// s*(u-8) = s*q exactly (both products fit the fp32 significand), so the
// only rounding is the final bf16 RNE.
// (a & m) | o in one instruction: the compiler otherwise emits two, since a
// VOP3 operand cannot be a 32-bit literal on this target.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
  uint32_t d;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(m), "v"(o));
  return d;
}

__device__ __forceinline__ bf16x8 dequant8(uint32_t w, float s) {
  const uint32_t M = 0x000F000Fu, O = 0x64006400u;
  float c0 = -1032.0f * s;
  uint32_t r[4] = {and_or(w, M, O), and_or(w >> 4, M, O), and_or(w >> 8, M, O),
                   and_or(w >> 12, M, O)};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    half2v h = __builtin_bit_cast(half2v, r[i]);
    float a = __builtin_fmaf((float)h.x, s, c0);
    float b = __builtin_fmaf((float)h.y, s, c0);
    o[i] = pack_bf16x2(a, b);
  }
  uint4 v = make_uint4(o[0], o[1], o[2], o[3]);
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ float fp16_bits_to_f32(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Record a first-error key (integer atomic: order independent).
__device__ __forceinline__ void record_err(unsigned long long* status, uint64_t key) {
  atomicMin(status, (unsigned long long)key);
}

// ---- cross-workgroup handoff inside one launch -----------------------------
// Data handed between workgroups is written and read with agent-scope relaxed
// atomics: they go to the device-coherent level and bypass the per-XCD L2,
// so no cache write-back / invalidate fences are needed.  A producer writes
// its data, waits for the stores to complete, then bumps a counter; a
// consumer polls the counter, then reads the data.
__device__ __forceinline__ void st_coh(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_coh_u32(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_coh_u64(const void* p) {
  return __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<void*>(p)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh_u64(void* p, uint64_t v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A plain store (no cache-control bits): it lands in the L2 of the XCD the
// workgroup runs on, where agent-scope loads (ld_coh_u64) of workgroups on
// the same XCD see it; workgroups on other XCDs do not see it before the
// kernel ends.  For hand-offs whose producer and consumers share an XCD.
__device__ __forceinline__ void st_l2_u64(void* p, uint64_t v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_WAVEFRONT);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Every vector memory operation of this wave (loads and stores) complete.
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---- wave-wide reductions with DPP (row shifts, then row broadcasts) --------
// The result is exact for max/min (order independent), read from lane 63.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false));
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  const int id = -1;
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x111, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x112, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x114, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x118, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x142, 0xA, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x143, 0xC, 0xF, false));
  return __builtin_amdgcn_readlane(v, 63);
}
// max of floats via the order-preserving map of IEEE bits to unsigned
__device__ __forceinline__ uint32_t f2key(float f) {
  const uint32_t u = f2u(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
  return u2f((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Bounded poll until *c reaches target (wrap-safe).  About one second at the
// limit; on timeout records a sync error and returns false so that the
// caller skips later waits and the grid always drains.
constexpr long kSpinLimit = 1l << 20;
__device__ __forceinline__ bool wait_count(const unsigned* c, unsigned target,
                                           unsigned long long* status) {
  for (long i = 0; i < kSpinLimit; ++i) {
    if ((int)(ld_coh_u32(c) - target) >= 0) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  record_err(status, err_key(kPhSync, 0, 0, 0, 0));
  return false;
}

// The softmax normaliser, summed sequentially in expert order
// (src/layers/router.mojo:160-170), read from LDS in batches of 64 values.
__device__ __forceinline__ float seq_sum(const float* v, int n) {
  float s = 0.0f;
  const float4* v4 = reinterpret_cast<const float4*>(v);
  const int n4 = n >> 2;
  for (int b0 = 0; b0 < n4; b0 += 16) {
    float4 t[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) t[u] = b0 + u < n4 ? v4[b0 + u] : make_float4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (b0 + u < n4) {
        s = s + t[u].x;
        s = s + t[u].y;
        s = s + t[u].z;
        s = s + t[u].w;
      }
    }
  }
  for (int e = n4 * 4; e < n; ++e) s = s + v[e];
  return s;
}

// ---- A16 tile access ------------------------------------------------------
struct ExpertView {
  const uint8_t* nib;   // A16 matrix
  const uint16_t* sc;
  int rows, cols;
};

__device__ __forceinline__ void load_chunk(const ExpertView& v, int rb, int gq, int lane,
                                           uint4& w, uint2& s) {
  const int nGQ = v.cols / kQuadCols;
  w = *reinterpret_cast<const uint4*>(v.nib + a16_nib_offset(nGQ, rb, gq, lane));
  s = *reinterpret_cast<const uint2*>(v.sc + a16_sc_offset(nGQ, rb, gq, lane & 15));
}

// The same with non-temporal loads: for weights read once per use (routed
// experts), so that they do not evict data reused across launches from L2.
__device__ __forceinline__ void load_chunk_nt(const ExpertView& v, int rb, int gq, int lane,
                                              uint4& w, uint2& s) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const int nGQ = v.cols / kQuadCols;
  const u32x4 a = __builtin_nontemporal_load(
      reinterpret_cast<const u32x4*>(v.nib + a16_nib_offset(nGQ, rb, gq, lane)));
  const u32x2 c = __builtin_nontemporal_load(
      reinterpret_cast<const u32x2*>(v.sc + a16_sc_offset(nGQ, rb, gq, lane & 15)));
  w = make_uint4(a.x, a.y, a.z, a.w);
  s = make_uint2(c.x, c.y);
}

__device__ __forceinline__ float scale_of(const uint2& s, int c) {
  const uint32_t word = c < 2 ? s.x : s.y;
  return fp16_bits_to_f32((c & 1) ? (word >> 16) : (word & 0xFFFFu));
}

__device__ __forceinline__ uint32_t word_of(const uint4& w, int c) {
  return c == 0 ? w.x : c == 1 ? w.y : c == 2 ? w.z : w.w;
}

// Stage an fp32 vector v[n] (n % 32 == 0) as B-operand blocks in LDS:
// blk[(g*4 + q)*3 + {0: hi, 1: lo, 2: zero}] holds columns 32g+8q..+7.
__device__ __forceinline__ void stage_split(const float* __restrict__ v, int n, uint4* blk) {
  for (int i = threadIdx.x; i < n / 8; i += blockDim.x) {
    float f[8];
    const float4 a = reinterpret_cast<const float4*>(v)[2 * i];
    const float4 b = reinterpret_cast<const float4*>(v)[2 * i + 1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    uint4 hi, lo;
    split8(f, hi, lo);
    blk[3 * i + 0] = hi;
    blk[3 * i + 1] = lo;
    blk[3 * i + 2] = make_uint4(0, 0, 0, 0);
  }
}

// Columns 0 (hi) + 1 (lo) of an MFMA accumulator: after the exchange, lanes
// with (lane & 15) == 0 hold rows 4*(lane>>4) + i.
__device__ __forceinline__ void fold_cols(f32x4& acc) {
  // quad_perm [1,0,3,2]: lane l reads lane l^1
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = acc[i];
    const float o = __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    acc[i] = v + o;
  }
}

}  // namespace dm
