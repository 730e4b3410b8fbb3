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
// SiLU of the experts' hidden values, z / (1 + e^-z), from the hardware's
// exp2 and reciprocal (v_exp_f32, v_rcp_f32: about 2 ulp in all, where the
// expert outputs are held to 1e-3 of their RMS): 7 instructions instead of
// the 30-odd of z * dm_sigmoid(z) with its bit-exact exp and IEEE divide,
// which made the SiLU half of the prefill gate/up epilogue.  Finite z gives
// a finite value of the reference's sign (z < -88.7: -0, as z * 0); NaN ->
// NaN, +inf -> +inf, -inf -> 0 as the reference's silu(z) = z * sigmoid(z)
// (src/layers/swiglu.mojo).
__device__ __forceinline__ float dm_silu(float z) {
  const float e = __builtin_amdgcn_exp2f(z * -0x1.715476p+0f);  // e^-z; +inf for z < -88.7
  const float s = z * __builtin_amdgcn_rcpf(1.0f + e);         // rcp(inf) = 0
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

// The same weights from four shifted copies of the word (two instructions
// more per 8 weights).  The one-token fused kernels keep this form for their
// gate/up tiles: the XCD-sliced kernel's step measured 13.4 us with it
// against 14.0 us with dequant8 below there (dequant8 in its down operands:
// 13.35 against 13.39 us).
__device__ __forceinline__ bf16x8 dequant8_shifted(uint32_t w, float s) {
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

// The codes at bits 4-7 of each half are taken where they lie: the half
// 0x5400|(u<<4) is 64+u exactly (exponent 6, mantissa step 1/16), and
// fma(64+u, s, -72*s) = s*q as exactly; only nibble pairs 2 and 3 need a
// shift.  Both offsets -1032*s and -72*s are exact (the fp32 significand
// holds them), each one instruction on the fp16 scale.
__device__ __forceinline__ bf16x8 dequant8(uint32_t w, float s) {
  const uint32_t M0 = 0x000F000Fu, M1 = 0x00F000F0u;
  const uint32_t O0 = 0x64006400u, O1 = 0x54005400u;
  const float c0 = __builtin_fmaf(s, -1032.0f, 0.0f);
  const float c1 = __builtin_fmaf(s, -72.0f, 0.0f);
  const uint32_t w8 = w >> 8;
  uint32_t r[4] = {and_or(w, M0, O0), and_or(w, M1, O1), and_or(w8, M0, O0), and_or(w8, M1, O1)};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    half2v h = __builtin_bit_cast(half2v, r[i]);
    const float c = (i & 1) ? c1 : c0;
    float a = __builtin_fmaf((float)h.x, s, c);
    float b = __builtin_fmaf((float)h.y, s, c);
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

// 16 bytes per lane from p to the LDS byte address m + 16 * lane (m uniform),
// without passing through registers (global_load_lds_dwordx4).  Issued as
// inline assembly: the caller counts these loads itself (s_waitcnt vmcnt); a
// load the compiler tracks is only ever waited for longer because of them.
// M0 (the LDS address) is saved and restored around the load.
__device__ __forceinline__ void dma16_lds(const void* p, uint32_t m) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(p), "s"(__builtin_amdgcn_readfirstlane(m))
      : "memory");
}
// The LDS byte address of a __shared__ object: the low word of its generic
// address (the shared aperture's base is a multiple of 2^32).
__device__ __forceinline__ uint32_t lds_u32(const void* p) { return (uint32_t)(uintptr_t)p; }

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
__device__ __forceinline__ void st_coh_i32(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_coh_i32(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Polls between kernels' workgroups are bounded (kDefaultSpinLimit polls
// unless the context sets another bound), then the caller records a sync
// error and goes on, so that the grid always drains.  The bound is a launch
// argument: a context can lower it so that waits give up early (the tests of
// the time-out path).

// The softmax normaliser, summed sequentially in expert order
// (src/layers/router.mojo:160-170), read from LDS in batches of 64 values.
__device__ __forceinline__ float seq_sum(const float* v, int n) {
  float s = 0.0f;
  const float4* v4 = reinterpret_cast<const float4*>(v);
  const int n32 = n & ~31;
  for (int k = 0; k < n32 / 4; k += 8) {  // eight float4 read ahead of their adds
    float4 t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = v4[k + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      s = s + t[u].x;
      s = s + t[u].y;
      s = s + t[u].z;
      s = s + t[u].w;
    }
  }
  for (int e = n32; e < n; ++e) s = s + v[e];
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

// One step of a wave-wide top-8 reduction: every lane holds 8 keys in
// descending order; it takes the 8 keys of the lane the DPP control names
// (in reverse order), keeps the elementwise maxima (a bitonic sequence that
// holds the 8 largest of the 16) and sorts them with a bitonic network.
// Lanes without a source lane take zeros (no keys).  The shift and row
// broadcast controls of the usual reduction leave the top 8 of all lanes in
// lane 63.
template <int CTRL, int RM>
__device__ __forceinline__ void top8_step(uint32_t (&a)[8]) {
  uint32_t c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t bv = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a[7 - i], CTRL, RM, 0xF, false);
    c[i] = a[i] > bv ? a[i] : bv;
  }
  auto cx = [](uint32_t& p, uint32_t& q) {  // p >= q afterwards
    const uint32_t hi = p > q ? p : q, lo = p > q ? q : p;
    p = hi;
    q = lo;
  };
#pragma unroll
  for (int i = 0; i < 4; ++i) cx(c[i], c[i + 4]);
  cx(c[0], c[2]);
  cx(c[1], c[3]);
  cx(c[4], c[6]);
  cx(c[5], c[7]);
#pragma unroll
  for (int i = 0; i < 8; i += 2) cx(c[i], c[i + 1]);
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = c[i];
}

// ---- top-k on tagged logits (shared by the decode and GGUF kernels) ----------
// One selection round set over NK keys per lane (lane l owns experts
// l + 64 i, i < NK): `rounds` times take the largest remaining key, the
// lowest id on equal keys (lowest i first, then lowest lane).  Winners go to ids[].
// Returns the key of each round through kr (kr[0] = first, kr[1] = last,
// kr[2] = the best key left after `rounds` rounds when want_next).
template <int NK>
__device__ __forceinline__ void select_keys(const uint32_t (&key)[NK], int rounds, int E,
                                            int* ids, bool want_next, uint32_t (&kr)[3]) {
  const int lane = threadIdx.x & 63;
  uint32_t taken = 0;
  kr[0] = kr[1] = kr[2] = 0;
  for (int it = 0; it <= rounds; ++it) {
    uint32_t lm = 0;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const uint32_t kv = (taken >> i & 1u) ? 0u : key[i];
      lm = kv > lm ? kv : lm;
    }
    const uint32_t gm = wave_max_u32(lm);
    if (it == rounds) {
      kr[2] = gm;
      break;
    }
    if (it == 0) kr[0] = gm;
    kr[1] = gm;
    int wi = -1, wl = 0;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const uint64_t mk = __builtin_amdgcn_ballot_w64(!(taken >> i & 1u) && key[i] == gm);
      if (wi < 0 && mk) {
        wi = i;
        wl = (int)__builtin_ctzll(mk);
      }
    }
    if (wi < 0) wi = 0;
    if (lane == wl) taken |= 1u << wi;
    if (lane == 0) {
      const int e = 64 * wi + wl;
      ids[it] = e < E ? e : E - 1;
    }
    if (!want_next && it == rounds - 1) break;
  }
}

template <int R>
__device__ __forceinline__ void issue_logits(const uint64_t* zt, int E, bool gate,
                                             uint64_t (&v)[4 * R + 1]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 4 * R; ++i) v[i] = ld_coh_u64(zt + min(lane + 64 * i, E - 1));
  v[4 * R] = gate ? ld_coh_u64(zt + E) : 0;
}
template <int R>
__device__ __forceinline__ bool logits_ready(const uint64_t (&v)[4 * R + 1], unsigned tag, int E,
                                             bool gate, float (&z)[4 * R], float* gl) {
  const int lane = threadIdx.x & 63;
  bool ready = true;
#pragma unroll
  for (int i = 0; i < 4 * R; ++i) {
    z[i] = 0.0f;
    if (lane + 64 * i < E) {
      z[i] = u2f((uint32_t)v[i]);
      ready &= (uint32_t)(v[i] >> 32) == tag;
    }
  }
  if (gate && lane == 0) {
    *gl = u2f((uint32_t)v[4 * R]);
    ready &= (uint32_t)(v[4 * R] >> 32) == tag;
  }
  return __builtin_amdgcn_ballot_w64(!ready) == 0;
}

// Poll the tagged logits until every entry carries this launch's tag.  Lane
// l holds experts l + 64 i (coalesced loads); lane 0 also the shared-gate
// logit (entry E) when gl is given.  One poll in flight at a time: loads
// left in flight would stall the first later reuse of their registers.
// Returns false after lim polls.
template <int R>
__device__ __forceinline__ bool poll_logits(const uint64_t* zt, unsigned tag, int E, float (&z)[4 * R],
                                            float* gl, long lim) {
  const bool gate = gl != nullptr;
  uint64_t v[4 * R + 1];
  for (long spin = 0; spin < lim; ++spin) {
    issue_logits<R>(zt, E, gate, v);
    if (logits_ready<R>(v, tag, E, gate, z, gl)) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// A workgroup barrier for data passed through LDS only.  __syncthreads()
// is a release and acquire at workgroup scope, and its release waits for
// every global load the wave has in flight (s_waitcnt vmcnt(0)): for waves
// holding cold weight loads that is microseconds.  Here each wave waits only
// for its own LDS operations, so LDS written by any wave before the barrier
// is visible to every wave after it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Top-K of one token's router logits on one wave, the selection step of
// router_forward (src/layers/router.mojo:188-210 with select_topk of
// src/layers/topk.mojo:79-128) done on the logits: lane l holds z[i] of
// expert l + 64 i (i < 4R; entries past E are never selected).  Unique
// 32-bit keys (the high bits of the logit's order key, then the inverted
// expert id, so equal logits order by the lower id); K rounds, or one
// top-8 reduction for 256 experts or fewer.  Lane k < K receives the
// expert of the k-th largest key in myid and fk[] the logits' order keys.
// Returns true when the margin check below fails: the caller then selects
// on the exact probabilities p = exp(z - max) * (1/S) with the lowest-id
// tie-break.  Otherwise the selected set is exactly the K largest p, each
// strictly above every unselected p (their order among themselves by p
// is the caller's to form).
template <int R>
__device__ __forceinline__ bool topk_on_logits(const float (&z)[4 * R], int E, int K, int lane,
                                               uint32_t (&fk)[4 * R], int& myid) {
  constexpr int NK = 4 * R;
  constexpr int IDB = R == 1 ? 8 : 11;  // id bits of a selection key
  constexpr uint32_t IDM = (1u << IDB) - 1;
  uint32_t key[NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    const int e = lane + 64 * i;
    const bool in = e < E;
    fk[i] = in ? f2key(z[i]) : 0u;
    key[i] = in ? (((fk[i] >> IDB) << IDB) | (IDM - (uint32_t)e)) : 0u;
  }
  // K rounds: the largest remaining key; its low bits name the expert.  Lane
  // `it` keeps the id of round it (no branches inside the loop).  With four
  // keys a lane sorts them once, so a round is one wave-wide max of the lane
  // heads and a shift in the winning lane.  A last max gives the largest
  // unselected key.
  uint32_t gm = 0, gu = 0, gtop = 0;
  if constexpr (NK == 4) {
    uint32_t k0 = key[0], k1 = key[1], k2 = key[2], k3 = key[3];
    auto cx = [](uint32_t& a, uint32_t& b) {  // a >= b afterwards
      const uint32_t hi = a > b ? a : b, lo = a > b ? b : a;
      a = hi;
      b = lo;
    };
    cx(k0, k1);
    cx(k2, k3);
    cx(k0, k2);
    cx(k1, k3);
    cx(k1, k2);
    if (K <= 8) {
      // one wave-wide top-8 reduction (bitonic merges along the DPP
      // reduction tree) instead of K rounds of wave maxima
      uint32_t a[8] = {k0, k1, k2, k3, 0u, 0u, 0u, 0u};
      top8_step<0x111, 0xF>(a);
      top8_step<0x112, 0xF>(a);
      top8_step<0x114, 0xF>(a);
      top8_step<0x118, 0xF>(a);
      top8_step<0x142, 0xA>(a);
      top8_step<0x143, 0xC>(a);
      uint32_t T[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) T[i] = __builtin_amdgcn_readlane(a[i], 63);
      gtop = T[0];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i == K - 1) gm = T[i];
        if (i == K && K < E) gu = T[i];
        myid = lane == i ? (int)(IDM - (T[i] & IDM)) : myid;
      }
      if (K == 8 && K < E) {
        // the largest key outside the top 8: each lane's first key below T7
        const uint32_t t7 = T[7];
        const uint32_t c = k0 < t7 ? k0 : k1 < t7 ? k1 : k2 < t7 ? k2 : k3 < t7 ? k3 : 0u;
        gu = wave_max_u32(c);
      }
    } else {
#pragma unroll 8
      for (int it = 0; it < K; ++it) {
        gm = wave_max_u32(k0);
        gtop = it == 0 ? gm : gtop;
        const bool win = k0 == gm;
        k0 = win ? k1 : k0;
        k1 = win ? k2 : k1;
        k2 = win ? k3 : k2;
        k3 = win ? 0u : k3;
        myid = lane == it ? (int)(IDM - (gm & IDM)) : myid;
      }
      if (K < E) gu = wave_max_u32(k0);
    }
  } else {
    uint32_t kw[NK];
#pragma unroll
    for (int i = 0; i < NK; ++i) kw[i] = key[i];
#pragma unroll 8
    for (int it = 0; it < K; ++it) {
      uint32_t km = 0;
#pragma unroll
      for (int i = 0; i < NK; ++i) km = kw[i] > km ? kw[i] : km;
      gm = wave_max_u32(km);
      gtop = it == 0 ? gm : gtop;
#pragma unroll
      for (int i = 0; i < NK; ++i) kw[i] = kw[i] == gm ? 0u : kw[i];
      myid = lane == it ? (int)(IDM - (gm & IDM)) : myid;
    }
    if (K < E) {
      uint32_t km = 0;
#pragma unroll
      for (int i = 0; i < NK; ++i) km = kw[i] > km ? kw[i] : km;
      gu = wave_max_u32(km);
    }
  }
  // Margin check on bounds from the keys: every selected logit is at least
  // zs (the K-th key with its id bits cleared) and every unselected one at
  // most zu (the largest unselected key with its id bits set), so
  // e(zs) > e(zu) (1 + 2^-20) implies the same for the exact boundary logits
  // (exp is monotone to within an ulp, far inside the 2^-20 margin).
  // Fast sufficient test first: with zmax an upper bound of the largest
  // logit (the top key with its id bits set), the rounded arguments zs - m
  // and zu - m differ by at least (zs - zu) - 2^-23 (zmax - zu), and the
  // computed exponentials (within 2^-21 relative of exp) keep their order by
  // more than 2^-20 once that difference exceeds 2^-18; so when
  // zs - zu > 2^-17 + 2^-21 (zmax - zu) and zmax - zs < 64 (no underflow of
  // e(zs)) the exact maximum and both exponentials are not needed.  Any
  // non-finite bound fails the test and takes the full check.
  bool unsafe = false;
  if (K < E) {
    const float zs = key2f(gm & ~IDM), zu = key2f(gu | IDM), zmax = key2f(gtop | IDM);
    const bool clear = (zs - zu) > 0x1p-17f + (zmax - zu) * 0x1p-21f && (zmax - zs) < 64.0f;
    if (!clear) {
      uint32_t lmax = 0;
#pragma unroll
      for (int i = 0; i < NK; ++i) lmax = fk[i] > lmax ? fk[i] : lmax;
      const float m = key2f(wave_max_u32(lmax));
      const float ek = dm_expf(zs - m), en = dm_expf(zu - m);
      unsafe = !(ek > en + en * 0x1p-20f);
    }
  }
  return unsafe;
}

// ---- softmax + top-k + shared gate of one token ------------------------------
// router_softmax (src/layers/router.mojo:140-183: sequential max, exp, sum,
// p = e * (1/sum)) and select_topk (src/layers/topk.mojo:79-128: largest p,
// lowest expert id on ties, K rounds; sum and renormalisation-leak checks).
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// NE values per lane: element e = lane + 64 i.  Probabilities stay in
// registers; each selection round is two wave-wide maxima: of the key
// f2u(p) + 1 (p >= 0, so its bits order like p; 0 marks "no candidate") and,
// among the lanes holding that key, of 0xFFFF - e (the lowest expert id).
// Token t on one wave (lane 0..63), with sm (((E + 3) & ~3) + 4 floats of
// LDS) its own; sync() orders the wave's LDS writes before reads by other
// lanes (a workgroup barrier when the wave is the whole workgroup).  COH:
// the logits are read, and the ids written, with agent-scope accesses
// (producer and consumer are other workgroups of the same launch).
template <int NE, bool COH, class Sync>
__device__ __forceinline__ void route_select_token(const float* __restrict__ z, int ldz, int E,
                                                   int K, int has_sh, int t, int lane, float* sm,
                                                   int32_t* __restrict__ ids,
                                                   float* __restrict__ probs,
                                                   float* __restrict__ shg,
                                                   unsigned long long* status, Sync sync) {
  float* pv = sm;
  float* scal = sm + ((E + 3) & ~3);
  const float* zr = z + (size_t)t * ldz;
  // the shared-gate logit is requested with the others: a load issued after
  // the stores below would wait for them
  const float lg = has_sh && lane == 0 ? (COH ? ld_coh(zr + E) : zr[E]) : 0.0f;
  float zv[NE];
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const int e = lane + 64 * i;
    zv[i] = e < E ? (COH ? ld_coh(zr + e) : zr[e]) : -__builtin_inff();
    if (e < E && !finite_f(zv[i])) record_err(status, err_key(kPhLogit, t, 0, e, 0));
    m = zv[i] > m ? zv[i] : m;
  }
  m = __ockl_wfred_max_f32(m);
  if (lane == 0 && !finite_f(m)) record_err(status, err_key(kPhSoftmax, t, 0, 0, 0));
  float p[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const int e = lane + 64 * i;
    if (e < E) {
      p[i] = dm_expf(zv[i] - m);
      if (!finite_f(p[i])) record_err(status, err_key(kPhSoftmax, t, 0, 1 + e, 0));
      pv[e] = p[i];
    }
  }
  sync();
  if (lane == 0) {
    const float s = seq_sum(pv, E);
    if (!(s > 0.0f) || !finite_f(s)) record_err(status, err_key(kPhSoftmax, t, 0, 1 + E, 0));
    scal[0] = 1.0f / s;
  }
  sync();
  const float inv = scal[0];
  uint32_t key[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const int e = lane + 64 * i;
    p[i] = p[i] * inv;
    key[i] = e < E ? f2u(p[i]) + 1u : 0u;
  }
  sync();  // pv is rewritten with the probabilities for the leak check
#pragma unroll
  for (int i = 0; i < NE; ++i)
    if (lane + 64 * i < E) pv[lane + 64 * i] = p[i];
  float sum_topk = 0.0f;
  bool done = false;
  if constexpr (NE <= 4) {
    // Fast path (E <= 256, K <= 8): one wave-wide top-8 reduction of 32-bit
    // keys, the probability bits with their low 8 bits replaced by 255 - e.
    // It is the exact selection when the truncated probabilities of the K
    // selected experts and of the best unselected one are strictly
    // decreasing (no tie or near tie the truncation could reorder) and the
    // K-th is nonzero; otherwise the K exact rounds below run.
    if (K <= 8) {
      uint32_t k4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = lane + 64 * i;
        k4[i] = i < NE && e < E ? ((key[i < NE ? i : 0] >> 8) << 8) | (255u - (uint32_t)e) : 0u;
      }
      auto cx = [](uint32_t& a, uint32_t& b) {  // a >= b afterwards
        const uint32_t hi = a > b ? a : b, lo = a > b ? b : a;
        a = hi;
        b = lo;
      };
      cx(k4[0], k4[1]);
      cx(k4[2], k4[3]);
      cx(k4[0], k4[2]);
      cx(k4[1], k4[3]);
      cx(k4[1], k4[2]);
      uint32_t a[8] = {k4[0], k4[1], k4[2], k4[3], 0u, 0u, 0u, 0u};
      top8_step<0x111, 0xF>(a);
      top8_step<0x112, 0xF>(a);
      top8_step<0x114, 0xF>(a);
      top8_step<0x118, 0xF>(a);
      top8_step<0x142, 0xA>(a);
      top8_step<0x143, 0xC>(a);
      uint32_t T[9];
#pragma unroll
      for (int i = 0; i < 8; ++i) T[i] = __builtin_amdgcn_readlane(a[i], 63);
      T[8] = 0u;
      if (K == 8 && K < E) {  // the largest key outside the top 8
        const uint32_t t7 = T[7];
        const uint32_t c = k4[0] < t7 ? k4[0] : k4[1] < t7 ? k4[1] : k4[2] < t7 ? k4[2]
                         : k4[3] < t7 ? k4[3] : 0u;
        T[8] = wave_max_u32(c);
      }
      bool clean = true;
#pragma unroll
      for (int r = 0; r < 8; ++r)
        if (r < K) clean = clean && (T[r] >> 8) > (T[r + 1] >> 8);
      if (clean) {
        sync();  // pv (the probabilities) is read by other lanes
        // lane r < K reads and writes rank r; lane 0 sums them in rank order
        int win = 0;
#pragma unroll
        for (int r = 0; r < 8; ++r) win = lane == r ? 255 - (int)(T[r] & 255u) : win;
        const float bv = lane < K ? pv[win] : 0.0f;
        if (lane < K) {
          if (COH)
            st_coh_i32(ids + (size_t)t * K + lane, win);
          else
            ids[(size_t)t * K + lane] = win;
          probs[(size_t)t * K + lane] = bv;
        }
#pragma unroll
        for (int r = 0; r < 8; ++r)
          if (r < K) sum_topk = sum_topk + u2f(__builtin_amdgcn_readlane(f2u(bv), r));
        done = true;
      }
    }
  }
  for (int r = 0; r < K && !done; ++r) {
    uint32_t bk = 0;
    int bi = 0xFFFF;
#pragma unroll
    for (int i = 0; i < NE; ++i)  // ascending e within the lane: first of equal keys wins
      if (key[i] > bk) { bk = key[i]; bi = lane + 64 * i; }
    const uint32_t mk = __ockl_wfred_max_u32(bk);
    const uint32_t me = __ockl_wfred_max_u32(bk == mk && mk != 0u ? 0xFFFFu - (uint32_t)bi : 0u);
    int win = (int)(0xFFFFu - me);
    if (mk == 0u || win < 0 || win >= E) win = 0;  // only reachable after a recorded error
    const float bv = u2f(mk - 1u);
#pragma unroll
    for (int i = 0; i < NE; ++i)
      if (lane + 64 * i == win) key[i] = 0u;
    sum_topk = sum_topk + bv;
    if (lane == 0) {
      if (COH)
        st_coh_i32(ids + (size_t)t * K + r, win);
      else
        ids[(size_t)t * K + r] = win;
      probs[(size_t)t * K + r] = bv;
    }
  }
  if (lane == 0) {
    if (sum_topk > 1.00001f) record_err(status, err_key(kPhTopk, t, 0, 0, kTkSum));
    if (K < E && __builtin_fabsf(sum_topk - 1.0f) < 1e-6f) {
      const float sum_all = seq_sum(pv, E);
      if (sum_all - sum_topk > 1e-5f) record_err(status, err_key(kPhTopk, t, 0, 0, kTkLeak));
    }
    if (has_sh) {
      if (!finite_f(lg)) record_err(status, err_key(kPhGate, t, 0, 0, kGkLogit));
      const float s = dm_sigmoid(lg);
      if (!finite_f(s) || s < 0.0f || s > 1.0f)
        record_err(status, err_key(kPhGate, t, 0, 0, kGkRange));
      shg[t] = s;
    }
  }
}


// One router logit chain of the R16 layer form: row e, lane partial l of
// router_project (src/layers/router.mojo:80-104): k = l, l + 16, ... with
// separate multiply and add, x (one token, fp32) staged in LDS.
// The weights are requested eight 128-column chunks at a time (clamped
// loads, all in flight together) ahead of their multiply-adds.
__device__ __forceinline__ float router_chain(const uint16_t* __restrict__ router, int H, int e,
                                              int l, const float* xs) {
  float acc = 0.0f;
  const uint4* wp = reinterpret_cast<const uint4*>(router + r16_index(H, e, l));
  const int nj8 = H / 128;
  for (int j0 = 0; j0 < nj8; j0 += 8) {
    uint4 w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = wp[(size_t)min(j0 + u, nj8 - 1) * 16];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (j0 + u < nj8) {  // uniform
        const uint32_t ww[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
        const float* xc = xs + (j0 + u) * 128 + l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc = acc + xc[(2 * i) * 16] * bf16lo(ww[i]);
          acc = acc + xc[(2 * i + 1) * 16] * bf16hi(ww[i]);
        }
      }
    }
  }
  return acc;
}

}  // namespace dm
