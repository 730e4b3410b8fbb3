// dm_gguf.hip -- GGUF tensor payloads to fp32 on the GPU: the Q8_0, Q4_K and
// Q3_K block layouts of src/format/gguf.mojo:414-560 and the F32 / BF16
// branches of stream_gguf_tensor_f32 (gguf.mojo:598-613).
//
// Byte work, bound by HBM: per 256 weights a Q3_K block reads 114 B and
// writes 1 KiB of fp32, so the stores are 90% of the traffic.  Each thread
// produces 4 consecutive outputs and the lanes of a wave consecutive float4s,
// so every (non-temporal) store instruction fills whole cache lines: with 8
// outputs per thread as two float4 stores, each instruction left every line
// half written and the kernel ran at a third of this rate.  The block header
// bytes that neighbouring threads share come from the lines just fetched.
// No status: the reference's dequantizers accept every byte pattern
// (non-finite super-scales propagate as IEEE products).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dm_device.h"
#include "dm_gguf.h"
#include "dm_grouped.h"
#include "dm_layout.h"

namespace dm {
namespace {

__device__ __forceinline__ float h2f(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// The 4 outputs at element e0 (a multiple of 4) of a type whose whole
// blocks cover them.
template <int T>
__device__ __forceinline__ f32x4 values4(const uint8_t* raw, int64_t e0, int layout) {
  f32x4 v;
  if constexpr (T == kGgmlQ8_0) {
    // 34-byte blocks: fp16 d, 32 int8 codes
    const uint8_t* blk = raw + (e0 >> 5) * 34;
    const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
    const float d = h2f(h[0]);
    const int r = (int)(e0 & 31);
    const uint32_t w0 = h[1 + (r >> 1)], w1 = h[2 + (r >> 1)];
    v.x = d * (float)(int8_t)(w0 & 0xFF);
    v.y = d * (float)(int8_t)(w0 >> 8);
    v.z = d * (float)(int8_t)(w1 & 0xFF);
    v.w = d * (float)(int8_t)(w1 >> 8);
  } else if constexpr (T == kGgmlQ4_K) {
    // 144-byte blocks: fp16 d, fp16 dmin, 12 packed scale/min bytes, 128
    // code bytes; sub-block j holds 32 weights in code bytes 16j..16j+15,
    // the low nibbles first
    const uint8_t* blk = raw + (e0 >> 8) * 144;
    const uint32_t* w32 = reinterpret_cast<const uint32_t*>(blk);
    const int e = (int)(e0 & 255), j = e >> 5, r = e & 31;
    auto qb = [&](int i) -> int { return (int)((w32[1 + (i >> 2)] >> ((i & 3) * 8)) & 0xFF); };
    int sc, mn;
    if (j < 4) {
      sc = qb(j) & 63;
      mn = qb(j + 4) & 63;
    } else {
      // gguf.mojo:482-488 takes the low bits from byte j of the packed
      // scales; the reference's Python twin (oracle_port.py:104-110) from j+4
      const int lo = layout ? qb(j + 4) : qb(j);
      sc = (lo & 15) | ((qb(j - 4) >> 6) << 4);
      mn = (lo >> 4) | ((qb(j) >> 6) << 4);
    }
    const uint32_t hd = w32[0];
    const float fs = (float)sc * h2f(hd & 0xFFFF);
    const float fm = (float)mn * h2f(hd >> 16);
    const uint32_t c = w32[(16 + j * 16 + (r & 15)) >> 2] >> (r < 16 ? 0 : 4);
    v.x = fs * (float)(c & 15) - fm;
    v.y = fs * (float)((c >> 8) & 15) - fm;
    v.z = fs * (float)((c >> 16) & 15) - fm;
    v.w = fs * (float)((c >> 24) & 15) - fm;
  } else if constexpr (T == kGgmlQ3_K) {
    // 114-byte blocks: hmask[32] (bit e of the 256), qs[64] (2 bits each),
    // 16 scale bytes (value - 32), fp16 d at 112
    const uint8_t* blk = raw + (e0 >> 8) * 114;
    const int e = (int)(e0 & 255);
    const uint32_t hm = blk[e >> 3] >> (e & 7);
    const uint32_t qs = blk[32 + (e >> 2)];
    const float fs = (float)((int)blk[96 + (e >> 4)] - 32) *
                     h2f(reinterpret_cast<const uint16_t*>(blk)[56]);
    v.x = fs * (float)((int)(((hm & 1) << 2) | (qs & 3)) - 4);
    v.y = fs * (float)((int)((((hm >> 1) & 1) << 2) | ((qs >> 2) & 3)) - 4);
    v.z = fs * (float)((int)((((hm >> 2) & 1) << 2) | ((qs >> 4) & 3)) - 4);
    v.w = fs * (float)((int)((((hm >> 3) & 1) << 2) | ((qs >> 6) & 3)) - 4);
  } else if constexpr (T == kGgmlBF16) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(raw + e0 * 2);
    const uint32_t a = w[0], b = w[1];
    v.x = __builtin_bit_cast(float, a << 16);
    v.y = __builtin_bit_cast(float, a & 0xFFFF0000u);
    v.z = __builtin_bit_cast(float, b << 16);
    v.w = __builtin_bit_cast(float, b & 0xFFFF0000u);
  } else {  // F32
    const float* f = reinterpret_cast<const float*>(raw) + e0;
    v.x = f[0];
    v.y = f[1];
    v.z = f[2];
    v.w = f[3];
  }
  return v;
}

// n outputs; whole blocks cover n_blk of them (a multiple of 32 for the
// block types, n for F32 / BF16), the rest is 0.0.  Thread f writes elements
// 4f .. 4f+3; the last float4 may be partial.
template <int T>
__global__ __launch_bounds__(256) void k_dequant_gguf(const uint8_t* __restrict__ raw,
                                                      int64_t n, int64_t n_blk, int layout,
                                                      float* __restrict__ out) {
  // Workgroups are dispatched round-robin over the 8 XCDs, each with its own
  // L2.  For the K-quant types give XCD x one contiguous run of the
  // workgroup range, so that a 114- or 144-byte block straddling two
  // workgroups' ranges is fetched once, not once per XCD (Q3_K: 1.26x ->
  // 1.0x of the payload bytes; measured slower for Q8_0, which keeps the
  // plain order).
  uint32_t wg = blockIdx.x;
  if constexpr (T == kGgmlQ3_K || T == kGgmlQ4_K) {
    const uint32_t G = gridDim.x, q = G >> 3, r = G & 7;
    const uint32_t x = blockIdx.x & 7, pos = blockIdx.x >> 3;
    wg = x * q + (x < r ? x : r) + pos;
  }
  const int64_t f = (int64_t)wg * 256 + threadIdx.x;
  const int64_t e0 = f * 4;
  if constexpr (T == kGgmlQ4_K) {
    // A workgroup's 1024 outputs are 4 whole Q4_K blocks, 576 contiguous
    // bytes at a 4-byte aligned offset: load them with coalesced dwords into
    // LDS and decode from there, instead of each lane issuing five dword
    // loads into the same lines (Q4_K 203 -> 161 us per layer; the same for
    // Q8_0's 1088 bytes measured slower, 251 -> 303 us).
    constexpr int kBytes = 576;
    __shared__ __attribute__((aligned(16))) uint32_t sblk[kBytes / 4];
    const int64_t w0 = (int64_t)wg * 1024;  // first output of the workgroup
    if (w0 + 1024 <= n_blk) {                // uniform over the workgroup
      const uint32_t* src = reinterpret_cast<const uint32_t*>(raw + (w0 >> 8) * 144);
      for (int i = threadIdx.x; i < kBytes / 4; i += 256) sblk[i] = src[i];
      __syncthreads();
      const f32x4 v = values4<T>(reinterpret_cast<const uint8_t*>(sblk), e0 - w0, layout);
      __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(out + e0));
      return;
    }
  }
  if (e0 >= n) return;
  f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
  if (e0 + 4 <= n_blk) {
    v = values4<T>(raw, e0, layout);
  } else if (e0 < n_blk) {  // F32 / BF16 tail, element by element
    for (int i = 0; i < 4 && e0 + i < n_blk; ++i) {
      float x;
      if constexpr (T == kGgmlBF16)
        x = __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t*>(raw)[e0 + i] << 16);
      else
        x = reinterpret_cast<const float*>(raw)[e0 + i];
      v[i] = x;
    }
  }
  if (e0 + 4 <= n) {
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(out + e0));
  } else {
    for (int i = 0; i < 4 && e0 + i < n; ++i) out[e0 + i] = v[i];
  }
}


// ---- MoE experts straight from GGUF blocks ---------------------------------
// One wave per output row: the 64 lanes walk the row in float4 chunks (the
// row's weights decoded from their blocks as in k_dequant_gguf), accumulate
// in fp32 and reduce across the wave.  Decode reads each selected expert's
// payload once (Q3_K: 0.445 B per weight) instead of converting the layer's
// 256 experts to fp32 first.

// Sum over the 64 lanes by DPP row shifts and row broadcasts (the result of
// lane 63, broadcast): a few cycles per step where a shuffle goes through
// the LDS crossbar.  Every expert kernel of this file reduces in this order,
// so a token's outputs do not depend on the launch form that computed them.
template <int CTRL, int RM>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                               RM, 0xF, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = v + dpp_f<0x111, 0xF>(v);  // row_shr:1
  v = v + dpp_f<0x112, 0xF>(v);  // row_shr:2
  v = v + dpp_f<0x114, 0xF>(v);  // row_shr:4
  v = v + dpp_f<0x118, 0xF>(v);  // row_shr:8
  v = v + dpp_f<0x142, 0xA>(v);  // row_bcast:15
  v = v + dpp_f<0x143, 0xC>(v);  // row_bcast:31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}


__device__ __forceinline__ float dot4(f32x4 a, f32x4 b, float acc) {
  acc = __builtin_fmaf(a.x, b.x, acc);
  acc = __builtin_fmaf(a.y, b.y, acc);
  acc = __builtin_fmaf(a.z, b.z, acc);
  return __builtin_fmaf(a.w, b.w, acc);
}

// The 3-bit codes of sixteen Q3_K weights (qs: their 2-bit low parts, code
// i at bits 2i; hm: their high bits, bit i) as bytes, four weights per
// word: byte m of qw[k] = code of weight 4m + k.  A word costs a shift, a
// mask and a merge of each part (the high bits first moved so that nibble m
// of hm is the low nibble of byte m), where a code taken alone costs two
// bit-field extractions and a merge; a byte then converts in one
// instruction (v_cvt_f32_ubyte0..3).
__device__ __forceinline__ void q3_codes(uint32_t qs, uint32_t hm, uint32_t (&qw)[4]) {
  uint32_t t = (hm | (hm << 8)) & 0x00FF00FFu;
  const uint32_t hs = (t | (t << 4)) & 0x0F0F0F0Fu;  // bit k of byte m = hm bit 4m + k
  qw[0] = ((hs << 2) & 0x04040404u) | (qs & 0x03030303u);
  qw[1] = ((hs << 1) & 0x04040404u) | ((qs >> 2) & 0x03030303u);
  qw[2] = (hs & 0x04040404u) | ((qs >> 4) & 0x03030303u);
  qw[3] = ((hs >> 1) & 0x04040404u) | ((qs >> 6) & 0x03030303u);
}
// code i of q3_codes' words as a float
__device__ __forceinline__ float q3_code(const uint32_t (&qw)[4], int i) {
  return (float)((qw[i & 3] >> (8 * (i >> 2))) & 0xFFu);
}

// W consecutive weights at element e0 (a multiple of W, W in {4, 8, 16}).
// For Q3_K eight weights share one hmask byte, two code bytes, the scale
// byte and d, so the block header is decoded once per eight (sixteen).
template <int T, int W>
__device__ __forceinline__ void valuesW(const uint8_t* raw, int64_t e0, int layout, f32x4 (&v)[W / 4]) {
  static_assert(!(T == kGgmlQ3_K && W == 16), "Q3_K gate/up rows go through gu_dot16");
  if constexpr (T == kGgmlQ3_K && W == 8) {
    const uint8_t* blk = raw + (e0 >> 8) * 114;
    const int e = (int)(e0 & 255);
    const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
    const uint32_t hm = blk[e >> 3];
    const uint32_t qs = h[16 + (e >> 3)];  // code bytes 32 + e/4 and the next
    const float fs = (float)((int)blk[96 + (e >> 4)] - 32) * h2f(h[56]);
    // fs (q - 4) rounded once: fma(fs, q, -4 fs), -4 fs being exact
    const float m4 = -4.0f * fs;
    uint32_t qw[4];
    q3_codes(qs, hm, qw);
    float w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = __builtin_fmaf(fs, q3_code(qw, i), m4);
    v[0] = f32x4{w[0], w[1], w[2], w[3]};
    v[1] = f32x4{w[4], w[5], w[6], w[7]};
  } else {
#pragma unroll
    for (int j = 0; j < W / 4; ++j) v[j] = values4<T>(raw, e0 + 4 * j, layout);
  }
}

// The bytes of W consecutive Q3_K weights (W = 8 or 16, at an element that
// is a multiple of W) as separate loads, so that a wave can request every
// chunk it needs before decoding the first.
template <int W>
struct Q3Raw {
  uint32_t hm, q0, q1, sc, d;
};
template <int W>
__device__ __forceinline__ Q3Raw<W> q3_load(const uint8_t* raw, int64_t e0) {
  const uint8_t* blk = raw + (e0 >> 8) * 114;
  const int e = (int)(e0 & 255);
  const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
  Q3Raw<W> r;
  if constexpr (W == 16) {
    r.hm = h[e >> 4];
    r.q0 = h[16 + (e >> 3)];
    r.q1 = h[17 + (e >> 3)];
  } else {
    r.hm = blk[e >> 3];
    r.q0 = h[16 + (e >> 3)];
    r.q1 = 0;
  }
  r.sc = blk[96 + (e >> 4)];
  r.d = h[56];
  return r;
}
// the same values valuesW<kGgmlQ3_K, W> forms from these bytes
template <int W>
__device__ __forceinline__ void q3_decode(const Q3Raw<W>& r, f32x4 (&v)[W / 4]) {
  const uint32_t qs = r.q0 | (r.q1 << 16);
  const float fs = (float)((int)r.sc - 32) * h2f(r.d);
  const float m4 = -4.0f * fs;  // fs (q - 4) rounded once, as valuesW forms it
  uint32_t qw[4];
  q3_codes(qs, r.hm, qw);
  float w[W];
#pragma unroll
  for (int i = 0; i < W; ++i) w[i] = __builtin_fmaf(fs, q3_code(qw, i), m4);
#pragma unroll
  for (int j = 0; j < W / 4; ++j) v[j] = f32x4{w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
}

// x[0] + x[1] + ... + x[15] in element order: the chunk term of q3_dot16.
__device__ __forceinline__ float xsum16(const f32x4 (&x)[4]) {
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    s = s + x[u].x;
    s = s + x[u].y;
    s = s + x[u].z;
    s = s + x[u].w;
  }
  return s;
}

// acc + sum_i w_i x_i over sixteen Q3_K weights w_i = fs (q_i - 4) of one
// 16-weight scale group, formed as fs (sum_i q_i x_i - 4 xs) with xs =
// xsum16(x): the 3-bit codes enter the products as they are, so a weight
// costs its share of q3_codes, a conversion and a multiply-add.
__device__ __forceinline__ float q3_dot16(const Q3Raw<16>& r, const f32x4 (&x)[4], float xs,
                                          float acc) {
  const uint32_t qs = r.q0 | (r.q1 << 16);
  const float fs = (float)((int)r.sc - 32) * h2f(r.d);
  uint32_t qw[4];
  q3_codes(qs, r.hm, qw);
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) t = __builtin_fmaf(q3_code(qw, i), x[i >> 2][i & 3], t);
  return __builtin_fmaf(fs, __builtin_fmaf(-4.0f, xs, t), acc);
}

// Gate and up dot-product terms of the sixteen weights at e0 of a row pair
// (x: the sixteen activations): Q3_K through q3_dot16, the other types as
// dequantised values.  Shared by every gate/up kernel, so that one token
// gives the same bits whichever launch form computes it.
template <int T>
__device__ __forceinline__ void gu_dot16(const uint8_t* wg, const uint8_t* wu, int64_t e0,
                                         int layout, const f32x4 (&xv)[4], float& ag, float& au) {
  if constexpr (T == kGgmlQ3_K) {
    const float xs = xsum16(xv);
    ag = q3_dot16(q3_load<16>(wg, e0), xv, xs, ag);
    au = q3_dot16(q3_load<16>(wu, e0), xv, xs, au);
  } else {
    f32x4 g4[4], u4[4];
    valuesW<T, 16>(wg, e0, layout, g4);
    valuesW<T, 16>(wu, e0, layout, u4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ag = dot4(g4[j], xv[j], ag);
      au = dot4(u4[j], xv[j], au);
    }
  }
}

template <int T, int W>
__global__ __launch_bounds__(256) void k_gguf_gateup(GgufMoeDev L, const float* __restrict__ x,
                                                     const int32_t* __restrict__ ids,
                                                     float* __restrict__ h, int ldh,
                                                     unsigned long long* status, int t0) {
  const int lane = threadIdx.x & 63;
  const int slot = (int)(blockIdx.y % (unsigned)(L.K + 1));
  const int t = t0 + (int)(blockIdx.y / (unsigned)(L.K + 1));
  const bool sh = slot == L.K;
  const int rows = sh ? L.Ish : L.I;
  const int r = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int e = sh ? L.E : ids[(size_t)t * L.K + slot];
  const uint8_t* wg = L.raw + L.off[(size_t)e * 3 + 0];
  const uint8_t* wu = L.raw + L.off[(size_t)e * 3 + 1];
  const float* xt = x + (size_t)t * L.H;
  const int64_t base = (int64_t)r * L.H;
  float ag = 0.0f, au = 0.0f;
  for (int c = lane * W; c < L.H; c += 64 * W) {
    if constexpr (W == 16) {
      f32x4 xv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[j] = *reinterpret_cast<const f32x4*>(xt + c + 4 * j);
      gu_dot16<T>(wg, wu, base + c, L.layout, xv, ag, au);
    } else {
      f32x4 g4[W / 4], u4[W / 4];
      valuesW<T, W>(wg, base + c, L.layout, g4);
      valuesW<T, W>(wu, base + c, L.layout, u4);
#pragma unroll
      for (int j = 0; j < W / 4; ++j) {
        const f32x4 xv = *reinterpret_cast<const f32x4*>(xt + c + 4 * j);
        ag = dot4(g4[j], xv, ag);
        au = dot4(u4[j], xv, au);
      }
    }
  }
  ag = wave_sum_dpp(ag);
  au = wave_sum_dpp(au);
  if (lane == 0) {
    const float hv = dm_silu(ag) * au;
    const uint32_t ph = sh ? kPhShared : kPhExpert, sl = sh ? 0 : (uint32_t)slot;
    if (!finite_f(ag)) record_err(status, err_key(ph, t, sl, r, kEkGate));
    if (!finite_f(au)) record_err(status, err_key(ph, t, sl, r, kEkUp));
    if (!finite_f(hv)) record_err(status, err_key(ph, t, sl, r, kEkH));
    h[((size_t)t * (L.K + 1) + slot) * ldh + r] = hv;
  }
}

// Down projections and moe_aggregate_forward in one launch: workgroup (d, t)
// computes output row d of every slot of token t (wave w takes slots w, w+4,
// ...), then one thread combines them in the reference order, y = sum_k p_k
// r_k + g r_sh (+ residual), with separate multiply and add.
template <int T, int W>
__global__ __launch_bounds__(256) void k_gguf_down_combine(
    GgufMoeDev L, const float* __restrict__ h, int ldh, const int32_t* __restrict__ ids,
    const float* __restrict__ probs, const float* __restrict__ shg,
    const float* __restrict__ residual, float* __restrict__ y, unsigned long long* status,
    int t0) {
  __shared__ float part[33];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int d = (int)blockIdx.x, t = t0 + (int)blockIdx.y;
  for (int slot = wave; slot <= L.K; slot += 4) {
    const bool sh = slot == L.K;
    const int n = sh ? L.Ish : L.I;
    const int e = sh ? L.E : ids[(size_t)t * L.K + slot];
    const uint8_t* wd = L.raw + L.off[(size_t)e * 3 + 2];
    const float* hv = h + ((size_t)t * (L.K + 1) + slot) * ldh;
    const int64_t base = (int64_t)d * n;
    float a = 0.0f;
    for (int c = lane * W; c < n; c += 64 * W) {
      f32x4 w4[W / 4];
      valuesW<T, W>(wd, base + c, L.layout, w4);
#pragma unroll
      for (int j = 0; j < W / 4; ++j)
        a = dot4(w4[j], *reinterpret_cast<const f32x4*>(hv + c + 4 * j), a);
    }
    a = wave_sum_dpp(a);
    if (lane == 0) {
      if (!finite_f(a))
        record_err(status, err_key(sh ? kPhShared : kPhExpert, t, sh ? 0 : slot, n + d, kEkDown));
      part[slot] = a;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float acc = 0.0f;
    for (int k = 0; k < L.K; ++k) acc = acc + probs[(size_t)t * L.K + k] * part[k];
    float total = acc + shg[t] * part[L.K];
    if (residual) total = total + residual[(size_t)t * L.H + d];
    if (!finite_f(total)) record_err(status, err_key(kPhAgg, t, 0, d, 0));
    y[(size_t)t * L.H + d] = total;
  }
}

// ---- several tokens grouped by expert --------------------------------------
// The units of launch_group_build: an expert's row is read once per unit (up
// to 128 tokens) and its weights decoded once per pass of kGgufUnitTok
// tokens.  Each token's lane sums and wave reductions are those of
// k_gguf_gateup / k_gguf_down_combine (the same helpers, the same order), so
// a token's outputs do not depend on the form that computed them.
constexpr int kGgufUnitTok = 8;

struct GgufUnit {
  int e, p0, n;  // expert (E: shared), first position (shared: first token), tokens
  bool sh;
};
__device__ __forceinline__ GgufUnit gguf_unit(const int2* units, const int32_t* meta,
                                              const int32_t* off, int u, int E, int T) {
  const int2 v = units[u];
  const int size = u < meta[1] ? kUnitBig : kUnitSmall;
  GgufUnit r;
  r.sh = v.x >= E;
  r.e = r.sh ? E : v.x;
  r.p0 = r.sh ? v.y : off[v.x] + v.y;
  r.n = min(size, (r.sh ? T : off[v.x + 1]) - r.p0);
  return r;
}
// token and slot (K: the shared expert) of the unit's position i
__device__ __forceinline__ void gguf_unit_pos(const GgufUnit& ut, const int32_t* perm, int K,
                                              int i, int& t, int& slot) {
  if (ut.sh) {
    t = ut.p0 + i;
    slot = K;
  } else {
    const int a = perm[ut.p0 + i];
    t = a / K;
    slot = a % K;
  }
}

// Workgroup (rb, u): rows 4 rb + wave of unit u0 + u's expert, h as
// k_gguf_gateup writes it.
template <int T, int W>
__global__ __launch_bounds__(256) void k_gguf_gateup_units(
    GgufMoeDev L, const float* __restrict__ x, const int32_t* __restrict__ off,
    const int32_t* __restrict__ perm, const int2* __restrict__ units,
    const int32_t* __restrict__ meta, int ntok, float* __restrict__ h, int ldh,
    unsigned long long* status, int u0) {
  const int u = u0 + (int)blockIdx.y;
  if (u >= meta[0]) return;
  const GgufUnit ut = gguf_unit(units, meta, off, u, L.E, ntok);
  const int rows = ut.sh ? L.Ish : L.I;
  const int r = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows || ut.n <= 0) return;
  const int lane = threadIdx.x & 63;
  const uint8_t* wg = L.raw + L.off[(size_t)ut.e * 3 + 0];
  const uint8_t* wu = L.raw + L.off[(size_t)ut.e * 3 + 1];
  const int64_t base = (int64_t)r * L.H;
  for (int i0 = 0; i0 < ut.n; i0 += kGgufUnitTok) {
    int tt[kGgufUnitTok], sl[kGgufUnitTok];
    float ag[kGgufUnitTok], au[kGgufUnitTok];
#pragma unroll
    for (int k = 0; k < kGgufUnitTok; ++k) {
      gguf_unit_pos(ut, perm, L.K, min(i0 + k, ut.n - 1), tt[k], sl[k]);
      ag[k] = 0.0f;
      au[k] = 0.0f;
    }
    const int nk = min(kGgufUnitTok, ut.n - i0);
    for (int c = lane * W; c < L.H; c += 64 * W) {
#pragma unroll
      for (int k = 0; k < kGgufUnitTok; ++k) {
        if (k >= nk) break;  // uniform per wave
        const float* xt = x + (size_t)tt[k] * L.H;
        if constexpr (W == 16) {
          f32x4 xv[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) xv[j] = *reinterpret_cast<const f32x4*>(xt + c + 4 * j);
          gu_dot16<T>(wg, wu, base + c, L.layout, xv, ag[k], au[k]);
        } else {
          f32x4 g4[W / 4], u4[W / 4];
          valuesW<T, W>(wg, base + c, L.layout, g4);
          valuesW<T, W>(wu, base + c, L.layout, u4);
#pragma unroll
          for (int j = 0; j < W / 4; ++j) {
            const f32x4 xv = *reinterpret_cast<const f32x4*>(xt + c + 4 * j);
            ag[k] = dot4(g4[j], xv, ag[k]);
            au[k] = dot4(u4[j], xv, au[k]);
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kGgufUnitTok; ++k) {
      if (i0 + k >= ut.n) break;  // uniform per wave
      const float g = wave_sum_dpp(ag[k]), uu = wave_sum_dpp(au[k]);
      if (lane == 0) {
        const int t = tt[k], slot = sl[k];
        const float hv = dm_silu(g) * uu;
        const uint32_t ph = ut.sh ? kPhShared : kPhExpert, sp = ut.sh ? 0 : (uint32_t)slot;
        if (!finite_f(g)) record_err(status, err_key(ph, t, sp, r, kEkGate));
        if (!finite_f(uu)) record_err(status, err_key(ph, t, sp, r, kEkUp));
        if (!finite_f(hv)) record_err(status, err_key(ph, t, sp, r, kEkH));
        h[((size_t)t * (L.K + 1) + slot) * ldh + r] = hv;
      }
    }
  }
}

// Workgroup (db, u): output rows 4 db + wave of unit u0 + u's down
// projection, parts[t][slot][d] as k_gguf_down_combine forms part[slot].
template <int T, int W>
__global__ __launch_bounds__(256) void k_gguf_down_units(
    GgufMoeDev L, const float* __restrict__ h, int ldh, const int32_t* __restrict__ off,
    const int32_t* __restrict__ perm, const int2* __restrict__ units,
    const int32_t* __restrict__ meta, int ntok, float* __restrict__ parts,
    unsigned long long* status, int u0) {
  const int u = u0 + (int)blockIdx.y;
  if (u >= meta[0]) return;
  const GgufUnit ut = gguf_unit(units, meta, off, u, L.E, ntok);
  const int d = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (d >= L.H || ut.n <= 0) return;
  const int lane = threadIdx.x & 63;
  const int n = ut.sh ? L.Ish : L.I;
  const uint8_t* wd = L.raw + L.off[(size_t)ut.e * 3 + 2];
  const int64_t base = (int64_t)d * n;
  for (int i0 = 0; i0 < ut.n; i0 += kGgufUnitTok) {
    int tt[kGgufUnitTok], sl[kGgufUnitTok];
    float a[kGgufUnitTok];
#pragma unroll
    for (int k = 0; k < kGgufUnitTok; ++k) {
      gguf_unit_pos(ut, perm, L.K, min(i0 + k, ut.n - 1), tt[k], sl[k]);
      a[k] = 0.0f;
    }
    const int nk = min(kGgufUnitTok, ut.n - i0);
    for (int c = lane * W; c < n; c += 64 * W) {
      f32x4 w4[W / 4];
      valuesW<T, W>(wd, base + c, L.layout, w4);
#pragma unroll
      for (int k = 0; k < kGgufUnitTok; ++k) {
        if (k >= nk) break;  // uniform per wave
        const float* hv = h + ((size_t)tt[k] * (L.K + 1) + sl[k]) * ldh;
#pragma unroll
        for (int j = 0; j < W / 4; ++j)
          a[k] = dot4(w4[j], *reinterpret_cast<const f32x4*>(hv + c + 4 * j), a[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < kGgufUnitTok; ++k) {
      if (i0 + k >= ut.n) break;  // uniform per wave
      const float v = wave_sum_dpp(a[k]);
      if (lane == 0) {
        const int t = tt[k], slot = sl[k];
        if (!finite_f(v))
          record_err(status, err_key(ut.sh ? kPhShared : kPhExpert, t, ut.sh ? 0 : slot, n + d,
                                     kEkDown));
        parts[((size_t)t * (L.K + 1) + slot) * L.H + d] = v;
      }
    }
  }
}

// Blocked forms (the common shapes): a wave keeps the activations of
// kGgufBlkTok tokens in registers (its lane's chunks, at most kGgufBlkCh of
// them) across rpw rows (1 .. kGgufBlkRowsMax, more when the units hold
// more tokens), so that a row costs its weights and the
// products, not another read of every token's x (or h) from the caches.
// The lane sums run over the same chunks in the same order as above.
constexpr int kGgufBlkTok = 4, kGgufBlkCh = 2, kGgufBlkRowsMax = 8;

// gate/up, sixteen weights per lane (gu_dot16), H <= 64 * 16 * kGgufBlkCh
template <int T>
__global__ __launch_bounds__(256) void k_gguf_gateup_units_blk(
    GgufMoeDev L, const float* __restrict__ x, const int32_t* __restrict__ off,
    const int32_t* __restrict__ perm, const int2* __restrict__ units,
    const int32_t* __restrict__ meta, int ntok, float* __restrict__ h, int ldh,
    unsigned long long* status, int u0, int rpw) {
  const int u = u0 + (int)blockIdx.y;
  if (u >= meta[0]) return;
  const GgufUnit ut = gguf_unit(units, meta, off, u, L.E, ntok);
  const int rows = ut.sh ? L.Ish : L.I;
  const int row0 = ((int)blockIdx.x * 4 + (threadIdx.x >> 6)) * rpw;
  if (row0 >= rows || ut.n <= 0) return;
  const int lane = threadIdx.x & 63;
  const uint8_t* wg = L.raw + L.off[(size_t)ut.e * 3 + 0];
  const uint8_t* wu = L.raw + L.off[(size_t)ut.e * 3 + 1];
  for (int i0 = 0; i0 < ut.n; i0 += kGgufBlkTok) {
    const int nk = min(kGgufBlkTok, ut.n - i0);
    int tt[kGgufBlkTok], sl[kGgufBlkTok];
    f32x4 xv[kGgufBlkTok][kGgufBlkCh][4];
#pragma unroll
    for (int k = 0; k < kGgufBlkTok; ++k) {
      gguf_unit_pos(ut, perm, L.K, min(i0 + k, ut.n - 1), tt[k], sl[k]);
      const float* xt = x + (size_t)tt[k] * L.H;
#pragma unroll
      for (int ch = 0; ch < kGgufBlkCh; ++ch) {
        const int c = lane * 16 + 1024 * ch;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          xv[k][ch][j] = c < L.H ? *reinterpret_cast<const f32x4*>(xt + c + 4 * j)
                                 : f32x4{0, 0, 0, 0};
      }
    }
    // Q3_K: the next row's bytes are requested before this row's products
    // (q3_dot16 on them is gu_dot16's arithmetic)
    Q3Raw<16> pg[kGgufBlkCh], pu[kGgufBlkCh];
    auto q3_fetch = [&](int r) {
#pragma unroll
      for (int ch = 0; ch < kGgufBlkCh; ++ch) {
        const int c = min(lane * 16 + 1024 * ch, L.H - 16);
        pg[ch] = q3_load<16>(wg, (int64_t)r * L.H + c);
        pu[ch] = q3_load<16>(wu, (int64_t)r * L.H + c);
      }
    };
    if constexpr (T == kGgmlQ3_K) q3_fetch(row0);
    for (int rr = 0; rr < rpw; ++rr) {
      const int r = row0 + rr;
      if (r >= rows) break;  // uniform per wave
      const int64_t base = (int64_t)r * L.H;
      float ag[kGgufBlkTok], au[kGgufBlkTok];
#pragma unroll
      for (int k = 0; k < kGgufBlkTok; ++k) ag[k] = au[k] = 0.0f;
      if constexpr (T == kGgmlQ3_K) {
        Q3Raw<16> cg[kGgufBlkCh], cu[kGgufBlkCh];
#pragma unroll
        for (int ch = 0; ch < kGgufBlkCh; ++ch) {
          cg[ch] = pg[ch];
          cu[ch] = pu[ch];
        }
        if (rr + 1 < rpw && r + 1 < rows) q3_fetch(r + 1);
#pragma unroll
        for (int ch = 0; ch < kGgufBlkCh; ++ch) {
          const int c = lane * 16 + 1024 * ch;
          if (c < L.H) {
#pragma unroll
            for (int k = 0; k < kGgufBlkTok; ++k)
              if (k < nk) {
                const float xs = xsum16(xv[k][ch]);
                ag[k] = q3_dot16(cg[ch], xv[k][ch], xs, ag[k]);
                au[k] = q3_dot16(cu[ch], xv[k][ch], xs, au[k]);
              }
          }
        }
      } else {
#pragma unroll
        for (int ch = 0; ch < kGgufBlkCh; ++ch) {
          const int c = lane * 16 + 1024 * ch;
          if (c < L.H) {
#pragma unroll
            for (int k = 0; k < kGgufBlkTok; ++k)
              if (k < nk) gu_dot16<T>(wg, wu, base + c, L.layout, xv[k][ch], ag[k], au[k]);
          }
        }
      }
#pragma unroll
      for (int k = 0; k < kGgufBlkTok; ++k) {
        if (k >= nk) break;  // uniform per wave
        const float g = wave_sum_dpp(ag[k]), uu = wave_sum_dpp(au[k]);
        if (lane == 0) {
          const int t = tt[k], slot = sl[k];
          const float hv = dm_silu(g) * uu;
          const uint32_t ph = ut.sh ? kPhShared : kPhExpert, sp = ut.sh ? 0 : (uint32_t)slot;
          if (!finite_f(g)) record_err(status, err_key(ph, t, sp, r, kEkGate));
          if (!finite_f(uu)) record_err(status, err_key(ph, t, sp, r, kEkUp));
          if (!finite_f(hv)) record_err(status, err_key(ph, t, sp, r, kEkH));
          h[((size_t)t * (L.K + 1) + slot) * ldh + r] = hv;
        }
      }
    }
  }
}

// down, eight weights per lane, I and Ish <= 64 * 8 * kGgufBlkCh
template <int T>
__global__ __launch_bounds__(256) void k_gguf_down_units_blk(
    GgufMoeDev L, const float* __restrict__ h, int ldh, const int32_t* __restrict__ off,
    const int32_t* __restrict__ perm, const int2* __restrict__ units,
    const int32_t* __restrict__ meta, int ntok, float* __restrict__ parts,
    unsigned long long* status, int u0, int rpw) {
  const int u = u0 + (int)blockIdx.y;
  if (u >= meta[0]) return;
  const GgufUnit ut = gguf_unit(units, meta, off, u, L.E, ntok);
  const int d0 = ((int)blockIdx.x * 4 + (threadIdx.x >> 6)) * rpw;
  if (d0 >= L.H || ut.n <= 0) return;
  const int lane = threadIdx.x & 63;
  const int n = ut.sh ? L.Ish : L.I;
  const uint8_t* wd = L.raw + L.off[(size_t)ut.e * 3 + 2];
  for (int i0 = 0; i0 < ut.n; i0 += kGgufBlkTok) {
    const int nk = min(kGgufBlkTok, ut.n - i0);
    int tt[kGgufBlkTok], sl[kGgufBlkTok];
    f32x4 hv[kGgufBlkTok][kGgufBlkCh][2];
#pragma unroll
    for (int k = 0; k < kGgufBlkTok; ++k) {
      gguf_unit_pos(ut, perm, L.K, min(i0 + k, ut.n - 1), tt[k], sl[k]);
      const float* ht = h + ((size_t)tt[k] * (L.K + 1) + sl[k]) * ldh;
#pragma unroll
      for (int ch = 0; ch < kGgufBlkCh; ++ch) {
        const int c = lane * 8 + 512 * ch;
#pragma unroll
        for (int j = 0; j < 2; ++j)
          hv[k][ch][j] = c < n ? *reinterpret_cast<const f32x4*>(ht + c + 4 * j)
                               : f32x4{0, 0, 0, 0};
      }
    }
    // Q3_K: the next row's bytes are requested before this row's products
    // (q3_decode on them forms valuesW's values)
    Q3Raw<8> pd[kGgufBlkCh];
    auto q3_fetch = [&](int d) {
#pragma unroll
      for (int ch = 0; ch < kGgufBlkCh; ++ch)
        pd[ch] = q3_load<8>(wd, (int64_t)d * n + min(lane * 8 + 512 * ch, n - 8));
    };
    if constexpr (T == kGgmlQ3_K) q3_fetch(d0);
    for (int rr = 0; rr < rpw; ++rr) {
      const int d = d0 + rr;
      if (d >= L.H) break;  // uniform per wave
      const int64_t base = (int64_t)d * n;
      float a[kGgufBlkTok];
#pragma unroll
      for (int k = 0; k < kGgufBlkTok; ++k) a[k] = 0.0f;
      Q3Raw<8> cd[kGgufBlkCh];
      if constexpr (T == kGgmlQ3_K) {
#pragma unroll
        for (int ch = 0; ch < kGgufBlkCh; ++ch) cd[ch] = pd[ch];
        if (rr + 1 < rpw && d + 1 < L.H) q3_fetch(d + 1);
      }
#pragma unroll
      for (int ch = 0; ch < kGgufBlkCh; ++ch) {
        const int c = lane * 8 + 512 * ch;
        if (c < n) {
          f32x4 w4[2];
          if constexpr (T == kGgmlQ3_K)
            q3_decode<8>(cd[ch], w4);
          else
            valuesW<T, 8>(wd, base + c, L.layout, w4);
#pragma unroll
          for (int k = 0; k < kGgufBlkTok; ++k)
            if (k < nk) {
#pragma unroll
              for (int j = 0; j < 2; ++j) a[k] = dot4(w4[j], hv[k][ch][j], a[k]);
            }
        }
      }
#pragma unroll
      for (int k = 0; k < kGgufBlkTok; ++k) {
        if (k >= nk) break;  // uniform per wave
        const float v = wave_sum_dpp(a[k]);
        if (lane == 0) {
          const int t = tt[k], slot = sl[k];
          if (!finite_f(v))
            record_err(status, err_key(ut.sh ? kPhShared : kPhExpert, t, ut.sh ? 0 : slot,
                                       n + d, kEkDown));
          parts[((size_t)t * (L.K + 1) + slot) * L.H + d] = v;
        }
      }
    }
  }
}

// y[t][d] from parts[t][0..K][d]: k_gguf_down_combine's combine, thread per (t, d).
__global__ __launch_bounds__(256) void k_gguf_combine_parts(int K, int H, int ntok,
                                                            const float* __restrict__ parts,
                                                            const float* __restrict__ probs,
                                                            const float* __restrict__ shg,
                                                            const float* __restrict__ residual,
                                                            float* __restrict__ y,
                                                            unsigned long long* status) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)ntok * H) return;
  const int t = (int)(i / H), d = (int)(i % H);
  const float* pp = parts + (size_t)t * (K + 1) * H + d;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) acc = acc + probs[(size_t)t * K + k] * pp[(size_t)k * H];
  float total = acc + shg[t] * pp[(size_t)K * H];
  if (residual) total = total + residual[(size_t)t * H + d];
  if (!finite_f(total)) record_err(status, err_key(kPhAgg, t, 0, d, 0));
  y[(size_t)t * H + d] = total;
}

// ---- one token in one launch ------------------------------------------------
// k_gguf_one: one workgroup of 8 waves per CU, all resident together.  The
// routing runs as one task per wave (the tasks below): router groups on
// wave 0 of workgroups 0 .. nR - 1, the selection on wave 1 of workgroup 0,
// the softmax terms on wave 1 of workgroup 1, the shared expert's h rows on
// waves 2 .. 7 (row r on wave 2 + r % 6 of workgroup r / 6); each result is
// handed over as tagged words (launch << 32 | bits) at the device-coherent
// level, and every wait on them is a bounded poll.
constexpr int kFrontMaxH = 2048;
// sync area head: slot s's h count at 128 + 64 s, the selected experts as
// tagged words at kSelOff, the softmax terms (max, 1/S, shared gate) as
// tagged words at kSelOff + 64; then the tagged logits, the shared
// expert's h as tagged words and the routed slots' h
constexpr size_t kSyncHead = 1024;
constexpr size_t kSelOff = 768;
constexpr int kFrontRows = 4;
constexpr int kChainS = kFrontMaxH / 16 + 4;  // LDS row of x in chain order (4 pad floats)

// whether any of four values is not finite, without branches
__device__ __forceinline__ bool nonfinite4(const f32x4& q) {
  constexpr uint32_t e = 0x7F800000u;
  const int n = ((f2u(q.x) & e) == e) + ((f2u(q.y) & e) == e) + ((f2u(q.z) & e) == e) +
                ((f2u(q.w) & e) == e);
  return n != 0;
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ uint64_t tagged(unsigned launch, float v) {
  return ((uint64_t)launch << 32) | f2u(v);
}

// The shared expert's gate / up row r (as k_gguf_gateup's slot K) on one
// wave, h published as a tagged word.
template <int T>
__device__ __forceinline__ void shared_row_task(const GgufMoeDev& L, const float* __restrict__ x,
                                                int r, uint64_t* hsh, unsigned launch,
                                                unsigned long long* status) {
  const int lane = threadIdx.x & 63, H = L.H, E = L.E;
  const uint8_t* wg = L.raw + L.off[(size_t)E * 3 + 0];
  const uint8_t* wu = L.raw + L.off[(size_t)E * 3 + 1];
  const int64_t base = (int64_t)r * H;
  float ag = 0.0f, au = 0.0f;
  for (int c = lane * 16; c < H; c += 64 * 16) {
    f32x4 xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xv[j] = *reinterpret_cast<const f32x4*>(x + c + 4 * j);
    gu_dot16<T>(wg, wu, base + c, L.layout, xv, ag, au);
  }
  ag = wave_sum_dpp(ag);
  au = wave_sum_dpp(au);
  if (lane == 0) {
    const float hv = dm_silu(ag) * au;
    if (!finite_f(ag)) record_err(status, err_key(kPhShared, 0, 0, r, kEkGate));
    if (!finite_f(au)) record_err(status, err_key(kPhShared, 0, 0, r, kEkUp));
    if (!finite_f(hv)) record_err(status, err_key(kPhShared, 0, 0, r, kEkH));
    st_coh_u64(hsh + r, tagged(launch, hv));
  }
}

// Router rows 4 grp .. 4 grp + 3 (row E: the shared-expert gate) on one
// wave: lane 16 r + c runs chain c of row r (k = c, c + 16, ..., separate
// multiply and add), then the halving tree of the router kernels.  The
// chain's weights come four steps per float4 from the chain-ordered copy of
// the router (k_chain_router, rows of kFrontMaxH floats, zero past H), x
// from xt (LDS, this wave's) in chain order (zero past H: the extra steps
// add +0.0 to a sum that is never -0.0, which leaves it unchanged).  Each
// logit is published as a tagged word.
__device__ __forceinline__ void router_task(const GgufMoeDev& L, const float* __restrict__ x,
                                            int grp, uint64_t* zt, unsigned launch, float* xt,
                                            unsigned long long* status) {
  const int lane = threadIdx.x & 63, H = L.H, E = L.E;
  const int r = lane >> 4, c = lane & 15;
  const int e = grp * kFrontRows + r;
  const bool row = e <= E, chk = row && e != E;
  constexpr int kJ = kFrontMaxH / 256;  // float4 of x per lane
  constexpr int kQ = kFrontMaxH / 64;   // float4 of a chain
  // every load (clamped to the data) before the first LDS store
  f32x4 xv[kJ], wv[kQ];
#pragma unroll
  for (int j = 0; j < kJ; ++j)
    xv[j] = *reinterpret_cast<const f32x4*>(x + min(4 * lane + 256 * j, H - 4));
  const float* wr = L.rchain + (int64_t)min(e, E) * kFrontMaxH + 4 * c;
#pragma unroll
  for (int q = 0; q < kQ; ++q) wv[q] = *reinterpret_cast<const f32x4*>(wr + 64 * q);
  if (H < kFrontMaxH) {  // steps past H read zeros
    for (int i = lane; i < 16 * kChainS; i += 64) xt[i] = 0.0f;
  }
  // x to LDS in chain order (element k at (k & 15) kChainS + (k >> 4); the
  // clamped duplicates past H to the pad columns), every value checked
  bool bad_x = false, bad_w = false;
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const int k = 4 * lane + 256 * j;
    const bool in = k < H;
    const f32x4 q = xv[j];
    bad_x |= in && nonfinite4(q);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int kk = k + u;
      xt[(kk & 15) * kChainS + (in ? kk >> 4 : kFrontMaxH / 16 + ((kk >> 4) & 3))] = q[u];
    }
  }
#pragma unroll
  for (int q = 0; q < kQ; ++q) bad_w |= nonfinite4(wv[q]);
  bad_w = bad_w && chk;
  if (bad_x) record_err(status, err_key(kPhX, 0, 0, 0, 0));
  if (bad_w) record_err(status, err_key(kPhRouterW, 0, 0, 0, 0));
  wave_sync();
  float acc = 0.0f;
  const float* xc = xt + c * kChainS;
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const f32x4 xq = *reinterpret_cast<const f32x4*>(xc + 4 * q);
    acc = acc + xq.x * wv[q].x;
    acc = acc + xq.y * wv[q].y;
    acc = acc + xq.z * wv[q].z;
    acc = acc + xq.w * wv[q].w;
  }
#pragma unroll
  for (int wdt = 8; wdt >= 1; wdt >>= 1) {
    const float o = __shfl_down(acc, wdt, 16);
    if (c < wdt) acc = acc + o;
  }
  if (row && c == 0) {
    if (e != E && !finite_f(acc)) record_err(status, err_key(kPhLogit, 0, 0, e, 0));
    st_coh_u64(zt + e, tagged(launch, acc));
  }
}

// The top K on one wave: poll the tagged logits (bounded), topk_on_logits
// (on a near tie at the boundary the exact-probability rounds of
// route_select_token, on scratch in LDS), and the K experts, ordered by
// logit (then id), published as tagged words sel[k] (launch << 32 | id).
template <int R>
__device__ __forceinline__ void select_task(const GgufMoeDev& L, const uint64_t* zt,
                                            unsigned launch, uint64_t* sel, float* scr,
                                            unsigned long long* status, long lim) {
  const int lane = threadIdx.x & 63, E = L.E, K = L.K;
  float z[4 * R];
  if (!poll_logits<R>(zt, launch, E, z, nullptr, lim) && lane == 0)
    record_err(status, err_key(kPhSync, 0, 0, 0, 0));
  uint32_t fk[4 * R];
  int myid = 0;
  if (!topk_on_logits<R>(z, E, K, lane, fk, myid)) {
    // lane k < K: the k-th by key; ordered by (logit, then lower id), the
    // order the softmax's probabilities keep unless two of them round to
    // the same value (the probabilities' own order is formed later)
    myid = min(max(myid, 0), E - 1);
    // the logit of expert e sits in lane e & 63, entry e >> 6
    float zk = 0.0f;
#pragma unroll
    for (int i = 0; i < 4 * R; ++i) {
      const float zo = u2f((uint32_t)__builtin_amdgcn_ds_bpermute(4 * (myid & 63), (int)f2u(z[i])));
      zk = (myid >> 6) == i ? zo : zk;
    }
    const uint32_t kk = f2key(zk);
    int rank = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)kk, j);
      const int ij = __builtin_amdgcn_readlane(myid, j);
      if (j < K && lane < K)
        rank += (kj > kk || (kj == kk && (ij < myid || (ij == myid && j < lane)))) ? 1 : 0;
    }
    if (lane < K) st_coh_u64(sel + rank, ((uint64_t)launch << 32) | (uint32_t)myid);
  } else {
    // a near tie at the top-k boundary: the exact probabilities decide
    float* sz = scr;
    float* sm = scr + 512;
    int32_t* ids = reinterpret_cast<int32_t*>(scr + 1040);
    float* pr = scr + 1048;
#pragma unroll
    for (int i = 0; i < 4 * R; ++i)
      if (lane + 64 * i < E) sz[lane + 64 * i] = z[i];
    wave_sync();
    route_select_token<4 * R, false>(sz, 0, E, K, 0, 0, lane, sm, ids, pr, nullptr, status,
                                     [] { wave_sync(); });
    wave_sync();
    if (lane < K)
      st_coh_u64(sel + lane, ((uint64_t)launch << 32) | (uint32_t)min(max(ids[lane], 0), E - 1));
  }
}

// The softmax terms on one wave: poll the tagged logits and the
// shared-gate logit (bounded), then max z, 1/S (S the sum of
// exp(z - max) in expert order) and the shared gate with router_softmax's
// and the gate's checks (src/layers/router.mojo:140-183,
// src/layers/moe.mojo:70-100), published as tagged words soft[0..2].
template <int R>
__device__ __forceinline__ void softmax_task(const GgufMoeDev& L, const uint64_t* zt,
                                             unsigned launch, uint64_t* soft, float* scr,
                                             unsigned long long* status, long lim) {
  const int lane = threadIdx.x & 63, E = L.E;
  float z[4 * R], gl = 0.0f;
  if (!poll_logits<R>(zt, launch, E, z, &gl, lim) && lane == 0)
    record_err(status, err_key(kPhSync, 0, 0, 0, 0));
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < 4 * R; ++i)
    if (lane + 64 * i < E) m = z[i] > m ? z[i] : m;
  m = __ockl_wfred_max_f32(m);
  if (lane == 0 && !finite_f(m)) record_err(status, err_key(kPhSoftmax, 0, 0, 0, 0));
#pragma unroll
  for (int i = 0; i < 4 * R; ++i) {
    const int e = lane + 64 * i;
    if (e < E) {
      const float ev = dm_expf(z[i] - m);
      if (!finite_f(ev)) record_err(status, err_key(kPhSoftmax, 0, 0, 1 + e, 0));
      scr[e] = ev;
    }
  }
  wave_sync();
  if (lane == 0) {
    const float s = seq_sum(scr, E);
    if (!(s > 0.0f) || !finite_f(s)) record_err(status, err_key(kPhSoftmax, 0, 0, 1 + E, 0));
    if (!finite_f(gl)) record_err(status, err_key(kPhGate, 0, 0, 0, kGkLogit));
    const float g = dm_sigmoid(gl);
    if (!finite_f(g) || g < 0.0f || g > 1.0f)
      record_err(status, err_key(kPhGate, 0, 0, 0, kGkRange));
    st_coh_u64(soft + 0, tagged(launch, m));
    st_coh_u64(soft + 1, tagged(launch, 1.0f / s));
    st_coh_u64(soft + 2, tagged(launch, g));
  }
}

// Bounded poll of n (<= 64) tagged words, word l on lane l; their values
// (as bits) to v.  False on reaching the limit.
__device__ __forceinline__ bool poll_words(const uint64_t* p, int n, unsigned tag, long limit,
                                           uint32_t& v) {
  const int lane = threadIdx.x & 63;
  for (long spin = 0; spin < limit; ++spin) {
    const uint64_t wd = lane < n ? ld_coh_u64(p + lane) : 0;
    v = (uint32_t)wd;
    if (__builtin_amdgcn_ballot_w64(lane < n && (uint32_t)(wd >> 32) != tag) == 0) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// The chain-ordered copy of the router and the shared gate for router_task:
// rows of kFrontMaxH floats (row E: the shared gate) as float4 groups
// g = 16 q + c holding the elements c + 16 (4q + u), u = 0..3 (chain c's
// steps 4q .. 4q + 3; zero past H), so that group q of the 16 chains is one
// contiguous 256-byte read.
__global__ void k_chain_router(const float* __restrict__ router, const float* __restrict__ shgate,
                               int E, int H, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)(E + 1) * kFrontMaxH) return;
  const int e = (int)(i / kFrontMaxH), p = (int)(i % kFrontMaxH);
  const int q = p >> 6, c = (p >> 2) & 15, u = p & 3;
  const int k = c + 64 * q + 16 * u;
  const float* src = e == E ? shgate : router + (int64_t)e * H;
  out[i] = k < H ? src[k] : 0.0f;
}

// After the routing tasks every wave polls the selected experts.  Phase 1:
// the K x I routed (gate, up) row pairs in blocks of 16 per workgroup, every
// weight chunk requested before the first is used; a block's h goes to the
// device-coherent level as one write and the block is counted in its slot's
// counter (hcnt[16 s]).  Phase 2: workgroup b owns output rows 8b .. 8b + 7
// (and 8b + 8G ..): wave w requests the chunks of row 8b + w of the shared
// expert and of the 8 rows of routed slot w, polls the shared h, waits for
// slot w's count, and forms the dot products; eight lanes then combine each
// row in moe_aggregate_forward's order (y = sum_k p_k r_k + g r_sh
// (+ residual), k in probability order).  Wave kSoftWave forms the K
// probabilities and their order before phase 2 (gguf_slot_probs);
// workgroup 0 writes ids, probs and the shared gate.  Q3_K experts take
// the separate-load path (q3_load / q3_dot16); other types decode as they
// load.
// Bounded poll until *c reaches target (wrap-safe); on reaching the limit
// records a sync error and returns false, so that the caller skips later
// waits and the grid drains.
__device__ __forceinline__ bool wait_count(const unsigned* c, unsigned target,
                                           unsigned long long* status, long lim) {
  for (long i = 0; i < lim; ++i) {
    const unsigned v =
        __hip_atomic_load(const_cast<unsigned*>(c), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((int)(v - target) >= 0) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  record_err(status, err_key(kPhSync, 0, 0, 0, 0));
  return false;
}

__device__ __forceinline__ int64_t lane64(int64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// p_k = exp(z_k - max) * (1/S) for the K experts of the token (lane k < K:
// slot k's expert idk and its logit zk; max and 1/S from softmax_task,
// router_softmax's terms, src/layers/router.mojo:140-183), their
// (p desc, id asc) order and select_topk's checks (src/layers/topk.mojo:
// 109-128) on one wave.  To LDS: sp[r], sslot[r], sid[r] (probability, slot
// and id of rank r).  Only the `record` workgroup writes error keys; the
// renormalisation-leak check re-forms every probability from the tagged
// logits.
constexpr int kSoftWave = 7;
template <int R>
__device__ __forceinline__ void gguf_slot_probs(float zk, int idk, float m, float inv,
                                                const uint64_t* zt, int E, int K, float* sev,
                                                float* sp, int* sslot, int* sid, bool record,
                                                unsigned long long* status) {
  const int lane = threadIdx.x & 63;
  auto wave_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  };
  const float pk = lane < K ? dm_expf(zk - m) * inv : 0.0f;
  // rank of slot k: (p desc, id asc; the slot breaks any remaining tie so
  // that the ranks are a permutation whatever the inputs)
  const uint32_t kk = f2key(pk);
  int rank = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)kk, j);
    const int ij = __builtin_amdgcn_readlane(idk, j);
    if (j < K && lane < K)
      rank += (kj > kk || (kj == kk && (ij < idk || (ij == idk && j < lane)))) ? 1 : 0;
  }
  if (lane < K) {
    sp[rank] = pk;
    sslot[rank] = lane;
    sid[rank] = idk;
  }
  if (!record) return;
  wave_sync();
  float sum_topk = 0.0f;
#pragma unroll
  for (int r = 0; r < 8; ++r)
    if (r < K) sum_topk = sum_topk + sp[r];
  if (lane == 0 && sum_topk > 1.00001f) record_err(status, err_key(kPhTopk, 0, 0, 0, kTkSum));
  if (K < E && __builtin_fabsf(sum_topk - 1.0f) < 1e-6f) {
#pragma unroll
    for (int i = 0; i < 4 * R; ++i) {
      const int e = lane + 64 * i;
      if (e < E) sev[e] = dm_expf(u2f((uint32_t)ld_coh_u64(zt + e)) - m) * inv;
    }
    wave_sync();
    const float sum_all = seq_sum(sev, E);
    if (lane == 0 && sum_all - sum_topk > 1e-5f)
      record_err(status, err_key(kPhTopk, 0, 0, 0, kTkLeak));
  }
}

// Bounded poll of a lane's eight tagged words (launch << 32 | bits) until
// every lane's words carry this launch's tag; false on reaching the limit.
__device__ __forceinline__ bool poll8(const uint64_t* p, unsigned tag, long limit,
                                      f32x4 (&v)[2]) {
  for (long spin = 0; spin < limit; ++spin) {
    uint64_t wd[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) wd[q] = ld_coh_u64(p + q);
    bool ok = true;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      ok &= (uint32_t)(wd[q] >> 32) == tag;
      v[q >> 2][q & 3] = u2f((uint32_t)wd[q]);
    }
    if (__builtin_amdgcn_ballot_w64(!ok) == 0) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

template <int T, int R>
// The leading arguments (what the routing and shared-expert tasks need for
// their first loads) are preloaded into scalar registers at dispatch
// (dm_gguf.hip is compiled with -amdgpu-kernarg-preload-count): those loads
// are issued without waiting for a read of the argument segment.
__global__ __launch_bounds__(512) void k_gguf_one(
    const float* __restrict__ x, const float* __restrict__ rchain_, const uint8_t* raw_,
    const int64_t* off_, int H_, int E_, int Ish_, int nR, GgufMoeDev Lk, uint64_t* zt,
    uint64_t* sel,
    uint64_t* soft, uint64_t* hsh, const float* __restrict__ residual, float* __restrict__ y,
    int32_t* __restrict__ ids, float* __restrict__ probs, float* __restrict__ shg,
    float* __restrict__ h, int ldh, unsigned* hcnt, unsigned target, unsigned launch,
    unsigned long long* status, long lim) {
  __shared__ __attribute__((aligned(16))) float xt[16 * kChainS];
  __shared__ __attribute__((aligned(16))) float scr[1056];
  __shared__ float part[8][33];
  __shared__ float sev[256 * R];
  __shared__ float sp[8];
  __shared__ int sslot[8], sid[8];
  GgufMoeDev L = Lk;  // the entry fields from the preloaded arguments
  L.H = H_;
  L.E = E_;
  L.Ish = Ish_;
  L.rchain = rchain_;
  L.raw = raw_;
  L.off = off_;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wid = __builtin_amdgcn_readfirstlane(w);  // w as a uniform value
  const int G = (int)gridDim.x, b = (int)blockIdx.x;
  const int H = L.H, E = L.E, K = L.K, I = L.I, Ish = L.Ish;
  // ---- the routing and the shared expert's h, one task per wave
  if (wid == 0) {
    if (b < nR) router_task(L, x, b, zt, launch, xt, status);
  } else if (wid == 1) {
    if (b == 0) select_task<R>(L, zt, launch, sel, scr, status, lim);
    if (b == 1) softmax_task<R>(L, zt, launch, soft, scr, status, lim);
  } else if (6 * b + wid - 2 < Ish) {
    shared_row_task<T>(L, x, 6 * b + wid - 2, hsh, launch, status);
  }
  // the selected experts: one wave per workgroup polls them (a poll by
  // every wave would crowd the memory the routing tasks are using); wave 0,
  // whose router task ends before the selection does (wave 1 of workgroup
  // 1 forms the softmax terms until after the ids are out)
  __shared__ int sel_ids[8];
  if (wid == 0) {
    uint32_t sv = 0;
    if (!poll_words(sel, K, launch, lim, sv) && lane == 0)
      record_err(status, err_key(kPhSync, 0, 0, 0, 0));
    if (lane < K) sel_ids[lane] = min(max((int)sv, 0), E - 1);
  }
  __syncthreads();
  // lane s < K: the expert and payload offsets of routed slot s
  const int es = sel_ids[min(lane, K - 1)];
  int64_t og, ou, od;
  if (L.estride > 0) {
    og = (int64_t)(3 * es) * L.estride;
    ou = og + L.estride;
    od = ou + L.estride;
  } else {
    og = L.off[(size_t)es * 3 + 0];
    ou = L.off[(size_t)es * 3 + 1];
    od = L.off[(size_t)es * 3 + 2];
  }
  // for the combine: the slot's logit (requested after the offsets, so
  // that waiting for those does not wait for it)
  const float zk = u2f((uint32_t)ld_coh_u64(zt + es));
  const uint8_t* wsh = L.raw + L.off[(size_t)E * 3 + 2];
  const int cs = min(lane * 8, Ish - 8), cr = min(lane * 8, I - 8);
  const int dfirst = (int)blockIdx.x * 8;
  // Done once, in the shadow of the first gate / up requests (or after phase
  // 1 when the workgroup has no block): wave 0 reads the shared expert's h
  // into LDS, wave kSoftWave forms the K probabilities and their order.
  __shared__ float sg;  // the shared gate
  __shared__ __attribute__((aligned(16))) float hshl[512];
  bool side_done = false;
  auto side_work = [&]() {
    side_done = true;
    if (wid == 0) {
      f32x4 hv[2];
      if (!poll8(hsh + cs, launch, lim, hv) && lane == 0)
        record_err(status, err_key(kPhSync, 0, 0, 0, 0));
      if (lane * 8 < Ish) {
        *reinterpret_cast<f32x4*>(hshl + lane * 8) = hv[0];
        *reinterpret_cast<f32x4*>(hshl + lane * 8 + 4) = hv[1];
      }
    }
    if (wid == kSoftWave) {
      uint32_t tv = 0;
      if (!poll_words(soft, 3, launch, lim, tv) && lane == 0)
        record_err(status, err_key(kPhSync, 0, 0, 0, 0));
      const float sm_max = u2f((uint32_t)__builtin_amdgcn_readlane((int)tv, 0));
      const float sm_inv = u2f((uint32_t)__builtin_amdgcn_readlane((int)tv, 1));
      if (lane == 2) sg = u2f(tv);
      gguf_slot_probs<R>(zk, es, sm_max, sm_inv, zt, E, K, sev, sp, sslot, sid, b == 0, status);
    }
  };
  // ---- phase 1: routed gate / up.  Workgroup b takes blocks of 16 row
  // pairs (16 pb .. 16 pb + 15 of slot 16 pb / I; wave w rows 2w, 2w + 1),
  // publishes the block's 16 h values as one write and counts the block in
  // its slot's counter.
  __shared__ float hs[16];
  for (int pb = (int)blockIdx.x; pb < K * I / 16; pb += G) {
    const int slot = pb * 16 / I, r0 = pb * 16 - slot * I + 2 * w;
    float ag[2] = {0.0f, 0.0f}, au[2] = {0.0f, 0.0f};
    const uint8_t* wg = L.raw + lane64(og, slot);
    const uint8_t* wu = L.raw + lane64(ou, slot);
    if constexpr (T == kGgmlQ3_K) {
      constexpr int NJ = kFrontMaxH / 1024;  // chunks of 16 weights per lane and row
      Q3Raw<16> rg[2][NJ], ru[2][NJ];
      f32x4 xv[NJ][4];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int c = min(lane * 16 + 1024 * j, H - 16);
          rg[q][j] = q3_load<16>(wg, (int64_t)(r0 + q) * H + c);
          ru[q][j] = q3_load<16>(wu, (int64_t)(r0 + q) * H + c);
        }
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int c = min(lane * 16 + 1024 * j, H - 16);
#pragma unroll
        for (int u = 0; u < 4; ++u) xv[j][u] = *reinterpret_cast<const f32x4*>(x + c + 4 * u);
      }
      if (!side_done) side_work();
      float xs[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) xs[j] = xsum16(xv[j]);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          // every chunk is used (an unused load left in flight would hold
          // its registers); chunks past H do not enter the sums
          const bool in = lane * 16 + 1024 * j < H;
          const float a = q3_dot16(rg[q][j], xv[j], xs[j], ag[q]);
          const float bu = q3_dot16(ru[q][j], xv[j], xs[j], au[q]);
          ag[q] = in ? a : ag[q];
          au[q] = in ? bu : au[q];
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int64_t base = (int64_t)(r0 + q) * H;
        for (int c = lane * 16; c < H; c += 64 * 16) {
          f32x4 g4[4], u4[4];
          valuesW<T, 16>(wg, base + c, L.layout, g4);
          valuesW<T, 16>(wu, base + c, L.layout, u4);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const f32x4 xq = *reinterpret_cast<const f32x4*>(x + c + 4 * u);
            ag[q] = dot4(g4[u], xq, ag[q]);
            au[q] = dot4(u4[u], xq, au[q]);
          }
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float a = wave_sum_dpp(ag[q]), b = wave_sum_dpp(au[q]);
      if (lane == 0) {
        const float hv = dm_silu(a) * b;
        if (!finite_f(a)) record_err(status, err_key(kPhExpert, 0, slot, r0 + q, kEkGate));
        if (!finite_f(b)) record_err(status, err_key(kPhExpert, 0, slot, r0 + q, kEkUp));
        if (!finite_f(hv)) record_err(status, err_key(kPhExpert, 0, slot, r0 + q, kEkH));
        hs[2 * w + q] = hv;
      }
    }
    __syncthreads();
    if (threadIdx.x < 16) {
      st_coh(h + (size_t)slot * ldh + pb * 16 - slot * I + threadIdx.x, hs[threadIdx.x]);
      wait_stores();
    }
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(hcnt + 16 * slot, 1u);
  }
  // phase 2's first rows: their down chunks requested now, in flight
  // while the slots' h counts are awaited (Q3_K)
  const uint8_t* wrd = L.raw + lane64(od, min(w, K - 1));
  Q3Raw<8> pre_s, pre_r[8];
  if constexpr (T == kGgmlQ3_K) {
    pre_s = q3_load<8>(wsh, (int64_t)min(dfirst + w, H - 1) * Ish + cs);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      pre_r[i] = q3_load<8>(wrd, (int64_t)min(dfirst + i, H - 1) * I + cr);
  }
  if (!side_done) side_work();
  __syncthreads();  // hshl, sp, sslot, sid, sg
  // ---- phase 2: down projections and the combine
  bool ready = false;
  const bool ls = lane * 8 < Ish, lr = lane * 8 < I;
  for (int d0 = (int)blockIdx.x * 8; d0 < H; d0 += 8 * G) {
    const int nd = min(8, H - d0);
    f32x4 ws[2], wr[8][2];
    if constexpr (T == kGgmlQ3_K) {
      if (d0 != dfirst) {
        pre_s = q3_load<8>(wsh, (int64_t)min(d0 + w, H - 1) * Ish + cs);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          pre_r[i] = q3_load<8>(wrd, (int64_t)min(d0 + i, H - 1) * I + cr);
      }
      q3_decode<8>(pre_s, ws);
#pragma unroll
      for (int i = 0; i < 8; ++i) q3_decode<8>(pre_r[i], wr[i]);
    } else {
      valuesW<T, 8>(wsh, (int64_t)min(d0 + w, H - 1) * Ish + cs, L.layout, ws);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        valuesW<T, 8>(wrd, (int64_t)min(d0 + i, H - 1) * I + cr, L.layout, wr[i]);
    }
    // the shared expert's row d0 + w
    {
      const float* hp = hshl + cs;
      float a = dot4(ws[0], *reinterpret_cast<const f32x4*>(hp), 0.0f);
      a = dot4(ws[1], *reinterpret_cast<const f32x4*>(hp + 4), a);
      a = wave_sum_dpp(ls ? a : 0.0f);
      if (lane == 0 && w < nd) {
        if (!finite_f(a)) record_err(status, err_key(kPhShared, 0, 0, Ish + d0 + w, kEkDown));
        part[w][K] = a;
      }
    }
    if (w < K) {
      if (!ready) ready = wait_count(hcnt + 16 * w, target, status, lim);
      f32x4 hv[2];
      const float* hp = h + (size_t)w * ldh + cr;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint64_t v = ld_coh_u64(hp + 2 * q);
        hv[q >> 1][(q & 1) * 2] = u2f((uint32_t)v);
        hv[q >> 1][(q & 1) * 2 + 1] = u2f((uint32_t)(v >> 32));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float a = dot4(wr[i][0], hv[0], 0.0f);
        a = dot4(wr[i][1], hv[1], a);
        a = wave_sum_dpp(lr ? a : 0.0f);
        if (i < nd && lane == 0) {
          if (!finite_f(a)) record_err(status, err_key(kPhExpert, 0, w, I + d0 + i, kEkDown));
          part[i][w] = a;
        }
      }
    }
    const float res = residual && (int)threadIdx.x < nd ? residual[d0 + threadIdx.x] : 0.0f;
    __syncthreads();
    if ((int)threadIdx.x < nd) {
      const int i = threadIdx.x, d = d0 + i;
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < K) acc = acc + sp[k] * part[i][sslot[k]];
      float total = acc + sg * part[i][K];
      if (residual) total = total + res;
      if (!finite_f(total)) record_err(status, err_key(kPhAgg, 0, 0, d, 0));
      y[d] = total;
    }
    if (blockIdx.x == 0 && d0 == 0) {
      if ((int)threadIdx.x < K) {
        ids[threadIdx.x] = sid[threadIdx.x];
        probs[threadIdx.x] = sp[threadIdx.x];
      }
      if (threadIdx.x == 0) shg[0] = sg;
    }
    __syncthreads();
  }
}

}  // namespace

int gguf_block_spec(int t, int* bs, int* bpb) {
  switch (t) {
    case kGgmlF32: *bs = 1; *bpb = 4; return 0;
    case kGgmlBF16: *bs = 1; *bpb = 2; return 0;
    case kGgmlQ8_0: *bs = 32; *bpb = 34; return 0;
    case kGgmlQ4_K: *bs = 256; *bpb = 144; return 0;
    case kGgmlQ3_K: *bs = 256; *bpb = 114; return 0;
    default: return -1;
  }
}

hipError_t launch_dequant_gguf(int t, const uint8_t* raw, int64_t n, int layout, float* out,
                               hipStream_t st) {
  int bs = 0, bpb = 0;
  if (gguf_block_spec(t, &bs, &bpb) || n <= 0) return hipErrorInvalidValue;
  const int64_t n_blk = n / bs * bs;
  const int64_t quads = (n + 3) / 4;
  if ((quads + 255) / 256 > 0x7FFFFFFF) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((quads + 255) / 256)), block(256);
  switch (t) {
    case kGgmlQ8_0: k_dequant_gguf<kGgmlQ8_0><<<grid, block, 0, st>>>(raw, n, n_blk, layout, out); break;
    case kGgmlQ4_K: k_dequant_gguf<kGgmlQ4_K><<<grid, block, 0, st>>>(raw, n, n_blk, layout, out); break;
    case kGgmlQ3_K: k_dequant_gguf<kGgmlQ3_K><<<grid, block, 0, st>>>(raw, n, n_blk, layout, out); break;
    case kGgmlBF16: k_dequant_gguf<kGgmlBF16><<<grid, block, 0, st>>>(raw, n, n_blk, layout, out); break;
    default: k_dequant_gguf<kGgmlF32><<<grid, block, 0, st>>>(raw, n, n_blk, layout, out); break;
  }
  return hipGetLastError();
}

// eight weights per lane when every row length allows it, else four
#define DM_GGUF_DISPATCH_W(KERNEL, W, GRID, ...)                                          \
  switch (L.type) {                                                                       \
    case kGgmlQ8_0: KERNEL<kGgmlQ8_0, W><<<GRID, 256, 0, st>>>(__VA_ARGS__); break;       \
    case kGgmlQ4_K: KERNEL<kGgmlQ4_K, W><<<GRID, 256, 0, st>>>(__VA_ARGS__); break;       \
    case kGgmlQ3_K: KERNEL<kGgmlQ3_K, W><<<GRID, 256, 0, st>>>(__VA_ARGS__); break;       \
    case kGgmlBF16: KERNEL<kGgmlBF16, W><<<GRID, 256, 0, st>>>(__VA_ARGS__); break;       \
    case kGgmlF32: KERNEL<kGgmlF32, W><<<GRID, 256, 0, st>>>(__VA_ARGS__); break;         \
    default: return hipErrorInvalidValue;                                                 \
  }
#define DM_GGUF_DISPATCH_T(KERNEL, GRID, ...)                                             \
  switch (L.type) {                                                                       \
    case kGgmlQ8_0: KERNEL<kGgmlQ8_0><<<GRID, 256, 0, st>>>(__VA_ARGS__); break;          \
    case kGgmlQ4_K: KERNEL<kGgmlQ4_K><<<GRID, 256, 0, st>>>(__VA_ARGS__); break;          \
    case kGgmlQ3_K: KERNEL<kGgmlQ3_K><<<GRID, 256, 0, st>>>(__VA_ARGS__); break;          \
    case kGgmlBF16: KERNEL<kGgmlBF16><<<GRID, 256, 0, st>>>(__VA_ARGS__); break;          \
    case kGgmlF32: KERNEL<kGgmlF32><<<GRID, 256, 0, st>>>(__VA_ARGS__); break;            \
    default: return hipErrorInvalidValue;                                                 \
  }
#define DM_GGUF_DISPATCH(KERNEL, GRID, ...)                                               \
  if (L.H % 8 == 0 && L.I % 8 == 0 && L.Ish % 8 == 0) {                                   \
    DM_GGUF_DISPATCH_W(KERNEL, 8, GRID, __VA_ARGS__)                                      \
  } else {                                                                                \
    DM_GGUF_DISPATCH_W(KERNEL, 4, GRID, __VA_ARGS__)                                      \
  }

hipError_t launch_gguf_gateup(const GgufMoeDev& L, const float* x, int T, const int32_t* ids,
                              float* h, int ldh, unsigned long long* status, hipStream_t st) {
  if (T <= 0 || L.H % 4 || L.I % 4 || L.Ish % 4 || ldh % 4 || ldh < L.I || ldh < L.Ish)
    return hipErrorInvalidValue;
  const int rows = L.I > L.Ish ? L.I : L.Ish;
  const int chunk = 65535 / (L.K + 1);  // tokens per launch: grid.y <= 65535
  for (int t0 = 0; t0 < T; t0 += chunk) {
    const int n = T - t0 < chunk ? T - t0 : chunk;
    const dim3 grid((unsigned)((rows + 3) / 4), (unsigned)(n * (L.K + 1)));
    if (L.H % 16 == 0) {  // rows of H weights: sixteen per lane
      DM_GGUF_DISPATCH_W(k_gguf_gateup, 16, grid, L, x, ids, h, ldh, status, t0)
    } else {
      DM_GGUF_DISPATCH(k_gguf_gateup, grid, L, x, ids, h, ldh, status, t0)
    }
  }
  return hipGetLastError();
}

hipError_t launch_gguf_down_combine(const GgufMoeDev& L, const float* h, int ldh, int T,
                                    const int32_t* ids, const float* probs, const float* shg,
                                    const float* residual, float* y, unsigned long long* status,
                                    hipStream_t st) {
  if (T <= 0 || L.K > 32 || L.H % 4 || L.I % 4 || L.Ish % 4 || ldh % 4)
    return hipErrorInvalidValue;
  for (int t0 = 0; t0 < T; t0 += 65535) {
    const int n = T - t0 < 65535 ? T - t0 : 65535;
    const dim3 grid((unsigned)L.H, (unsigned)n);
    DM_GGUF_DISPATCH(k_gguf_down_combine, grid, L, h, ldh, ids, probs, shg, residual, y, status, t0)
  }
  return hipGetLastError();
}
hipError_t launch_gguf_units(const GgufMoeDev& L, const float* x, int T, const int32_t* off,
                             const int32_t* perm, const int2* units, const int32_t* meta,
                             int nunits, float* h, int ldh, float* parts, const float* probs,
                             const float* shg, const float* residual, float* y,
                             unsigned long long* status, hipStream_t st) {
  if (T <= 0 || nunits <= 0 || L.K <= 0 || L.H % 4 || L.I % 4 || L.Ish % 4 || ldh % 4 ||
      ldh < L.I || ldh < L.Ish)
    return hipErrorInvalidValue;
  const int rows = L.I > L.Ish ? L.I : L.Ish;
  // rows per wave of the blocked forms: one for few tokens (the units hold
  // one or two, and more waves hide more latency), up to eight as the units fill
  const int rpw = T >= 512 ? kGgufBlkRowsMax : T >= 128 ? 4 : T >= 32 ? 2 : 1;  // (T >= 128 in use)
  for (int u0 = 0; u0 < nunits; u0 += 65535) {
    const int n = nunits - u0 < 65535 ? nunits - u0 : 65535;
    const dim3 grid((unsigned)((rows + 3) / 4), (unsigned)n);
    if (L.H % 16 == 0 && L.H <= 64 * 16 * kGgufBlkCh) {  // as launch_gguf_gateup: W = 16
      const dim3 gb((unsigned)((rows + 4 * rpw - 1) / (4 * rpw)), (unsigned)n);
      DM_GGUF_DISPATCH_T(k_gguf_gateup_units_blk, gb, L, x, off, perm, units, meta, T, h, ldh,
                         status, u0, rpw)
    } else if (L.H % 16 == 0) {
      DM_GGUF_DISPATCH_W(k_gguf_gateup_units, 16, grid, L, x, off, perm, units, meta, T, h, ldh,
                         status, u0)
    } else {
      DM_GGUF_DISPATCH(k_gguf_gateup_units, grid, L, x, off, perm, units, meta, T, h, ldh, status,
                       u0)
    }
  }
  for (int u0 = 0; u0 < nunits; u0 += 65535) {
    const int n = nunits - u0 < 65535 ? nunits - u0 : 65535;
    const dim3 grid((unsigned)((L.H + 3) / 4), (unsigned)n);
    const int nmax = L.I > L.Ish ? L.I : L.Ish;
    if (L.H % 8 == 0 && L.I % 8 == 0 && L.Ish % 8 == 0 && nmax <= 64 * 8 * kGgufBlkCh) {
      // as launch_gguf_down_combine: W = 8
      const dim3 gb((unsigned)((L.H + 4 * rpw - 1) / (4 * rpw)), (unsigned)n);
      DM_GGUF_DISPATCH_T(k_gguf_down_units_blk, gb, L, h, ldh, off, perm, units, meta, T, parts,
                         status, u0, rpw)
    } else {
      DM_GGUF_DISPATCH(k_gguf_down_units, grid, L, h, ldh, off, perm, units, meta, T, parts,
                       status, u0)
    }
  }
  const int64_t nt = (int64_t)T * L.H;
  hipLaunchKernelGGL(k_gguf_combine_parts, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, st,
                     L.K, L.H, T, parts, probs, shg, residual, y, status);
  return hipGetLastError();
}
#undef DM_GGUF_DISPATCH
#undef DM_GGUF_DISPATCH_W
#undef DM_GGUF_DISPATCH_T

bool gguf_one_token_supported(const GgufMoeDev& L) {
  return L.H % 64 == 0 && L.H <= kFrontMaxH && L.I % 16 == 0 && L.I <= 512 && L.Ish % 8 == 0 &&
         L.Ish <= 512 && L.K <= 8 && L.E + 1 <= 512 && L.type != kGgmlF32 && L.type != kGgmlBF16;
}

static size_t zt_bytes(const GgufMoeDev& L) { return ((size_t)(L.E + 1) * 8 + 255) & ~(size_t)255; }

static size_t hsh_bytes(const GgufMoeDev& L) { return ((size_t)L.Ish * 8 + 255) & ~(size_t)255; }

size_t gguf_one_token_sync_bytes(const GgufMoeDev& L) {
  return kSyncHead + zt_bytes(L) + hsh_bytes(L) + (size_t)L.K * L.I * 4;
}

size_t gguf_chain_router_bytes(const GgufMoeDev& L) {
  return (size_t)(L.E + 1) * kFrontMaxH * sizeof(float);
}

hipError_t launch_chain_router(const GgufMoeDev& L, float* out, hipStream_t st) {
  if (L.H % 64 || L.H > kFrontMaxH || L.E < 1) return hipErrorInvalidValue;
  const int64_t n = (int64_t)(L.E + 1) * kFrontMaxH;
  k_chain_router<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(L.router, L.shgate, L.E, L.H, out);
  return hipGetLastError();
}

bool gguf_one_token_grid_ok(const GgufMoeDev& L, int grid) {
  const int nR = (L.E + 1 + kFrontRows - 1) / kFrontRows;
  return grid >= 2 && grid >= nR && 6 * grid >= L.Ish;
}

int gguf_experts_occupancy(const GgufMoeDev& L, int* per_cu) {
  hipError_t e = hipErrorInvalidValue;
  const bool r1 = L.E <= 256;
#define DM_OCC(TY)                                                                                \
  e = r1 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, k_gguf_one<TY, 1>, 512, 0)   \
         : hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, k_gguf_one<TY, 2>, 512, 0)
  switch (L.type) {
    case kGgmlQ8_0: DM_OCC(kGgmlQ8_0); break;
    case kGgmlQ4_K: DM_OCC(kGgmlQ4_K); break;
    case kGgmlQ3_K: DM_OCC(kGgmlQ3_K); break;
    default: break;
  }
#undef DM_OCC
  return e == hipSuccess ? 0 : -1;
}

hipError_t launch_gguf_one_token(const GgufMoeDev& L, const float* x, const float* residual,
                                 float* y, int32_t* ids, float* probs, float* shg, void* sync,
                                 unsigned launch, int grid, unsigned long long* status,
                                 hipStream_t st, long spin) {
  const int nR = (L.E + 1 + kFrontRows - 1) / kFrontRows;
  if (!gguf_one_token_supported(L) || !L.rchain || !gguf_one_token_grid_ok(L, grid) ||
      launch == 0)
    return hipErrorInvalidValue;
  uint8_t* sb = static_cast<uint8_t*>(sync);
  unsigned* hcnt = reinterpret_cast<unsigned*>(sb + 128);  // slot s at 64 s bytes
  uint64_t* sel = reinterpret_cast<uint64_t*>(sb + kSelOff);
  uint64_t* soft = reinterpret_cast<uint64_t*>(sb + kSelOff + 64);
  uint64_t* zt = reinterpret_cast<uint64_t*>(sb + kSyncHead);
  uint64_t* hsh = reinterpret_cast<uint64_t*>(sb + kSyncHead + zt_bytes(L));
  float* h = reinterpret_cast<float*>(sb + kSyncHead + zt_bytes(L) + hsh_bytes(L));
  const unsigned target = launch * (unsigned)(L.I / 16);  // blocks per slot
#define DM_ONE(TY, R)                                                                          \
  k_gguf_one<TY, R><<<grid, 512, 0, st>>>(x, L.rchain, L.raw, L.off, L.H, L.E, L.Ish, nR, L, zt, \
                                          sel, soft, hsh, residual, y, ids, probs,             \
                                          shg, h, L.I, hcnt, target, launch, status, spin)
#define DM_ONE_R(TY)    \
  if (L.E <= 256) {     \
    DM_ONE(TY, 1);      \
  } else {              \
    DM_ONE(TY, 2);      \
  }
  switch (L.type) {
    case kGgmlQ8_0: DM_ONE_R(kGgmlQ8_0) break;
    case kGgmlQ4_K: DM_ONE_R(kGgmlQ4_K) break;
    case kGgmlQ3_K: DM_ONE_R(kGgmlQ3_K) break;
    default: return hipErrorInvalidValue;
  }
#undef DM_ONE_R
#undef DM_ONE
  return hipGetLastError();
}

}  // namespace dm
