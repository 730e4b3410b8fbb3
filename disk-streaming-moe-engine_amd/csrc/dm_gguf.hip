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

// W consecutive weights at element e0 (a multiple of W, W in {4, 8, 16}).
// For Q3_K eight weights share one hmask byte, two code bytes, the scale
// byte and d, so the block header is decoded once per eight (sixteen).
template <int T, int W>
__device__ __forceinline__ void valuesW(const uint8_t* raw, int64_t e0, int layout, f32x4 (&v)[W / 4]) {
  if constexpr (T == kGgmlQ3_K && W == 16) {
    // sixteen weights: two hmask bytes, four code bytes, one scale byte
    const uint8_t* blk = raw + (e0 >> 8) * 114;
    const int e = (int)(e0 & 255);
    const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
    const uint32_t hm = h[e >> 4];
    const uint32_t qs = (uint32_t)h[16 + (e >> 3)] | ((uint32_t)h[17 + (e >> 3)] << 16);
    const float fs = (float)((int)blk[96 + (e >> 4)] - 32) * h2f(h[56]);
    float w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      w[i] = fs * (float)((int)((((hm >> i) & 1) << 2) | ((qs >> (2 * i)) & 3)) - 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = f32x4{w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
  } else if constexpr (T == kGgmlQ3_K && W == 8) {
    const uint8_t* blk = raw + (e0 >> 8) * 114;
    const int e = (int)(e0 & 255);
    const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
    const uint32_t hm = blk[e >> 3];
    const uint32_t qs = h[16 + (e >> 3)];  // code bytes 32 + e/4 and the next
    const float fs = (float)((int)blk[96 + (e >> 4)] - 32) * h2f(h[56]);
    float w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      w[i] = fs * (float)((int)((((hm >> i) & 1) << 2) | ((qs >> (2 * i)) & 3)) - 4);
    v[0] = f32x4{w[0], w[1], w[2], w[3]};
    v[1] = f32x4{w[4], w[5], w[6], w[7]};
  } else {
#pragma unroll
    for (int j = 0; j < W / 4; ++j) v[j] = values4<T>(raw, e0 + 4 * j, layout);
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

// ---- one token in two launches ----------------------------------------------
// The bytes of W consecutive Q3_K weights (W = 8 or 16, at an element that
// is a multiple of W) as separate loads, so that a wave can request every
// chunk it needs before decoding the first (valuesW decodes as it loads).
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
  float w[W];
#pragma unroll
  for (int i = 0; i < W; ++i)
    w[i] = fs * (float)((int)((((r.hm >> i) & 1) << 2) | ((qs >> (2 * i)) & 3)) - 4);
#pragma unroll
  for (int j = 0; j < W / 4; ++j) v[j] = f32x4{w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
}

// k_gguf_front: workgroups 0 .. nR - 1 (one wave each) form the router logits
// of rows 2b and 2b + 1 (row E: the shared-expert gate) in router_project's
// order (16 lane chains k = l, l + 16, ..., the halving tree, the tail on
// lane 0: the order of the router kernels), and publish them at the
// device-coherent level; the last of them to arrive runs the softmax / top-k
// (route_select_token).  Workgroups nR .. nR + Ish - 1 form the shared
// expert's h rows meanwhile (they do not depend on the routing).
constexpr int kFrontMaxH = 2048;
constexpr size_t kSyncHead = 1024;  // counters: front at 0, slot s's h count at 128 + 64 s
constexpr int kFrontRows = 2;

template <int T, int W, int NE>
__global__ __launch_bounds__(64) void k_gguf_front(GgufMoeDev L, const float* __restrict__ x,
                                                   int nR, float* __restrict__ z,
                                                   float* __restrict__ h, int ldh,
                                                   unsigned* front, int32_t* __restrict__ ids,
                                                   float* __restrict__ probs,
                                                   float* __restrict__ shg,
                                                   unsigned long long* status) {
  __shared__ __attribute__((aligned(16))) float sx[kFrontMaxH];
  __shared__ __attribute__((aligned(16))) float sw[kFrontRows][kFrontMaxH + 16];
  const int lane = threadIdx.x, H = L.H, E = L.E;
  if ((int)blockIdx.x >= nR) {
    // the shared expert's gate / up row r (as k_gguf_gateup's slot K)
    const int r = (int)blockIdx.x - nR;
    const uint8_t* wg = L.raw + L.off[(size_t)E * 3 + 0];
    const uint8_t* wu = L.raw + L.off[(size_t)E * 3 + 1];
    const int64_t base = (int64_t)r * H;
    float ag = 0.0f, au = 0.0f;
    for (int c = lane * W; c < H; c += 64 * W) {
      f32x4 g4[W / 4], u4[W / 4];
      valuesW<T, W>(wg, base + c, L.layout, g4);
      valuesW<T, W>(wu, base + c, L.layout, u4);
#pragma unroll
      for (int j = 0; j < W / 4; ++j) {
        const f32x4 xv = *reinterpret_cast<const f32x4*>(x + c + 4 * j);
        ag = dot4(g4[j], xv, ag);
        au = dot4(u4[j], xv, au);
      }
    }
    ag = wave_sum_dpp(ag);
    au = wave_sum_dpp(au);
    if (lane == 0) {
      const float hv = dm_silu(ag) * au;
      if (!finite_f(ag)) record_err(status, err_key(kPhShared, 0, 0, r, kEkGate));
      if (!finite_f(au)) record_err(status, err_key(kPhShared, 0, 0, r, kEkUp));
      if (!finite_f(hv)) record_err(status, err_key(kPhShared, 0, 0, r, kEkH));
      h[(size_t)L.K * ldh + r] = hv;
    }
    return;
  }
  // x and the workgroup's rows to LDS, every value checked as it is read
  const int row0 = (int)blockIdx.x * kFrontRows;
  bool bad_x = false, bad_w = false;
  {
    // x and the rows: every load (clamped to the data) issued before the
    // first LDS store
    constexpr int kJ = kFrontMaxH / 256;
    f32x4 v[kFrontRows + 1][kJ];
#pragma unroll
    for (int r = 0; r <= kFrontRows; ++r) {
      const int e = min(row0 + r - 1, E);
      const float* src = r == 0 ? x : e == E ? L.shgate : L.router + (int64_t)e * H;
#pragma unroll
      for (int j = 0; j < kJ; ++j)
        v[r][j] = *reinterpret_cast<const f32x4*>(src + min(4 * lane + 256 * j, H - 4));
    }
#pragma unroll
    for (int r = 0; r <= kFrontRows; ++r) {
      const int e = row0 + r - 1;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int k = 4 * lane + 256 * j;
        if (k >= H || (r > 0 && e > E)) continue;
        const f32x4 q = v[r][j];
        const bool bad = !finite_f(q.x) || !finite_f(q.y) || !finite_f(q.z) || !finite_f(q.w);
        if (r == 0) {
          bad_x |= bad;
          *reinterpret_cast<f32x4*>(&sx[k]) = q;
        } else {
          if (e != E) bad_w |= bad;
          *reinterpret_cast<f32x4*>(&sw[r - 1][k]) = q;
        }
      }
    }
  }
  if (bad_x) record_err(status, err_key(kPhX, 0, 0, 0, 0));
  if (bad_w) record_err(status, err_key(kPhRouterW, 0, 0, 0, 0));
  __syncthreads();
  const int l = lane & 15, r = lane >> 4, e = row0 + r;
  const bool row = r < kFrontRows && e <= E;
  const int h16 = H & ~15;
  float acc = 0.0f;
  if (row) {
#pragma unroll 8
    for (int k = l; k < h16; k += 16) acc = acc + sx[k] * sw[r][k];
  }
#pragma unroll
  for (int wdt = 8; wdt >= 1; wdt >>= 1) {
    const float o = __shfl_down(acc, wdt, 16);
    if (l < wdt) acc = acc + o;
  }
  if (row && l == 0) {
    float sv = acc;
    for (int k = h16; k < H; ++k) sv = sv + sx[k] * sw[r][k];
    if (e != E && !finite_f(sv)) record_err(status, err_key(kPhLogit, 0, 0, e, 0));
    st_coh(z + e, sv);
  }
  wait_stores();
  __syncthreads();
  unsigned last = 0;
  if (lane == 0) last = atomicAdd(front, 1u) == (unsigned)(nR - 1);
  last = __shfl(last, 0);
  if (!last) return;
  if (lane == 0) atomicExch(front, 0u);
  route_select_token<NE, true>(z, E + 1, E, L.K, 1, 0, lane, &sw[0][0], ids, probs, shg, status,
                               [] {
                                 __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                                 __builtin_amdgcn_wave_barrier();
                               });
}

// k_gguf_experts: one workgroup of 8 waves per CU, all resident together.
// Phase 1: the K x I routed (gate, up) row pairs in blocks of 16 per
// workgroup, every weight chunk requested before the first is decoded; a
// block's h goes to the device-coherent level as one write and the block is
// counted in its slot's counter (hcnt[16 s]).  Phase 2: workgroup b owns output rows 8b .. 8b + 7 (and
// 8b + 8G ..): wave w requests the chunks of row 8b + w of the shared
// expert (whose h the front launch wrote) and of the 8 rows of routed slot
// w, waits for slot w's count, and forms the dot products; eight lanes
// then combine each row in moe_aggregate_forward's order
// (y = sum_k p_k r_k + g r_sh (+ residual)).  Q3_K experts take the
// separate-load path (q3_load / q3_decode); other types decode as they load.
__device__ __forceinline__ int64_t lane64(int64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <int T>
__global__ __launch_bounds__(512) void k_gguf_experts(
    GgufMoeDev L, const float* __restrict__ x, const int32_t* __restrict__ ids,
    const float* __restrict__ probs, const float* __restrict__ shg,
    const float* __restrict__ residual, float* __restrict__ y, float* __restrict__ h, int ldh,
    unsigned* hcnt, unsigned target, unsigned long long* status) {
  __shared__ float part[8][33];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int G = (int)gridDim.x;
  const int H = L.H, E = L.E, K = L.K, I = L.I, Ish = L.Ish;
  // lane s < K: the payload offsets of routed slot s
  const int es = min(max((int)ids[min(lane, K - 1)], 0), E - 1);
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
  // what the combine reads, requested now: the K probabilities and the
  // shared gate (every lane), the residual of this lane's row
  float pk[8], g_sh = shg[0];
#pragma unroll
  for (int k = 0; k < 8; ++k) pk[k] = probs[min(k, K - 1)];
  // phase 2's first rows: their down chunks requested before phase 1 (Q3_K)
  const uint8_t* wsh = L.raw + L.off[(size_t)E * 3 + 2];
  const int cs = min(lane * 8, Ish - 8), cr = min(lane * 8, I - 8);
  const int dfirst = (int)blockIdx.x * 8;
  Q3Raw<8> pre_s, pre_r[8];
  if constexpr (T == kGgmlQ3_K) {
    const uint8_t* wrd0 = L.raw + lane64(od, min(w, K - 1));
    pre_s = q3_load<8>(wsh, (int64_t)min(dfirst + w, H - 1) * Ish + cs);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      pre_r[i] = q3_load<8>(wrd0, (int64_t)min(dfirst + i, H - 1) * I + cr);
  }
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
#pragma unroll
      for (int q = 0; q < 2; ++q) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          if (lane * 16 + 1024 * j >= H) continue;
          f32x4 g4[4], u4[4];
          q3_decode<16>(rg[q][j], g4);
          q3_decode<16>(ru[q][j], u4);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            ag[q] = dot4(g4[u], xv[j][u], ag[q]);
            au[q] = dot4(u4[u], xv[j][u], au[q]);
          }
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
  // ---- phase 2: down projections and the combine
  bool ready = false;
  const uint8_t* wrd = L.raw + lane64(od, min(w, K - 1));
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
    // the shared expert's row d0 + w (h written by the front launch)
    {
      const float* hp = h + (size_t)K * ldh + cs;
      float a = dot4(ws[0], *reinterpret_cast<const f32x4*>(hp), 0.0f);
      a = dot4(ws[1], *reinterpret_cast<const f32x4*>(hp + 4), a);
      a = wave_sum_dpp(ls ? a : 0.0f);
      if (lane == 0 && w < nd) {
        if (!finite_f(a)) record_err(status, err_key(kPhShared, 0, 0, Ish + d0 + w, kEkDown));
        part[w][K] = a;
      }
    }
    if (w < K) {
      if (!ready) ready = wait_count(hcnt + 16 * w, target, status);
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
        if (k < K) acc = acc + pk[k] * part[i][k];
      float total = acc + g_sh * part[i][K];
      if (residual) total = total + res;
      if (!finite_f(total)) record_err(status, err_key(kPhAgg, 0, 0, d, 0));
      y[d] = total;
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
#undef DM_GGUF_DISPATCH
#undef DM_GGUF_DISPATCH_W

bool gguf_one_token_supported(const GgufMoeDev& L) {
  return L.H % 16 == 0 && L.H <= kFrontMaxH && L.I % 16 == 0 && L.I <= 512 && L.Ish % 8 == 0 &&
         L.Ish <= 512 && L.K <= 8 && L.E + 1 <= 512 && L.type != kGgmlF32 && L.type != kGgmlBF16;
}

size_t gguf_one_token_sync_bytes(const GgufMoeDev& L) {
  const int ldh = L.I > L.Ish ? L.I : L.Ish;
  return kSyncHead + (((size_t)(L.E + 1) * 4 + 255) & ~(size_t)255) + (size_t)(L.K + 1) * ldh * 4;
}

int gguf_experts_occupancy(const GgufMoeDev& L, int* per_cu) {
  hipError_t e = hipErrorInvalidValue;
  switch (L.type) {
    case kGgmlQ8_0: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, k_gguf_experts<kGgmlQ8_0>, 512, 0); break;
    case kGgmlQ4_K: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, k_gguf_experts<kGgmlQ4_K>, 512, 0); break;
    case kGgmlQ3_K: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, k_gguf_experts<kGgmlQ3_K>, 512, 0); break;
    default: break;
  }
  return e == hipSuccess ? 0 : -1;
}

hipError_t launch_gguf_one_token(const GgufMoeDev& L, const float* x, const float* residual,
                                 float* y, int32_t* ids, float* probs, float* shg, void* sync,
                                 unsigned launch, int grid, unsigned long long* status,
                                 hipStream_t st) {
  if (!gguf_one_token_supported(L) || grid <= 0 || launch == 0) return hipErrorInvalidValue;
  const int ldh = L.I > L.Ish ? L.I : L.Ish;
  uint8_t* sb = static_cast<uint8_t*>(sync);
  unsigned* front = reinterpret_cast<unsigned*>(sb);
  unsigned* hcnt = reinterpret_cast<unsigned*>(sb + 128);  // slot s at 64 s bytes
  float* z = reinterpret_cast<float*>(sb + kSyncHead);
  float* h = reinterpret_cast<float*>(sb + kSyncHead + (((size_t)(L.E + 1) * 4 + 255) & ~(size_t)255));
  const int nR = (L.E + 1 + kFrontRows - 1) / kFrontRows;
  const dim3 g1((unsigned)(nR + L.Ish)), g2((unsigned)grid);
  const unsigned target = launch * (unsigned)(L.I / 16);  // blocks per slot
  const int ne = (L.E + 63) / 64;
#define DM_FRONT(TY, N)                                                                      \
  k_gguf_front<TY, 16, N><<<g1, 64, 0, st>>>(L, x, nR, z, h, ldh, front, ids, probs, shg, status)
#define DM_FRONT_NE(TY)              \
  if (ne <= 1) DM_FRONT(TY, 1);      \
  else if (ne <= 2) DM_FRONT(TY, 2); \
  else if (ne <= 4) DM_FRONT(TY, 4); \
  else DM_FRONT(TY, 8);
  switch (L.type) {
    case kGgmlQ8_0: DM_FRONT_NE(kGgmlQ8_0)
      k_gguf_experts<kGgmlQ8_0><<<g2, 512, 0, st>>>(L, x, ids, probs, shg, residual, y, h, ldh, hcnt, target, status);
      break;
    case kGgmlQ4_K: DM_FRONT_NE(kGgmlQ4_K)
      k_gguf_experts<kGgmlQ4_K><<<g2, 512, 0, st>>>(L, x, ids, probs, shg, residual, y, h, ldh, hcnt, target, status);
      break;
    case kGgmlQ3_K: DM_FRONT_NE(kGgmlQ3_K)
      k_gguf_experts<kGgmlQ3_K><<<g2, 512, 0, st>>>(L, x, ids, probs, shg, residual, y, h, ldh, hcnt, target, status);
      break;
    default: return hipErrorInvalidValue;
  }
#undef DM_FRONT_NE
#undef DM_FRONT
  return hipGetLastError();
}

}  // namespace dm
