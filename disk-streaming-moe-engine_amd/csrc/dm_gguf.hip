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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
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
  ag = wave_sum(ag);
  au = wave_sum(au);
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
    a = wave_sum(a);
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

}  // namespace dm
