// dm_grouped.hip -- the MoE block for several tokens at once (small batches
// and prefill): tokens are grouped by expert on the GPU and every expert runs
// as a grouped GEMM on MFMA.
//
// Reference composition (src/layers/moe_block.mojo:20-138): router for all
// tokens, then the routed experts per (token, k) with
// src/layers/swiglu.mojo:52-230, then the shared expert for all tokens, then
// the combine of src/layers/moe.mojo:105-177.  Here:
//
//   k_router_dec / k_router_select (dm_kernels.hip)  logits, softmax, top-k
//   k_group_build   one workgroup: count assignments per expert, scan,
//                   scatter them into expert order, emit the work units
//                   (expert, 64-token tile); the shared expert follows as
//                   expert E over all tokens
//   k_split_rows    activations -> bf16 hi / lo rows (lo only when needed)
//   k_gu_grouped    h = SiLU(W_g x) * (W_u x): per unit and 64-feature block,
//                   A = dequantized 4-bit weights (16 features x 32 k per
//                   MFMA), B = 16 gathered tokens; one dequantized tile feeds
//                   every token sub-tile of the unit
//   k_down_grouped  r = W_d h, B = h split into bf16 hi / lo on the fly
//   k_combine       y = sum_k p_k r_k + g r_sh (+ residual), reference order
//
// Each token's outputs depend only on its own column of the MFMA tiles, so
// the placement of tokens inside an expert's tiles (atomic scatter) does not
// change any result bit.
#include <hip/hip_runtime.h>

#include "dm_device.h"
#include "dm_grouped.h"

namespace dm {

constexpr int kMT = 64;       // tokens per work unit (4 MFMA column tiles of 16)
constexpr int kGThreads = 256;

// ---------------------------------------------------------------------------
// One workgroup of 1024 threads.  ids [T*K] in the reference order (slot k of
// token t at t*K + k).  Outputs: off [E+1] expert offsets into perm, perm
// [T*K] assignment indices grouped by expert, units [nmax] (expert, tile),
// meta[0] = number of units.
__global__ __launch_bounds__(1024) void k_group_build(const int32_t* __restrict__ ids, int T, int K,
                                                      int E, int32_t* __restrict__ off,
                                                      int32_t* __restrict__ perm,
                                                      int2* __restrict__ units,
                                                      int32_t* __restrict__ meta) {
  extern __shared__ int lds[];  // cnt[E] | cur[E] | part[1024] | upart[1024]
  int* cnt = lds;
  int* cur = lds + E;
  int* part = lds + 2 * E;
  int* upart = part + 1024;
  const int tid = threadIdx.x, TK = T * K;
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int a = tid; a < TK; a += 1024) {
    const int e = min(max((int)ids[a], 0), E - 1);
    atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // scan of counts and of unit counts: thread tid owns experts [e0, e1)
  const int per = (E + 1023) / 1024, e0 = min(tid * per, E), e1 = min(e0 + per, E);
  int s = 0, us = 0;
  for (int e = e0; e < e1; ++e) {
    s += cnt[e];
    us += (cnt[e] + kMT - 1) / kMT;
  }
  part[tid] = s;
  upart[tid] = us;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {  // inclusive Hillis-Steele scan
    const int a = tid >= d ? part[tid - d] : 0, b = tid >= d ? upart[tid - d] : 0;
    __syncthreads();
    part[tid] += a;
    upart[tid] += b;
    __syncthreads();
  }
  int base = part[tid] - s, ubase = upart[tid] - us;
  for (int e = e0; e < e1; ++e) {
    off[e] = base;
    cur[e] = base;
    const int nt = (cnt[e] + kMT - 1) / kMT;
    for (int tc = 0; tc < nt; ++tc) units[ubase + tc] = make_int2(e, tc);
    base += cnt[e];
    ubase += nt;
  }
  const int nrouted = upart[1023];
  if (tid == 0) off[E] = TK;
  __syncthreads();
  for (int a = tid; a < TK; a += 1024) {
    const int e = min(max((int)ids[a], 0), E - 1);
    perm[atomicAdd(&cur[e], 1)] = a;
  }
  const int nsh = (T + kMT - 1) / kMT;
  for (int tc = tid; tc < nsh; tc += 1024) units[nrouted + tc] = make_int2(E, tc);
  if (tid == 0) meta[0] = nrouted + nsh;
}

hipError_t launch_group_build(const int32_t* ids, int T, int K, int E, int32_t* off,
                              int32_t* perm, int2* units, int32_t* meta, hipStream_t st) {
  const size_t lds = (size_t)(2 * E + 2048) * sizeof(int);
  hipLaunchKernelGGL(k_group_build, dim3(1), dim3(1024), lds, st, ids, T, K, E, off, perm, units,
                     meta);
  return hipGetLastError();
}

int group_units_max(int T, int K, int E) {
  return E + (T * K + kMT - 1) / kMT + (T + kMT - 1) / kMT;
}

// ---------------------------------------------------------------------------
// rows [T][n] fp32 -> bf16 hi / lo; *need_lo |= 1 when some lo part is nonzero.
__global__ __launch_bounds__(256) void k_split_rows(const float* __restrict__ x, int64_t count8,
                                                    uint4* __restrict__ hi, uint4* __restrict__ lo,
                                                    int* __restrict__ need_lo) {
  bool nz = false;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < count8; i += (int64_t)gridDim.x * 256) {
    const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
    const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
    const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint4 h, l;
    split8(f, h, l);
    hi[i] = h;
    lo[i] = l;
    nz |= (l.x | l.y | l.z | l.w) != 0u;
  }
  if (__builtin_amdgcn_ballot_w64(nz) != 0 && (threadIdx.x & 63) == 0) atomicOr(need_lo, 1);
}

hipError_t launch_split_rows(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, int* need_lo,
                             hipStream_t st) {
  const int64_t c8 = n / 8;
  const int blocks = (int)((c8 + 255) / 256 < 2048 ? (c8 + 255) / 256 : 2048);
  hipLaunchKernelGGL(k_split_rows, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, st, x, c8,
                     reinterpret_cast<uint4*>(hi), reinterpret_cast<uint4*>(lo), need_lo);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Token rows of a unit: column c of tile (e, tc) is position p = off[e] +
// 64 tc + c of the expert order, i.e. assignment a = perm[p] of token a / K;
// for the shared expert (e == E) column c is token 64 tc + c itself.
struct UnitTokens {
  int e, p0, n;   // expert, first position, tokens in this unit
  bool shared;
};
__device__ __forceinline__ UnitTokens unit_tokens(int2 u, const int32_t* off, int E, int T) {
  UnitTokens r;
  r.e = u.x;
  r.shared = u.x >= E;
  if (r.shared) {
    r.p0 = kMT * u.y;
    r.n = min(kMT, T - r.p0);
  } else {
    r.p0 = off[u.x] + kMT * u.y;
    r.n = min(kMT, off[u.x + 1] - r.p0);
  }
  return r;
}

// ---------------------------------------------------------------------------
// Gate/up: blockIdx.x = unit, blockIdx.y = block of 64 features (4 row tiles,
// wave w owns tile 4*blockIdx.y + w) of the gate and the up matrix.  Output
// h [p][I] fp32 at the unit's positions (routed) or hs [t][Ish] (shared).
__global__ __launch_bounds__(kGThreads) void k_gu_grouped(
    LayerDev L, const uint16_t* __restrict__ xhi, const uint16_t* __restrict__ xlo,
    const int* __restrict__ need_lo, const int32_t* __restrict__ off,
    const int32_t* __restrict__ perm, const int2* __restrict__ units,
    const int32_t* __restrict__ meta, int T, float* __restrict__ hr, float* __restrict__ hs,
    unsigned long long* status) {
  if ((int)blockIdx.x >= meta[0]) return;
  const UnitTokens ut = unit_tokens(units[blockIdx.x], off, L.E, T);
  const int H = L.H, K = L.K;
  const int I = ut.shared ? L.Ish : L.I;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15;
  const int rb = blockIdx.y * 4 + w;
  if (rb * kTileRows >= I) return;  // (uniform per wave; no barriers below)
  const size_t mat = (size_t)I * H;
  ExpertView gv, uv;
  if (ut.shared) {
    gv = {L.sgu_nib, L.sgu_sc, I, H};
  } else {
    gv = {L.gu_nib + (size_t)ut.e * mat, L.gu_sc + (size_t)ut.e * 2 * (mat / kGroup), I, H};
  }
  uv = {gv.nib + mat / 2, gv.sc + mat / kGroup, I, H};
  const bool lo = need_lo[0] != 0;
  // token row of each column tile for this lane (column j)
  int tok[4];
  bool valid[4];
#pragma unroll
  for (int ts = 0; ts < 4; ++ts) {
    const int c = 16 * ts + j;
    valid[ts] = c < ut.n;
    const int cc = valid[ts] ? c : 0;
    tok[ts] = ut.shared ? ut.p0 + cc : perm[ut.p0 + cc] / K;
  }
  f32x4 ag[4], au[4];
#pragma unroll
  for (int ts = 0; ts < 4; ++ts) ag[ts] = au[ts] = f32x4{0, 0, 0, 0};
  const int nGQ = H / kQuadCols;
  const int nts = (ut.n + 15) / 16;
  for (int gq = 0; gq < nGQ; ++gq) {
    uint4 wg, wu;
    uint2 sg, su;
    load_chunk_nt(gv, rb, gq, lane, wg, sg);
    load_chunk_nt(uv, rb, gq, lane, wu, su);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bf16x8 a_g = dequant8(word_of(wg, c), scale_of(sg, c));
      const bf16x8 a_u = dequant8(word_of(wu, c), scale_of(su, c));
      const int k0 = gq * kQuadCols + c * kGroup + 8 * q;
#pragma unroll
      for (int ts = 0; ts < 4; ++ts) {
        if (ts < nts) {
          uint4 bv = *reinterpret_cast<const uint4*>(xhi + (size_t)tok[ts] * H + k0);
          if (!valid[ts]) bv = make_uint4(0, 0, 0, 0);
          const bf16x8 b = __builtin_bit_cast(bf16x8, bv);
          ag[ts] = mfma16(a_g, b, ag[ts]);
          au[ts] = mfma16(a_u, b, au[ts]);
          if (lo) {
            uint4 lv = *reinterpret_cast<const uint4*>(xlo + (size_t)tok[ts] * H + k0);
            if (!valid[ts]) lv = make_uint4(0, 0, 0, 0);
            const bf16x8 bl = __builtin_bit_cast(bf16x8, lv);
            ag[ts] = mfma16(a_g, bl, ag[ts]);
            au[ts] = mfma16(a_u, bl, au[ts]);
          }
        }
      }
    }
  }
  // D: lane (q, j) holds features 16 rb + 4q + i of column j
#pragma unroll
  for (int ts = 0; ts < 4; ++ts) {
    if (ts < nts && valid[ts]) {
      const int c = 16 * ts + j;
      const int p = ut.p0 + c;
      const int a = ut.shared ? p : perm[p];
      const int t = ut.shared ? p : a / K, k = ut.shared ? 0 : a % K;
      float hv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rb * kTileRows + 4 * q + i;
        const float g = ag[ts][i], u = au[ts][i];
        hv[i] = dm_silu(g) * u;
        if (!finite_f(g) || !finite_f(u) || !finite_f(hv[i])) {
          const uint32_t ph = ut.shared ? kPhShared : kPhExpert;
          const uint32_t kind = !finite_f(g) ? kEkGate : !finite_f(u) ? kEkUp : kEkH;
          record_err(status, err_key(ph, t, k, row, kind));
        }
      }
      float* dst = ut.shared ? hs + (size_t)t * I : hr + (size_t)p * I;
      *reinterpret_cast<float4*>(dst + rb * kTileRows + 4 * q) = make_float4(hv[0], hv[1], hv[2], hv[3]);
    }
  }
}

// ---------------------------------------------------------------------------
// Down: blockIdx.x = unit, blockIdx.y = block of 64 output rows.  B = h of the
// unit's tokens split into bf16 hi / lo on the fly.  Output r [a][H]
// (routed, a = assignment) or rs [t][H] (shared).
__global__ __launch_bounds__(kGThreads) void k_down_grouped(
    LayerDev L, const int32_t* __restrict__ off, const int32_t* __restrict__ perm,
    const int2* __restrict__ units, const int32_t* __restrict__ meta, int T,
    const float* __restrict__ hr, const float* __restrict__ hs, float* __restrict__ r,
    float* __restrict__ rs, unsigned long long* status) {
  if ((int)blockIdx.x >= meta[0]) return;
  const UnitTokens ut = unit_tokens(units[blockIdx.x], off, L.E, T);
  const int H = L.H, K = L.K;
  const int I = ut.shared ? L.Ish : L.I;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15;
  const int rb = blockIdx.y * 4 + w;
  if (rb * kTileRows >= H) return;
  const size_t mat = (size_t)H * I;
  const ExpertView dv = ut.shared ? ExpertView{L.sd_nib, L.sd_sc, H, I}
                                  : ExpertView{L.d_nib + (size_t)ut.e * (mat / 2),
                                               L.d_sc + (size_t)ut.e * (mat / kGroup), H, I};
  const float* hrow[4];
  bool valid[4];
#pragma unroll
  for (int ts = 0; ts < 4; ++ts) {
    const int c = 16 * ts + j;
    valid[ts] = c < ut.n;
    const int p = ut.p0 + (valid[ts] ? c : 0);
    hrow[ts] = ut.shared ? hs + (size_t)p * I : hr + (size_t)p * I;
  }
  f32x4 acc[4];
#pragma unroll
  for (int ts = 0; ts < 4; ++ts) acc[ts] = f32x4{0, 0, 0, 0};
  const int nGQ = I / kQuadCols;
  const int nts = (ut.n + 15) / 16;
  for (int gq = 0; gq < nGQ; ++gq) {
    uint4 wd;
    uint2 sd;
    load_chunk_nt(dv, rb, gq, lane, wd, sd);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bf16x8 a = dequant8(word_of(wd, c), scale_of(sd, c));
      const int k0 = gq * kQuadCols + c * kGroup + 8 * q;
#pragma unroll
      for (int ts = 0; ts < 4; ++ts) {
        if (ts < nts) {
          const float4 u0 = *reinterpret_cast<const float4*>(hrow[ts] + k0);
          const float4 u1 = *reinterpret_cast<const float4*>(hrow[ts] + k0 + 4);
          float f[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
          if (!valid[ts])
#pragma unroll
            for (int z = 0; z < 8; ++z) f[z] = 0.0f;
          uint4 bh, bl;
          split8(f, bh, bl);
          acc[ts] = mfma16(a, __builtin_bit_cast(bf16x8, bh), acc[ts]);
          acc[ts] = mfma16(a, __builtin_bit_cast(bf16x8, bl), acc[ts]);
        }
      }
    }
  }
#pragma unroll
  for (int ts = 0; ts < 4; ++ts) {
    if (ts < nts && valid[ts]) {
      const int c = 16 * ts + j;
      const int p = ut.p0 + c;
      const int a = ut.shared ? p : perm[p];
      const int t = ut.shared ? p : a / K, k = ut.shared ? 0 : a % K;
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = acc[ts][i];
        if (!finite_f(v[i])) {
          const uint32_t ph = ut.shared ? kPhShared : kPhExpert;
          record_err(status, err_key(ph, t, k, I + rb * kTileRows + 4 * q + i, kEkDown));
        }
      }
      float* dst = ut.shared ? rs + (size_t)t * H : r + (size_t)a * H;
      *reinterpret_cast<float4*>(dst + rb * kTileRows + 4 * q) = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
}

hipError_t launch_experts_grouped(const LayerDev& L, const uint16_t* xhi, const uint16_t* xlo,
                                  const int* need_lo, const int32_t* off, const int32_t* perm,
                                  const int2* units, const int32_t* meta, int T, float* hr,
                                  float* hs, float* r, float* rs, unsigned long long* status,
                                  hipStream_t st) {
  const int nu = group_units_max(T, L.K, L.E);
  const int imax = L.I > L.Ish ? L.I : L.Ish;
  hipLaunchKernelGGL(k_gu_grouped, dim3(nu, (imax + 63) / 64), dim3(kGThreads), 0, st, L, xhi,
                     xlo, need_lo, off, perm, units, meta, T, hr, hs, status);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_down_grouped, dim3(nu, (L.H + 63) / 64), dim3(kGThreads), 0, st, L, off,
                     perm, units, meta, T, hr, hs, r, rs, status);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// y[t][d] = (sum_k p[t][k] r[t*K+k][d]) + g[t] rs[t][d] (+ residual[t][d]):
// routed experts in the reference order, then the shared expert, then the
// residual (src/layers/moe.mojo:157-166, src/layers/forward_layer.mojo:226-238).
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ r,
                                                  const float* __restrict__ rs,
                                                  const float* __restrict__ probs,
                                                  const float* __restrict__ shg,
                                                  const float* __restrict__ residual, int H, int K,
                                                  float* __restrict__ y,
                                                  unsigned long long* status) {
  const int t = blockIdx.y, d = blockIdx.x * 256 + threadIdx.x;
  if (d >= H) return;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) acc = acc + probs[(size_t)t * K + k] * r[((size_t)t * K + k) * H + d];
  float total = acc + shg[t] * rs[(size_t)t * H + d];
  if (residual) total = total + residual[(size_t)t * H + d];
  if (!finite_f(total)) record_err(status, err_key(kPhAgg, t, 0, d, 0));
  y[(size_t)t * H + d] = total;
}

hipError_t launch_combine(const float* r, const float* rs, const float* probs, const float* shg,
                          const float* residual, int T, int H, int K, float* y,
                          unsigned long long* status, hipStream_t st) {
  hipLaunchKernelGGL(k_combine, dim3((H + 255) / 256, T), dim3(256), 0, st, r, rs, probs, shg,
                     residual, H, K, y, status);
  return hipGetLastError();
}

}  // namespace dm
