// dm_grouped.hip -- the MoE block for several tokens at once (small batches
// and prefill): tokens are grouped by expert on the GPU and every expert runs
// as a grouped GEMM on MFMA.
//
// Reference composition (src/layers/moe_block.mojo:20-138): router for all
// tokens, then the routed experts per (token, k) with
// src/layers/swiglu.mojo:52-230, then the shared expert for all tokens, then
// the combine of src/layers/moe.mojo:105-177.  Here:
//
//   k_router_mfma / k_router_dec, k_router_select (dm_kernels.hip)  logits
//                   (matrix cores for bf16 activations), softmax, top-k
//   k_group_build   one workgroup: count assignments per expert, scan,
//                   scatter them into expert order, emit the work units
//                   (expert, tile of up to 128 tokens); the shared expert is
//                   expert E over all tokens.  Units of more than 16 tokens
//                   ("big") come first, then the small ones.
//   k_split_rows    activations -> bf16 hi / lo rows
//   k_big<true>     h = SiLU(W_g x) * (W_u x) for big units: token rows,
//                   4-bit weights and scales all staged in LDS by
//                   direct-to-LDS loads, three stages in flight, weights
//                   dequantised from LDS (16 features x 32 k per MFMA)
//   k_gu_small      the same for units of <= 16 tokens: B fragments straight
//                   from memory, no LDS and no barriers, deeper prefetch
//   k_big<false> / k_down_small   r = W_d h, B = h as bf16 hi + lo parts
//   k_combine       y = sum_k p_k r_k + g r_sh (+ residual), reference order
//
// Each token's outputs depend only on its own column of the MFMA tiles, so
// the placement of tokens inside an expert's tiles (atomic scatter) does not
// change any result bit.
#include <hip/hip_runtime.h>

#include <atomic>

#include "dm_device.h"
#include "dm_grouped.h"

namespace dm {

constexpr int kMT = 128;       // tokens per big work unit (8 MFMA column tiles of 16)
constexpr int kNCT = kMT / 16;
constexpr int kSmallMax = 16;  // units of at most this many tokens are small
constexpr int kGThreads = 256;

// ---------------------------------------------------------------------------
// One workgroup of 1024 threads.  ids [T*K] in the reference order (slot k of
// token t at t*K + k).  Outputs: off [E+1] expert offsets into perm, perm
// [T*K] assignment indices grouped by expert, units [nmax] = (expert, first
// position within the expert), meta[0] = number of units, meta[1] = number of
// big units.  An expert's c tokens form c / 128 full big units; a remainder
// r > 32 is one more big unit, a remainder r <= 32 becomes ceil(r / 16) small
// units.  Order: full routed units, full shared units, partial big routed
// units, a partial big shared unit, then the small routed and shared units,
// so that the costly workgroups start first.
__device__ __forceinline__ void unit_split(int c, int& nf, int& pb, int& ps) {
  const int r = c % kMT;
  nf = c / kMT;
  pb = r > 2 * kSmallMax;
  ps = (r > 0 && r <= 2 * kSmallMax) ? (r + kSmallMax - 1) / kSmallMax : 0;
}

// The grouping on one workgroup of 1024 threads, lds: (2 E + 64) ints.
// COH: ids are read with agent-scope loads (written in the same launch).
template <bool COH>
__device__ __forceinline__ void group_build_wg(const int32_t* __restrict__ ids, int T, int K, int E,
                                               int32_t* __restrict__ off,
                                               int32_t* __restrict__ perm,
                                               int2* __restrict__ units,
                                               int32_t* __restrict__ meta, int* lds) {
  // cnt[E] | cur[E] | wave totals of the 4 scans (counts, full units,
  // partial big, small units), 16 waves each
  int* cnt = lds;
  int* cur = lds + E;
  int* sc = lds + 2 * E;
  const int tid = threadIdx.x, TK = T * K;
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  // the first kCache expert ids of this thread stay in registers for the
  // scatter below (a load issued after the stores of the units would wait
  // for them)
  constexpr int kCache = 16;
  int ec[kCache];
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    const int a = tid + 1024 * i;
    ec[i] = a < TK ? min(max((int)(COH ? ld_coh_i32(ids + a) : ids[a]), 0), E - 1) : 0;
  }
#pragma unroll
  for (int i = 0; i < kCache; ++i)
    if (tid + 1024 * i < TK) atomicAdd(&cnt[ec[i]], 1);
  for (int a = tid + 1024 * kCache; a < TK; a += 1024) {
    const int e = min(max((int)(COH ? ld_coh_i32(ids + a) : ids[a]), 0), E - 1);
    atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // thread tid owns experts [e0, e1)
  const int per = (E + 1023) / 1024, e0 = min(tid * per, E), e1 = min(e0 + per, E);
  int v[4] = {0, 0, 0, 0};
  for (int e = e0; e < e1; ++e) {
    int nf, pb, ps;
    unit_split(cnt[e], nf, pb, ps);
    v[0] += cnt[e];
    v[1] += nf;
    v[2] += pb;
    v[3] += ps;
  }
  // exclusive prefix sums of the four counts over the threads: inclusive
  // scans inside each wave (shuffles), then the 16 wave totals from LDS
  const int lane = tid & 63, wv = tid >> 6;
  int incl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int a = v[i];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(a, d, 64);
      a += lane >= d ? o : 0;
    }
    incl[i] = a;
    if (lane == 63) sc[i * 16 + wv] = a;
  }
  __syncthreads();
  int pre[4], tot[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int p = 0, t = 0;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int wt = sc[i * 16 + u];
      p += u < wv ? wt : 0;
      t += wt;
    }
    pre[i] = p + incl[i] - v[i];
    tot[i] = t;
  }
  const int nf = tot[1], npb = tot[2], nps = tot[3];
  int snf, spb, sps;
  unit_split(T, snf, spb, sps);
  const int pb0 = nf + snf, s0 = pb0 + npb + spb;
  int base = pre[0], fb = pre[1], pb = pb0 + pre[2], ps = s0 + pre[3];
  for (int e = e0; e < e1; ++e) {
    int nfe, pbe, pse;
    unit_split(cnt[e], nfe, pbe, pse);
    off[e] = base;
    cur[e] = base;
    for (int i = 0; i < nfe; ++i) units[fb + i] = make_int2(e, kMT * i);
    if (pbe) units[pb++] = make_int2(e, kMT * nfe);
    for (int i = 0; i < pse; ++i) units[ps++] = make_int2(e, kMT * nfe + kSmallMax * i);
    base += cnt[e];
    fb += nfe;
  }
  if (tid == 0) off[E] = TK;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    const int a = tid + 1024 * i;
    if (a < TK) perm[atomicAdd(&cur[ec[i]], 1)] = a;
  }
  for (int a = tid + 1024 * kCache; a < TK; a += 1024) {
    const int e = min(max((int)(COH ? ld_coh_i32(ids + a) : ids[a]), 0), E - 1);
    perm[atomicAdd(&cur[e], 1)] = a;
  }
  for (int i = tid; i < snf; i += 1024) units[nf + i] = make_int2(E, kMT * i);
  if (tid == 0) {
    if (spb) units[pb0 + npb] = make_int2(E, kMT * snf);
    for (int i = 0; i < sps; ++i) units[s0 + nps + i] = make_int2(E, kMT * snf + kSmallMax * i);
    meta[0] = s0 + nps + sps;
    meta[1] = s0;
  }
}

__global__ __launch_bounds__(1024) void k_group_build(const int32_t* __restrict__ ids, int T, int K,
                                                      int E, int32_t* __restrict__ off,
                                                      int32_t* __restrict__ perm,
                                                      int2* __restrict__ units,
                                                      int32_t* __restrict__ meta) {
  extern __shared__ int lds[];
  group_build_wg<false>(ids, T, K, E, off, perm, units, meta, lds);
}

hipError_t launch_group_build(const int32_t* ids, int T, int K, int E, int32_t* off,
                              int32_t* perm, int2* units, int32_t* meta, hipStream_t st) {
  const size_t lds = (size_t)(2 * E + 64) * sizeof(int);
  hipLaunchKernelGGL(k_group_build, dim3(1), dim3(1024), lds, st, ids, T, K, E, off, perm, units,
                     meta);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The front end of a small batch in one launch (T tokens, 2 <= T < 64):
// workgroup (b, t) stages token t's x in LDS, computes router rows
// 64 b .. 64 b + 63 (16 lanes each, the chains of router_chain and the
// halving tree of k_router_dec: the same logits bit for bit), and workgroup
// (0, t) also writes t's bf16 hi / lo rows and the need-lo flag.  Each
// workgroup then counts itself in token t's counter flags[2 + t]; the last
// of them (the logits are written and read at the device-coherent level, so
// that those of workgroups on other XCDs are visible) runs t's softmax /
// top-k on one wave (route_select_token) and counts the token in flags[1];
// the last token's workgroup groups the assignments (group_build_wg).  Each
// counter is reset by the workgroup that saw it complete.  No workgroup
// waits for another.
template <int NE>
__global__ __launch_bounds__(1024) void k_front(const float* __restrict__ x,
                                                const uint16_t* __restrict__ router_, int H_,
                                                int E_, LayerDev Lk, int T,
                                                float* __restrict__ z, uint4* __restrict__ xhi,
                                                uint4* __restrict__ xlo, int* flags,
                                                int32_t* __restrict__ ids,
                                                float* __restrict__ probs,
                                                float* __restrict__ shg, int32_t* __restrict__ off,
                                                int32_t* __restrict__ perm,
                                                int2* __restrict__ units,
                                                int32_t* __restrict__ meta,
                                                unsigned long long* status) {
  extern __shared__ __attribute__((aligned(16))) float fl[];
  __shared__ int last, last_tok;
  LayerDev L = Lk;  // the entry fields from the preloaded leading arguments
  L.H = H_;
  L.E = E_;
  L.router = router_;
  const int tid = threadIdx.x, H = L.H, E = L.E, t = blockIdx.y;
  const float* xr = x + (size_t)t * H;
  bool bad = false;
  for (int i = tid; i < H; i += 1024) {
    const float v = xr[i];
    bad |= !finite_f(v);
    fl[i] = v;
  }
  if (bad && blockIdx.x == 0) record_err(status, err_key(kPhX, 0, 0, 0, 0));
  if (blockIdx.x == 0) {
    bool nz = false;
    for (int i = tid; i < H / 8; i += 1024) {
      uint4 h, l;
      split8(xr + 8 * i, h, l);
      xhi[(size_t)t * (H / 8) + i] = h;
      xlo[(size_t)t * (H / 8) + i] = l;
      nz |= (l.x | l.y | l.z | l.w) != 0u;
    }
    if (__builtin_amdgcn_ballot_w64(nz) != 0 && (tid & 63) == 0) atomicOr(&flags[0], 1);
  }
  __syncthreads();
  const int l = tid & 15, e = blockIdx.x * 64 + (tid >> 4);
  float acc = e <= E ? router_chain(L.router, H, e, l, fl) : 0.0f;
#pragma unroll
  for (int wdt = 8; wdt >= 1; wdt >>= 1) acc = acc + __shfl_down(acc, wdt, 16);
  // logits to the device-coherent level (agent-scope stores, complete before
  // the count), read back by the last workgroup with agent-scope loads: no
  // write-back or invalidation of the whole L2
  if (l == 0 && e <= E) st_coh(z + (size_t)t * (E + 1) + e, acc);
  wait_stores();
  __syncthreads();
  // the last of token t's workgroups selects its experts (wave 0) ...
  if (tid == 0) last = atomicAdd(&flags[2 + t], 1) == (int)gridDim.x - 1;
  __syncthreads();
  if (!last) return;
  const int lane = tid & 63, w = tid >> 6, K = L.K;
  auto wsync = [] {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  };
  // Two waves at once: wave 0 picks the top K on the logits (topk_on_logits:
  // the same set as the reference's rounds on the probabilities whenever its
  // margin check passes), wave 1 forms the softmax terms (max, the
  // exponentials, their sum in expert order) and the shared gate, as
  // router_softmax does (src/layers/router.mojo:140-183).  Then wave 0
  // forms the K probabilities e_k * (1/S) and orders them (p desc, id asc),
  // as select_topk (src/layers/topk.mojo:79-128).  On a near tie at the
  // boundary wave 0 runs the exact rounds (route_select_token) instead.
  constexpr int R = NE <= 4 ? 1 : 2;
  __shared__ float sm_terms[2];  // max, 1/S
  __shared__ int sm_unsafe;
  float* sev = fl;               // [E] exponentials (the staged x is no longer read)
  const float* zr = z + (size_t)t * (E + 1);
  int myid = 0;
  float zk = 0.0f;
  if (w == 0) {
    if (tid == 0) atomicExch(&flags[2 + t], 0);
    float zv[4 * R];
#pragma unroll
    for (int i = 0; i < 4 * R; ++i) {
      const int e = lane + 64 * i;
      zv[i] = e < E ? ld_coh(zr + e) : -__builtin_inff();
    }
    uint32_t fk[4 * R];
    const bool unsafe = topk_on_logits<R>(zv, E, K, lane, fk, myid);
    myid = min(max(myid, 0), E - 1);
    // the logit of expert myid sits in lane myid & 63, entry myid >> 6
#pragma unroll
    for (int i = 0; i < 4 * R; ++i) {
      const float zo = u2f((uint32_t)__builtin_amdgcn_ds_bpermute(4 * (myid & 63), (int)f2u(zv[i])));
      zk = (myid >> 6) == i ? zo : zk;
    }
    if (lane == 0) sm_unsafe = unsafe || K > 8 ? 1 : 0;  // (the ranks below take K <= 8)
  } else if (w == 1) {
    const float lg = lane == 0 ? ld_coh(zr + E) : 0.0f;
    float zv[NE];
    float m = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int e = lane + 64 * i;
      zv[i] = e < E ? ld_coh(zr + e) : -__builtin_inff();
      if (e < E && !finite_f(zv[i])) record_err(status, err_key(kPhLogit, t, 0, e, 0));
      m = zv[i] > m ? zv[i] : m;
    }
    m = __ockl_wfred_max_f32(m);
    if (lane == 0 && !finite_f(m)) record_err(status, err_key(kPhSoftmax, t, 0, 0, 0));
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int e = lane + 64 * i;
      if (e < E) {
        const float ev = dm_expf(zv[i] - m);
        if (!finite_f(ev)) record_err(status, err_key(kPhSoftmax, t, 0, 1 + e, 0));
        sev[e] = ev;
      }
    }
    wsync();
    if (lane == 0) {
      const float sum = seq_sum(sev, E);
      if (!(sum > 0.0f) || !finite_f(sum)) record_err(status, err_key(kPhSoftmax, t, 0, 1 + E, 0));
      sm_terms[0] = m;
      sm_terms[1] = 1.0f / sum;
      if (!finite_f(lg)) record_err(status, err_key(kPhGate, t, 0, 0, kGkLogit));
      const float g = dm_sigmoid(lg);
      if (!finite_f(g) || g < 0.0f || g > 1.0f) record_err(status, err_key(kPhGate, t, 0, 0, kGkRange));
      shg[t] = g;
    }
  }
  __syncthreads();
  if (w == 0) {
    if (sm_unsafe) {
      route_select_token<NE, true>(z, E + 1, E, K, 1, t, lane, fl, ids, probs, shg, status, wsync);
    } else {
      const float m = sm_terms[0], inv = sm_terms[1];
      const float pk = lane < K ? dm_expf(zk - m) * inv : 0.0f;
      // rank of slot k: (p desc, id asc); the ids are distinct
      const uint32_t kk = f2key(pk);
      int rank = 0;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)kk, jj);
        const int ij = __builtin_amdgcn_readlane(myid, jj);
        if (jj < K && lane < K) rank += (kj > kk || (kj == kk && ij < myid)) ? 1 : 0;
      }
      if (lane < K) {
        st_coh_i32(ids + (size_t)t * K + rank, myid);
        probs[(size_t)t * K + rank] = pk;
      }
      // the checks of select_topk in rank order
      float* sp = sev + ((E + 3) & ~3);  // [8] probabilities by rank
      if (lane < K) sp[rank] = pk;
      wsync();
      if (lane == 0) {
        float sum_topk = 0.0f;
        for (int r = 0; r < K; ++r) sum_topk = sum_topk + sp[r];
        if (sum_topk > 1.00001f) record_err(status, err_key(kPhTopk, t, 0, 0, kTkSum));
        if (K < E && __builtin_fabsf(sum_topk - 1.0f) < 1e-6f) {
          float sum_all = 0.0f;
          for (int e = 0; e < E; ++e) sum_all = sum_all + sev[e] * inv;
          if (sum_all - sum_topk > 1e-5f) record_err(status, err_key(kPhTopk, t, 0, 0, kTkLeak));
        }
      }
    }
    wait_stores();
    // ... and the last token to be selected groups the assignments
    if (tid == 0) last_tok = atomicAdd(&flags[1], 1) == T - 1;
  }
  __syncthreads();
  if (!last_tok) return;
  if (tid == 0) atomicExch(&flags[1], 0);
  group_build_wg<true>(ids, T, L.K, E, off, perm, units, meta, reinterpret_cast<int*>(fl));
}

bool front_supported(const LayerDev& L, int T) {
  return T >= 2 && T <= kFrontMaxT && L.E <= kFrontMaxE && L.H % 128 == 0;
}

hipError_t launch_front(const LayerDev& L, const float* x, int T, float* z, uint16_t* xhi,
                        uint16_t* xlo, int* flags, int32_t* ids, float* probs, float* shg,
                        int32_t* off, int32_t* perm, int2* units, int32_t* meta,
                        unsigned long long* status, hipStream_t st) {
  if (!front_supported(L, T)) return hipErrorInvalidValue;
  const size_t sel = (size_t)(((L.E + 3) & ~3) + 8) * sizeof(float);
  const size_t bld = (size_t)(2 * L.E + 64) * sizeof(int);
  const size_t xs = (size_t)L.H * sizeof(float);
  const size_t lds = sel > bld ? (sel > xs ? sel : xs) : (bld > xs ? bld : xs);
  const dim3 grid((L.E + 1 + 63) / 64, T);
  uint4* hi = reinterpret_cast<uint4*>(xhi);
  uint4* lo = reinterpret_cast<uint4*>(xlo);
  const int ne = (L.E + 63) / 64;
#define DM_FRONT(N)                                                                             \
  hipLaunchKernelGGL(k_front<N>, grid, dim3(1024), lds, st, x, L.router, L.H, L.E, L, T, z, hi, \
                     lo, flags, ids, probs, shg, off, perm, units, meta, status)
  if (ne <= 1) DM_FRONT(1);
  else if (ne <= 2) DM_FRONT(2);
  else if (ne <= 4) DM_FRONT(4);
  else DM_FRONT(8);
#undef DM_FRONT
  return hipGetLastError();
}

int group_units_max(int T, int K, int E) {
  // per expert at most c / 128 + 2 units (two small units of a remainder <= 32)
  return 2 * E + (T * K + kMT - 1) / kMT + (T + kMT - 1) / kMT + 2;
}

// Bounds of the two unit kinds, for the launch grids (the exact counts are
// known on the device only).  Small units: each holds at least one
// assignment and an expert has at most two (its remainder <= 32), the
// shared expert at most two as well.  Big units: the full ones of all
// assignments (routed and shared), plus at most one partial per expert with
// more than 32 tokens in its remainder, and the shared expert's.
static int small_units_max(int T, int K, int E) {
  const long tk = (long)T * K;
  return (int)(tk < 2L * E ? tk : 2L * E) + 2;
}
static int big_units_max(int T, int K, int E) {
  const long tk = (long)T * K;
  const long partial = tk / (2 * kSmallMax + 1);
  return (int)(tk / kMT + T / kMT + (partial < E ? partial : E) + 1);
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
  // a plain store of 1, not an atomic: thousands of waves may set the flag,
  // and same-address atomics would be serialised one after another
  if (__builtin_amdgcn_ballot_w64(nz) != 0 && (threadIdx.x & 63) == 0) *need_lo = 1;
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
// Token rows of a unit (e, start): row r is position p = off[e] + start + r
// of the expert order, i.e. assignment a = perm[p] of token a / K; for the
// shared expert (e == E) row r is token start + r itself.  Big units hold up
// to kMT rows, small units up to kSmallMax.
struct UnitTokens {
  int e, p0, n;   // expert, first position, tokens in this unit
  bool shared;
};
__device__ __forceinline__ UnitTokens unit_tokens(int2 u, const int32_t* off, int E, int T,
                                                  int size) {
  UnitTokens r;
  r.e = u.x;
  r.shared = u.x >= E;
  if (r.shared) {
    r.p0 = u.y;
    r.n = min(size, T - r.p0);
  } else {
    r.p0 = off[u.x] + u.y;
    r.n = min(size, off[u.x + 1] - r.p0);
  }
  return r;
}

struct GroupArgs {
  LayerDev L;
  const uint16_t* xhi;   // [T][H] bf16 parts of the activations
  const uint16_t* xlo;
  const int* need_lo;    // nonzero: some activation is not a bf16 value
  const int32_t* off;
  const int32_t* perm;
  const int2* units;
  const int32_t* meta;
  int T;
  uint16_t* hrh;         // h of routed positions [T*K][I], bf16 hi / lo
  uint16_t* hrl;
  uint16_t* hsh;         // h of the shared expert [T][Ish]
  uint16_t* hsl;
  float* r;              // routed down outputs [T*K][H] by assignment
  float* rs;             // shared down outputs [T][H]
  unsigned long long* status;
};

__device__ __forceinline__ int gwave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// The A chunks (16 rows x 128 columns, 4-bit + scales) of NT tiles for one
// k-step.  Gate/up (GU): tiles 0..NT/2-1 are gate tiles rb0 + t, tiles
// NT/2.. the up tiles at the same rows; down: tiles rb0 + t of one matrix.
template <int NT>
struct AChunks {
  uint4 w[NT];
  uint2 s[NT];
};

template <int NT, bool GU>
__device__ __forceinline__ void load_a(const ExpertView& v0, const ExpertView& v1, int rb0, int s,
                                       int lane, AChunks<NT>& a) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (GU)
      load_chunk_nt(t < NT / 2 ? v0 : v1, rb0 + (t % (NT / 2)), s, lane, a.w[t], a.s[t]);
    else
      load_chunk_nt(v0, rb0 + t, s, lane, a.w[t], a.s[t]);
  }
}

template <int NT>
__device__ __forceinline__ void dequant_a(const AChunks<NT>& a, int kk, bf16x8 (&av)[NT]) {
#pragma unroll
  for (int tl = 0; tl < NT; ++tl) av[tl] = dequant8(word_of(a.w[tl], kk), scale_of(a.s[tl], kk));
}

__device__ __forceinline__ void split4(const float* v, uint2& hi, uint2& lo) {
  float h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t hb = pack_bf16x2(v[i], 0.0f) & 0xFFFFu;
    h[i] = u2f(hb << 16);
    l[i] = v[i] - h[i];
  }
  hi = make_uint2(pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3]));
  lo = make_uint2(pack_bf16x2(l[0], l[1]), pack_bf16x2(l[2], l[3]));
}

// ---- epilogues -------------------------------------------------------------
// Gate/up: tile t < NT/2 holds gate features f0 + 16 t + 4q + i, tile
// NT/2 + t the same up features; h = SiLU(g) * u with the reference's checks
// (src/layers/swiglu.mojo:191-201), stored as bf16 hi / lo.
// The assignment (token * K + slot; the token for the shared expert) of
// column j of each of the unit's NC column tiles, all requested before the
// first store: a load issued after stores waits for them to complete (one
// counter covers both), which would serialise the epilogue on store latency.
template <int NC>
__device__ __forceinline__ void unit_assignments(const GroupArgs& g, const UnitTokens& ut, int j,
                                                 int (&aa)[NC]) {
// (The load is unconditional — perm has T * K >= T entries — so that no
// path joins with loads of unknown count in flight.)
#pragma unroll
  for (int ct = 0; ct < NC; ++ct) {
    const int p = ut.p0 + min(16 * ct + j, ut.n - 1);
    const int a = g.perm[p];
    aa[ct] = ut.shared ? p : a;
  }
}

// (aa: the unit's assignments of column j, unit_assignments)
template <int NT, int NC>
__device__ __forceinline__ void gu_epilogue(const GroupArgs& g, const UnitTokens& ut, int I,
                                            int f0, int q, int j, const f32x4 (&acc)[NT][NC],
                                            const int (&aa)[NC]) {
  const int K = g.L.K;
#pragma unroll
  for (int ct = 0; ct < NC; ++ct) {
    const int c = 16 * ct + j;
    if (c < ut.n) {
      const int p = ut.p0 + c;
#pragma unroll
      for (int half = 0; half < NT / 2; ++half) {
        const int fr = f0 + 16 * half + 4 * q;
        float hv[4];
        bool bad = false;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gg = acc[half][ct][i], u = acc[NT / 2 + half][ct][i];
          hv[i] = dm_silu(gg) * u;
          bad |= !finite_f(gg) || !finite_f(u) || !finite_f(hv[i]);
        }
        uint2 h2, l2;
        split4(hv, h2, l2);
        const size_t o = (size_t)p * I + fr;
        *reinterpret_cast<uint2*>((ut.shared ? g.hsh : g.hrh) + o) = h2;
        *reinterpret_cast<uint2*>((ut.shared ? g.hsl : g.hrl) + o) = l2;
        if (bad) {  // the error key needs token and slot (a division by K): only here
          const int a = aa[ct];
          const int t = ut.shared ? p : a / K, k = ut.shared ? 0 : a % K;
          const uint32_t ph = ut.shared ? kPhShared : kPhExpert;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float gg = acc[half][ct][i], u = acc[NT / 2 + half][ct][i];
            if (!finite_f(gg) || !finite_f(u) || !finite_f(hv[i])) {
              const uint32_t kind = !finite_f(gg) ? kEkGate : !finite_f(u) ? kEkUp : kEkH;
              record_err(g.status, err_key(ph, t, k, fr + i, kind));
            }
          }
        }
      }
    }
  }
}

// Down: tile tl holds output rows row0 + 16 tl + 4q + i of column j.
template <int NT, int NC>
__device__ __forceinline__ void down_epilogue(const GroupArgs& g, const UnitTokens& ut, int I,
                                              int row0, int q, int j, const f32x4 (&acc)[NT][NC],
                                              const int (&aa)[NC]) {
  const int H = g.L.H, K = g.L.K;
#pragma unroll
  for (int ct = 0; ct < NC; ++ct) {
    const int c = 16 * ct + j;
    if (c < ut.n) {
      const int p = ut.p0 + c;
      const int a = aa[ct];
      float* dst = ut.shared ? g.rs + (size_t)p * H : g.r + (size_t)a * H;
#pragma unroll
      for (int tl = 0; tl < NT; ++tl) {
        const int d0 = row0 + 16 * tl + 4 * q;
        const float* v = reinterpret_cast<const float*>(&acc[tl][ct]);
        *reinterpret_cast<float4*>(dst + d0) = make_float4(v[0], v[1], v[2], v[3]);
        if (!finite_f(v[0]) || !finite_f(v[1]) || !finite_f(v[2]) || !finite_f(v[3])) {
          // the error key needs token and slot (a division by K): only here
          const int t = ut.shared ? p : a / K, k = ut.shared ? 0 : a % K;
          const uint32_t ph = ut.shared ? kPhShared : kPhExpert;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (!finite_f(v[i])) record_err(g.status, err_key(ph, t, k, I + d0 + i, kEkDown));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Big-unit workgroups come in classes b % 8, and the dispatcher places all
// workgroups of a class on one XCD (it hands a launch's workgroups to the
// XCDs in rotation).  The big units are cut into 8 contiguous ranges (the
// units of one expert are adjacent in the unit list) and range c runs in
// class c with each unit's feature blocks next to each other: the blocks of
// a unit share that XCD's L2 for the unit's token rows, and the units of an
// expert share it for the expert's weights.  Item (unit u, block f) of
// workgroup b; false when b has no item.
__device__ __forceinline__ bool big_item(int b, int nbig, int nblk, int& u, int& f) {
  const int c = b & 7, idx = b >> 3;
  const int span = (nbig + 7) >> 3;
  const int ul = idx / nblk;
  u = c * span + ul;
  f = idx - ul * nblk;
  return ul < span && u < nbig;
}
static int big_grid(int nbig, int nblk) { return 8 * ((nbig + 7) / 8) * nblk; }

// ---------------------------------------------------------------------------
// Big units (17..128 tokens): k_big<GU>.  A workgroup of 8 waves takes one
// unit and 128 features (gate/up: gate and up tiles rb0 + w of wave w, so
// that h = SiLU(g) * u is formed in its registers) or 256 output rows (down:
// tiles rb0 + 2w, rb0 + 2w + 1 of wave w), all 8 column tiles of the unit
// (columns past its tokens are never stored).  Every operand is staged in
// LDS by direct-to-LDS loads (global_load_lds_dwordx4: 16 bytes per lane
// land in LDS without passing through registers), three stages in flight:
//   - B rows: 128 rows x 256 bytes per k-step, segment sigma of row r stored
//     at position sigma ^ (r & 15) of its row, so that the 16 rows of one
//     MFMA B operand read distinct LDS banks;
//   - A: the step's 16 A16 chunks (2 per wave) as they lie in memory, and
//     their scales.
// B rows are bf16 hi parts, and when the activations are not all bf16
// values (h always; x when the need-lo flag is set) the lo parts too: then
// a k-step is two stages, hi then lo, with the same A (read twice, the
// second time from L2) and both products summed into the accumulators.
// One barrier per stage: after it, stage s is complete everywhere and the
// buffer of stage s - 1 is free for stage s + 2.
constexpr int kB2Threads = 512;
constexpr int kB2Stages = 3;
constexpr int kB2RowBytes = kQuadCols * 2;                // one token row of a k-step
constexpr int kB2BBytes = kMT * kB2RowBytes;               // 32 KB
constexpr int kB2ABytes = 16 * 1024;                       // 16 A16 chunks
constexpr int kB2SBytes = 16 * 128;                        // their scales
constexpr int kB2Stage = kB2BBytes + kB2ABytes + kB2SBytes;  // 51200 bytes
constexpr size_t kB2Lds = (size_t)kB2Stages * kB2Stage;    // 153600 bytes
constexpr int kB2DmaPerStage = 7;                          // DMA instructions per wave and stage

// 16 bytes per lane from p to LDS at byte address m + 16 * lane (m uniform
// per wave): dma16_lds, inline assembly.  The compiler, which cannot tell the
// stages of one LDS array apart, would otherwise wait for every load in
// flight before any LDS read.  The kernel counts these loads itself
// (s_waitcnt vmcnt); a load the compiler tracks is only ever waited for longer
// because of them.  LDS addresses are 32-bit offsets from lds_u32 of the
// array: arithmetic on a generic pointer into LDS makes the compiler build
// the 64-bit address, which it cannot always lower.
// The B fragments of 8 column tiles (rows 16 ct + j of a staged k-step,
// 16 * 256 bytes apart) as 8 LDS reads in flight together.  Inline assembly
// again: the compiler would otherwise sink each read next to its first use,
// leaving two in flight.  Their registers are not valid before lds_wait8.
__device__ __forceinline__ void lds_read8(uint32_t a, bf16x8 (&b)[kNCT]) {
  static_assert(kNCT == 8 && 16 * kB2RowBytes == 4096, "offsets below");
  asm volatile(
      "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:4096\n\t"
      "ds_read_b128 %2, %8 offset:8192\n\tds_read_b128 %3, %8 offset:12288\n\t"
      "ds_read_b128 %4, %8 offset:16384\n\tds_read_b128 %5, %8 offset:20480\n\t"
      "ds_read_b128 %6, %8 offset:24576\n\tds_read_b128 %7, %8 offset:28672"
      : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5]),
        "=&v"(b[6]), "=&v"(b[7])
      : "v"(a));
}
// Wait until at most N LDS operations are in flight (LDS operations complete
// in order, so every read issued before the last N has landed); b's
// registers are tied to the wait, so no use of them moves above it.
template <int N>
__device__ __forceinline__ void lds_wait8(bf16x8 (&b)[kNCT]) {
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]), "+v"(b[4]), "+v"(b[5]),
                 "+v"(b[6]), "+v"(b[7])
               : "n"(N));
}

__device__ __forceinline__ void gu_small_part(const GroupArgs& g, int bx, int by, int w);
__device__ __forceinline__ void down_small_part(const GroupArgs& g, int bx, int by, int w);

// One big item (unit ui, feature / row block fb) as seen by one lane: what
// the DMA of its stages needs (its A views and tiles, its B rows) and what
// its epilogue needs.
struct BigItem {
  bool valid;
  UnitTokens ut;
  int I, fb, nst, nGQ, KD, t0, t1, st_;
  bool lo;
  ExpertView v0, v1;
  const uint16_t* bhi;
  const uint16_t* blo;
  uint32_t rowo[4];  // this lane's B row offsets (elements) of the four DMA rows
};

template <bool GU>
__device__ __forceinline__ BigItem big_item_state(const GroupArgs& g, int idx, int items,
                                                  int nblk, int w, int lane) {
  BigItem it;
  it.valid = false;
  int ui, fb;
  if (idx >= items || !big_item(idx, g.meta[1], nblk, ui, fb)) return it;
  const LayerDev& L = g.L;
  const int H = L.H, K = L.K;
  it.ut = unit_tokens(g.units[ui], g.off, L.E, g.T, kMT);
  it.I = it.ut.shared ? L.Ish : L.I;
  it.fb = fb;
  if (GU && fb * 128 >= it.I) return it;  // uniform per workgroup
  it.KD = GU ? H : it.I;  // reduction length
  it.nGQ = it.KD / kQuadCols;
  it.lo = GU ? g.need_lo[0] != 0 : true;
  it.nst = it.lo ? 2 * it.nGQ : it.nGQ;
  if (GU) {
    const size_t mat = (size_t)it.I * H;
    it.v0 = it.ut.shared ? ExpertView{L.sgu_nib, L.sgu_sc, it.I, H}
                         : ExpertView{L.gu_nib + (size_t)it.ut.e * mat,
                                      L.gu_sc + (size_t)it.ut.e * 2 * (mat / kGroup), it.I, H};
    it.v1 = {it.v0.nib + mat / 2, it.v0.sc + mat / kGroup, it.I, H};
    it.t0 = it.t1 = fb * 8 + w;
  } else {
    const size_t mat = (size_t)H * it.I;
    it.v0 = it.ut.shared ? ExpertView{L.sd_nib, L.sd_sc, H, it.I}
                         : ExpertView{L.d_nib + (size_t)it.ut.e * (mat / 2),
                                      L.d_sc + (size_t)it.ut.e * (mat / kGroup), H, it.I};
    it.v1 = it.v0;
    // H is a multiple of 128, so the last block may hold 128 rows: waves
    // past H load tiles 0 and 1 (their share of the B rows is still needed)
    // and store nothing
    it.t0 = fb * 256 + 32 * w < H ? fb * 16 + 2 * w : 0;
    it.t1 = it.t0 + 1;
  }
  it.bhi = GU ? g.xhi : (it.ut.shared ? g.hsh : g.hrh);
  it.blo = GU ? g.xlo : (it.ut.shared ? g.hsl : g.hrl);
  // B rows: instructions i = w + 8 m (m < 4) carry rows 4i..4i+3, lane L
  // row 4i + L/16, stored segment L % 16 = global segment (L % 16) ^ (row & 15)
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int r = 4 * (w + 8 * m) + (lane >> 4);
    const int p = it.ut.p0 + min(r, it.ut.n - 1);
    const int sg = (lane & 15) ^ (r & 15);
    const int row = !GU ? p : it.ut.shared ? p : g.perm[p] / K;  // h rows by position, x by token
    it.rowo[m] = (uint32_t)row * (uint32_t)it.KD + sg * 8;
  }
  it.st_ = lane < 8 ? it.t0 : it.t1;
  it.valid = true;
  return it;
}

// The first valid item at idx, idx + step, ... (idx advanced past it).
template <bool GU>
__device__ __forceinline__ BigItem big_next_item(const GroupArgs& g, int& idx, int step, int items,
                                                 int nblk, int w, int lane) {
  BigItem it;
  it.valid = false;
  while (idx < items) {
    it = big_item_state<GU>(g, idx, items, nblk, w, lane);
    idx += step;
    if (it.valid) break;
  }
  return it;
}

// Workgroups 0 .. big_wgs - 1 are persistent: workgroup b takes the big
// items (big_item index space 0 .. items - 1) b, b + big_wgs, ...; with
// big_wgs a multiple of 8, every item of b is of class b % 8, on b's XCD.
// The stage pipeline runs on across items: the first two stages of the
// next item are requested during the last two stages of the current one,
// so they land while its epilogue runs (the start latency of a workgroup,
// ~3.4 us, is paid once per workgroup instead of once per item).
// Workgroups from big_wgs on run the small units of the same stage (sx x sy
// four-wave parts, two per workgroup): dispatched after every big one, they
// fill the CUs the big items' last round leaves idle.
// (The grouping's arrays lead the arguments, preloaded at dispatch: they
// start each workgroup's chain of dependent loads.)
template <bool GU>
__global__ __launch_bounds__(kB2Threads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_big(int items, int big_wgs, const int32_t* meta, const int2* units, const int32_t* off,
           const int32_t* perm, const int* need_lo, GroupArgs gk, int sx, int sy) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds2[];
  GroupArgs g = gk;
  g.meta = meta;
  g.units = units;
  g.off = off;
  g.perm = perm;
  g.need_lo = need_lo;
  if ((int)blockIdx.x >= big_wgs) {
    const int w = gwave_id();
    const int s = 2 * ((int)blockIdx.x - big_wgs) + (w >> 2);
    if (s < sx * sy) {
      if (GU)
        gu_small_part(g, s % sx, s / sx, w & 3);
      else
        down_small_part(g, s % sx, s / sx, w & 3);
    }
    return;
  }
  const LayerDev& L = g.L;
  const int H = L.H;
  const int nblk = GU ? ((L.I > L.Ish ? L.I : L.Ish) + 127) / 128 : (H + 255) / 256;
  const int tid = threadIdx.x, w = gwave_id(), lane = tid & 63, q = lane >> 4, j = lane & 15;
  int idx = blockIdx.x;
  BigItem cur = big_next_item<GU>(g, idx, big_wgs, items, nblk, w, lane);
  if (!cur.valid) return;  // uniform per workgroup
  // this lane's part of the DMA of a stage:
  //   B rows: 4 instructions of 4 rows (rowo)
  //   A: chunk 2w (tile t0) and chunk 2w + 1 (tile t1)
  //   scales: lanes 0..15 carry the 2 x 128 bytes of the same two chunks
  auto issue = [&](const BigItem& it, int ps, int buf) {
    const int s = it.lo ? ps >> 1 : ps;
    const uint16_t* src = (it.lo && (ps & 1)) ? it.blo : it.bhi;
    const uint32_t st = lds_u32(lds2) + (uint32_t)(buf * kB2Stage);
#pragma unroll
    for (int m = 0; m < 4; ++m)
      dma16_lds(src + it.rowo[m] + s * kQuadCols, st + (uint32_t)((w + 8 * m) * 1024));
    dma16_lds(it.v0.nib + a16_nib_offset(it.nGQ, it.t0, s, lane), st + (uint32_t)(kB2BBytes + 2 * w * 1024));
    dma16_lds(it.v1.nib + a16_nib_offset(it.nGQ, it.t1, s, lane),
              st + (uint32_t)(kB2BBytes + (2 * w + 1) * 1024));
    // scales of the two chunks: 128 bytes each, lanes 0..7 and 8..15 (only
    // 16 lanes write: 256 bytes at the wave's own place)
    if (lane < 16)
      dma16_lds(reinterpret_cast<const unsigned char*>((lane < 8 ? it.v0 : it.v1).sc +
                                                       a16_sc_offset(it.nGQ, it.st_, s, 0)) +
                    (lane & 7) * 16,
                st + (uint32_t)(kB2BBytes + kB2ABytes + w * 256));
  };
  issue(cur, 0, 0);
  issue(cur, 1, 1);  // every item has at least two stages (checked at launch)
  int gb = 0;        // stage count of the items before cur (buffer of its stage ps: (gb + ps) % 3)
  while (true) {
    // the next item's state (its loads wait, at the latest, for cur's first
    // two stages, which stage 0 waits for anyway)
    const BigItem nxt = big_next_item<GU>(g, idx, big_wgs, items, nblk, w, lane);
    // the epilogue's assignments, requested now: a load issued after the next
    // item's first stages would wait for them
    int aa[kNCT];
    unit_assignments<kNCT>(g, cur.ut, j, aa);
    f32x4 acc[2][kNCT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int ct = 0; ct < kNCT; ++ct) acc[t][ct] = f32x4{0, 0, 0, 0};
    for (int ps = 0; ps < cur.nst; ++ps) {
      // this wave's loads of stage ps have landed (one later stage may be in flight)
      // (the first stage of an item after the first: everything, since the
      // previous epilogue's stores were issued after this stage's loads and
      // a count of outstanding operations cannot tell them apart)
      static_assert(kB2DmaPerStage == 7, "the wait below counts one stage of 7 loads");
      if ((ps + 1 < cur.nst || nxt.valid) && !(ps == 0 && gb > 0))
        asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      // every wave's loads of stage ps have landed, and every wave has finished
      // reading stage ps - 1 (whose buffer the next issue overwrites)
      __builtin_amdgcn_s_barrier();
      const int gs = gb + ps;
      if (ps + 2 < cur.nst)
        issue(cur, ps + 2, (gs + 2) % kB2Stages);
      else if (nxt.valid)
        issue(nxt, ps + 2 - cur.nst, (gs + 2) % kB2Stages);
      const unsigned char* st = lds2 + (gs % kB2Stages) * kB2Stage;
      const uint4 c0 = *reinterpret_cast<const uint4*>(st + kB2BBytes + 2 * w * 1024 + lane * 16);
      const uint4 c1 =
          *reinterpret_cast<const uint4*>(st + kB2BBytes + (2 * w + 1) * 1024 + lane * 16);
      const uint2 s0 =
          *reinterpret_cast<const uint2*>(st + kB2BBytes + kB2ABytes + w * 256 + j * 8);
      const uint2 s1 =
          *reinterpret_cast<const uint2*>(st + kB2BBytes + kB2ABytes + w * 256 + 128 + j * 8);
      // The 8 B fragments of k-group kk + 1 are read while kk computes.
      bf16x8 bc[kNCT], bn[kNCT];
      const uint32_t bp = lds_u32(lds2) + (uint32_t)((gs % kB2Stages) * kB2Stage + j * kB2RowBytes);
      lds_read8(bp + (q ^ j) * 16, bc);
#pragma unroll
      for (int kk = 0; kk < kGroupsPerQuad; ++kk) {
        if (kk + 1 < kGroupsPerQuad) lds_read8(bp + ((4 * (kk + 1) + q) ^ j) * 16, bn);
        const bf16x8 a0 = dequant8(word_of(c0, kk), scale_of(s0, kk));
        const bf16x8 a1 = dequant8(word_of(c1, kk), scale_of(s1, kk));
        if (kk + 1 < kGroupsPerQuad)
          lds_wait8<kNCT>(bc);
        else
          lds_wait8<0>(bc);
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct) {
          acc[0][ct] = mfma16(a0, bc[ct], acc[0][ct]);
          acc[1][ct] = mfma16(a1, bc[ct], acc[1][ct]);
        }
        if (kk + 1 < kGroupsPerQuad) {
#pragma unroll
          for (int ct = 0; ct < kNCT; ++ct) bc[ct] = bn[ct];
        }
      }
    }
    if (GU)
      gu_epilogue<2, kNCT>(g, cur.ut, cur.I, cur.fb * 128 + 16 * w, q, j, acc, aa);
    else if (cur.fb * 256 + 32 * w < H)
      down_epilogue<2, kNCT>(g, cur.ut, cur.I, cur.fb * 256 + 32 * w, q, j, acc, aa);
    if (!nxt.valid) break;  // uniform
    gb += cur.nst;
    cur = nxt;
  }
}

// k_big's LDS (150 KB) is above the default limit of a launch: raised once
// per device.
static hipError_t big_attrs() {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev < 64 ? 1ull << dev : 0;
  if (bit && (done.load() & bit)) return hipSuccess;
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_big<true>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kB2Lds);
  if (e == hipSuccess)
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_big<false>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kB2Lds);
  if (e == hipSuccess) done.fetch_or(bit);
  return e;
}

// Persistent big workgroups of this device: its CU count rounded down to a
// multiple of 8 (0 when it cannot be read).
static int big_persistent_wgs() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cus[dev].load();
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    n &= ~7;
    cus[dev].store(n);
  }
  return n;
}

// ---------------------------------------------------------------------------
// Small units (<= 16 tokens): one column tile.  Waves are independent (no
// LDS, no barrier): each wave owns 2 A tiles (gate/up: 16 features, gate and
// up tile; down: 32 output rows) and reads its B fragments (lane (q, j):
// token j, columns 8q..8q+7 of each group) straight from memory into the
// same prefetch ring as the A chunks, P k-steps ahead.  At most 168 registers
// per lane, so that three waves share a SIMD and their loads overlap.
constexpr int kSmallTiles = 2;

template <bool LO>
struct SmallStep {
  AChunks<kSmallTiles> a;
  v4u b[kGroupsPerQuad];
  v4u bl[LO ? kGroupsPerQuad : 1];
};

template <bool LO, bool GU>
__device__ __forceinline__ void small_load(const ExpertView& v0, const ExpertView& v1, int rb0,
                                           int s, int lane, const uint16_t* bh,
                                           const uint16_t* bl, SmallStep<LO>& st) {
  load_a<kSmallTiles, GU>(v0, v1, rb0, s, lane, st.a);
#pragma unroll
  for (int kk = 0; kk < kGroupsPerQuad; ++kk) {
    const int o = s * kQuadCols + kk * kGroup;
    st.b[kk] = *reinterpret_cast<const v4u*>(bh + o);
    if (LO) st.bl[kk] = *reinterpret_cast<const v4u*>(bl + o);
  }
}

template <bool LO>
__device__ __forceinline__ void small_step(const SmallStep<LO>& st,
                                           f32x4 (&acc)[kSmallTiles][1]) {
#pragma unroll
  for (int kk = 0; kk < kGroupsPerQuad; ++kk) {
    bf16x8 av[kSmallTiles];
    dequant_a<kSmallTiles>(st.a, kk, av);
    const bf16x8 b = __builtin_bit_cast(bf16x8, st.b[kk]);
#pragma unroll
    for (int tl = 0; tl < kSmallTiles; ++tl) acc[tl][0] = mfma16(av[tl], b, acc[tl][0]);
    if (LO) {
      const bf16x8 b2 = __builtin_bit_cast(bf16x8, st.bl[kk]);
#pragma unroll
      for (int tl = 0; tl < kSmallTiles; ++tl) acc[tl][0] = mfma16(av[tl], b2, acc[tl][0]);
    }
  }
}

// bh / bl point at this lane's B row (+ 8q) at column 0.  The ring slot of a
// step is a constant of the unrolled body; steps past the last are clamped
// to it (redundant loads only when ns % P != 0).
template <bool LO, bool GU, int P>
__device__ __forceinline__ void small_loop(const ExpertView& v0, const ExpertView& v1, int rb0,
                                           const uint16_t* bh, const uint16_t* bl, int ns,
                                           f32x4 (&acc)[kSmallTiles][1]) {
  const int lane = threadIdx.x & 63;
  SmallStep<LO> ring[P];
#pragma unroll
  for (int u = 0; u < P; ++u) small_load<LO, GU>(v0, v1, rb0, min(u, ns - 1), lane, bh, bl, ring[u]);
#pragma unroll
  for (int tl = 0; tl < kSmallTiles; ++tl) acc[tl][0] = f32x4{0, 0, 0, 0};
  int s0 = 0;
  for (; s0 + P < ns; s0 += P) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      small_step<LO>(ring[u], acc);
      small_load<LO, GU>(v0, v1, rb0, min(s0 + u + P, ns - 1), lane, bh, bl, ring[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < P; ++u)
    if (s0 + u < ns) small_step<LO>(ring[u], acc);
}

static_assert(kMT == kUnitBig && kSmallMax == kUnitSmall, "unit sizes of dm_grouped.h");
constexpr int kSmallGuCols = 4 * 16;   // features per small gate/up workgroup
constexpr int kSmallDnRows = 4 * 32;   // output rows per small down workgroup

// Small gate/up unit bx (of those after the big ones), features by * 64 ..,
// on wave w of four; no barriers, so that four waves of a larger workgroup
// can run it too.
__device__ __forceinline__ void gu_small_part(const GroupArgs& g, int bx, int by, int w) {
  const int ui = g.meta[1] + bx;
  if (ui >= g.meta[0]) return;
  const UnitTokens ut = unit_tokens(g.units[ui], g.off, g.L.E, g.T, kSmallMax);
  const LayerDev& L = g.L;
  const int H = L.H, K = L.K, I = ut.shared ? L.Ish : L.I;
  const int lane = threadIdx.x & 63, q = lane >> 4, j = lane & 15;
  const int f0 = by * kSmallGuCols + 16 * w;
  if (f0 >= I) return;  // uniform per wave
  const size_t mat = (size_t)I * H;
  const ExpertView gv = ut.shared ? ExpertView{L.sgu_nib, L.sgu_sc, I, H}
                                  : ExpertView{L.gu_nib + (size_t)ut.e * mat,
                                               L.gu_sc + (size_t)ut.e * 2 * (mat / kGroup), I, H};
  const ExpertView uv = {gv.nib + mat / 2, gv.sc + mat / kGroup, I, H};
  const int r = min(j, ut.n - 1);
  const int t = ut.shared ? ut.p0 + r : g.perm[ut.p0 + r] / K;
  const size_t o = (size_t)t * H + 8 * q;
  f32x4 acc[kSmallTiles][1];
  const int ns = H / kQuadCols;
  if (g.need_lo[0] != 0)
    small_loop<true, true, 2>(gv, uv, f0 / kTileRows, g.xhi + o, g.xlo + o, ns, acc);
  else
    small_loop<false, true, 4>(gv, uv, f0 / kTileRows, g.xhi + o, g.xlo + o, ns, acc);
  int aa[1];
  unit_assignments<1>(g, ut, j, aa);
  gu_epilogue<kSmallTiles, 1>(g, ut, I, f0, q, j, acc, aa);
}

// Small down unit bx, output rows by * 128 .., on wave w of four.
__device__ __forceinline__ void down_small_part(const GroupArgs& g, int bx, int by, int w) {
  const int ui = g.meta[1] + bx;
  if (ui >= g.meta[0]) return;
  const UnitTokens ut = unit_tokens(g.units[ui], g.off, g.L.E, g.T, kSmallMax);
  const LayerDev& L = g.L;
  const int H = L.H, I = ut.shared ? L.Ish : L.I;
  const int lane = threadIdx.x & 63, q = lane >> 4, j = lane & 15;
  const int row0 = by * kSmallDnRows + 32 * w;
  if (row0 >= H) return;
  const size_t mat = (size_t)H * I;
  const ExpertView dv = ut.shared ? ExpertView{L.sd_nib, L.sd_sc, H, I}
                                  : ExpertView{L.d_nib + (size_t)ut.e * (mat / 2),
                                               L.d_sc + (size_t)ut.e * (mat / kGroup), H, I};
  const size_t o = (size_t)(ut.p0 + min(j, ut.n - 1)) * I + 8 * q;
  f32x4 acc[kSmallTiles][1];
  small_loop<true, false, 2>(dv, dv, row0 / kTileRows, (ut.shared ? g.hsh : g.hrh) + o,
                             (ut.shared ? g.hsl : g.hrl) + o, I / kQuadCols, acc);
  int aa[1];
  unit_assignments<1>(g, ut, j, aa);
  down_epilogue<kSmallTiles, 1>(g, ut, I, row0, q, j, acc, aa);
}

// The grouping's arrays come first among the arguments: they start each
// workgroup's chain of dependent loads (meta -> units -> off -> perm) and
// are preloaded into scalar registers at dispatch.
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(3))) void k_gu_small(
    const int32_t* meta, const int2* units, const int32_t* off, const int32_t* perm,
    GroupArgs gk) {
  GroupArgs g = gk;
  g.meta = meta;
  g.units = units;
  g.off = off;
  g.perm = perm;
  gu_small_part(g, blockIdx.x, blockIdx.y, gwave_id());
}

__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(3))) void k_down_small(
    const int32_t* meta, const int2* units, const int32_t* off, const int32_t* perm,
    GroupArgs gk) {
  GroupArgs g = gk;
  g.meta = meta;
  g.units = units;
  g.off = off;
  g.perm = perm;
  down_small_part(g, blockIdx.x, blockIdx.y, gwave_id());
}

hipError_t launch_experts_grouped(const LayerDev& L, const uint16_t* xhi, const uint16_t* xlo,
                                  const int* need_lo, const int32_t* off, const int32_t* perm,
                                  const int2* units, const int32_t* meta, int T, uint16_t* hrh,
                                  uint16_t* hrl, uint16_t* hsh, uint16_t* hsl, float* r,
                                  float* rs, unsigned long long* status, hipStream_t st) {
  const GroupArgs g = {L, xhi, xlo, need_lo, off, perm, units, meta, T,
                       hrh, hrl, hsh, hsl, r, rs, status};
  const int nu = group_units_max(T, L.K, L.E);
  // grids sized by the bound of each unit kind, so that few workgroups
  // start only to find no unit (each still costs a dispatch and its first
  // instructions)
  const int nbig = min(nu, big_units_max(T, L.K, L.E));
  const int nsmall = min(nu, small_units_max(T, L.K, L.E));
  const int imax = L.I > L.Ish ? L.I : L.Ish;
  // an expert holds at most T tokens (its ids per token are distinct), so
  // units of more than 2 * kSmallMax tokens need T > 2 * kSmallMax
  const bool big = T > 2 * kSmallMax;
  // the big items' B row offsets are 32-bit element offsets
  if ((size_t)T * L.K * imax >= (1ull << 32) || (size_t)T * L.H >= (1ull << 32))
    return hipErrorInvalidValue;
  if (big) {
    const hipError_t e = big_attrs();
    if (e != hipSuccess) return e;
  }
  const int gy = (imax + kSmallGuCols - 1) / kSmallGuCols, dy = (L.H + kSmallDnRows - 1) / kSmallDnRows;
  if (big) {
    // the small gate/up units ride in the big gate/up grid, after the big
    // units, and fill the CUs its last round leaves idle; the down stage's
    // big units run about five rounds, so its small units keep their own
    // launch (dispatched after every big one they would add rounds)
    const int bg = big_grid(nbig, (imax + 127) / 128), bd = big_grid(nbig, (L.H + 255) / 256);
    // persistent big workgroups: one per CU (150 KB of LDS each), a multiple
    // of 8 so that an item keeps its class; every item needs two stages or
    // more (gate/up: H / 128 of them, down: 2 I / 128)
    const int pw = L.H >= 256 ? big_persistent_wgs() : 0;
    const int wg_g = pw > 0 && pw < bg ? pw : bg, wg_d = pw > 0 && pw < bd ? pw : bd;
    hipLaunchKernelGGL(k_big<true>, dim3(wg_g + (nsmall * gy + 1) / 2), dim3(kB2Threads), kB2Lds,
                       st, bg, wg_g, meta, units, off, perm, need_lo, g, nsmall, gy);
    hipLaunchKernelGGL(k_big<false>, dim3(wg_d), dim3(kB2Threads), kB2Lds, st, bd, wg_d, meta,
                       units, off, perm, need_lo, g, 0, 0);
  } else {
    hipLaunchKernelGGL(k_gu_small, dim3(nsmall, gy), dim3(kGThreads), 0, st, meta, units, off, perm,
                       g);
  }
  hipLaunchKernelGGL(k_down_small, dim3(nsmall, dy), dim3(kGThreads), 0, st, meta, units, off,
                     perm, g);
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
                                                  unsigned long long* status,
                                                  int* __restrict__ clear_flag) {
  // four consecutive outputs per thread (H % 4 == 0); the slots' rows are
  // requested eight at a time before their products
  const int t = blockIdx.y, d = (blockIdx.x * 256 + threadIdx.x) * 4;
  // the last kernel of a call clears the call's need-lo flag for the next
  if (clear_flag && t == 0 && d == 0) *clear_flag = 0;
  if (d >= H) return;
  const float* pt = probs + (size_t)t * K;
  float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = 0; k0 < K; k0 += 8) {
    float4 rv[8];
    float pv[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const int k = min(k0 + kk, K - 1);
      rv[kk] = *reinterpret_cast<const float4*>(r + ((size_t)t * K + k) * H + d);
      pv[kk] = pt[k];
    }
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      if (k0 + kk < K) {
        a[0] = a[0] + pv[kk] * rv[kk].x;
        a[1] = a[1] + pv[kk] * rv[kk].y;
        a[2] = a[2] + pv[kk] * rv[kk].z;
        a[3] = a[3] + pv[kk] * rv[kk].w;
      }
    }
  }
  const float g = shg[t];
  const float4 sv = *reinterpret_cast<const float4*>(rs + (size_t)t * H + d);
  float tot[4] = {a[0] + g * sv.x, a[1] + g * sv.y, a[2] + g * sv.z, a[3] + g * sv.w};
  if (residual) {
    const float4 rr = *reinterpret_cast<const float4*>(residual + (size_t)t * H + d);
    tot[0] = tot[0] + rr.x;
    tot[1] = tot[1] + rr.y;
    tot[2] = tot[2] + rr.z;
    tot[3] = tot[3] + rr.w;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (!finite_f(tot[i])) record_err(status, err_key(kPhAgg, t, 0, d + i, 0));
  *reinterpret_cast<float4*>(y + (size_t)t * H + d) = make_float4(tot[0], tot[1], tot[2], tot[3]);
}

hipError_t launch_combine(const float* r, const float* rs, const float* probs, const float* shg,
                          const float* residual, int T, int H, int K, float* y,
                          unsigned long long* status, hipStream_t st, int* clear_flag) {
  if (H % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_combine, dim3((H / 4 + 255) / 256, T), dim3(256), 0, st, r, rs, probs, shg,
                     residual, H, K, y, status, clear_flag);
  return hipGetLastError();
}

}  // namespace dm
