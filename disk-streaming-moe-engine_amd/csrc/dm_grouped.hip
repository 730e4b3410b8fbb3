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
//   k_gu_big2       h = SiLU(W_g x) * (W_u x) for big units of bf16
//                   activations: token rows, 4-bit weights and scales all
//                   staged in LDS by direct-to-LDS loads, three k-steps in
//                   flight, weights dequantised from LDS (16 features x 32 k
//                   per MFMA)
//   k_gu_big        the same when activations carry lo parts: A = 4-bit
//                   weights dequantised in registers, B = the unit's token
//                   rows (hi and lo) staged in LDS per 128-column step
//                   (double-buffered, one barrier per step)
//   k_gu_small      the same for units of <= 16 tokens: B fragments straight
//                   from memory, no LDS and no barriers, deeper prefetch
//   k_down_big / k_down_small   r = W_d h, B = h as bf16 hi + lo parts
//   k_combine       y = sum_k p_k r_k + g r_sh (+ residual), reference order
//
// Each token's outputs depend only on its own column of the MFMA tiles, so
// the placement of tokens inside an expert's tiles (atomic scatter) does not
// change any result bit.
#include <hip/hip_runtime.h>

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

__global__ __launch_bounds__(1024) void k_group_build(const int32_t* __restrict__ ids, int T, int K,
                                                      int E, int32_t* __restrict__ off,
                                                      int32_t* __restrict__ perm,
                                                      int2* __restrict__ units,
                                                      int32_t* __restrict__ meta) {
  // cnt[E] | cur[E] | 4 scans of 1024: counts, full units, partial big, small
  extern __shared__ int lds[];
  int* cnt = lds;
  int* cur = lds + E;
  int* sc = lds + 2 * E;
  const int tid = threadIdx.x, TK = T * K;
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int a = tid; a < TK; a += 1024) {
    const int e = min(max((int)ids[a], 0), E - 1);
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
#pragma unroll
  for (int i = 0; i < 4; ++i) sc[i * 1024 + tid] = v[i];
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {  // inclusive Hillis-Steele scans
    int a[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = tid >= d ? sc[i * 1024 + tid - d] : 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i * 1024 + tid] += a[i];
    __syncthreads();
  }
  const int nf = sc[1024 + 1023], npb = sc[2048 + 1023], nps = sc[3072 + 1023];
  int snf, spb, sps;
  unit_split(T, snf, spb, sps);
  const int pb0 = nf + snf, s0 = pb0 + npb + spb;
  int base = sc[tid] - v[0], fb = sc[1024 + tid] - v[1], pb = pb0 + sc[2048 + tid] - v[2],
      ps = s0 + sc[3072 + tid] - v[3];
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
  for (int a = tid; a < TK; a += 1024) {
    const int e = min(max((int)ids[a], 0), E - 1);
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

hipError_t launch_group_build(const int32_t* ids, int T, int K, int E, int32_t* off,
                              int32_t* perm, int2* units, int32_t* meta, hipStream_t st) {
  const size_t lds = (size_t)(2 * E + 4096) * sizeof(int);
  hipLaunchKernelGGL(k_group_build, dim3(1), dim3(1024), lds, st, ids, T, K, E, off, perm, units,
                     meta);
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
template <int NT, int NC>
__device__ __forceinline__ void gu_epilogue(const GroupArgs& g, const UnitTokens& ut, int I,
                                            int f0, int q, int j, const f32x4 (&acc)[NT][NC]) {
  const int K = g.L.K;
#pragma unroll
  for (int ct = 0; ct < NC; ++ct) {
    const int c = 16 * ct + j;
    if (c < ut.n) {
      const int p = ut.p0 + c;
      const int a = ut.shared ? p : g.perm[p];
      const int t = ut.shared ? p : a / K, k = ut.shared ? 0 : a % K;
#pragma unroll
      for (int half = 0; half < NT / 2; ++half) {
        const int fr = f0 + 16 * half + 4 * q;
        float hv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gg = acc[half][ct][i], u = acc[NT / 2 + half][ct][i];
          hv[i] = dm_silu(gg) * u;
          if (!finite_f(gg) || !finite_f(u) || !finite_f(hv[i])) {
            const uint32_t ph = ut.shared ? kPhShared : kPhExpert;
            const uint32_t kind = !finite_f(gg) ? kEkGate : !finite_f(u) ? kEkUp : kEkH;
            record_err(g.status, err_key(ph, t, k, fr + i, kind));
          }
        }
        uint2 h2, l2;
        split4(hv, h2, l2);
        const size_t o = (size_t)p * I + fr;
        *reinterpret_cast<uint2*>((ut.shared ? g.hsh : g.hrh) + o) = h2;
        *reinterpret_cast<uint2*>((ut.shared ? g.hsl : g.hrl) + o) = l2;
      }
    }
  }
}

// Down: tile tl holds output rows row0 + 16 tl + 4q + i of column j.
template <int NT, int NC>
__device__ __forceinline__ void down_epilogue(const GroupArgs& g, const UnitTokens& ut, int I,
                                              int row0, int q, int j,
                                              const f32x4 (&acc)[NT][NC]) {
  const int H = g.L.H, K = g.L.K;
#pragma unroll
  for (int ct = 0; ct < NC; ++ct) {
    const int c = 16 * ct + j;
    if (c < ut.n) {
      const int p = ut.p0 + c;
      const int a = ut.shared ? p : g.perm[p];
      const int t = ut.shared ? p : a / K, k = ut.shared ? 0 : a % K;
      float* dst = ut.shared ? g.rs + (size_t)t * H : g.r + (size_t)a * H;
#pragma unroll
      for (int tl = 0; tl < NT; ++tl) {
        const int d0 = row0 + 16 * tl + 4 * q;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = acc[tl][ct][i];
          if (!finite_f(v[i])) {
            const uint32_t ph = ut.shared ? kPhShared : kPhExpert;
            record_err(g.status, err_key(ph, t, k, I + d0 + i, kEkDown));
          }
        }
        *reinterpret_cast<float4*>(dst + d0) = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Big units.  A workgroup of 4 waves takes one unit (17..128 tokens) and
// 128 features (gate/up: wave w owns features f0 = 128 blockIdx.y + 32 w ..
// f0 + 31, i.e. gate tiles f0, f0 + 16 and the same up tiles) or 256 output
// rows (down: wave w owns rows 256 blockIdx.y + 64 w .. + 63).  All 8 column
// tiles are computed (columns past the unit's tokens are never stored).
//
// B staging: per k-step of 128 columns, the unit's 128 rows (row r clamped
// to the last token) move global -> registers -> LDS: thread tid carries the
// 16-byte segment tid & 15 of rows (tid >> 4) + 16 i.  Two LDS buffers: step
// s computes from buffer s & 1 while the rows of step s + 1 are written to
// the other and those of step s + 2 are in flight; one barrier per step.
// Rows are padded to kBPitch elements so that the 16 rows of one MFMA operand
// fetch (ds_read_b128 by lanes j = 0..15 at one q) fall on 16 distinct
// 4-bank groups.  A: the chunks of step s + 2 are requested while step s
// computes (kBigPre = 2, which also keeps the buffer index of each unrolled
// step a constant).
constexpr int kBPitch = kQuadCols + 8;
constexpr int kBTile = kMT * kBPitch;  // elements per staged plane
constexpr int kBigPre = 2;
constexpr size_t kBigLds = 2 * 2 * kBTile * sizeof(uint16_t);  // 2 buffers x (hi, lo)

__device__ __forceinline__ bf16x8 lds_b(const uint16_t* bs, int ct, int kk, int q, int j) {
  return *reinterpret_cast<const bf16x8*>(bs + (ct * 16 + j) * kBPitch + kk * kGroup + 8 * q);
}

template <bool LO>
__device__ __forceinline__ void rows_load(const uint16_t* __restrict__ sh,
                                          const uint16_t* __restrict__ sl,
                                          const int (&roff)[kNCT], int s, v4u (&bh)[kNCT],
                                          v4u (&bl)[kNCT]) {
#pragma unroll
  for (int i = 0; i < kNCT; ++i) {
    const uint32_t o = (uint32_t)roff[i] + (uint32_t)(s * kQuadCols);
    bh[i] = *reinterpret_cast<const v4u*>(sh + o);
    if (LO) bl[i] = *reinterpret_cast<const v4u*>(sl + o);
  }
}

template <bool LO>
__device__ __forceinline__ void rows_store(uint16_t* bs, int srow, int seg, const v4u (&bh)[kNCT],
                                           const v4u (&bl)[kNCT]) {
#pragma unroll
  for (int i = 0; i < kNCT; ++i) {
    const int o = (srow + 16 * i) * kBPitch + seg * 8;
    *reinterpret_cast<v4u*>(bs + o) = bh[i];
    if (LO) *reinterpret_cast<v4u*>(bs + kBTile + o) = bl[i];
  }
}

// One k-step of a big unit: 4 k-groups x (4 A tiles x 8 column tiles).
template <bool LO>
__device__ __forceinline__ void big_step(const uint16_t* bs, const AChunks<4>& a, int q, int j,
                                         f32x4 (&acc)[4][kNCT]) {
#pragma unroll
  for (int kk = 0; kk < kGroupsPerQuad; ++kk) {
    bf16x8 av[4];
    dequant_a<4>(a, kk, av);
#pragma unroll
    for (int ct = 0; ct < kNCT; ++ct) {
      const bf16x8 b = lds_b(bs, ct, kk, q, j);
#pragma unroll
      for (int tl = 0; tl < 4; ++tl) acc[tl][ct] = mfma16(av[tl], b, acc[tl][ct]);
      if (LO) {
        const bf16x8 b2 = lds_b(bs + kBTile, ct, kk, q, j);
#pragma unroll
        for (int tl = 0; tl < 4; ++tl) acc[tl][ct] = mfma16(av[tl], b2, acc[tl][ct]);
      }
    }
  }
}

// The k-loop of a big unit over ns steps (A views, staged rows from sh/sl).
template <bool LO, bool GU>
__device__ __forceinline__ void big_loop(uint16_t* lds, const ExpertView& v0,
                                         const ExpertView& v1, int rb0, bool active,
                                         const uint16_t* sh, const uint16_t* sl,
                                         const int (&roff)[kNCT], int ns, f32x4 (&acc)[4][kNCT]) {
  const int tid = threadIdx.x, lane = tid & 63, q = lane >> 4, j = lane & 15;
  const int seg = tid & 15, srow = tid >> 4;
  constexpr int kBuf = 2 * kBTile;  // elements per buffer (hi, lo planes)
  v4u bh[kNCT], bl[kNCT];
  rows_load<LO>(sh, sl, roff, 0, bh, bl);
  rows_store<LO>(lds, srow, seg, bh, bl);
  rows_load<LO>(sh, sl, roff, min(1, ns - 1), bh, bl);
  AChunks<4> ring[kBigPre];
  if (active) {
#pragma unroll
    for (int u = 0; u < kBigPre; ++u) load_a<4, GU>(v0, v1, rb0, min(u, ns - 1), lane, ring[u]);
  }
#pragma unroll
  for (int tl = 0; tl < 4; ++tl)
#pragma unroll
    for (int ct = 0; ct < kNCT; ++ct) acc[tl][ct] = f32x4{0, 0, 0, 0};
  __syncthreads();
  int s0 = 0;
  for (; s0 + kBigPre < ns; s0 += kBigPre) {
#pragma unroll
    for (int u = 0; u < kBigPre; ++u) {
      const int s = s0 + u;
      rows_store<LO>(lds + ((u + 1) & 1) * kBuf, srow, seg, bh, bl);
      rows_load<LO>(sh, sl, roff, min(s + 2, ns - 1), bh, bl);
      if (active) {
        big_step<LO>(lds + (u & 1) * kBuf, ring[u], q, j, acc);
        load_a<4, GU>(v0, v1, rb0, s + kBigPre, lane, ring[u]);
      }
      __syncthreads();
    }
  }
  // the last 1..kBigPre steps: nothing left to request
#pragma unroll
  for (int u = 0; u < kBigPre; ++u) {
    const int s = s0 + u;
    if (s < ns) {
      if (s + 1 < ns) rows_store<LO>(lds + ((u + 1) & 1) * kBuf, srow, seg, bh, bl);
      if (active) big_step<LO>(lds + (u & 1) * kBuf, ring[u], q, j, acc);
      __syncthreads();
    }
  }
}

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

__global__ __launch_bounds__(kGThreads) void k_gu_big(GroupArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint16_t glds[];
  if (g.need_lo[0] == 0) return;  // bf16 activations: k_gu_big2
  int ui, fb;
  const int nblk = ((g.L.I > g.L.Ish ? g.L.I : g.L.Ish) + 127) / 128;
  if (!big_item(blockIdx.x, g.meta[1], nblk, ui, fb)) return;
  const UnitTokens ut = unit_tokens(g.units[ui], g.off, g.L.E, g.T, kMT);
  const LayerDev& L = g.L;
  const int H = L.H, K = L.K, I = ut.shared ? L.Ish : L.I;
  if (fb * 128 >= I) return;  // uniform per workgroup
  const int tid = threadIdx.x, w = gwave_id(), lane = tid & 63, q = lane >> 4, j = lane & 15;
  const int f0 = fb * 128 + 32 * w;
  const bool active = f0 < I;  // uniform per wave
  const int rb0 = active ? f0 / kTileRows : 0;
  const size_t mat = (size_t)I * H;
  const ExpertView gv = ut.shared ? ExpertView{L.sgu_nib, L.sgu_sc, I, H}
                                  : ExpertView{L.gu_nib + (size_t)ut.e * mat,
                                               L.gu_sc + (size_t)ut.e * 2 * (mat / kGroup), I, H};
  const ExpertView uv = {gv.nib + mat / 2, gv.sc + mat / kGroup, I, H};
  int roff[kNCT];
  const int seg = tid & 15, srow = tid >> 4;
#pragma unroll
  for (int i = 0; i < kNCT; ++i) {
    const int r = min(srow + 16 * i, ut.n - 1);
    const int t = ut.shared ? ut.p0 + r : g.perm[ut.p0 + r] / K;
    roff[i] = t * H + seg * 8;
  }
  f32x4 acc[4][kNCT];
  big_loop<true, true>(glds, gv, uv, rb0, active, g.xhi, g.xlo, roff, H / kQuadCols, acc);
  if (active) gu_epilogue<4, kNCT>(g, ut, I, f0, q, j, acc);
}

// ---------------------------------------------------------------------------
// Big units for bf16 activations (no lo parts), gate/up: k_gu_big2.  The same
// work item as k_gu_big (a unit of up to 128 tokens x 128 features), on 8
// waves, with every operand staged in LDS by direct-to-LDS loads
// (global_load_lds_dwordx4: 16 bytes per lane land in LDS without passing
// through registers), three k-steps in flight:
//   - token rows: 128 rows x 256 bytes per k-step, segment sigma of row r
//     stored at position sigma ^ (r & 15) of its row, so that the 16 rows of
//     one MFMA B operand read distinct LDS banks;
//   - A: the 16 A16 chunks of the step (8 gate tiles, 8 up tiles of the
//     workgroup's 128 features) as they lie in memory, and their scales.
// Wave w owns gate tile w and up tile w (features 16w..16w+15 of the block)
// and all 8 column tiles, so h = SiLU(g) * u is formed in its registers.
// One barrier per k-step: after it, stage s is complete everywhere and the
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

typedef __attribute__((address_space(3))) void lptr_t;
// 16 bytes per lane from p to LDS at dst + 16 * lane (dst uniform per wave).
// Issued as inline assembly: the compiler, which cannot tell the stages of
// one LDS array apart, would otherwise wait for every load in flight before
// any LDS read.  The kernel counts these loads itself (s_waitcnt vmcnt); a
// load the compiler tracks is only ever waited for longer because of them.
__device__ __forceinline__ void dma16(const void* p, void* dst) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lptr_t*)dst);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(p), "s"(m)
               : "memory", "m0");
}

__global__ __launch_bounds__(kB2Threads) void k_gu_big2(GroupArgs g) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds2[];
  if (g.need_lo[0] != 0) return;  // activations with lo parts: k_gu_big
  int ui, fb;
  const int nblk = ((g.L.I > g.L.Ish ? g.L.I : g.L.Ish) + 127) / 128;
  if (!big_item(blockIdx.x, g.meta[1], nblk, ui, fb)) return;
  const UnitTokens ut = unit_tokens(g.units[ui], g.off, g.L.E, g.T, kMT);
  const LayerDev& L = g.L;
  const int H = L.H, K = L.K, I = ut.shared ? L.Ish : L.I;
  if (fb * 128 >= I) return;  // uniform per workgroup
  const int tid = threadIdx.x, w = gwave_id(), lane = tid & 63, q = lane >> 4, j = lane & 15;
  const int rb0 = fb * 8;  // first 16-row tile of the block (gate and up)
  const int nGQ = H / kQuadCols, ns = nGQ;
  const size_t mat = (size_t)I * H;
  const ExpertView gv = ut.shared ? ExpertView{L.sgu_nib, L.sgu_sc, I, H}
                                  : ExpertView{L.gu_nib + (size_t)ut.e * mat,
                                               L.gu_sc + (size_t)ut.e * 2 * (mat / kGroup), I, H};
  const ExpertView uv = {gv.nib + mat / 2, gv.sc + mat / kGroup, I, H};
  // this lane's part of the DMA of a stage:
  //   token rows: instructions i = w + 8 m (m < 4) carry rows 4i..4i+3, lane
  //   L row 4i + L/16, stored segment L % 16 = global segment (L % 16) ^ (row & 15)
  //   A: chunk w (gate tile rb0 + w) and chunk 8 + w (up tile rb0 + w)
  //   scales: lanes 0..15 carry the 2 x 128 bytes of the same two chunks
  const uint16_t* rowp[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int r = 4 * (w + 8 * m) + (lane >> 4);
    const int rc = min(r, ut.n - 1);
    const int t = ut.shared ? ut.p0 + rc : g.perm[ut.p0 + rc] / K;
    const int sg = (lane & 15) ^ (r & 15);
    rowp[m] = g.xhi + (size_t)t * H + sg * 8;
  }
  const ExpertView& sv = lane < 8 ? gv : uv;  // scale piece owner (lanes 0..15)
  auto issue = [&](int s, int buf) {
    unsigned char* st = lds2 + buf * kB2Stage;
#pragma unroll
    for (int m = 0; m < 4; ++m) dma16(rowp[m] + s * kQuadCols, st + (w + 8 * m) * 1024);
    dma16(gv.nib + a16_nib_offset(nGQ, rb0 + w, s, lane), st + kB2BBytes + w * 1024);
    dma16(uv.nib + a16_nib_offset(nGQ, rb0 + w, s, lane), st + kB2BBytes + (8 + w) * 1024);
    // scales of (gate tile w, up tile w): 128 bytes each, lanes 0..7 and 8..15
    // (only 16 lanes write: 256 bytes at the wave's own place)
    if (lane < 16)
      dma16(reinterpret_cast<const unsigned char*>(sv.sc + a16_sc_offset(nGQ, rb0 + w, s, 0)) +
                (lane & 7) * 16,
            st + kB2BBytes + kB2ABytes + w * 256);
  };
  f32x4 acc[2][kNCT];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int ct = 0; ct < kNCT; ++ct) acc[t][ct] = f32x4{0, 0, 0, 0};
  issue(0, 0);
  if (ns > 1) issue(1, 1);
  for (int s = 0; s < ns; ++s) {
    // this wave's loads of stage s have landed (one later stage may be in flight)
    static_assert(kB2DmaPerStage == 7, "the wait below counts one stage of 7 loads");
    if (s + 1 < ns)
      asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // every wave's loads of stage s have landed, and every wave has finished
    // reading stage s - 1 (whose buffer the next issue overwrites)
    __builtin_amdgcn_s_barrier();
    if (s + 2 < ns) issue(s + 2, (s + 2) % kB2Stages);
    const unsigned char* st = lds2 + (s % kB2Stages) * kB2Stage;
    const uint4 cg = *reinterpret_cast<const uint4*>(st + kB2BBytes + w * 1024 + lane * 16);
    const uint4 cu = *reinterpret_cast<const uint4*>(st + kB2BBytes + (8 + w) * 1024 + lane * 16);
    const uint2 sgs = *reinterpret_cast<const uint2*>(st + kB2BBytes + kB2ABytes + w * 256 + j * 8);
    const uint2 sus =
        *reinterpret_cast<const uint2*>(st + kB2BBytes + kB2ABytes + w * 256 + 128 + j * 8);
#pragma unroll
    for (int kk = 0; kk < kGroupsPerQuad; ++kk) {
      const bf16x8 ag = dequant8(word_of(cg, kk), scale_of(sgs, kk));
      const bf16x8 au = dequant8(word_of(cu, kk), scale_of(sus, kk));
      const int sg = (4 * kk + q) ^ j;
#pragma unroll
      for (int ct = 0; ct < kNCT; ++ct) {
        const bf16x8 b =
            *reinterpret_cast<const bf16x8*>(st + (ct * 16 + j) * kB2RowBytes + sg * 16);
        acc[0][ct] = mfma16(ag, b, acc[0][ct]);
        acc[1][ct] = mfma16(au, b, acc[1][ct]);
      }
    }
  }
  gu_epilogue<2, kNCT>(g, ut, I, fb * 128 + 16 * w, q, j, acc);
}

__global__ __launch_bounds__(kGThreads) void k_down_big(GroupArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint16_t glds[];
  int ui, rbk;
  if (!big_item(blockIdx.x, g.meta[1], (g.L.H + 255) / 256, ui, rbk)) return;
  const UnitTokens ut = unit_tokens(g.units[ui], g.off, g.L.E, g.T, kMT);
  const LayerDev& L = g.L;
  const int H = L.H, I = ut.shared ? L.Ish : L.I;
  const int tid = threadIdx.x, w = gwave_id(), lane = tid & 63, q = lane >> 4, j = lane & 15;
  const int row0 = rbk * 256 + 64 * w;
  const bool active = row0 < H;
  const int rb0 = active ? row0 / kTileRows : 0;
  const size_t mat = (size_t)H * I;
  const ExpertView dv = ut.shared ? ExpertView{L.sd_nib, L.sd_sc, H, I}
                                  : ExpertView{L.d_nib + (size_t)ut.e * (mat / 2),
                                               L.d_sc + (size_t)ut.e * (mat / kGroup), H, I};
  int roff[kNCT];
  const int seg = tid & 15, srow = tid >> 4;
#pragma unroll
  for (int i = 0; i < kNCT; ++i) roff[i] = (ut.p0 + min(srow + 16 * i, ut.n - 1)) * I + seg * 8;
  f32x4 acc[4][kNCT];
  big_loop<true, false>(glds, dv, dv, rb0, active, ut.shared ? g.hsh : g.hrh,
                        ut.shared ? g.hsl : g.hrl, roff, I / kQuadCols, acc);
  if (active) down_epilogue<4, kNCT>(g, ut, I, row0, q, j, acc);
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

constexpr int kSmallGuCols = 4 * 16;   // features per small gate/up workgroup
constexpr int kSmallDnRows = 4 * 32;   // output rows per small down workgroup

__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(3))) void k_gu_small(
    GroupArgs g) {
  const int ui = g.meta[1] + blockIdx.x;
  if (ui >= g.meta[0]) return;
  const UnitTokens ut = unit_tokens(g.units[ui], g.off, g.L.E, g.T, kSmallMax);
  const LayerDev& L = g.L;
  const int H = L.H, K = L.K, I = ut.shared ? L.Ish : L.I;
  const int w = gwave_id(), lane = threadIdx.x & 63, q = lane >> 4, j = lane & 15;
  const int f0 = blockIdx.y * kSmallGuCols + 16 * w;
  if (f0 >= I) return;  // uniform per wave; no barriers in this kernel
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
  gu_epilogue<kSmallTiles, 1>(g, ut, I, f0, q, j, acc);
}

__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(3))) void k_down_small(
    GroupArgs g) {
  const int ui = g.meta[1] + blockIdx.x;
  if (ui >= g.meta[0]) return;
  const UnitTokens ut = unit_tokens(g.units[ui], g.off, g.L.E, g.T, kSmallMax);
  const LayerDev& L = g.L;
  const int H = L.H, I = ut.shared ? L.Ish : L.I;
  const int w = gwave_id(), lane = threadIdx.x & 63, q = lane >> 4, j = lane & 15;
  const int row0 = blockIdx.y * kSmallDnRows + 32 * w;
  if (row0 >= H) return;
  const size_t mat = (size_t)H * I;
  const ExpertView dv = ut.shared ? ExpertView{L.sd_nib, L.sd_sc, H, I}
                                  : ExpertView{L.d_nib + (size_t)ut.e * (mat / 2),
                                               L.d_sc + (size_t)ut.e * (mat / kGroup), H, I};
  const size_t o = (size_t)(ut.p0 + min(j, ut.n - 1)) * I + 8 * q;
  f32x4 acc[kSmallTiles][1];
  small_loop<true, false, 2>(dv, dv, row0 / kTileRows, (ut.shared ? g.hsh : g.hrh) + o,
                             (ut.shared ? g.hsl : g.hrl) + o, I / kQuadCols, acc);
  down_epilogue<kSmallTiles, 1>(g, ut, I, row0, q, j, acc);
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
  if (big) {
    // I and Ish are multiples of 128 (checked at upload): every block of
    // k_gu_big2 is a whole 128-feature block.  Exactly one of the two
    // kernels does the work, chosen on the device by the need-lo flag.
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(k_gu_big2), hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)kB2Lds);
    if (attr != hipSuccess) return attr;
    const int gsz = big_grid(nbig, (imax + 127) / 128);
    hipLaunchKernelGGL(k_gu_big2, dim3(gsz), dim3(kB2Threads), kB2Lds, st, g);
    hipLaunchKernelGGL(k_gu_big, dim3(gsz), dim3(kGThreads), kBigLds, st, g);
  }
  hipLaunchKernelGGL(k_gu_small, dim3(nsmall, (imax + kSmallGuCols - 1) / kSmallGuCols),
                     dim3(kGThreads), 0, st, g);
  if (big)
    hipLaunchKernelGGL(k_down_big, dim3(big_grid(nbig, (L.H + 255) / 256)), dim3(kGThreads),
                       kBigLds, st, g);
  hipLaunchKernelGGL(k_down_small, dim3(nsmall, (L.H + kSmallDnRows - 1) / kSmallDnRows),
                     dim3(kGThreads), 0, st, g);
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
  const int t = blockIdx.y, d = blockIdx.x * 256 + threadIdx.x;
  // the last kernel of a call clears the call's need-lo flag for the next
  if (clear_flag && t == 0 && d == 0) *clear_flag = 0;
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
                          unsigned long long* status, hipStream_t st, int* clear_flag) {
  hipLaunchKernelGGL(k_combine, dim3((H + 255) / 256, T), dim3(256), 0, st, r, rs, probs, shg,
                     residual, H, K, y, status, clear_flag);
  return hipGetLastError();
}

}  // namespace dm
