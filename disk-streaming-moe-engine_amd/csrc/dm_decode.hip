// dm_decode.hip -- the fused single-launch decode kernel of the MoE block.
//
// One launch computes the whole block for one token (forward_moe_block,
// src/layers/moe_block.mojo:20-138, with the routed experts of
// src/layers/swiglu.mojo:52-230 and the combine of src/layers/moe.mojo:150-175
// / src/layers/forward_layer.mojo:226-238).  The grid is one persistent
// workgroup per CU; the phases hand data to each other through coherent
// counters instead of kernel boundaries:
//
//   P1  router rows (16 per WG, exact 16-lane order)          -> z
//       shared-expert gate/up tiles (independent of routing)  -> h[K], cnt_h[K]
//   P2  every WG: poll z, top-k itself (identical result everywhere, so no
//       broadcast handoff), issue its down-projection loads
//   P3  routed gate/up tile (slot, 16 rows), full reduction in the WG -> h[k]
//   P4  down unit (16 output rows, half of the K+1 slots): dequantise the
//       prefetched weights, wait for h of its slots (meanwhile one wave forms
//       the softmax normaliser), MFMA, partial combine; the unit of half 0
//       adds the partial of half 1 and writes y.
//
// Small hand-offs (logits, half partials) travel as 64-bit (launch tag,
// value) words, so the consumer polls the data itself: one round trip, no
// counter.  The h tiles use per-slot counters polled in parallel.
//
// Top-k runs on e = exp(z - max) before the softmax normaliser S is known:
// p = e * (1/S) is a monotone map, so the (p desc, id asc) order equals the
// (e desc, id asc) order unless rounding merges two distinct e values.  That
// can only happen when the k-th and (k+1)-th e are within a few ulp; then
// the kernel forms S first and selects on the exact p (rare slow path).
//
// Counters only grow and tags are the launch index, so launch n of a layer
// waits for n * (arrivals per launch) or tag n: nothing is reset between
// launches.  Every wait is bounded.
#include <hip/hip_runtime.h>

#include "dm_decode.h"
#include "dm_device.h"

namespace dm {

constexpr int kDownBatch = 8;   // routed down chunks per wave held in registers
constexpr int kShBatch = 1;     // shared-expert down chunks per wave held in registers
constexpr int kPollItems = 2;   // h items (8 values) per thread per poll batch
constexpr int kSelRMax = 8;     // top-k: lane owns e = 256 r + 4 lane + i, r < R <= 8

// Gate/up of one 16-row tile: h = SiLU(W_g x) * (W_u x) for rows 16rb..+15,
// reduced over all H columns inside the workgroup (wave w owns the 128-column
// chunks w, w+4, ...).  gu_load issues the tile's loads; gu_compute consumes
// them and stores the 16 h values as (tag, value) words to hdst[row].
template <int GQW>
__device__ __forceinline__ void gu_load(const ExpertView& gv, const ExpertView& uv, int rb,
                                        uint4 (&wg)[GQW], uint4 (&wu)[GQW], uint2 (&sg)[GQW],
                                        uint2 (&su)[GQW]) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nGQ = gv.cols / kQuadCols;
#pragma unroll
  for (int i = 0; i < GQW; ++i) {
    const int gq = w + 4 * i;
    if (gq < nGQ) {
      load_chunk(gv, rb, gq, lane, wg[i], sg[i]);
      load_chunk(uv, rb, gq, lane, wu[i], su[i]);
    }
  }
}

template <int GQW>
__device__ __forceinline__ void gu_compute(const ExpertView& gv, int rb, const uint4 (&wg)[GQW],
                                           const uint4 (&wu)[GQW], const uint2 (&sg)[GQW],
                                           const uint2 (&su)[GQW], const uint4* xb, float* red,
                                           uint64_t* hdst, unsigned tag, uint32_t phase,
                                           uint32_t token, uint32_t slot,
                                           unsigned long long* status) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15, jsel = j < 2 ? j : 2;
  const int nGQ = gv.cols / kQuadCols;
  f32x4 ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < GQW; ++i) {
    const int gq = w + 4 * i;
    if (gq < nGQ) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int g = gq * 4 + c;
        const bf16x8 b = __builtin_bit_cast(bf16x8, xb[(g * 4 + q) * 3 + jsel]);
        ag = mfma16(dequant8(word_of(wg[i], c), scale_of(sg[i], c)), b, ag);
        au = mfma16(dequant8(word_of(wu[i], c), scale_of(su[i], c)), b, au);
      }
    }
  }
  fold_cols(ag);
  fold_cols(au);
  if (j == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[(w * 2 + 0) * 16 + 4 * q + i] = ag[i];
      red[(w * 2 + 1) * 16 + 4 * q + i] = au[i];
    }
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int r = threadIdx.x, row = rb * kTileRows + r;
    const float g = ((red[0 * 32 + r] + red[1 * 32 + r]) + red[2 * 32 + r]) + red[3 * 32 + r];
    const float u = ((red[0 * 32 + 16 + r] + red[1 * 32 + 16 + r]) + red[2 * 32 + 16 + r]) +
                    red[3 * 32 + 16 + r];
    if (!finite_f(g)) record_err(status, err_key(phase, token, slot, row, kEkGate));
    if (!finite_f(u)) record_err(status, err_key(phase, token, slot, row, kEkUp));
    const float h = dm_silu(g) * u;
    if (!finite_f(h)) record_err(status, err_key(phase, token, slot, row, kEkH));
    st_coh_u64(hdst + row, ((uint64_t)tag << 32) | f2u(h));
  }
  __syncthreads();
}

// Router row e (row E = shared-expert gate), lane chain l = threadIdx & 15:
// sequential chain over the preloaded R16 chunk wv, halving tree over the 16
// chains, (tag, logit) stored to zt[e].  xs = fp32 x in LDS.
template <int NJ8>
__device__ __forceinline__ void router_compute(const LayerDev& L, const uint4 (&wv)[NJ8], int e,
                                               const float* xs, uint64_t* zt, unsigned tag) {
  const int l = threadIdx.x & 15;
  const int nj8 = L.H / 128;
  float acc = 0.0f;
  if (e <= L.E) {
#pragma unroll
    for (int j8 = 0; j8 < NJ8; ++j8) {
      if (j8 < nj8) {
        const uint32_t ww[4] = {wv[j8].x, wv[j8].y, wv[j8].z, wv[j8].w};
        const float* xc = xs + j8 * 128 + l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc = acc + xc[(2 * i) * 16] * bf16lo(ww[i]);
          acc = acc + xc[(2 * i + 1) * 16] * bf16hi(ww[i]);
        }
      }
    }
  }
#pragma unroll
  for (int wdt = 8; wdt >= 1; wdt >>= 1) acc = acc + __shfl_down(acc, wdt, 16);
  if (l == 0 && e <= L.E) st_coh_u64(zt + e, ((uint64_t)tag << 32) | f2u(acc));
}

// Shared LDS state of the routing decision.
struct SelState {
  float* ev;     // [E] e = exp(z - max)
  int* ids;      // [K] selected experts, (e desc, id asc) = slot order
  float* eval;   // [K] their e
  float* p;      // [K] their probabilities (after the normaliser)
  int* order;    // [K] slots in (p desc, id asc) order
  float* g;      // [1] shared-expert gate
  float* inv;    // [1] 1 / S
  int* exact;    // [1] 1 when the selection was made on p (S already known)
};

// One K-round selection on keys (key > 0 valid), lowest id on equal keys.
// Returns (key of the K-th selected, best unselected key).
struct KeyPair {
  uint32_t kth, next;
};
template <int R>
__device__ __forceinline__ KeyPair select_rounds(uint32_t (&key)[R][4], int K, int E, int* ids_out) {
  const int lane = threadIdx.x & 63;
  uint32_t taken[R];
#pragma unroll
  for (int r = 0; r < R; ++r) taken[r] = 0;
  uint32_t kth = 0, next = 0;
  for (int it = 0; it <= K; ++it) {
    uint32_t lmax = 0;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!(taken[r] >> i & 1u) && key[r][i] > lmax) lmax = key[r][i];
    const uint32_t gmax = wave_max_u32(lmax);
    if (it == K) {  // the best unselected key
      next = gmax;
      break;
    }
    uint32_t lid = 0xFFFFFFFFu;
#pragma unroll
    for (int r = R - 1; r >= 0; --r)
#pragma unroll
      for (int i = 3; i >= 0; --i)
        if (!(taken[r] >> i & 1u) && key[r][i] == gmax) lid = 256 * r + 4 * lane + i;
    uint32_t gid = wave_min_u32(lid);
    if (gid >= (uint32_t)E) gid = 0;  // only after a recorded error
    if (((gid >> 2) & 63) == (uint32_t)lane) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if ((uint32_t)r == (gid >> 8)) taken[r] |= 1u << (gid & 3);
    }
    if (lane == 0) ids_out[it] = (int)gid;
    kth = gmax;
  }
  return {kth, next};
}

// Top-k of src/layers/topk.mojo:79-128 over the softmax of
// src/layers/router.mojo:140-183, on wave 0.  Polls the tagged logits until
// every entry carries this launch's tag.  Identical in every workgroup; only
// `record` workgroups write error keys.  Returns false on a poll timeout.
template <int R>
__device__ __forceinline__ bool route(const uint64_t* zt, unsigned tag, int E, int K, SelState& st,
                                      bool record, int token, unsigned long long* status) {
  if (threadIdx.x >= 64) return true;
  const int lane = threadIdx.x;
  float zv[R][4];
  float gl = 0.0f;
  bool ok = false;
  for (long spin = 0; spin < kSpinLimit; ++spin) {
    bool ready = true;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 256 * r + 4 * lane + i;
        const uint64_t v = ld_coh_u64(zt + e);
        zv[r][i] = u2f((uint32_t)v);
        if (e < E && (uint32_t)(v >> 32) != tag) ready = false;
      }
    if (lane == 0) {
      const uint64_t v = ld_coh_u64(zt + E);
      gl = u2f((uint32_t)v);
      if ((uint32_t)(v >> 32) != tag) ready = false;
    }
    if (__builtin_amdgcn_ballot_w64(!ready) == 0) {
      ok = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (!ok && lane == 0) record_err(status, err_key(kPhSync, 0, 0, 0, 0));
  // max (exact in any order)
  uint32_t lm = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 256 * r + 4 * lane + i;
      if (e < E) {
        if (record && !finite_f(zv[r][i])) record_err(status, err_key(kPhLogit, token, 0, e, 0));
        const uint32_t k = f2key(zv[r][i]);
        lm = k > lm ? k : lm;
      }
    }
  const float m = key2f(wave_max_u32(lm));
  if (record && lane == 0 && !finite_f(m)) record_err(status, err_key(kPhSoftmax, token, 0, 0, 0));
  uint32_t key[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      key[r][i] = 0;
      const int e = 256 * r + 4 * lane + i;
      if (e < E) {
        const float ev = dm_expf(zv[r][i] - m);
        if (record && !finite_f(ev)) record_err(status, err_key(kPhSoftmax, token, 0, 1 + e, 0));
        st.ev[e] = ev;
        key[r][i] = f2u(ev) + 1u;
      }
    }
  KeyPair kp = select_rounds<R>(key, K, E, st.ids);
  // exactness guard: e_k and e_(k+1) within a few ulp -> select on exact p
  const float ek = u2f(kp.kth - 1u);
  const float en = kp.next ? u2f(kp.next - 1u) : 0.0f;
  const bool unsafe = K < E && ek > en && ek <= en + en * 0x1p-20f;
  if (lane == 0) *st.exact = unsafe;
  if (unsafe) {
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    float inv = 0.0f;
    if (lane == 0) {
      float s = 0.0f;
      for (int e = 0; e < E; ++e) s = s + st.ev[e];
      inv = 1.0f / s;
    }
    inv = __shfl(inv, 0);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (key[r][i]) key[r][i] = f2u(u2f(key[r][i] - 1u) * inv) + 1u;
    select_rounds<R>(key, K, E, st.ids);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  if (lane < K) st.eval[lane] = st.ev[st.ids[lane]];
  if (lane == 0) {
    if (record && !finite_f(gl)) record_err(status, err_key(kPhGate, token, 0, 0, kGkLogit));
    const float sg = dm_sigmoid(gl);
    if (record && (!finite_f(sg) || sg < 0.0f || sg > 1.0f))
      record_err(status, err_key(kPhGate, token, 0, 0, kGkRange));
    *st.g = sg;
  }
  return ok;
}

// The softmax normaliser (sequential over e, src/layers/router.mojo:160-170),
// the K probabilities and the checks of src/layers/topk.mojo:109-128, run by
// lane 0 of the calling wave; `outputs` additionally writes ids / probs in
// (p desc, id asc) order.
__device__ __forceinline__ void finish_probs(int E, int K, SelState& st, bool record, int token,
                                             unsigned long long* status, int32_t* ids_out,
                                             float* probs_out, float* shg_out) {
  if ((threadIdx.x & 63) != 0) return;
  float s = 0.0f;
  for (int e = 0; e < E; ++e) s = s + st.ev[e];
  if (record && (!(s > 0.0f) || !finite_f(s)))
    record_err(status, err_key(kPhSoftmax, token, 0, 1 + E, 0));
  const float inv = 1.0f / s;
  *st.inv = inv;
  float sum_topk = 0.0f;
  int* order = st.order;
  for (int k = 0; k < K; ++k) {
    st.p[k] = st.eval[k] * inv;
    order[k] = k;
  }
  // (p desc, id asc); equal p can only come from near-equal e in slot order
  for (int a = 1; a < K; ++a) {
    const int v = order[a];
    int b = a - 1;
    while (b >= 0 && (st.p[order[b]] < st.p[v] ||
                      (st.p[order[b]] == st.p[v] && st.ids[order[b]] > st.ids[v]))) {
      order[b + 1] = order[b];
      --b;
    }
    order[b + 1] = v;
  }
  for (int k = 0; k < K; ++k) sum_topk = sum_topk + st.p[order[k]];
  if (record) {
    if (sum_topk > 1.00001f) record_err(status, err_key(kPhTopk, token, 0, 0, kTkSum));
    if (K < E && __builtin_fabsf(sum_topk - 1.0f) < 1e-6f) {
      float sum_all = 0.0f;
      for (int e = 0; e < E; ++e) sum_all = sum_all + st.ev[e] * inv;
      if (sum_all - sum_topk > 1e-5f) record_err(status, err_key(kPhTopk, token, 0, 0, kTkLeak));
    }
  }
  if (ids_out) {
    for (int k = 0; k < K; ++k) {
      ids_out[k] = st.ids[order[k]];
      probs_out[k] = st.p[order[k]];
    }
    shg_out[0] = *st.g;
  }
}

template <int GQW, int R>
__global__ __launch_bounds__(256) void k_moe_decode(LayerDev L, DecodePlan P, const float* __restrict__ x,
                                                     const float* __restrict__ residual,
                                                     float* __restrict__ y, int32_t* __restrict__ ids_out,
                                                     float* __restrict__ probs_out,
                                                     float* __restrict__ shg_out, DecodeSync S,
                                                     unsigned long long* status, int token) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* xs = reinterpret_cast<float*>(smem + P.off_xs);
  uint4* xb = reinterpret_cast<uint4*>(smem + P.off_xb);
  float* red = reinterpret_cast<float*>(smem + P.off_red);
  uint4* hb = reinterpret_cast<uint4*>(smem + P.off_hb);
  float* redd = reinterpret_cast<float*>(smem + P.off_redd);
  unsigned char* sel = smem + P.off_sel;
  SelState st{reinterpret_cast<float*>(smem + P.off_pv), reinterpret_cast<int*>(sel),
              reinterpret_cast<float*>(sel + 256), reinterpret_cast<float*>(sel + 512),
              reinterpret_cast<int*>(sel + 768),   reinterpret_cast<float*>(sel + 1024),
              reinterpret_cast<float*>(sel + 1028), reinterpret_cast<int*>(sel + 1032)};
  int* flag = reinterpret_cast<int*>(sel + 1036);

  const int H = L.H, K = L.K, E = L.E;
  const int b = blockIdx.x, nb = gridDim.x;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15, jsel = j < 2 ? j : 2;
  const unsigned n = S.n;
  const int nrbo = H / kTileRows;
  const bool down_wg = b < nrbo;     // one 16-row output tile per WG, all K+1 slots
  const int nsh = L.Ish / kTileRows;  // shared-expert gate/up tiles
  const int sh_tile = (b + nb - P.n_router_wg % nb) % nb;
  const int nGQI = L.I / kQuadCols, nGQS = L.Ish / kQuadCols;

  // ---- entry: issue every load that does not depend on x or on routing -----
  uint4 rw[4 * GQW];  // router row chunk (R16 layout)
  const bool router_wg = b < P.n_router_wg;
  const int re = b * 16 + (threadIdx.x >> 4);
  if (router_wg && re <= E) {
    const uint4* wp = reinterpret_cast<const uint4*>(L.router + r16_index(H, re, threadIdx.x & 15));
#pragma unroll
    for (int j8 = 0; j8 < 4 * GQW; ++j8)
      if (j8 < H / 128) rw[j8] = wp[(size_t)j8 * 16];
  }
  const size_t matS = (size_t)L.Ish * H;
  const ExpertView sgv = {L.sgu_nib, L.sgu_sc, L.Ish, H};
  const ExpertView suv = {L.sgu_nib + matS / 2, L.sgu_sc + matS / kGroup, L.Ish, H};
  uint4 swg[GQW], swu[GQW];
  uint2 ssg[GQW], ssu[GQW];
  if (sh_tile < nsh) gu_load<GQW>(sgv, suv, sh_tile, swg, swu, ssg, ssu);
  const ExpertView sdv = {L.sd_nib, L.sd_sc, H, L.Ish};
  uint4 sdw[kShBatch];
  uint2 sds[kShBatch];
  const int my_sh = down_wg ? (nGQS - w + 3) / 4 : 0;
#pragma unroll
  for (int i = 0; i < kShBatch; ++i)
    if (i < my_sh) load_chunk(sdv, b, w + 4 * i, lane, sdw[i], sds[i]);

  // ---- stage x: fp32 copy (router chains) and bf16 hi/lo B blocks ----------
  {
    bool bad = false;
    for (int i = threadIdx.x; i < H / 8; i += 256) {
      const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
      const float4 c = reinterpret_cast<const float4*>(x)[2 * i + 1];
      const float f[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
      for (int k2 = 0; k2 < 8; ++k2) {
        bad |= !finite_f(f[k2]);
        xs[8 * i + k2] = f[k2];
      }
      uint4 hi, lo;
      split8(f, hi, lo);
      xb[3 * i + 0] = hi;
      xb[3 * i + 1] = lo;
      xb[3 * i + 2] = make_uint4(0, 0, 0, 0);
    }
    if (bad && b == 0) record_err(status, err_key(kPhX, 0, 0, 0, 0));
  }
  __syncthreads();

  // ---- P1: router rows; shared-expert gate/up tile --------------------------
  if (router_wg) router_compute<4 * GQW>(L, rw, re, xs, S.zt, n);
  for (int rr = b + nb; rr < P.n_router_wg; rr += nb) {  // only when the grid is small
    const int e2 = rr * 16 + (threadIdx.x >> 4);
    if (e2 <= E) {
      const uint4* wp = reinterpret_cast<const uint4*>(L.router + r16_index(H, e2, threadIdx.x & 15));
#pragma unroll
      for (int j8 = 0; j8 < 4 * GQW; ++j8)
        if (j8 < H / 128) rw[j8] = wp[(size_t)j8 * 16];
    }
    router_compute<4 * GQW>(L, rw, e2, xs, S.zt, n);
  }
  for (int t = sh_tile; t < nsh; t += nb) {
    if (t != sh_tile) gu_load<GQW>(sgv, suv, t, swg, swu, ssg, ssu);
    gu_compute<GQW>(sgv, t, swg, swu, ssg, ssu, xb, red, S.ht + (size_t)K * P.ldh, n, kPhShared,
                    token, 0, status);
  }

  // ---- P2: routing (every WG computes the same top-k) -----------------------
  if (threadIdx.x < 64) {
    const bool rok = route<R>(S.zt, n, E, K, st, b == 0, token, status);
    if (threadIdx.x == 0) flag[0] = rok;
  }
  __syncthreads();
  bool ok = flag[0];

  // ---- P3: routed gate/up tile; routed down chunks of this WG's output tile --
  const int nrb = L.I / kTileRows;
  const size_t matI = (size_t)L.I * H;
  auto gu_views = [&](int t, ExpertView& gv, ExpertView& uv) {
    int e = st.ids[t / nrb];
    if (e < 0 || e >= E) e = 0;
    gv = {L.gu_nib + (size_t)e * matI, L.gu_sc + (size_t)e * 2 * (matI / kGroup), L.I, H};
    uv = {gv.nib + matI / 2, gv.sc + matI / kGroup, L.I, H};
  };
  uint4 gwg[GQW], gwu[GQW];
  uint2 gsg[GQW], gsu[GQW];
  ExpertView gv, uv;
  if (b < K * nrb) {
    gu_views(b, gv, uv);
    gu_load<GQW>(gv, uv, b % nrb, gwg, gwu, gsg, gsu);
  }
  auto down_view = [&](int s) -> ExpertView {
    int e = st.ids[s];
    if (e < 0 || e >= E) e = 0;
    const size_t mat = (size_t)H * L.I;
    return {L.d_nib + (size_t)e * (mat / 2), L.d_sc + (size_t)e * (mat / kGroup), H, L.I};
  };
  const int nchunk = K * nGQI;  // routed down chunks of the tile: c -> (slot c / nGQI, gq c % nGQI)
  const int my_chunks = down_wg ? (nchunk - w + 3) / 4 : 0;
  uint4 dw[kDownBatch];
  uint2 ds[kDownBatch];
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i)
    if (i < my_chunks) {
      const int c = w + 4 * i;
      load_chunk(down_view(c / nGQI), b, c % nGQI, lane, dw[i], ds[i]);
    }
  if (w == 1 && down_wg)  // softmax normaliser while the loads are in flight
    finish_probs(E, K, st, b == 0, token, status, b == 0 ? ids_out : nullptr, probs_out, shg_out);
  for (int t = b; t < K * nrb; t += nb) {
    if (t != b) {
      gu_views(t, gv, uv);
      gu_load<GQW>(gv, uv, t % nrb, gwg, gwu, gsg, gsu);
    }
    const int k = t / nrb;
    gu_compute<GQW>(gv, t % nrb, gwg, gwu, gsg, gsu, xb, red, S.ht + (size_t)k * P.ldh, n,
                    kPhExpert, token, k, status);
  }
  if (!down_wg) return;

  // ---- P4: down projection of the 16 output rows of this WG, all slots -------
  bf16x8 A[kDownBatch][4];
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i)
    if (i < my_chunks)
#pragma unroll
      for (int c = 0; c < 4; ++c) A[i][c] = dequant8(word_of(dw[i], c), scale_of(ds[i], c));
  bf16x8 As[kShBatch][4];
#pragma unroll
  for (int i = 0; i < kShBatch; ++i)
    if (i < my_sh)
#pragma unroll
      for (int c = 0; c < 4; ++c) As[i][c] = dequant8(word_of(sdw[i], c), scale_of(sds[i], c));
  // poll the tagged h of all slots until every value carries this launch's
  // tag, then stage it as B blocks
  const int nblk_slot = (P.ldh / 8) * 3;
  const int items_r = K * (L.I / 8), items = items_r + L.Ish / 8;
  {
    bool done = false;
    for (long spin = 0; spin < kSpinLimit; ++spin) {
      bool mine = true;
      for (int base = threadIdx.x; base < items; base += 256 * kPollItems) {
        uint64_t v[kPollItems][8];
#pragma unroll
        for (int bi = 0; bi < kPollItems; ++bi) {  // all loads of the batch first
          const int it = base + 256 * bi;
          if (it < items) {
            const int s = it < items_r ? it / (L.I / 8) : K;
            const int ii = it < items_r ? it % (L.I / 8) : it - items_r;
            const uint64_t* src = S.ht + (size_t)s * P.ldh + 8 * ii;
#pragma unroll
            for (int k2 = 0; k2 < 8; ++k2) v[bi][k2] = ld_coh_u64(src + k2);
          }
        }
#pragma unroll
        for (int bi = 0; bi < kPollItems; ++bi) {
          const int it = base + 256 * bi;
          if (it < items) {
            const int s = it < items_r ? it / (L.I / 8) : K;
            const int ii = it < items_r ? it % (L.I / 8) : it - items_r;
            float f[8];
#pragma unroll
            for (int k2 = 0; k2 < 8; ++k2) {
              mine &= (uint32_t)(v[bi][k2] >> 32) == n;
              f[k2] = u2f((uint32_t)v[bi][k2]);
            }
            uint4 hi, lo;
            split8(f, hi, lo);
            uint4* dst = hb + (size_t)s * nblk_slot + 3 * ii;
            dst[0] = hi;
            dst[1] = lo;
            dst[2] = make_uint4(0, 0, 0, 0);
          }
        }
      }
      if (__syncthreads_and(mine || !ok)) {
        done = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!done && threadIdx.x == 0) record_err(status, err_key(kPhSync, 0, 0, 0, 0));
  }
  // MFMA: chunk partials to LDS redd[slot][gq][16]
  for (int base = 0; base < my_chunks; base += kDownBatch) {
    if (base > 0) {  // chunks beyond the register batch
#pragma unroll
      for (int i = 0; i < kDownBatch; ++i)
        if (base + i < my_chunks) {
          const int c = w + 4 * (base + i);
          load_chunk(down_view(c / nGQI), b, c % nGQI, lane, dw[i], ds[i]);
        }
#pragma unroll
      for (int i = 0; i < kDownBatch; ++i)
        if (base + i < my_chunks)
#pragma unroll
          for (int c = 0; c < 4; ++c) A[i][c] = dequant8(word_of(dw[i], c), scale_of(ds[i], c));
    }
#pragma unroll
    for (int i = 0; i < kDownBatch; ++i) {
      if (base + i < my_chunks) {
        const int c = w + 4 * (base + i);
        const int s = c / nGQI, gq = c % nGQI;
        const uint4* hbs = hb + (size_t)s * nblk_slot;
        f32x4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
          acc = mfma16(A[i][cc], __builtin_bit_cast(bf16x8, hbs[((gq * 4 + cc) * 4 + q) * 3 + jsel]), acc);
        fold_cols(acc);
        if (j == 0) {
#pragma unroll
          for (int r = 0; r < 4; ++r) redd[c * 16 + 4 * q + r] = acc[r];
        }
      }
    }
  }
  for (int i = 0; i < (my_sh + kShBatch - 1) / kShBatch * kShBatch; i += kShBatch) {
    if (i > 0) {
#pragma unroll
      for (int i2 = 0; i2 < kShBatch; ++i2)
        if (i + i2 < my_sh) {
          load_chunk(sdv, b, w + 4 * (i + i2), lane, sdw[i2], sds[i2]);
#pragma unroll
          for (int c = 0; c < 4; ++c) As[i2][c] = dequant8(word_of(sdw[i2], c), scale_of(sds[i2], c));
        }
    }
#pragma unroll
    for (int i2 = 0; i2 < kShBatch; ++i2) {
      if (i + i2 < my_sh) {
        const int gq = w + 4 * (i + i2);
        const uint4* hbs = hb + (size_t)K * nblk_slot;
        f32x4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
          acc = mfma16(As[i2][cc], __builtin_bit_cast(bf16x8, hbs[((gq * 4 + cc) * 4 + q) * 3 + jsel]), acc);
        fold_cols(acc);
        if (j == 0) {
#pragma unroll
          for (int r = 0; r < 4; ++r) redd[(nchunk + gq) * 16 + 4 * q + r] = acc[r];
        }
      }
    }
  }
  __syncthreads();
  // combine in the reference order: routed experts in routing order, then the
  // shared expert, then the residual (src/layers/moe.mojo:157-166)
  if (threadIdx.x < 16) {
    const int r = threadIdx.x, d = b * kTileRows + r;
    float rs = 0.0f;
    for (int k = 0; k < K; ++k) {
      const int s = st.order[k];
      float v = 0.0f;
      for (int g = 0; g < nGQI; ++g) v = v + redd[(s * nGQI + g) * 16 + r];
      if (!finite_f(v)) record_err(status, err_key(kPhExpert, token, s, P.ldh + d, kEkDown));
      rs = rs + st.p[s] * v;
    }
    float vsh = 0.0f;
    for (int g = 0; g < nGQS; ++g) vsh = vsh + redd[(nchunk + g) * 16 + r];
    if (!finite_f(vsh)) record_err(status, err_key(kPhShared, token, 0, P.ldh + d, kEkDown));
    float total = rs + *st.g * vsh;
    if (residual) total = total + residual[d];
    if (!finite_f(total)) record_err(status, err_key(kPhAgg, token, 0, d, 0));
    y[d] = total;
  }
}

static int align16(int v) { return (v + 15) & ~15; }
static size_t align256z(size_t v) { return (v + 255) & ~(size_t)255; }

size_t decode_sync_bytes(const LayerDev& L) {
  const int ldh = L.I > L.Ish ? L.I : L.Ish;
  const size_t R = (size_t)(L.E + 255) / 256;
  return align256z((256 * R + 64) * 8) + align256z((size_t)(L.K + 1) * ldh * 8);
}

DecodeSync decode_sync_carve(const LayerDev& L, void* base) {
  const size_t R = (size_t)(L.E + 255) / 256;
  unsigned char* p = (unsigned char*)base;
  DecodeSync S{};
  S.zt = (uint64_t*)p; p += align256z((256 * R + 64) * 8);
  S.ht = (uint64_t*)p;
  return S;
}

DecodePlan make_decode_plan(const LayerDev& L, int num_cus) {
  DecodePlan P{};
  P.ldh = L.I > L.Ish ? L.I : L.Ish;
  P.n_router_wg = (L.E + 1 + 15) / 16;
  P.s0 = (L.K + 2) / 2;
  int nch0 = 0, nch1 = 0;
  for (int s = 0; s <= L.K; ++s) {
    const int ng = (s < L.K ? L.I : L.Ish) / kQuadCols;
    (s < P.s0 ? nch0 : nch1) += ng;
  }
  (void)nch0;
  (void)nch1;
  const int nch = L.K * (L.I / kQuadCols) + L.Ish / kQuadCols;
  const int slots = L.K + 1;
  int off = 0;
  P.off_xs = off; off += align16(4 * L.H);
  P.off_xb = off; off += align16(6 * L.H);
  P.off_pv = off; off += align16(4 * (L.E + 2));
  P.off_sel = off; off += 1056;
  P.off_red = off; off += 512;
  P.off_hb = off; off += align16(slots * (P.ldh / 8) * 3 * 16);
  P.off_redd = off; off += align16(nch * 64);
  P.lds_bytes = off;
  P.grid = num_cus > L.H / kTileRows ? num_cus : L.H / kTileRows;
  return P;
}

template <int GQW>
static const void* pick_r(int R) {
  return R <= 1 ? (const void*)k_moe_decode<GQW, 1> : R <= 2 ? (const void*)k_moe_decode<GQW, 2>
       : R <= 4 ? (const void*)k_moe_decode<GQW, 4> : (const void*)k_moe_decode<GQW, 8>;
}

static const void* pick_kernel(const LayerDev& L) {
  const int gqw = (L.H / kQuadCols + 3) / 4;
  const int R = (L.E + 255) / 256;
  if (R > kSelRMax) return nullptr;
  return gqw <= 1 ? pick_r<1>(R) : gqw <= 2 ? pick_r<2>(R) : gqw <= 4 ? pick_r<4>(R)
       : gqw <= 8 ? pick_r<8>(R) : gqw <= 16 ? pick_r<16>(R) : nullptr;
}

hipError_t decode_occupancy(const LayerDev& L, const DecodePlan& P, int* blocks_per_cu) {
  const void* fn = pick_kernel(L);
  if (!fn) return hipErrorInvalidValue;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, 256, P.lds_bytes);
}

hipError_t launch_moe_decode(const LayerDev& L, const DecodePlan& P, const float* x,
                             const float* residual, float* y, int32_t* ids, float* probs,
                             float* shg, const DecodeSync& S, unsigned long long* status, int token,
                             hipStream_t st) {
  const void* fn = pick_kernel(L);
  if (!fn) return hipErrorInvalidValue;
  LayerDev Lc = L;
  DecodePlan Pc = P;
  DecodeSync Sc = S;
  const float* xc = x;
  const float* rc = residual;
  void* args[] = {&Lc, &Pc, &xc, &rc, &y, &ids, &probs, &shg, &Sc, &status, &token};
  return hipLaunchKernel(fn, dim3(P.grid), dim3(256), args, P.lds_bytes, st);
}

}  // namespace dm
