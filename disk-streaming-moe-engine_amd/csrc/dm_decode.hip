// dm_decode.hip -- the fused single-launch decode kernel of the MoE block.
//
// One launch computes the whole block for one token (forward_moe_block,
// src/layers/moe_block.mojo:20-138, with the routed experts of
// src/layers/swiglu.mojo:52-230 and the combine of src/layers/moe.mojo:150-175
// / src/layers/forward_layer.mojo:226-238).  The grid is one persistent
// 512-thread workgroup (8 waves, two per SIMD) per CU; phases hand data to
// each other through tagged words in global memory instead of kernel
// boundaries:
//
//   entry  every workgroup issues the loads that do not depend on x or on
//          routing: router rows, a shared-expert gate/up tile, shared-expert
//          down chunks.
//   P1     router rows (16 per router workgroup, the exact 16-lane order of
//          router_project) -> z;  shared-expert gate/up tile -> h[K].
//   P2     every workgroup polls z and selects the top-k itself (identical
//          everywhere, so no broadcast hand-off), then issues its routed
//          gate/up and down loads.  One wave forms the softmax normaliser and
//          the probabilities while the loads are in flight.
//   P3     routed gate/up tile (slot, 16 rows) -> h[k].
//   P4     down tile (16 output rows, all K+1 slots): poll h, scale each slot
//          by its weight (p_k, or the shared gate), one MFMA chain per wave,
//          residual, y.
//
// Hand-offs are 64-bit (launch tag, value) words: the consumer polls the data
// itself (one round trip, no counters, nothing reset between launches).
// Every wait is bounded; a timeout records an error and skips later waits so
// the grid always drains.
//
// Top-k is selected on the logits z: e = exp(z - max) and p = e * (1/S) are
// monotone in z, so the top-k set on z equals the set on p unless the k-th
// and (k+1)-th values merge under rounding.  The kernel checks the margin
// e_k > e_(k+1) (1 + 2^-20), which keeps p_k > p_(k+1) strict; otherwise it
// forms S first and selects on the exact p with the lowest-id tie-break
// (rare slow path).  The order inside the selected set is always decided on
// p (descending, lowest id first), as select_topk does (src/layers/topk.mojo:79-128).
#include <hip/hip_runtime.h>

#include "dm_decode.h"
#include "dm_device.h"

namespace dm {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kRouterRows = 16;      // router rows per router workgroup (waves 0..3)
constexpr int kRwMax = 16;           // router chain chunks (8 bf16 each) held per lane
constexpr int kDownBatch = 5;        // down chunks per wave held in registers
constexpr int kPollItems = 2;        // h items (8 values) per thread per poll pass
constexpr int kProbWave = kWaves - 1;

// LDS state of the routing decision.
struct SelState {
  float* zv;    // [256R] logits
  float* ev;    // [256R] e = exp(z - max)
  int* ids;     // [32] selected experts, slot order
  int* rank;    // [32] position of each slot in the (p desc, id asc) order
  float* pw;    // [33] B-operand weight of slot s: p_s; slot K: the shared gate
  float* misc;  // [0] shared gate, [1] max logit, [2] ok flag
  float* p;     // [32] probabilities by slot
  int* order;   // [32] slots in (p desc, id asc) order
};

// B operand of a 16x16x32 MFMA from split blocks blk2[2*b + {hi, lo}]:
// lane (q, j) holds rows 8q..8q+7 of column j; columns 0/1 carry hi/lo, the
// others are zero.
__device__ __forceinline__ bf16x8 ld_b(const uint4* blk2, int blk, int j) {
  uint4 v = blk2[2 * blk + (j & 1)];
  if (j >= 2) v = make_uint4(0, 0, 0, 0);
  return __builtin_bit_cast(bf16x8, v);
}

// ---------------------------------------------------------------------------
// Gate/up of one 16-row tile: h = SiLU(W_g x) * (W_u x) for rows 16rb..+15,
// reduced over all H columns inside the workgroup (wave w owns the 128-column
// chunks w, w+8, ...).  gu_load issues the loads; gu_compute consumes them and
// stores the 16 h values as (tag, value) words to hdst[row].
template <int GQW>
__device__ __forceinline__ void gu_load(const ExpertView& gv, const ExpertView& uv, int rb,
                                        uint4 (&wg)[GQW], uint4 (&wu)[GQW], uint2 (&sg)[GQW],
                                        uint2 (&su)[GQW]) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nGQ = gv.cols / kQuadCols;
#pragma unroll
  for (int i = 0; i < GQW; ++i) {
    const int gq = w + kWaves * i;
    if (gq < nGQ) {
      load_chunk(gv, rb, gq, lane, wg[i], sg[i]);
      load_chunk(uv, rb, gq, lane, wu[i], su[i]);
    }
  }
}

template <int GQW>
__device__ __forceinline__ void gu_compute(const ExpertView& gv, int rb, const uint4 (&wg)[GQW],
                                           const uint4 (&wu)[GQW], const uint2 (&sg)[GQW],
                                           const uint2 (&su)[GQW], const uint4* xb2, float* red,
                                           uint64_t* hdst, unsigned tag, uint32_t phase,
                                           uint32_t token, int slot, const int* rank,
                                           unsigned long long* status) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15;
  const int nGQ = gv.cols / kQuadCols;
  f32x4 ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < GQW; ++i) {
    const int gq = w + kWaves * i;
    if (gq < nGQ) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const bf16x8 b = ld_b(xb2, (gq * 4 + c) * 4 + q, j);
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
    // error keys name the slot by its position in the reference's order
    const uint32_t sl = rank ? (uint32_t)rank[slot] : (uint32_t)slot;
    float g = 0.0f, u = 0.0f;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
      g = g + red[v * 32 + r];
      u = u + red[v * 32 + 16 + r];
    }
    if (!finite_f(g)) record_err(status, err_key(phase, token, sl, row, kEkGate));
    if (!finite_f(u)) record_err(status, err_key(phase, token, sl, row, kEkUp));
    const float h = dm_silu(g) * u;
    if (!finite_f(h)) record_err(status, err_key(phase, token, sl, row, kEkH));
    st_coh_u64(hdst + row, ((uint64_t)tag << 32) | f2u(h));
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Router row e (row E = shared-expert gate), lane chain l = threadIdx & 15:
// the sequential chain k = l, l+16, ... (router_project,
// src/layers/router.mojo:84-96) over the R16 chunks rw (first kRwMax
// preloaded, the rest loaded here), the halving tree over the 16 chains, and
// the (tag, logit) word stored to zt[e].  xt = x transposed: xt[l*xts + j] =
// x[16j + l], row stride xts = H/16 + 4 floats.
__device__ __forceinline__ void router_compute(const LayerDev& L, uint4 (&rw)[kRwMax], int e,
                                               const float* xt, uint64_t* zt, unsigned tag) {
  const int l = threadIdx.x & 15;
  const int nj8 = L.H / 128;
  const float4* xr = reinterpret_cast<const float4*>(xt + l * (L.H / 16 + 4));
  float acc = 0.0f;
  if (e <= L.E) {
    const uint4* wp = reinterpret_cast<const uint4*>(L.router + r16_index(L.H, e, l));
    for (int base = 0; base < nj8; base += kRwMax) {
      if (base > 0) {
#pragma unroll
        for (int j8 = 0; j8 < kRwMax; ++j8)
          if (base + j8 < nj8) rw[j8] = wp[(size_t)(base + j8) * 16];
      }
#pragma unroll
      for (int j8 = 0; j8 < kRwMax; ++j8) {
        if (base + j8 < nj8) {
          const float4 xa = xr[2 * (base + j8)], xc = xr[2 * (base + j8) + 1];
          const uint4 ww = rw[j8];
          acc = acc + xa.x * bf16lo(ww.x);
          acc = acc + xa.y * bf16hi(ww.x);
          acc = acc + xa.z * bf16lo(ww.y);
          acc = acc + xa.w * bf16hi(ww.y);
          acc = acc + xc.x * bf16lo(ww.z);
          acc = acc + xc.y * bf16hi(ww.z);
          acc = acc + xc.z * bf16lo(ww.w);
          acc = acc + xc.w * bf16hi(ww.w);
        }
      }
    }
  }
  // halving tree: lane l += lane l + w for w = 8, 4, 2, 1 (row_shl within 16 lanes)
  acc = acc + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, acc), 0x108, 0xF, 0xF, true));
  acc = acc + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, acc), 0x104, 0xF, 0xF, true));
  acc = acc + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, acc), 0x102, 0xF, 0xF, true));
  acc = acc + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, acc), 0x101, 0xF, 0xF, true));
  if (l == 0 && e <= L.E) st_coh_u64(zt + e, ((uint64_t)tag << 32) | f2u(acc));
}

// ---------------------------------------------------------------------------
// One selection round set over NK keys per lane (lane l owns experts
// NK*l .. NK*l+NK-1, so lane order is id order): `rounds` times take the
// largest remaining key, the lowest id on equal keys.  Winners go to ids[].
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
    const uint64_t bal = __builtin_amdgcn_ballot_w64(lm == gm);
    const int fl = bal ? (int)__builtin_ctzll(bal) : 0;
    if (lane == fl) {
      int si = 0;
#pragma unroll
      for (int i = NK - 1; i >= 0; --i)
        if (!(taken >> i & 1u) && key[i] == gm) si = i;
      taken |= 1u << si;
      const int e = NK * lane + si;
      ids[it] = e < E ? e : E - 1;
    }
    if (!want_next && it == rounds - 1) break;
  }
}

// Routing on wave 0: poll the tagged logits until every entry carries this
// launch's tag, select the top-k (fast path on z, exact path on p), the
// shared gate sigmoid(z_E) (src/layers/moe.mojo:70-100).  Identical in every
// workgroup; only `record` workgroups write error keys.  Returns false on a
// poll timeout.
template <int R>
__device__ __forceinline__ bool route(const uint64_t* zt, unsigned tag, int E, int K, SelState& st,
                                      bool record, int token, unsigned long long* status) {
  constexpr int NK = 4 * R;
  const int lane = threadIdx.x & 63;
  const int e0 = NK * lane;
  float z[NK];
  float gl = 0.0f;
  bool ok = false;
  for (long spin = 0; spin < kSpinLimit; ++spin) {
    bool ready = true;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      z[i] = 0.0f;
      if (e0 + i < E) {
        const uint64_t v = ld_coh_u64(zt + e0 + i);
        z[i] = u2f((uint32_t)v);
        ready &= (uint32_t)(v >> 32) == tag;
      }
    }
    if (lane == 0) {
      const uint64_t v = ld_coh_u64(zt + E);
      gl = u2f((uint32_t)v);
      ready &= (uint32_t)(v >> 32) == tag;
    }
    if (__builtin_amdgcn_ballot_w64(!ready) == 0) {
      ok = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (!ok && lane == 0) record_err(status, err_key(kPhSync, 0, 0, 0, 0));
  uint32_t key[NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    key[i] = 0;
    const int e = e0 + i;
    if (e < E) {
      st.zv[e] = z[i];
      if (record && !finite_f(z[i])) record_err(status, err_key(kPhLogit, token, 0, e, 0));
      key[i] = f2key(z[i]);
    }
  }
  uint32_t kr[3];
  select_keys<NK>(key, K, E, st.ids, K < E, kr);
  const float m = key2f(kr[0]);
  if (record && lane == 0 && !finite_f(m)) record_err(status, err_key(kPhSoftmax, token, 0, 0, 0));
  bool unsafe = false;
  if (K < E) {
    const float ek = dm_expf(key2f(kr[1]) - m), en = dm_expf(key2f(kr[2]) - m);
    unsafe = !(ek > en + en * 0x1p-20f);
  }
  if (unsafe) {  // select on the exact probabilities
    float ev[NK];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      ev[i] = 0.0f;
      if (e0 + i < E) {
        ev[i] = dm_expf(z[i] - m);
        st.ev[e0 + i] = ev[i];
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    float s = 0.0f;
    for (int e = 0; e < E; ++e) s = s + st.ev[e];
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < NK; ++i) key[i] = e0 + i < E ? f2u(ev[i] * inv) + 1u : 0u;
    select_keys<NK>(key, K, E, st.ids, false, kr);
  }
  if (lane == 0) {
    if (record && !finite_f(gl)) record_err(status, err_key(kPhGate, token, 0, 0, kGkLogit));
    const float sg = dm_sigmoid(gl);
    if (record && (!finite_f(sg) || sg < 0.0f || sg > 1.0f))
      record_err(status, err_key(kPhGate, token, 0, 0, kGkRange));
    st.misc[0] = sg;
    st.misc[1] = m;
  }
  return ok;
}

// The softmax normaliser (sequential over e, src/layers/router.mojo:150-183),
// the K probabilities, their (p desc, id asc) order and the checks of
// src/layers/topk.mojo:109-128, on one wave.  Writes the slot weights pw[]
// (p_k; the shared gate for slot K) and ranks; `outputs` also writes ids /
// probs / shared gate in the reference's order.
template <int R>
__device__ __forceinline__ void finish_probs(int E, int K, SelState& st, bool record, int token,
                                             unsigned long long* status, int32_t* ids_out,
                                             float* probs_out, float* shg_out) {
  constexpr int NK = 4 * R;
  const int lane = threadIdx.x & 63, e0 = NK * lane;
  const float m = st.misc[1];
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    const int e = e0 + i;
    if (e < E) {
      const float ev = dm_expf(st.zv[e] - m);
      if (record && !finite_f(ev)) record_err(status, err_key(kPhSoftmax, token, 0, 1 + e, 0));
      st.ev[e] = ev;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  if (lane != 0) return;
  float s = 0.0f;
  const float4* ev4 = reinterpret_cast<const float4*>(st.ev);
  int e = 0;
#pragma unroll 8
  for (; e + 4 <= E; e += 4) {
    const float4 v = ev4[e >> 2];
    s = s + v.x;
    s = s + v.y;
    s = s + v.z;
    s = s + v.w;
  }
  for (; e < E; ++e) s = s + st.ev[e];
  if (record && (!(s > 0.0f) || !finite_f(s)))
    record_err(status, err_key(kPhSoftmax, token, 0, 1 + E, 0));
  const float inv = 1.0f / s;
  float* p = st.p;
  int* order = st.order;
  for (int k = 0; k < K; ++k) {
    p[k] = st.ev[st.ids[k]] * inv;
    order[k] = k;
  }
  for (int a = 1; a < K; ++a) {  // (p desc, id asc)
    const int v = order[a];
    int b = a - 1;
    while (b >= 0 && (p[order[b]] < p[v] || (p[order[b]] == p[v] && st.ids[order[b]] > st.ids[v]))) {
      order[b + 1] = order[b];
      --b;
    }
    order[b + 1] = v;
  }
  float sum_topk = 0.0f;
  for (int k = 0; k < K; ++k) {
    sum_topk = sum_topk + p[order[k]];
    st.rank[order[k]] = k;
    st.pw[k] = p[k];
  }
  st.pw[K] = st.misc[0];
  if (record) {
    if (sum_topk > 1.00001f) record_err(status, err_key(kPhTopk, token, 0, 0, kTkSum));
    if (K < E && __builtin_fabsf(sum_topk - 1.0f) < 1e-6f) {
      float sum_all = 0.0f;
      for (int e2 = 0; e2 < E; ++e2) sum_all = sum_all + st.ev[e2] * inv;
      if (sum_all - sum_topk > 1e-5f) record_err(status, err_key(kPhTopk, token, 0, 0, kTkLeak));
    }
  }
  if (ids_out) {
    for (int k = 0; k < K; ++k) {
      ids_out[k] = st.ids[order[k]];
      probs_out[k] = p[order[k]];
    }
    shg_out[0] = st.misc[0];
  }
}

// ---------------------------------------------------------------------------
template <int GQW, int R>
__global__ __launch_bounds__(kThreads) void k_moe_decode(
    LayerDev L, DecodePlan P, const float* __restrict__ x, const float* __restrict__ residual,
    float* __restrict__ y, int32_t* __restrict__ ids_out, float* __restrict__ probs_out,
    float* __restrict__ shg_out, DecodeSync S, unsigned long long* status, int token) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* xt = reinterpret_cast<float*>(smem + P.off_xt);
  uint4* xb2 = reinterpret_cast<uint4*>(smem + P.off_xb);
  float* red = reinterpret_cast<float*>(smem + P.off_red);
  uint4* hb2 = reinterpret_cast<uint4*>(smem + P.off_hb);
  float* yred = reinterpret_cast<float*>(smem + P.off_yred);
  unsigned char* sel = smem + P.off_sel;
  SelState st{reinterpret_cast<float*>(smem + P.off_zv), reinterpret_cast<float*>(smem + P.off_ev),
              reinterpret_cast<int*>(sel),         reinterpret_cast<int*>(sel + 128),
              reinterpret_cast<float*>(sel + 256), reinterpret_cast<float*>(sel + 400),
              reinterpret_cast<float*>(sel + 416), reinterpret_cast<int*>(sel + 544)};

  const int H = L.H, K = L.K, E = L.E;
  const int b = blockIdx.x, nb = gridDim.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int q = lane >> 4, j = lane & 15;
  const unsigned n = S.n;
  const int nGQI = L.I / kQuadCols, nGQS = L.Ish / kQuadCols;
  const int nrb = L.I / kTileRows;          // routed gate/up tiles per slot
  const int nsh = L.Ish / kTileRows;        // shared-expert gate/up tiles
  const bool down_wg = b < H / kTileRows;   // one 16-row output tile per workgroup
  const int nch_r = K * nGQI, nch = nch_r + nGQS;  // down chunks of an output tile
  const int my_chunks = down_wg ? (nch - w + kWaves - 1) / kWaves : 0;
  const bool router_wg = b < P.n_router_wg;
  const int sh_tile = (b + nb - P.n_router_wg % nb) % nb;

  // ---- entry: every load that depends on neither x nor routing --------------
  uint4 rw[kRwMax];
  const int re = b * kRouterRows + (tid >> 4);
  if (router_wg && tid < kRouterRows * 16 && re <= E) {
    const uint4* wp = reinterpret_cast<const uint4*>(L.router + r16_index(H, re, tid & 15));
#pragma unroll
    for (int j8 = 0; j8 < kRwMax; ++j8)
      if (j8 < H / 128) rw[j8] = wp[(size_t)j8 * 16];
  }
  const size_t matS = (size_t)L.Ish * H;
  const ExpertView sgv = {L.sgu_nib, L.sgu_sc, L.Ish, H};
  const ExpertView suv = {L.sgu_nib + matS / 2, L.sgu_sc + matS / kGroup, L.Ish, H};
  uint4 swg[GQW], swu[GQW];
  uint2 ssg[GQW], ssu[GQW];
  if (sh_tile < nsh) gu_load<GQW>(sgv, suv, sh_tile, swg, swu, ssg, ssu);
  const ExpertView sdv = {L.sd_nib, L.sd_sc, H, L.Ish};
  uint4 dw[kDownBatch];
  uint2 ds[kDownBatch];
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i) {
    const int c = w + kWaves * i;
    if (i < my_chunks && c >= nch_r) load_chunk(sdv, b, c - nch_r, lane, dw[i], ds[i]);
  }

  // ---- stage x: transposed fp32 (router chains) and bf16 hi/lo B blocks -----
  {
    bool bad = false;
    for (int i = tid; i < H / 8; i += kThreads) {
      const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
      const float4 c = reinterpret_cast<const float4*>(x)[2 * i + 1];
      const float f[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
      for (int k2 = 0; k2 < 8; ++k2) bad |= !finite_f(f[k2]);
      if (router_wg) {
        // columns 8i..8i+7 are chains l = 8(i&1)+k2 at step j = i/2
        const int xts = H / 16 + 4;
        float* dst = xt + (8 * (i & 1)) * xts + (i >> 1);
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) dst[k2 * xts] = f[k2];
      }
      uint4 hi, lo;
      split8(f, hi, lo);
      xb2[2 * i + 0] = hi;
      xb2[2 * i + 1] = lo;
    }
    if (bad && b == 0) record_err(status, err_key(kPhX, 0, 0, 0, 0));
  }
  __syncthreads();

  // ---- P1: router rows; shared-expert gate/up tile --------------------------
  if (router_wg && tid < kRouterRows * 16) router_compute(L, rw, re, xt, S.zt, n);
  for (int rr = b + nb; rr < P.n_router_wg; rr += nb) {  // only when the grid is small
    if (tid < kRouterRows * 16) {
      // the transposed x is staged only by router workgroups, which this one is
      const int e2 = rr * kRouterRows + (tid >> 4);
      if (e2 <= E) {
        const uint4* wp = reinterpret_cast<const uint4*>(L.router + r16_index(H, e2, tid & 15));
#pragma unroll
        for (int j8 = 0; j8 < kRwMax; ++j8)
          if (j8 < H / 128) rw[j8] = wp[(size_t)j8 * 16];
      }
      router_compute(L, rw, e2, xt, S.zt, n);
    }
  }
  for (int t = sh_tile; t < nsh; t += nb) {
    if (t != sh_tile) gu_load<GQW>(sgv, suv, t, swg, swu, ssg, ssu);
    gu_compute<GQW>(sgv, t, swg, swu, ssg, ssu, xb2, red, S.ht + (size_t)K * P.ldh, n, kPhShared,
                    token, 0, nullptr, status);
  }

  // ---- P2: routing (every workgroup computes the same top-k) ----------------
  if (w == 0) {
    const bool rok = route<R>(S.zt, n, E, K, st, b == 0, token, status);
    if (lane == 0) st.misc[2] = rok ? 1.0f : 0.0f;
  }
  __syncthreads();
  const bool ok = st.misc[2] != 0.0f;

  // ---- P3: routed loads; normaliser; routed gate/up tile --------------------
  const size_t matI = (size_t)L.I * H;
  auto gu_views = [&](int t, ExpertView& gv, ExpertView& uv) {
    const int e = st.ids[t / nrb];
    gv = {L.gu_nib + (size_t)e * matI, L.gu_sc + (size_t)e * 2 * (matI / kGroup), L.I, H};
    uv = {gv.nib + matI / 2, gv.sc + matI / kGroup, L.I, H};
  };
  const size_t matD = (size_t)H * L.I;
  auto down_view = [&](int s) -> ExpertView {
    const int e = st.ids[s];
    return {L.d_nib + (size_t)e * (matD / 2), L.d_sc + (size_t)e * (matD / kGroup), H, L.I};
  };
  uint4 gwg[GQW], gwu[GQW];
  uint2 gsg[GQW], gsu[GQW];
  ExpertView gv, uv;
  if (b < K * nrb) {
    gu_views(b, gv, uv);
    gu_load<GQW>(gv, uv, b % nrb, gwg, gwu, gsg, gsu);
  }
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i) {
    const int c = w + kWaves * i;
    if (i < my_chunks && c < nch_r) load_chunk(down_view(c / nGQI), b, c % nGQI, lane, dw[i], ds[i]);
  }
  if (w == kProbWave)
    finish_probs<R>(E, K, st, b == 0, token, status, b == 0 ? ids_out : nullptr, probs_out,
                    shg_out);
  for (int t = b; t < K * nrb; t += nb) {
    if (t != b) {
      gu_views(t, gv, uv);
      gu_load<GQW>(gv, uv, t % nrb, gwg, gwu, gsg, gsu);
    }
    const int k = t / nrb;
    // (the first barrier inside also publishes the normaliser wave's results)
    gu_compute<GQW>(gv, t % nrb, gwg, gwu, gsg, gsu, xb2, red, S.ht + (size_t)k * P.ldh, n,
                    kPhExpert, token, k, st.rank, status);
  }
  if (K * nrb <= b) __syncthreads();  // publish the normaliser results here instead
  if (!down_wg) return;

  // ---- P4: down projection of this workgroup's 16 output rows ---------------
  bf16x8 A[kDownBatch][4];
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i)
    if (i < my_chunks)
#pragma unroll
      for (int c = 0; c < 4; ++c) A[i][c] = dequant8(word_of(dw[i], c), scale_of(ds[i], c));
  // poll the tagged h of all slots; stage h * weight(slot) as split B blocks
  const int nblk_slot = P.ldh / 8;
  const int items_r = K * (L.I / 8), items = items_r + L.Ish / 8;
  {
    bool done = false;
    uint32_t have = 0;
    for (long spin = 0; spin < kSpinLimit; ++spin) {
      bool mine = true;
      uint64_t v[kPollItems][8];
#pragma unroll
      for (int bi = 0; bi < kPollItems; ++bi) {  // all loads of the pass first
        const int it = tid + kThreads * bi;
        if (it < items && !(have >> bi & 1u)) {
          const int s = it < items_r ? it / (L.I / 8) : K;
          const int ii = it < items_r ? it % (L.I / 8) : it - items_r;
          const uint64_t* src = S.ht + (size_t)s * P.ldh + 8 * ii;
#pragma unroll
          for (int k2 = 0; k2 < 8; ++k2) v[bi][k2] = ld_coh_u64(src + k2);
        }
      }
#pragma unroll
      for (int bi = 0; bi < kPollItems; ++bi) {
        const int it = tid + kThreads * bi;
        if (it < items && !(have >> bi & 1u)) {
          const int s = it < items_r ? it / (L.I / 8) : K;
          const int ii = it < items_r ? it % (L.I / 8) : it - items_r;
          bool tags = true;
          float f[8];
          const float wgt = st.pw[s];
#pragma unroll
          for (int k2 = 0; k2 < 8; ++k2) {
            tags &= (uint32_t)(v[bi][k2] >> 32) == n;
            f[k2] = u2f((uint32_t)v[bi][k2]) * wgt;
          }
          if (tags) {
            uint4 hi, lo;
            split8(f, hi, lo);
            uint4* dst = hb2 + 2 * ((size_t)s * nblk_slot + ii);
            dst[0] = hi;
            dst[1] = lo;
            have |= 1u << bi;
          } else {
            mine = false;
          }
        }
      }
      if (__syncthreads_and(mine || !ok)) {
        done = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!done && tid == 0) record_err(status, err_key(kPhSync, 0, 0, 0, 0));
  }
  // one MFMA chain per wave over its chunks: sum_k W_k (p_k h_k) + W_sh (g h_sh)
  f32x4 acc = {0, 0, 0, 0};
  for (int base = 0; base < my_chunks; base += kDownBatch) {
    if (base > 0) {  // chunks beyond the register batch
#pragma unroll
      for (int i = 0; i < kDownBatch; ++i) {
        const int c = w + kWaves * (base + i);
        if (base + i < my_chunks) {
          if (c < nch_r) load_chunk(down_view(c / nGQI), b, c % nGQI, lane, dw[i], ds[i]);
          else load_chunk(sdv, b, c - nch_r, lane, dw[i], ds[i]);
        }
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
        const int c = w + kWaves * (base + i);
        const int s = c < nch_r ? c / nGQI : K, gq = c < nch_r ? c % nGQI : c - nch_r;
        const uint4* hbs = hb2 + 2 * (size_t)s * nblk_slot;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) acc = mfma16(A[i][cc], ld_b(hbs, (gq * 4 + cc) * 4 + q, j), acc);
      }
    }
  }
  fold_cols(acc);
  if (j == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) yred[w * 16 + 4 * q + r] = acc[r];
  }
  __syncthreads();
  if (tid < 16) {
    const int d = b * kTileRows + tid;
    float total = 0.0f;
#pragma unroll
    for (int v2 = 0; v2 < kWaves; ++v2) total = total + yred[v2 * 16 + tid];
    if (residual) total = total + residual[d];
    // a non-finite output: the host re-derives which check of the reference fires first
    if (!finite_f(total)) record_err(status, err_key(kPhExpert, token, 0, 0, kEkRecheck));
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
  S.zt = (uint64_t*)p;
  p += align256z((256 * R + 64) * 8);
  S.ht = (uint64_t*)p;
  return S;
}

DecodePlan make_decode_plan(const LayerDev& L, int num_cus) {
  DecodePlan P{};
  P.ldh = L.I > L.Ish ? L.I : L.Ish;
  P.n_router_wg = (L.E + 1 + kRouterRows - 1) / kRouterRows;
  const int R = (L.E + 255) / 256;
  const int slots = L.K + 1;
  int off = 0;
  P.off_xt = off; off += align16(4 * kRouterRows * (L.H / 16 + 4));
  P.off_xb = off; off += align16(4 * L.H);
  P.off_zv = off; off += align16(4 * 256 * R);
  P.off_ev = off; off += align16(4 * 256 * R);
  P.off_sel = off; off += 768;
  P.off_red = off; off += align16(kWaves * 2 * 16 * 4);
  P.off_hb = off; off += align16(slots * (P.ldh / 8) * 32);
  P.off_yred = off; off += align16(kWaves * 16 * 4);
  P.lds_bytes = off;
  P.threads = kThreads;
  P.grid = num_cus > L.H / kTileRows ? num_cus : L.H / kTileRows;
  return P;
}

template <int GQW>
static const void* pick_r(int R) {
  return R <= 1 ? (const void*)k_moe_decode<GQW, 1> : (const void*)k_moe_decode<GQW, 8>;
}

static const void* pick_kernel(const LayerDev& L) {
  const int gqw = (L.H / kQuadCols + kWaves - 1) / kWaves;
  const int R = (L.E + 255) / 256;
  if (R > 8 || L.K > 32) return nullptr;
  return gqw <= 2 ? pick_r<2>(R) : gqw <= 8 ? pick_r<8>(R) : nullptr;
}

hipError_t decode_occupancy(const LayerDev& L, const DecodePlan& P, int* blocks_per_cu) {
  const void* fn = pick_kernel(L);
  if (!fn) return hipErrorInvalidValue;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, P.threads, P.lds_bytes);
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
  return hipLaunchKernel(fn, dim3(P.grid), dim3(P.threads), args, P.lds_bytes, st);
}

}  // namespace dm
