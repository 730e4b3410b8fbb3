// dm_decode.hip -- the fused single-launch decode kernel of the MoE block.
//
// One launch computes the whole block for one token (forward_moe_block,
// src/layers/moe_block.mojo:20-138, with the routed experts of
// src/layers/swiglu.mojo:52-230 and the combine of src/layers/moe.mojo:150-175
// / src/layers/forward_layer.mojo:226-238).  The grid is one persistent
// workgroup per CU; the phases hand data to each other through coherent
// counters instead of kernel boundaries:
//
//   P1  router rows (16 per WG, exact 16-lane order)          -> z, cnt_router
//       shared-expert gate/up tiles (independent of routing)  -> h[K], cnt_h[K]
//   P2  every WG: wait cnt_router, softmax + top-k itself (identical result
//       everywhere, so no broadcast handoff), issue its down-projection loads
//   P3  routed gate/up tile (slot, 16 rows), full reduction in the WG -> h[k]
//   P4  down unit (16 output rows, half of the K+1 slots): dequantise the
//       prefetched weights, wait for h of its slots, MFMA, partial combine;
//       the second arriver of the two halves writes y (last-arriver, no wait).
//
// Counters only grow: launch n waits for n * (arrivals per launch), so they
// never need a reset between launches.  Every wait is bounded.
#include <hip/hip_runtime.h>

#include "dm_decode.h"
#include "dm_device.h"

namespace dm {

constexpr int kDownBatch = 8;  // down chunks per wave held in registers

// Gate/up of one 16-row tile: h = SiLU(W_g x) * (W_u x) for rows 16rb..+15,
// reduction over all H columns inside the workgroup (4 waves x nGQ/4 chunks).
// Result rows are stored coherently to hdst[row]; returns after the stores
// of wave 0 completed (the caller then signals).
template <int GQW>
__device__ __forceinline__ void gateup_tile(const ExpertView& gv, const ExpertView& uv, int rb,
                                            const uint4* xb, float* red, float* hdst,
                                            uint32_t phase, uint32_t token, uint32_t slot,
                                            unsigned long long* status) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15, jsel = j < 2 ? j : 2;
  const int nGQ = gv.cols / kQuadCols;
  uint4 wg[GQW], wu[GQW];
  uint2 sg[GQW], su[GQW];
#pragma unroll
  for (int i = 0; i < GQW; ++i) {
    const int gq = w + 4 * i;
    if (gq < nGQ) {
      load_chunk(gv, rb, gq, lane, wg[i], sg[i]);
      load_chunk(uv, rb, gq, lane, wu[i], su[i]);
    }
  }
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
    st_coh(hdst + row, h);
    wait_stores();
  }
  __syncthreads();
}

// Router rows 16*b..16*b+15 (row E = shared-expert gate): one lane per
// (row, chain l), sequential chains, halving tree; xs = fp32 x in LDS.
__device__ __forceinline__ void router_rows(const LayerDev& L, int b, const float* xs, float* z) {
  const int H = L.H;
  const int l = threadIdx.x & 15;
  const int e = b * 16 + (threadIdx.x >> 4);
  float acc = 0.0f;
  if (e <= L.E) {
    const uint4* wp = reinterpret_cast<const uint4*>(L.router + r16_index(H, e, l));
    const int nj8 = H / 128;
    for (int j8 = 0; j8 < nj8; ++j8) {
      const uint4 w = wp[(size_t)j8 * 16];
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
      const float* xc = xs + j8 * 128 + l;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc = acc + xc[(2 * i) * 16] * bf16lo(ww[i]);
        acc = acc + xc[(2 * i + 1) * 16] * bf16hi(ww[i]);
      }
    }
  }
#pragma unroll
  for (int wdt = 8; wdt >= 1; wdt >>= 1) acc = acc + __shfl_down(acc, wdt, 16);
  if (l == 0 && e <= L.E) st_coh(z + e, acc);
  wait_stores();
}

// Softmax + top-k of src/layers/router.mojo:140-183 and
// src/layers/topk.mojo:79-128 on wave 0, result in LDS.  Identical in every
// workgroup; only `record` workgroups write error keys.
__device__ __forceinline__ void select_topk(const float* z, int E, int K, float* pv, int* sel_ids,
                                            float* sel_p, float* sel_g, bool record, int token,
                                            unsigned long long* status) {
  const int lane = threadIdx.x;
  if (lane >= 64) return;
  float m = -__builtin_inff();
  for (int e = lane; e < E; e += 64) {
    const float v = ld_coh(z + e);
    pv[e] = v;
    if (record && !finite_f(v)) record_err(status, err_key(kPhLogit, token, 0, e, 0));
    m = v > m ? v : m;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float other = __shfl_xor(m, o);
    m = other > m ? other : m;
  }
  if (record && lane == 0 && !finite_f(m)) record_err(status, err_key(kPhSoftmax, token, 0, 0, 0));
  for (int e = lane; e < E; e += 64) {
    const float ev = dm_expf(pv[e] - m);
    if (record && !finite_f(ev)) record_err(status, err_key(kPhSoftmax, token, 0, 1 + e, 0));
    pv[e] = ev;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  float inv = 0.0f;
  if (lane == 0) {
    float s = 0.0f;
    for (int e = 0; e < E; ++e) s = s + pv[e];
    if (record && (!(s > 0.0f) || !finite_f(s)))
      record_err(status, err_key(kPhSoftmax, token, 0, 1 + E, 0));
    inv = 1.0f / s;
  }
  inv = __shfl(inv, 0);
  for (int e = lane; e < E; e += 64) pv[e] = pv[e] * inv;
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  uint32_t taken = 0;
  float sum_topk = 0.0f;
  for (int i = 0; i < K; ++i) {
    float bv = -1.0f;
    int bi = 0x7FFFFFFF;
    for (int e = lane, s = 0; e < E; e += 64, ++s) {
      if (taken >> s & 1u) continue;
      const float v = pv[e];
      if (v > bv || (v == bv && e < bi)) { bv = v; bi = e; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (bi < 0 || bi >= E) bi = 0;
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    sum_topk = sum_topk + bv;
    if (lane == 0) {
      sel_ids[i] = bi;
      sel_p[i] = bv;
    }
  }
  if (lane == 0) {
    if (record && sum_topk > 1.00001f) record_err(status, err_key(kPhTopk, token, 0, 0, kTkSum));
    if (record && K < E && __builtin_fabsf(sum_topk - 1.0f) < 1e-6f) {
      float sum_all = 0.0f;
      for (int e = 0; e < E; ++e) sum_all = sum_all + pv[e];
      if (sum_all - sum_topk > 1e-5f) record_err(status, err_key(kPhTopk, token, 0, 0, kTkLeak));
    }
    const float lg = ld_coh(z + E);
    if (record && !finite_f(lg)) record_err(status, err_key(kPhGate, token, 0, 0, kGkLogit));
    const float sg = dm_sigmoid(lg);
    if (record && (!finite_f(sg) || sg < 0.0f || sg > 1.0f))
      record_err(status, err_key(kPhGate, token, 0, 0, kGkRange));
    *sel_g = sg;
  }
}

template <int GQW>
__global__ __launch_bounds__(256) void k_moe_decode(LayerDev L, DecodePlan P, const float* __restrict__ x,
                                                     const float* __restrict__ residual,
                                                     float* __restrict__ y, int32_t* __restrict__ ids_out,
                                                     float* __restrict__ probs_out,
                                                     float* __restrict__ shg_out, DecodeSync S,
                                                     unsigned long long* status, int token) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* xs = reinterpret_cast<float*>(smem + P.off_xs);
  uint4* xb = reinterpret_cast<uint4*>(smem + P.off_xb);
  float* pv = reinterpret_cast<float*>(smem + P.off_pv);
  int* sel_ids = reinterpret_cast<int*>(smem + P.off_sel);
  float* sel_p = reinterpret_cast<float*>(smem + P.off_sel + 4 * 64);
  float* sel_g = reinterpret_cast<float*>(smem + P.off_sel + 8 * 64);
  float* red = reinterpret_cast<float*>(smem + P.off_red);
  uint4* hb = reinterpret_cast<uint4*>(smem + P.off_hb);
  float* redd = reinterpret_cast<float*>(smem + P.off_redd);
  int* flag = reinterpret_cast<int*>(smem + P.off_sel + 8 * 64 + 16);

  const int H = L.H, K = L.K, E = L.E;
  const int b = blockIdx.x, nb = gridDim.x;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const unsigned n = S.n;
  bool ok = true;  // false after a timed-out wait: skip later waits

  // ---- stage x: fp32 copy (router chains) and bf16 hi/lo B blocks ----------
  bool bad = false;
  for (int i = threadIdx.x; i < H; i += 256) {
    const float v = x[i];
    bad |= !finite_f(v);
    xs[i] = v;
  }
  if (bad && b == 0) record_err(status, err_key(kPhX, 0, 0, 0, 0));
  stage_split(x, H, xb);
  __syncthreads();

  // ---- P1: router rows; shared-expert gate/up tiles ------------------------
  for (int rw = b; rw < P.n_router_wg; rw += nb) {
    router_rows(L, rw, xs, S.z);
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(S.cnt_router, 1u);
  }
  {
    const int nsh = L.Ish / kTileRows;
    const size_t mat = (size_t)L.Ish * H;
    const ExpertView gv = {L.sgu_nib, L.sgu_sc, L.Ish, H};
    const ExpertView uv = {L.sgu_nib + mat / 2, L.sgu_sc + mat / kGroup, L.Ish, H};
    for (int t = (b + nb - P.n_router_wg % nb) % nb; t < nsh; t += nb) {
      gateup_tile<GQW>(gv, uv, t, xb, red, S.h + (size_t)K * P.ldh, kPhShared, token, 0, status);
      if (threadIdx.x == 0) atomicAdd(S.cnt_h + K, 1u);
    }
  }

  // ---- P2: routing (every WG computes the same top-k) -----------------------
  if (threadIdx.x == 0) {
    ok = wait_count(S.cnt_router, n * (unsigned)P.n_router_wg, status);
    flag[0] = ok;
  }
  __syncthreads();
  ok = flag[0];
  select_topk(S.z, E, K, pv, sel_ids, sel_p, sel_g, b == 0, token, status);
  __syncthreads();
  if (b == 0 && threadIdx.x < K) {
    ids_out[threadIdx.x] = sel_ids[threadIdx.x];
    probs_out[threadIdx.x] = sel_p[threadIdx.x];
    if (threadIdx.x == 0) shg_out[0] = *sel_g;
  }

  // ---- P4 prologue: down unit of this WG, loads issued before P3 ----------
  const int nrbo = H / kTileRows;
  const int unit = b < 2 * nrbo ? b : -1;  // one down unit per WG (2*H/16 <= grid)
  const int half = unit >= 0 ? unit / nrbo : 0;
  const int rbo = unit >= 0 ? unit % nrbo : 0;
  const int s_lo = half == 0 ? 0 : P.s0, s_hi = half == 0 ? P.s0 : K + 1;
  // the wave's chunk list: index c = w + 4*i over (slot s, gq) in slot order
  int nchunk = 0;
  for (int s = s_lo; s < s_hi; ++s) nchunk += (s < K ? L.I : L.Ish) / kQuadCols;
  uint4 dw[kDownBatch];
  uint2 ds[kDownBatch];
  int dslot[kDownBatch], dgq[kDownBatch];
  auto chunk_at = [&](int c, int& s, int& gq) {
    s = s_lo;
    int cc = c;
    for (;;) {
      const int ng = (s < K ? L.I : L.Ish) / kQuadCols;
      if (cc < ng) break;
      cc -= ng;
      ++s;
    }
    gq = cc;
  };
  auto view_of = [&](int s) -> ExpertView {
    if (s < K) {
      int e = sel_ids[s];
      if (e < 0 || e >= E) e = 0;
      const size_t mat = (size_t)H * L.I;
      return {L.d_nib + (size_t)e * (mat / 2), L.d_sc + (size_t)e * (mat / kGroup), H, L.I};
    }
    return {L.sd_nib, L.sd_sc, H, L.Ish};
  };
  const int my_chunks = unit >= 0 ? (nchunk - w + 3) / 4 : 0;
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i) {
    dslot[i] = 0;
    dgq[i] = 0;
    if (i < my_chunks) {
      chunk_at(w + 4 * i, dslot[i], dgq[i]);
      load_chunk(view_of(dslot[i]), rbo, dgq[i], lane, dw[i], ds[i]);
    }
  }

  // ---- P3: routed gate/up tiles ---------------------------------------------
  {
    const int nrb = L.I / kTileRows;
    const size_t mat = (size_t)L.I * H;
    for (int t = b; t < K * nrb; t += nb) {
      const int k = t / nrb, rb = t % nrb;
      int e = sel_ids[k];
      if (e < 0 || e >= E) e = 0;
      const ExpertView gv = {L.gu_nib + (size_t)e * mat, L.gu_sc + (size_t)e * 2 * (mat / kGroup),
                             L.I, H};
      const ExpertView uv = {gv.nib + mat / 2, gv.sc + mat / kGroup, L.I, H};
      gateup_tile<GQW>(gv, uv, rb, xb, red, S.h + (size_t)k * P.ldh, kPhExpert, token, k, status);
      if (threadIdx.x == 0) atomicAdd(S.cnt_h + k, 1u);
    }
  }

  // ---- P4: down projection + combine ----------------------------------------
  if (unit < 0) return;
  // dequantise the prefetched chunks while the h tiles are still arriving
  bf16x8 A[kDownBatch][4];
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i)
    if (i < my_chunks)
#pragma unroll
      for (int c = 0; c < 4; ++c) A[i][c] = dequant8(word_of(dw[i], c), scale_of(ds[i], c));
  if (threadIdx.x == 0) {
    for (int s = s_lo; s < s_hi && ok; ++s) {
      const unsigned tiles = (unsigned)((s < K ? L.I : L.Ish) / kTileRows);
      ok = wait_count(S.cnt_h + s, n * tiles, status);
    }
    flag[0] = ok;
  }
  __syncthreads();
  ok = flag[0];
  // stage h of the half's slots as B blocks (coherent reads)
  const int nblk_slot = (P.ldh / 8) * 3;
  for (int s = s_lo; s < s_hi; ++s) {
    const int Is = s < K ? L.I : L.Ish;
    const float* hs = S.h + (size_t)s * P.ldh;
    uint4* dst = hb + (size_t)(s - s_lo) * nblk_slot;
    for (int i = threadIdx.x; i < Is / 8; i += 256) {
      float f[8];
#pragma unroll
      for (int k2 = 0; k2 < 8; ++k2) f[k2] = ld_coh(hs + 8 * i + k2);
      uint4 hi, lo;
      split8(f, hi, lo);
      dst[3 * i + 0] = hi;
      dst[3 * i + 1] = lo;
      dst[3 * i + 2] = make_uint4(0, 0, 0, 0);
    }
  }
  __syncthreads();
  const int q = lane >> 4, j = lane & 15, jsel = j < 2 ? j : 2;
  for (int base = 0; base < my_chunks; base += kDownBatch) {
    if (base > 0) {  // chunks beyond the prefetched batch
#pragma unroll
      for (int i = 0; i < kDownBatch; ++i)
        if (base + i < my_chunks) {
          chunk_at(w + 4 * (base + i), dslot[i], dgq[i]);
          load_chunk(view_of(dslot[i]), rbo, dgq[i], lane, dw[i], ds[i]);
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
        const uint4* hbs = hb + (size_t)(dslot[i] - s_lo) * nblk_slot;
        f32x4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int g = dgq[i] * 4 + c;
          acc = mfma16(A[i][c], __builtin_bit_cast(bf16x8, hbs[(g * 4 + q) * 3 + jsel]), acc);
        }
        fold_cols(acc);
        const int cidx = w + 4 * (base + i);
        if (j == 0) {
#pragma unroll
          for (int r = 0; r < 4; ++r) redd[cidx * 16 + 4 * q + r] = acc[r];
        }
      }
    }
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int r = threadIdx.x, d = rbo * kTileRows + r;
    float part = 0.0f;
    int c = 0;
    for (int s = s_lo; s < s_hi; ++s) {
      const int ng = (s < K ? L.I : L.Ish) / kQuadCols;
      float rs = 0.0f;
      for (int g = 0; g < ng; ++g, ++c) rs = rs + redd[c * 16 + r];
      if (s < K) {
        if (!finite_f(rs)) record_err(status, err_key(kPhExpert, token, s, P.ldh + d, kEkDown));
        part = part + sel_p[s] * rs;
      } else {
        if (!finite_f(rs)) record_err(status, err_key(kPhShared, token, 0, P.ldh + d, kEkDown));
        part = part + *sel_g * rs;
      }
    }
    st_coh(S.ypart + (size_t)half * H + d, part);
    wait_stores();
    unsigned old = 0;
    if (r == 0) old = atomicAdd(S.cnt_y + rbo, 1u);
    old = __shfl(old, 0, 16);
    if (old == 2 * n - 1) {  // second arriver of the two halves combines
      const float p0 = half == 0 ? part : ld_coh(S.ypart + d);
      const float p1 = half == 1 ? part : ld_coh(S.ypart + H + d);
      float total = p0 + p1;
      if (residual) total = total + residual[d];
      if (!finite_f(total)) record_err(status, err_key(kPhAgg, token, 0, d, 0));
      y[d] = total;
    }
  }
}

static int align16(int v) { return (v + 15) & ~15; }

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
  const int nch = nch0 > nch1 ? nch0 : nch1;
  const int slots = P.s0 > L.K + 1 - P.s0 ? P.s0 : L.K + 1 - P.s0;
  int off = 0;
  P.off_xs = off; off += align16(4 * L.H);
  P.off_xb = off; off += align16(6 * L.H);
  P.off_pv = off; off += align16(4 * (L.E + 2));
  P.off_sel = off; off += 640;
  P.off_red = off; off += 512;
  P.off_hb = off; off += align16(slots * (P.ldh / 8) * 3 * 16);
  P.off_redd = off; off += align16(nch * 64);
  P.lds_bytes = off;
  P.grid = num_cus > 2 * (L.H / kTileRows) ? num_cus : 2 * (L.H / kTileRows);
  return P;
}

hipError_t decode_occupancy(const LayerDev& L, const DecodePlan& P, int* blocks_per_cu) {
  const int gqw = (L.H / kQuadCols + 3) / 4;
  const void* fn = gqw <= 1 ? (const void*)k_moe_decode<1> : gqw <= 2 ? (const void*)k_moe_decode<2>
                 : gqw <= 4 ? (const void*)k_moe_decode<4> : gqw <= 8 ? (const void*)k_moe_decode<8>
                            : (const void*)k_moe_decode<16>;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, 256, P.lds_bytes);
}

hipError_t launch_moe_decode(const LayerDev& L, const DecodePlan& P, const float* x,
                             const float* residual, float* y, int32_t* ids, float* probs,
                             float* shg, const DecodeSync& S, unsigned long long* status, int token,
                             hipStream_t st) {
  const int gqw = (L.H / kQuadCols + 3) / 4;
#define DM_LAUNCH(G)                                                                          \
  hipLaunchKernelGGL(k_moe_decode<G>, dim3(P.grid), dim3(256), P.lds_bytes, st, L, P, x,     \
                     residual, y, ids, probs, shg, S, status, token)
  if (gqw <= 1) DM_LAUNCH(1);
  else if (gqw <= 2) DM_LAUNCH(2);
  else if (gqw <= 4) DM_LAUNCH(4);
  else if (gqw <= 8) DM_LAUNCH(8);
  else if (gqw <= 16) DM_LAUNCH(16);
  else return hipErrorInvalidValue;
#undef DM_LAUNCH
  return hipGetLastError();
}

}  // namespace dm
