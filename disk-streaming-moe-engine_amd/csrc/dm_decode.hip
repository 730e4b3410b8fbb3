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
//   entry  x first, then the loads that depend on neither x nor routing:
//          router rows, a shared-expert gate/up tile.
//   P1     router rows (4 per router workgroup, the exact 16-lane order of
//          router_project) -> z;  shared-expert gate/up tile -> h[K].
//   P2     every workgroup polls z and selects the top-k itself on wave 0
//          (identical everywhere, so no broadcast hand-off) while wave 7
//          forms the softmax normaliser and the shared gate.
//   P3     routed gate/up and down loads; routed gate/up tile (slot, 16
//          rows) -> h[k], published with its bf16 hi/lo split.
//   P4     down tile (16 output rows, all K+1 slots): poll h, dequantize the
//          down chunks and (wave 7) form the probabilities meanwhile, MFMA
//          per chunk scaled by its slot's weight
//          (p_k, or the shared gate), residual, y.
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

#include <atomic>
#include <vector>

#include "dm_decode.h"
#include "dm_device.h"

namespace dm {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kRouterRows = 4;       // router rows per router workgroup (wave 0)
constexpr int kRwMax = 16;           // router chain chunks (8 bf16 each) held per lane
constexpr int kDownBatch = 5;        // down chunks per wave held in registers
constexpr int kHw = 5;               // h words per thread (all polled at once)
constexpr int kNormWave = 7;          // softmax normaliser during routing; probabilities after the gate/up tile

// LDS state of the routing decision.
struct SelState {
  float* zv;    // [256R] logits
  float* ev;    // [256R] e = exp(z - max)
  int* ids;     // [32] selected experts, slot order
  int* rank;    // [32] position of each slot in the (p desc, id asc) order
  float* pw;    // [33] B-operand weight of slot s: p_s; slot K: the shared gate
  float* misc;  // [0] shared gate, [2] ok flag, [3] 1/S
  float* scr;   // [64] p by slot, then p by rank (16-byte aligned)
};

// The wave index as a uniform (scalar) value: derived from threadIdx the
// compiler treats it as divergent and masks every per-wave branch.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// B operand of a 16x16x32 MFMA from split blocks blk2[2*b + {hi, lo}]:
// lane (q, j) holds rows 8q..8q+7 of column j; columns 0/1 carry hi/lo.  The
// other columns repeat them: column j of the product depends on column j of
// B only, and only columns 0 and 1 are ever read (fold_cols, then j == 0),
// so they need no zeroing.
__device__ __forceinline__ bf16x8 ld_b(const uint4* blk2, int blk, int j) {
  return __builtin_bit_cast(bf16x8, blk2[2 * blk + (j & 1)]);
}

// The same operand from separate bf16 arrays hi[] / lo[] (8 values per block).
__device__ __forceinline__ bf16x8 ld_b2(const uint16_t* hi, const uint16_t* lo, int blk, int j) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>((j & 1 ? lo : hi) + 8 * blk));
}

// fp32 -> bf16 hi + bf16 lo (v ~= hi + lo within 2^-17 relative).
__device__ __forceinline__ void split1(float v, uint16_t& hi, uint16_t& lo) {
  const uint32_t h = pack_bf16x2(v, 0.0f) & 0xFFFFu;
  hi = (uint16_t)h;
  lo = (uint16_t)(pack_bf16x2(v - u2f(h << 16), 0.0f) & 0xFFFFu);
}

// h hand-off word: two values (rows 2i and 2i+1 of a slot) and the low 16
// bits of the launch tag, (tag16 << 48) | (v1 << 24) | v0, each value the top
// 24 bits of its float encoding rounded to nearest (16 significant bits, the
// precision of the bf16 hi + lo pair the down tile's MFMA operand is formed
// from).  Half the words of a one-value-per-word hand-off, so each poll of h
// moves half the bytes.
__device__ __forceinline__ uint32_t h24(float v) { return (f2u(v) + 0x80u) >> 8; }
__device__ __forceinline__ uint64_t pack_h2(unsigned tag, float v0, float v1) {
  return ((uint64_t)(tag & 0xFFFFu) << 48) | ((uint64_t)h24(v1) << 24) | h24(v0);
}
__device__ __forceinline__ bool h2_current(uint64_t wd, unsigned tag) {
  return (uint32_t)(wd >> 48) == (tag & 0xFFFFu);
}
__device__ __forceinline__ float h2_v0(uint64_t wd) { return u2f((uint32_t)wd << 8); }
__device__ __forceinline__ float h2_v1(uint64_t wd) { return u2f((uint32_t)(wd >> 24) << 8); }

// ---------------------------------------------------------------------------
// Gate/up of one 16-row tile: h = SiLU(W_g x) * (W_u x) for rows 16rb..+15,
// reduced over all H columns inside the workgroup (wave w owns the 128-column
// chunks w, w+8, ...).  gu_load issues the loads; gu_compute consumes them and
// stores the 16 h values as 8 pack_h2 words to hdst[row / 2].
template <int GQW, bool NT>
__device__ __forceinline__ void gu_load(const ExpertView& gv, const ExpertView& uv, int rb,
                                        uint4 (&wg)[GQW], uint4 (&wu)[GQW], uint2 (&sg)[GQW],
                                        uint2 (&su)[GQW]) {
  const int w = wave_id(), lane = threadIdx.x & 63;
  const int nGQ = gv.cols / kQuadCols;
  // unconditional loads (a chunk past the end re-reads the last one and is
  // not used): conditional loads in unrolled code get serialized
#pragma unroll
  for (int i = 0; i < GQW; ++i) {
    const int gq = min(w + kWaves * i, nGQ - 1);
    if (NT) {
      load_chunk_nt(gv, rb, gq, lane, wg[i], sg[i]);
      load_chunk_nt(uv, rb, gq, lane, wu[i], su[i]);
    } else {
      load_chunk(gv, rb, gq, lane, wg[i], sg[i]);
      load_chunk(uv, rb, gq, lane, wu[i], su[i]);
    }
  }
}

// The products of one 16-row tile for this wave's chunks (w, w+8, ...):
// gate and up partial sums over its columns, folded to column 0, stored to
// red[(w * 2 + {0: gate, 1: up}) * 16 + row].
// kShifted: dequant8_shifted (the one-token kernels), else dequant8.
template <int GQW, bool kShifted>
__device__ __forceinline__ void gu_products(const ExpertView& gv, const uint4 (&wg)[GQW],
                                            const uint4 (&wu)[GQW], const uint2 (&sg)[GQW],
                                            const uint2 (&su)[GQW], const uint4* xb2,
                                            float* red) {
  const int w = wave_id(), lane = threadIdx.x & 63;
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
        const uint32_t wgc = word_of(wg[i], c), wuc = word_of(wu[i], c);
        const float sgc = scale_of(sg[i], c), suc = scale_of(su[i], c);
        ag = mfma16(kShifted ? dequant8_shifted(wgc, sgc) : dequant8(wgc, sgc), b, ag);
        au = mfma16(kShifted ? dequant8_shifted(wuc, suc) : dequant8(wuc, suc), b, au);
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
}

// hdst: the tile's 8 hand-off words.  LOCAL: plain stores, read only by
// workgroups on the same XCD (through its L2); otherwise agent-scope stores.
template <int GQW, bool LOCAL = false>
__device__ __forceinline__ void gu_compute(const ExpertView& gv, int rb, const uint4 (&wg)[GQW],
                                           const uint4 (&wu)[GQW], const uint2 (&sg)[GQW],
                                           const uint2 (&su)[GQW], const uint4* xb2, float* red,
                                           uint64_t* hdst, unsigned tag, uint32_t phase,
                                           uint32_t token, unsigned long long* status) {
  gu_products<GQW, true>(gv, wg, wu, sg, su, xb2, red);
  __syncthreads();
  if (threadIdx.x < 16) {
    const int r = threadIdx.x, row = rb * kTileRows + r;
    float g = 0.0f, u = 0.0f;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
      g = g + red[v * 32 + r];
      u = u + red[v * 32 + 16 + r];
    }
    const float h = dm_silu(g) * u;
    if (!finite_f(g) || !finite_f(u) || !finite_f(h)) {
      // shared expert: the exact key (slot 0); routed expert: the slot's
      // position in the reference's order is formed later, so the host
      // re-derives the first failing check
      if (phase == kPhShared)
        record_err(status, err_key(phase, token, 0, row,
                                   !finite_f(g) ? kEkGate : !finite_f(u) ? kEkUp : kEkH));
      else
        record_err(status, err_key(kPhExpert, token, 0, 0, kEkRecheck));
    }
    // published in pairs of rows (2i, 2i+1) as one word (hand-off format
    // of pack_h2); the partner's value comes from the neighbouring lane
    const float hn = __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, h), 0xB1, 0xF, 0xF, true));
    if ((r & 1) == 0) {
      if (LOCAL)
        st_l2_u64(hdst + (r >> 1), pack_h2(tag, h, hn));
      else
        st_coh_u64(hdst + (r >> 1), pack_h2(tag, h, hn));
    }
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
template <bool LOCAL = false>
__device__ __forceinline__ void router_compute(const LayerDev& L, uint4 (&rw)[kRwMax], int e,
                                               const float* xt, uint64_t* zt, unsigned tag) {
  const int l = threadIdx.x & 15;
  const int nj8 = L.H / 128;
  const float4* xr = reinterpret_cast<const float4*>(xt + l * (L.H / 16 + 4));
  float acc = 0.0f;
  if (e <= L.E && nj8 == kRwMax) {
    // every chunk preloaded (H = 2048): one straight-line block, so the x
    // reads from LDS are issued ahead of the chain instead of one chunk at a
    // time behind a branch
    // x of four chunks in flight ahead of the chain (the compiler otherwise
    // reads each chunk just before its products and waits for it)
    constexpr int kAhead = 4;
    float4 xq[kAhead][2];
#pragma unroll
    for (int t = 0; t < kAhead; ++t) {
      xq[t][0] = xr[2 * t];
      xq[t][1] = xr[2 * t + 1];
    }
#pragma unroll
    for (int j8 = 0; j8 < kRwMax; ++j8) {
      const float4 xa = xq[j8 % kAhead][0], xc = xq[j8 % kAhead][1];
      if (j8 + kAhead < kRwMax) {
        xq[j8 % kAhead][0] = xr[2 * (j8 + kAhead)];
        xq[j8 % kAhead][1] = xr[2 * (j8 + kAhead) + 1];
      }
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
  } else if (e <= L.E) {
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
  if (l == 0 && e <= L.E) {
    if (LOCAL)
      st_l2_u64(zt + e, ((uint64_t)tag << 32) | f2u(acc));
    else
      st_coh_u64(zt + e, ((uint64_t)tag << 32) | f2u(acc));
  }
}


// Routing on wave 0.  Selects the K largest logits with unique 32-bit keys
// (the high bits of the logit's order key, then the inverted expert id, so
// equal logits order by the lower id), then checks that the smallest
// selected logit and the largest unselected one are far enough apart that
// p = exp(z - max) * (1/S) keeps them strictly ordered; otherwise it forms S
// and selects on the exact probabilities with the lowest-id tie-break.
// Identical in every workgroup; only `record` workgroups write error keys.
template <int R>
__device__ __forceinline__ bool route(const uint64_t* zt, unsigned tag, int E, int K, SelState& st,
                                      bool record, int token, unsigned long long* status,
                                      long lim) {
  constexpr int NK = 4 * R;
  const int lane = threadIdx.x & 63;
  float z[NK];
  const bool ok = poll_logits<R>(zt, tag, E, z, nullptr, lim);
  if (!ok && lane == 0) record_err(status, err_key(kPhSync, 0, 0, 0, 0));
  // the logits' copy for the exact path; non-finite logits are recorded on
  // a separate, rarely taken path
  bool bad = false;
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    const int e = lane + 64 * i;
    const bool in = e < E;
    st.zv[min(e, 256 * R - 1)] = in ? z[i] : 0.0f;
    bad |= in && !finite_f(z[i]);
  }
  if (record && __builtin_amdgcn_ballot_w64(bad) != 0) {
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int e = lane + 64 * i;
      if (e < E && !finite_f(z[i])) record_err(status, err_key(kPhLogit, token, 0, e, 0));
    }
  }
  uint32_t fk[NK], key[NK];
  int myid = 0;
  const bool unsafe = topk_on_logits<R>(z, E, K, lane, fk, myid);
  if (lane < K) st.ids[lane] = myid < E ? myid : E - 1;
  if (unsafe) {  // select on the exact probabilities
    uint32_t lmax = 0;
#pragma unroll
    for (int i = 0; i < NK; ++i) lmax = fk[i] > lmax ? fk[i] : lmax;
    const float m = key2f(wave_max_u32(lmax));
    float ev[NK];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      ev[i] = lane + 64 * i < E ? dm_expf(z[i] - m) : 0.0f;
      st.ev[lane + 64 * i] = ev[i];
    }
    wait_lds();
    __builtin_amdgcn_wave_barrier();
    const float inv = 1.0f / seq_sum(st.ev, 256 * R);
#pragma unroll
    for (int i = 0; i < NK; ++i) key[i] = lane + 64 * i < E ? f2u(ev[i] * inv) + 1u : 0u;
    uint32_t kr[3];
    select_keys<NK>(key, K, E, st.ids, false, kr);
  }
  return ok;
}

// The softmax numerators on another wave while wave 0 selects: max, e =
// exp(z - max) (zero-padded to 256R entries) to ev[] (src/layers/router.mojo:
// 140-183), and the shared-expert gate to misc[0].  Their sum is formed later
// (softmax_sum), off the routing path.
template <int R>
__device__ __forceinline__ void softmax_exp(const uint64_t* zt, unsigned tag, int E, SelState& st,
                                            bool record, int token, unsigned long long* status,
                                            long lim) {
  constexpr int NK = 4 * R;
  const int lane = threadIdx.x & 63;
  float z[NK];
  float gl = 0.0f;
  (void)poll_logits<R>(zt, tag, E, z, &gl, lim);  // wave 0 reports a timeout
  uint32_t lm = 0;
#pragma unroll
  for (int i = 0; i < NK; ++i)
    if (lane + 64 * i < E) {
      const uint32_t k = f2key(z[i]);
      lm = k > lm ? k : lm;
    }
  const float m = key2f(wave_max_u32(lm));
  if (record && lane == 0 && !finite_f(m)) record_err(status, err_key(kPhSoftmax, token, 0, 0, 0));
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    const int e = lane + 64 * i;
    float ev = 0.0f;
    if (e < E) {
      ev = dm_expf(z[i] - m);
      if (record && !finite_f(ev)) record_err(status, err_key(kPhSoftmax, token, 0, 1 + e, 0));
    }
    st.ev[e] = ev;
  }
  if (lane == 0) {
    // the shared-expert gate sigmoid(z_E) (src/layers/moe.mojo:70-100)
    if (record && !finite_f(gl)) record_err(status, err_key(kPhGate, token, 0, 0, kGkLogit));
    const float sg = dm_sigmoid(gl);
    if (record && (!finite_f(sg) || sg < 0.0f || sg > 1.0f))
      record_err(status, err_key(kPhGate, token, 0, 0, kGkRange));
    st.misc[0] = sg;
  }
}

// S = sum of ev[] in expert order (sequential, as src/layers/router.mojo:
// 140-183 sums it) on every lane of one wave, 1/S to misc[3], and the slot
// weights of the down tile: pw[k] = e_(ids[k]) / S (the routed probability
// p_k) and pw[K] = the shared gate.  Published by the caller's next barrier.
template <int R>
__device__ __forceinline__ void softmax_sum(int E, int K, SelState& st, bool record, int token,
                                            unsigned long long* status) {
  const int lane = threadIdx.x & 63;
  const float s = seq_sum(st.ev, 256 * R);
  const float inv = 1.0f / s;
  if (lane < K) st.pw[lane] = st.ev[st.ids[lane]] * inv;
  if (lane == 0) {
    if (record && (!(s > 0.0f) || !finite_f(s)))
      record_err(status, err_key(kPhSoftmax, token, 0, 1 + E, 0));
    st.misc[3] = inv;
    st.pw[K] = st.misc[0];
  }
}

// After routing, on one wave: the K probabilities p_k = e_k * (1/S), their
// (p desc, id asc) order and the checks of src/layers/topk.mojo:109-128.
// Lane k < K owns slot k and counts the slots ahead of it, which is its
// rank; the top-k sum is then formed in rank order.  Writes the ranks;
// `outputs` also writes ids / probs / shared gate in the reference's order.
// Runs in one workgroup after the gate/up tile.  Every slot's (p, id)
// is read as broadcast LDS vectors, all reads before the compares: a round
// trip per slot, or cross-lane reads into scalar registers, made this wave
// the last to reach the down tile's barrier.
__device__ __forceinline__ void finish_probs(int E, int K, SelState& st, bool record, int token,
                                             unsigned long long* status, int32_t* ids_out,
                                             float* probs_out, float* shg_out) {
  const int lane = threadIdx.x & 63;
  const float inv = st.misc[3];
  const int idk = lane < K ? st.ids[lane] : 0;
  const float pk = lane < K ? st.ev[idk] * inv : 0.0f;
  float* ps = st.scr;           // [32] p by slot
  float* sorted = st.scr + 32;  // [32] p by rank
  if (lane < K) ps[lane] = pk;
  wait_lds();
  __builtin_amdgcn_wave_barrier();
  int rank = 0;
  for (int jb = 0; jb < K; jb += 8) {  // K <= 32; entries past K are masked
    const float4 pa = *reinterpret_cast<const float4*>(ps + jb);
    const float4 pb = *reinterpret_cast<const float4*>(ps + jb + 4);
    const int4 ia = *reinterpret_cast<const int4*>(st.ids + jb);
    const int4 ib = *reinterpret_cast<const int4*>(st.ids + jb + 4);
    const float pj[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
    const int ij[8] = {ia.x, ia.y, ia.z, ia.w, ib.x, ib.y, ib.z, ib.w};
#pragma unroll
    for (int u = 0; u < 8; ++u)
      rank += (jb + u < K && (pj[u] > pk || (pj[u] == pk && ij[u] < idk))) ? 1 : 0;
  }
  if (lane < K) {
    sorted[rank] = pk;
    st.rank[lane] = rank;
    if (ids_out) {
      ids_out[rank] = idk;
      probs_out[rank] = pk;
    }
  }
  wait_lds();
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) {
    float sum_topk = 0.0f;  // in the reference's order
    for (int jb = 0; jb < K; jb += 8) {
      const float4 sa = *reinterpret_cast<const float4*>(sorted + jb);
      const float4 sb = *reinterpret_cast<const float4*>(sorted + jb + 4);
      const float sv[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (jb + u < K) sum_topk = sum_topk + sv[u];
    }
    if (ids_out) shg_out[0] = st.misc[0];
    if (record) {
      if (sum_topk > 1.00001f) record_err(status, err_key(kPhTopk, token, 0, 0, kTkSum));
      if (K < E && __builtin_fabsf(sum_topk - 1.0f) < 1e-6f) {
        float sum_all = 0.0f;
        for (int e2 = 0; e2 < E; ++e2) sum_all = sum_all + st.ev[e2] * inv;
        if (sum_all - sum_topk > 1e-5f) record_err(status, err_key(kPhTopk, token, 0, 0, kTkLeak));
      }
    }
  }
}

// The end of a workgroup when status_out is set (the host waits on these
// words instead of synchronising the stream): once this workgroup's output
// stores and its own error records (atomicMin on *status) have completed,
// thread 0 reads the key and stores it to status_out[blockIdx.x].  Each
// entry is the minimum of a set of records that holds at least the
// workgroup's own, so the minimum over all entries is the launch's
// first-error key: no counter, no atomic shared by the grid.  Launches
// without status_out pay nothing.
//
// The key is a system-scope release: the workgroup's outputs (written
// before the barrier by any of its waves) are visible to the host before the
// key that says they are complete, whatever memory type the host block has.
// It costs an L2 write-back per workgroup: the host-pointer call measured
// about 4.8 us slower than with a plain store of the key, whose ordering
// after the outputs the memory model does not promise.  (System-scope output
// stores waited on before the key, and a host-side sentinel check of every
// output word, measured as slow.)
__device__ __forceinline__ void end_workgroup(const unsigned long long* status,
                                              unsigned long long* status_out) {
  if (!status_out) return;
  wait_vm();
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_store(status_out + blockIdx.x, ld_coh_u64(status), __ATOMIC_RELEASE,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}

// The sum of the squares sq[0..n) one after another (rmsnorm's order,
// src/layers/rmsnorm.mojo:41-44) on one thread: a chain of n dependent adds
// (about 6.7 us at n = 2048 on MI355X; a double-buffered variant of the LDS
// reads measured slower).  n % 32 == 0.
__device__ __forceinline__ float seq_sum_squares(const float* sq, int n) {
  const float4* s4 = reinterpret_cast<const float4*>(sq);
  float a = 0.0f;
  for (int k = 0; k < n / 4; k += 8) {  // reads 8 float4 ahead of the adds
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = s4[k + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      a = a + v[u].x;
      a = a + v[u].y;
      a = a + v[u].z;
      a = a + v[u].w;
    }
  }
  return a;
}

// The same sum on one wave, every lane holding per <= kSeqPerLane of the
// squares in registers: lane l the elements l*per .. l*per + per - 1, read
// from sqT[i * 64 + l] = element l*per + i.  Round l adds every lane's
// values to the running sum; lane l's total is then the sum through its
// last element and is broadcast to all lanes for round l + 1.  The adds are
// the same dependent chain in the same order, without LDS reads on it:
// 2048 squares in about 4.2 us on MI355X against 6.5-7.2 us for the LDS
// loop (one chain of plain register adds: 3.8-4.7 us).
constexpr int kSeqPerLane = 32;
__device__ __forceinline__ float seq_sum_wave_rounds(const float* sqT, int per) {
  const int lane = threadIdx.x & 63;
  float r[kSeqPerLane];
#pragma unroll
  for (int i = 0; i < kSeqPerLane; ++i) r[i] = i < per ? sqT[i * 64 + lane] : 0.0f;
  float a = 0.0f;
  if (per == kSeqPerLane) {
    for (int l = 0; l < 64; ++l) {
#pragma unroll
      for (int i = 0; i < kSeqPerLane; ++i) a = a + r[i];
      a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), l));
    }
  } else {
    for (int l = 0; l < 64; ++l) {
#pragma unroll
      for (int i = 0; i < kSeqPerLane; ++i)
        if (i < per) a = a + r[i];
      a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), l));
    }
  }
  return a;
}

// The block-edge norm's sum of squares of x, left in red[0] (read by every
// thread after the final barrier; the barriers are LDS-only, so the weight
// loads in flight go on landing while the sum runs).  Thread tid holds x[8i .. 8i+7] for
// i = tid, tid + kThreads in xr.  sq: H floats of LDS.
// NORM 1: 256 strided partials and a halving tree (partial t + partial
//   t + wd, wd = 128 .. 1, the order of or_rmsnorm_tree256); the levels
//   below 64 are shuffles inside one wave, which pair the same partials.
// NORM 2: the reference's order, x_0^2 + x_1^2 + ... one add after another
//   (src/layers/rmsnorm.mojo:41-44): on one wave in rounds
//   (seq_sum_wave_rounds) when H <= 64 kSeqPerLane, else on one thread.
template <int NORM>
__device__ __forceinline__ void norm_sum_squares(const float4 (&xr)[2][2], int H, float* sq,
                                                 float* red) {
  const int tid = threadIdx.x;
  const bool rounds = NORM == 2 && H <= 64 * kSeqPerLane;
  const int per = H / 64;
#pragma unroll
  for (int ii = 0; ii < 2; ++ii) {
    const int i = tid + kThreads * ii;
    if (i < H / 8) {
      const float4 a = xr[ii][0], c = xr[ii][1];
      const float f[8] = {a.x * a.x, a.y * a.y, a.z * a.z, a.w * a.w,
                          c.x * c.x, c.y * c.y, c.z * c.z, c.w * c.w};
      if (rounds) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int k = 8 * i + j;
          sq[(k % per) * 64 + k / per] = f[j];
        }
      } else {
        reinterpret_cast<float4*>(sq)[2 * i] = make_float4(f[0], f[1], f[2], f[3]);
        reinterpret_cast<float4*>(sq)[2 * i + 1] = make_float4(f[4], f[5], f[6], f[7]);
      }
    }
  }
  lds_barrier();
  if constexpr (NORM == 1) {
    if (tid < 256) {
      float a = 0.0f;
      for (int k = tid; k < H; k += 256) a = a + sq[k];
      red[tid] = a;
    }
    lds_barrier();
    if (tid < 128) red[tid] = red[tid] + red[tid + 128];
    lds_barrier();
    if (tid < 64) {
      float v = red[tid] + red[tid + 64];
#pragma unroll
      for (int wd = 32; wd >= 1; wd >>= 1) v = v + __shfl_down(v, wd, 64);
      if (tid == 0) red[0] = v;
    }
  } else if (rounds) {
    if (tid < 64) {
      const float a = seq_sum_wave_rounds(sq, per);
      if (tid == 0) red[0] = a;
    }
  } else {
    if (tid == 0) red[0] = seq_sum_squares(sq, H);
  }
  lds_barrier();
}

// ---------------------------------------------------------------------------
// NORM: 0 the block input is x; 1 / 2 it is rmsnorm(x, gamma, eps) with the
// sum of squares as a 256-partial tree (1) or in element order (2, the
// reference's order, src/layers/rmsnorm.mojo:41-44).
template <int GQW, int R, int NORM>
__global__ __launch_bounds__(kThreads) void k_moe_decode(
    const float* __restrict__ x, const uint16_t* __restrict__ router,
    const float* __restrict__ gamma, int H_, int E_, int nx_, int nrw_, int nb_, LayerDev L,
    DecodePlan P,
    const float* __restrict__ residual, float* __restrict__ y, int32_t* __restrict__ ids_out,
    float* __restrict__ probs_out, float* __restrict__ shg_out, DecodeSync S,
    unsigned long long* status, int token, NormSpec nm, unsigned long long* status_out) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* xt = reinterpret_cast<float*>(smem + P.off_xt);
  uint4* xb2 = reinterpret_cast<uint4*>(smem + P.off_xb);
  float* red = reinterpret_cast<float*>(smem + P.off_red);
  float* yred = reinterpret_cast<float*>(smem + P.off_yred);
  unsigned char* sel = smem + P.off_sel;
  SelState st{reinterpret_cast<float*>(smem + P.off_zv), reinterpret_cast<float*>(smem + P.off_ev),
              reinterpret_cast<int*>(sel), reinterpret_cast<int*>(sel + 128),
              reinterpret_cast<float*>(sel + 256), reinterpret_cast<float*>(sel + 400),
              reinterpret_cast<float*>(sel + 512)};

  const int H = H_, K = L.K, E = E_;  // (preloaded entry arguments)
  const int b = blockIdx.x, nb = gridDim.x;
  const int tid = threadIdx.x, w = wave_id(), lane = tid & 63;
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

  // ---- entry: the router rows first (their arrival gates the logits, the
  // first hand-off), then x, then every other load that depends on neither
  // x nor routing (a wave's loads complete in order).  With the norm, x and
  // gamma come first instead: the norm's sum needs them, and runs while the
  // router rows land.
  uint4 rw[kRwMax];
  const int re = b * kRouterRows + (tid >> 4);
  auto load_rw = [&]() {
    if (router_wg && tid < kRouterRows * 16) {
      const uint4* wp =
          reinterpret_cast<const uint4*>(router + r16_index(H, min(re, E), tid & 15));
#pragma unroll
      for (int j8 = 0; j8 < kRwMax; ++j8) rw[j8] = wp[(size_t)min(j8, H / 128 - 1) * 16];
    }
  };
  if constexpr (NORM == 0) load_rw();
  float4 xr[2][2];
#pragma unroll
  for (int ii = 0; ii < 2; ++ii) {
    const int i = min(tid + kThreads * ii, H / 8 - 1);
    xr[ii][0] = reinterpret_cast<const float4*>(x)[2 * i];
    xr[ii][1] = reinterpret_cast<const float4*>(x)[2 * i + 1];
  }
  [[maybe_unused]] float4 gr[2][2];  // gamma of the same columns (the norm forms only)
  if constexpr (NORM != 0) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = min(tid + kThreads * ii, H / 8 - 1);
      gr[ii][0] = reinterpret_cast<const float4*>(gamma)[2 * i];
      gr[ii][1] = reinterpret_cast<const float4*>(gamma)[2 * i + 1];
    }
    load_rw();
  }
  const size_t matS = (size_t)L.Ish * H;
  const ExpertView sgv = {L.sgu_nib, L.sgu_sc, L.Ish, H};
  const ExpertView suv = {L.sgu_nib + matS / 2, L.sgu_sc + matS / kGroup, L.Ish, H};
  uint4 swg[GQW], swu[GQW];
  uint2 ssg[GQW], ssu[GQW];
  if (sh_tile < nsh) gu_load<GQW, false>(sgv, suv, sh_tile, swg, swu, ssg, ssu);
  const ExpertView sdv = {L.sd_nib, L.sd_sc, H, L.Ish};
  uint4 dw[kDownBatch];
  uint2 ds[kDownBatch];

  // ---- optional RMSNorm of x (the port block's post-attention norm,
  // src/layers/port_scheduler.mojo:383-385): every workgroup forms the sum of
  // squares itself while the weight loads above are in flight, then
  // x / denominator * gamma.  NORM 1: 256 strided partials and a halving tree;
  // NORM 2: one lane adds the squares in element order (rmsnorm.mojo:41-44).
  // The B-block area holds the squares and the reduction area the partials
  // until the staging below.
  if constexpr (NORM != 0) {
    norm_sum_squares<NORM>(xr, H, reinterpret_cast<float*>(xb2), red);
    const float denom = __builtin_sqrtf(red[0] / (float)H + nm.eps);
    auto nrm = [&](float4 v, float4 g) {
      return make_float4((v.x / denom) * g.x, (v.y / denom) * g.y, (v.z / denom) * g.z,
                         (v.w / denom) * g.w);
    };
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      xr[ii][0] = nrm(xr[ii][0], gr[ii][0]);
      xr[ii][1] = nrm(xr[ii][1], gr[ii][1]);
    }
    lds_barrier();  // the squares and partials are overwritten below
  }

  // ---- stage x: transposed fp32 (router chains) and bf16 hi/lo B blocks -----
  {
    bool bad = false;
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = tid + kThreads * ii;
      if (i < H / 8) {  // (loaded unconditionally above, used only when valid)
        const float f[8] = {xr[ii][0].x, xr[ii][0].y, xr[ii][0].z, xr[ii][0].w,
                            xr[ii][1].x, xr[ii][1].y, xr[ii][1].z, xr[ii][1].w};
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
    }
    if (bad && b == 0) record_err(status, err_key(kPhX, 0, 0, 0, 0));
  }
  __syncthreads();

  // ---- P1: router rows (wave 0); shared-expert gate/up tile ------------------
  if (router_wg && tid < kRouterRows * 16) router_compute(L, rw, re, xt, S.zt, n);
  for (int rr = b + nb; rr < P.n_router_wg; rr += nb) {  // only when the grid is small
    // (every workgroup is then a router workgroup and has staged xt)
    if (tid < kRouterRows * 16) {
      const int e2 = rr * kRouterRows + (tid >> 4);
      {
        const uint4* wp =
            reinterpret_cast<const uint4*>(router + r16_index(H, min(e2, E), tid & 15));
#pragma unroll
        for (int j8 = 0; j8 < kRwMax; ++j8) rw[j8] = wp[(size_t)min(j8, H / 128 - 1) * 16];
      }
      router_compute(L, rw, e2, xt, S.zt, n);
    }
  }
  for (int t = sh_tile; t < nsh; t += nb) {
    if (t != sh_tile) gu_load<GQW, false>(sgv, suv, t, swg, swu, ssg, ssu);
    gu_compute<GQW>(sgv, t, swg, swu, ssg, ssu, xb2, red,
                    S.ht + ((size_t)K << (P.ldh_log2 - 1)) + (size_t)t * (kTileRows / 2), n,
                    kPhShared, token, status);
  }

  // ---- P2: routing on wave 0, softmax numerators on wave 7 (every
  // workgroup computes the same result, so there is no broadcast hand-off) --
  if (w == 0) {
    const bool rok = route<R>(S.zt, n, E, K, st, b == 0, token, status, S.spin);
    if (lane == 0) st.misc[2] = rok ? 1.0f : 0.0f;
  } else if (w == kNormWave) {
    softmax_exp<R>(S.zt, n, E, st, b == 0, token, status, S.spin);
  }
  __syncthreads();
  const bool ok = st.misc[2] != 0.0f;

  // ---- P3: routed loads; softmax sum and slot weights; routed gate/up tile --
  const size_t matI = (size_t)L.I * H;
  auto gu_views = [&](int t, ExpertView& gv, ExpertView& uv) {
    const int e = __builtin_amdgcn_readfirstlane(st.ids[t / nrb]);
    gv = {L.gu_nib + (size_t)e * matI, L.gu_sc + (size_t)e * 2 * (matI / kGroup), L.I, H};
    uv = {gv.nib + matI / 2, gv.sc + matI / kGroup, L.I, H};
  };
  const size_t matD = (size_t)H * L.I;
  auto down_view = [&](int s) -> ExpertView {
    const int e = __builtin_amdgcn_readfirstlane(st.ids[s]);
    return {L.d_nib + (size_t)e * (matD / 2), L.d_sc + (size_t)e * (matD / kGroup), H, L.I};
  };
  uint4 gwg[GQW], gwu[GQW];
  uint2 gsg[GQW], gsu[GQW];
  ExpertView gv, uv;
  // every address first, then all loads of the phase back to back: with
  // address arithmetic between them the compiler waited for the gate/up
  // loads before issuing the down loads
  ExpertView dv[kDownBatch];
  int dgq[kDownBatch], dsl[kDownBatch];  // chunk within its slot; the slot (K: shared)
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i) {
    const int c = min(w + kWaves * i, nch - 1);
    const bool routed = c < nch_r;
    dv[i] = routed ? down_view(c / nGQI) : sdv;
    dgq[i] = routed ? c % nGQI : c - nch_r;
    dsl[i] = routed ? c / nGQI : K;
  }
  // (a workgroup past the routed tiles loads the last tile and ignores it)
  const int t0 = min(b, K * nrb - 1);
  gu_views(t0, gv, uv);
  gu_load<GQW, true>(gv, uv, t0 % nrb, gwg, gwu, gsg, gsu);
  // the softmax sum and the slot weights while the loads are in flight
  // (published by the first barrier of the gate/up tile, or the one below)
  if (w == kNormWave) softmax_sum<R>(E, K, st, b == 0, token, status);
  // The down chunks of this workgroup's output tile only once this wave's
  // gate/up bytes have landed: every workgroup's gate/up tile gates the h
  // hand-off, while the down chunks are needed only after it, so they do
  // not share the memory system with the gate/up loads (routed:
  // non-temporal; shared: cached).  Unconditional: loads under a branch
  // left their registers to be copied at the join, which waited for every
  // load in flight.  Workgroups without an output tile all read the first
  // chunk of the shared down matrix (one cached line set) and ignore it.
  wait_vm();
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i)
    load_chunk_nt(down_wg ? dv[i] : sdv, down_wg ? b : 0, down_wg ? dgq[i] : 0, lane, dw[i],
                  ds[i]);
  for (int t = b; t < K * nrb; t += nb) {
    if (t != b) {
      gu_views(t, gv, uv);
      gu_load<GQW, true>(gv, uv, t % nrb, gwg, gwu, gsg, gsu);
    }
    const int k = t / nrb;
    gu_compute<GQW>(gv, t % nrb, gwg, gwu, gsg, gsu, xb2, red,
                    S.ht + ((size_t)k << (P.ldh_log2 - 1)) + (size_t)(t % nrb) * (kTileRows / 2),
                    n, kPhExpert, token, status);
  }
  if (K * nrb <= b) __syncthreads();
  // the ranks, the outputs in the reference's order and the top-k checks:
  // in the first workgroup without an output tile (idle from here on), or
  // after the output tile in workgroup 0 when every workgroup has one
  const int fin_wg = nb > H / kTileRows ? H / kTileRows : 0;
  if (!down_wg) {
    if (b == fin_wg && w == 0)
      finish_probs(E, K, st, true, token, status, ids_out, probs_out, shg_out);
    end_workgroup(status, status_out);
    return;
  }

  // ---- P4: down projection of this workgroup's 16 output rows ---------------
  // Dequantize the down chunks first, then poll h (thread t reads words t,
  // t + 512, ...): the last gate/up tiles are published around the time the
  // dequantization ends, and a poll issued earlier comes back stale and
  // costs a round trip more.  (The empty asm statements pin the order: the
  // compiler would otherwise sink the dequantization below the poll.)
  const int lg = P.ldh_log2;
  const int lgw = lg - 1;                                          // words per slot: ldh / 2
  uint16_t* hbh = reinterpret_cast<uint16_t*>(smem + P.off_hb);  // [K+1][ldh] bf16 hi
  uint16_t* hbl = hbh + ((size_t)(K + 1) << lg);                  // [K+1][ldh] bf16 lo
  const int nwords = (K + 1) << lgw;
  auto pin = [&](int i) {
    asm volatile("" : "+v"(dw[i].x), "+v"(dw[i].y), "+v"(dw[i].z), "+v"(dw[i].w), "+v"(ds[i].x),
                 "+v"(ds[i].y)::"memory");
  };
  bf16x8 A[kDownBatch][4];
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i) pin(i);
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i)
    if (i < my_chunks)
#pragma unroll
      for (int c = 0; c < 4; ++c) A[i][c] = dequant8_shifted(word_of(dw[i], c), scale_of(ds[i], c));
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(A[i][c])::"memory");
  uint64_t hv[kHw];
#pragma unroll
  for (int u = 0; u < kHw; ++u) hv[u] = ld_coh_u64(S.ht + min(tid + kThreads * u, nwords - 1));
  {
    // Each word carries rows 2i, 2i+1 of one slot; they are staged scaled by
    // the slot's weight (p_k, or the shared gate) as bf16 hi / lo pairs, so
    // every chunk of the tile accumulates into the same MFMA chains.
    // Padding entries of a slot row are never written: they count as
    // staged; each thread re-polls only its own stale words and the
    // workgroup meets once at the end.
    uint32_t have = 0;
#pragma unroll
    for (int u = 0; u < kHw; ++u) {
      const int wd = min(tid + kThreads * u, nwords - 1), s2 = wd >> lgw;
      const int idx = 2 * (wd & ((1 << lgw) - 1));
      if (idx >= (s2 < K ? L.I : L.Ish)) have |= 1u << u;
    }
    const uint32_t all = (1u << min(kHw, (nwords - tid + kThreads - 1) / kThreads)) - 1u;
    have &= all;
    for (long spin = 0; spin < S.spin && ok; ++spin) {
#pragma unroll
      for (int u = 0; u < kHw; ++u) {
        if (!(have >> u & 1u) && (all >> u & 1u)) {
          const int wd = tid + kThreads * u;
          if (h2_current(hv[u], n)) {
            const int s2 = wd >> lgw, at = (s2 << lg) + 2 * (wd & ((1 << lgw) - 1));
            const float wgt = st.pw[s2];
            uint16_t h0, l0, h1, l1;
            split1(h2_v0(hv[u]) * wgt, h0, l0);
            split1(h2_v1(hv[u]) * wgt, h1, l1);
            *reinterpret_cast<uint32_t*>(hbh + at) = (uint32_t)h0 | ((uint32_t)h1 << 16);
            *reinterpret_cast<uint32_t*>(hbl + at) = (uint32_t)l0 | ((uint32_t)l1 << 16);
            have |= 1u << u;
          }
        }
      }
      if (have == all) break;
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int u = 0; u < kHw; ++u)  // unconditional loads stay in flight together
        hv[u] = ld_coh_u64(S.ht + min(tid + kThreads * u, nwords - 1));
    }
    if (!__syncthreads_and(have == all || !ok) && tid == 0)
      record_err(status, err_key(kPhSync, 0, 0, 0, 0));
  }
  // y = sum_k W_k (p_k h_k) + W_sh (g h_sh): every chunk of the wave into two
  // MFMA chains (the weights are in the staged operand); the next chunk's B
  // operand is read while the current one's products run
  f32x4 acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
  auto ld_chunk_b = [&](int s, int gq, bf16x8 (&B)[4]) {
    const uint16_t* hs = hbh + ((size_t)s << lg);
    const uint16_t* ls = hbl + ((size_t)s << lg);
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) B[cc] = ld_b2(hs, ls, (gq * 4 + cc) * 4 + q, j);
  };
  bf16x8 Bb[2][4];
  ld_chunk_b(dsl[0], dgq[0], Bb[0]);
#pragma unroll
  for (int i = 0; i < kDownBatch; ++i) {
    if (i < my_chunks) {
      if (i + 1 < kDownBatch) ld_chunk_b(dsl[min(i + 1, kDownBatch - 1)],
                                         dgq[min(i + 1, kDownBatch - 1)], Bb[(i + 1) & 1]);
      const bf16x8(&B)[4] = Bb[i & 1];
      acc0 = mfma16(A[i][0], B[0], acc0);
      acc1 = mfma16(A[i][1], B[1], acc1);
      acc0 = mfma16(A[i][2], B[2], acc0);
      acc1 = mfma16(A[i][3], B[3], acc1);
    }
  }
  // chunks beyond the register batch (only when a wave has more than
  // kDownBatch chunks)
  for (int base = kDownBatch; base < my_chunks; base += kDownBatch) {
#pragma unroll
    for (int i = 0; i < kDownBatch; ++i) {
      const int c = w + kWaves * (base + i);
      if (base + i < my_chunks) {
        const bool routed = c < nch_r;
        const ExpertView v = routed ? down_view(c / nGQI) : sdv;
        load_chunk_nt(v, b, routed ? c % nGQI : c - nch_r, lane, dw[i], ds[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < kDownBatch; ++i)
      if (base + i < my_chunks)
#pragma unroll
        for (int c = 0; c < 4; ++c) A[i][c] = dequant8_shifted(word_of(dw[i], c), scale_of(ds[i], c));
#pragma unroll
    for (int i = 0; i < kDownBatch; ++i) {
      if (base + i < my_chunks) {
        const int c = w + kWaves * (base + i);
        const int s = c < nch_r ? c / nGQI : K, gq = c < nch_r ? c % nGQI : c - nch_r;
        bf16x8 B[4];
        ld_chunk_b(s, gq, B);
        acc0 = mfma16(A[i][0], B[0], acc0);
        acc1 = mfma16(A[i][1], B[1], acc1);
        acc0 = mfma16(A[i][2], B[2], acc0);
        acc1 = mfma16(A[i][3], B[3], acc1);
      }
    }
  }
  f32x4 acc;
#pragma unroll
  for (int r = 0; r < 4; ++r) acc[r] = acc0[r] + acc1[r];
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
  if (b == fin_wg && fin_wg == 0 && w == 0)
    finish_probs(E, K, st, true, token, status, ids_out, probs_out, shg_out);
  end_workgroup(status, status_out);
}

// ---------------------------------------------------------------------------
// The XCD-sliced form of the same launch.  The dispatcher places the
// workgroups of a launch on the nx XCDs in rotation (b on XCD (b + r) % nx,
// with r varying between launches), so every XCD holds nb / nx of them; each
// workgroup reads its XCD from the hardware.  Hand-offs between workgroups
// of one XCD go
// through that XCD's L2 (plain stores, agent-scope polls: about a quarter of
// the round trip of a hand-off through memory), so the expert work is cut
// along XCDs:
//
//   pair p = (slot k, 128-row slice c of I) for the K routed slots, then the
//   shared expert's slices.  XCD x owns the pairs p = x, x + nx, ...:
//   - their gate/up tiles (8 tiles of 16 rows per pair, one per workgroup of
//     the XCD at the Qwen3.6 shape), h published XCD-locally;
//   - columns 128c..128c+127 of their down matrices for every output row:
//     workgroup m of the XCD owns output tiles m*rpw..m*rpw+rpw-1, and its
//     waves take the (tile, pair) A16 tiles, so each wave accumulates one
//     output tile over its pairs.
//   The XCD's partial output vector (its pairs' share of sum_k p_k W_k h_k +
//   g W_sh h_sh) is published once; the final sum of the nx partials (XCD
//   order) plus the residual forms y, rows spread over all workgroups.
//
// Every XCD forms all E+1 router logits itself (its workgroups share the
// rows) and hands them on through its L2, so routing needs no hand-off
// between XCDs; every workgroup then selects the same top-k as in the
// original form.  The shared expert needs no routing: its h rows are formed
// before the routing decision, two per workgroup, and handed to the XCDs
// holding its slices through memory.
constexpr int kXsR = 2;   // routed (output tile, pair) down tiles per wave, A operands in registers
constexpr int kXsS = 1;   // shared-expert down tiles per wave
constexpr int kXsHw = 2;     // XCD-local h words per thread
constexpr int kXsRouterWaves = 4;  // waves holding router rows (4 rows each)

__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xFu;
}

#ifdef DM_PHASE_TRACE
// Tracing build: workgroup b (< 256) of a launch with S.trace = slot stores
// wall_clock64() at point k to g_phase_trace[(slot * 256 + b) * 8 + k]:
// 0 entry, 1 norm sum done, 2 x staged, 3 routing done, 4 h staged,
// 5 partial published, 6 partials polled, 7 end; in k_moe_tokens: 0 entry,
// 1 x staged, 2 routing done, 3 gate/up tasks done, 4 h staged, 5 down
// products done, 7 end.
__device__ unsigned long long g_phase_trace[kTraceSlots * 256 * kTracePoints];
#define DM_TR(k)                                                                      \
  do {                                                                                \
    if (S.trace >= 0 && S.trace < kTraceSlots && blockIdx.x < 256 && threadIdx.x == 0) \
      g_phase_trace[((size_t)S.trace * 256 + blockIdx.x) * kTracePoints + (k)] =       \
          wall_clock64();                                                             \
  } while (0)
#else
#define DM_TR(k) \
  do {           \
  } while (0)
#endif

template <int GQW, int R, int NORM>
__global__ __launch_bounds__(kThreads) void k_moe_decode_xs(
    const float* __restrict__ x, const uint16_t* __restrict__ router,
    const float* __restrict__ gamma, int H_, int E_, int nx_, int nrw_, int nb_, LayerDev L,
    DecodePlan P,
    const float* __restrict__ residual, float* __restrict__ y, int32_t* __restrict__ ids_out,
    float* __restrict__ probs_out, float* __restrict__ shg_out, DecodeSync S,
    unsigned long long* status, int token, NormSpec nm, unsigned long long* status_out) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  DM_TR(0);
  // ---- entry: router rows, x, gamma (with the norm: x, gamma, router
  // rows, as in the original form), requested first, from the preloaded
  // leading arguments only --------------------------------------------------
  const int H = H_, E = E_;
  const int b = blockIdx.x, nb = nb_;
  const int tid = threadIdx.x, w = wave_id(), lane = tid & 63;
  // The dispatcher hands workgroups to the XCDs in rotation, starting at an
  // XCD that varies from launch to launch: the XCD a workgroup runs on is
  // read from the hardware, and b / nx numbers the workgroups of one XCD.
  const int nx = nx_, nmx = nb / nx, m = b / nx;
  // router rows of this workgroup: every XCD forms all E+1 logits itself, so
  // routing needs no hand-off between XCDs; wave w < nrw, lane group g owns
  // row m + nmx*(4w + g)
  const int nrw = nrw_;
  uint4 rw[kRwMax];
  const int re = m + nmx * (4 * w + (lane >> 4));
  auto load_rw = [&]() {
    if (w < nrw) {
      const uint4* wp =
          reinterpret_cast<const uint4*>(router + r16_index(H, min(re, E), lane & 15));
#pragma unroll
      for (int j8 = 0; j8 < kRwMax; ++j8) rw[j8] = wp[(size_t)min(j8, H / 128 - 1) * 16];
    }
  };
  if constexpr (NORM == 0) load_rw();
  float4 xr[2][2];
#pragma unroll
  for (int ii = 0; ii < 2; ++ii) {
    const int i = min(tid + kThreads * ii, H / 8 - 1);
    xr[ii][0] = reinterpret_cast<const float4*>(x)[2 * i];
    xr[ii][1] = reinterpret_cast<const float4*>(x)[2 * i + 1];
  }
  [[maybe_unused]] float4 gr[2][2];
  if constexpr (NORM != 0) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = min(tid + kThreads * ii, H / 8 - 1);
      gr[ii][0] = reinterpret_cast<const float4*>(gamma)[2 * i];
      gr[ii][1] = reinterpret_cast<const float4*>(gamma)[2 * i + 1];
    }
    load_rw();
  }
  float* xt = reinterpret_cast<float*>(smem + P.off_xt);
  uint4* xb2 = reinterpret_cast<uint4*>(smem + P.off_xb);
  float* red = reinterpret_cast<float*>(smem + P.off_red);
  float* yred = reinterpret_cast<float*>(smem + P.off_yred);
  float* fin = reinterpret_cast<float*>(smem + P.off_fin);
  uint16_t* hbh = reinterpret_cast<uint16_t*>(smem + P.off_hb);  // [npx][128] bf16 hi
  uint16_t* hbl = hbh + (size_t)P.xs_npx * kQuadCols;             // [npx][128] bf16 lo
  unsigned char* sel = smem + P.off_sel;
  SelState st{reinterpret_cast<float*>(smem + P.off_zv), reinterpret_cast<float*>(smem + P.off_ev),
              reinterpret_cast<int*>(sel), reinterpret_cast<int*>(sel + 128),
              reinterpret_cast<float*>(sel + 256), reinterpret_cast<float*>(sel + 400),
              reinterpret_cast<float*>(sel + 512)};

  const int K = L.K;
  const int q = lane >> 4, j = lane & 15;
  const unsigned n = S.n;
  const int xc = (int)xcc_id();
  const int nT = L.I / kQuadCols, KT = K * nT, NP = KT + L.Ish / kQuadCols;
  const int npx = NP > xc ? (NP - xc + nx - 1) / nx : 0;   // pairs of this XCD
  const int nrpx = KT > xc ? (KT - xc + nx - 1) / nx : 0;  // routed ones (they come first)
  const int ntr = nrpx * 8;  // routed gate/up tiles of 16 rows on this XCD
  const int rpw = P.xs_rpw, rb0 = m * rpw, nrt = H / kTileRows;
  const int my_rt = max(0, min(rpw, nrt - rb0));  // output tiles of this workgroup
  // this wave's down tiles: items jj = 0, 1, ...: output tile rb0 + ri of
  // pair lp0 + lstep*jj (rpw divides the wave count, so ri is fixed)
  const int ri = w & (rpw - 1), lp0 = w / rpw, lstep = kWaves / rpw;
  const int nit = (ri < my_rt && lp0 < npx) ? (npx - lp0 + lstep - 1) / lstep : 0;
  const int nit_r = (ri < my_rt && lp0 < nrpx) ? min(nit, (nrpx - lp0 + lstep - 1) / lstep) : 0;
  const int nit_s = nit - nit_r;  // the plan keeps nit_r <= kXsR and nit_s <= kXsS
  const int rbc = min(rb0 + ri, nrt - 1);  // a valid output tile for unused load slots
  const int zs = 256 * R + 64;            // logit words per XCD
  uint64_t* zl = S.zt + (size_t)xc * zs;  // this XCD's logits
  if (xc >= nx) {  // (never: the count was probed on this device)
    if (tid == 0) record_err(status, err_key(kPhSync, 0, 0, 1, 0));
    end_workgroup(status, status_out);
    return;
  }

  const size_t matS = (size_t)L.Ish * H;
  const ExpertView sgv = {L.sgu_nib, L.sgu_sc, L.Ish, H};
  const ExpertView suv = {L.sgu_nib + matS / 2, L.sgu_sc + matS / kGroup, L.Ish, H};
  const ExpertView sdv = {L.sd_nib, L.sd_sc, H, L.Ish};
  // down A operands: routed tiles jr (pair lp0 + lstep*jr), then the shared
  // tile (pair lp0 + lstep*nit_r).  Every load slot is always issued (an
  // unused slot re-reads a valid tile): loads under a branch make the
  // compiler wait for every load in flight before their first use.
  uint4 dwr[kXsR], dws;
  uint2 dsr[kXsR], dss;
  bf16x8 Ar[kXsR][4], As[4];
  // The shared expert's h: workgroup b forms rows 2b and 2b+1 (one hand-off
  // word) as wave-level dot products, wave 2 row 2b and wave 3 row 2b+1 (gate
  // and up each; at the Qwen3.6 shape neither holds router rows outside
  // workgroup 0), lane = one 16-byte piece of the row (groups 4gq..4gq+3,
  // columns 8q..8q+7 of each).  Spread over every workgroup it costs each
  // one a few hundred instructions before routing, on SIMDs the router
  // chains do not use.
  const bool shw = w == 2 || w == 3;
  const int nGQs = H / kQuadCols;
  uint4 shc[2];
  uint2 shs[2];
  if (shw) {
    const int r = min(2 * b + (w - 2), L.Ish - 1);
    const int pc = min(lane, nGQs * 4 - 1);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const ExpertView& v = mt ? suv : sgv;
      shc[mt] = *reinterpret_cast<const uint4*>(
          v.nib + a16_nib_offset(nGQs, r >> 4, pc >> 2, (pc & 3) * 16 + (r & 15)));
      shs[mt] = *reinterpret_cast<const uint2*>(v.sc + a16_sc_offset(nGQs, r >> 4, pc >> 2, r & 15));
    }
  }
  // the shared down operand (dequantized after routing)
  load_chunk(sdv, rbc, nit_s > 0 ? xc + nx * (lp0 + lstep * nit_r) - KT : 0, lane, dws, dss);
  float* shv = reinterpret_cast<float*>(sel + 448);  // [4] the four dot products

  // ---- optional RMSNorm of x (as in the original form) ---------------------
  if constexpr (NORM != 0) {
    norm_sum_squares<NORM>(xr, H, reinterpret_cast<float*>(xb2), red);
    DM_TR(1);
    const float denom = __builtin_sqrtf(red[0] / (float)H + nm.eps);
    auto nrm = [&](float4 v, float4 g) {
      return make_float4((v.x / denom) * g.x, (v.y / denom) * g.y, (v.z / denom) * g.z,
                         (v.w / denom) * g.w);
    };
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      xr[ii][0] = nrm(xr[ii][0], gr[ii][0]);
      xr[ii][1] = nrm(xr[ii][1], gr[ii][1]);
    }
    lds_barrier();  // the squares and partials are overwritten below
  }

  // ---- stage x --------------------------------------------------------------
  {
    bool bad = false;
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = tid + kThreads * ii;
      if (i < H / 8) {
        const float f[8] = {xr[ii][0].x, xr[ii][0].y, xr[ii][0].z, xr[ii][0].w,
                            xr[ii][1].x, xr[ii][1].y, xr[ii][1].z, xr[ii][1].w};
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) bad |= !finite_f(f[k2]);
        {
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
    }
    if (bad && b == 0) record_err(status, err_key(kPhX, 0, 0, 0, 0));
  }
  __syncthreads();
  DM_TR(2);

  // ---- router rows (XCD-local logits), the shared expert's rows ---------------
  if (w < nrw) router_compute<true>(L, rw, re, xt, zl, n);
  if (shw) {
    float a[2] = {0.0f, 0.0f};  // gate, up
    if (lane < nGQs * 4) {
      const int gq = lane >> 2, q = lane & 3;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int blk = (4 * gq + c) * 4 + q;  // x columns 32(4gq+c) + 8q .. +7
        const uint4 xh = xb2[2 * blk], xl = xb2[2 * blk + 1];
        const uint32_t hd[4] = {xh.x, xh.y, xh.z, xh.w};
        const uint32_t ld[4] = {xl.x, xl.y, xl.z, xl.w};
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const uint4 wv =
              __builtin_bit_cast(uint4, dequant8(word_of(shc[mt], c), scale_of(shs[mt], c)));
          const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            a[mt] = __builtin_fmaf(bf16lo(wd[u]), bf16lo(hd[u]) + bf16lo(ld[u]), a[mt]);
            a[mt] = __builtin_fmaf(bf16hi(wd[u]), bf16hi(hd[u]) + bf16hi(ld[u]), a[mt]);
          }
        }
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      a[0] = a[0] + __shfl_xor(a[0], off);
      a[1] = a[1] + __shfl_xor(a[1], off);
    }
    if (lane == 0) {
      shv[w - 2] = a[0];      // gate of row 2b + (w - 2)
      shv[2 + w - 2] = a[1];  // up
    }
  }

  // ---- routing (as in the original form) ------------------------------------
  if (w == 0) {
    const bool rok = route<R>(zl, n, E, K, st, b == 0, token, status, S.spin);
    if (lane == 0) st.misc[2] = rok ? 1.0f : 0.0f;
  } else if (w == kNormWave) {
    softmax_exp<R>(zl, n, E, st, b == 0, token, status, S.spin);
  }
  __syncthreads();
  DM_TR(3);
  const bool ok = st.misc[2] != 0.0f;

  // ---- routed loads: this workgroup's gate/up tile, this wave's down tiles ---
  const size_t matI = (size_t)L.I * H, matD = (size_t)H * L.I;
  auto task_views = [&](int tr, ExpertView& gv, ExpertView& uv) -> int {
    const int p = xc + nx * (tr / 8);
    const int e = __builtin_amdgcn_readfirstlane(st.ids[p / nT]);
    gv = {L.gu_nib + (size_t)e * matI, L.gu_sc + (size_t)e * 2 * (matI / kGroup), L.I, H};
    uv = {gv.nib + matI / 2, gv.sc + matI / kGroup, L.I, H};
    return (p % nT) * 8 + tr % 8;
  };
  // this wave's routed down tiles first: they are few bytes, land first and
  // are dequantized while the gate/up bytes are still in flight
#pragma unroll
  for (int jr = 0; jr < kXsR; ++jr) {
    ExpertView dv = sdv;
    int gq = 0;
    if (nit_r > 0) {
      const int p = xc + nx * (lp0 + lstep * min(jr, nit_r - 1));
      const int e = __builtin_amdgcn_readfirstlane(st.ids[p / nT]);
      dv = {L.d_nib + (size_t)e * (matD / 2), L.d_sc + (size_t)e * (matD / kGroup), H, L.I};
      gq = p % nT;
    }
    load_chunk_nt(dv, rbc, gq, lane, dwr[jr], dsr[jr]);
  }
  uint4 gwg[GQW], gwu[GQW];
  uint2 gsg[GQW], gsu[GQW];
  ExpertView gv = sgv, uv = suv;
  int grb = 0;
  if (ntr > 0) grb = task_views(min(m, ntr - 1), gv, uv);  // (a spare workgroup re-reads a tile)
  gu_load<GQW, true>(gv, uv, grb, gwg, gwu, gsg, gsu);

  // while the routed loads are in flight: the shared rows' h (its thread
  // would otherwise issue its loads late) and the shared down operand
  if (tid == 64 && 2 * b < L.Ish) {
    // h of shared rows 2b, 2b+1 (swiglu_forward's gate, up, product checks)
    const int r0 = 2 * b;
    const float g0 = shv[0], g1 = shv[1], u0 = shv[2], u1 = shv[3];
    const float h0 = dm_silu(g0) * u0, h1 = dm_silu(g1) * u1;
    auto chk = [&](int r, float g, float u, float hh) {
      if (!finite_f(g) || !finite_f(u) || !finite_f(hh))
        record_err(status, err_key(kPhShared, token, 0, r,
                                   !finite_f(g) ? kEkGate : !finite_f(u) ? kEkUp : kEkH));
    };
    chk(r0, g0, u0, h0);
    chk(r0 + 1, g1, u1, h1);
    // read by the XCD holding the shared slice r0 / 128 (any XCD): agent scope
    st_coh_u64(S.hl + (size_t)(KT + r0 / kQuadCols) * 64 + (r0 % kQuadCols) / 2,
               pack_h2(n, h0, h1));
  }

#pragma unroll
  for (int c = 0; c < 4; ++c) As[c] = dequant8(word_of(dws, c), scale_of(dss, c));
  // the softmax sum and slot weights while the loads are in flight; the
  // ranks and outputs in the reference's order in one workgroup
  const int fin_wg = nb - 1;
  if (w == kNormWave) {
    softmax_sum<R>(E, K, st, b == 0, token, status);
    if (b == fin_wg)
      finish_probs(E, K, st, true, token, status, ids_out, probs_out, shg_out);
  }
#pragma unroll
  for (int jr = 0; jr < kXsR; ++jr)
#pragma unroll
    for (int c = 0; c < 4; ++c) Ar[jr][c] = dequant8(word_of(dwr[jr], c), scale_of(dsr[jr], c));
  // (the empty asm statements keep the dequantization here, ahead of the
  // gate/up tile; the compiler would otherwise sink it to the products)
#pragma unroll
  for (int jr = 0; jr < kXsR; ++jr)
#pragma unroll
    for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(Ar[jr][c])::"memory");
#pragma unroll
  for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(As[c])::"memory");
  for (int tr = m; tr < ntr; tr += nmx) {
    if (tr != m) {
      grb = task_views(tr, gv, uv);
      gu_load<GQW, true>(gv, uv, grb, gwg, gwu, gsg, gsu);
    }
    const int p = xc + nx * (tr / 8);
    gu_compute<GQW, true>(gv, grb, gwg, gwu, gsg, gsu, xb2, red,
                          S.hl + (size_t)p * 64 + (tr % 8) * 8, n, kPhExpert, token, status);
  }
  if (m >= ntr) __syncthreads();  // publishes the slot weights

  // ---- down: this XCD's pairs, columns of its slices, this workgroup's rows --
  {
    // h of every pair of the XCD, staged scaled by its slot's weight (p_k,
    // or the shared gate) as bf16 hi / lo pairs; stale words are polled
    // again.
    const int nwords = my_rt > 0 ? npx * 64 : 0;
    uint64_t hv[kXsHw];
    uint32_t have = 0, all = 0;
    if (nwords > 0) {
#pragma unroll
      for (int u = 0; u < kXsHw; ++u) {
        const int wd = min(tid + kThreads * u, nwords - 1);
        if (tid + kThreads * u < nwords) all |= 1u << u;
        hv[u] = ld_coh_u64(S.hl + (size_t)(xc + nx * (wd >> 6)) * 64 + (wd & 63));
      }
    }
    for (long spin = 0; spin < S.spin && ok && have != all; ++spin) {
#pragma unroll
      for (int u = 0; u < kXsHw; ++u) {
        if ((all >> u & 1u) && !(have >> u & 1u) && h2_current(hv[u], n)) {
          const int wd = tid + kThreads * u, lp = wd >> 6, iw = wd & 63;
          const int p = xc + nx * lp;
          const float wgt = st.pw[p < KT ? p / nT : K];
          uint16_t h0, l0, h1, l1;
          split1(h2_v0(hv[u]) * wgt, h0, l0);
          split1(h2_v1(hv[u]) * wgt, h1, l1);
          const int at = lp * kQuadCols + 2 * iw;
          *reinterpret_cast<uint32_t*>(hbh + at) = (uint32_t)h0 | ((uint32_t)h1 << 16);
          *reinterpret_cast<uint32_t*>(hbl + at) = (uint32_t)l0 | ((uint32_t)l1 << 16);
          have |= 1u << u;
        }
      }
      if (have == all) break;
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int u = 0; u < kXsHw; ++u) {
        const int wd = min(tid + kThreads * u, nwords - 1);
        hv[u] = ld_coh_u64(S.hl + (size_t)(xc + nx * (wd >> 6)) * 64 + (wd & 63));
      }
    }
    if (!__syncthreads_and(have == all || !ok) && tid == 0)
      record_err(status, err_key(kPhSync, 0, 0, 2, 0));
  }
  DM_TR(4);
  f32x4 acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
  auto tile_mfma = [&](const bf16x8 (&Aop)[4], int lp) {
    const uint16_t* hs = hbh + lp * kQuadCols;
    const uint16_t* ls = hbl + lp * kQuadCols;
    bf16x8 B[4];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) B[cc] = ld_b2(hs, ls, cc * 4 + q, j);
    acc0 = mfma16(Aop[0], B[0], acc0);
    acc1 = mfma16(Aop[1], B[1], acc1);
    acc0 = mfma16(Aop[2], B[2], acc0);
    acc1 = mfma16(Aop[3], B[3], acc1);
  };
#pragma unroll
  for (int jr = 0; jr < kXsR; ++jr)
    if (jr < nit_r) tile_mfma(Ar[jr], lp0 + lstep * jr);
  if (nit_s > 0) tile_mfma(As, lp0 + lstep * nit_r);
  {
    f32x4 acc;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = acc0[r] + acc1[r];
    fold_cols(acc);
    if (j == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) yred[w * 16 + 4 * q + r] = acc[r];
    }
  }
  __syncthreads();
  if (npx > 0 && tid < kTileRows * my_rt) {
    // the XCD's partial of rows (rb0 + tid/16)*16 + tid%16, waves in order
    const int t2 = tid >> 4, r = tid & 15;
    float s = 0.0f;
    for (int w2 = t2; w2 < kWaves; w2 += rpw) s = s + yred[w2 * 16 + r];
    st_coh_u64(S.pt + (size_t)xc * H + (rb0 + t2) * kTileRows + r, ((uint64_t)n << 32) | f2u(s));
  }
  DM_TR(5);

  // ---- the final sum: rows b*rpf .. b*rpf + rpf - 1 -------------------------
  {
    const int rpf = P.xs_rpf, nxa = min(nx, NP);
    const int r0 = b * rpf, nfr = max(0, min(rpf, H - r0));
    bool fok = true;
    if (tid < nxa * rpf && tid % rpf < nfr) {
      const int xx = tid / rpf, rr = tid % rpf;
      const uint64_t* src = S.pt + (size_t)xx * H + r0 + rr;
      // two polls in flight: while the older one is checked the newer one
      // travels, so a partial is seen about half a round trip sooner
      uint64_t v = ld_coh_u64(src), nv = ld_coh_u64(src);
      for (long spin = 0; spin < S.spin && ok && (uint32_t)(v >> 32) != n; ++spin) {
        v = nv;
        nv = ld_coh_u64(src);
      }
      fok = (uint32_t)(v >> 32) == n;
      fin[xx * rpf + rr] = u2f((uint32_t)v);
    }
    if (!__syncthreads_and(fok || !ok) && tid == 0)
      record_err(status, err_key(kPhSync, 0, 0, 3, 0));
    DM_TR(6);
    if (tid < nfr) {
      const int d = r0 + tid;
      float total = 0.0f;
      for (int xx = 0; xx < nxa; ++xx) total = total + fin[xx * rpf + tid];
      if (residual) total = total + residual[d];
      if (!finite_f(total)) record_err(status, err_key(kPhExpert, token, 0, 0, kEkRecheck));
      y[d] = total;
    }
  }
  DM_TR(7);
  end_workgroup(status, status_out);
}

// ---------------------------------------------------------------------------
// Several tokens in one launch (launch_moe_tokens): the XCD-sliced grid, XCD
// c taking token c (T <= nx) and its whole block on its own nmx = nb / nx
// workgroups (workgroup m = b / nx of the XCD), so every hand-off stays in
// that XCD's L2 and no partial output crosses XCDs:
//   routing  as in k_moe_decode_xs: the XCD forms all E+1 logits and every
//            workgroup selects the top k itself;
//   gate/up  the token's NP pairs (a routed slot's or the shared expert's
//            128-row slice of I) x 8 tiles of 16 rows: tasks m, m + nmx, ...
//            of workgroup m, streamed through an LDS ring by direct-to-LDS
//            loads; each wave's partial sums of every task kept in LDS, then
//            one barrier and every task's h formed and published
//            XCD-locally, one tagged word per value;
//   down     workgroup m owns the output tiles m rpw ..; wave w takes tile
//            w % rpw and the pairs w / rpw, + kWaves / rpw, ... (A16 chunks
//            kTokRing ahead, the first ones requested right after routing),
//            with h of every pair staged in LDS scaled by its slot's weight
//            (p_k, or the shared gate); y = the waves' sums (+ residual).
// Routing is bit for bit that of the single-token kernels (the same chains,
// tree and selection); the expert sums run in another order, within the
// same tolerance.  Loads past a workgroup's or wave's last task read fixed
// bytes of the shared expert instead (every such request hits the same
// lines), so that no load is issued under a branch.
constexpr int kTokHw = 12;   // h words per thread in the staging poll
constexpr int kTokRing = 4;  // down chunks per wave in flight
constexpr int kTokGu = 3;    // gate/up task slots of the LDS ring
constexpr int kTokSlotW = 4 * 1024 + 4 * 128;  // one wave's part of a slot
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

template <int GQW, int R>
__global__ __launch_bounds__(kThreads) void k_moe_tokens(
    const float* __restrict__ x, const uint16_t* __restrict__ router, int H_, int E_, int nx_,
    int nrw_, int nb_, int T, LayerDev L, DecodePlan P, const float* __restrict__ residual,
    float* __restrict__ y, int32_t* __restrict__ ids_out, float* __restrict__ probs_out,
    float* __restrict__ shg_out, DecodeSync S, unsigned long long* status) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  DM_TR(0);
  const int H = H_, E = E_;
  const int b = blockIdx.x, nb = nb_;
  const int tid = threadIdx.x, w = wave_id(), lane = tid & 63;
  const int nx = nx_, nmx = nb / nx, m = b / nx;
  // router rows of this workgroup (as in k_moe_decode_xs)
  const int nrw = nrw_;
  const int re = m + nmx * (4 * w + (lane >> 4));
  float* xt = reinterpret_cast<float*>(smem + P.off_xt);
  uint4* xb2 = reinterpret_cast<uint4*>(smem + P.off_xb);
  float* yred = reinterpret_cast<float*>(smem + P.tok_off_yred);
  const int K = L.K;
  const int nT = L.I / kQuadCols, KT = K * nT, NP = KT + L.Ish / kQuadCols;
  uint16_t* hbh = reinterpret_cast<uint16_t*>(smem + P.tok_off_hb);  // [NP][128] bf16 hi
  uint16_t* hbl = hbh + (size_t)NP * kQuadCols;                      // [NP][128] bf16 lo
  unsigned char* sel = smem + P.off_sel;
  SelState st{reinterpret_cast<float*>(smem + P.off_zv), reinterpret_cast<float*>(smem + P.off_ev),
              reinterpret_cast<int*>(sel), reinterpret_cast<int*>(sel + 128),
              reinterpret_cast<float*>(sel + 256), reinterpret_cast<float*>(sel + 400),
              reinterpret_cast<float*>(sel + 512)};
  const int q = lane >> 4, j = lane & 15;
  const unsigned n = S.n;
  const int xc = (int)xcc_id();
  const int rpw = P.xs_rpw, rb0 = m * rpw, nrt = H / kTileRows;
  const int my_rt = max(0, min(rpw, nrt - rb0));  // output tiles of this workgroup
  const int ri = w & (rpw - 1), lp0 = w / rpw, lstep = kWaves / rpw;
  const int nit = (ri < my_rt && lp0 < NP) ? (NP - lp0 + lstep - 1) / lstep : 0;
  const int rbc = min(rb0 + ri, nrt - 1);
  const int zs = 256 * R + 64;
  const int ntask = NP * (kQuadCols / kTileRows);
  // pair p: the shared expert's slices first (their tasks need no routing,
  // and task m of every workgroup is one of them), then the routed slots'
  const int nGS = L.Ish / kQuadCols;
  auto pair_of = [&](int p, int& shared, int& slot, int& slice) {
    shared = p < nGS;
    slot = shared ? K : (p - nGS) / nT;
    slice = shared ? p : (p - nGS) % nT;
  };
  const size_t matI = (size_t)L.I * H, matD = (size_t)H * L.I, matS = (size_t)L.Ish * H;
  const ExpertView sgv = {L.sgu_nib, L.sgu_sc, L.Ish, H};
  const ExpertView suv = {L.sgu_nib + matS / 2, L.sgu_sc + matS / kGroup, L.Ish, H};
  const ExpertView sdv = {L.sd_nib, L.sd_sc, H, L.Ish};
  if (xc >= nx) {  // (never: the count was probed on this device)
    if (tid == 0) record_err(status, err_key(kPhSync, 0, 0, 1, 0));
    return;
  }
  // token t = xc (T <= nx: at most one token per XCD; the other XCDs' workgroups end here)
  const int t = xc;
  if (t >= T) return;
  {
    uint4 rw[kRwMax];
    if (w < nrw) {
      const uint4* wp =
          reinterpret_cast<const uint4*>(router + r16_index(H, min(re, E), lane & 15));
#pragma unroll
      for (int j8 = 0; j8 < kRwMax; ++j8) rw[j8] = wp[(size_t)min(j8, H / 128 - 1) * 16];
    }
    uint64_t* zl = S.zt + (size_t)t * zs;                    // token t's logits
    uint64_t* hk = S.htk + (size_t)t * NP * kQuadCols;       // token t's h words
    const float* xg = x + (size_t)t * H;

    // ---- x staged (chains: transposed fp32; MFMA: bf16 hi / lo) -------------
    {
      bool bad = false;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
        const int i = tid + kThreads * ii;
        if (i < H / 8) {
          const float4 a = reinterpret_cast<const float4*>(xg)[2 * i];
          const float4 c = reinterpret_cast<const float4*>(xg)[2 * i + 1];
          const float f[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
          for (int k2 = 0; k2 < 8; ++k2) bad |= !finite_f(f[k2]);
          const int xts = H / 16 + 4;
          float* dst = xt + (8 * (i & 1)) * xts + (i >> 1);
#pragma unroll
          for (int k2 = 0; k2 < 8; ++k2) dst[k2 * xts] = f[k2];
          uint4 hi, lo;
          split8(f, hi, lo);
          xb2[2 * i + 0] = hi;
          xb2[2 * i + 1] = lo;
        }
      }
      if (bad && m == 0) record_err(status, err_key(kPhX, 0, 0, 0, 0));
    }
    __syncthreads();
    DM_TR(1);

    // ---- gate/up tasks (views, and their loads into the LDS ring) -----------
    auto tview = [&](int tr, ExpertView& gv, ExpertView& uv, int& rb, uint32_t& ph) {
      gv = sgv;
      uv = suv;
      rb = 0;
      ph = kPhShared;
      if (tr < ntask) {
        int sh, slot, sli;
        pair_of(tr >> 3, sh, slot, sli);
        rb = sli * 8 + (tr & 7);
        if (!sh) {
          const int e = __builtin_amdgcn_readfirstlane(st.ids[slot]);
          gv = {L.gu_nib + (size_t)e * matI, L.gu_sc + (size_t)e * 2 * (matI / kGroup), L.I, H};
          uv = {gv.nib + matI / 2, gv.sc + matI / kGroup, L.I, H};
          ph = kPhExpert;
        }
      }
    };
    static_assert(GQW == 2, "the ring holds two chunk pairs per wave");
    // each task's partial sums: [task of this workgroup][wave][gate 16, up 16]
    // in the h staging area (not used before the h poll)
    float* rall = reinterpret_cast<float*>(smem + P.tok_off_hb);
    const uint32_t ring = lds_u32(smem + P.tok_off_ring) + w * kTokSlotW;
    auto issue = [&](int tr, int k) {
      ExpertView gv, uv;
      int rb;
      uint32_t ph;
      tview(tr, gv, uv, rb, ph);
      const int nGQ = gv.cols / kQuadCols;
      const uint32_t sl = ring + k * kWaves * kTokSlotW;
#pragma unroll
      for (int c = 0; c < 2 * GQW; ++c) {
        const int gq = min(w + kWaves * (c >> 1), nGQ - 1);
        dma16_lds(((c & 1) ? uv : gv).nib + a16_nib_offset(nGQ, rb, gq, lane), sl + c * 1024);
      }
      // the four chunks' scales: 128 bytes each, 8 lanes per chunk
      if (lane < 8 * 2 * GQW) {
        const int c = lane >> 3;
        const int gq = min(w + kWaves * (c >> 1), nGQ - 1);
        dma16_lds(reinterpret_cast<const unsigned char*>(((c & 1) ? uv : gv).sc +
                                                         a16_sc_offset(nGQ, rb, gq, 0)) +
                      (lane & 7) * 16,
                  sl + 2 * GQW * 1024);
      }
    };

    // ---- router rows, then routing (as in k_moe_decode_xs) ---------------------
    // task m is a shared slice's (m < 8 nGS): it needs no routing, so its
    // loads go out now on the waves that neither poll nor select
    const bool early = m < nGS * (kQuadCols / kTileRows);
    if (w < nrw) router_compute<true>(L, rw, re, xt, zl, n);
    if (early && w != 0 && w != kNormWave) issue(m, 0);
    if (w == 0) {
      const bool rok = route<R>(zl, n, E, K, st, m == 0, t, status, S.spin);
      if (lane == 0) st.misc[2] = rok ? 1.0f : 0.0f;
    } else if (w == kNormWave) {
      softmax_exp<R>(zl, n, E, st, m == 0, t, status, S.spin);
    }
    lds_barrier();  // the routing state (LDS); task m's loads stay in flight
    DM_TR(2);
    const bool ok = st.misc[2] != 0.0f;

    // ---- this wave's first down chunks (they need the routing only) ----------
    auto dload = [&](int i, uint4& wv, uint2& sv) {
      ExpertView dv = sdv;
      int gq = 0;
      if (i < nit) {
        int sh, slot, sli;
        pair_of(lp0 + lstep * i, sh, slot, sli);
        gq = sli;
        if (!sh) {
          const int e = __builtin_amdgcn_readfirstlane(st.ids[slot]);
          dv = {L.d_nib + (size_t)e * (matD / 2), L.d_sc + (size_t)e * (matD / kGroup), H, L.I};
        }
      }
      load_chunk_nt(dv, i < nit ? rbc : 0, gq, lane, wv, sv);
    };
    uint4 dw[kTokRing];
    uint2 ds[kTokRing];
#pragma unroll
    for (int u = 0; u < kTokRing; ++u) dload(u, dw[u], ds[u]);

    // ---- slot weights; ids / probs / gate of the token in one workgroup ------
    if (w == kNormWave) {
      softmax_sum<R>(E, K, st, m == 0, t, status);
      if (m == nmx - 1)
        finish_probs(E, K, st, true, t, status, ids_out + (size_t)t * K,
                     probs_out + (size_t)t * K, shg_out + t);
    }

    {
      // A ring of kTokGu task slots in LDS, filled by direct-to-LDS loads
      // (loads into registers stall at a few tens of KB in flight per CU):
      // wave w's part of a slot holds its 2 GQW chunks (gate, up of chunk
      // w + 8 i) and their scales, and only wave w reads it, so the ring needs
      // no barrier; the loads of the next kTokGu - 1 tasks are in flight
      // while one task's products run.
      static_assert(kTokGu == 3, "tasks m and m + nmx are the two issued ahead");
      if (!early || w == 0 || w == kNormWave) issue(m, 0);
      issue(m + nmx, 1);

      for (int tr = m; tr < ntask; tr += kTokGu * nmx) {
#pragma unroll
        for (int k = 0; k < kTokGu; ++k) {
          issue(tr + (k + kTokGu - 1) * nmx, (k + kTokGu - 1) % kTokGu);
          const int tk = tr + k * nmx;
          // this slot's loads have landed: only the later tasks' loads (five
          // per task) may still be in flight
          asm volatile("s_waitcnt vmcnt(%0)" ::"n"((kTokGu - 1) * (2 * GQW + 1)) : "memory");
          if (tk < ntask) {
            ExpertView gv, uv;
            int rb;
            uint32_t ph;
            tview(tk, gv, uv, rb, ph);
            (void)rb;
            (void)ph;
            const uint32_t sl = ring + k * kWaves * kTokSlotW;
            uint4 wg[GQW], wu[GQW];
            uint2 sg[GQW], su[GQW];
#pragma unroll
            for (int i = 0; i < GQW; ++i) {
              const v4u a = *(const __attribute__((address_space(3))) v4u*)(size_t)(
                  sl + (2 * i) * 1024 + lane * 16);
              const v4u c = *(const __attribute__((address_space(3))) v4u*)(size_t)(
                  sl + (2 * i + 1) * 1024 + lane * 16);
              const v2u d = *(const __attribute__((address_space(3))) v2u*)(size_t)(
                  sl + 2 * GQW * 1024 + (2 * i) * 128 + j * 8);
              const v2u e2 = *(const __attribute__((address_space(3))) v2u*)(size_t)(
                  sl + 2 * GQW * 1024 + (2 * i + 1) * 128 + j * 8);
              wg[i] = make_uint4(a.x, a.y, a.z, a.w);
              wu[i] = make_uint4(c.x, c.y, c.z, c.w);
              sg[i] = make_uint2(d.x, d.y);
              su[i] = make_uint2(e2.x, e2.y);
            }
            gu_products<GQW, false>(gv, wg, wu, sg, su, xb2, rall + (size_t)((tk - m) / nmx) * 256);
          }
        }
      }
      // every task's partials in LDS: one barrier, then 16 threads per task
      // form its h (swiglu_forward's SiLU, product and checks) and publish it
      lds_barrier();
      const int ntk = m < ntask ? (ntask - m + nmx - 1) / nmx : 0;
      if (tid < kTileRows * ntk) {
        const int kt = tid >> 4, r = tid & 15, tk = m + kt * nmx;
        const float* rp = rall + (size_t)kt * 256;
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) {
          g = g + rp[v * 32 + r];
          u = u + rp[v * 32 + 16 + r];
        }
        const float h = dm_silu(g) * u;
        if (!finite_f(g) || !finite_f(u) || !finite_f(h)) {
          // shared expert: the exact key; routed: the host re-derives it
          int sh, slot, sli;
          pair_of(tk >> 3, sh, slot, sli);
          if (sh)
            record_err(status, err_key(kPhShared, t, 0, (sli * 8 + (tk & 7)) * kTileRows + r,
                                       !finite_f(g) ? kEkGate : !finite_f(u) ? kEkUp : kEkH));
          else
            record_err(status, err_key(kPhExpert, t, 0, 0, kEkRecheck));
        }
        st_l2_u64(hk + (size_t)tk * kTileRows + r, ((uint64_t)n << 32) | f2u(h));
      }
    }
    __syncthreads();  // (a workgroup without tasks) publishes the slot weights
    DM_TR(3);

    // ---- every pair's h, staged scaled by its slot's weight --------------------
    {
      const int nwords = NP * kQuadCols;
      uint64_t hv[kTokHw];
      uint32_t have = 0, all = 0;
#pragma unroll
      for (int u = 0; u < kTokHw; ++u) {
        const int wd = tid + kThreads * u;
        if (wd < nwords) all |= 1u << u;
        hv[u] = ld_coh_u64(hk + min(wd, nwords - 1));
      }
      for (long spin = 0; spin < S.spin && ok && have != all; ++spin) {
#pragma unroll
        for (int u = 0; u < kTokHw; ++u) {
          if ((all >> u & 1u) && !(have >> u & 1u) && (uint32_t)(hv[u] >> 32) == n) {
            const int wd = tid + kThreads * u;
            int sh, slot, sli;
            pair_of(wd / kQuadCols, sh, slot, sli);
            const float wgt = st.pw[slot];
            uint16_t h0, l0;
            split1(u2f((uint32_t)hv[u]) * wgt, h0, l0);
            hbh[wd] = h0;
            hbl[wd] = l0;
            have |= 1u << u;
          }
        }
        if (have == all) break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int u = 0; u < kTokHw; ++u) {
          const int wd = tid + kThreads * u;
          hv[u] = ld_coh_u64(hk + min(wd, nwords - 1));
        }
      }
      if (!__syncthreads_and(have == all || !ok) && tid == 0)
        record_err(status, err_key(kPhSync, 0, 0, 2, 0));
    }
    DM_TR(4);

    // ---- down: this wave's tile over its pairs ------------------------------
    f32x4 acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
    for (int i0 = 0; i0 < nit; i0 += kTokRing) {
#pragma unroll
      for (int u = 0; u < kTokRing; ++u) {
        const int i = i0 + u;
        if (i < nit) {
          const int lp = lp0 + lstep * i;
          bf16x8 A[4], B[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) A[c] = dequant8(word_of(dw[u], c), scale_of(ds[u], c));
          const uint16_t* hs = hbh + lp * kQuadCols;
          const uint16_t* ls = hbl + lp * kQuadCols;
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) B[cc] = ld_b2(hs, ls, cc * 4 + q, j);
          acc0 = mfma16(A[0], B[0], acc0);
          acc1 = mfma16(A[1], B[1], acc1);
          acc0 = mfma16(A[2], B[2], acc0);
          acc1 = mfma16(A[3], B[3], acc1);
        }
        dload(i + kTokRing, dw[u], ds[u]);
      }
    }
    DM_TR(5);
    {
      f32x4 acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = acc0[r] + acc1[r];
      fold_cols(acc);
      if (j == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) yred[w * 16 + 4 * q + r] = acc[r];
      }
    }
    __syncthreads();
    if (tid < kTileRows * my_rt) {
      // rows (rb0 + t2) * 16 + r: the waves of tile t2 in order, the residual
      const int t2 = tid >> 4, r = tid & 15;
      float sum = 0.0f;
      for (int w2 = t2; w2 < kWaves; w2 += rpw) sum = sum + yred[w2 * 16 + r];
      const int d = (rb0 + t2) * kTileRows + r;
      if (residual) sum = sum + residual[(size_t)t * H + d];
      // a non-finite output: the host re-derives which check fires first
      if (!finite_f(sum)) record_err(status, err_key(kPhExpert, t, 0, 0, kEkRecheck));
      y[(size_t)t * H + d] = sum;
    }
    DM_TR(7);
  }
}

static int ldh_log2_of(const LayerDev& L) {
  const int m = L.I > L.Ish ? L.I : L.Ish;
  int lg = 0;
  while ((1 << lg) < m) ++lg;
  return lg;
}

static int align16(int v) { return (v + 15) & ~15; }
static size_t align256z(size_t v) { return (v + 255) & ~(size_t)255; }

static int xs_pairs(const LayerDev& L) { return L.K * (L.I / kQuadCols) + L.Ish / kQuadCols; }

size_t decode_sync_bytes(const LayerDev& L, const DecodePlan& P) {
  const size_t R = (size_t)(L.E + 255) / 256;
  const size_t z = align256z((256 * R + 64) * 8 * (P.xs ? P.xs_nx : 1));
  if (P.xs)
    return z + align256z((size_t)xs_pairs(L) * 64 * 8) + align256z((size_t)P.xs_nx * L.H * 8) +
           (P.tok ? align256z((size_t)kTokMaxT * xs_pairs(L) * kQuadCols * 8) : 0);
  const size_t ldh = (size_t)1 << ldh_log2_of(L);
  return z + align256z((size_t)(L.K + 1) * ldh * 8);
}

DecodeSync decode_sync_carve(const LayerDev& L, const DecodePlan& P, void* base) {
  const size_t R = (size_t)(L.E + 255) / 256;
  unsigned char* p = (unsigned char*)base;
  DecodeSync S{};
  S.spin = kDefaultSpinLimit;
  S.trace = -1;
  S.zt = (uint64_t*)p;
  p += align256z((256 * R + 64) * 8 * (P.xs ? P.xs_nx : 1));
  if (P.xs) {
    S.hl = (uint64_t*)p;
    p += align256z((size_t)xs_pairs(L) * 64 * 8);
    S.pt = (uint64_t*)p;
    p += align256z((size_t)P.xs_nx * L.H * 8);
    if (P.tok) S.htk = (uint64_t*)p;
  } else {
    S.ht = (uint64_t*)p;
  }
  return S;
}

// The XCD-sliced form's geometry, when the layer's shape fits it.
static bool plan_xs(const LayerDev& L, int num_cus, int nx, DecodePlan& P) {
  if (nx <= 0 || num_cus < nx || num_cus % nx != 0) return false;
  if (L.I % kQuadCols != 0 || L.Ish % kQuadCols != 0 || L.K > 32 || L.E > 2048) return false;
  const int nmx = num_cus / nx, nrt = L.H / kTileRows;
  const int need = (nrt + nmx - 1) / nmx;
  int rpw = 1;
  while (rpw < need) rpw *= 2;
  if (rpw > kWaves) return false;
  const int NP = xs_pairs(L), npx = (NP + nx - 1) / nx;
  const int KT = L.K * (L.I / kQuadCols);
  // down tiles per wave: routed ones in registers (kXsR), shared ones (kXsS)
  for (int xc = 0; xc < nx; ++xc) {
    const int np_x = NP > xc ? (NP - xc + nx - 1) / nx : 0;
    const int nr_x = KT > xc ? (KT - xc + nx - 1) / nx : 0;
    for (int w = 0; w < kWaves; ++w) {
      const int lp0 = w / rpw, lstep = kWaves / rpw;
      const int nit = lp0 < np_x ? (np_x - lp0 + lstep - 1) / lstep : 0;
      const int nit_r = lp0 < nr_x ? (nr_x - lp0 + lstep - 1) / lstep : 0;
      if (nit_r > kXsR || nit - nit_r > kXsS) return false;
    }
  }
  const int rpf = (L.H + num_cus - 1) / num_cus;
  const int nxa = nx < NP ? nx : NP;
  if (npx * 64 > kXsHw * kThreads || rpf * nxa > kThreads) return false;
  // the shared expert's rows: two per workgroup, one 16-byte piece per lane
  if (L.Ish > 2 * num_cus || L.H / kQuadCols * 4 > 64) return false;
  // every XCD forms all E+1 logits: rows per workgroup, four per wave
  const int rows = (L.E + 1 + nmx - 1) / nmx;
  const int nrw = (rows + 3) / 4;
  if (nrw > kXsRouterWaves) return false;
  P.xs_nrw = nrw;
  P.xs = 1;
  P.xs_nx = nx;
  P.xs_rpw = rpw;
  P.xs_rpf = rpf;
  P.xs_npx = npx;
  return true;
}

DecodePlan make_decode_plan(const LayerDev& L, int num_cus, int nx) {
  DecodePlan P{};
  P.ldh_log2 = ldh_log2_of(L);
  const int ldh = 1 << P.ldh_log2;
  P.n_router_wg = (L.E + 1 + kRouterRows - 1) / kRouterRows;
  const int R = (L.E + 255) / 256;
  const int slots = L.K + 1;
  const bool xs = plan_xs(L, num_cus, nx, P);
  int off = 0;
  P.off_xt = off; off += align16(4 * 16 * (L.H / 16 + 4));  // 16 chains
  P.off_xb = off; off += align16(4 * L.H);
  P.off_zv = off; off += align16(4 * 256 * R);
  P.off_ev = off; off += align16(4 * 256 * R);
  P.off_sel = off; off += 768;
  P.off_red = off; off += align16(kWaves * 2 * 16 * 4);
  P.off_hb = off; off += align16(xs ? P.xs_npx * kQuadCols * 4 : slots * ldh * 4);
  P.off_yred = off; off += align16(kWaves * 16 * 4);
  P.off_fin = off; off += align16(xs ? P.xs_rpf * (P.xs_nx < xs_pairs(L) ? P.xs_nx : xs_pairs(L)) * 4 : 0);
  P.lds_bytes = off;
  // the several-token form: every pair's h polled by the whole workgroup
  // (kTokHw words per thread), the router rows as in the sliced form
  // (H <= 2048: two chunk pairs per wave in the LDS ring of gate/up tasks)
  if (xs && xs_pairs(L) * kQuadCols <= kTokHw * kThreads && L.H <= 2 * kWaves * kQuadCols) {
    int o = P.off_hb;
    P.tok_off_hb = o; o += align16(xs_pairs(L) * kQuadCols * 4);
    P.tok_off_yred = o; o += align16(kWaves * 16 * 4);
    P.tok_off_ring = o; o += kTokGu * kWaves * kTokSlotW;
    P.tok_lds_bytes = o;
    // each workgroup's task partials (1 KB per task) fit the h staging area
    const int nmx = num_cus / nx;
    const int ntk = (xs_pairs(L) * (kQuadCols / kTileRows) + nmx - 1) / nmx;
    P.tok = o <= kTokMaxLds && ntk * 1024 <= xs_pairs(L) * kQuadCols * 4 ? 1 : 0;
  }
  P.threads = kThreads;
  P.grid = xs ? num_cus : num_cus > L.H / kTileRows ? num_cus : L.H / kTileRows;
  return P;
}

template <int GQW, int NORM, bool XS>
static const void* pick_r(int R) {
  if (XS)
    return R <= 1 ? (const void*)k_moe_decode_xs<GQW, 1, NORM>
                  : (const void*)k_moe_decode_xs<GQW, 8, NORM>;
  return R <= 1 ? (const void*)k_moe_decode<GQW, 1, NORM>
                : (const void*)k_moe_decode<GQW, 8, NORM>;
}

template <int NORM, bool XS>
static const void* pick_gqw(int gqw, int R) {
  return gqw <= 2 ? pick_r<2, NORM, XS>(R) : gqw <= 8 ? pick_r<8, NORM, XS>(R) : nullptr;
}

static int norm_mode(const NormSpec& nm) { return nm.eps > 0.0f ? (nm.seq ? 2 : 1) : 0; }

template <bool XS>
static const void* pick_norm(int norm, int gqw, int R) {
  return norm == 0 ? pick_gqw<0, XS>(gqw, R) : norm == 1 ? pick_gqw<1, XS>(gqw, R)
                                                         : pick_gqw<2, XS>(gqw, R);
}

static const void* pick_kernel(const LayerDev& L, const DecodePlan& P, int norm) {
  const int gqw = (L.H / kQuadCols + kWaves - 1) / kWaves;
  const int R = (L.E + 255) / 256;
  const int ldh = 1 << ldh_log2_of(L);
  if (R > 8 || L.K > 32 || ldh < 2) return nullptr;
  if (P.xs) return pick_norm<true>(norm, gqw, R);
  if ((L.K + 1) * (ldh / 2) > kHw * kThreads) return nullptr;
  return pick_norm<false>(norm, gqw, R);
}

hipError_t decode_occupancy(const LayerDev& L, const DecodePlan& P, int* blocks_per_cu) {
  // every norm form must fit: the launch picks one per call
  int best = 1 << 30;
  for (int norm = 0; norm < 3; ++norm) {
    const void* fn = pick_kernel(L, P, norm);
    if (!fn) return hipErrorInvalidValue;
    int b = 0;
    const hipError_t e =
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, fn, P.threads, P.lds_bytes);
    if (e != hipSuccess) return e;
    best = b < best ? b : best;
  }
  *blocks_per_cu = best;
  return hipSuccess;
}

static const void* pick_tok(int R) {
  return R <= 1 ? (const void*)k_moe_tokens<2, 1> : (const void*)k_moe_tokens<2, 8>;
}

// the several-token kernel's LDS (its gate/up ring) is above the default
// limit of a launch: raised once per device
static hipError_t tok_attrs() {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev < 64 ? 1ull << dev : 0;
  if (bit && (done.load() & bit)) return hipSuccess;
  for (int r : {1, 8}) {
    e = hipFuncSetAttribute(pick_tok(r), hipFuncAttributeMaxDynamicSharedMemorySize, kTokMaxLds);
    if (e != hipSuccess) return e;
  }
  done.fetch_or(bit);
  return hipSuccess;
}

hipError_t launch_moe_tokens(const LayerDev& L, const DecodePlan& P, const float* x, int T,
                             const float* residual, float* y, int32_t* ids, float* probs,
                             float* shg, const DecodeSync& S, unsigned long long* status,
                             hipStream_t st, bool cooperative) {
  if (!P.xs || !P.tok || !S.htk || T < 2 || T > kTokMaxT || T > P.xs_nx)
    return hipErrorInvalidValue;
  const int R = (L.E + 255) / 256;
  if (R > 8 || L.K > 32 || L.H > 2 * kWaves * kQuadCols || P.tok_lds_bytes > kTokMaxLds)
    return hipErrorInvalidValue;
  const void* fn = pick_tok(R);
  const hipError_t ea = tok_attrs();
  if (ea != hipSuccess) return ea;
  LayerDev Lc = L;
  DecodePlan Pc = P;
  DecodeSync Sc = S;
  const float* xc = x;
  const float* rc = residual;
  // (leading arguments preloaded into scalar registers, as in launch_moe_decode)
  const uint16_t* router = L.router;
  int eH = L.H, eE = L.E, enx = P.xs_nx, enrw = P.xs_nrw, enb = P.grid, eT = T;
  void* args[] = {&xc, &router, &eH, &eE, &enx,   &enrw, &enb,   &eT, &Lc,
                  &Pc, &rc,     &y,  &ids, &probs, &shg,  &Sc, &status};
  // every workgroup of an XCD waits for words its other workgroups publish:
  // all must be resident at once (the rule of launch_moe_decode)
  if (cooperative)
    return hipLaunchCooperativeKernel(fn, dim3(P.grid), dim3(P.threads), args, P.tok_lds_bytes,
                                      st);
  return hipLaunchKernel(fn, dim3(P.grid), dim3(P.threads), args, P.tok_lds_bytes, st);
}

hipError_t launch_moe_decode(const LayerDev& L, const DecodePlan& P, const float* x,
                             const float* residual, float* y, int32_t* ids, float* probs,
                             float* shg, const DecodeSync& S, unsigned long long* status, int token,
                             hipStream_t st, const NormSpec& nm, bool cooperative,
                             unsigned long long* status_out) {
  const int norm = norm_mode(nm);
  if (norm != 0 && !nm.gamma) return hipErrorInvalidValue;
  const void* fn = pick_kernel(L, P, norm);
  if (!fn) return hipErrorInvalidValue;
  LayerDev Lc = L;
  DecodePlan Pc = P;
  DecodeSync Sc = S;
  NormSpec nc = nm;
  const float* xc = x;
  const float* rc = residual;
  // The arguments every workgroup needs for its first loads come first:
  // gfx950 preloads the leading kernel arguments into scalar registers
  // (dm_decode.hip is compiled with -amdgpu-kernarg-preload-count), so the
  // loads of x, gamma and the router rows are issued without waiting for a
  // read of the argument segment, which the host has just written.
  const uint16_t* router = L.router;
  const float* gamma = nm.gamma;
  int eH = L.H, eE = L.E, enx = P.xs_nx, enrw = P.xs_nrw, enb = P.grid;
  void* args[] = {&xc,  &router, &gamma, &eH,    &eE,  &enx, &enrw,   &enb,   &Lc, &Pc,
                  &rc,  &y,      &ids,   &probs, &shg, &Sc,  &status, &token, &nc, &status_out};
  // Every workgroup waits for words other workgroups publish, so all of them
  // must be resident at once.  A cooperative launch guarantees it (or fails
  // at launch) but costs about 18 us more per launch than the plain one on
  // MI355X; the caller asks for it when another persistent grid of this
  // library may run concurrently on the device.  Work of other kernels only
  // delays the plain launch's workgroups, and every wait is bounded.
  if (cooperative)
    return hipLaunchCooperativeKernel(fn, dim3(P.grid), dim3(P.threads), args, P.lds_bytes, st);
  return hipLaunchKernel(fn, dim3(P.grid), dim3(P.threads), args, P.lds_bytes, st);
}

}  // namespace dm

namespace dm {

__global__ void k_xcc_map(unsigned* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

hipError_t probe_xcd_map(int num_cus, int* nx) {
  *nx = 0;
  if (num_cus <= 0) return hipSuccess;
  unsigned* d = nullptr;
  hipError_t e = hipMalloc(&d, sizeof(unsigned) * num_cus);
  if (e != hipSuccess) return e;
  std::vector<unsigned> h(num_cus, 0u);
  hipLaunchKernelGGL(k_xcc_map, dim3(num_cus), dim3(64), 0, 0, d);
  e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpy(h.data(), d, sizeof(unsigned) * num_cus, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return e;
  *nx = xcd_rotation(h.data(), num_cus);
  return hipSuccess;
}

int xcd_rotation(const unsigned* xcd, int nwg) {
  if (!xcd || nwg <= 0) return 0;
  unsigned mx = 0;
  for (int b = 0; b < nwg; ++b) mx = xcd[b] > mx ? xcd[b] : mx;
  if (mx >= 64) return 0;  // not an XCD number
  const int n = (int)mx + 1;
  if (nwg % n != 0) return 0;
  // a rotation: workgroup b on XCD (b + r) % n for the one r of workgroup 0
  const unsigned r = xcd[0];
  for (int b = 0; b < nwg; ++b)
    if (xcd[b] != (unsigned)((b + (int)r) % n)) return 0;
  return n;
}

}  // namespace dm

#ifdef DM_PHASE_TRACE
// The phase timestamps of a tracing build (kTraceSlots x 256 x kTracePoints
// 64-bit words, zero where no launch stored one); not in the normal build.
extern "C" int dmh_phase_trace_fetch(void* dst, size_t bytes) {
  if (!dst || bytes < sizeof(dm::g_phase_trace)) return 1;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(dm::g_phase_trace), sizeof(dm::g_phase_trace)) ==
                 hipSuccess
             ? 0
             : 3;
}
#endif
