// dm_kernels.hip -- gfx950 kernels of the MoE FFN block (router, top-k,
// 4-bit SwiGLU experts, shared expert, combine) and their upload helpers.
//
// Reference path (CPU, Mojo): src/layers/router.mojo:15-210,
// src/layers/topk.mojo:11-133, src/layers/swiglu.mojo:11-230,
// src/layers/moe.mojo:17-177, src/layers/forward_layer.mojo:181-247,
// src/quant/dequant_kernel.mojo:22-155.
#include <hip/hip_runtime.h>

#include "dm_device.h"
#include "dm_kernels.h"

namespace dm {

// ===========================================================================
// Upload: reference 4-bit layout -> A16 tiles, with the validation of
// src/quant/dequant_kernel.mojo:68-108 (scale NaN/Inf, scale <= 0, code -8).
// One thread per (matrix, tile, lane): reads 4 aligned words of the source
// row (32 codes per word group), writes 16 bytes; q == 0 lanes move scales.
// The source group size gsrc is any of {32, 64, 128, 256}: groups run over
// the flattened row-major index (quant_format.md:117-161), every 32-column
// chunk of a row lies inside one source group (row * C and the chunk start
// are multiples of 32), and that group's scale is written for the chunk.
// bf16(fp32(s) * q) depends on s and q only, so the tiles compute the same
// values at every source group size.
// Validation key: tensor << 34 | (2*group + kind) for scale errors
// (kind 0 NaN/Inf, 1 non-positive; group in the source numbering),
// tensor << 34 | 1 << 33 for code -8.
// ===========================================================================
__global__ __launch_bounds__(256) void k_repack_a16(const uint8_t* __restrict__ src_nib,
                                                     const uint16_t* __restrict__ src_sc,
                                                     uint8_t* __restrict__ dst_nib,
                                                     uint16_t* __restrict__ dst_sc, int R, int C,
                                                     int nmat, int tensor_base, int gsrc,
                                                     unsigned long long* vkey) {
  const int nRB = R / kTileRows, nGQ = C / kQuadCols;
  const int64_t per_mat = (int64_t)nRB * nGQ * 64;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= per_mat * nmat) return;
  const int m = (int)(gid / per_mat);
  int64_t rem = gid - (int64_t)m * per_mat;
  const int lane = (int)(rem & 63);
  rem >>= 6;
  const int gq = (int)(rem % nGQ);
  const int rb = (int)(rem / nGQ);
  const int r = lane & 15, q = lane >> 4;
  const int row = rb * kTileRows + r;
  const size_t mat_nib = (size_t)R * C / 2, mat_sc = (size_t)R * C / kGroup;
  const uint8_t* sn = src_nib + (size_t)m * mat_nib;
  const uint16_t* ss = src_sc + (size_t)m * ((size_t)R * C / gsrc);
  uint32_t out[4];
  bool reserved = false;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int g = gq * 4 + c;
    const size_t e0 = (size_t)row * C + (size_t)g * kGroup + 8 * q;  // first element
    const uint32_t win = *reinterpret_cast<const uint32_t*>(sn + e0 / 2);
    uint32_t wo = 0;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const uint32_t nib = (win >> (4 * kk)) & 0xFu;  // element e0+kk (low nibble = even)
      reserved |= (nib == 8u);
      wo |= (nib ^ 8u) << (4 * a16_slot_of_kk(kk));
    }
    out[c] = wo;
  }
  *reinterpret_cast<uint4*>(dst_nib + (size_t)m * mat_nib + a16_nib_offset(nGQ, rb, gq, lane)) =
      make_uint4(out[0], out[1], out[2], out[3]);
  uint64_t key = kNoError;
  const uint64_t tens = (uint64_t)(tensor_base + m) << 34;
  if (reserved) key = tens | (1ull << 33);
  if (q == 0) {
    uint16_t sv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int g = gq * 4 + c;
      // source group index inside the tensor
      const size_t gidx = ((size_t)row * C + (size_t)g * kGroup) / (size_t)gsrc;
      const uint16_t u = ss[gidx];
      sv[c] = u;
      uint64_t k2 = kNoError;
      if (((u >> 10) & 0x1Fu) == 0x1Fu) k2 = tens | (2ull * gidx);
      else if ((u & 0x8000u) || (u & 0x7FFFu) == 0) k2 = tens | (2ull * gidx + 1);
      if (k2 < key) key = k2;
    }
    uint2 pk = make_uint2((uint32_t)sv[0] | ((uint32_t)sv[1] << 16),
                          (uint32_t)sv[2] | ((uint32_t)sv[3] << 16));
    *reinterpret_cast<uint2*>(dst_sc + (size_t)m * mat_sc + a16_sc_offset(nGQ, rb, gq, r)) = pk;
  }
  if (key != kNoError) atomicMin(vkey, (unsigned long long)key);
}

hipError_t launch_repack_a16(const uint8_t* src_nib, const uint16_t* src_sc, uint8_t* dst_nib,
                             uint16_t* dst_sc, int R, int C, int nmat, int tensor_base, int gsrc,
                             unsigned long long* vkey, hipStream_t st) {
  if (gsrc != 32 && gsrc != 64 && gsrc != 128 && gsrc != 256) return hipErrorInvalidValue;
  const int64_t n = (int64_t)(R / kTileRows) * (C / kQuadCols) * 64 * nmat;
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(k_repack_a16, dim3((unsigned)blocks), dim3(256), 0, st, src_nib, src_sc,
                     dst_nib, dst_sc, R, C, nmat, tensor_base, gsrc, vkey);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_repack_router(const uint16_t* __restrict__ router,
                                                        const uint16_t* __restrict__ shgate,
                                                        uint16_t* __restrict__ dst, int E, int H,
                                                        unsigned* flags) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)(E + 1) * H) return;
  const int e = (int)(gid / H), k = (int)(gid % H);
  uint16_t v;
  if (e < E) {
    v = router[gid];
    if ((v & 0x7F80u) == 0x7F80u) atomicOr(flags, 1u);  // bf16 NaN/Inf
  } else {
    v = shgate[k];
  }
  dst[r16_index(H, e, k)] = v;
}

hipError_t launch_repack_router(const uint16_t* router, const uint16_t* shgate, uint16_t* dst,
                                int E, int H, unsigned* flags, hipStream_t st) {
  const int64_t n = (int64_t)(E + 1) * H;
  hipLaunchKernelGGL(k_repack_router, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     router, shgate, dst, E, H, flags);
  return hipGetLastError();
}

// ===========================================================================
// Unit dequant (dequant_kernel_simd, src/quant/dequant_kernel.mojo:22-124):
// reference layout in, bf16 out.  Each thread owns 8 codes (4 bytes).
// vkey: scale errors 2*group+kind (kind 0 NaN/Inf, 1 <= 0); code -8 -> 1<<40.
// ===========================================================================
__global__ __launch_bounds__(256) void k_dequant_ref(const uint16_t* __restrict__ scales,
                                                      const uint8_t* __restrict__ packed, int64_t n,
                                                      int group, uint16_t* __restrict__ out,
                                                      unsigned long long* vkey) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t e0 = gid * 8;
  if (e0 >= n) return;
  const int64_t g = e0 / group;
  const uint16_t su = scales[g];
  uint64_t key = kNoError;
  if (e0 % group == 0) {  // one thread per group checks its scale
    if (((su >> 10) & 0x1Fu) == 0x1Fu) key = 2ull * g;
    else if ((su & 0x8000u) || (su & 0x7FFFu) == 0) key = 2ull * g + 1;
  }
  const float s = fp16_bits_to_f32(su);
  const uint32_t w = *reinterpret_cast<const uint32_t*>(packed + e0 / 2);
  uint32_t o[4];
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t b = (w >> (8 * i)) & 0xFFu;
    const int lo = (int)((b & 0xFu) ^ 8u) - 8;  // sign-extended low nibble
    const int hi = (int)((b >> 4) ^ 8u) - 8;
    bad |= (lo == -8) | (hi == -8);
    o[i] = pack_bf16x2(s * (float)lo, s * (float)hi);
  }
  if (bad && (1ull << 40) < key) key = 1ull << 40;
  *reinterpret_cast<uint4*>(out + e0) = make_uint4(o[0], o[1], o[2], o[3]);
  if (key != kNoError) atomicMin(vkey, (unsigned long long)key);
}

hipError_t launch_dequant_ref(const uint16_t* scales, const uint8_t* packed, int64_t n,
                              int group, uint16_t* out, unsigned long long* vkey,
                              hipStream_t st) {
  const int64_t threads = n / 8;
  hipLaunchKernelGGL(k_dequant_ref, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                     scales, packed, n, group, out, vkey);
  return hipGetLastError();
}

// ===========================================================================
// Router logits with the association order of router_project
// (src/layers/router.mojo:80-104): 16 strided lane partials accumulated
// sequentially, halving tree, scalar tail.
// ===========================================================================

// Generic form for the unit entry point: fp32 weights [E][H], any H.  Each
// row's 16 lane partials (router.mojo:75-106) are 16 lanes of a wave: lane l
// runs the chain k = l, l+16, ... with separate multiply and add, the
// halving tree pairs lanes through shuffles inside the 16-lane group, and
// lane 0 adds the tail.  A workgroup holds 16 rows of one token; every lane
// checks the activations and weights it reads, which together cover x and w
// (router.mojo:57-72).
__global__ __launch_bounds__(256) void k_router_generic(const float* __restrict__ x,
                                                         const float* __restrict__ w, int T,
                                                         int H, int E, float* __restrict__ z,
                                                         unsigned long long* status, int t0,
                                                         const float* __restrict__ w_sh) {
  const int l = threadIdx.x & 15;
  const int e = (int)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int t = t0 + (int)blockIdx.y;
  // row E, when w_sh is given, is the shared-expert gate: same order, its
  // checks are the gate's own and run where the logit is used
  const int ldz = w_sh ? E + 1 : E;
  const bool row = e < ldz, gate = e == E;
  const float* xr = x + (int64_t)t * H;
  const float* wr = gate ? w_sh : w + (int64_t)(row ? e : 0) * H;
  const int h16 = H & ~15;
  float acc = 0.0f;
  bool bad_x = false, bad_w = false;
  if (row) {
#pragma unroll 8
    for (int k = l; k < h16; k += 16) {
      const float xv = xr[k], wv = wr[k];
      bad_x |= !finite_f(xv);
      bad_w |= !finite_f(wv);
      acc = acc + xv * wv;
    }
  }
#pragma unroll
  for (int wdt = 8; wdt >= 1; wdt >>= 1) {
    const float o = __shfl_down(acc, wdt, 16);
    if (l < wdt) acc = acc + o;
  }
  if (row && l == 0) {
    float s = acc;
    for (int k = h16; k < H; ++k) {
      const float xv = xr[k], wv = wr[k];
      bad_x |= !finite_f(xv);
      bad_w |= !finite_f(wv);
      s = s + xv * wv;
    }
    if (!gate && !finite_f(s)) record_err(status, err_key(kPhLogit, t, 0, e, 0));
    z[(int64_t)t * ldz + e] = s;
  }
  if (bad_x) record_err(status, err_key(kPhX, 0, 0, 0, 0));
  if (bad_w && !gate) record_err(status, err_key(kPhRouterW, 0, 0, 0, 0));
}

// The same rows with H <= 2048 staged in LDS first: a one-wave workgroup of
// 4 rows loads them and x with 16-byte loads all in flight (one memory round
// trip instead of one per step of the chains), checks every element once,
// then runs the 16-lane chains from LDS.  Row stride H + 16 floats keeps the
// two rows a half-wave reads on different banks.
constexpr int kRouterLdsMaxH = 2048;
__global__ __launch_bounds__(64) void k_router_lds(const float* __restrict__ x,
                                                    const float* __restrict__ w, int T, int H,
                                                    int E, float* __restrict__ z,
                                                    unsigned long long* status, int t0,
                                                    const float* __restrict__ w_sh) {
  __shared__ __attribute__((aligned(16))) float sx[kRouterLdsMaxH];
  __shared__ __attribute__((aligned(16))) float sw[4][kRouterLdsMaxH + 16];
  const int tid = threadIdx.x;
  const int t = t0 + (int)blockIdx.y;
  const int ldz = w_sh ? E + 1 : E;
  const int row0 = (int)blockIdx.x * 4;
  const float* xr = x + (int64_t)t * H;
  bool bad_x = false, bad_w = false;
  // x and the 4 rows: lane tid takes columns 4 (tid + 64 j) of each, all
  // 40 loads issued before the first LDS store
  constexpr int kJ = kRouterLdsMaxH / 256;
  f32x4 v[5][kJ];
#pragma unroll
  for (int r = 0; r < 5; ++r) {
    const int e = row0 + r - 1;  // r = 0: x
    const float* src = r == 0 ? xr : e == E ? w_sh : w + (int64_t)(e < ldz ? e : 0) * H;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const int k = (tid + 64 * j) * 4;
      v[r][j] = (k < H && (r == 0 || e < ldz)) ? *reinterpret_cast<const f32x4*>(src + k)
                                               : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
#pragma unroll
  for (int r = 0; r < 5; ++r) {
    const int e = row0 + r - 1;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const int k = (tid + 64 * j) * 4;
      if (k >= H) continue;
      const f32x4 q = v[r][j];
      const bool bad = !finite_f(q.x) || !finite_f(q.y) || !finite_f(q.z) || !finite_f(q.w);
      if (r == 0) {
        bad_x |= bad;
        *reinterpret_cast<f32x4*>(&sx[k]) = q;
      } else if (e < ldz) {
        if (e != E) bad_w |= bad;
        *reinterpret_cast<f32x4*>(&sw[r - 1][k]) = q;
      }
    }
  }
  __syncthreads();
  const int l = tid & 15, r = tid >> 4, e = row0 + r;
  const bool row = e < ldz, gate = e == E;
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
    float s = acc;
    for (int k = h16; k < H; ++k) s = s + sx[k] * sw[r][k];
    if (!gate && !finite_f(s)) record_err(status, err_key(kPhLogit, t, 0, e, 0));
    z[(int64_t)t * ldz + e] = s;
  }
  if (bad_x) record_err(status, err_key(kPhX, 0, 0, 0, 0));
  if (bad_w) record_err(status, err_key(kPhRouterW, 0, 0, 0, 0));
}

hipError_t launch_router_generic(const float* x, const float* w, int T, int H, int E, float* z,
                                 unsigned long long* status, hipStream_t st, const float* w_sh) {
  if (T <= 0 || E <= 0) return hipErrorInvalidValue;
  const int rows = w_sh ? E + 1 : E;
  const bool lds = H <= kRouterLdsMaxH && H % 4 == 0 &&
                   (((uintptr_t)x | (uintptr_t)w | (uintptr_t)w_sh) & 15) == 0;
  for (int t0 = 0; t0 < T; t0 += 65535) {  // grid.y holds at most 65535 tokens
    const int n = T - t0 < 65535 ? T - t0 : 65535;
    if (lds)
      hipLaunchKernelGGL(k_router_lds, dim3((unsigned)((rows + 3) / 4), (unsigned)n), dim3(64), 0,
                         st, x, w, T, H, E, z, status, t0, w_sh);
    else
      hipLaunchKernelGGL(k_router_generic, dim3((unsigned)((rows + 15) / 16), (unsigned)n),
                         dim3(256), 0, st, x, w, T, H, E, z, status, t0, w_sh);
  }
  return hipGetLastError();
}

// Layer form: R16 bf16 weights with E+1 rows (row E = shared-expert gate,
// which shared_gate_forward, src/layers/moe.mojo:70-100, reduces in the same
// 16-lane order).  One lane per (row, chain l); 16 rows per 256-thread block;
// blockIdx.y = token.  x is staged in LDS once per block.  With gate set, the
// kernel runs only when *gate is nonzero (activations that are not all bf16
// values, which k_router_mfma leaves to it).
__global__ __launch_bounds__(256) void k_router_dec(LayerDev L, const float* __restrict__ x, int T,
                                                     float* __restrict__ z,
                                                     unsigned long long* status,
                                                     const int* __restrict__ gate) {
  extern __shared__ float xs[];
  if (gate && gate[0] == 0) return;  // uniform: k_router_mfma computed these logits
  const int H = L.H;
  const int l = threadIdx.x & 15;
  const int e = blockIdx.x * 16 + (threadIdx.x >> 4);
  for (int t = blockIdx.y; t < T; t += gridDim.y) {
    const float* xr = x + (size_t)t * H;
    bool bad = false;
    for (int i = threadIdx.x; i < H; i += 256) {
      const float v = xr[i];
      bad |= !finite_f(v);
      xs[i] = v;
    }
    if (bad && blockIdx.x == 0) record_err(status, err_key(kPhX, 0, 0, 0, 0));
    __syncthreads();
    float acc = e <= L.E ? router_chain(L.router, H, e, l, xs) : 0.0f;
    // halving tree over the 16 chains of a row: lane l += lane l + w
#pragma unroll
    for (int wdt = 8; wdt >= 1; wdt >>= 1) acc = acc + __shfl_down(acc, wdt, 16);
    if (l == 0 && e <= L.E) z[(size_t)t * (L.E + 1) + e] = acc;
    __syncthreads();  // xs is restaged for the next token
  }
}

// The same logits for many tokens: each thread keeps its chain's H / 16
// router weights (bf16, 8 per register quad) in registers for all the tokens
// of its workgroup, instead of reading the rows again for every token, and
// runs kRdTok tokens per pass, whose activations are staged in LDS as
// xs[k][token] (one 16-byte read gives a step's value for every token of the
// pass).  Each token's 16 chains are the reference's, element for element:
// acc_l = acc_l + x[16 s + l] * w[16 s + l] in s order, multiply and add
// rounded separately, then the halving tree, so every logit has the bits of
// k_router_dec's.
// NJ8 = H / 128 words of 8 steps per chain (a compile-time count: the step
// loop is straight-line code).  The activations of 4 steps (one 16-byte
// read per step) are read by inline assembly one group ahead of their
// products, with a wait tied to their registers: the compiler, left to
// itself, hoisted every read of the loop to its start and spilled.  At
// H = 2048 the kernel holds 127 registers, so four waves share a SIMD and
// the ~1000 workgroups of the launch run in one round.
constexpr int kRdTok = 4;
// the 4 steps' reads: a, a + 256, a + 512, a + 768 (steps 16 floats x 4
// tokens apart)
__device__ __forceinline__ void lds_read_steps4(uint32_t a, f32x4 (&v)[4]) {
  asm volatile(
      "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:256\n\t"
      "ds_read_b128 %2, %4 offset:512\n\tds_read_b128 %3, %4 offset:768"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
      : "v"(a));
}
// wait until at most N LDS operations are in flight (they complete in
// order); v's registers are tied to the wait
template <int N>
__device__ __forceinline__ void lds_wait_steps4(f32x4 (&v)[4]) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]) : "n"(N));
}
template <int NJ8>
__global__ __launch_bounds__(256) void k_router_rows(
    const float* __restrict__ x, const int* __restrict__ gate, const uint16_t* __restrict__ router_,
    int E_, int T, int tpw, LayerDev Lk, float* __restrict__ z, unsigned long long* status) {
  LayerDev L = Lk;  // the entry fields from the preloaded leading arguments
  L.router = router_;
  L.E = E_;
  extern __shared__ __attribute__((aligned(16))) float xs4[];  // [H][kRdTok]
  if (gate && gate[0] == 0) return;  // uniform: k_router_mfma computed these logits
  constexpr int H = NJ8 * 128;
  const int l = threadIdx.x & 15;
  const int e = blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool wave_live = blockIdx.x * 16 + (threadIdx.x >> 6) * 4 <= L.E;  // uniform per wave
  uint4 wr[NJ8];
  {
    const uint4* wp = reinterpret_cast<const uint4*>(L.router + r16_index(H, min(e, L.E), l));
#pragma unroll
    for (int u = 0; u < NJ8; ++u) wr[u] = wp[(size_t)u * 16];
  }
  const int tb = blockIdx.y * tpw, te = min(T, tb + tpw);
  static_assert(kRdTok == 4, "the float4 staging below");
  for (int t0 = tb; t0 < te; t0 += kRdTok) {
    const int nt = min(kRdTok, te - t0);
    bool bad = false;
    for (int k = threadIdx.x; k < H; k += 256) {
      float v[kRdTok];
#pragma unroll
      for (int tt = 0; tt < kRdTok; ++tt) {
        v[tt] = x[(size_t)(t0 + min(tt, nt - 1)) * H + k];
        bad |= tt < nt && !finite_f(v[tt]);
      }
      *reinterpret_cast<float4*>(xs4 + (size_t)k * kRdTok) = make_float4(v[0], v[1], v[2], v[3]);
    }
    if (bad && blockIdx.x == 0) record_err(status, err_key(kPhX, 0, 0, 0, 0));
    __syncthreads();
    // a wave whose four rows are all past row E (the last block's tail)
    // only helps to stage the activations
    if (wave_live) {
      float acc[kRdTok] = {0.0f, 0.0f, 0.0f, 0.0f};
      // group c of 4 steps: steps 4c .. 4c + 3, i.e. word u = c / 2, registers
      // i = 2 (c % 2) and i + 1 (step 8u + 2i: low half, 8u + 2i + 1: high)
      const uint32_t xa0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)(
          xs4 + (size_t)l * kRdTok);
      f32x4 xc[4], xn[4];
      lds_read_steps4(xa0, xc);
#pragma unroll
      for (int c = 0; c < 2 * NJ8; ++c) {
        if (c + 1 < 2 * NJ8) {
          lds_read_steps4(xa0 + (c + 1) * 4 * 256, xn);
          lds_wait_steps4<4>(xc);
        } else {
          lds_wait_steps4<0>(xc);
        }
        const int u = c >> 1;
        // this group's two weight words pass through an empty asm, so their
        // conversions stay in the group (hoisted to the top of the token loop as
        // 128 floats they did not fit in the registers)
        uint32_t wg[2] = {(c & 1) ? wr[u].z : wr[u].x, (c & 1) ? wr[u].w : wr[u].y};
        asm volatile("" : "+v"(wg[0]), "+v"(wg[1]));
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const f32x4 xa = xc[2 * i2], xb = xc[2 * i2 + 1];
          const float wl = bf16lo(wg[i2]), wh = bf16hi(wg[i2]);
          acc[0] = acc[0] + xa[0] * wl;
          acc[1] = acc[1] + xa[1] * wl;
          acc[2] = acc[2] + xa[2] * wl;
          acc[3] = acc[3] + xa[3] * wl;
          acc[0] = acc[0] + xb[0] * wh;
          acc[1] = acc[1] + xb[1] * wh;
          acc[2] = acc[2] + xb[2] * wh;
          acc[3] = acc[3] + xb[3] * wh;
        }
        // (the four chains are complete at every group: sunk below the
        // first token's store, the others kept every read of the pass live)
        asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
        if (c + 1 < 2 * NJ8) {
#pragma unroll
          for (int k = 0; k < 4; ++k) xc[k] = xn[k];
        }
      }
#pragma unroll
      for (int tt = 0; tt < kRdTok; ++tt) {
        // halving tree over the 16 chains of a row: lane l += lane l + w
#pragma unroll
        for (int wdt = 8; wdt >= 1; wdt >>= 1) acc[tt] = acc[tt] + __shfl_down(acc[tt], wdt, 16);
        if (l == 0 && e <= L.E && tt < nt) z[(size_t)(t0 + tt) * (L.E + 1) + e] = acc[tt];
      }
    }
    __syncthreads();  // xs4 is restaged for the next tokens
  }
}

// The fp32 router of the GGUF layers for many tokens: k_router_rows' form
// (each lane's chain of weights in registers, four tokens per pass, the
// activations from LDS) on the chain-ordered fp32 copy of the router and the
// shared gate (launch_chain_router: rows of rs floats, float4 group 16 q + l
// = steps 4q .. 4q + 3 of chain l), with k_router_lds's checks: a
// non-finite activation (kPhX), routed router weight (kPhRouterW) or routed
// logit (kPhLogit).  The chains, their order and the halving tree are
// k_router_lds's (H % 16 == 0: no tail), so the logits are its bits.
template <int NQ>
__global__ __launch_bounds__(256) void k_router_rows_f32(const float* __restrict__ x,
                                                         const float* __restrict__ rchain, int rs,
                                                         int E, int T, int tpw,
                                                         float* __restrict__ z,
                                                         unsigned long long* status) {
  extern __shared__ __attribute__((aligned(16))) float xs4[];  // [H][kRdTok]
  constexpr int H = NQ * 64;
  const int l = threadIdx.x & 15;
  const int e = blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool wave_live = blockIdx.x * 16 + (threadIdx.x >> 6) * 4 <= E;  // uniform per wave
  f32x4 wf[NQ];
  {
    const f32x4* wp = reinterpret_cast<const f32x4*>(rchain + (size_t)min(e, E) * rs) + l;
#pragma unroll
    for (int q = 0; q < NQ; ++q) wf[q] = wp[16 * q];
  }
  if (blockIdx.y == 0 && e < E) {
    bool bad = false;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      bad |= !finite_f(wf[q].x) || !finite_f(wf[q].y) || !finite_f(wf[q].z) || !finite_f(wf[q].w);
    if (bad) record_err(status, err_key(kPhRouterW, 0, 0, 0, 0));
  }
  const int tb = blockIdx.y * tpw, te = min(T, tb + tpw);
  for (int t0 = tb; t0 < te; t0 += kRdTok) {
    const int nt = min(kRdTok, te - t0);
    bool bad = false;
    for (int k = threadIdx.x; k < H; k += 256) {
      float v[kRdTok];
#pragma unroll
      for (int tt = 0; tt < kRdTok; ++tt) {
        v[tt] = x[(size_t)(t0 + min(tt, nt - 1)) * H + k];
        bad |= tt < nt && !finite_f(v[tt]);
      }
      *reinterpret_cast<float4*>(xs4 + (size_t)k * kRdTok) = make_float4(v[0], v[1], v[2], v[3]);
    }
    if (bad && blockIdx.x == 0) record_err(status, err_key(kPhX, 0, 0, 0, 0));
    __syncthreads();
    if (wave_live) {
      float acc[kRdTok] = {0.0f, 0.0f, 0.0f, 0.0f};
      const uint32_t xa0 = lds_u32(xs4 + (size_t)l * kRdTok);
      f32x4 xc[4], xn[4];
      lds_read_steps4(xa0, xc);
#pragma unroll
      for (int c = 0; c < NQ; ++c) {
        if (c + 1 < NQ) {
          lds_read_steps4(xa0 + (c + 1) * 4 * 256, xn);
          lds_wait_steps4<4>(xc);
        } else {
          lds_wait_steps4<0>(xc);
        }
        // steps 4c .. 4c + 3 of chain l, in order
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float wv = wf[c][u];
          acc[0] = acc[0] + xc[u][0] * wv;
          acc[1] = acc[1] + xc[u][1] * wv;
          acc[2] = acc[2] + xc[u][2] * wv;
          acc[3] = acc[3] + xc[u][3] * wv;
        }
        asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
        if (c + 1 < NQ) {
#pragma unroll
          for (int k = 0; k < 4; ++k) xc[k] = xn[k];
        }
      }
#pragma unroll
      for (int tt = 0; tt < kRdTok; ++tt) {
#pragma unroll
        for (int wdt = 8; wdt >= 1; wdt >>= 1) acc[tt] = acc[tt] + __shfl_down(acc[tt], wdt, 16);
        if (l == 0 && e <= E && tt < nt) {
          if (e < E && !finite_f(acc[tt])) record_err(status, err_key(kPhLogit, t0 + tt, 0, e, 0));
          z[(size_t)(t0 + tt) * (E + 1) + e] = acc[tt];
        }
      }
    }
    __syncthreads();  // xs4 is restaged for the next tokens
  }
}

bool router_rows_f32_ok(int T, int H, int E, int rs) {
  const int nq = H % 64 == 0 ? H / 64 : 0;
  return T >= 2 * kRdTok && (nq == 32 || nq == 16 || nq == 8) && rs >= H && rs % 4 == 0 && E >= 1;
}

hipError_t launch_router_rows_f32(const float* x, const float* rchain, int rs, int T, int H, int E,
                                  float* z, unsigned long long* status, hipStream_t st) {
  if (!router_rows_f32_ok(T, H, E, rs)) return hipErrorInvalidValue;
  const int blocks = (E + 1 + 15) / 16;
  const int want = (1024 + blocks - 1) / blocks;
  int tpw = (T + want - 1) / want;
  tpw = ((tpw + kRdTok - 1) / kRdTok) * kRdTok;
  const dim3 g(blocks, (T + tpw - 1) / tpw);
  const size_t lds = (size_t)H * kRdTok * sizeof(float);
  switch (H / 64) {
    case 32: hipLaunchKernelGGL(k_router_rows_f32<32>, g, dim3(256), lds, st, x, rchain, rs, E, T, tpw, z, status); break;
    case 16: hipLaunchKernelGGL(k_router_rows_f32<16>, g, dim3(256), lds, st, x, rchain, rs, E, T, tpw, z, status); break;
    default: hipLaunchKernelGGL(k_router_rows_f32<8>, g, dim3(256), lds, st, x, rchain, rs, E, T, tpw, z, status); break;
  }
  return hipGetLastError();
}

hipError_t launch_router_dec(const LayerDev& L, const float* x, int T, float* z,
                             unsigned long long* status, hipStream_t st, const int* gate) {
  const int blocks = (L.E + 1 + 15) / 16;
  const int nj8 = L.H % 128 == 0 ? L.H / 128 : 0;
  if (T >= 2 * kRdTok && (nj8 == 2 || nj8 == 4 || nj8 == 8 || nj8 == 16)) {
    // tokens per workgroup: a multiple of kRdTok, about 1024 workgroups
    const int want = (1024 + blocks - 1) / blocks;
    int tpw = (T + want - 1) / want;
    tpw = ((tpw + kRdTok - 1) / kRdTok) * kRdTok;
    const int ty = (T + tpw - 1) / tpw;
    const size_t lds = (size_t)L.H * kRdTok * sizeof(float);
    const dim3 g(blocks, ty);
    if (nj8 == 16)
      hipLaunchKernelGGL(k_router_rows<16>, g, dim3(256), lds, st, x, gate, L.router, L.E, T, tpw,
                         L, z, status);
    else if (nj8 == 8)
      hipLaunchKernelGGL(k_router_rows<8>, g, dim3(256), lds, st, x, gate, L.router, L.E, T, tpw,
                         L, z, status);
    else if (nj8 == 4)
      hipLaunchKernelGGL(k_router_rows<4>, g, dim3(256), lds, st, x, gate, L.router, L.E, T, tpw,
                         L, z, status);
    else
      hipLaunchKernelGGL(k_router_rows<2>, g, dim3(256), lds, st, x, gate, L.router, L.E, T, tpw,
                         L, z, status);
    return hipGetLastError();
  }
  const int ty = T < 256 ? T : 256;  // workgroups loop over the tokens beyond
  hipLaunchKernelGGL(k_router_dec, dim3(blocks, ty), dim3(256), (size_t)L.H * sizeof(float), st, L,
                     x, T, z, status, gate);
  return hipGetLastError();
}

// ===========================================================================
// Router logits for many tokens on the matrix cores, for activations that
// are bf16 values (need_lo == 0; otherwise the workgroups return and
// k_router_dec computes the logits).  Every chain of router_project
// (src/layers/router.mojo:15-106) is acc_l = acc_l + x[16s+l] * w[16s+l] in s
// order; with x and w bf16 the product is exact in fp32, so an fp32 MFMA with
// a reduction depth of 1 (v_mfma_f32_16x16x1f32: four blocks of 16x16 outer
// products, one rounding per accumulation) computes exactly that step for 16
// tokens x 16 experts at once.  Block b of instruction g carries chain
// l = 4g + b; the output of block b for (token i, expert j) sits in lane
// j + 16 (i / 4), register 4b + i % 4, so the 16 chains of one logit share a
// lane and the halving tree (l += l + w, w = 8, 4, 2, 1) is plain adds.
//
// Workgroup: 16 tokens x 64 experts (wave w: experts 64 blockIdx.x + 16 w);
// the last column of workgroups computes the shared-expert gate logit (row E)
// with one lane per (token, chain) instead.  The tokens' activations are
// staged once in LDS in chain-major order: xs[i][l][s] = x[t0 + i][16 s + l]
// (bf16), rows padded by 16 bytes so that the 16 lanes of one operand fetch
// hit distinct banks.
// ===========================================================================
typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void k_router_mfma(const uint16_t* __restrict__ xhi,
                                                      const int* __restrict__ need_lo,
                                                      const uint16_t* __restrict__ router_, int H_,
                                                      int E_, int T, LayerDev Lk,
                                                      float* __restrict__ z) {
  LayerDev L = Lk;  // the entry fields from the preloaded leading arguments
  L.router = router_;
  L.H = H_;
  L.E = E_;
  extern __shared__ __attribute__((aligned(16))) uint16_t xs_chain[];
  uint16_t* xs = xs_chain;
  if (need_lo[0] != 0) return;  // uniform: k_router_dec takes these tokens
  const int H = L.H, E = L.E, ns = H / 16;
  const int pitch = 16 * ns + 8;  // elements per staged token (16 B of padding)
  const int t0 = blockIdx.y * 16, tid = threadIdx.x;
  // stage: thread item (token i, step pair sp) reads x[32 sp .. 32 sp + 31]
  // and writes, for each chain l, steps 2 sp and 2 sp + 1 as one word.
  // The reads of up to kStage items are all requested before the first
  // write (one round trip instead of one per item: x was just written by
  // another launch, so it comes from beyond this XCD's L2).
  constexpr int kStage = 4;
  const int npair = ns / 2;
  for (int idx0 = tid; idx0 < 16 * npair; idx0 += 256 * kStage) {
    uint4 xv[kStage][4];
#pragma unroll
    for (int it = 0; it < kStage; ++it) {
      const int idx = min(idx0 + 256 * it, 16 * npair - 1);
      const int i = idx / npair, sp = idx % npair;
      const uint4* src =
          reinterpret_cast<const uint4*>(xhi + (size_t)min(t0 + i, T - 1) * H + 32 * sp);
#pragma unroll
      for (int c = 0; c < 4; ++c) xv[it][c] = src[c];
    }
#pragma unroll
    for (int it = 0; it < kStage; ++it) {
      const int idx = idx0 + 256 * it;
      if (idx < 16 * npair) {
        const int i = idx / npair, sp = idx % npair;
        uint32_t v[16];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const bool in = t0 + i < T;  // tokens past T stage zeros
          v[4 * c] = in ? xv[it][c].x : 0u;
          v[4 * c + 1] = in ? xv[it][c].y : 0u;
          v[4 * c + 2] = in ? xv[it][c].z : 0u;
          v[4 * c + 3] = in ? xv[it][c].w : 0u;
        }
#pragma unroll
        for (int l = 0; l < 16; ++l) {
          const uint32_t a = (v[l >> 1] >> (16 * (l & 1))) & 0xFFFFu;          // step 2 sp
          const uint32_t bq = (v[8 + (l >> 1)] >> (16 * (l & 1))) & 0xFFFFu;   // step 2 sp + 1
          *reinterpret_cast<uint32_t*>(xs + i * pitch + l * ns + 2 * sp) = a | (bq << 16);
        }
      }
    }
  }
  __syncthreads();
  const int lane = tid & 63, w = tid >> 6;
  if ((int)blockIdx.x == (E + 63) / 64) {
    // shared-expert gate: lane (token i, chain l), 8 steps per 16-byte read
    const int i = tid >> 4, l = tid & 15;
    const uint16_t* xr = xs + i * pitch + l * ns;
    const uint16_t* wr = L.router + r16_index(H, E, l);
    float acc = 0.0f;
    // the chain's gate words sixteen rounds at a time, all requested before
    // the first product (one round trip per sixteen rounds; requested one
    // per round they made these workgroups the launch's longest)
    constexpr int kGw = 16;
    const int nc = ns / 8;
    for (int c0 = 0; c0 < nc; c0 += kGw) {
      uint4 wv[kGw];
#pragma unroll
      for (int u = 0; u < kGw; ++u)
        wv[u] = *reinterpret_cast<const uint4*>(wr + (size_t)min(c0 + u, nc - 1) * 128);
#pragma unroll
      for (int u = 0; u < kGw; ++u) {
        if (c0 + u < nc) {  // uniform
          const uint4 xv = *reinterpret_cast<const uint4*>(xr + 8 * (c0 + u));
          const uint32_t xa[4] = {xv.x, xv.y, xv.z, xv.w};
          const uint32_t wa[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            acc = acc + bf16lo(xa[k]) * bf16lo(wa[k]);
            acc = acc + bf16hi(xa[k]) * bf16hi(wa[k]);
          }
        }
      }
    }
#pragma unroll
    for (int wdt = 8; wdt >= 1; wdt >>= 1) acc = acc + __shfl_down(acc, wdt, 16);
    if (l == 0 && t0 + i < T) z[(size_t)(t0 + i) * (E + 1) + E] = acc;
    return;
  }
  const int e0 = blockIdx.x * 64 + 16 * w;
  if (e0 >= E) return;  // uniform per wave (no barrier below)
  const int b = lane >> 4, jj = lane & 15;
  const int er = min(e0 + jj, E - 1);
  // A: token jj (as row i = lane & 15 of block b), chain 4g + b
  const uint16_t* xa = xs + jj * pitch + b * ns;
  const uint16_t* wb = L.router + r16_index(H, er, b);
  f32x16 acc[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) acc[g] = f32x16{};
  // steps 8c .. 8c + 7 of the wave's chains: the router words two rounds
  // ahead of their products (a ring of two, requests clamped to the last
  // round), x from LDS one round ahead
  const int nc = ns / 8;
  uint4 wr[2][4], xr[2][4];
  auto load_w = [&](int c, uint4 (&d)[4]) {
    const int cc = min(c, nc - 1);
#pragma unroll
    for (int g = 0; g < 4; ++g)
      d[g] = *reinterpret_cast<const uint4*>(wb + (size_t)cc * 128 + 4 * g * 8);
  };
  auto load_x = [&](int c, uint4 (&d)[4]) {
    const int cc = min(c, nc - 1);
#pragma unroll
    for (int g = 0; g < 4; ++g) d[g] = *reinterpret_cast<const uint4*>(xa + 4 * g * ns + 8 * cc);
  };
  // the four accumulators' steps interleaved (each one's steps in order),
  // so that consecutive matrix instructions are independent
  auto steps = [&](const uint4 (&xv)[4], const uint4 (&wv)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t xw = u == 0 ? xv[g].x : u == 1 ? xv[g].y : u == 2 ? xv[g].z : xv[g].w;
        const uint32_t ww = u == 0 ? wv[g].x : u == 1 ? wv[g].y : u == 2 ? wv[g].z : wv[g].w;
        acc[g] = __builtin_amdgcn_mfma_f32_16x16x1f32(bf16lo(xw), bf16lo(ww), acc[g], 0, 0, 0);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t xw = u == 0 ? xv[g].x : u == 1 ? xv[g].y : u == 2 ? xv[g].z : xv[g].w;
        const uint32_t ww = u == 0 ? wv[g].x : u == 1 ? wv[g].y : u == 2 ? wv[g].z : wv[g].w;
        acc[g] = __builtin_amdgcn_mfma_f32_16x16x1f32(bf16hi(xw), bf16hi(ww), acc[g], 0, 0, 0);
      }
    }
  };
  load_w(0, wr[0]);
  load_w(1, wr[1]);
  load_x(0, xr[0]);
  int c = 0;
  for (; c + 1 < nc; c += 2) {
    load_x(c + 1, xr[1]);
    steps(xr[0], wr[0]);
    load_w(c + 2, wr[0]);
    load_x(c + 2, xr[0]);
    steps(xr[1], wr[1]);
    load_w(c + 3, wr[1]);
  }
  if (c < nc) steps(xr[0], wr[0]);
  // lane holds tokens t0 + 4 b + r, expert e0 + jj; chain 4g + bb at acc[g][4 bb + r]
  const int e = e0 + jj;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) v[g][bb] = acc[g][4 * bb + r];
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {  // w = 8: chain l += chain l + 8
      v[0][bb] = v[0][bb] + v[2][bb];
      v[1][bb] = v[1][bb] + v[3][bb];
    }
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) v[0][bb] = v[0][bb] + v[1][bb];  // w = 4
    v[0][0] = v[0][0] + v[0][2];  // w = 2
    v[0][1] = v[0][1] + v[0][3];
    const float s = v[0][0] + v[0][1];  // w = 1
    const int t = t0 + 4 * b + r;
    if (t < T && e < E) z[(size_t)t * (E + 1) + e] = s;
  }
}

hipError_t launch_router_mfma(const LayerDev& L, const uint16_t* xhi, const int* need_lo, int T,
                              float* z, hipStream_t st) {
  const size_t lds = (size_t)16 * (16 * (L.H / 16) + 8) * sizeof(uint16_t);
  hipLaunchKernelGGL(k_router_mfma, dim3((L.E + 63) / 64 + 1, (T + 15) / 16), dim3(256), lds, st,
                     xhi, need_lo, L.router, L.H, L.E, T, L, z);
  return hipGetLastError();
}

// ===========================================================================
// Softmax + top-k + shared gate, one 64-lane wave per token
// (route_select_token).
// ===========================================================================
template <int NE>
__global__ __launch_bounds__(64) void k_router_select(const float* __restrict__ z, int ldz, int E,
                                                       int K, int has_sh,
                                                       int32_t* __restrict__ ids,
                                                       float* __restrict__ probs,
                                                       float* __restrict__ shg,
                                                       unsigned long long* status) {
  extern __shared__ __attribute__((aligned(16))) float sm[];  // e[E] (padded), then 1/S
  route_select_token<NE, false>(z, ldz, E, K, has_sh, (int)blockIdx.x, threadIdx.x, sm, ids, probs, shg,
                         status, [] { __syncthreads(); });
}

hipError_t launch_router_select(const float* z, int ldz, int T, int E, int K, int has_sh,
                                int32_t* ids, float* probs, float* shg,
                                unsigned long long* status, hipStream_t st) {
  const size_t lds = (size_t)(((E + 3) & ~3) + 4) * sizeof(float);
  const int ne = (E + 63) / 64;
#define DM_SELECT(N)                                                                         \
  hipLaunchKernelGGL(k_router_select<N>, dim3(T), dim3(64), lds, st, z, ldz, E, K, has_sh, ids, \
                     probs, shg, status)
  if (ne <= 1) DM_SELECT(1);
  else if (ne <= 2) DM_SELECT(2);
  else if (ne <= 4) DM_SELECT(4);
  else if (ne <= 8) DM_SELECT(8);
  else if (ne <= 16) DM_SELECT(16);
  else DM_SELECT(32);
#undef DM_SELECT
  return hipGetLastError();
}

// ===========================================================================
// Decode gate/up: h = SiLU(W_gate x) * (W_up x) for the K routed experts and
// the shared expert (src/layers/swiglu.mojo:134-201, fp32 h).  Block =
// (slot, 16-row tile); its 4 waves split the 128-column chunks of the
// reduction and meet in LDS.  Each MFMA step dequantises one group of the
// 16 rows into bf16 (bit-exact bf16_rne(s*q)) and multiplies it by the
// activation split into bf16 hi/lo columns 0 and 1 of the B operand.
// ===========================================================================
__global__ __launch_bounds__(256) void k_gateup_dec(LayerDev L, const float* __restrict__ x,
                                                     const int32_t* __restrict__ ids,
                                                     float* __restrict__ hout, int ldh, int token,
                                                     unsigned long long* status) {
  extern __shared__ uint4 xb[];  // (H/8)*3 blocks
  __shared__ float red[4][2][16];
  const int H = L.H;
  const int nrb_r = L.I / kTileRows;
  int slot, rb, I;
  ExpertView gv, uv;
  if ((int)blockIdx.x < L.K * nrb_r) {
    slot = blockIdx.x / nrb_r;
    rb = blockIdx.x % nrb_r;
    I = L.I;
    int e = ids[slot];
    if (e < 0 || e >= L.E) e = 0;  // invalid ids come with a recorded router error
    const size_t mat = (size_t)I * H;
    gv = {L.gu_nib + (size_t)e * mat, L.gu_sc + (size_t)e * 2 * (mat / kGroup), I, H};
    uv = {gv.nib + mat / 2, gv.sc + mat / kGroup, I, H};
  } else {
    slot = L.K;
    rb = blockIdx.x - L.K * nrb_r;
    I = L.Ish;
    const size_t mat = (size_t)I * H;
    gv = {L.sgu_nib, L.sgu_sc, I, H};
    uv = {L.sgu_nib + mat / 2, L.sgu_sc + mat / kGroup, I, H};
  }
  stage_split(x, H, xb);
  __syncthreads();
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15, jsel = j < 2 ? j : 2;
  const int nGQ = H / kQuadCols;
  f32x4 ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
  for (int gq = w; gq < nGQ; gq += 4) {
    uint4 wg, wu;
    uint2 sg, su;
    load_chunk(gv, rb, gq, lane, wg, sg);
    load_chunk(uv, rb, gq, lane, wu, su);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int g = gq * 4 + c;
      const bf16x8 b = __builtin_bit_cast(bf16x8, xb[(g * 4 + q) * 3 + jsel]);
      ag = mfma16(dequant8(word_of(wg, c), scale_of(sg, c)), b, ag);
      au = mfma16(dequant8(word_of(wu, c), scale_of(su, c)), b, au);
    }
  }
  fold_cols(ag);
  fold_cols(au);
  if (j == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[w][0][4 * q + i] = ag[i];
      red[w][1][4 * q + i] = au[i];
    }
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int r = threadIdx.x, row = rb * kTileRows + r;
    const float g = ((red[0][0][r] + red[1][0][r]) + red[2][0][r]) + red[3][0][r];
    const float u = ((red[0][1][r] + red[1][1][r]) + red[2][1][r]) + red[3][1][r];
    const uint32_t ph = slot < L.K ? kPhExpert : kPhShared;
    const uint32_t sl = slot < L.K ? slot : 0;
    if (!finite_f(g)) record_err(status, err_key(ph, token, sl, row, kEkGate));
    if (!finite_f(u)) record_err(status, err_key(ph, token, sl, row, kEkUp));
    const float h = dm_silu(g) * u;
    if (!finite_f(h)) record_err(status, err_key(ph, token, sl, row, kEkH));
    hout[(size_t)slot * ldh + row] = h;
  }
}

hipError_t launch_gateup_dec(const LayerDev& L, const float* x, const int32_t* ids, float* h,
                             int ldh, int token, unsigned long long* status, hipStream_t st) {
  const int blocks = L.K * (L.I / kTileRows) + L.Ish / kTileRows;
  hipLaunchKernelGGL(k_gateup_dec, dim3(blocks), dim3(256), (size_t)(L.H / 8) * 3 * sizeof(uint4),
                     st, L, x, ids, h, ldh, token, status);
  return hipGetLastError();
}

// ===========================================================================
// Decode down projection + combine: y_d = sum_k p_k (W_down_k h_k)_d
// + g_sh (W_down_sh h_sh)_d (+ residual), k in routed order first, then the
// shared expert, then the residual (src/layers/moe.mojo:157-166,
// src/layers/forward_layer.mojo:226-238).  Block = 16 output rows; wave w
// owns slots w, w+4, ...; the combine is one ordered pass, no atomics.
// ===========================================================================
__global__ __launch_bounds__(256) void k_down_dec(LayerDev L, const float* __restrict__ hin,
                                                   int ldh, const int32_t* __restrict__ ids,
                                                   const float* __restrict__ probs,
                                                   const float* __restrict__ shg,
                                                   const float* __restrict__ residual,
                                                   float* __restrict__ y, int token,
                                                   unsigned long long* status) {
  extern __shared__ uint4 hb[];  // (K+1) * (ldh/8) * 3 blocks
  __shared__ float red[33][16];
  const int H = L.H, K = L.K;
  const int rb = blockIdx.x;
  const int nblk_slot = (ldh / 8) * 3;
  for (int s = 0; s <= K; ++s) {
    const int Is = s < K ? L.I : L.Ish;
    stage_split(hin + (size_t)s * ldh, Is, hb + (size_t)s * nblk_slot);
  }
  __syncthreads();
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15, jsel = j < 2 ? j : 2;
  for (int s = w; s <= K; s += 4) {
    ExpertView dv;
    if (s < K) {
      int e = ids[s];
      if (e < 0 || e >= L.E) e = 0;
      const size_t mat = (size_t)H * L.I;
      dv = {L.d_nib + (size_t)e * (mat / 2), L.d_sc + (size_t)e * (mat / kGroup), H, L.I};
    } else {
      dv = {L.sd_nib, L.sd_sc, H, L.Ish};
    }
    const int nGQ = dv.cols / kQuadCols;
    const uint4* hbs = hb + (size_t)s * nblk_slot;
    f32x4 acc = {0, 0, 0, 0};
    for (int gq = 0; gq < nGQ; ++gq) {
      uint4 wd;
      uint2 sd;
      load_chunk(dv, rb, gq, lane, wd, sd);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int g = gq * 4 + c;
        const bf16x8 b = __builtin_bit_cast(bf16x8, hbs[(g * 4 + q) * 3 + jsel]);
        acc = mfma16(dequant8(word_of(wd, c), scale_of(sd, c)), b, acc);
      }
    }
    fold_cols(acc);
    if (j == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) red[s][4 * q + i] = acc[i];
    }
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int r = threadIdx.x, d = rb * kTileRows + r;
    float rs = 0.0f;
    for (int s = 0; s < K; ++s) {
      const float v = red[s][r];
      if (!finite_f(v)) record_err(status, err_key(kPhExpert, token, s, ldh + d, kEkDown));
      rs = rs + probs[s] * v;
    }
    const float vsh = red[K][r];
    if (!finite_f(vsh)) record_err(status, err_key(kPhShared, token, 0, ldh + d, kEkDown));
    float total = rs + shg[0] * vsh;
    if (residual) total = total + residual[d];
    if (!finite_f(total)) record_err(status, err_key(kPhAgg, token, 0, d, 0));
    y[d] = total;
  }
}

hipError_t launch_down_dec(const LayerDev& L, const float* h, int ldh, const int32_t* ids,
                           const float* probs, const float* shg, const float* residual,
                           float* y, int token, unsigned long long* status, hipStream_t st) {
  if (L.K + 1 > 33) return hipErrorInvalidValue;
  const size_t lds = (size_t)(L.K + 1) * (ldh / 8) * 3 * sizeof(uint4);
  hipLaunchKernelGGL(k_down_dec, dim3(L.H / kTileRows), dim3(256), lds, st, L, h, ldh, ids, probs,
                     shg, residual, y, token, status);
  return hipGetLastError();
}

// ===========================================================================
// RMSNorm per token (src/layers/rmsnorm.mojo:41-48): out = x / denom *
// gamma, denom = sqrt(sum(x * x) / H + eps), for the block-edge norm of
// several tokens.  SEQ: the squares staged in LDS and added in element order
// by one lane, the reference's order; otherwise 256 strided partials and a
// halving tree (the order of the fused decode kernel's tree mode).
// ===========================================================================
template <bool SEQ>
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float* __restrict__ x, int H,
                                                       float eps, const float* __restrict__ gamma,
                                                       float* __restrict__ out) {
  __shared__ float part[SEQ ? kNormMaxH : 256];
  const int t = blockIdx.x;
  const float* xr = x + (size_t)t * H;
  if (SEQ) {
    for (int i = threadIdx.x; i < H; i += 256) part[i] = xr[i] * xr[i];
    __syncthreads();
    if (threadIdx.x == 0) {
      float a = 0.0f;
      int i = 0;
      for (; i + 8 <= H; i += 8) {  // reads 8 ahead of the adds
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = part[i + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) a = a + v[u];
      }
      for (; i < H; ++i) a = a + part[i];
      part[0] = a;
    }
    __syncthreads();
  } else {
    float acc = 0.0f;
    for (int i = threadIdx.x; i < H; i += 256) acc = acc + xr[i] * xr[i];
    part[threadIdx.x] = acc;
    __syncthreads();
    for (int wdt = 128; wdt >= 1; wdt >>= 1) {
      if ((int)threadIdx.x < wdt) part[threadIdx.x] = part[threadIdx.x] + part[threadIdx.x + wdt];
      __syncthreads();
    }
  }
  const float denom = __builtin_sqrtf(part[0] / (float)H + eps);
  for (int i = threadIdx.x; i < H; i += 256) out[(size_t)t * H + i] = (xr[i] / denom) * gamma[i];
}

hipError_t launch_rmsnorm_rows(const float* x, int T, int H, const NormSpec& nm, float* out,
                               hipStream_t st) {
  if (H <= 0 || H > kNormMaxH || !nm.gamma) return hipErrorInvalidValue;
  if (nm.seq)
    hipLaunchKernelGGL(k_rmsnorm_rows<true>, dim3(T), dim3(256), 0, st, x, H, nm.eps, nm.gamma,
                       out);
  else
    hipLaunchKernelGGL(k_rmsnorm_rows<false>, dim3(T), dim3(256), 0, st, x, H, nm.eps, nm.gamma,
                       out);
  return hipGetLastError();
}

// ---- a small fill kernel ---------------------------------------------------
// Clears flags and counters in code a caller may capture into a HIP graph
// (a kernel node instead of a memset node).
__global__ __launch_bounds__(256) void k_fill_i32(int32_t* __restrict__ p, int n, int32_t v) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

hipError_t launch_fill_i32(int32_t* p, int n, int32_t v, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_i32, dim3((n + 255) / 256), dim3(256), 0, st, p, n, v);
  return hipGetLastError();
}

// ---- shared gate scores and expert-id checks (unit entry points) ----------
// One thread per token: sigmoid of the gate logit with the two checks of
// shared_gate_forward (src/layers/moe.mojo:83-100) in its order.
__global__ __launch_bounds__(256) void k_shared_gate_scores(const float* __restrict__ z, int ldz,
                                                            int T, float* __restrict__ scores,
                                                            unsigned long long* status) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= T) return;
  const float logit = z[(size_t)t * ldz];
  if (!finite_f(logit)) record_err(status, err_key(kPhGate, t, 0, 0, kGkLogit));
  const float sg = dm_sigmoid(logit);
  if (!finite_f(sg) || sg < 0.0f || sg > 1.0f)
    record_err(status, err_key(kPhGate, t, 0, 0, kGkRange));
  scores[t] = sg;
}

hipError_t launch_shared_gate_scores(const float* z, int ldz, int T, float* scores,
                                     unsigned long long* status, hipStream_t st) {
  hipLaunchKernelGGL(k_shared_gate_scores, dim3((T + 255) / 256), dim3(256), 0, st, z, ldz, T,
                     scores, status);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_check_ids(const int32_t* __restrict__ ids, int n, int K,
                                                   int E, int32_t* __restrict__ out,
                                                   unsigned long long* status) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int32_t e = ids[i];
  const bool ok = e >= 0 && e < E;
  if (!ok) record_err(status, err_key(kPhExpert, i / K, i % K, (uint32_t)e & 0xFFFFFFFu, kEkBadId));
  out[i] = ok ? e : 0;
}

hipError_t launch_check_ids(const int32_t* ids, int T, int K, int E, int32_t* out,
                            unsigned long long* status, hipStream_t st) {
  const int n = T * K;
  hipLaunchKernelGGL(k_check_ids, dim3((n + 255) / 256), dim3(256), 0, st, ids, n, K, E, out,
                     status);
  return hipGetLastError();
}

}  // namespace dm
