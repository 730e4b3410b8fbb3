/*
 * dm_oracle.c -- CPU restatement of the reference engine's 4-bit MoE FFN path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for libdismoen_hip.so, never the
 * product.  Built with -O2 -ffp-contract=off so every multiply and add rounds
 * separately, as the Mojo sources do.
 *
 * What pins each function (tests/test_oracle_*.py):
 *   or_fp16_to_f32 / or_f32_to_bf16_rne / or_dequant_q4_*: numpy's float16
 *       widening and torch's float32->bfloat16 cast over all 65536 fp16
 *       patterns x all 15 codes; the 225-pair exhaustive test and the pack
 *       known answers of tests/unit/test_m6_dequant.mojo:48-86 and
 *       tests/unit/test_m6_quant_format.mojo:139-144; the seed-42 G-M6-K
 *       fixture (regenerated in tests/golden); fixtures/m10_quant_mini.bin.
 *   or_expf: float64 exp (<= 2 ulp), monotonicity sweep, exp(0)=1, ties.
 *   or_sigmoid_f32 / or_silu_f32: tests/unit/test_moe.mojo:23-48 known values,
 *       float64 closed forms.
 *   or_router_project / softmax / select_topk: tests/unit/test_router_ops.mojo
 *       and test_router_topk.mojo known answers, float64 dot products,
 *       brute-force (-p, id) sort on tiny inputs, renorm-leak case.
 *   or_swiglu_forward / or_shared_gate_forward / or_moe_aggregate: known
 *       answers of tests/unit/test_moe.mojo:51-175 and a float64 numpy MoE.
 *   or_pool_*: partition_range invariants and serial == parallel bit-exact
 *       (tests/unit/test_m11_w1_workerpool.mojo:23-221).
 *   or_dequant_gguf: the closed forms of the synthetic blocks of
 *       fixtures/m9_port_mini.gguf (tools/fixtures/generate_m9_gguf_fixture.py:
 *       47-91); vectors of the reference's Python twin tools/oracle/
 *       oracle_port.py:68-160 on random blocks (Q8_0, Q3_K, Q4_K layout 1);
 *       Q4_K layout 0 through the byte substitution that maps it onto layout
 *       1 (bytes 12..15 := bytes 8..11, read from gguf.mojo:482-488).
 * Parity unpinned (no toolchain for the reference here): the exact bits of
 * Mojo's std.math.exp and the association order of SIMD.reduce_add; this file
 * fixes exp = or_expf and reduce_add = halving tree.
 */
#define _GNU_SOURCE
#include "dm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static int seterr(char* err, size_t errlen, const char* fmt, ...) {
  if (err && errlen) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
  }
  return 1;
}

static inline int finite_f(float v) { return isfinite(v) != 0; }

/* 16-lane strided dot product: lane l accumulates k = l, l+16, ... in order,
 * then the halving tree, then the scalar tail (router.mojo:84-96,
 * swiglu.mojo:138-150). */
static inline float dot16(const float* a, const float* b, int n) {
  float acc[16];
  for (int l = 0; l < 16; ++l) acc[l] = 0.0f;
  int k = 0;
  for (; k + 16 <= n; k += 16)
    for (int l = 0; l < 16; ++l) {
      float prod = a[k + l] * b[k + l];
      acc[l] = acc[l] + prod;
    }
  for (int w = 8; w >= 1; w >>= 1)
    for (int l = 0; l < w; ++l) acc[l] = acc[l] + acc[l + w];
  float s = acc[0];
  for (; k < n; ++k) {
    float prod = a[k] * b[k];
    s = s + prod;
  }
  return s;
}

/* ---- scalar helpers ------------------------------------------------------ */
float or_fp16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
  uint32_t m = (uint32_t)h & 0x3FFu;
  if (e == 0) {
    if (m == 0) return u2f(sign);
    float v = (float)m * 0x1p-24f; /* exact: m < 2^10 */
    return u2f(f2u(v) | sign);
  }
  if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t or_f32_to_bf16_rne(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* exp(x): Cody & Waite range reduction x = k*ln2 + r (ln2 split in a 15-bit
 * head and a tail), exp(r) by the degree-7 Taylor polynomial in Horner form
 * with fused multiply-adds, scaling by 2^k through the exponent field.  The
 * HIP kernels evaluate the identical operation sequence, so both sides agree
 * bit for bit. */
float or_expf(float x) {
  if (x != x) return x;
  if (x > 0x1.62e43p+6f) return INFINITY;
  if (x < -0x1.9fe36ap+6f) return 0.0f;
  float kf = rintf(x * 0x1.715476p+0f);
  float r = fmaf(kf, -0x1.62e4p-1f, x);
  r = fmaf(kf, -0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0x1p-1f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int k = (int)kf;
  if (k > 127) {
    p = p * 0x1p127f;
    k -= 127;
  }
  if (k < -126) {
    p = p * u2f((uint32_t)(k + 227) << 23);
    return p * 0x1p-100f;
  }
  return p * u2f((uint32_t)(k + 127) << 23);
}

/* sigmoid_f32, src/layers/swiglu.mojo:11-26 */
float or_sigmoid_f32(float z) {
  if (z != z) return z;
  if (z < -88.0f) return 0.0f;
  if (z > 88.0f) return 1.0f;
  if (z < 0.0f) {
    float ez = or_expf(z);
    return ez / (1.0f + ez);
  }
  return 1.0f / (1.0f + or_expf(-z));
}

/* silu_f32, src/layers/swiglu.mojo:29-38 */
float or_silu_f32(float z) {
  if (z != z) return z;
  if (isinf(z)) return z > 0.0f ? z : 0.0f;
  return z * or_sigmoid_f32(z);
}

/* pack_4bit_pair / unpack_4bit_pair, src/format/half_float.mojo:34-58 */
int or_pack_4bit_pair(int w0, int w1, uint8_t* out) {
  if (w0 < -7 || w0 > 7 || w1 < -7 || w1 > 7) return 1;
  *out = (uint8_t)(((w1 & 0x0F) << 4) | (w0 & 0x0F));
  return 0;
}

int or_unpack_4bit_pair(uint8_t b, int* w0, int* w1) {
  int u0 = b & 0x0F, u1 = (b >> 4) & 0x0F;
  if (u0 == 8 || u1 == 8) return 1;
  *w0 = u0 >= 8 ? u0 - 16 : u0;
  *w1 = u1 >= 8 ? u1 - 16 : u1;
  return 0;
}

/* is_allowed_group_size, src/format/half_float.mojo:24-31 */
int or_is_allowed_group_size(int g) { return g == 32 || g == 64 || g == 128 || g == 256; }

/* fp16 RNE of a float32 (normal range only is needed by the scale rule). */
static uint16_t f32_to_fp16_rne(float f) {
  uint32_t u = f2u(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (a > 0x7F800000u ? 0x200u : 0));
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to inf */
  if (a < 0x38800000u) { /* fp16 subnormal or zero: value = a * 2^24 units */
    float v = u2f(a) * 0x1p24f; /* exact scaling */
    float rv = rintf(v);
    return (uint16_t)(sign | (uint32_t)rv);
  }
  uint32_t e = (a >> 23) - 112u;
  uint32_t m = a & 0x7FFFFFu;
  uint32_t h = (e << 10) | (m >> 13);
  uint32_t rest = m & 0x1FFFu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1;
  return (uint16_t)(sign | h);
}

/* compute_fp16_scale_ceil, src/format/half_float.mojo:77-97 */
uint16_t or_compute_fp16_scale_ceil(float max_abs, int* status) {
  *status = 0;
  if (max_abs != max_abs || isinf(max_abs)) { *status = 1; return 0; }
  if (max_abs <= 0.0f) return 0x3C00u;
  float target = max_abs / 7.0f;
  uint16_t s = f32_to_fp16_rne(target);
  if (or_fp16_to_f32(s) * 7.0f < max_abs) {
    if (s >= 0x7C00u) { *status = 2; return 0; }
    s = (uint16_t)(s + 1u);
  }
  return s;
}

/* ---- dequant_kernel_simd, src/quant/dequant_kernel.mojo:22-124 ----------- */
int or_dequant_q4_bf16(const uint16_t* scales, int64_t n_scales,
                       const uint8_t* packed, int64_t n_packed,
                       int64_t num_elements, int group_size,
                       uint16_t* out, char* err, size_t errlen) {
  if (!or_is_allowed_group_size(group_size))
    return seterr(err, errlen,
                  "dequant_kernel: group_size must be in {32, 64, 128, 256}, got %d",
                  group_size);
  if (num_elements <= 0)
    return seterr(err, errlen, "dequant_kernel: num_elements must be positive");
  if (num_elements % group_size != 0)
    return seterr(err, errlen,
                  "M6_ERR_INPUT: N %% G != 0 (tail group not supported): N=%lld, G=%d",
                  (long long)num_elements, group_size);
  int64_t num_groups = num_elements / group_size;
  if (n_scales != num_groups)
    return seterr(err, errlen,
                  "dequant_kernel: scales length mismatch: expected %lld, got %lld",
                  (long long)num_groups, (long long)n_scales);
  int64_t exp_packed = (num_elements + 1) / 2;
  if (n_packed != exp_packed)
    return seterr(err, errlen,
                  "dequant_kernel: packed weights length mismatch: expected %lld, got %lld",
                  (long long)exp_packed, (long long)n_packed);
  for (int64_t g = 0; g < num_groups; ++g) {
    uint16_t u = scales[g];
    if (((u >> 10) & 0x1Fu) == 0x1Fu)
      return seterr(err, errlen, "dequant_kernel: scale is NaN or Inf at group %lld",
                    (long long)g);
    if ((u & 0x8000u) || (u & 0x7FFFu) == 0)
      return seterr(err, errlen, "dequant_kernel: scale is non-positive at group %lld",
                    (long long)g);
  }
  int bytes_in_group = group_size / 2;
  for (int64_t g = 0; g < num_groups; ++g) {
    float s = or_fp16_to_f32(scales[g]);
    int64_t eb = g * group_size, bb = g * bytes_in_group;
    for (int b = 0; b + 8 <= bytes_in_group; b += 8) {
      int lo[8], hi[8], bad = 0;
      for (int j = 0; j < 8; ++j) {
        uint8_t raw = packed[bb + b + j];
        lo[j] = (int)(int8_t)(uint8_t)(raw << 4) >> 4;
        hi[j] = (int)(int8_t)raw >> 4;
        if (lo[j] < -7 || hi[j] < -7) bad = 1;
      }
      if (bad)
        return seterr(err, errlen,
                      "dequant_kernel: reserved nibble 0b1000 (-8) encountered");
      for (int j = 0; j < 8; ++j) {
        out[eb + 2 * (b + j)] = or_f32_to_bf16_rne(s * (float)lo[j]);
        out[eb + 2 * (b + j) + 1] = or_f32_to_bf16_rne(s * (float)hi[j]);
      }
    }
  }
  return 0;
}

/* dequant_kernel_simd_f32, src/quant/dequant_kernel.mojo:127-155 */
int or_dequant_q4_f32(const uint16_t* scales, int64_t n_scales,
                      const uint8_t* packed, int64_t n_packed,
                      int64_t num_elements, int group_size, float* out,
                      char* err, size_t errlen) {
  if (num_elements <= 0 || num_elements > ((int64_t)1 << 40))
    return or_dequant_q4_bf16(scales, n_scales, packed, n_packed, num_elements,
                              group_size, NULL, err, errlen);
  uint16_t* tmp = (uint16_t*)malloc((size_t)num_elements * 2);
  if (!tmp) return seterr(err, errlen, "dequant_kernel: out of memory");
  int st = or_dequant_q4_bf16(scales, n_scales, packed, n_packed, num_elements,
                              group_size, tmp, err, errlen);
  if (st == 0)
    for (int64_t i = 0; i < num_elements; ++i) out[i] = or_bf16_to_f32(tmp[i]);
  free(tmp);
  return st;
}

/* ---- GGUF payloads ------------------------------------------------------- */
/* get_ggml_block_specs, src/format/gguf.mojo:76-102, for the types that
 * stream_gguf_tensor_f32 (gguf.mojo:598-626) dequantizes. */
int or_gguf_block_spec(int t, int* bs, int* bpb) {
  switch (t) {
    case 0: *bs = 1; *bpb = 4; return 0;      /* F32 */
    case 30: *bs = 1; *bpb = 2; return 0;     /* BF16 */
    case 8: *bs = 32; *bpb = 34; return 0;    /* Q8_0 */
    case 12: *bs = 256; *bpb = 144; return 0; /* Q4_K */
    case 11: *bs = 256; *bpb = 114; return 0; /* Q3_K */
    default: return -1;
  }
}

static uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Scale code and min code of sub-block j of a Q4_K block (12 packed bytes
 * q = block + 4).  layout 0: gguf.mojo:473-488 (for j >= 4 the low bits of
 * both come from q[j]); layout 1: oracle_port.py:100-110 (from q[j + 4]). */
static void q4k_scale_min(const uint8_t* q, int j, int layout, int* sc, int* mn) {
  if (j < 4) {
    *sc = q[j] & 63;
    *mn = q[j + 4] & 63;
    return;
  }
  const int lo = layout ? q[j + 4] : q[j];
  *sc = (lo & 15) | ((q[j - 4] >> 6) << 4);
  *mn = (lo >> 4) | ((q[j] >> 6) << 4);
}

/* dequantize_q8_0 (gguf.mojo:414-441), dequantize_q4_k (:444-506),
 * dequantize_q3_k (:509-560) and the F32 / BF16 copies of
 * stream_gguf_tensor_f32 (:598-613).  Each output is one fp32 product of
 * exactly representable factors (Q4_K: minus the min, one rounding). */
int or_dequant_gguf(int t, const uint8_t* raw, int64_t raw_bytes, int64_t n, int layout,
                    float* out, char* err, size_t errlen) {
  int bs, bpb;
  if (or_gguf_block_spec(t, &bs, &bpb))
    return seterr(err, errlen, "GGUF_UNSUPPORTED_DTYPE: unsupported GGML type %d", t);
  if (n < 0) return seterr(err, errlen, "or_dequant_gguf: negative num_elements");
  const int64_t nb = n / bs;
  if (raw_bytes < nb * bpb)
    return seterr(err, errlen, "or_dequant_gguf: %lld bytes < %lld blocks x %d",
                  (long long)raw_bytes, (long long)nb, bpb);
  for (int64_t i = nb * bs; i < n; ++i) out[i] = 0.0f;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* blk = raw + b * bpb;
    float* o = out + b * bs;
    if (t == 0) {
      memcpy(o, blk, 4);
    } else if (t == 30) {
      o[0] = or_bf16_to_f32(rd_u16(blk));
    } else if (t == 8) {
      const float d = or_fp16_to_f32(rd_u16(blk));
      for (int i = 0; i < 32; ++i) o[i] = d * (float)(int8_t)blk[2 + i];
    } else if (t == 12) {
      const float d = or_fp16_to_f32(rd_u16(blk));
      const float dmin = or_fp16_to_f32(rd_u16(blk + 2));
      for (int e = 0; e < 256; ++e) {
        const int j = e >> 5, r = e & 31; /* sub-block, position in it */
        int sc, mn;
        q4k_scale_min(blk + 4, j, layout, &sc, &mn);
        const uint8_t byte = blk[16 + j * 16 + (r & 15)];
        const int q = r < 16 ? (byte & 15) : (byte >> 4);
        const float fs = (float)sc * d, fm = (float)mn * dmin;
        o[e] = fs * (float)q - fm;
      }
    } else { /* Q3_K: hmask [0,32), qs [32,96), scales [96,112), d [112,114) */
      const float d = or_fp16_to_f32(rd_u16(blk + 112));
      for (int e = 0; e < 256; ++e) {
        const int hi = (blk[e >> 3] >> (e & 7)) & 1;
        const int lo = (blk[32 + (e >> 2)] >> ((e & 3) * 2)) & 3;
        const float fs = (float)((int)blk[96 + (e >> 4)] - 32) * d;
        o[e] = fs * (float)((hi << 2 | lo) - 4);
      }
    }
  }
  return 0;
}

/* ---- router -------------------------------------------------------------- */
/* RouterConfig.validate, src/layers/router_types.mojo:9-44 */
int or_router_config_validate(int num_experts, int top_k, int norm, char* err,
                              size_t errlen) {
  if (num_experts <= 0)
    return seterr(err, errlen,
                  "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"num_experts must be"
                  " positive\",\"stage\":\"router\"}");
  if (top_k <= 0)
    return seterr(err, errlen,
                  "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"num_experts_per_tok"
                  " must be positive\",\"stage\":\"router\"}");
  if (top_k > num_experts)
    return seterr(err, errlen,
                  "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"num_experts_per_tok"
                  " cannot exceed num_experts\",\"stage\":\"router\"}");
  if (norm)
    return seterr(err, errlen,
                  "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"norm_topk_prob=true"
                  " forbidden; unrenormalized routing invariant"
                  " violated\",\"stage\":\"router\"}");
  return 0;
}

/* router_project, src/layers/router.mojo:15-106 */
int or_router_project(const float* x, int64_t n_x, const float* w, int64_t n_w,
                      int T, int H, int E, int layer, float* out, char* err,
                      size_t errlen) {
  if (T <= 0 || H <= 0 || E <= 0)
    return seterr(err, errlen,
                  "{\"error_type\":\"ACT_LOAD_FAILED\",\"detail\":\"dimensions must be"
                  " positive\",\"stage\":\"router\",\"layer\":%d}", layer);
  if (n_x != (int64_t)T * H)
    return seterr(err, errlen,
                  "{\"error_type\":\"ACT_LOAD_FAILED\",\"detail\":\"activation length"
                  " mismatch: expected %lld got %lld\",\"stage\":\"router\",\"layer\":%d}",
                  (long long)T * H, (long long)n_x, layer);
  if (n_w != (int64_t)E * H)
    return seterr(err, errlen,
                  "{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"weight length"
                  " mismatch: expected %lld got %lld\",\"stage\":\"router\",\"layer\":%d}",
                  (long long)E * H, (long long)n_w, layer);
  for (int64_t i = 0; i < n_x; ++i)
    if (!finite_f(x[i]))
      return seterr(err, errlen,
                    "{\"error_type\":\"ACT_LOAD_FAILED\",\"detail\":\"non-finite value in"
                    " activation\",\"stage\":\"router\",\"layer\":%d}", layer);
  for (int64_t i = 0; i < n_w; ++i)
    if (!finite_f(w[i]))
      return seterr(err, errlen,
                    "{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"non-finite value"
                    " in router weight\",\"stage\":\"router\",\"layer\":%d}", layer);
  for (int t = 0; t < T; ++t)
    for (int e = 0; e < E; ++e) {
      float acc = dot16(x + (int64_t)t * H, w + (int64_t)e * H, H);
      if (!finite_f(acc))
        return seterr(err, errlen,
                      "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"non-finite router"
                      " logit computed\",\"stage\":\"router\",\"layer\":%d}", layer);
      out[(int64_t)t * E + e] = acc;
    }
  return 0;
}

/* router_softmax, src/layers/router.mojo:109-185 */
int or_router_softmax(const float* z, int64_t n_z, int T, int E, int layer,
                      float* probs, char* err, size_t errlen) {
  if (T <= 0 || E <= 0)
    return seterr(err, errlen,
                  "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"dimensions must be"
                  " positive\",\"stage\":\"router\",\"layer\":%d}", layer);
  if (n_z != (int64_t)T * E)
    return seterr(err, errlen,
                  "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"logits length mismatch:"
                  " expected %lld got %lld\",\"stage\":\"router\",\"layer\":%d}",
                  (long long)T * E, (long long)n_z, layer);
  float* tmp = (float*)malloc(sizeof(float) * (size_t)E);
  if (!tmp) return seterr(err, errlen, "oracle: out of memory");
  for (int t = 0; t < T; ++t) {
    const float* zr = z + (int64_t)t * E;
    float m = zr[0];
    for (int e = 1; e < E; ++e)
      if (zr[e] > m) m = zr[e];
    if (!finite_f(m)) {
      free(tmp);
      return seterr(err, errlen,
                    "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"non-finite max logit in"
                    " router softmax\",\"stage\":\"router\",\"layer\":%d}", layer);
    }
    float sum = 0.0f;
    for (int e = 0; e < E; ++e) {
      float ev = or_expf(zr[e] - m);
      if (!finite_f(ev)) {
        free(tmp);
        return seterr(err, errlen,
                      "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"non-finite exp in"
                      " router softmax\",\"stage\":\"router\",\"layer\":%d}", layer);
      }
      tmp[e] = ev;
      sum = sum + ev;
    }
    if (sum <= 0.0f || !finite_f(sum)) {
      free(tmp);
      return seterr(err, errlen,
                    "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"invalid sum_exp in"
                    " router softmax\",\"stage\":\"router\",\"layer\":%d}", layer);
    }
    float inv = 1.0f / sum;
    for (int e = 0; e < E; ++e) probs[(int64_t)t * E + e] = tmp[e] * inv;
  }
  free(tmp);
  return 0;
}

/* select_topk, src/layers/topk.mojo:11-133 (selection sort, lowest id wins
 * ties, no renormalisation). */
int or_select_topk(const float* probs, int64_t n_probs, int T, int E, int K,
                   int norm, int layer, int32_t* out_ids, float* out_vals,
                   char* err, size_t errlen) {
  if (norm)
    return seterr(err, errlen,
                  "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"norm_topk_prob=true"
                  " forbidden; unrenormalized routing invariant"
                  " violated\",\"stage\":\"router\",\"layer\":%d}", layer);
  if (T <= 0 || E <= 0 || K <= 0)
    return seterr(err, errlen,
                  "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"dimensions must be"
                  " positive\",\"stage\":\"router\",\"layer\":%d}", layer);
  if (K > E)
    return seterr(err, errlen,
                  "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"top_k cannot exceed"
                  " num_experts\",\"stage\":\"router\",\"layer\":%d}", layer);
  if (n_probs != (int64_t)T * E)
    return seterr(err, errlen,
                  "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"probabilities length"
                  " mismatch: expected %lld got %lld\",\"stage\":\"router\",\"layer\":%d}",
                  (long long)T * E, (long long)n_probs, layer);
  int* ids = (int*)malloc(sizeof(int) * (size_t)E);
  float* vals = (float*)malloc(sizeof(float) * (size_t)E);
  if (!ids || !vals) {
    free(ids); free(vals);
    return seterr(err, errlen, "oracle: out of memory");
  }
  int st = 0;
  for (int t = 0; t < T && !st; ++t) {
    const float* pr = probs + (int64_t)t * E;
    float sum_all = 0.0f;
    for (int e = 0; e < E; ++e) {
      ids[e] = e;
      vals[e] = pr[e];
      sum_all = sum_all + pr[e];
    }
    for (int i = 0; i < K; ++i) {
      int mi = i;
      float mv = vals[i];
      for (int j = i + 1; j < E; ++j) {
        if (vals[j] > mv) {
          mv = vals[j];
          mi = j;
        } else if (vals[j] == mv && ids[j] < ids[mi]) {
          mv = vals[j];
          mi = j;
        }
      }
      if (mi != i) {
        float tv = vals[i]; vals[i] = vals[mi]; vals[mi] = tv;
        int ti = ids[i]; ids[i] = ids[mi]; ids[mi] = ti;
      }
    }
    float sum_topk = 0.0f;
    for (int i = 0; i < K; ++i) {
      out_ids[(int64_t)t * K + i] = ids[i];
      out_vals[(int64_t)t * K + i] = vals[i];
      sum_topk = sum_topk + vals[i];
    }
    if (sum_topk > 1.00001f) {
      st = seterr(err, errlen,
                  "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"sum of top-k"
                  " probabilities exceeds 1.0\",\"stage\":\"router\",\"layer\":%d}", layer);
      break;
    }
    if (K < E) {
      float rem = sum_all - sum_topk;
      if (rem > 1e-5f && fabsf(sum_topk - 1.0f) < 1e-6f) {
        st = seterr(err, errlen,
                    "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"renormalization"
                    " leak detected: sum of top-k probabilities is"
                    " 1.0\",\"stage\":\"router\",\"layer\":%d}", layer);
        break;
      }
    }
  }
  free(ids);
  free(vals);
  return st;
}

/* router_forward, src/layers/router.mojo:188-210 */
int or_router_forward(const float* x, int64_t n_x, const float* w, int64_t n_w,
                      int T, int H, int E, int K, int norm, int layer,
                      int32_t* ids, float* vals, char* err, size_t errlen) {
  if (or_router_config_validate(E, K, norm, err, errlen)) return 1;
  float* z = (float*)malloc(sizeof(float) * (size_t)T * (size_t)(E > 0 ? E : 1));
  float* p = (float*)malloc(sizeof(float) * (size_t)T * (size_t)(E > 0 ? E : 1));
  int st = (!z || !p) ? seterr(err, errlen, "oracle: out of memory") : 0;
  if (!st) st = or_router_project(x, n_x, w, n_w, T, H, E, layer, z, err, errlen);
  if (!st) st = or_router_softmax(z, (int64_t)T * E, T, E, layer, p, err, errlen);
  if (!st) st = or_select_topk(p, (int64_t)T * E, T, E, K, norm, layer, ids, vals, err, errlen);
  free(z);
  free(p);
  return st;
}

/* ---- experts ------------------------------------------------------------- */
#define SWIGLU_ERR(kind, detail)                                                   \
  seterr(err, errlen,                                                              \
         "{\"error_type\":\"" kind "\",\"detail\":\"" detail                      \
         "\",\"stage\":\"swiglu\",\"layer\":%d,\"expert_id\":%d}", layer, expert_id)

/* swiglu_forward, src/layers/swiglu.mojo:52-230 */
int or_swiglu_forward(const float* x, int64_t n_x, const float* wg,
                      const float* wu, const float* wd, int64_t n_g,
                      int64_t n_u, int64_t n_d, int T, int H, int I, int layer,
                      int expert_id, float* out, char* err, size_t errlen) {
  if (T <= 0 || H <= 0 || I <= 0) return SWIGLU_ERR("EXPERT_ERROR", "dimensions must be positive");
  if (n_x != (int64_t)T * H)
    return seterr(err, errlen,
                  "{\"error_type\":\"ACT_LOAD_FAILED\",\"detail\":\"activation length"
                  " mismatch: expected %lld got %lld\",\"stage\":\"swiglu\",\"layer\":%d,"
                  "\"expert_id\":%d}", (long long)T * H, (long long)n_x, layer, expert_id);
  if (n_g != (int64_t)I * H || n_u != (int64_t)I * H)
    return SWIGLU_ERR("WEIGHT_LOAD_FAILED", "gate/up weight length mismatch");
  if (n_d != (int64_t)H * I) return SWIGLU_ERR("WEIGHT_LOAD_FAILED", "down weight length mismatch");
  for (int64_t i = 0; i < n_x; ++i)
    if (!finite_f(x[i])) return SWIGLU_ERR("ACT_LOAD_FAILED", "non-finite value in activation");
  float* h = (float*)malloc(sizeof(float) * (size_t)I);
  if (!h) return seterr(err, errlen, "oracle: out of memory");
  for (int t = 0; t < T; ++t) {
    const float* xr = x + (int64_t)t * H;
    for (int j = 0; j < I; ++j) {
      float g = dot16(xr, wg + (int64_t)j * H, H);
      if (!finite_f(g)) { free(h); return SWIGLU_ERR("EXPERT_ERROR", "non-finite in gate projection"); }
      float ga = or_silu_f32(g);
      float u = dot16(xr, wu + (int64_t)j * H, H);
      if (!finite_f(u)) { free(h); return SWIGLU_ERR("EXPERT_ERROR", "non-finite in up projection"); }
      float hj = ga * u;
      if (!finite_f(hj)) { free(h); return SWIGLU_ERR("SWIGLU_ERROR", "non-finite in element-wise product"); }
      h[j] = hj;
    }
    for (int d = 0; d < H; ++d) {
      float y = dot16(h, wd + (int64_t)d * I, I);
      if (!finite_f(y)) { free(h); return SWIGLU_ERR("EXPERT_ERROR", "non-finite in down projection"); }
      out[(int64_t)t * H + d] = y;
    }
  }
  free(h);
  return 0;
}

/* shared_gate_forward, src/layers/moe.mojo:17-102 */
int or_shared_gate_forward(const float* x, int64_t n_x, const float* w,
                           int64_t n_w, int T, int H, int layer,
                           const char* mode, float* scores, char* err,
                           size_t errlen) {
  if (!mode || strcmp(mode, "sigmoid") != 0)
    return seterr(err, errlen,
                  "{\"error_type\":\"GATE_ERROR\",\"detail\":\"shared expert gate must be"
                  " sigmoid; non-sigmoid gate forbidden (invariant"
                  " #2)\",\"stage\":\"shared\",\"layer\":%d}", layer);
  if (T <= 0 || H <= 0)
    return seterr(err, errlen,
                  "{\"error_type\":\"GATE_ERROR\",\"detail\":\"dimensions must be"
                  " positive\",\"stage\":\"shared\",\"layer\":%d}", layer);
  if (n_x != (int64_t)T * H)
    return seterr(err, errlen,
                  "{\"error_type\":\"ACT_LOAD_FAILED\",\"detail\":\"activation length"
                  " mismatch\",\"stage\":\"shared\",\"layer\":%d}", layer);
  if (n_w != H)
    return seterr(err, errlen,
                  "{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"shared gate weight"
                  " length mismatch: expected %d got %lld\",\"stage\":\"shared\",\"layer\":%d}",
                  H, (long long)n_w, layer);
  for (int t = 0; t < T; ++t) {
    float logit = dot16(x + (int64_t)t * H, w, H);
    if (!finite_f(logit))
      return seterr(err, errlen,
                    "{\"error_type\":\"GATE_ERROR\",\"detail\":\"non-finite shared gate"
                    " logit\",\"stage\":\"shared\",\"layer\":%d}", layer);
    float s = or_sigmoid_f32(logit);
    if (!finite_f(s) || s < 0.0f || s > 1.0f)
      return seterr(err, errlen,
                    "{\"error_type\":\"GATE_ERROR\",\"detail\":\"shared gate score outside"
                    " (0, 1)\",\"stage\":\"shared\",\"layer\":%d}", layer);
    scores[t] = s;
  }
  return 0;
}

/* moe_aggregate_forward, src/layers/moe.mojo:105-177 (residual != NULL) and
 * moe_combine_no_residual, src/layers/forward_layer.mojo:181-247. */
int or_moe_aggregate(const float* residual, const float* routed,
                     const float* probs, const float* sh, const float* gates,
                     int T, int H, int K, int layer, float* out, char* err,
                     size_t errlen) {
  if (T <= 0 || H <= 0)
    return seterr(err, errlen,
                  "{\"error_type\":\"EXPERT_ERROR\",\"detail\":\"dimensions must be"
                  " positive\",\"stage\":\"aggregation\",\"layer\":%d}", layer);
  for (int t = 0; t < T; ++t) {
    float g = gates[t];
    const float* r = routed + (int64_t)t * K * H;
    const float* p = probs + (int64_t)t * K;
    for (int d = 0; d < H; ++d) {
      float rs = 0.0f;
      for (int k = 0; k < K; ++k) {
        float prod = p[k] * r[(int64_t)k * H + d];
        rs = rs + prod;
      }
      float shv = g * sh[(int64_t)t * H + d];
      float total = rs + shv;
      if (residual) total = total + residual[(int64_t)t * H + d];
      if (!finite_f(total))
        return seterr(err, errlen,
                      "{\"error_type\":\"EXPERT_ERROR\",\"detail\":\"non-finite value in"
                      " aggregation\",\"stage\":\"aggregation\",\"layer\":%d}", layer);
      out[(int64_t)t * H + d] = total;
    }
  }
  return 0;
}

/* ---- glue ---------------------------------------------------------------- */
/* rmsnorm, src/layers/rmsnorm.mojo:10-48 */
int or_rmsnorm(const float* x, const float* gamma, int n, float eps, float* out,
               char* err, size_t errlen) {
  if (n <= 0)
    return seterr(err, errlen,
                  "{\"error_type\":\"NORM_ERROR\",\"detail\":\"empty input\",\"stage\":\"rmsnorm\"}");
  if (eps != eps || isinf(eps) || eps <= 0.0f)
    return seterr(err, errlen,
                  "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"rms_norm_eps must be"
                  " finite and > 0\",\"stage\":\"config\"}");
  float acc = 0.0f;
  for (int i = 0; i < n; ++i) {
    float sq = x[i] * x[i];
    acc = acc + sq;
  }
  float denom = sqrtf(acc / (float)n + eps);
  for (int i = 0; i < n; ++i) {
    float q = x[i] / denom;
    out[i] = q * (gamma ? gamma[i] : 1.0f);
  }
  return 0;
}

/* The fast-mode RMSNorm of the library: the arithmetic of
 * src/layers/rmsnorm.mojo:41-48 (x / denom * gamma, gamma NULL = 1) except
 * that the sum of squares is reduced as 256 strided partials (partial i sums
 * x[i], x[i+256], ... in order) and a halving tree, the order of the GPU's
 * tree mode.  The reference sums sequentially (or_rmsnorm); the two agree to
 * a few ulp (tests/test_oracle_moe.py). */
int or_rmsnorm_tree256(const float* x, const float* gamma, int n, float eps, float* out,
                       char* err, size_t errlen) {
  if (n <= 0)
    return seterr(err, errlen,
                  "{\"error_type\":\"NORM_ERROR\",\"detail\":\"empty input\",\"stage\":\"rmsnorm\"}");
  if (eps != eps || isinf(eps) || eps <= 0.0f)
    return seterr(err, errlen,
                  "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"rms_norm_eps must be"
                  " finite and > 0\",\"stage\":\"config\"}");
  float part[256];
  for (int i = 0; i < 256; ++i) {
    float a = 0.0f;
    for (int k = i; k < n; k += 256) {
      float sq = x[k] * x[k];
      a = a + sq;
    }
    part[i] = a;
  }
  for (int w = 128; w >= 1; w >>= 1)
    for (int i = 0; i < w; ++i) part[i] = part[i] + part[i + w];
  float denom = sqrtf(part[0] / (float)n + eps);
  for (int i = 0; i < n; ++i) {
    float q = x[i] / denom;
    out[i] = q * (gamma ? gamma[i] : 1.0f);
  }
  return 0;
}

/* add_residual, src/layers/residual.mojo:10-51 */
int or_add_residual(const float* y, const float* x, int64_t n, int layer,
                    float* out, char* err, size_t errlen) {
  for (int64_t i = 0; i < n; ++i) {
    if (!finite_f(y[i]) || !finite_f(x[i]))
      return seterr(err, errlen,
                    "{\"error_type\":\"ATTENTION_ERROR\",\"detail\":\"non-finite value in"
                    " residual\",\"stage\":\"residual\",\"layer\":%d}", layer);
    float v = y[i] + x[i];
    if (!finite_f(v))
      return seterr(err, errlen,
                    "{\"error_type\":\"ATTENTION_ERROR\",\"detail\":\"overflow in"
                    " residual addition\",\"stage\":\"residual\",\"layer\":%d}", layer);
    out[i] = v;
  }
  return 0;
}

/* ---- worker pool, src/core/worker_pool.mojo ------------------------------ */
/* partition_range, src/core/worker_pool.mojo:29-49 */
void or_partition_range(int64_t total, int64_t tid, int64_t n, int64_t* start,
                        int64_t* end) {
  if (n <= 1) { *start = 0; *end = total; return; }
  if (total <= 0) { *start = 0; *end = 0; return; }
  int64_t chunk = total / n, rem = total % n;
  int64_t s = tid * chunk + (tid < rem ? tid : rem);
  int64_t c = chunk + (tid < rem ? 1 : 0);
  *start = s;
  *end = s + c;
}

struct or_pool {
  int n;
  pthread_t* th;
  pthread_barrier_t bar_start, bar_done;
  int quit;
  /* TASK_MOE_EXPERTS arguments */
  int top_k, hidden, inter;
  const float* x_tok;
  float* out_routed;
  const int64_t* selected;
  const float* const* wg;
  const float* const* wu;
  const float* const* wd;
  float* h_scratch; /* [n][inter] */
  int h_cap;
};

typedef struct { or_pool* p; int id; } worker_arg;

/* _worker_moe_task, src/core/worker_pool.mojo:108-189 */
static void moe_task(or_pool* p, int wid) {
  int64_t s, e;
  or_partition_range(p->top_k, wid, p->n, &s, &e);
  int H = p->hidden, I = p->inter;
  float* h = p->h_scratch + (int64_t)wid * p->h_cap;
  for (int64_t k = s; k < e; ++k) {
    int64_t id = p->selected[k];
    const float* wg = p->wg[id];
    const float* wu = p->wu[id];
    const float* wd = p->wd[id];
    float* out = p->out_routed + k * H;
    for (int j = 0; j < I; ++j) {
      float ga[16], ua[16];
      for (int l = 0; l < 16; ++l) ga[l] = ua[l] = 0.0f;
      int c = 0;
      const float* gr = wg + (int64_t)j * H;
      const float* ur = wu + (int64_t)j * H;
      for (; c + 16 <= H; c += 16)
        for (int l = 0; l < 16; ++l) {
          float xv = p->x_tok[c + l];
          float pg = xv * gr[c + l];
          float pu = xv * ur[c + l];
          ga[l] = ga[l] + pg;
          ua[l] = ua[l] + pu;
        }
      for (int w = 8; w >= 1; w >>= 1)
        for (int l = 0; l < w; ++l) {
          ga[l] = ga[l] + ga[l + w];
          ua[l] = ua[l] + ua[l + w];
        }
      float g = ga[0], u = ua[0];
      for (; c < H; ++c) {
        float xv = p->x_tok[c];
        float pg = xv * gr[c];
        float pu = xv * ur[c];
        g = g + pg;
        u = u + pu;
      }
      h[j] = or_silu_f32(g) * u;
    }
    for (int d = 0; d < H; ++d) out[d] = dot16(wd + (int64_t)d * I, h, I);
  }
}

static void* worker_main(void* arg) {
  worker_arg* a = (worker_arg*)arg;
  or_pool* p = a->p;
  int id = a->id;
  free(a);
  for (;;) {
    pthread_barrier_wait(&p->bar_start);
    if (p->quit) break;
    moe_task(p, id);
    pthread_barrier_wait(&p->bar_done);
  }
  return NULL;
}

or_pool* or_pool_create(int n) {
  if (n < 1) n = 1;
  or_pool* p = (or_pool*)calloc(1, sizeof(or_pool));
  if (!p) return NULL;
  p->n = n;
  if (n > 1) {
    pthread_barrier_init(&p->bar_start, NULL, (unsigned)n);
    pthread_barrier_init(&p->bar_done, NULL, (unsigned)n);
    p->th = (pthread_t*)calloc((size_t)n, sizeof(pthread_t));
    for (int i = 1; i < n; ++i) {
      worker_arg* a = (worker_arg*)malloc(sizeof(worker_arg));
      a->p = p;
      a->id = i;
      pthread_create(&p->th[i], NULL, worker_main, a);
    }
  }
  return p;
}

void or_pool_destroy(or_pool* p) {
  if (!p) return;
  if (p->n > 1) {
    p->quit = 1;
    pthread_barrier_wait(&p->bar_start);
    for (int i = 1; i < p->n; ++i) pthread_join(p->th[i], NULL);
    pthread_barrier_destroy(&p->bar_start);
    pthread_barrier_destroy(&p->bar_done);
    free(p->th);
  }
  free(p->h_scratch);
  free(p);
}

int or_pool_num_threads(const or_pool* p) { return p ? p->n : 1; }

/* WorkerPool.parallel_moe_experts, src/core/worker_pool.mojo:383-438 (the
 * coordinator acts as worker 0). */
int or_pool_parallel_moe_experts(or_pool* p, int top_k, int hidden, int inter,
                                 const float* x_tok, float* out_routed,
                                 const int64_t* selected,
                                 const float* const* wg, const float* const* wu,
                                 const float* const* wd) {
  if (!p) return 1;
  if (p->h_cap < inter) {
    free(p->h_scratch);
    p->h_scratch = (float*)malloc(sizeof(float) * (size_t)inter * (size_t)p->n);
    if (!p->h_scratch) { p->h_cap = 0; return 1; }
    p->h_cap = inter;
  }
  p->top_k = top_k; p->hidden = hidden; p->inter = inter;
  p->x_tok = x_tok; p->out_routed = out_routed; p->selected = selected;
  p->wg = wg; p->wu = wu; p->wd = wd;
  if (p->n > 1) pthread_barrier_wait(&p->bar_start);
  moe_task(p, 0);
  if (p->n > 1) pthread_barrier_wait(&p->bar_done);
  return 0;
}

/* ---- the 4-bit MoE layer ------------------------------------------------- */
typedef struct {
  float* wg; float* wu; float* wd; /* [I][H], [I][H], [H][I] */
} expert_f32;

struct or_layer_cache {
  int E;
  expert_f32* ex;
  expert_f32 sh;
};

static void expert_free(expert_f32* e) {
  free(e->wg); free(e->wu); free(e->wd);
  e->wg = e->wu = e->wd = NULL;
}

/* load_quant_routed_expert_weights / load_quant_shared_expert_weights,
 * src/layers/quant_loader.mojo:89-136: each of gate/up/down is its own
 * 4-bit tensor, dequantized through bf16 into fresh fp32 storage. */
static int load_expert(const or_layer_q4* L, int e, expert_f32* out, char* err,
                       size_t errlen) {
  int H = L->hidden, G = L->group_size;
  int I = e >= 0 ? L->inter : L->inter_sh;
  int64_t nih = (int64_t)I * H;
  const uint16_t* gus = e >= 0 ? L->gu_scales + (int64_t)e * 2 * nih / G : L->sh_gu_scales;
  const uint8_t* gup = e >= 0 ? L->gu_packed + (int64_t)e * nih : L->sh_gu_packed;
  const uint16_t* ds = e >= 0 ? L->d_scales + (int64_t)e * nih / G : L->sh_d_scales;
  const uint8_t* dp = e >= 0 ? L->d_packed + (int64_t)e * nih / 2 : L->sh_d_packed;
  out->wg = (float*)malloc(sizeof(float) * (size_t)nih);
  out->wu = (float*)malloc(sizeof(float) * (size_t)nih);
  out->wd = (float*)malloc(sizeof(float) * (size_t)nih);
  if (!out->wg || !out->wu || !out->wd) {
    expert_free(out);
    return seterr(err, errlen, "oracle: out of memory");
  }
  int st = or_dequant_q4_f32(gus, nih / G, gup, nih / 2, nih, G, out->wg, err, errlen);
  if (!st) st = or_dequant_q4_f32(gus + nih / G, nih / G, gup + nih / 2, nih / 2, nih, G,
                                  out->wu, err, errlen);
  if (!st) st = or_dequant_q4_f32(ds, nih / G, dp, nih / 2, nih, G, out->wd, err, errlen);
  if (st) expert_free(out);
  return st;
}

/* The cache is built by nthreads threads (experts split by partition_range,
 * the shared expert on thread 0); every expert's dequantization is the same
 * single-threaded routine, so the contents do not depend on nthreads. */
typedef struct {
  const or_layer_q4* L;
  or_layer_cache* c;
  int tid, n, st;
  char err[256];
} cache_job;

static void* cache_worker(void* arg) {
  cache_job* j = (cache_job*)arg;
  int64_t b, e;
  or_partition_range(j->c->E, j->tid, j->n, &b, &e);
  for (int64_t x = b; x < e && !j->st; ++x)
    j->st = load_expert(j->L, (int)x, &j->c->ex[x], j->err, sizeof(j->err));
  if (!j->st && j->tid == 0) j->st = load_expert(j->L, -1, &j->c->sh, j->err, sizeof(j->err));
  return NULL;
}

or_layer_cache* or_layer_cache_build_mt(const or_layer_q4* L, int nthreads, char* err,
                                        size_t errlen) {
  or_layer_cache* c = (or_layer_cache*)calloc(1, sizeof(or_layer_cache));
  if (!c) return NULL;
  c->E = L->num_experts;
  c->ex = (expert_f32*)calloc((size_t)c->E, sizeof(expert_f32));
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 64) nthreads = 64;
  cache_job jobs[64];
  pthread_t th[64];
  for (int t = 0; t < nthreads; ++t) {
    jobs[t].L = L; jobs[t].c = c; jobs[t].tid = t; jobs[t].n = nthreads; jobs[t].st = 0;
    jobs[t].err[0] = 0;
    if (t > 0) pthread_create(&th[t], NULL, cache_worker, &jobs[t]);
  }
  cache_worker(&jobs[0]);
  for (int t = 1; t < nthreads; ++t) pthread_join(th[t], NULL);
  for (int t = 0; t < nthreads; ++t)
    if (jobs[t].st) {
      if (err && errlen) snprintf(err, errlen, "%s", jobs[t].err);
      or_layer_cache_free(c);
      return NULL;
    }
  return c;
}

or_layer_cache* or_layer_cache_build(const or_layer_q4* L, char* err, size_t errlen) {
  return or_layer_cache_build_mt(L, 1, err, errlen);
}

void or_layer_cache_free(or_layer_cache* c) {
  if (!c) return;
  if (c->ex)
    for (int e = 0; e < c->E; ++e) expert_free(&c->ex[e]);
  free(c->ex);
  expert_free(&c->sh);
  free(c);
}

/* forward_moe_block, src/layers/moe_block.mojo:20-138, over the 4-bit
 * weights; with a pool of >1 threads the routed experts of each token run
 * through parallel_moe_experts as in src/layers/port_scheduler.mojo:398-444. */
int or_moe_layer_q4(const or_layer_q4* L, const or_layer_cache* cache,
                    or_pool* pool, const float* x, const float* residual,
                    int T, int layer, float* y, int32_t* ids, float* probs,
                    float* shgate, char* err, size_t errlen) {
  int H = L->hidden, E = L->num_experts, K = L->top_k, I = L->inter, Ish = L->inter_sh;
  int st = 0;
  if (or_router_config_validate(E, K, 0, err, errlen)) return 1;
  /* each tensor is dequantized as one flat array (quant_loader.mojo:27-41,
   * dequant_kernel.mojo:40-46): N % G == 0, a group may span two rows */
  if (T <= 0 || H <= 0 || I <= 0 || Ish <= 0 || !or_is_allowed_group_size(L->group_size) ||
      ((int64_t)I * H) % L->group_size || ((int64_t)Ish * H) % L->group_size)
    return seterr(err, errlen,
                  "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"invalid MoE layer"
                  " dimensions\",\"stage\":\"moe\",\"layer\":%d}", layer);
  int64_t TH = (int64_t)T * H;
  float* wr = (float*)malloc(sizeof(float) * (size_t)E * H);
  float* wsh = (float*)malloc(sizeof(float) * (size_t)H);
  float* routed = (float*)malloc(sizeof(float) * (size_t)TH * K);
  float* shout = (float*)malloc(sizeof(float) * (size_t)TH);
  float* gates = (float*)malloc(sizeof(float) * (size_t)T);
  int* uniq = (int*)malloc(sizeof(int) * (size_t)T * K);
  expert_f32* loaded = (expert_f32*)calloc((size_t)T * K, sizeof(expert_f32));
  expert_f32 shw = {0, 0, 0};
  const float** pg = (const float**)calloc((size_t)E, sizeof(float*));
  const float** pu = (const float**)calloc((size_t)E, sizeof(float*));
  const float** pd = (const float**)calloc((size_t)E, sizeof(float*));
  int64_t* sel = (int64_t*)malloc(sizeof(int64_t) * (size_t)K);
  int32_t* ids_own = ids ? NULL : (int32_t*)malloc(sizeof(int32_t) * (size_t)T * K);
  float* probs_own = probs ? NULL : (float*)malloc(sizeof(float) * (size_t)T * K);
  int64_t IH = (int64_t)I * H, ISH = (int64_t)Ish * H;
  int nuniq = 0;
  if (!ids) ids = ids_own;
  if (!probs) probs = probs_own;
  if (!ids || !probs || !wr || !wsh || !routed || !shout || !gates || !uniq || !loaded || !pg || !pu || !pd || !sel) {
    st = seterr(err, errlen, "oracle: out of memory");
    goto done;
  }
  /* load_layer_router_weights: bf16 -> f32 exact widening (router.mojo:213-257) */
  for (int64_t i = 0; i < (int64_t)E * H; ++i) wr[i] = or_bf16_to_f32(L->router_bf16[i]);
  for (int i = 0; i < H; ++i) wsh[i] = or_bf16_to_f32(L->shgate_bf16[i]);
  st = or_router_forward(x, TH, wr, (int64_t)E * H, T, H, E, K, 0, layer, ids, probs, err, errlen);
  if (st) goto done;
  /* unique experts in first-appearance order (moe_block.mojo:47-59) */
  for (int64_t i = 0; i < (int64_t)T * K; ++i) {
    int f = 0;
    for (int u = 0; u < nuniq; ++u)
      if (uniq[u] == ids[i]) { f = 1; break; }
    if (!f) uniq[nuniq++] = ids[i];
  }
  for (int u = 0; u < nuniq; ++u) {
    if (cache) {
      loaded[u] = cache->ex[uniq[u]];
    } else if ((st = load_expert(L, uniq[u], &loaded[u], err, errlen))) {
      goto done;
    }
    pg[uniq[u]] = loaded[u].wg;
    pu[uniq[u]] = loaded[u].wu;
    pd[uniq[u]] = loaded[u].wd;
  }
  for (int t = 0; t < T; ++t) {
    const float* xt = x + (int64_t)t * H;
    float* rt = routed + (int64_t)t * K * H;
    if (pool && or_pool_num_threads(pool) > 1) {
      for (int k = 0; k < K; ++k) sel[k] = ids[(int64_t)t * K + k];
      or_pool_parallel_moe_experts(pool, K, H, I, xt, rt, sel, pg, pu, pd);
    } else {
      for (int k = 0; k < K; ++k) {
        int e = ids[(int64_t)t * K + k];
        st = or_swiglu_forward(xt, H, pg[e], pu[e], pd[e], IH, IH, IH, 1, H, I, layer, e,
                               rt + (int64_t)k * H, err, errlen);
        if (st) goto done;
      }
    }
  }
  if (cache) {
    shw = cache->sh;
  } else if ((st = load_expert(L, -1, &shw, err, errlen))) {
    goto done;
  }
  st = or_swiglu_forward(x, TH, shw.wg, shw.wu, shw.wd, ISH, ISH, ISH, T, H, Ish, layer, -1,
                         shout, err, errlen);
  if (st) goto done;
  st = or_shared_gate_forward(x, TH, wsh, H, T, H, layer, "sigmoid", gates, err, errlen);
  if (st) goto done;
  st = or_moe_aggregate(residual, routed, probs, shout, gates, T, H, K, layer, y, err, errlen);
  if (!st && shgate) memcpy(shgate, gates, sizeof(float) * (size_t)T);
done:
  if (!cache) {
    if (loaded)
      for (int u = 0; u < nuniq; ++u) expert_free(&loaded[u]);
    expert_free(&shw);
  }
  free(wr); free(wsh); free(routed); free(shout); free(gates); free(uniq); free(loaded);
  free(pg); free(pu); free(pd); free(sel); free(ids_own); free(probs_own);
  return st;
}

/* Stack of MoE blocks with the token mixer replaced by identity: the MoE
 * section of forward_port_block (src/layers/port_scheduler.mojo:381-482):
 * x_norm = rmsnorm(h, gamma_l, eps) (apply_rmsnorm_sequence, :383-385;
 * gammas[l] NULL or gammas NULL: gamma = 1), then
 * h <- moe_aggregate_forward(h, MoE(x_norm)) (:469-479).  tree != 0 reduces
 * the sum of squares in the library's fast-mode order (or_rmsnorm_tree256)
 * instead of the reference's sequential order (or_rmsnorm). */
int or_moe_stack_q4(const or_layer_q4* layers, int nl, const float* const* gammas, int tree,
                    or_pool* pool, const float* x, int T, float eps, float* out, int32_t* ids,
                    float* probs, char* err, size_t errlen) {
  int H = layers[0].hidden;
  int64_t TH = (int64_t)T * H;
  float* h = (float*)malloc(sizeof(float) * (size_t)TH);
  float* xn = (float*)malloc(sizeof(float) * (size_t)TH);
  float* nh = (float*)malloc(sizeof(float) * (size_t)TH);
  int st = (!h || !xn || !nh) ? seterr(err, errlen, "oracle: out of memory") : 0;
  if (!st) memcpy(h, x, sizeof(float) * (size_t)TH);
  for (int l = 0; l < nl && !st; ++l) {
    int K = layers[l].top_k;
    const float* g = gammas ? gammas[l] : NULL;
    for (int t = 0; t < T && !st; ++t)
      st = tree ? or_rmsnorm_tree256(h + (int64_t)t * H, g, H, eps, xn + (int64_t)t * H, err,
                                     errlen)
                : or_rmsnorm(h + (int64_t)t * H, g, H, eps, xn + (int64_t)t * H, err, errlen);
    if (!st)
      st = or_moe_layer_q4(&layers[l], NULL, pool, xn, h, T, l, nh,
                           ids ? ids + (int64_t)l * T * K : NULL,
                           probs ? probs + (int64_t)l * T * K : NULL, NULL, err, errlen);
    float* tmp = h; h = nh; nh = tmp;
  }
  if (!st) memcpy(out, h, sizeof(float) * (size_t)TH);
  free(h); free(xn); free(nh);
  return st;
}
