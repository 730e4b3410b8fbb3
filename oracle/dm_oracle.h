/*
 * dm_oracle.h -- CPU restatement of the reference engine's 4-bit MoE FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * implementation in libdismoen_hip.so.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it; the product path never does.
 *
 * Every function restates one reference function (cited file:line, paths
 * relative to the reference repository root) with the same arithmetic order:
 *   - dot products use 16 strided fp32 lane partials accumulated sequentially,
 *     then a halving tree (lane i += lane i+8, +4, +2, +1), then a scalar tail,
 *     as `SIMD[float32,16]` accumulate + `reduce_add()` in the Mojo sources;
 *   - no fused multiply-add anywhere (built with -ffp-contract=off);
 *   - exp() is or_expf(): Cody-Waite reduction + degree-7 Taylor polynomial,
 *     the same function the HIP kernels evaluate (see or_expf in the .c).
 * Errors are reported as the reference's JSON error strings in `err`, and the
 * function returns a nonzero status.
 *
 * Parity status (which checks pin each function) is listed in the header of
 * dm_oracle.c.
 */
#ifndef DM_ORACLE_H
#define DM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers (src/format/half_float.mojo, src/layers/swiglu.mojo) ---- */
float or_fp16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16_rne(float f);
float or_bf16_to_f32(uint16_t b);
float or_expf(float x);
float or_sigmoid_f32(float z);
float or_silu_f32(float z);
int or_pack_4bit_pair(int w0, int w1, uint8_t* out);
int or_unpack_4bit_pair(uint8_t b, int* w0, int* w1);
int or_is_allowed_group_size(int g);
uint16_t or_compute_fp16_scale_ceil(float max_abs, int* status);

/* ---- dequant (src/quant/dequant_kernel.mojo:22-155) ---- */
int or_dequant_q4_bf16(const uint16_t* scales, int64_t n_scales,
                       const uint8_t* packed, int64_t n_packed,
                       int64_t num_elements, int group_size,
                       uint16_t* out_bf16, char* err, size_t errlen);
int or_dequant_q4_f32(const uint16_t* scales, int64_t n_scales,
                      const uint8_t* packed, int64_t n_packed,
                      int64_t num_elements, int group_size,
                      float* out_f32, char* err, size_t errlen);

/* ---- GGUF tensor payloads -> fp32 (src/format/gguf.mojo:414-626) ----
 * ggml_type: 0 F32, 30 BF16, 8 Q8_0 (32 weights / 34 B), 12 Q4_K (256 / 144 B),
 * 11 Q3_K (256 / 114 B), the reference's own block layouts.  Elements past
 * the last whole block stay 0.0, as in the reference.  q4k_layout 0 follows
 * dequantize_q4_k of gguf.mojo:444-506; 1 follows the reference's Python twin
 * (tools/oracle/oracle_port.py:86-127), which packs the scales and mins of
 * sub-blocks 4..7 differently (gguf.mojo:482-488 vs oracle_port.py:104-110). */
int or_gguf_block_spec(int ggml_type, int* block_size, int* bytes_per_block);
int or_dequant_gguf(int ggml_type, const uint8_t* raw, int64_t raw_bytes,
                    int64_t num_elements, int q4k_layout, float* out, char* err,
                    size_t errlen);

/* ---- router (src/layers/router.mojo, topk.mojo, router_types.mojo) ---- */
int or_router_config_validate(int num_experts, int top_k, int norm_topk_prob,
                              char* err, size_t errlen);
int or_router_project(const float* x, int64_t n_x, const float* w, int64_t n_w,
                      int seq_len, int hidden, int num_experts, int layer,
                      float* logits, char* err, size_t errlen);
int or_router_softmax(const float* logits, int64_t n_logits, int seq_len,
                      int num_experts, int layer, float* probs, char* err,
                      size_t errlen);
int or_select_topk(const float* probs, int64_t n_probs, int seq_len,
                   int num_experts, int top_k, int norm_topk_prob, int layer,
                   int32_t* ids, float* vals, char* err, size_t errlen);
int or_router_forward(const float* x, int64_t n_x, const float* w, int64_t n_w,
                      int seq_len, int hidden, int num_experts, int top_k,
                      int norm_topk_prob, int layer, int32_t* ids, float* vals,
                      char* err, size_t errlen);

/* ---- experts (src/layers/swiglu.mojo, moe.mojo, forward_layer.mojo) ---- */
int or_swiglu_forward(const float* x, int64_t n_x, const float* w_gate,
                      const float* w_up, const float* w_down, int64_t n_gate,
                      int64_t n_up, int64_t n_down, int seq_len, int hidden,
                      int inter, int layer, int expert_id, float* out,
                      char* err, size_t errlen);
int or_shared_gate_forward(const float* x, int64_t n_x, const float* w,
                           int64_t n_w, int seq_len, int hidden, int layer,
                           const char* gate_mode, float* scores, char* err,
                           size_t errlen);
/* routed: [seq_len][top_k*hidden]; probs: [seq_len][top_k];
 * residual == NULL -> moe_combine_no_residual, else moe_aggregate_forward. */
int or_moe_aggregate(const float* residual, const float* routed,
                     const float* probs, const float* shared_out,
                     const float* shared_gates, int seq_len, int hidden,
                     int top_k, int layer, float* out, char* err,
                     size_t errlen);

/* ---- glue (src/layers/rmsnorm.mojo, residual.mojo) ---- */
int or_rmsnorm(const float* x, const float* gamma, int n, float eps, float* out,
               char* err, size_t errlen);
int or_rmsnorm_tree256(const float* x, const float* gamma, int n, float eps, float* out, char* err,
                       size_t errlen);
int or_add_residual(const float* y, const float* x, int64_t n, int layer,
                    float* out, char* err, size_t errlen);

/* ---- worker pool (src/core/worker_pool.mojo) ---- */
void or_partition_range(int64_t total, int64_t tid, int64_t nthreads,
                        int64_t* start, int64_t* end);
typedef struct or_pool or_pool;
or_pool* or_pool_create(int num_threads);
void or_pool_destroy(or_pool* p);
int or_pool_num_threads(const or_pool* p);
/* parallel_moe_experts: w_*_ptrs index by expert id; out_routed [top_k*hidden] */
int or_pool_parallel_moe_experts(or_pool* p, int top_k, int hidden, int inter,
                                 const float* x_tok, float* out_routed,
                                 const int64_t* selected,
                                 const float* const* w_gate_ptrs,
                                 const float* const* w_up_ptrs,
                                 const float* const* w_down_ptrs);

/* ---- the 4-bit MoE layer composition ---- */
typedef struct {
  int hidden, num_experts, top_k, inter, inter_sh, group_size;
  const uint16_t* router_bf16;   /* [E][H] */
  const uint16_t* shgate_bf16;   /* [H]    */
  const uint16_t* gu_scales;     /* [E][2I][H/G] fp16 bits (gate rows, then up rows) */
  const uint8_t* gu_packed;      /* [E][2I][H/2] */
  const uint16_t* d_scales;      /* [E][H][I/G] */
  const uint8_t* d_packed;       /* [E][H][I/2] */
  const uint16_t* sh_gu_scales;  /* [2Ish][H/G] */
  const uint8_t* sh_gu_packed;   /* [2Ish][H/2] */
  const uint16_t* sh_d_scales;   /* [H][Ish/G] */
  const uint8_t* sh_d_packed;    /* [H][Ish/2] */
} or_layer_q4;

/* Optional fp32 cache of every dequantized expert (the "pre-dequantized
 * resident" CPU variant).  Built once by or_layer_cache_build. */
typedef struct or_layer_cache or_layer_cache;
or_layer_cache* or_layer_cache_build(const or_layer_q4* L, char* err,
                                     size_t errlen);
/* The same cache built by nthreads threads (identical contents). */
or_layer_cache* or_layer_cache_build_mt(const or_layer_q4* L, int nthreads, char* err,
                                        size_t errlen);
void or_layer_cache_free(or_layer_cache* c);

/* forward_moe_block for the 4-bit layer.  residual == NULL gives the
 * no-residual combine.  cache may be NULL (dequant-per-use) and pool may be
 * NULL (serial experts). */
int or_moe_layer_q4(const or_layer_q4* L, const or_layer_cache* cache,
                    or_pool* pool, const float* x, const float* residual,
                    int seq_len, int layer, float* y, int32_t* ids,
                    float* probs, float* shgate, char* err, size_t errlen);

/* 40-layer style stack: h <- h + MoE_l(RMSNorm_{gamma_l,eps}(h)), the norm
 * in the reference's sequential order, or the tree order when tree != 0.
 * gammas: [num_layers] pointers to [H] (NULL entries or NULL: gamma = 1). */
int or_moe_stack_q4(const or_layer_q4* layers, int num_layers,
                    const float* const* gammas, int tree, or_pool* pool,
                    const float* x, int seq_len, float eps, float* out,
                    int32_t* ids, float* probs, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif
#endif
