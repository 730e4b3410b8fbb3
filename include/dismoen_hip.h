/*
 * dismoen_hip.h -- C ABI of libdismoen_hip.so, the gfx950 (MI355X) MoE FFN
 * block of the disk-streaming MoE engine: router (logits, softmax, top-k),
 * 4-bit group-quantised SwiGLU experts, the sigmoid-gated shared expert and
 * the weighted combine.
 *
 * Plain C types only.  Every function returns DMH_OK (0) or a DMH_ERR_*
 * code and, when err != NULL, writes the reference's error text into
 * err[0..errlen): the JSON objects raised by the Mojo layers
 * ({"error_type":...,"detail":...,"stage":...,"layer":...}) or the plain
 * dequant strings, so a Mojo shim can `raise Error(String(err))` unchanged.
 *
 * Memory: by default every pointer is host memory and the call is
 * synchronous (a single token's block runs with x and the outputs in a
 * page-locked block of the context that the kernel reads and writes itself:
 * one launch and one synchronisation per call, no copy operations).  With
 * DMH_F_DEVICE every activation/output pointer is device
 * memory, the call is ordered on the context's stream and returns at once;
 * errors found on the device are then sticky and reported by dmh_sync().
 *
 * Threading: one context per host thread; a context is not re-entrant.
 * Reference paths below are relative to the reference repository root.
 */
#ifndef DISMOEN_HIP_H
#define DISMOEN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DMH_ABI_VERSION 1

enum {
  DMH_OK = 0,
  DMH_ERR_INVALID_ARG = 1,  /* null pointer, bad length, unknown layer */
  DMH_ERR_CONFIG = 2,       /* CONFIG_ERROR: dimensions the path does not support */
  DMH_ERR_HIP = 3,          /* HIP runtime failure */
  DMH_ERR_NO_MEMORY = 4,
  DMH_ERR_DEQUANT = 5,      /* invalid 4-bit payload (reserved code, bad scale) */
  DMH_ERR_ACT = 6,          /* ACT_LOAD_FAILED */
  DMH_ERR_WEIGHT = 7,       /* WEIGHT_LOAD_FAILED */
  DMH_ERR_ROUTER = 8,       /* ROUTER_ERROR */
  DMH_ERR_EXPERT = 9,       /* EXPERT_ERROR */
  DMH_ERR_SWIGLU = 10,      /* SWIGLU_ERROR */
  DMH_ERR_GATE = 11,        /* GATE_ERROR */
  DMH_ERR_NORM = 12,        /* NORM_ERROR */
  DMH_ERR_FORMAT = 13,      /* a weight file fails its format checks */
};

#define DMH_F_DEVICE 0x1u   /* pointers are device memory; stream-ordered, no sync */
/* Block-edge RMSNorm in the library's fast order: the sum of squares as 256
 * strided partials and a halving tree.  Without it the squares are added in
 * element order, as rmsnorm does (src/layers/rmsnorm.mojo:41-44). */
#define DMH_F_NORM_TREE 0x20u

typedef struct dmh_ctx dmh_ctx;

/* Fields of ModelConfig that the block uses (src/core/config.mojo:11-174,
 * src/layers/router_types.mojo:9-44).  group_size is one of the quantizer's
 * sizes {32, 64, 128, 256} (src/format/half_float.mojo:9,24-31; the format's
 * default is 128); hidden, inter and inter_sh must be multiples of 128;
 * norm_topk_prob must be 0. */
typedef struct {
  int32_t hidden;          /* H */
  int32_t num_experts;     /* E */
  int32_t top_k;           /* K: num_experts_per_tok */
  int32_t inter;           /* I: moe_intermediate_size */
  int32_t inter_sh;        /* I_sh: shared_expert_intermediate_size */
  int32_t group_size;      /* G */
  int32_t norm_topk_prob;  /* forbidden (raises) when nonzero */
} dmh_moe_dims;

/* One layer's weights in the reference layouts.  4-bit tensors follow
 * docs/format/quant_format.md:117-161: fp16 scales [N/G] then packed codes
 * [N/2] (element i in byte i/2, low nibble = even i), groups along the input
 * dimension.  gu_* is the fused experts.gate_up_proj [E][2I][H] (gate rows
 * 0..I-1 then up rows I..2I-1 per expert, src/layers/moe_loader.mojo:47-72),
 * which is the per-expert gate_proj [I][H] and up_proj [I][H] tensors of
 * src/layers/quant_loader.mojo:89-111 laid end to end; d_* is
 * experts.down_proj [E][H][I]; sh_* the shared expert
 * (src/layers/quant_loader.mojo:114-136).  router_bf16 [E][H] is mlp.gate
 * (src/layers/router.mojo:213-257) and shgate_bf16 [H] mlp.shared_expert_gate. */
typedef struct {
  const uint16_t* router_bf16;
  const uint16_t* shgate_bf16;
  const uint16_t* gu_scales;    /* [E*2I*H/G] fp16 bits */
  const uint8_t* gu_packed;     /* [E*2I*H/2] */
  const uint16_t* d_scales;     /* [E*H*I/G] */
  const uint8_t* d_packed;      /* [E*H*I/2] */
  const uint16_t* sh_gu_scales; /* [2*Ish*H/G] */
  const uint8_t* sh_gu_packed;  /* [2*Ish*H/2] */
  const uint16_t* sh_d_scales;  /* [H*Ish/G] */
  const uint8_t* sh_d_packed;   /* [H*Ish/2] */
} dmh_moe_weights;

/* Library version string, e.g. "dismoen_hip 1 gfx950". */
const char* dmh_version(void);

/* Create a context on HIP device `device` with its own stream.  Replaces the
 * engine's WorkerPool construction (src/core/worker_pool.mojo:228-294): the
 * context owns all device memory of the block. */
int dmh_create(int device, dmh_ctx** out, char* err, size_t errlen);
int dmh_destroy(dmh_ctx* ctx);

/* Use another HIP stream (a hipStream_t) for subsequent calls; NULL restores
 * the context's own stream.  Work already queued on the previous stream is
 * ordered before anything issued on the new one.  Calls made while the
 * stream is being captured into a HIP graph take the multi-kernel path (the
 * single-launch decode kernel tags its hand-offs per launch on the host, so
 * a replayed capture would repeat a tag); buffers a call allocates on first
 * use must be allocated by an uncaptured call first. */
int dmh_set_stream(dmh_ctx* ctx, void* hip_stream);
void* dmh_get_stream(dmh_ctx* ctx);

/* Wait for the stream; return the first device-side error recorded since
 * the last dmh_sync (DMH_F_DEVICE calls), then clear it. */
int dmh_sync(dmh_ctx* ctx, char* err, size_t errlen);

/* The single-token kernels run all their workgroups at once and pass data
 * between them through polled words; every such wait gives up after a bound
 * of polls (default 2^20, about one second) and records a sync error.  A
 * host-pointer call whose wait gave up (another process's kernels held CUs
 * the grid needed) restarts the layer's tags and reruns the call on the
 * multi-kernel path, which has no such waits; DMH_F_DEVICE calls report the
 * error at dmh_sync.  dmh_set_spin_limit sets the bound: polls >= 0 polls
 * (0: every wait gives up at once, for tests of this path), polls < 0 the
 * default.  dmh_sync_fallbacks reports how many host-pointer calls of the
 * context were rerun this way.  No counterpart in the reference (its block
 * runs on CPU threads that do not wait on each other this way). */
int dmh_set_spin_limit(dmh_ctx* ctx, int64_t polls);
int dmh_sync_fallbacks(dmh_ctx* ctx, int64_t* count);

/* The decision the library makes once per device at dmh_create: given the
 * XCD each workgroup of a one-workgroup-per-CU launch ran on
 * (xcd_of_workgroup[b], read from the hardware), the XCD count n when
 * workgroup b ran on XCD (b + r) % n for a single r and n divides
 * num_workgroups (the dispatcher's rotation the XCD-sliced decode kernel
 * relies on), else 0 (that kernel form is not used).  No counterpart in the
 * reference (a host-side diagnostic of the gfx950 launch geometry). */
int dmh_xcd_rotation(const uint32_t* xcd_of_workgroup, int num_workgroups);

/* Upload one layer once into HBM, re-tiled for the gfx950 kernels and
 * validated (reserved code 0x8, fp16 scale NaN/Inf or <= 0: the checks of
 * src/quant/dequant_kernel.mojo:68-108; non-finite router weights: the scan
 * of src/layers/router.mojo:65-72, reported when the layer is used).
 * Replaces the per-use pread + dequant of load_quant_routed_expert_weights /
 * load_quant_shared_expert_weights (src/layers/quant_loader.mojo:89-136) and
 * load_layer_router_weights (src/layers/router.mojo:213-257).
 * flags & DMH_F_DEVICE: the weight pointers are device memory. */
int dmh_upload_moe_layer(dmh_ctx* ctx, int layer, const dmh_moe_dims* dims,
                         const dmh_moe_weights* w, unsigned flags, char* err,
                         size_t errlen);
int dmh_free_layer(dmh_ctx* ctx, int layer);
/* Device bytes held by an uploaded layer. */
int dmh_layer_bytes(dmh_ctx* ctx, int layer, int64_t* bytes);

/* The MoE block for seq_len tokens of one uploaded layer: router_forward ->
 * routed SwiGLU experts -> shared expert + sigmoid gate -> combine.
 * Replaces forward_moe_block (src/layers/moe_block.mojo:20-138) and the MoE
 * section of forward_port_block (src/layers/port_scheduler.mojo:381-482).
 *   x        [seq_len][H] fp32 input of the router and experts
 *   residual [seq_len][H] fp32 or NULL.  Non-NULL: moe_aggregate_forward
 *            (src/layers/moe.mojo:105-177), y = routed + shared + residual;
 *            NULL: moe_combine_no_residual (src/layers/forward_layer.mojo:181-247).
 *   y        [seq_len][H] fp32 output
 *   ids      [seq_len][K] int32 selected experts (RoutingInfo.selected_experts,
 *            src/layers/router_types.mojo:47-81), p descending, lowest id on ties;
 *            may be NULL
 *   probs    [seq_len][K] fp32 raw softmax probabilities (no renormalisation); may be NULL
 *   shared_gate [seq_len] fp32 sigmoid(w_sh . x); may be NULL */
int dmh_moe_forward(dmh_ctx* ctx, int layer, const float* x, const float* residual,
                    int seq_len, float* y, int32_t* ids, float* probs,
                    float* shared_gate, unsigned flags, char* err, size_t errlen);

/* dmh_moe_forward that allocates nothing: no counterpart in the reference;
 * for callers that cannot allocate device or host memory during a call
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  DMH_F_DEVICE is required (host pointers would need staging
 * buffers).  Every buffer of the call (logits, grouping, h, partial outputs,
 * and ids / probs / shared_gate when NULL) is carved from one static 8 MiB
 * array per device that the library holds until the process ends; a call
 * that needs more (about 80 tokens at the Qwen3.6 layer shape) fails with
 * DMH_ERR_INVALID_ARG and changes nothing.  All calls on a device share its
 * array, which keeps the last call's contents, so the library puts them in
 * one order: each call's stream waits for an event the device's previous
 * call (from any context or stream) recorded after its kernels.  A call made
 * while its stream is captured into a HIP graph is not chained that way (a
 * capture cannot wait on outside work): replays of such a graph must not
 * overlap other calls of this entry point on the device.  Outputs equal
 * dmh_moe_forward's bit for bit. */
int dmh_moe_forward_noalloc(dmh_ctx* ctx, int layer, const float* x, const float* residual,
                            int seq_len, float* y, int32_t* ids, float* probs,
                            float* shared_gate, unsigned flags, char* err, size_t errlen);

/* The post-attention RMSNorm weight of an uploaded layer: gamma [hidden] fp32
 * (PortBlockWeights.post_attention_layernorm_gamma,
 * src/layers/port_scheduler.mojo:65-86, used at :383-385), copied to the
 * device; NULL restores gamma = 1.  hidden must equal the layer's (else the
 * NORM_ERROR "length mismatch" of rmsnorm.mojo:31-35).  flags & DMH_F_DEVICE:
 * gamma is device memory. */
int dmh_set_layer_norm(dmh_ctx* ctx, int layer, const float* gamma, int hidden,
                       unsigned flags, char* err, size_t errlen);

/* The MoE section of forward_port_block (src/layers/port_scheduler.mojo:
 * 381-482) with its RMSNorm: xn = rmsnorm(x_mid, gamma, eps)
 * (apply_rmsnorm_sequence, :383-385, gamma the layer's), y = MoE(xn) +
 * x_mid.  Outputs as dmh_moe_forward.  eps NaN/Inf/<= 0 gives rmsnorm's
 * CONFIG_ERROR.  flags: DMH_F_DEVICE, DMH_F_NORM_TREE. */
int dmh_port_moe_forward(dmh_ctx* ctx, int layer, const float* x_mid, int seq_len, float eps,
                         float* y, int32_t* ids, float* probs, float* shared_gate,
                         unsigned flags, char* err, size_t errlen);

/* num_layers consecutive uploaded layers, token mixer replaced by identity:
 * per layer h <- dmh_port_moe_forward(h), i.e. h + MoE(rmsnorm(h, gamma_l,
 * eps)), the composition of src/layers/port_scheduler.mojo:381-482 with
 * gamma_l each layer's (dmh_set_layer_norm).  ids/probs
 * [num_layers][seq_len][K] may be NULL.  flags: DMH_F_DEVICE,
 * DMH_F_NORM_TREE. */
int dmh_moe_stack_forward(dmh_ctx* ctx, int first_layer, int num_layers, float eps,
                          const float* x, int seq_len, float* out, int32_t* ids,
                          float* probs, unsigned flags, char* err, size_t errlen);

/* router_forward (src/layers/router.mojo:188-210) with fp32 weights
 * w_router [E][H]: router_project + router_softmax + select_topk. */
int dmh_router_forward(dmh_ctx* ctx, const float* x, const float* w_router, int seq_len,
                       int hidden, int num_experts, int top_k, int norm_topk_prob,
                       int layer, int32_t* ids, float* probs, unsigned flags, char* err,
                       size_t errlen);

/* dequant_kernel_simd (src/quant/dequant_kernel.mojo:22-124): 4-bit codes +
 * fp16 scales -> bf16 bits, out[i] = bf16_rne(fp32(s_g) * q_i). */
int dmh_dequant_q4_bf16(dmh_ctx* ctx, const uint16_t* scales, int64_t n_scales,
                        const uint8_t* packed, int64_t n_packed, int64_t num_elements,
                        int group_size, uint16_t* out, unsigned flags, char* err,
                        size_t errlen);

/* The SwiGLU experts of given assignments on an uploaded layer's 4-bit
 * weights, unweighted: out[t][k][H] = W_down_e (SiLU(W_gate_e x_t) * (W_up_e
 * x_t)) with e = ids[t][k], k < top_k (1..64; any expert ids in [0, E), repeats
 * allowed).  Replaces WorkerPool.parallel_moe_experts
 * (src/core/worker_pool.mojo:383-438, out_routed[k*H + d] for one token) and
 * the per-(token, expert) swiglu_forward calls (src/layers/swiglu.mojo:52-230)
 * of forward_moe_block.  shared_out [seq_len][H] (may be NULL) receives the
 * shared expert's output.  A non-finite gate/up/product/output raises the
 * EXPERT_ERROR / SWIGLU_ERROR text of swiglu_forward with the expert id; an id
 * outside [0, E) raises EXPERT_ERROR "expert id out of range". */
int dmh_experts_forward(dmh_ctx* ctx, int layer, const float* x, int seq_len,
                        const int32_t* ids, int top_k, float* out, float* shared_out,
                        unsigned flags, char* err, size_t errlen);

/* shared_gate_forward (src/layers/moe.mojo:17-102) with gate_mode "sigmoid" and
 * the uploaded layer's bf16 gate vector: scores[t] = sigmoid(w_sh . x_t), the
 * dot product in the 16-lane order of the reference; GATE_ERROR texts. */
int dmh_shared_gate_forward(dmh_ctx* ctx, int layer, const float* x, int seq_len,
                            float* scores, unsigned flags, char* err, size_t errlen);

/* moe_aggregate_forward (src/layers/moe.mojo:105-177) on given parts, or
 * moe_combine_no_residual (src/layers/forward_layer.mojo:181-247) when
 * residual is NULL: y[t][d] = (sum_k probs[t][k] routed[t][k][d]) +
 * shared_gates[t] shared_out[t][d] (+ residual[t][d]), in that order.  layer
 * is used in the error text only. */
int dmh_moe_aggregate(dmh_ctx* ctx, const float* residual, const float* routed,
                      const float* probs, const float* shared_out, const float* shared_gates,
                      int seq_len, int hidden, int top_k, int layer, float* out,
                      unsigned flags, char* err, size_t errlen);

/* ---- weight files ---------------------------------------------------------
 * Readers of the reference's weight files on the host (no GPU needed), and
 * the upload of one layer straight from them.  They replace, for this block,
 * the per-use pread + dequant of src/layers/quant_loader.mojo and the
 * router's safetensors load (src/layers/router.mojo:213-257). */
typedef struct dmh_quant_file dmh_quant_file;
typedef struct dmh_st_file dmh_st_file;

/* One tensor of a weight file; name and dtype stay valid while the file
 * handle is open.  Offsets are absolute file offsets. */
typedef struct {
  const char* name;
  const char* dtype;        /* safetensors dtype, or the quant meta's "dtype" */
  int32_t ndim;
  int64_t shape[8];
  int32_t group_size;       /* quant files */
  int64_t num_groups;       /* quant files */
  int64_t scales_offset;    /* quant files: fp16 LE group scales */
  int64_t scales_bytes;
  int64_t data_offset;      /* quant: packed codes; safetensors: the payload */
  int64_t data_bytes;
} dmh_tensor_info;

/* scan_quant_file (src/format/quant_reader.mojo:487-662): header, every
 * record and the SEC-4 checks; on failure err receives the reference's text
 * ("scan_quant_file: ...") and DMH_ERR_FORMAT is returned. */
int dmh_quant_open(const char* path, dmh_quant_file** out, char* err, size_t errlen);
void dmh_quant_close(dmh_quant_file* f);
int dmh_quant_num_tensors(const dmh_quant_file* f);
/* QuantModelIndex.tensor_map lookup (quant_reader.mojo:631): index, or -1. */
int dmh_quant_find(const dmh_quant_file* f, const char* name);
int dmh_quant_tensor_info(const dmh_quant_file* f, int idx, dmh_tensor_info* info);
/* pread_tensor_quant (quant_reader.mojo:665-692): fp16 scale bits
 * [num_groups] and packed codes [data_bytes]. */
int dmh_quant_read(const dmh_quant_file* f, int idx, uint16_t* scales, int64_t n_scales,
                   uint8_t* packed, int64_t n_packed, char* err, size_t errlen);

/* read_header (src/format/reader.mojo:21-297): safetensors header parse and
 * the F15 checks (dtype, offsets, layout, no holes or overlap); errors are
 * the reference's {"error_type","detail","shard","tensor_name"} objects. */
int dmh_st_open(const char* path, dmh_st_file** out, char* err, size_t errlen);
void dmh_st_close(dmh_st_file* f);
int dmh_st_num_tensors(const dmh_st_file* f);
int dmh_st_find(const dmh_st_file* f, const char* name);
int dmh_st_tensor_info(const dmh_st_file* f, int idx, dmh_tensor_info* info);
/* The payload bytes of tensor idx; bytes must equal its size. */
int dmh_st_read(const dmh_st_file* f, int idx, void* out, int64_t bytes, char* err,
                size_t errlen);

/* dmh_upload_moe_layer from the files of model layer model_layer: routed
 * experts model.layers.{l}.mlp.experts.{e}.{gate,up,down}_proj.weight and
 * model.layers.{l}.mlp.shared_expert.{gate,up,down}_proj.weight from the
 * quant model (src/layers/quant_loader.mojo:89-136); the router mlp.gate.weight
 * (language-model prefix first, src/layers/router.mojo:234-247) and
 * mlp.shared_expert_gate.weight as BF16 from the safetensors shard, the
 * shared gate falling back to the quant model's 4-bit tensor.
 * dims->group_size 0 takes the quant model's own group size,
 * quantization.group_size of its header (docs/format/quant_format.md:76). */
int dmh_upload_moe_layer_files(dmh_ctx* ctx, int layer, const dmh_moe_dims* dims,
                               const dmh_quant_file* quant, const dmh_st_file* shard,
                               int model_layer, char* err, size_t errlen);

/* ---- GGUF ------------------------------------------------------------------
 * The container and the expert formats of the reference's Qwen3.6 port
 * decode (src/format/gguf.mojo, read by src/layers/gguf_port_loader.mojo).
 * GGML type codes with a dequantizer: */
#define DMH_GGML_F32 0
#define DMH_GGML_Q8_0 8   /* 32 weights in 34 bytes: fp16 d, 32 int8 */
#define DMH_GGML_Q3_K 11  /* 256 weights in 114 bytes (the reference's layout) */
#define DMH_GGML_Q4_K 12  /* 256 weights in 144 bytes (the reference's layout) */
#define DMH_GGML_BF16 30
/* Q4_K sub-blocks 4..7 with the scale/min packing of the reference's Python
 * twin (tools/oracle/oracle_port.py:104-110) instead of gguf.mojo:482-488. */
#define DMH_F_Q4K_PY_SCALES 0x10u

typedef struct dmh_gguf_file dmh_gguf_file;

/* GGUFTensorInfo (gguf.mojo:104-114); name valid while the file is open.
 * offset is relative to the data section, file_offset absolute. */
typedef struct {
  const char* name;
  int32_t ndim;
  int64_t dims[8];
  int32_t ggml_type;
  int64_t offset;
  int64_t file_offset;
  int64_t num_elements;
  int64_t raw_bytes;
} dmh_gguf_tensor;

/* The scalar fields of GGUFIndex (gguf.mojo:117-141). */
typedef struct {
  int32_t version;
  int64_t tensor_count;
  int64_t metadata_kv_count;
  int64_t data_section_offset;
  int64_t expected_file_size;
  int64_t alignment;
} dmh_gguf_header;

/* parse_gguf_index (gguf.mojo:257-411): magic, version 2/3, metadata, tensor
 * directory, general.alignment, and the exact file size rule (F11b); on
 * failure err receives the reference's "GGUF..." text, DMH_ERR_FORMAT. */
int dmh_gguf_open(const char* path, dmh_gguf_file** out, char* err, size_t errlen);
void dmh_gguf_close(dmh_gguf_file* f);
int dmh_gguf_get_header(const dmh_gguf_file* f, dmh_gguf_header* h);
int dmh_gguf_num_tensors(const dmh_gguf_file* f);
/* GGUFIndex.tensor_map lookup: the last tensor of that name, or -1. */
int dmh_gguf_find(const dmh_gguf_file* f, const char* name);
int dmh_gguf_tensor_info(const dmh_gguf_file* f, int idx, dmh_gguf_tensor* info);
/* GGUFIndex.metadata[key] as text (scalars in decimal, arrays as
 * "[Array of N elements]"), or NULL. */
const char* dmh_gguf_metadata(const dmh_gguf_file* f, const char* key);
/* The raw payload bytes of tensor idx; bytes must equal its raw_bytes. */
int dmh_gguf_read(const dmh_gguf_file* f, int idx, void* out, int64_t bytes, char* err,
                  size_t errlen);

/* dequantize_q8_0 / dequantize_q4_k / dequantize_q3_k (gguf.mojo:414-560)
 * and the F32 / BF16 copies of stream_gguf_tensor_f32 (:598-613) on the GPU:
 * out[num_elements] fp32, elements past the last whole block 0.0.  raw holds
 * at least the whole blocks.  flags: DMH_F_DEVICE (raw and out are device
 * memory, raw 4-byte and out 16-byte aligned), DMH_F_Q4K_PY_SCALES.  Unknown
 * types: "GGUF_UNSUPPORTED_DTYPE: unsupported GGML type T", DMH_ERR_FORMAT. */
int dmh_dequant_gguf(dmh_ctx* ctx, int ggml_type, const void* raw, int64_t raw_bytes,
                     int64_t num_elements, float* out, unsigned flags, char* err,
                     size_t errlen);

/* stream_gguf_tensor_f32 (gguf.mojo:563-626): read one tensor's bytes from
 * the file and dequantize them on the GPU into out[n_out] (n_out must equal
 * num_elements).  flags: DMH_F_DEVICE (out is device memory),
 * DMH_F_Q4K_PY_SCALES.  Errors: WEIGHT_LOAD_FAILED (name not in the index),
 * GGUF_READ_ERROR (truncated read), GGUF_UNSUPPORTED_DTYPE. */
int dmh_gguf_stream_tensor_f32(dmh_ctx* ctx, const dmh_gguf_file* f, const char* name,
                               float* out, int64_t n_out, unsigned flags, char* err,
                               size_t errlen);

/* load_port_block_from_gguf's MoE tensors (src/layers/gguf_port_loader.mojo:
 * 207-256) of model layer model_layer into GGUF layer slot `layer` (slots
 * separate from dmh_upload_moe_layer's): router blk.{l}.ffn_gate_exps.weight
 * [E*H] and shared gate blk.{l}.shared_gate.weight [H] dequantized to fp32;
 * blk.{l}.ffn_{gate,up,down}.{e}.weight and blk.{l}.ffn_shared_{gate,up,down}
 * .weight kept in their GGUF blocks in HBM (one GGML type for all of them).
 * Errors: the loader's WEIGHT_LOAD_FAILED / GGUF_READ_ERROR /
 * GGUF_UNSUPPORTED_DTYPE / "GGUF_FILE_CORRUPT: dimension mismatch" texts in
 * its order.  dims: hidden, inter, inter_sh multiples of 4; group_size is
 * ignored.  flags: DMH_F_Q4K_PY_SCALES. */
int dmh_upload_moe_layer_gguf(dmh_ctx* ctx, int layer, const dmh_moe_dims* dims,
                              const dmh_gguf_file* f, int model_layer, unsigned flags, char* err,
                              size_t errlen);
int dmh_free_layer_gguf(dmh_ctx* ctx, int layer);

/* The MoE section of forward_port_block (src/layers/port_scheduler.mojo:
 * 381-482) on a GGUF layer, as dmh_moe_forward: x is the post-attention
 * RMSNorm output [seq_len][H], residual (x_mid, may be NULL) is added last;
 * ids / probs [seq_len][K] and shg [seq_len] may be NULL.  Router, top-k,
 * shared gate and aggregation are bit-exact with the reference's fp32
 * order; the experts accumulate in fp32 in another order.  Expert error
 * texts carry hidden as "layer" and the intermediate size as "expert_id", as
 * forward_port_block's swiglu_forward calls do (port_scheduler.mojo:450-464).
 * DMH_F_DEVICE: x, residual and y 16-byte aligned device memory. */
int dmh_moe_forward_gguf(dmh_ctx* ctx, int layer, const float* x, const float* residual,
                         int seq_len, float* y, int32_t* ids, float* probs, float* shg,
                         unsigned flags, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif
#endif /* DISMOEN_HIP_H */
