// dm_gguf.h -- GGUF container index (host) and the payload dequantizer (GPU).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

struct dmh_ctx;

namespace dm {

// GGML type codes of src/format/gguf.mojo:19-30 that have a dequantizer.
constexpr int kGgmlF32 = 0;
constexpr int kGgmlQ8_0 = 8;
constexpr int kGgmlQ3_K = 11;
constexpr int kGgmlQ4_K = 12;
constexpr int kGgmlBF16 = 30;

// (block_size, bytes_per_block) of a type with a dequantizer; -1 otherwise.
int gguf_block_spec(int ggml_type, int* block_size, int* bytes_per_block);

// out[0, n) = the fp32 values of the payload raw (device memory, 4-byte
// aligned; out 16-byte aligned) of n weights of ggml_type; elements past the
// last whole block are 0.0.  q4k_layout 1 selects the scale packing of the
// reference's Python twin for Q4_K sub-blocks 4..7.
hipError_t launch_dequant_gguf(int ggml_type, const uint8_t* raw, int64_t n, int q4k_layout,
                               float* out, hipStream_t st);

// One MoE layer uploaded from GGUF (the tensors of
// src/layers/gguf_port_loader.mojo:207-256): expert payloads stay in their
// GGUF blocks in HBM, the router and the shared-expert gate are fp32.
struct GgufMoeDev {
  int H, E, K, I, Ish;
  int type;            // GGML type of every expert tensor
  int layout;          // Q4_K scale packing (see launch_dequant_gguf)
  const uint8_t* raw;  // expert payloads
  const int64_t* off;  // [E + 1][3] byte offsets of gate, up, down in raw; row E = shared expert
  const float* router; // [E][H]
  const float* shgate; // [H]
  int64_t estride;     // > 0: off[3e + k] = (3e + k) * estride for the routed experts (else 0)
  const float* rchain; // [E + 1][H] router and shared gate in chain order (one-token form), or null
};

// h[t][s][i] = SiLU(W_gate x_t)_i * (W_up x_t)_i for slots s < K (expert
// ids[t][s]) and s = K (the shared expert), rows i < I (Ish); ldh >= max(I,
// Ish), a multiple of 4.  Non-finite gate / up / product values record the
// first-error keys of swiglu_forward (phase expert or shared).
hipError_t launch_gguf_gateup(const GgufMoeDev& L, const float* x, int T, const int32_t* ids,
                              float* h, int ldh, unsigned long long* status, hipStream_t st);
// y[t][d] = sum_k probs[t][k] (W_down h[t][k])_d + shg[t] (W_sh_down
// h[t][K])_d (+ residual[t][d]): the down projections and
// moe_aggregate_forward's order in one launch per 65535 tokens; K <= 32.
hipError_t launch_gguf_down_combine(const GgufMoeDev& L, const float* h, int ldh, int T,
                                    const int32_t* ids, const float* probs, const float* shg,
                                    const float* residual, float* y, unsigned long long* status,
                                    hipStream_t st);

// The same outputs for T tokens grouped by expert (off, perm, units, meta
// of launch_group_build on ids; nunits = group_units_max(T, K, E)): each
// expert row is read once per unit of up to 128 tokens instead of once per
// (token, slot).  Three launches: gate/up into h as launch_gguf_gateup, the
// down projections into parts [T][K+1][H], then moe_aggregate_forward's
// combine.  Every token's sums are formed by the same helpers in the same
// order as launch_gguf_gateup / launch_gguf_down_combine: the same bits.
hipError_t launch_gguf_units(const GgufMoeDev& L, const float* x, int T, const int32_t* off,
                             const int32_t* perm, const int2* units, const int32_t* meta,
                             int nunits, float* h, int ldh, float* parts, const float* probs,
                             const float* shg, const float* residual, float* y,
                             unsigned long long* status, hipStream_t st);

// One token in one launch of grid workgroups of 512 threads that must all
// be resident (gguf_experts_occupancy >= 1 per CU, gguf_one_token_grid_ok):
// the router logits, the top-k selection, the softmax terms and the shared
// expert's h as wave tasks handed over in words tagged with the launch
// number n, then the routed experts (one hand-off of the routed h counted
// per slot), the down projections and the combine.  L.rchain must be set
// (launch_chain_router).  sync: gguf_one_token_sync_bytes of device
// memory, zero before the first launch; launch n of a layer (n = 1, 2, ...)
// waits for words tagged n and for n * I / 16 counts per slot (compared
// modulo 2^32), so the caller keeps n per layer.
bool gguf_one_token_supported(const GgufMoeDev& L);
// rchain for the one-token form: row e's element c + 16 (4q + u) at
// 4 (16 q + c) + u (the steps of router_project's lane chains, four per
// float4; zero past H), rows 0 .. E - 1 the router, row E the shared gate;
// out holds gguf_chain_router_bytes(L) bytes, H a multiple of 64.
size_t gguf_chain_router_bytes(const GgufMoeDev& L);
hipError_t launch_chain_router(const GgufMoeDev& L, float* out, hipStream_t st);
size_t gguf_one_token_sync_bytes(const GgufMoeDev& L);
bool gguf_one_token_grid_ok(const GgufMoeDev& L, int grid);
int gguf_experts_occupancy(const GgufMoeDev& L, int* per_cu);
hipError_t launch_gguf_one_token(const GgufMoeDev& L, const float* x, const float* residual,
                                 float* y, int32_t* ids, float* probs, float* shg, void* sync,
                                 unsigned launch, int grid, unsigned long long* status,
                                 hipStream_t st, long spin);

// GGUFTensorInfo (gguf.mojo:104-114); offset is relative to the data section.
struct GgufTensor {
  std::string name;
  std::vector<int64_t> dims;
  int type = 0;
  int64_t offset = 0, num_elements = 0, raw_bytes = 0;
};

// GGUFIndex (gguf.mojo:117-141).
struct GgufFile {
  std::string path;
  int64_t filesize = 0;
  int version = 0;
  int64_t tensor_count = 0, metadata_kv_count = 0;
  int64_t data_section_offset = 0, expected_file_size = 0, alignment = 32;
  std::vector<GgufTensor> tensors;
  std::unordered_map<std::string, int> tensor_map;           // name -> last index
  std::vector<std::pair<std::string, std::string>> metadata;  // first-seen order
  std::unordered_map<std::string, size_t> meta_pos;
  int find(const std::string& name) const;
  const std::string* meta(const std::string& key) const;
};

// parse_gguf_index (gguf.mojo:257-411): header, metadata, tensor directory
// and the exact-size rule; err receives the reference's text.
bool parse_gguf_index(const std::string& path, GgufFile* out, std::string* err);

// The raw payload of tensor idx (raw_bytes bytes) read from the file; the
// truncated-read text of stream_gguf_tensor_f32 (gguf.mojo:586-596).
bool read_gguf_tensor(const GgufFile& f, int idx, std::vector<uint8_t>* out, std::string* err);

// The body of dmh_dequant_gguf with the memory kind of raw and out given
// separately (defined in dm_api.cpp).
int api_dequant_gguf(::dmh_ctx* c, int ggml_type, const void* raw, bool raw_dev,
                     int64_t raw_bytes, int64_t n, float* out, bool out_dev, int q4k_layout,
                     char* err, size_t errlen);

}  // namespace dm

// The C ABI's GGUF file handle.
struct dmh_gguf_file {
  dm::GgufFile f;
};
