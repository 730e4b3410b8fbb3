// dm_files_api.cpp -- C ABI over the weight-file readers (dm_formats.cpp) and
// the upload of one MoE layer straight from the reference's files.
#include <stdio.h>
#include <string.h>

#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/dismoen_hip.h"
#include "dm_api_internal.h"
#include "dm_formats.h"
#include "dm_gguf.h"

struct dmh_quant_file {
  dm::QuantFile f;
};
struct dmh_st_file {
  dm::SafetensorsFile f;
};


namespace {

int put_err(char* err, size_t errlen, int code, const std::string& msg) {
  if (err && errlen) {
    const size_t n = msg.size() < errlen - 1 ? msg.size() : errlen - 1;
    memcpy(err, msg.data(), n);
    err[n] = '\0';
  }
  return code;
}

void fill_info(const dm::FileTensor& t, dmh_tensor_info* info) {
  memset(info, 0, sizeof(*info));
  info->name = t.name.c_str();
  info->dtype = t.dtype.c_str();
  info->ndim = (int32_t)t.shape.size();
  for (size_t i = 0; i < t.shape.size() && i < 8; ++i) info->shape[i] = t.shape[i];
  info->group_size = t.group_size;
  info->num_groups = t.num_groups;
  info->scales_offset = t.scales_offset;
  info->scales_bytes = t.scales_bytes;
  info->data_offset = t.data_offset;
  info->data_bytes = t.data_bytes;
}

int upload_files(dmh_ctx* ctx, int layer, const dmh_moe_dims* d, const dm::QuantFile& q,
                 const dm::SafetensorsFile& s, int model_layer, char* err, size_t errlen);

std::string not_in_quant(const std::string& name) {  // src/layers/quant_loader.mojo:33-40
  return "{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"tensor not found in quant model\","
         "\"tensor\":\"" + name + "\"}";
}

std::string shape_str(const std::vector<int64_t>& s) {
  std::string o = "[";
  for (size_t i = 0; i < s.size(); ++i) o += (i ? "," : "") + std::to_string(s[i]);
  return o + "]";
}

// One 4-bit tensor of [rows][cols] with group size G appended to the staging
// vectors (scales, then codes).
int append_quant(const dm::QuantFile& q, const std::string& name, int64_t rows, int64_t cols,
                 int G, std::vector<uint16_t>& sc, std::vector<uint8_t>& pk, char* err,
                 size_t errlen) {
  const int idx = q.find(name);
  if (idx < 0) return put_err(err, errlen, DMH_ERR_WEIGHT, not_in_quant(name));
  const dm::FileTensor& t = q.tensors[idx];
  const bool shape_ok = (t.shape.size() == 2 && t.shape[0] == rows && t.shape[1] == cols);
  if (!shape_ok || t.group_size != G)
    return put_err(err, errlen, DMH_ERR_WEIGHT,
                   "{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"expected shape [" +
                       std::to_string(rows) + "," + std::to_string(cols) + "] group " +
                       std::to_string(G) + ", file has " + shape_str(t.shape) + " group " +
                       std::to_string(t.group_size) + "\",\"tensor\":\"" + name + "\"}");
  const size_t s0 = sc.size(), p0 = pk.size();
  sc.resize(s0 + (size_t)t.num_groups);
  pk.resize(p0 + (size_t)t.data_bytes);
  std::string e;
  if (!dm::read_quant_tensor(q, idx, sc.data() + s0, pk.data() + p0, &e))
    return put_err(err, errlen, DMH_ERR_WEIGHT, e);
  return DMH_OK;
}

// A bf16 tensor of n elements from the safetensors shard under the first of
// the candidate names that exists.
int read_bf16(const dm::SafetensorsFile& s, const std::vector<std::string>& names, int64_t n,
              std::vector<uint16_t>& out, std::string* found) {
  for (const std::string& nm : names) {
    const int idx = s.find(nm);
    if (idx < 0) continue;
    const dm::FileTensor& t = s.tensors[idx];
    int64_t numel = 1;
    for (int64_t d : t.shape) numel *= d;
    if (t.dtype != "BF16" || numel != n) return -2;
    out.resize((size_t)n);
    std::string e;
    if (!dm::read_safetensors_tensor(s, idx, out.data(), n * 2, &e)) return -3;
    *found = nm;
    return idx;
  }
  return -1;
}

}  // namespace

extern "C" {

int dmh_quant_open(const char* path, dmh_quant_file** out, char* err, size_t errlen) {
  if (!path || !out) return put_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_quant_open: NULL argument");
  *out = nullptr;
  dmh_quant_file* h = new dmh_quant_file();
  std::string e;
  if (!dm::scan_quant_file(path, &h->f, &e)) {
    delete h;
    return put_err(err, errlen, DMH_ERR_FORMAT, e);
  }
  *out = h;
  return DMH_OK;
}

void dmh_quant_close(dmh_quant_file* f) { delete f; }

int dmh_quant_num_tensors(const dmh_quant_file* f) { return f ? (int)f->f.tensors.size() : -1; }

int dmh_quant_find(const dmh_quant_file* f, const char* name) {
  return (f && name) ? f->f.find(name) : -1;
}

int dmh_quant_tensor_info(const dmh_quant_file* f, int idx, dmh_tensor_info* info) {
  if (!f || !info || idx < 0 || idx >= (int)f->f.tensors.size()) return DMH_ERR_INVALID_ARG;
  fill_info(f->f.tensors[idx], info);
  return DMH_OK;
}

int dmh_quant_read(const dmh_quant_file* f, int idx, uint16_t* scales, int64_t n_scales,
                   uint8_t* packed, int64_t n_packed, char* err, size_t errlen) {
  if (!f || !scales || !packed || idx < 0 || idx >= (int)f->f.tensors.size())
    return put_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_quant_read: bad arguments");
  const dm::FileTensor& t = f->f.tensors[idx];
  if (n_scales != t.num_groups || n_packed != t.data_bytes)
    return put_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_quant_read: buffers of " + std::to_string(n_scales) + " scales / " +
                       std::to_string(n_packed) + " bytes, tensor has " +
                       std::to_string(t.num_groups) + " / " + std::to_string(t.data_bytes));
  std::string e;
  if (!dm::read_quant_tensor(f->f, idx, scales, packed, &e))
    return put_err(err, errlen, DMH_ERR_WEIGHT, e);
  return DMH_OK;
}

int dmh_st_open(const char* path, dmh_st_file** out, char* err, size_t errlen) {
  if (!path || !out) return put_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_st_open: NULL argument");
  *out = nullptr;
  dmh_st_file* h = new dmh_st_file();
  std::string e;
  if (!dm::read_safetensors_header(path, &h->f, &e)) {
    delete h;
    return put_err(err, errlen, DMH_ERR_FORMAT, e);
  }
  *out = h;
  return DMH_OK;
}

void dmh_st_close(dmh_st_file* f) { delete f; }

int dmh_st_num_tensors(const dmh_st_file* f) { return f ? (int)f->f.tensors.size() : -1; }

int dmh_st_find(const dmh_st_file* f, const char* name) {
  return (f && name) ? f->f.find(name) : -1;
}

int dmh_st_tensor_info(const dmh_st_file* f, int idx, dmh_tensor_info* info) {
  if (!f || !info || idx < 0 || idx >= (int)f->f.tensors.size()) return DMH_ERR_INVALID_ARG;
  fill_info(f->f.tensors[idx], info);
  return DMH_OK;
}

int dmh_st_read(const dmh_st_file* f, int idx, void* out, int64_t bytes, char* err,
                size_t errlen) {
  if (!f || !out) return put_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_st_read: bad arguments");
  std::string e;
  if (!dm::read_safetensors_tensor(f->f, idx, out, bytes, &e))
    return put_err(err, errlen, DMH_ERR_FORMAT, e);
  return DMH_OK;
}

int dmh_upload_moe_layer_files(dmh_ctx* ctx, int layer, const dmh_moe_dims* d,
                               const dmh_quant_file* qf, const dmh_st_file* sf, int model_layer,
                               char* err, size_t errlen) {
  if (!d || !qf || !sf)
    return put_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_upload_moe_layer_files: NULL argument");
  // group_size 0: the quant model's own, quantization.group_size of its
  // header (docs/format/quant_format.md:76,212)
  dmh_moe_dims dd = *d;
  if (dd.group_size == 0) dd.group_size = qf->f.group_size;
  d = &dd;
  // the dims are checked before any size arithmetic (a zero or negative
  // group size would divide by zero below) and nothing throws across the ABI
  const int rc = dm::api_moe_dims_check(d, layer, err, errlen);
  if (rc != DMH_OK) return rc;
  if (!ctx)
    return put_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_upload_moe_layer_files: NULL context");
  try {
    return upload_files(ctx, layer, d, qf->f, sf->f, model_layer, err, errlen);
  } catch (const std::bad_alloc&) {
    return put_err(err, errlen, DMH_ERR_NO_MEMORY, "dmh_upload_moe_layer_files: out of host memory");
  } catch (const std::exception& ex) {
    return put_err(err, errlen, DMH_ERR_NO_MEMORY,
                   std::string("dmh_upload_moe_layer_files: ") + ex.what());
  }
}

}  // extern "C"

namespace {

int upload_files(dmh_ctx* ctx, int layer, const dmh_moe_dims* d, const dm::QuantFile& q,
                 const dm::SafetensorsFile& s, int model_layer, char* err, size_t errlen) {
  const int64_t H = d->hidden, E = d->num_experts, I = d->inter, Ish = d->inter_sh;
  const int G = d->group_size;
  const std::string L = std::to_string(model_layer);
  // router gate (src/layers/router.mojo:234-247): language-model prefix first
  std::vector<uint16_t> router, shgate;
  std::string rn;
  const std::string r_lm = "model.language_model.layers." + L + ".mlp.gate.weight";
  const std::string r_old = "model.layers." + L + ".mlp.gate.weight";
  int rc = read_bf16(s, {r_lm, r_old}, E * H, router, &rn);
  if (rc == -1)
    return put_err(err, errlen, DMH_ERR_WEIGHT,
                   "{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"required router gate"
                   " tensor not in weight_map: " + r_old + "\",\"shard\":\"\",\"tensor_name\":\"" +
                       r_old + "\"}");
  if (rc < 0)
    return put_err(err, errlen, DMH_ERR_WEIGHT,
                   "{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"router gate must be BF16"
                   " [" + std::to_string(E) + "," + std::to_string(H) + "]\",\"shard\":\"" +
                       s.path + "\",\"tensor_name\":\"" + r_old + "\"}");
  // shared-expert gate: bf16 from the shard, else the 4-bit tensor of the
  // quant model (src/layers/quant_loader.mojo:132-135), whose dequantised
  // values are bf16 numbers
  const std::string g_lm = "model.language_model.layers." + L + ".mlp.shared_expert_gate.weight";
  const std::string g_old = "model.layers." + L + ".mlp.shared_expert_gate.weight";
  rc = read_bf16(s, {g_lm, g_old}, H, shgate, &rn);
  if (rc == -1) {
    const int gi = q.find(g_old);
    if (gi < 0) return put_err(err, errlen, DMH_ERR_WEIGHT, not_in_quant(g_old));
    const dm::FileTensor& t = q.tensors[gi];
    int64_t numel = 1;
    for (int64_t v : t.shape) numel *= v;
    if (numel != H)
      return put_err(err, errlen, DMH_ERR_WEIGHT,
                     "{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"shared expert gate has " +
                         std::to_string(numel) + " elements, expected " + std::to_string(H) +
                         "\",\"tensor\":\"" + g_old + "\"}");
    std::vector<uint16_t> sc((size_t)t.num_groups);
    std::vector<uint8_t> pk((size_t)t.data_bytes);
    std::string e;
    if (!dm::read_quant_tensor(q, gi, sc.data(), pk.data(), &e))
      return put_err(err, errlen, DMH_ERR_WEIGHT, e);
    shgate.resize((size_t)H);
    uint16_t* tmp = shgate.data();
    char e2[512];
    const int r2 = dmh_dequant_q4_bf16(ctx, sc.data(), (int64_t)sc.size(), pk.data(),
                                       (int64_t)pk.size(), H, t.group_size, tmp, 0, e2,
                                       sizeof(e2));
    if (r2) return put_err(err, errlen, r2, e2);
  } else if (rc < 0) {
    return put_err(err, errlen, DMH_ERR_WEIGHT,
                   "{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"shared expert gate must be"
                   " BF16 with " + std::to_string(H) + " elements\",\"shard\":\"" + s.path +
                       "\",\"tensor_name\":\"" + g_old + "\"}");
  }
  // routed experts (src/layers/quant_loader.mojo:89-111) and the shared
  // expert (:114-130), gate then up rows per expert as in experts.gate_up_proj
  std::vector<uint16_t> gus, ds, sgus, sds;
  std::vector<uint8_t> gup, dp, sgup, sdp;
  gus.reserve((size_t)(E * 2 * I * H / G));
  gup.reserve((size_t)(E * 2 * I * H / 2));
  ds.reserve((size_t)(E * H * I / G));
  dp.reserve((size_t)(E * H * I / 2));
  for (int64_t e = 0; e < E; ++e) {
    const std::string p = "model.layers." + L + ".mlp.experts." + std::to_string(e) + ".";
    if ((rc = append_quant(q, p + "gate_proj.weight", I, H, G, gus, gup, err, errlen)) ||
        (rc = append_quant(q, p + "up_proj.weight", I, H, G, gus, gup, err, errlen)) ||
        (rc = append_quant(q, p + "down_proj.weight", H, I, G, ds, dp, err, errlen)))
      return rc;
  }
  const std::string sp = "model.layers." + L + ".mlp.shared_expert.";
  if ((rc = append_quant(q, sp + "gate_proj.weight", Ish, H, G, sgus, sgup, err, errlen)) ||
      (rc = append_quant(q, sp + "up_proj.weight", Ish, H, G, sgus, sgup, err, errlen)) ||
      (rc = append_quant(q, sp + "down_proj.weight", H, Ish, G, sds, sdp, err, errlen)))
    return rc;
  dmh_moe_weights w = {router.data(), shgate.data(), gus.data(), gup.data(), ds.data(),
                       dp.data(),     sgus.data(),   sgup.data(), sds.data(), sdp.data()};
  return dmh_upload_moe_layer(ctx, layer, d, &w, 0, err, errlen);
}

}  // namespace

extern "C" {

int dmh_gguf_open(const char* path, dmh_gguf_file** out, char* err, size_t errlen) {
  if (!path || !out) return put_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_gguf_open: NULL argument");
  *out = nullptr;
  dmh_gguf_file* h = new dmh_gguf_file();
  std::string e;
  if (!dm::parse_gguf_index(path, &h->f, &e)) {
    delete h;
    return put_err(err, errlen, DMH_ERR_FORMAT, e);
  }
  *out = h;
  return DMH_OK;
}

void dmh_gguf_close(dmh_gguf_file* f) { delete f; }

int dmh_gguf_get_header(const dmh_gguf_file* f, dmh_gguf_header* h) {
  if (!f || !h) return DMH_ERR_INVALID_ARG;
  h->version = f->f.version;
  h->tensor_count = f->f.tensor_count;
  h->metadata_kv_count = f->f.metadata_kv_count;
  h->data_section_offset = f->f.data_section_offset;
  h->expected_file_size = f->f.expected_file_size;
  h->alignment = f->f.alignment;
  return DMH_OK;
}

int dmh_gguf_num_tensors(const dmh_gguf_file* f) { return f ? (int)f->f.tensors.size() : -1; }

int dmh_gguf_find(const dmh_gguf_file* f, const char* name) {
  return (f && name) ? f->f.find(name) : -1;
}

int dmh_gguf_tensor_info(const dmh_gguf_file* f, int idx, dmh_gguf_tensor* info) {
  if (!f || !info || idx < 0 || idx >= (int)f->f.tensors.size()) return DMH_ERR_INVALID_ARG;
  const dm::GgufTensor& t = f->f.tensors[idx];
  memset(info, 0, sizeof(*info));
  info->name = t.name.c_str();
  info->ndim = (int32_t)t.dims.size();
  for (size_t i = 0; i < t.dims.size() && i < 8; ++i) info->dims[i] = t.dims[i];
  info->ggml_type = t.type;
  info->offset = t.offset;
  info->file_offset = f->f.data_section_offset + t.offset;
  info->num_elements = t.num_elements;
  info->raw_bytes = t.raw_bytes;
  return DMH_OK;
}

const char* dmh_gguf_metadata(const dmh_gguf_file* f, const char* key) {
  if (!f || !key) return nullptr;
  const std::string* v = f->f.meta(key);
  return v ? v->c_str() : nullptr;
}

int dmh_gguf_read(const dmh_gguf_file* f, int idx, void* out, int64_t bytes, char* err,
                  size_t errlen) {
  if (!f || !out || idx < 0 || idx >= (int)f->f.tensors.size())
    return put_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_gguf_read: bad arguments");
  const dm::GgufTensor& t = f->f.tensors[idx];
  if (bytes != t.raw_bytes)
    return put_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_gguf_read: buffer of " + std::to_string(bytes) + " bytes, tensor has " +
                       std::to_string(t.raw_bytes));
  std::vector<uint8_t> raw;
  std::string e;
  if (!dm::read_gguf_tensor(f->f, idx, &raw, &e)) return put_err(err, errlen, DMH_ERR_WEIGHT, e);
  memcpy(out, raw.data(), raw.size());
  return DMH_OK;
}

// stream_gguf_tensor_f32 (src/format/gguf.mojo:563-626): lookup, read, then
// the type check, in the reference's order.
int dmh_gguf_stream_tensor_f32(dmh_ctx* ctx, const dmh_gguf_file* f, const char* name, float* out,
                               int64_t n_out, unsigned flags, char* err, size_t errlen) {
  if (!ctx || !f || !name || !out)
    return put_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_gguf_stream_tensor_f32: NULL argument");
  const int idx = f->f.find(name);
  if (idx < 0)
    return put_err(err, errlen, DMH_ERR_WEIGHT,
                   std::string("{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"tensor not "
                               "found in GGUF index\",\"tensor\":\"") + name + "\"}");
  const dm::GgufTensor& t = f->f.tensors[idx];
  std::vector<uint8_t> raw;
  std::string e;
  if (!dm::read_gguf_tensor(f->f, idx, &raw, &e)) return put_err(err, errlen, DMH_ERR_WEIGHT, e);
  int bs, bpb;
  if (dm::gguf_block_spec(t.type, &bs, &bpb))
    return put_err(err, errlen, DMH_ERR_FORMAT,
                   "GGUF_UNSUPPORTED_DTYPE: unsupported GGML type " + std::to_string(t.type) +
                       " for tensor " + t.name);
  if (n_out != t.num_elements)
    return put_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_gguf_stream_tensor_f32: output of " + std::to_string(n_out) +
                       " elements, tensor has " + std::to_string(t.num_elements));
  return dm::api_dequant_gguf(ctx, t.type, raw.data(), false, (int64_t)raw.size(),
                              t.num_elements, out, (flags & DMH_F_DEVICE) != 0,
                              (flags & DMH_F_Q4K_PY_SCALES) ? 1 : 0, err, errlen);
}

}  // extern "C"
