// dm_formats.h -- host readers of the reference's weight files: the 4-bit
// per-group quant model (src/format/quant_reader.mojo) and safetensors shard
// headers with bf16 tensor reads (src/format/reader.mojo).  Pure host code:
// no HIP call, usable without a GPU.
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

namespace dm {

// One tensor of either file.  Offsets are absolute file offsets.
struct FileTensor {
  std::string name;
  std::vector<int64_t> shape;
  std::string dtype;            // safetensors dtype, or the quant meta's "dtype"
  std::string quantized_dtype;  // quant only
  int group_size = 0;           // quant only
  int64_t num_groups = 0;       // quant only
  int64_t scales_offset = 0, scales_bytes = 0;  // quant only
  int64_t data_offset = 0, data_bytes = 0;      // quant: packed codes; safetensors: payload
};

struct QuantFile {
  std::string path;
  int version = 0;
  std::string model, format, scale_dtype;
  int group_size = 0;
  int64_t num_tensors = 0, total_bytes = 0;
  std::vector<FileTensor> tensors;
  int find(const std::string& name) const;  // last entry of that name, -1 if none
};

struct SafetensorsFile {
  std::string path;
  int64_t filesize = 0, data_base = 0, header_len = 0;
  std::vector<FileTensor> tensors;
  int find(const std::string& name) const;
};

// scan_quant_file (quant_reader.mojo:487-662).  Returns false and the
// reference's message in *err on failure.
bool scan_quant_file(const std::string& path, QuantFile* out, std::string* err);
// pread_tensor_quant (quant_reader.mojo:665-692): fp16 scale bits and packed
// codes of tensor idx.
bool read_quant_tensor(const QuantFile& f, int idx, uint16_t* scales, uint8_t* packed,
                       std::string* err);

// read_header (reader.mojo:21-297): header parse and the F15 layout checks.
bool read_safetensors_header(const std::string& path, SafetensorsFile* out, std::string* err);
// Payload bytes of tensor idx (count bytes, which must equal its size).
bool read_safetensors_tensor(const SafetensorsFile& f, int idx, void* out, int64_t count,
                             std::string* err);

// The reference's four-field error object (types.mojo:103-122).
std::string error_json(const std::string& type, const std::string& detail,
                       const std::string& shard, const std::string& tensor);

}  // namespace dm
