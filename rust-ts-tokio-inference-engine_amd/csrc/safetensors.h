// Strict safetensors reader for rs_mlx_weights_load (native/mlx_bridge.cpp:108-118,
// which loads through mx::load_safetensors): an 8-byte little-endian header
// length, a JSON header {name: {dtype, shape, data_offsets}, "__metadata__":
// {...}}, then the tensor payload. The checks follow the reference's checkpoint
// manifest (src/serving/weights.rs:236-301): header length 2 B..8 MiB inside the
// file, dtypes F32/I32/U32/F16/BF16, rank 1..4 with positive dimensions,
// data_offsets spanning exactly shape x item bytes inside the payload, no two
// tensors overlapping, no duplicate keys.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace hb {

struct SafeTensor {
  std::string name;
  int dtype = 0;  // graph.h Dtype: 0 f32, 1 i32, 2 u32, 3 f16, 4 bf16
  std::vector<int32_t> shape;
  uint64_t begin = 0, end = 0;  // byte range inside the payload
};

struct SafeFile {
  uint64_t payload = 0;  // file offset of the payload
  std::vector<SafeTensor> tensors;
};

// Parses and validates the header of the file at `path` (throws
// std::invalid_argument with the reason when it is malformed).
SafeFile read_safetensors_header(const std::string& path);

// Parses a header given as bytes (the JSON after the length prefix) for a
// payload of `payload_bytes`; exposed for the parser tests.
std::vector<SafeTensor> parse_safetensors_header(const std::string& json, uint64_t payload_bytes);

}  // namespace hb
