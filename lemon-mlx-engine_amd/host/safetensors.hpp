// safetensors.hpp -- checkpoint files for the host classes: the safetensors
// reader and the directory resolution of the reference's
// load_safetensors_from_directory (src/common/safetensors.cpp:23-77).
//
// Reading is split in two steps.  read_safetensors* parses headers and maps
// the files read-only: a HostTensor is a view of its bytes in the mapping,
// nothing is copied or uploaded.  load_safetensors* uploads tensors to device
// `array`s, the form the reference's loaders return (mlx::core arrays).  The
// MoE sanitize step (per-expert stacking) runs on HostTensors, between the two,
// so a layer's experts are uploaded once, already stacked.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "switch_layers.hpp"

namespace mlx_lm {
namespace mi355x {

// One tensor of a checkpoint, in host memory.
struct HostTensor {
  std::string dtype;                   // safetensors dtype: "BF16", "F32", "U32", "I32", "F16", ...
  Shape shape;
  const uint8_t* data = nullptr;       // nbytes bytes, little-endian, row-major
  size_t nbytes = 0;
  std::shared_ptr<const void> owner;   // keeps the file mapping (or a stacked buffer) alive

  size_t numel() const;
};
using HostTensors = std::unordered_map<std::string, HostTensor>;

// Bytes per element of a safetensors dtype string; throws std::invalid_argument
// for an unknown one.
size_t safetensors_itemsize(const std::string& dtype);

// Parses one file (8-byte little-endian header length, JSON header, data
// section).  Validates every entry: known dtype, non-negative shape, offsets
// inside the data section and matching the shape's size.  "__metadata__" is
// skipped.  Throws std::runtime_error for I/O failures, std::invalid_argument
// for a malformed file.
HostTensors read_safetensors(const std::string& path);

// The files of a checkpoint directory, in the reference's order of preference:
// the shards named by model.safetensors.index.json's weight_map (sorted; a
// missing one throws "Missing shard file: ..."), else model.safetensors when it
// is larger than 1024 bytes, else every *.safetensors file of the directory
// (sorted by name; none throws "No .safetensors files found in ...").
std::vector<std::string> safetensors_files(const std::string& directory);

// All tensors of the directory's files; a name in several files takes the
// later file's tensor, as the reference's insert_or_assign does.
HostTensors read_safetensors_from_directory(const std::string& directory);

// Device copy of a host tensor (BF16, F32, U32, I32; other dtypes throw
// std::invalid_argument).  A 0-d tensor becomes shape {1}.
array to_device(const HostTensor& t);

// The reference's loaders (safetensors.cpp:17-77): every tensor uploaded.
// `keep` (optional) selects the names to upload.
using NameFilter = std::function<bool(const std::string&)>;
std::unordered_map<std::string, array> load_safetensors(const std::string& path, const NameFilter& keep = {});
std::unordered_map<std::string, array> load_safetensors_from_directory(const std::string& directory,
                                                                       const NameFilter& keep = {});

// CRC-32 (IEEE 802.3, reflected polynomial 0xEDB88320) of a byte range, the
// checksum zlib.crc32 computes; used to compare readers tensor by tensor.
uint32_t crc32(const void* data, size_t n, uint32_t crc = 0);

}  // namespace mi355x
}  // namespace mlx_lm
