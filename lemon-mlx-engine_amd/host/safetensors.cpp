// safetensors.cpp -- the reader and directory resolution declared in
// safetensors.hpp.
#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <set>
#include <sstream>
#include <stdexcept>

#include "json.hpp"

namespace fs = std::filesystem;

namespace mlx_lm {
namespace mi355x {

size_t HostTensor::numel() const {
  size_t n = 1;
  for (int32_t d : shape)
    if (__builtin_mul_overflow(n, static_cast<size_t>(d), &n))
      throw std::invalid_argument("tensor of " + std::to_string(shape.size()) + " dimensions: element count overflows");
  return n;
}

size_t safetensors_itemsize(const std::string& dt) {
  static const std::unordered_map<std::string, size_t> sizes = {
      {"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"F8_E5M2", 1}, {"F8_E4M3", 1}, {"U16", 2}, {"I16", 2}, {"F16", 2},
      {"BF16", 2}, {"U32", 4}, {"I32", 4}, {"F32", 4},     {"U64", 8},     {"I64", 8}, {"F64", 8}};
  const auto it = sizes.find(dt);
  if (it == sizes.end()) throw std::invalid_argument("safetensors: unknown dtype '" + dt + "'");
  return it->second;
}

namespace {

// A read-only private mapping of a whole file, unmapped with the last owner.
std::shared_ptr<const void> map_file(const std::string& path, size_t& size) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) throw std::runtime_error("safetensors: cannot open " + path + ": " + std::strerror(errno));
  struct stat st {};
  if (::fstat(fd, &st) != 0) {
    const int err = errno;
    ::close(fd);
    throw std::runtime_error("safetensors: cannot stat " + path + ": " + std::strerror(err));
  }
  size = static_cast<size_t>(st.st_size);
  if (size == 0) {
    ::close(fd);
    throw std::invalid_argument("safetensors: " + path + " is empty");
  }
  void* p = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  const int err = errno;
  ::close(fd);
  if (p == MAP_FAILED) throw std::runtime_error("safetensors: cannot map " + path + ": " + std::strerror(err));
  const size_t len = size;
  return std::shared_ptr<const void>(p, [len](const void* q) { ::munmap(const_cast<void*>(q), len); });
}

[[noreturn]] void bad(const std::string& path, const std::string& what) {
  throw std::invalid_argument("safetensors: " + path + ": " + what);
}

}  // namespace

HostTensors read_safetensors(const std::string& path) {
  size_t size = 0;
  std::shared_ptr<const void> map = map_file(path, size);
  const auto* base = static_cast<const uint8_t*>(map.get());
  if (size < 8) bad(path, "shorter than its header length field");
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | base[i];  // little-endian u64
  if (n > size - 8) bad(path, "header length " + std::to_string(n) + " exceeds the file");
  Json header;
  try {
    header = parse_json(std::string(reinterpret_cast<const char*>(base + 8), static_cast<size_t>(n)));
  } catch (const std::invalid_argument& e) {
    bad(path, std::string("bad header: ") + e.what());
  }
  if (!header.is_object()) bad(path, "header is not a JSON object");
  const uint8_t* data = base + 8 + n;
  const size_t data_size = size - 8 - static_cast<size_t>(n);
  HostTensors out;
  for (const auto& [name, info] : header.fields()) {
    if (name == "__metadata__") continue;
    try {
      HostTensor t;
      t.dtype = info.at("dtype").str();
      const size_t item = safetensors_itemsize(t.dtype);
      for (const Json& d : info.at("shape").items()) {
        const int64_t v = d.integer();
        if (v < 0 || v > 0x7fffffff) bad(path, name + ": bad dimension");
        t.shape.push_back(static_cast<int32_t>(v));
      }
      const auto& off = info.at("data_offsets").items();
      if (off.size() != 2) bad(path, name + ": data_offsets needs two entries");
      const int64_t b = off[0].integer(), e = off[1].integer();
      if (b < 0 || e < b || static_cast<uint64_t>(e) > data_size) bad(path, name + ": data_offsets out of range");
      t.nbytes = static_cast<size_t>(e - b);
      size_t want = 0;
      if (__builtin_mul_overflow(t.numel(), item, &want)) bad(path, name + ": tensor size overflows");
      if (t.nbytes != want) bad(path, name + ": data_offsets do not match dtype and shape");
      t.data = data + b;
      t.owner = map;
      out.insert_or_assign(name, std::move(t));
    } catch (const std::invalid_argument& e) {
      const std::string msg = e.what();
      if (msg.rfind("safetensors: " + path, 0) == 0) throw;
      bad(path, name + ": " + msg);
    }
  }
  return out;
}

std::vector<std::string> safetensors_files(const std::string& directory) {
  const fs::path dir(directory);
  const fs::path index = dir / "model.safetensors.index.json";
  if (fs::exists(index)) {
    std::ifstream f(index);
    std::stringstream ss;
    ss << f.rdbuf();
    const Json j = parse_json(ss.str());
    if (j.contains("weight_map")) {
      std::set<std::string> shards;
      for (const auto& [name, file] : j.at("weight_map").fields()) shards.insert(file.str());
      std::vector<std::string> files;
      for (const std::string& s : shards) {
        const fs::path p = dir / s;
        if (!fs::exists(p)) throw std::runtime_error("Missing shard file: " + p.string());
        files.push_back(p.string());
      }
      return files;
    }
  }
  const fs::path single = dir / "model.safetensors";
  if (fs::exists(single) && fs::file_size(single) > 1024) return {single.string()};
  std::vector<std::string> files;
  for (const auto& entry : fs::directory_iterator(dir))
    if (entry.path().extension() == ".safetensors") files.push_back(entry.path().string());
  std::sort(files.begin(), files.end());
  if (files.empty()) throw std::runtime_error("No .safetensors files found in " + directory);
  return files;
}

HostTensors read_safetensors_from_directory(const std::string& directory) {
  HostTensors all;
  for (const std::string& f : safetensors_files(directory))
    for (auto& [name, t] : read_safetensors(f)) all.insert_or_assign(name, std::move(t));
  return all;
}

array to_device(const HostTensor& t) {
  Dtype d;
  if (t.dtype == "BF16") d = Dtype::bfloat16;
  else if (t.dtype == "F32") d = Dtype::float32;
  else if (t.dtype == "U32") d = Dtype::uint32;
  else if (t.dtype == "I32") d = Dtype::int32;
  else throw std::invalid_argument("to_device: dtype " + t.dtype + " has no device array type here");
  Shape s = t.shape.empty() ? Shape{1} : t.shape;
  return array::from_host(t.data, s, d);
}

std::unordered_map<std::string, array> load_safetensors(const std::string& path, const NameFilter& keep) {
  std::unordered_map<std::string, array> out;
  for (const auto& [name, t] : read_safetensors(path))
    if (!keep || keep(name)) out.insert_or_assign(name, to_device(t));
  return out;
}

std::unordered_map<std::string, array> load_safetensors_from_directory(const std::string& directory,
                                                                       const NameFilter& keep) {
  std::unordered_map<std::string, array> out;
  for (const auto& [name, t] : read_safetensors_from_directory(directory))
    if (!keep || keep(name)) out.insert_or_assign(name, to_device(t));
  return out;
}

uint32_t crc32(const void* data, size_t n, uint32_t crc) {
  static const auto table = [] {
    std::vector<uint32_t> tb(256);
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1u) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
      tb[i] = c;
    }
    return tb;
  }();
  const auto* p = static_cast<const uint8_t*>(data);
  crc = ~crc;
  for (size_t i = 0; i < n; ++i) crc = table[(crc ^ p[i]) & 0xffu] ^ (crc >> 8);
  return ~crc;
}

}  // namespace mi355x
}  // namespace mlx_lm
