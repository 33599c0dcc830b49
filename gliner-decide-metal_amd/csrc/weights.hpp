// Host-side weight store (WeightStore, Weights.swift:23-58).
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace gd {

int64_t dtype_size(int dtype);
const char* dtype_name(int dtype);

struct HostTensor {
  int dtype = 0;
  std::vector<int64_t> shape;
  std::vector<uint8_t> data;
  int64_t numel() const;
  std::string shape_string() const;
};

struct WeightStore {
  std::unordered_map<std::string, HostTensor> tensors;

  int add(const std::string& key, const void* data, int dtype, const int64_t* shape, int ndim);
  int load_safetensors(const std::string& path);
  const HostTensor* find(const std::string& key) const;
  int require(const std::string& key, const std::vector<int64_t>& shape, int dtype, const HostTensor** out) const;
};

}  // namespace gd
