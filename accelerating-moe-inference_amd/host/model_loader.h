// Weight-file reader of the drop-in API: the reference's model.bin format
// and ModelLoader interface (include/model_loader.h:9-23,
// src/model_loader.cu:14-50), re-implemented.
//
// Format: u32 count, then per tensor: u32 name_len, name bytes, u32 ndim,
// u32 dims[ndim], u64 offset, u64 bytes; every tensor is fp32 row-major at
// `offset` from the start of the file.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "tensor.h"

class ModelLoader {
public:
    explicit ModelLoader(const std::string& path);
    // Reads one tensor into host memory (std::runtime_error if it is absent,
    // not fp32-sized, or truncated).
    Tensor load(const std::string& name) const;
    bool has(const std::string& name) const { return entries_.count(name) != 0; }
    // Shape of a tensor without reading its data (an extension).
    const std::vector<std::size_t>& shape(const std::string& name) const;

private:
    struct Entry {
        std::vector<std::size_t> shape;
        std::uint64_t offset = 0;
        std::uint64_t bytes = 0;
    };
    std::string path_;
    std::unordered_map<std::string, Entry> entries_;
    const Entry& entry(const std::string& name) const;
};
