#include "model_loader.h"

#include <fstream>
#include <stdexcept>

namespace {

template <class T>
T read_value(std::ifstream& in) {
    T v{};
    in.read(reinterpret_cast<char*>(&v), sizeof(T));
    if (!in) throw std::runtime_error("truncated model.bin");
    return v;
}

}  // namespace

ModelLoader::ModelLoader(const std::string& path) : path_(path) {
    std::ifstream in(path_, std::ios::binary);
    if (!in) throw std::runtime_error("cannot open model: " + path_);
    const auto count = read_value<std::uint32_t>(in);
    for (std::uint32_t i = 0; i < count; ++i) {
        const auto len = read_value<std::uint32_t>(in);
        std::string name(len, '\0');
        in.read(&name[0], len);
        if (!in) throw std::runtime_error("truncated model.bin");
        Entry e;
        const auto ndim = read_value<std::uint32_t>(in);
        e.shape.reserve(ndim);
        for (std::uint32_t d = 0; d < ndim; ++d) e.shape.push_back(read_value<std::uint32_t>(in));
        e.offset = read_value<std::uint64_t>(in);
        e.bytes = read_value<std::uint64_t>(in);
        entries_[name] = std::move(e);
    }
}

const ModelLoader::Entry& ModelLoader::entry(const std::string& name) const {
    const auto it = entries_.find(name);
    if (it == entries_.end()) throw std::runtime_error("missing tensor: " + name);
    return it->second;
}

const std::vector<std::size_t>& ModelLoader::shape(const std::string& name) const {
    return entry(name).shape;
}

Tensor ModelLoader::load(const std::string& name) const {
    const Entry& e = entry(name);
    std::size_t elements = 1;
    for (std::size_t d : e.shape) elements *= d;
    if (e.bytes != elements * sizeof(float))
        throw std::runtime_error("tensor is not float32: " + name);
    Tensor t(e.shape);
    std::ifstream in(path_, std::ios::binary);
    if (!in) throw std::runtime_error("cannot reopen model: " + path_);
    in.seekg(static_cast<std::streamoff>(e.offset));
    in.read(reinterpret_cast<char*>(t.data()), static_cast<std::streamsize>(e.bytes));
    if (!in) throw std::runtime_error("truncated tensor: " + name);
    return t;
}
