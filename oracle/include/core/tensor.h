// ORACLE (test infrastructure only): storage for the CPU restatement: a 64-byte aligned buffer, the
// exact-size weights reader ("incorrect byte size" on mismatch) and a typed view with a static shape
// (chroma/_src/core/tensor.h:12-49).
#pragma once

#include "bfloat16.h"
#include "layout.h"
#include <cstdio>
#include <new>
#include <stdexcept>
#include <type_traits>

namespace chroma {
class Buffer {
public:
    explicit Buffer(size_t bytes) : bytes_(bytes), data_(allocate(bytes)) {}
    ~Buffer() { ::operator delete(data_, std::align_val_t{64}); }
    Buffer(const Buffer&) = delete;
    Buffer& operator=(const Buffer&) = delete;
    std::byte* data() { return data_; }
    const std::byte* data() const { return data_; }
    size_t size() const { return bytes_; }

private:
    static std::byte* allocate(size_t bytes) {
        return static_cast<std::byte*>(::operator new(bytes ? bytes : 1, std::align_val_t{64}));
    }
    size_t bytes_;
    std::byte* data_;
};

inline void read_weights(const char* path, void* destination, size_t bytes) {
    std::FILE* file = std::fopen(path, "rb");
    long size = -1;
    if (file && std::fseek(file, 0, SEEK_END) == 0) {
        size = std::ftell(file);
    }
    if (!file || size != static_cast<long>(bytes)) {
        if (file) {
            std::fclose(file);
        }
        throw std::runtime_error("Missing weights file or incorrect byte size");
    }
    std::rewind(file);
    const size_t read = bytes ? std::fread(destination, 1, bytes, file) : 0;
    std::fclose(file);
    if (read != bytes) {
        throw std::runtime_error("Cannot read weights");
    }
}

template <class T, auto Extents> struct TensorView {
    using value_type = std::remove_const_t<T>;
    static constexpr auto shape = Extents;
    T* data;
    value_type operator[](size_t i) const { return data[i]; }
};

template <class T, auto Extents> TensorView<T, Extents> view(T* data) { return {data}; }
}  // namespace chroma
