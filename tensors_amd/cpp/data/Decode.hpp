// Shared pieces of the file loaders: whole-file reads, big-endian fields,
// and the byte -> float decode through a per-channel table of 256 values
// (the normalisation applied once per byte value, not once per pixel), on
// the host or, from bytes copied to the device, by tf_decode_u8.
#pragma once
#include "tensor/Device.hpp"
#include "tensor/Tensor.hpp"

#include <array>
#include <cstdint>
#include <string>
#include <vector>

namespace tensorforge::data::detail {

// The file's bytes; throws std::runtime_error("<what>: cannot open <path>").
std::vector<uint8_t> read_file(const std::string& path, const char* what);

inline uint32_t be32(const uint8_t* p) {
    return (uint32_t(p[0]) << 24) | (uint32_t(p[1]) << 16) | (uint32_t(p[2]) << 8) | uint32_t(p[3]);
}

// table[c][b] = the normalised value of byte b in channel c.
using ByteTable = std::vector<std::array<float, 256>>;

// Float32 tensor `shape` on `device` whose element i is
// table[(i / plane) % channels][bytes[i]] (bytes holds shape.numel() values).
Tensor decode(const uint8_t* bytes, const Shape& shape, int64_t plane, const ByteTable& table, Device device);

// Int64 tensor [n] on `device` from n label bytes (each checked <= 9 by the caller).
Tensor labels(const uint8_t* bytes, int64_t n, Device device);

}  // namespace tensorforge::data::detail
