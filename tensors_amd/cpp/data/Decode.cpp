#include "data/Decode.hpp"

#include "hip/HipBackend.hpp"
#include "tf_hip.h"

#include <cstring>
#include <fstream>
#include <stdexcept>

namespace tensorforge::data::detail {

std::vector<uint8_t> read_file(const std::string& path, const char* what) {
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in) throw std::runtime_error(std::string(what) + ": cannot open " + path);
    const std::streamoff size = in.tellg();
    std::vector<uint8_t> buf(static_cast<size_t>(size));
    in.seekg(0);
    if (size > 0 && !in.read(reinterpret_cast<char*>(buf.data()), size))
        throw std::runtime_error(std::string(what) + ": read failed on " + path);
    return buf;
}

Tensor decode(const uint8_t* bytes, const Shape& shape, int64_t plane, const ByteTable& table, Device device) {
    const int64_t n = shape.numel();
    const int channels = static_cast<int>(table.size());
    if (device.type == DeviceType::CUDA) {
        // Raw bytes and the table to the device; the decode runs there.
        Tensor raw = Tensor::empty(Shape{n}, Dtype::Bool, Device::cpu());   // one byte per element
        std::memcpy(raw.data(), bytes, static_cast<size_t>(n));
        Tensor tab = Tensor::empty(Shape{channels, 256}, Dtype::Float32, Device::cpu());
        for (int c = 0; c < channels; ++c)
            std::memcpy(static_cast<float*>(tab.data()) + 256 * c, table[c].data(), 256 * sizeof(float));
        Tensor raw_d = raw.to(device), tab_d = tab.to(device);
        Tensor out = Tensor::empty(shape, Dtype::Float32, device);
        hip::check(tf_decode_u8(hip::context(device.index), static_cast<const uint8_t*>(raw_d.data()),
                                static_cast<float*>(out.data()), n, plane, channels,
                                static_cast<const float*>(tab_d.data())),
                   "data::decode");
        return out;
    }
    Tensor out = Tensor::empty(shape, Dtype::Float32, Device::cpu());
    float* o = static_cast<float*>(out.data());
    for (int64_t i = 0; i < n; ++i) o[i] = table[static_cast<size_t>((i / plane) % channels)][bytes[i]];
    return out;
}

Tensor labels(const uint8_t* bytes, int64_t n, Device device) {
    Tensor t = Tensor::empty(Shape{n}, Dtype::Int64, Device::cpu());
    int64_t* o = static_cast<int64_t*>(t.data());
    for (int64_t i = 0; i < n; ++i) o[i] = bytes[i];
    return device.type == DeviceType::CUDA ? t.to(device) : t;
}

}  // namespace tensorforge::data::detail
