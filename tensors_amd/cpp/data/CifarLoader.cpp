// CIFAR-10 binary loader (behaviour of reference data/CifarLoader.cpp:20-168).
#include "data/CifarLoader.hpp"

#include "data/Decode.hpp"

#include <stdexcept>
#include <string>
#include <vector>

namespace tensorforge::data {

namespace {

constexpr int64_t kPlane = 32 * 32;
constexpr int64_t kRecord = 1 + 3 * kPlane;

// The reference's normalisation, in its float operations:
// (p * (1 / 255) - mean[c]) / std[c], once per byte value and channel.
detail::ByteTable cifar_table() {
    const float inv255 = 1.0f / 255.0f;
    const float mean[3] = {0.4914f, 0.4822f, 0.4465f}, stdv[3] = {0.2470f, 0.2435f, 0.2616f};
    detail::ByteTable t(3);
    for (int c = 0; c < 3; ++c)
        for (int b = 0; b < 256; ++b) t[c][b] = (static_cast<float>(b) * inv255 - mean[c]) / stdv[c];
    return t;
}

std::pair<Tensor, Tensor> load(const std::string& dir, const std::vector<const char*>& files, Device device) {
    // Pixels of every record, label bytes apart: [N][3][1024] and [N].
    std::vector<uint8_t> pixels, labels;
    for (const char* f : files) {
        const std::string path = dir + "/" + f;
        const std::vector<uint8_t> buf = detail::read_file(path, "CIFAR-10");
        if (buf.size() % kRecord != 0)
            throw std::runtime_error("CIFAR-10: " + path + " holds " + std::to_string(buf.size()) +
                                     " bytes, not a whole number of " + std::to_string(kRecord) + "-byte records");
        for (size_t r = 0; r < buf.size(); r += kRecord) {
            if (buf[r] > 9)
                throw std::runtime_error("CIFAR-10: label " + std::to_string(buf[r]) + " out of range in " + path);
            labels.push_back(buf[r]);
            pixels.insert(pixels.end(), buf.begin() + static_cast<std::ptrdiff_t>(r + 1),
                          buf.begin() + static_cast<std::ptrdiff_t>(r + kRecord));
        }
    }
    const int64_t n = static_cast<int64_t>(labels.size());
    static const detail::ByteTable table = cifar_table();
    return {detail::decode(pixels.data(), Shape{n, 3, 32, 32}, kPlane, table, device),
            detail::labels(labels.data(), n, device)};
}

}  // namespace

std::pair<Tensor, Tensor> load_cifar10_train(const std::string& data_dir, Device device) {
    return load(data_dir, {"data_batch_1.bin", "data_batch_2.bin", "data_batch_3.bin", "data_batch_4.bin",
                           "data_batch_5.bin"},
                device);
}
std::pair<Tensor, Tensor> load_cifar10_test(const std::string& data_dir, Device device) {
    return load(data_dir, {"test_batch.bin"}, device);
}
std::pair<Tensor, Tensor> load_cifar10_train(const std::string& data_dir) {
    return load_cifar10_train(data_dir, Device::cpu());
}
std::pair<Tensor, Tensor> load_cifar10_test(const std::string& data_dir) {
    return load_cifar10_test(data_dir, Device::cpu());
}

}  // namespace tensorforge::data
