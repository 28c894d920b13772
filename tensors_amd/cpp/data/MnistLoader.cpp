// MNIST IDX loader (behaviour of reference data/MnistLoader.cpp:23-162).
// An image file is the big-endian header magic 0x00000803 | count | rows |
// cols followed by count * rows * cols pixel bytes; a label file is magic
// 0x00000801 | count followed by count label bytes.
#include "data/MnistLoader.hpp"

#include "data/Decode.hpp"

#include <stdexcept>
#include <string>

namespace tensorforge::data {

namespace {

constexpr uint32_t kImageMagic = 0x00000803u;
constexpr uint32_t kLabelMagic = 0x00000801u;

// The reference's normalisation, in its float operations:
// (p * (1 / 255) - 0.1307) * (1 / 0.3081), once per byte value.
detail::ByteTable mnist_table() {
    const float inv255 = 1.0f / 255.0f, mean = 0.1307f, inv_std = 1.0f / 0.3081f;
    detail::ByteTable t(1);
    for (int b = 0; b < 256; ++b) t[0][b] = (static_cast<float>(b) * inv255 - mean) * inv_std;
    return t;
}

std::pair<Tensor, Tensor> load(const std::string& dir, const char* images, const char* labels, Device device) {
    const std::string ip = dir + "/" + images, lp = dir + "/" + labels;
    const std::vector<uint8_t> fi = detail::read_file(ip, "MNIST IDX");
    const std::vector<uint8_t> fl = detail::read_file(lp, "MNIST IDX");
    if (fi.size() < 16 || detail::be32(fi.data()) != kImageMagic)
        throw std::runtime_error("MNIST IDX: " + ip + " is not an image file (bad magic or header)");
    const int64_t n = detail::be32(fi.data() + 4);
    const uint32_t rows = detail::be32(fi.data() + 8), cols = detail::be32(fi.data() + 12);
    if (rows != 28 || cols != 28)
        throw std::runtime_error("MNIST IDX: images are " + std::to_string(rows) + "x" + std::to_string(cols) +
                                 ", not 28x28");
    if (static_cast<int64_t>(fi.size()) - 16 < n * 784) throw std::runtime_error("MNIST IDX: " + ip + " is short");
    if (fl.size() < 8 || detail::be32(fl.data()) != kLabelMagic)
        throw std::runtime_error("MNIST IDX: " + lp + " is not a label file (bad magic or header)");
    const int64_t nl = detail::be32(fl.data() + 4);
    if (static_cast<int64_t>(fl.size()) - 8 < nl) throw std::runtime_error("MNIST IDX: " + lp + " is short");
    if (nl != n)
        throw std::runtime_error("MNIST IDX: " + std::to_string(n) + " images but " + std::to_string(nl) + " labels");
    for (int64_t i = 0; i < nl; ++i)
        if (fl[8 + i] > 9) throw std::runtime_error("MNIST IDX: label " + std::to_string(fl[8 + i]) + " out of range");
    static const detail::ByteTable table = mnist_table();
    return {detail::decode(fi.data() + 16, Shape{n, 1, 28, 28}, 784, table, device),
            detail::labels(fl.data() + 8, n, device)};
}

}  // namespace

std::pair<Tensor, Tensor> load_mnist_train(const std::string& data_dir, Device device) {
    return load(data_dir, "train-images-idx3-ubyte", "train-labels-idx1-ubyte", device);
}
std::pair<Tensor, Tensor> load_mnist_test(const std::string& data_dir, Device device) {
    return load(data_dir, "t10k-images-idx3-ubyte", "t10k-labels-idx1-ubyte", device);
}
std::pair<Tensor, Tensor> load_mnist_train(const std::string& data_dir) {
    return load_mnist_train(data_dir, Device::cpu());
}
std::pair<Tensor, Tensor> load_mnist_test(const std::string& data_dir) { return load_mnist_test(data_dir, Device::cpu()); }

}  // namespace tensorforge::data
