// MNIST from its IDX files (reference data/MnistLoader.hpp:8-20): images
// [N, 1, 28, 28] Float32, each pixel (p / 255 - 0.1307) / 0.3081; labels [N]
// Int64 in 0..9.  Errors (missing file, bad magic, not 28 x 28, short file,
// label > 9, image/label count mismatch) throw std::runtime_error.
//
// The Device overloads (an addition to the reference API) copy the raw bytes
// to the device and decode them there (a quarter of the bytes of the
// decoded floats cross the bus), with the same per-byte values as the host
// decode, bit for bit.
#pragma once
#include "tensor/Device.hpp"
#include "tensor/Tensor.hpp"

#include <string>
#include <utility>

namespace tensorforge::data {

std::pair<Tensor, Tensor> load_mnist_train(const std::string& data_dir);
std::pair<Tensor, Tensor> load_mnist_test(const std::string& data_dir);
std::pair<Tensor, Tensor> load_mnist_train(const std::string& data_dir, Device device);
std::pair<Tensor, Tensor> load_mnist_test(const std::string& data_dir, Device device);

}  // namespace tensorforge::data
