// CIFAR-10 from its binary batches (reference data/CifarLoader.hpp:8-20):
// each record is one label byte then 1024 R, 1024 G and 1024 B bytes;
// images [N, 3, 32, 32] Float32 NCHW, channel c normalised as
// (p / 255 - mean[c]) / std[c] with mean (0.4914, 0.4822, 0.4465) and std
// (0.2470, 0.2435, 0.2616); labels [N] Int64 in 0..9.  The training split
// concatenates data_batch_1.bin .. data_batch_5.bin, the test split is
// test_batch.bin.  Errors (missing file, size not a whole number of
// records, label > 9) throw std::runtime_error.  Device overloads as for
// MNIST: raw bytes to the device, decoded there, bit for bit the host values.
#pragma once
#include "tensor/Device.hpp"
#include "tensor/Tensor.hpp"

#include <string>
#include <utility>

namespace tensorforge::data {

std::pair<Tensor, Tensor> load_cifar10_train(const std::string& data_dir);
std::pair<Tensor, Tensor> load_cifar10_test(const std::string& data_dir);
std::pair<Tensor, Tensor> load_cifar10_train(const std::string& data_dir, Device device);
std::pair<Tensor, Tensor> load_cifar10_test(const std::string& data_dir, Device device);

}  // namespace tensorforge::data
