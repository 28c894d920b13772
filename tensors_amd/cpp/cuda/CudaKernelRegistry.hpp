// Elementwise kernel slots (reference cuda/CudaKernelRegistry.hpp:15-26, same
// API).  The HIP backend fills them with libtf_hip launchers at load time;
// a caller may register its own.  The stream argument is a hipStream_t.
#pragma once

#include "tensor/Dtype.hpp"

#include <cstdint>

namespace tensorforge {

using BinaryOpFn = void (*)(const void*, const void*, void*, int64_t, Dtype, void*);
using UnaryOpFn = void (*)(const void*, void*, int64_t, Dtype, void*);
using LeakyReluFn = void (*)(const void*, void*, int64_t, Dtype, float, void*);

void register_cuda_add(BinaryOpFn fn);
void register_cuda_mul(BinaryOpFn fn);
void register_cuda_relu(UnaryOpFn fn);
void register_cuda_sigmoid(UnaryOpFn fn);
void register_cuda_tanh(UnaryOpFn fn);
void register_cuda_leaky_relu(LeakyReluFn fn);
void register_current_stream(void* stream);

}  // namespace tensorforge
