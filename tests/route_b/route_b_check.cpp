// Route-B check: the reference's own tensor/ code, compiled from its sources,
// with the registrar of INTEGRATION.md (section B) linked in, so that its
// CUDA-device tensors allocate, copy and run the elementwise slots through
// libtf_hip.  Built by `make -C oracle routeb` into oracle/_ref/.
//
//   route_b_check registry   the registrar's static initialiser installed the
//                            allocator and the copy callback (no GPU needed)
//   route_b_check gpu        add, mul, relu, sigmoid, tanh and leaky_relu on
//                            device tensors against the reference's own CPU
//                            loops on the same inputs (tensor/Tensor.cpp)
//
// Bars: add, mul, relu and leaky_relu are single IEEE operations or
// selections, so bit-exact; sigmoid and tanh call the device's exp / tanh,
// within 1e-6 relative + 1e-7 absolute of the host's.
#include "tensor/CPUStorageAllocator.hpp"
#include "tensor/Tensor.hpp"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

using namespace tensorforge;

namespace {

Tensor filled(int64_t n, uint32_t seed) {
    Tensor t = Tensor::empty(Shape{n}, Dtype::Float32, Device::cpu());
    float* p = static_cast<float*>(t.data());
    uint32_t s = seed;
    for (int64_t i = 0; i < n; ++i) {
        s = s * 1664525u + 1013904223u;
        p[i] = (static_cast<float>(s >> 8) / 16777216.0f - 0.5f) * 16.0f;  // [-8, 8)
    }
    if (n >= 4) {
        p[0] = 0.0f;
        p[1] = -0.0f;
        p[2] = -1e-30f;
        p[3] = 1e30f;
    }
    return t;
}

int compare(const char* what, int64_t n, const Tensor& got_dev, const Tensor& want, double rtol, double atol) {
    Tensor got = got_dev.to(Device::cpu());
    const float* g = static_cast<const float*>(got.data());
    const float* w = static_cast<const float*>(want.data());
    int64_t bad = 0, first = -1;
    for (int64_t i = 0; i < n; ++i) {
        bool ok;
        if (rtol == 0.0 && atol == 0.0) ok = std::memcmp(&g[i], &w[i], sizeof(float)) == 0;
        else ok = std::fabs((double)g[i] - (double)w[i]) <= atol + rtol * std::fabs((double)w[i]);
        if (!ok) {
            if (first < 0) first = i;
            ++bad;
        }
    }
    if (bad) {
        std::printf("FAIL %s n=%lld: %lld mismatches, first at %lld: got %.9g want %.9g\n", what, (long long)n,
                    (long long)bad, (long long)first, g[first], w[first]);
        return 1;
    }
    std::printf("ok %s n=%lld\n", what, (long long)n);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "registry";
    if (allocator_dispatch::get_allocator(DeviceType::CUDA) == nullptr || !allocator_dispatch::cuda_copy_available()) {
        std::printf("FAIL the registrar did not install the CUDA allocator / copy callback\n");
        return 1;
    }
    if (mode == "registry") {
        std::printf("route B registry ok\n");
        return 0;
    }
    if (mode != "gpu") {
        std::printf("usage: route_b_check [registry|gpu]\n");
        return 2;
    }
    int fails = 0;
    try {
        for (int64_t n : {int64_t{1}, int64_t{1000}, int64_t{(1 << 20) + 3}}) {
            const Tensor a = filled(n, 11u + (uint32_t)n), b = filled(n, 29u + (uint32_t)n);
            const Tensor da = a.to(Device::cuda(0)), db = b.to(Device::cuda(0));
            fails += compare("add", n, da + db, a + b, 0, 0);
            fails += compare("mul", n, da * db, a * b, 0, 0);
            fails += compare("relu", n, da.relu(), a.relu(), 0, 0);
            fails += compare("leaky_relu", n, da.leaky_relu(0.1f), a.leaky_relu(0.1f), 0, 0);
            fails += compare("sigmoid", n, da.sigmoid(), a.sigmoid(), 1e-6, 1e-7);
            fails += compare("tanh", n, da.tanh(), a.tanh(), 1e-6, 1e-7);
        }
    } catch (const std::exception& e) {
        std::printf("FAIL exception: %s\n", e.what());
        return 1;
    }
    std::printf(fails ? "route B gpu: %d failures\n" : "route B gpu ok\n", fails);
    return fails ? 1 : 0;
}
