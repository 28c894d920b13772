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
// within 1e-6 relative + 1e-7 absolute of the host's.  The gpu mode repeats
// the six slots on Float16 device tensors (the dtype the reference's
// registry also serves, cuda/kernels/elementwise.cu:185-245): expected =
// the host's fp32 loop on the widened inputs, rounded to half (nearest
// even); bit-exact for the four exact ops, within one half step for
// sigmoid and tanh.
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

// IEEE binary16 from / to float32 (round to nearest even; no NaNs occur in
// the checks), written from the format: 5 exponent bits biased by 15,
// 10 fraction bits, subnormals k * 2^-24.
uint16_t to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xFFu, man = x & 0x7FFFFFu;
    if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    if (exp == 0u) return (uint16_t)sign;
    const int32_t e = (int32_t)exp - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    uint32_t q, rem, half;
    if (e >= 1) {
        q = ((uint32_t)e << 10) | (man >> 13);
        rem = man & 0x1FFFu;
        half = 0x1000u;
    } else {
        const int sh = 14 - e;
        if (sh > 25) return (uint16_t)sign;
        const uint32_t M = man | 0x800000u;
        q = M >> sh;
        rem = M & ((1u << sh) - 1u);
        half = 1u << (sh - 1);
    }
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

float from_half(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    float f;
    if (exp == 0u) {
        f = std::ldexp((float)man, -24);
        return sign ? -f : f;
    }
    const uint32_t x = exp == 31u ? (sign | 0x7F800000u | (man << 13)) : (sign | ((exp + 112u) << 23) | (man << 13));
    std::memcpy(&f, &x, sizeof f);
    return f;
}

// Half host tensor of the values of a float tensor (rounded), and the float
// tensor of its exact widening.
Tensor to_half_tensor(const Tensor& f) {
    Tensor h = Tensor::empty(f.shape(), Dtype::Float16, Device::cpu());
    const float* src = static_cast<const float*>(f.data());
    uint16_t* dst = static_cast<uint16_t*>(h.data());
    for (int64_t i = 0; i < f.numel(); ++i) dst[i] = to_half(src[i]);
    return h;
}
Tensor widen(const Tensor& h) {
    Tensor f = Tensor::empty(h.shape(), Dtype::Float32, Device::cpu());
    const uint16_t* src = static_cast<const uint16_t*>(h.data());
    float* dst = static_cast<float*>(f.data());
    for (int64_t i = 0; i < h.numel(); ++i) dst[i] = from_half(src[i]);
    return f;
}

// got (a Float16 device tensor) against the float tensor `want` rounded to
// half: bit-exact with steps == 0, else within `steps` half steps (relative
// 2^-10 per step, absolute 2^-24 near zero).
int compare_half(const char* what, int64_t n, const Tensor& got_dev, const Tensor& want, int steps) {
    Tensor got = got_dev.to(Device::cpu());
    if (got.dtype() != Dtype::Float16) {
        std::printf("FAIL %s: result dtype is not Float16\n", what);
        return 1;
    }
    const uint16_t* g = static_cast<const uint16_t*>(got.data());
    const float* w = static_cast<const float*>(want.data());
    int64_t bad = 0, first = -1;
    for (int64_t i = 0; i < n; ++i) {
        const uint16_t wh = to_half(w[i]);
        bool ok;
        if (steps == 0) ok = g[i] == wh;
        else {
            const double gv = from_half(g[i]), wv = from_half(wh);
            ok = std::fabs(gv - wv) <= steps * (std::ldexp(1.0, -24) + std::ldexp(std::fabs(wv), -10));
        }
        if (!ok) {
            if (first < 0) first = i;
            ++bad;
        }
    }
    if (bad) {
        std::printf("FAIL %s n=%lld: %lld mismatches, first at %lld: got 0x%04x want 0x%04x\n", what, (long long)n,
                    (long long)bad, (long long)first, g[first], to_half(w[first]));
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
            // Float16 device tensors through the same slots.
            const Tensor ha = to_half_tensor(a), hb = to_half_tensor(b);
            const Tensor wa = widen(ha), wb = widen(hb);
            const Tensor dha = ha.to(Device::cuda(0)), dhb = hb.to(Device::cuda(0));
            fails += compare_half("f16 add", n, dha + dhb, wa + wb, 0);
            fails += compare_half("f16 mul", n, dha * dhb, wa * wb, 0);
            fails += compare_half("f16 relu", n, dha.relu(), wa.relu(), 0);
            fails += compare_half("f16 leaky_relu", n, dha.leaky_relu(0.1f), wa.leaky_relu(0.1f), 0);
            fails += compare_half("f16 sigmoid", n, dha.sigmoid(), wa.sigmoid(), 1);
            fails += compare_half("f16 tanh", n, dha.tanh(), wa.tanh(), 1);
        }
    } catch (const std::exception& e) {
        std::printf("FAIL exception: %s\n", e.what());
        return 1;
    }
    std::printf(fails ? "route B gpu: %d failures\n" : "route B gpu ok\n", fails);
    return fails ? 1 : 0;
}
