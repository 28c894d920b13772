#include "tensor/Compat.hpp"

#include <atomic>

namespace tensorforge::compat {

namespace {
std::atomic<bool> g_linear_drops_bias{false};
std::atomic<bool> g_ln_stub{false};
}  // namespace

void set_reference_compat(bool on) {
    g_linear_drops_bias = on;
    g_ln_stub = on;
}
void set_linear_drops_bias(bool on) { g_linear_drops_bias = on; }
void set_layernorm_stub_backward(bool on) { g_ln_stub = on; }
bool linear_drops_bias() { return g_linear_drops_bias; }
bool layernorm_stub_backward() { return g_ln_stub; }

}  // namespace tensorforge::compat
