// Switches that reproduce documented reference behaviour where this backend
// otherwise corrects it.  Both default to the corrected behaviour.
//   linear_drops_bias:       nn::Linear::forward ignores its bias
//                            (reference nn/Linear.cpp:60-63).
//   layernorm_stub_backward: LayerNormBackward returns dx = dy * gamma and
//                            zero dgamma / dbeta (reference
//                            autograd/ops/LayerNormBackward.hpp:39-59).
#pragma once

namespace tensorforge::compat {

void set_reference_compat(bool on);  // sets both switches
void set_linear_drops_bias(bool on);
void set_layernorm_stub_backward(bool on);
[[nodiscard]] bool linear_drops_bias();
[[nodiscard]] bool layernorm_stub_backward();

}  // namespace tensorforge::compat
