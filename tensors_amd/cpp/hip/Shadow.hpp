// bf16 shadows of fp32 master parameters (mixed precision).  A module that
// computes in bf16 asks for the shadow of its fp32 weight; the SGD step
// writes the shadow in the same pass that updates the master
// (tf_sgd_momentum's p_bf16 output), so no separate cast runs per step.
// A shadow is refreshed by a cast when the master's version moved without it.
#pragma once

#include "tensor/Tensor.hpp"

namespace tensorforge::hip {

// bf16 copy of `master` (GPU, Float32), current with master's version.
[[nodiscard]] Tensor shadow_for(const Tensor& master);
// The registered shadow of `master`, or an empty tensor.
[[nodiscard]] Tensor find_shadow(const Tensor& master);
// Record that `shadow` now equals bf16(master) at master's current version.
void mark_shadow_current(const Tensor& master);

}  // namespace tensorforge::hip
