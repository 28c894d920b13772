// Activation modules (reference nn/Activations.hpp:12-26, same API).
#pragma once

#include "nn/Module.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge::nn {

class ReLU : public Module {
public:
    Tensor forward(Tensor x) override;
};

class Sigmoid : public Module {
public:
    Tensor forward(Tensor x) override;
};

class Tanh : public Module {
public:
    Tensor forward(Tensor x) override;
};

}  // namespace tensorforge::nn
