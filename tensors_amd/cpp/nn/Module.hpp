// Module tree and parameters (reference nn/Module.hpp:18-80, same API) plus
// Module::to(Device), which moves every parameter (recursively) to a device.
#pragma once

#include "tensor/Tensor.hpp"

#include <memory>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace tensorforge::nn {

class Parameter {
public:
    Tensor data_;

    Parameter() = default;
    explicit Parameter(Tensor t) : data_(std::move(t)) { data_.requires_grad(true); }
    Parameter(const Parameter&) = default;
    Parameter(Parameter&&) noexcept = default;
    Parameter& operator=(const Parameter&) = default;
    Parameter& operator=(Parameter&&) noexcept = default;
};

class Module {
public:
    Module() = default;
    virtual ~Module() = default;

    void register_parameter(const std::string& name, Parameter p);
    void register_module(const std::string& name, std::shared_ptr<Module> m);

    virtual Tensor forward(Tensor x) = 0;
    Tensor operator()(Tensor x) { return forward(std::move(x)); }

    std::vector<Parameter*> parameters();
    std::vector<std::pair<std::string, Parameter*>> named_parameters(const std::string& prefix = "");

    // Move all parameters (and submodules') to `device`; they keep
    // requires_grad.  Call before building the optimizer over parameters().
    void to(Device device);

    void train() { training_ = true; }
    void eval() { training_ = false; }
    [[nodiscard]] bool is_training() const noexcept { return training_; }

protected:
    std::unordered_map<std::string, Parameter> parameters_;
    std::unordered_map<std::string, std::shared_ptr<Module>> submodules_;

private:
    bool training_ = true;
};

}  // namespace tensorforge::nn
