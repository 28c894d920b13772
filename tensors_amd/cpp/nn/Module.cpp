#include "nn/Module.hpp"

namespace tensorforge::nn {

void Module::register_parameter(const std::string& name, Parameter p) { parameters_[name] = std::move(p); }

void Module::register_module(const std::string& name, std::shared_ptr<Module> m) { submodules_[name] = std::move(m); }

std::vector<Parameter*> Module::parameters() {
    std::vector<Parameter*> out;
    for (auto& kv : parameters_) out.push_back(&kv.second);
    for (auto& kv : submodules_)
        if (kv.second)
            for (Parameter* p : kv.second->parameters()) out.push_back(p);
    return out;
}

std::vector<std::pair<std::string, Parameter*>> Module::named_parameters(const std::string& prefix) {
    std::vector<std::pair<std::string, Parameter*>> out;
    for (auto& kv : parameters_) out.emplace_back(prefix.empty() ? kv.first : prefix + "." + kv.first, &kv.second);
    for (auto& kv : submodules_) {
        if (!kv.second) continue;
        for (auto& sub : kv.second->named_parameters(prefix.empty() ? kv.first : prefix + "." + kv.first))
            out.push_back(std::move(sub));
    }
    return out;
}

void Module::to(Device device) {
    for (auto& kv : parameters_) {
        Parameter& p = kv.second;
        if (p.data_.device() == device) continue;
        const bool req = p.data_.requires_grad();
        p.data_ = p.data_.to(device);
        p.data_.requires_grad(req);
    }
    for (auto& kv : submodules_)
        if (kv.second) kv.second->to(device);
}

}  // namespace tensorforge::nn
