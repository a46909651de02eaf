// module.h -- base of the layer modules (include/inferno/modules/module.h of
// the reference, module.cpp): named parameters, buffers and child modules,
// recursive parameters() / to() / state_dict().
#pragma once
#include <map>
#include <string>
#include <unordered_map>
#include <vector>
#include "inferno/core/ops.h"
#include "inferno/core/tensor.h"

namespace Inferno {

using StateDict = std::map<std::string, Tensor>;

class Module {
public:
    virtual ~Module() = default;
    virtual Tensor forward(Tensor& input);  // throws: a module without a one-input forward
    std::vector<Tensor*> parameters() const;
    void register_parameter(const std::string& name, Tensor* tensor);
    void register_module(const std::string& name, Module* module);
    void register_buffer(const std::string& name, Tensor* tensor);
    StateDict state_dict() const;
    void to(const Device& device);
    void collect_state_dict(StateDict& out, const std::string& prefix = "") const;

private:
    // Ordered by name (the reference uses unordered maps), so parameters() and
    // state_dict() have a stable order.
    std::map<std::string, Module*> _children;
    std::map<std::string, Tensor*> _parameters;
    std::map<std::string, Tensor*> _buffers;
};

}  // namespace Inferno
