// engine.h -- reverse-mode autograd (the reference's Engine, src/inferno/gradengine/engine.{h,cpp}).
//
// backward(root): order the nodes reachable from root's grad_edge
// topologically, seed the root's gradient (ones, or a given tensor), run every
// node's backward() in reverse order, then release() them all.  Gradients
// reaching the same (node, slot) are summed.  grad_enabled is a process-wide
// switch, as in the reference (engine.cpp:6); NoGradGuard clears it for a scope.
#pragma once

#include "inferno/core/tensor.h"

namespace Inferno {

class Node;

extern bool grad_enabled;

class NoGradGuard {
public:
    NoGradGuard() : m_prev(grad_enabled) { grad_enabled = false; }
    ~NoGradGuard() { grad_enabled = m_prev; }
    NoGradGuard(const NoGradGuard&) = delete;
    NoGradGuard& operator=(const NoGradGuard&) = delete;

private:
    bool m_prev;
};

class Engine {
public:
    static void backward(const Tensor& root);
    static void backward(const Tensor& root, const Tensor& seed);
    static void accumulate(Node* node, int slot, const Tensor& g);
    static Tensor grad_in(Node* node, int slot);
};

}  // namespace Inferno
