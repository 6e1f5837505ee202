// traced.hpp — drop-in for the traced layers' optimizer surface (autograd/traced/*.hpp).
//
// The reference's traced layers own pre-allocated weight and gradient buffers that every
// backward overwrites (autograd/traced/nn.hpp:54-69), and update themselves with
// sgd_step(lr) = `w - lr*dw` per tensor (autograd/traced/nn.hpp:93-96, 272-275, 317-321).
// Here the buffers are tensors of one ParamArena whose grads always exist (zero until a
// backward writes them), and each sgd_step is one launch over that module's tensors.
// TracedSGD (autograd/traced/optim.hpp:15-29) steps all its layers in one launch.
#pragma once

#include <initializer_list>
#include <vector>

#include "autograd/value.hpp"

namespace traced {

using autograd::ParamArena;
using autograd::ValuePtr;

namespace detail {
inline void sgd_on(const std::vector<ValuePtr>& ps, float lr) {
    if (ps.empty()) return;
    std::vector<uint32_t> idx;
    for (auto& p : ps) idx.push_back(p->index);
    ttp::SgdOptions o;
    o.lr = lr;
    ps.front()->store().sgd_step(o, &idx);
}
}  // namespace detail

// y = x @ weight.T + bias;  weight [out, in] filled with `init`, bias [1, out] zeros
// (autograd/traced/nn.hpp:61-68)
struct TracedLinear {
    ValuePtr weight, bias;  // d_weight / d_bias are weight->grad / bias->grad
    uint32_t in_features, out_features;

    TracedLinear(uint32_t in_f, uint32_t out_f, float init, ParamArena& arena)
        : weight(arena.parameter({out_f, in_f}, autograd::filled((uint64_t)out_f * in_f, init),
                                 "weight", true, /*grad_always=*/true)),
          bias(arena.parameter({1, out_f}, autograd::filled(out_f, 0.0f), "bias", false, true)),
          in_features(in_f),
          out_features(out_f) {}

    std::vector<ValuePtr> parameters() const { return {weight, bias}; }
    void sgd_step(float lr) { detail::sgd_on(parameters(), lr); }
};

// gamma ones, beta zeros (autograd/traced/nn.hpp LayerNorm)
struct TracedLayerNorm {
    ValuePtr gamma, beta;

    TracedLayerNorm(uint32_t dim, ParamArena& arena)
        : gamma(arena.parameter({1, dim}, autograd::filled(dim, 1.0f), "gamma", false, true)),
          beta(arena.parameter({1, dim}, autograd::filled(dim, 0.0f), "beta", false, true)) {}

    std::vector<ValuePtr> parameters() const { return {gamma, beta}; }
    void sgd_step(float lr) { detail::sgd_on(parameters(), lr); }
};

// [vocab, dim] table filled with `init` (autograd/traced/nn.hpp:308-315).  The reference
// untilizes d_weight before its update (:317-321); the flat store has a single row-major
// layout, so there is nothing to convert.
struct TracedEmbedding {
    ValuePtr weight;

    TracedEmbedding(uint32_t vocab, uint32_t dim, float init, ParamArena& arena)
        : weight(arena.parameter({vocab, dim}, autograd::filled((uint64_t)vocab * dim, init),
                                 "embedding", true, true)) {}

    std::vector<ValuePtr> parameters() const { return {weight}; }
    void sgd_step(float lr) { detail::sgd_on(parameters(), lr); }
};

// autograd/traced/ops.hpp:132-134: param = param - lr * grad (one tensor)
inline void sgd_update(const ValuePtr& param, float lr) { detail::sgd_on({param}, lr); }

// traced::TraceContext (autograd/traced/trace.hpp:21-88) over a ttp::Store: the first
// run(fn) captures the work fn queues on the store's stream into a hipGraph and executes it;
// later calls replay it.  Step the captured tensor sets once eagerly before the first run.
// Release (or destroy) the TraceContext before the store.
class TraceContext {
public:
    explicit TraceContext(ttp::Store& store) : store_(&store) {}
    TraceContext(const TraceContext&) = delete;
    TraceContext& operator=(const TraceContext&) = delete;
    TraceContext(TraceContext&&) = default;
    TraceContext& operator=(TraceContext&&) = default;

    template <typename Fn>
    void run(Fn&& fn) {
        if (!graph_) {
            store_->begin_capture();
            try {
                fn();
            } catch (...) {
                store_->discard_capture();
                throw;
            }
            graph_ = store_->end_capture();
        }
        graph_.launch();
    }
    bool is_captured() const { return (bool)graph_; }
    void release() { graph_.reset(); }
    void reset() { release(); }

private:
    ttp::Store* store_;
    ttp::Graph graph_;
};

struct TracedSGD {
    std::vector<TracedLinear*> layers;
    float lr;

    TracedSGD(std::initializer_list<TracedLinear*> ls, float learning_rate)
        : layers(ls), lr(learning_rate) {}

    // one launch over every layer's weight and bias
    void step() {
        std::vector<ValuePtr> ps;
        for (auto* l : layers) {
            ps.push_back(l->weight);
            ps.push_back(l->bias);
        }
        detail::sgd_on(ps, lr);
    }
    // no zero_grad: gradients are overwritten each backward pass (autograd/traced/optim.hpp:28)
};

}  // namespace traced
