// static.hpp — drop-in for the optimizer surface of the static autograd's layers
// (autograd/static/nn.hpp): Linear, LinearReLU, MLP and FusedMLP own weight/bias plus
// pre-allocated gradient buffers (d_weight/d_bias), update themselves with
// sgd_step(lr) = `w - lr*dw` per tensor (:92-95, :178-181, :213-216, :242-245) and reset the
// gradient buffers with zero_grad() = zeros_like (:98-101, :183-186, :218-221, :247-250).
// Here the buffers are tensors of one ParamArena; sgd_step is one launch over the module's
// tensors and zero_grad one fill launch (the gradients stay present, as zeros).  Forward and
// backward compute are not part of this engine: a backward writes d_weight / d_bias through
// grad_ptr() / accumulate_grad(...).
#pragma once

#include <vector>

#include "autograd/value.hpp"

namespace static_autograd {

using autograd::ParamArena;
using autograd::ValuePtr;

namespace detail {
inline std::vector<uint32_t> indices(const std::vector<ValuePtr>& ps) {
    std::vector<uint32_t> idx;
    for (auto& p : ps) idx.push_back(p->index);
    return idx;
}
inline void sgd(const std::vector<ValuePtr>& ps, float lr) {
    if (ps.empty()) return;
    ttp::SgdOptions o;
    o.lr = lr;
    auto idx = indices(ps);
    ps.front()->store().sgd_step(o, &idx);
}
// zeros_like gradients (autograd/static/nn.hpp:98-101): zeroed and present afterwards, so
// the next sgd_step updates every listed tensor even before a backward has written it
inline void zero(const std::vector<ValuePtr>& ps) {
    if (ps.empty()) return;
    ttp::Store& st = ps.front()->store();
    const auto idx = indices(ps);
    st.zero_grad(idx, /*set_to_none=*/false);
    for (uint32_t i : idx) st.set_has_grad(i, true);
}
}  // namespace detail

// weight [out, in] filled with `init`, bias [1, out] zeros (autograd/static/nn.hpp:40-52)
struct Linear {
    ValuePtr weight, bias;  // d_weight / d_bias are weight->grad / bias->grad
    uint32_t in_features, out_features, batch_size;

    Linear(uint32_t batch, uint32_t in_f, uint32_t out_f, float init, ParamArena& arena)
        : weight(arena.parameter({out_f, in_f}, autograd::filled((uint64_t)out_f * in_f, init),
                                 "weight", /*decay=*/true, /*grad_always=*/true)),
          bias(arena.parameter({1, out_f}, autograd::filled(out_f, 0.0f), "bias", false, true)),
          in_features(in_f),
          out_features(out_f),
          batch_size(batch) {}

    std::vector<ValuePtr> parameters() const { return {weight, bias}; }
    void sgd_step(float lr) { detail::sgd(parameters(), lr); }
    void zero_grad() { detail::zero(parameters()); }
};

// Linear with a fused ReLU (autograd/static/nn.hpp:108-186): the same parameters
struct LinearReLU : Linear {
    using Linear::Linear;
};

struct MLP {
    Linear layer1, layer2;

    MLP(uint32_t batch, uint32_t in_dim, uint32_t hidden_dim, uint32_t out_dim, float init,
        ParamArena& arena)
        : layer1(batch, in_dim, hidden_dim, init, arena),
          layer2(batch, hidden_dim, out_dim, init, arena) {}

    std::vector<ValuePtr> parameters() const {
        return {layer1.weight, layer1.bias, layer2.weight, layer2.bias};
    }
    void sgd_step(float lr) { detail::sgd(parameters(), lr); }  // one launch, both layers
    void zero_grad() { detail::zero(parameters()); }
};

struct FusedMLP {
    LinearReLU layer1;
    Linear layer2;

    FusedMLP(uint32_t batch, uint32_t in_dim, uint32_t hidden_dim, uint32_t out_dim, float init,
             ParamArena& arena)
        : layer1(batch, in_dim, hidden_dim, init, arena),
          layer2(batch, hidden_dim, out_dim, init, arena) {}

    std::vector<ValuePtr> parameters() const {
        return {layer1.weight, layer1.bias, layer2.weight, layer2.bias};
    }
    void sgd_step(float lr) { detail::sgd(parameters(), lr); }
    void zero_grad() { detail::zero(parameters()); }
};

// autograd/static/nn.hpp:257-345: two dim x dim Linear layers filled with 0.01 and a learning
// rate; the reference's train_step builds and runs the forward / backward graph (model
// compute, not this engine) and ends with layer1.sgd_step(lr); layer2.sgd_step(lr)
// (:343-344), which sgd_step() does here in one launch.
struct PersistentMLP {
    Linear layer1, layer2;
    float lr;

    PersistentMLP(uint32_t batch, uint32_t dim, float learning_rate, ParamArena& arena)
        : layer1(batch, dim, dim, 0.01f, arena),
          layer2(batch, dim, dim, 0.01f, arena),
          lr(learning_rate) {}

    std::vector<ValuePtr> parameters() const {
        return {layer1.weight, layer1.bias, layer2.weight, layer2.bias};
    }
    void sgd_step() { detail::sgd(parameters(), lr); }
    void zero_grad() { detail::zero(parameters()); }  // the graph's zero_grad: grads stay, zero
};

}  // namespace static_autograd
