// value.hpp — parameters of the drop-in autograd API, stored in one flat HBM store.
//
// The reference's autograd::Value owns its `data` tensor and an optional `grad`
// (autograd/dynamic/autograd.hpp:38-84); static_autograd::Value points at external
// buffers (autograd/static/value.hpp:27-48).  Here every parameter is a non-owning view
// (arena, index) into a ttp::Store that holds all parameters of a model contiguously, so an
// optimizer step over all of them is one launch.  Parameters are declared on a ParamArena;
// the store is created on first use, after which the parameter set is fixed.
#pragma once

#include <cstdint>
#include <algorithm>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "ttperf/ttperf.hpp"

namespace autograd {

class ParamArena;

// Which store layout an arena creates (ttp::Layout).  Auto: the SGD layout for a Mixed
// arena, unless an Adam / AdamW over its parameters was constructed before the store exists
// (the store is created on first use).  An Adam constructed later converts the store at its
// first step, once.
enum class ArenaLayout { Auto, Default, Sgd };

struct ArenaState {
    ttp::Mode mode = ttp::Mode::FP32;
    int device = 0;
    ArenaLayout layout = ArenaLayout::Auto;
    bool adam_declared = false;  // an Adam over this arena's parameters was constructed
    std::vector<ttp::TensorSpec> specs;
    std::vector<std::vector<float>> init;  // initial fp32 weights (uploaded at creation)
    std::vector<bool> grad_always;         // pre-allocated grads (traced/static layers)
    std::unique_ptr<ttp::Store> store;

    ttp::Layout store_layout() const {
        if (layout == ArenaLayout::Sgd) return ttp::Layout::Sgd;
        if (layout == ArenaLayout::Default) return ttp::Layout::Default;
        return mode == ttp::Mode::Mixed && !adam_declared ? ttp::Layout::Sgd
                                                          : ttp::Layout::Default;
    }

    ttp::Store& get() {
        if (!store) {
            store = std::make_unique<ttp::Store>(specs, mode, device, store_layout());
            for (uint32_t i = 0; i < specs.size(); ++i) {
                if (!init[i].empty()) store->set_weights(i, init[i]);
                if (grad_always[i]) store->set_has_grad(i, true);
            }
            init.clear();
            init.shrink_to_fit();
        }
        return *store;
    }
};

struct Value;
using ValuePtr = std::shared_ptr<Value>;

// `grad` of a parameter: empty (std::nullopt, py `None`) or a tensor in the store's grad
// buffer.  Same surface as std::optional<Tensor> for what the optimizers use.
class GradSlot {
public:
    GradSlot(std::shared_ptr<ArenaState> a, uint32_t i) : a_(std::move(a)), i_(i) {}
    bool has_value() const { return a_->get().has_grad(i_); }
    explicit operator bool() const { return has_value(); }
    std::vector<float> value() const {
        if (!has_value()) throw std::runtime_error("grad has no value");
        return a_->get().grad(i_);
    }
    GradSlot& operator=(std::nullopt_t) {
        a_->get().set_has_grad(i_, false);
        return *this;
    }
    GradSlot& operator=(const std::vector<float>& g) {
        a_->get().set_grad(i_, g);
        return *this;
    }

private:
    std::shared_ptr<ArenaState> a_;
    uint32_t i_;
};

struct Value {
    std::shared_ptr<ArenaState> arena;
    uint32_t index;
    GradSlot grad;
    bool requires_grad = true;
    std::string name;

    Value(std::shared_ptr<ArenaState> a, uint32_t i, std::string n)
        : arena(a), index(i), grad(a, i), name(std::move(n)) {}

    const std::vector<uint64_t>& shape() const { return arena->specs[index].shape; }
    uint64_t numel() const { return arena->specs[index].numel(); }
    ttp::Store& store() const { return arena->get(); }
    std::vector<float> data() const { return store().weights(index); }
    std::vector<float> master() const { return store().master(index); }
    void set_data(const std::vector<float>& w) { store().set_weights(index, w); }

    // autograd/dynamic/autograd.hpp:78-83: grad = grad + incoming, or the first assignment;
    // done on the GPU in the flat grad buffer (one launch, no host round trip of the grad)
    // sums: the same launch also stores this parameter's gradient sum of squares, so that an
    // optimizer with tensor_sums set needs no pass over the gradients after the backward
    void accumulate_grad(const std::vector<float>& incoming, bool sums = false) {
        if (!requires_grad) return;
        if (incoming.size() != numel()) throw std::invalid_argument("grad shape mismatch");
        store().accumulate_grad(index, incoming, sums);
    }
    // the same with a device-resident gradient (TTP_DTYPE_F32 or TTP_DTYPE_BF16)
    void accumulate_grad_device(const void* incoming, int dtype, bool sums = false) {
        if (!requires_grad) return;
        store().accumulate_grad_device(index, incoming, dtype, sums);
    }
    // device address of this parameter's gradient slice, for backward kernels that write it
    void* grad_ptr() { return store().device_ptr(TTP_BUF_GRAD, index); }
};

// A backward's bucket of parameter gradients (ttp_accumulate_grad_multi, at most
// TTP_ACCUM_MULTI_MAX per launch): params[k] receives incoming[k], device memory of one dtype
// for all, exactly as params[k]->accumulate_grad_device(incoming[k], dtype, sums) would.  The
// parameters belong to one arena; those without requires_grad are left out, as there.  A
// parameter listed twice and a null source of a non-empty parameter are refused before any
// launch, as the library refuses them within one call; a longer list is several calls, and
// one that the library refuses after another leaves the earlier calls' gradients in place.
inline void accumulate_grads_device(const std::vector<ValuePtr>& params,
                                    const std::vector<const void*>& incoming, int dtype,
                                    bool sums = false) {
    if (params.size() != incoming.size())
        throw std::invalid_argument("accumulate_grads_device: one source per parameter");
    if (params.empty()) return;
    std::vector<uint32_t> idx;
    std::vector<const void*> src;
    std::vector<bool> seen(params[0]->arena->specs.size(), false);
    for (size_t k = 0; k < params.size(); ++k) {
        if (params[k]->arena != params[0]->arena)
            throw std::invalid_argument("accumulate_grads_device: parameters of one arena");
        if (seen[params[k]->index])
            throw std::invalid_argument("accumulate_grads_device: a parameter listed twice");
        seen[params[k]->index] = true;
        if (!params[k]->requires_grad) continue;
        if (!incoming[k] && params[k]->numel())
            throw std::invalid_argument("accumulate_grads_device: a null source");
        idx.push_back(params[k]->index);
        src.push_back(incoming[k]);
    }
    ttp::Store& store = params[0]->store();
    for (size_t k = 0; k < idx.size(); k += TTP_ACCUM_MULTI_MAX) {
        const size_t e = std::min(idx.size(), k + TTP_ACCUM_MULTI_MAX);
        store.accumulate_grads_device(std::vector<uint32_t>(idx.begin() + k, idx.begin() + e),
                                      std::vector<const void*>(src.begin() + k, src.begin() + e),
                                      dtype, sums);
    }
}

// Declares parameters; all of them live in one store created on first use.
class ParamArena {
public:
    explicit ParamArena(ttp::Mode mode = ttp::Mode::FP32, int device = 0,
                        ArenaLayout layout = ArenaLayout::Auto)
        : s_(std::make_shared<ArenaState>()) {
        s_->mode = mode;
        s_->device = device;
        s_->layout = layout;
    }

    ValuePtr parameter(std::vector<uint64_t> shape, std::vector<float> init = {},
                       std::string name = "", bool decay = false, bool grad_always = false) {
        if (s_->store) throw std::logic_error("parameters must be declared before first use");
        ttp::TensorSpec spec{std::move(shape), decay, name};
        if (!init.empty() && init.size() != spec.numel())
            throw std::invalid_argument("initial value has the wrong size");
        const uint32_t idx = (uint32_t)s_->specs.size();
        s_->specs.push_back(spec);
        s_->init.push_back(std::move(init));
        s_->grad_always.push_back(grad_always);
        return std::make_shared<Value>(s_, idx, name);
    }

    ttp::Store& store() { return s_->get(); }
    const std::shared_ptr<ArenaState>& state() const { return s_; }
    size_t size() const { return s_->specs.size(); }

private:
    std::shared_ptr<ArenaState> s_;
};

inline std::vector<float> filled(uint64_t n, float v) { return std::vector<float>(n, v); }

}  // namespace autograd
