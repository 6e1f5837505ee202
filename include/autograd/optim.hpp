// optim.hpp — drop-in optimizers of the C++ autograd over libttperf_hip.
//
// autograd::SGD keeps the reference's shape exactly (autograd/dynamic/optim.hpp:13-35):
//   SGD sgd(model.parameters(), lr);  sgd.zero_grad();  ...  sgd.step();
// step() skips parameters without a grad and updates the others in place,
// `p = p - lr*g` rounded after the multiply and after the subtract as
// autograd/dynamic/optim.hpp:24-25 does — all parameters of one arena in one launch.
// Adam follows py/optim.py:30-92 (same defaults and validation); AdamW adds decoupled
// weight decay on the decay-flagged parameters.  Loss scaling and clipping are options.
//
// Every optimizer counts its own steps (py/optim.py:46,50), while the count the kernels read
// lives in the arena's store: when a different live optimizer stepped an arena last, its
// count is saved and this optimizer's restored (ttp::Store::claim_step_count: a synchronising
// read and a write, on a change of owner only; a graph hands the count back to the optimizer
// that held it at capture before each launch).  Copies of an optimizer share one count.
// With loss scaling on an arena stepped by several optimizers in one iteration, set
// opts.update_scale = false on every one but the last (or on all, then call the store's
// scaler_update()): the scale then moves once per iteration, from the overflow of all of
// them, as torch's GradScaler.step per optimizer followed by one GradScaler.update.
#pragma once

#include <algorithm>
#include <map>
#include <memory>
#include <stdexcept>
#include <utility>
#include <vector>

#include "autograd/value.hpp"

namespace autograd {

namespace detail {

// parameters grouped by arena: (state, indices, covers the whole arena)
struct Group {
    std::shared_ptr<ArenaState> arena;
    std::vector<uint32_t> indices;
    bool whole = false;
};

inline std::vector<Group> group(const std::vector<ValuePtr>& params) {
    std::map<ArenaState*, Group> m;
    std::vector<ArenaState*> order;
    for (const auto& p : params) {
        if (!p) throw std::invalid_argument("null parameter");
        auto it = m.find(p->arena.get());
        if (it == m.end()) {
            order.push_back(p->arena.get());
            it = m.emplace(p->arena.get(), Group{p->arena, {}, false}).first;
        }
        it->second.indices.push_back(p->index);
    }
    std::vector<Group> out;
    for (auto* a : order) {
        Group g = m[a];
        std::sort(g.indices.begin(), g.indices.end());
        g.indices.erase(std::unique(g.indices.begin(), g.indices.end()), g.indices.end());
        g.whole = g.indices.size() == g.arena->specs.size();
        out.push_back(std::move(g));
    }
    return out;
}

inline void zero_grad(const std::vector<ValuePtr>& params) {
    for (auto& g : group(params)) {
        if (g.whole) {
            g.arena->get().zero_grad(true);  // zeros + grad = nullopt for every parameter
        } else {
            for (uint32_t i : g.indices) g.arena->get().set_has_grad(i, false);
        }
    }
}

}  // namespace detail

struct SGD {
    std::vector<ValuePtr> params;
    float lr;
    ttp::SgdOptions opts;
    std::shared_ptr<ttp::StepCounts> counts = std::make_shared<ttp::StepCounts>();

    SGD(std::vector<ValuePtr> params_, float lr_, float momentum = 0.0f, float dampening = 0.0f,
        float weight_decay = 0.0f, bool nesterov = false)
        : params(std::move(params_)), lr(lr_) {
        if (!(lr_ > 0)) throw std::invalid_argument("lr must be > 0");
        opts.momentum = momentum;
        opts.dampening = dampening;
        opts.weight_decay = weight_decay;
        opts.nesterov = nesterov;
    }

    void step() {
        opts.lr = lr;
        for (auto& g : detail::group(params)) {
            g.arena->get().claim_step_count(counts);
            g.arena->get().sgd_step(opts, g.whole ? nullptr : &g.indices);
        }
    }

    void zero_grad() { detail::zero_grad(params); }
};

struct Adam {
    std::vector<ValuePtr> params;
    ttp::AdamOptions opts;
    std::shared_ptr<ttp::StepCounts> counts = std::make_shared<ttp::StepCounts>();

    explicit Adam(std::vector<ValuePtr> params_, float lr = 1e-3f,
                  std::pair<double, double> betas = {0.9, 0.999}, float eps = 1e-8f,
                  float weight_decay = 0.0f, double max_grad_norm = 0.0)
        : params(std::move(params_)) {
        // py/optim.py:33-41
        if (!(lr > 0)) throw std::invalid_argument("lr must be > 0");
        if (!(eps > 0)) throw std::invalid_argument("eps must be > 0");
        if (!(betas.first > 0 && betas.first < 1 && betas.second > 0 && betas.second < 1))
            throw std::invalid_argument("betas must be in (0, 1)");
        if (!(weight_decay >= 0)) throw std::invalid_argument("weight_decay must be >= 0");
        // an arena whose store does not exist yet is then created in Adam's layout; a Bf16
        // arena has no fp32 state for the moments
        for (const auto& p : params) {
            if (p && p->arena->mode == ttp::Mode::Bf16)
                throw std::invalid_argument("Adam needs fp32 moments: a Bf16 arena holds bf16 "
                                            "weights and gradients only; use a Mixed arena");
            if (p) p->arena->adam_declared = true;
        }
        opts.lr = lr;
        opts.beta1 = betas.first;
        opts.beta2 = betas.second;
        opts.eps = eps;
        opts.weight_decay = weight_decay;
        opts.decoupled = false;
        opts.max_grad_norm = max_grad_norm;
    }

    ttp_step_report step(bool want_report = false) {
        ttp_step_report last{};
        for (auto& g : detail::group(params)) {
            g.arena->get().claim_step_count(counts);
            last = g.arena->get().adam_step(opts, g.whole ? nullptr : &g.indices, want_report);
        }
        return last;
    }

    void zero_grad() { detail::zero_grad(params); }
};

struct AdamW : Adam {
    explicit AdamW(std::vector<ValuePtr> params_, float lr = 1e-3f,
                   std::pair<double, double> betas = {0.9, 0.999}, float eps = 1e-8f,
                   float weight_decay = 1e-2f, double max_grad_norm = 0.0)
        : Adam(std::move(params_), lr, betas, eps, weight_decay, max_grad_norm) {
        opts.decoupled = true;
    }
};

}  // namespace autograd
