// nn.hpp — parameter-holding layers of the drop-in API (the optimizer-facing part only).
//
// Linear and MLP have the parameter layout and parameters() order of the reference's
// dynamic layers (autograd/dynamic/nn.hpp:13-56): weight [out, in] ~ U(-0.1, 0.1), bias
// [1, out] zeros.  The "device" argument is the ParamArena their tensors are declared on.
// Forward/backward compute is not part of this engine: gradients come from the caller
// (Value::grad / accumulate_grad, or written straight into the store's grad buffer).
#pragma once

#include <cstdint>
#include <vector>

#include "autograd/value.hpp"

namespace autograd {

// deterministic U(lo, hi) fill (64-bit LCG), so examples and tests are reproducible
inline std::vector<float> uniform_init(uint64_t n, float lo, float hi, uint64_t seed) {
    std::vector<float> v(n);
    uint64_t x = seed * 6364136223846793005ull + 1442695040888963407ull;
    for (uint64_t i = 0; i < n; ++i) {
        x = x * 6364136223846793005ull + 1442695040888963407ull;
        const double u = (double)(x >> 11) * (1.0 / 9007199254740992.0);
        v[i] = (float)(lo + (hi - lo) * u);
    }
    return v;
}

struct Linear {
    ValuePtr weight;  // [out_features, in_features]
    ValuePtr bias;    // [1, out_features]

    Linear(uint32_t in_features, uint32_t out_features, ParamArena& arena, uint64_t seed = 1)
        : weight(arena.parameter({out_features, in_features},
                                 uniform_init((uint64_t)out_features * in_features, -0.1f, 0.1f, seed),
                                 "weight", /*decay=*/true)),
          bias(arena.parameter({1, out_features}, filled(out_features, 0.0f), "bias", false)) {}

    std::vector<ValuePtr> parameters() { return {weight, bias}; }
};

struct MLP {
    Linear layer1;
    Linear layer2;

    MLP(uint32_t in_dim, uint32_t hidden_dim, uint32_t out_dim, ParamArena& arena)
        : layer1(in_dim, hidden_dim, arena, 1), layer2(hidden_dim, out_dim, arena, 2) {}

    std::vector<ValuePtr> parameters() {
        return {layer1.weight, layer1.bias, layer2.weight, layer2.bias};
    }
};

}  // namespace autograd
