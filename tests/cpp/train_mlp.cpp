// train_mlp.cpp — the training loop of the reference's examples/train_mlp.cpp:48-140 with
// the drop-in optimizer: SGD sgd(model.parameters(), lr); per iteration zero_grad, forward,
// MSE loss, backward, sgd.step().  Forward/backward are not part of this engine (TTNN ops in
// the reference); a small host implementation produces the gradients, which are written into
// the store's grad buffer, and the step runs on the GPU.  The loss must fall monotonically.
#include <algorithm>
#include <cmath>

#include "autograd/nn.hpp"
#include "autograd/optim.hpp"
#include "common.hpp"

using namespace autograd;

int main() {
    test::DeviceGuard dg;
    const uint32_t batch = 64, in = 32, hidden = 64, out = 8;
    const float lr = 1.0f;  // mean-reduced MSE on a small batch: 0.1 falls only ~5% in 30 steps
    const int iters = 30;
    ParamArena arena(ttp::Mode::Mixed);  // bf16 weights, fp32 master (the reference's bf16)
    MLP model(in, hidden, out, arena);
    SGD sgd(model.parameters(), lr);

    std::vector<float> x = uniform_init((uint64_t)batch * in, -1.0f, 1.0f, 11);
    std::vector<float> target = uniform_init((uint64_t)batch * out, -1.0f, 1.0f, 12);
    std::vector<float> losses;
    for (int it = 0; it < iters; ++it) {
        sgd.zero_grad();
        // forward on the model-facing (bf16) weights: h = relu(x W1^T + b1), y = h W2^T + b2
        const auto W1 = model.layer1.weight->data(), b1 = model.layer1.bias->data();
        const auto W2 = model.layer2.weight->data(), b2 = model.layer2.bias->data();
        std::vector<float> h((size_t)batch * hidden), y((size_t)batch * out);
        for (uint32_t n = 0; n < batch; ++n) {
            for (uint32_t j = 0; j < hidden; ++j) {
                float s = b1[j];
                for (uint32_t k = 0; k < in; ++k) s += x[n * in + k] * W1[j * in + k];
                h[n * hidden + j] = std::max(s, 0.0f);
            }
            for (uint32_t j = 0; j < out; ++j) {
                float s = b2[j];
                for (uint32_t k = 0; k < hidden; ++k) s += h[n * hidden + k] * W2[j * hidden + k];
                y[n * out + j] = s;
            }
        }
        // MSE loss = mean((y - t)^2) and its backward
        float loss = 0.0f;
        std::vector<float> dy(y.size());
        for (size_t i = 0; i < y.size(); ++i) {
            const float d = y[i] - target[i];
            loss += d * d;
            dy[i] = 2.0f * d / (float)y.size();
        }
        loss /= (float)y.size();
        losses.push_back(loss);
        std::vector<float> dW2((size_t)out * hidden, 0.0f), db2(out, 0.0f);
        std::vector<float> dW1((size_t)hidden * in, 0.0f), db1(hidden, 0.0f), dh(h.size(), 0.0f);
        for (uint32_t n = 0; n < batch; ++n)
            for (uint32_t j = 0; j < out; ++j) {
                const float d = dy[n * out + j];
                db2[j] += d;
                for (uint32_t k = 0; k < hidden; ++k) {
                    dW2[j * hidden + k] += d * h[n * hidden + k];
                    dh[n * hidden + k] += d * W2[j * hidden + k];
                }
            }
        for (uint32_t n = 0; n < batch; ++n)
            for (uint32_t j = 0; j < hidden; ++j) {
                const float d = h[n * hidden + j] > 0.0f ? dh[n * hidden + j] : 0.0f;
                db1[j] += d;
                for (uint32_t k = 0; k < in; ++k) dW1[j * in + k] += d * x[n * in + k];
            }
        model.layer1.weight->accumulate_grad(dW1);  // autograd/dynamic/autograd.hpp:78-83
        model.layer1.bias->accumulate_grad(db1);
        model.layer2.weight->accumulate_grad(dW2);
        model.layer2.bias->accumulate_grad(db2);
        sgd.step();
        std::printf("iter %2d  loss %.6f\n", it, loss);
    }
    for (int it = 1; it < iters; ++it)
        test::check(losses[it] < losses[it - 1], "loss decreases at iteration " + std::to_string(it));
    test::check(losses.back() < 0.8f * losses.front(), "loss falls by > 20% in 30 iterations");
    return test::finish("train_mlp");
}
