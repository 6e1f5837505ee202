// test_sgd.cpp — autograd::SGD with a Linear layer: the known answers of the reference's
// autograd/tests/test_sgd.cpp:14-73 (bias grad 32 from a batch of ones; lr 0.01 gives
// bias -0.32, a second step -0.64), here checked bit-for-bit in bf16 params (Mixed), fp32
// params (FP32) and the reference's bf16-only storage (Bf16).  The gradients are the ones the reference's backward produces for
// y = x W^T + b with x = ones[32, 64] and dY = ones: dW = 32 everywhere, db = 32.
#include <cassert>

#include "autograd/nn.hpp"
#include "autograd/optim.hpp"
#include "common.hpp"

using namespace autograd;

static void run(ttp::Mode mode) {
    const bool mixed = mode == ttp::Mode::Mixed;
    const std::string tag = mixed ? "mixed" : "fp32";
    ParamArena arena(mode);
    Linear linear(64, 32, arena);

    SGD sgd(linear.parameters(), 0.01f);
    sgd.zero_grad();  // grad = nullopt, no tensor work
    test::check(!linear.weight->grad.has_value(), tag + ": weight grad cleared");
    test::check(!linear.bias->grad.has_value(), tag + ": bias grad cleared");

    std::vector<float> master = linear.weight->master();  // fp32 master (== data in FP32)
    const std::vector<float> w_before = linear.weight->data();
    test::check(w_before[0] == (mixed ? test::bf16_round(master[0]) : master[0]),
                tag + ": bf16 param is RNE of the master");

    for (int it = 1; it <= 2; ++it) {
        if (it == 2) sgd.zero_grad();
        // "backward": dW = dY^T x = 32, db = sum over the batch of dY = 32
        linear.weight->grad = std::vector<float>(64 * 32, 32.0f);
        linear.bias->grad = std::vector<float>(32, 32.0f);
        test::check(linear.weight->grad.has_value() && linear.bias->grad.has_value(),
                    tag + ": grads exist after backward");
        test::assert_all_close(linear.bias->grad.value(), 32.0f, 0.0f, tag + ": dBias = 32");

        sgd.step();

        // autograd/dynamic/optim.hpp:24-25: update = grad*lr (rounded), data - update (rounded)
        const float update = 32.0f * 0.01f;
        for (auto& m : master) m = m - update;
        test::assert_bits(linear.weight->master(), master, tag + ": weight master");
        std::vector<float> want_w(master.size());
        for (size_t i = 0; i < master.size(); ++i)
            want_w[i] = mixed ? test::bf16_round(master[i]) : master[i];
        test::assert_bits(linear.weight->data(), want_w, tag + ": weight data");

        // bias: 0 - 0.32 = -0.32, then -0.64 (reference tolerance 0.1; here exact)
        float b = 0.0f;
        for (int k = 0; k < it; ++k) b = b - update;
        const float want_b = mixed ? test::bf16_round(b) : b;
        test::assert_bits(linear.bias->data(), std::vector<float>(32, want_b),
                          tag + ": bias after step " + std::to_string(it));
        test::assert_all_close(linear.bias->data(), it == 1 ? -0.32f : -0.64f, 0.1f,
                               tag + ": reference known answer, step " + std::to_string(it));
    }
    std::printf("%s: w[0] %.6f -> %.6f, bias %.6f\n", tag.c_str(), w_before[0],
                linear.weight->data()[0], linear.bias->data()[0]);

    // a parameter whose grad is nullopt is skipped (autograd/dynamic/optim.hpp:23)
    sgd.zero_grad();
    linear.bias->grad = std::vector<float>(32, 1.0f);
    const std::vector<float> w_keep = linear.weight->master();
    sgd.step();
    test::assert_bits(linear.weight->master(), w_keep, tag + ": weight without grad untouched");
}

// The reference's own storage (Bf16 mode: bf16 weights and gradients, no master): each step is
// update = RNE_bf16(32 * 0.01f) = 0.3203125, data = RNE_bf16(data - update), the rounding of
// each ttnn op's bf16 result in autograd/dynamic/optim.hpp:24-25.
static void run_bf16() {
    const std::string tag = "bf16";
    ParamArena arena(ttp::Mode::Bf16);
    Linear linear(64, 32, arena);
    SGD sgd(linear.parameters(), 0.01f);
    sgd.zero_grad();
    std::vector<float> w = linear.weight->data();  // the bf16 weights, widened
    const float update = test::bf16_round(32.0f * 0.01f);
    test::check(update == 0.3203125f, tag + ": the update rounds to 0.3203125");
    for (int it = 1; it <= 2; ++it) {
        if (it == 2) sgd.zero_grad();
        linear.weight->grad = std::vector<float>(64 * 32, 32.0f);
        linear.bias->grad = std::vector<float>(32, 32.0f);
        sgd.step();
        for (auto& x : w) x = test::bf16_round(x - update);
        test::assert_bits(linear.weight->data(), w, tag + ": weight data");
        const float want_b = it == 1 ? -0.3203125f : -0.640625f;
        test::assert_bits(linear.bias->data(), std::vector<float>(32, want_b),
                          tag + ": bias after step " + std::to_string(it));
        test::assert_all_close(linear.bias->data(), it == 1 ? -0.32f : -0.64f, 0.1f,
                               tag + ": reference known answer, step " + std::to_string(it));
    }
    std::printf("%s: bias %.7f\n", tag.c_str(), linear.bias->data()[0]);
    // a parameter whose grad is nullopt is skipped
    sgd.zero_grad();
    linear.bias->grad = std::vector<float>(32, 1.0f);
    const std::vector<float> w_keep = linear.weight->data();
    sgd.step();
    test::assert_bits(linear.weight->data(), w_keep, tag + ": weight without grad untouched");
    // no fp32 state: SGD with momentum and Adam are refused, nothing changed
    bool threw = false;
    try {
        SGD mom(linear.parameters(), 0.01f, 0.9f);
        linear.weight->grad = std::vector<float>(64 * 32, 1.0f);
        mom.step();
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    test::check(threw, tag + ": SGD with momentum throws std::invalid_argument");
    threw = false;
    try {
        AdamW adam(linear.parameters(), 1e-3f);
        adam.step();
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    test::check(threw, tag + ": AdamW throws std::invalid_argument");
    test::assert_bits(linear.weight->data(), w_keep, tag + ": refused steps change nothing");
}

int main() {
    test::DeviceGuard dg;
    run(ttp::Mode::Mixed);
    run(ttp::Mode::FP32);
    run_bf16();
    // the reference raises nothing for lr <= 0 in C++; this engine rejects it like py/optim.py:9-10
    ParamArena arena;
    Linear l(4, 4, arena);
    bool threw = false;
    try {
        SGD bad(l.parameters(), 0.0f);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    test::check(threw, "SGD(lr = 0) throws std::invalid_argument");
    return test::finish("test_sgd");
}
