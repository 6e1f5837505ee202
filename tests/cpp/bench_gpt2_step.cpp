// bench_gpt2_step.cpp — the optimizer step of the reference's full-GPT benchmark model,
// timed through the drop-in C++ surface.
//
// The reference's bench/autograd/bench_gpt2_full.cpp:74-100 builds
// traced::TracedTransformerWithEmbedding<N> from BENCH_* environment variables
// (:103-121), runs warmup iterations, then times N_ITERS train steps between two device
// synchronisations with std::chrono.  This program builds the same model class over a
// mixed-precision ParamArena (bf16 weights and gradients, fp32 master) at GPT-2 small
// dimensions by default and times, the same way, the two optimizer surfaces a training loop
// calls on it, each on a model of its own:
//   - autograd::AdamW over model.parameters(), with dynamic loss scaling (2^16, growth 2x
//     every 2000 clean steps, backoff 0.5) and a global grad-norm clip at 1.0; the AdamW is
//     declared before the store exists, so the arena lays out master, m and v in records;
//   - the model's own sgd_step() (autograd/traced/transformer_train.hpp:487-494) on a model
//     whose arena only SGD steps, which therefore takes the SGD layout (contiguous master,
//     no m and v).
// The forward and backward passes are not part of this engine; the gradients are written
// once from the host, scaled by the loss scale.  Before the timed steps each surface runs
// back to back for BENCH_SETTLE_MS (200 by default): the GPU leaves its idle clocks during
// the first tens of milliseconds of work.
//
// Checks, after the timed steps: the step count and the scaler state follow the steps run;
// every bf16 weight is the round-to-nearest-even of its fp32 master; a gradient holding
// +inf makes the next step a skipped one (weights and count unchanged, scale halved); one
// sgd_step moves a tensor by exactly w - lr*g.  Prints one JSON line, then
// "bench_gpt2_step: PASS".
#include <chrono>
#include <cmath>
#include <limits>
#include <string>

#include "autograd/optim.hpp"
#include "autograd/traced.hpp"
#include "common.hpp"

using autograd::ParamArena;
using autograd::ValuePtr;
using clk = std::chrono::steady_clock;

namespace {

uint32_t env_u32(const char* name, uint32_t dflt) {
    const char* e = std::getenv(name);
    return e ? (uint32_t)std::stoul(e) : dflt;
}

// uniform values with standard deviation `sd` (xorshift32 per tensor, seeded by its index)
std::vector<float> grad_values(uint64_t n, float sd, uint32_t seed) {
    std::vector<float> g(n);
    uint32_t s = 0x9E3779B9u ^ (seed * 2654435761u);
    const float a = sd * std::sqrt(3.0f) / 2147483648.0f;
    for (uint64_t i = 0; i < n; ++i) {
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        g[i] = a * (float)((int64_t)s - 2147483648LL);
    }
    return g;
}

double ms_since(clk::time_point t0) {
    return std::chrono::duration<double, std::milli>(clk::now() - t0).count();
}

struct Timing {
    double ms_per_step = 0;
    int settle_steps = 0;
};

// settle (untimed, back to back, in batches of 20), warmup, then `iters` timed steps between
// two synchronisations (bench_gpt2_full.cpp:85-99)
template <class Step>
Timing time_steps(ttp::Store& s, Step step, uint32_t settle_ms, uint32_t warmup, uint32_t iters,
                  uint64_t* steps_run) {
    Timing t;
    s.sync();
    const auto t0 = clk::now();
    while (settle_ms && ms_since(t0) < settle_ms) {
        for (int k = 0; k < 20; ++k) step();
        s.sync();
        t.settle_steps += 20;
    }
    for (uint32_t k = 0; k < warmup; ++k) step();
    s.sync();
    const auto t1 = clk::now();
    for (uint32_t k = 0; k < iters; ++k) step();
    s.sync();
    t.ms_per_step = ms_since(t1) / iters;
    *steps_run += (uint64_t)t.settle_steps + warmup + iters;
    return t;
}

template <size_t N>
int run(uint32_t seq, uint32_t dim, uint32_t heads, uint32_t ffn, uint32_t vocab) {
    const uint32_t settle_ms = env_u32("BENCH_SETTLE_MS", 200);
    const uint32_t warmup = env_u32("BENCH_WARMUP", 5), iters = env_u32("BENCH_ITERS", 50);
    const float sgd_lr = 0.01f;  // bench_gpt2_full.cpp:110
    const double init_scale = 65536.0;

    ParamArena arena(ttp::Mode::Mixed);
    traced::TracedTransformerWithEmbedding<N> model(/*batch=*/8, seq, dim, heads, ffn, vocab,
                                                    sgd_lr, arena);
    const std::vector<ValuePtr> params = model.parameters();
    uint64_t numel = 0;
    for (auto& p : params) numel += p->numel();
    // 1) AdamW (config of the GPT-2 runs: lr 6e-4, betas (0.9, 0.95), wd 0.1, clip 1.0),
    // declared before the store exists: Adam's layout
    autograd::AdamW opt(params, 6e-4f, {0.9, 0.95}, 1e-8f, 0.1f, 1.0);
    ttp::Store& store = arena.store();
    test::check(store.layout() == ttp::Layout::Default, "AdamW's arena: the default layout");
    store.configure_scaler(init_scale, 2.0, 0.5, 2000, true);
    for (size_t k = 0; k < params.size(); ++k)
        params[k]->grad = grad_values(params[k]->numel(), 1e-3f * (float)init_scale, (uint32_t)k);
    std::printf("# GPT model (TracedTransformerWithEmbedding<%zu>): seq=%u dim=%u heads=%u "
                "ffn_mult=%u vocab=%u; %zu tensors, %llu params, mixed precision\n",
                N, seq, dim, heads, ffn, vocab, params.size(), (unsigned long long)numel);

    uint64_t adam_steps = 0;
    const Timing ta = time_steps(store, [&] { opt.step(); }, settle_ms, warmup, iters, &adam_steps);
    const double adam_gps = (double)numel / (ta.ms_per_step * 1e-3) / 1e9;
    std::printf("AdamW step: %.4f ms/step, %.1f Gparams/s (%.0f GB/s at 30 B/param)\n",
                ta.ms_per_step, adam_gps, adam_gps * 30.0);

    test::check(store.step_count() == adam_steps, "step count after the AdamW steps");
    const uint64_t growths = adam_steps / 2000;
    const auto [scale, tracker] = store.scaler_state();
    test::check(scale == (float)(init_scale * std::ldexp(1.0, (int)growths)) &&
                    tracker == (int32_t)(adam_steps % 2000),
                "scaler state after " + std::to_string(adam_steps) + " clean steps");
    for (size_t k = 0; k < params.size(); ++k) {
        const std::vector<float> m = params[k]->master(), w = params[k]->data();
        std::vector<float> want(m.size());
        for (size_t i = 0; i < m.size(); ++i) want[i] = test::bf16_round(m[i]);
        test::assert_bits(w, want, "bf16 weight = RNE(master), tensor " + std::to_string(k));
    }

    // 2) an overflow step through the drop-in optimizer: skipped, scale backs off
    const ValuePtr& probe = model.layers[0].ln1.beta;
    std::vector<float> g_inf = grad_values(probe->numel(), 1e-3f * scale, 7);
    const std::vector<float> g_keep = g_inf;
    g_inf[g_inf.size() / 2] = std::numeric_limits<float>::infinity();
    probe->grad = g_inf;
    const std::vector<float> before = probe->master(), before_wte = model.tok_emb.weight->master();
    opt.step();
    const auto [scale2, tracker2] = store.scaler_state();
    test::check(store.step_count() == adam_steps, "an overflow step leaves the step count");
    test::check(scale2 == scale * 0.5f && tracker2 == 0, "an overflow step halves the scale");
    test::assert_bits(probe->master(), before, "an overflow step leaves the weights");
    test::assert_bits(model.tok_emb.weight->master(), before_wte,
                      "an overflow step leaves the embedding");
    probe->grad = g_keep;

    // 3) sgd_step (w - lr*g per tensor, no loss scale) on a second model whose arena only SGD
    // steps: timed, then one exact check
    ParamArena sgd_arena(ttp::Mode::Mixed);
    traced::TracedTransformerWithEmbedding<N> sgd_model(/*batch=*/8, seq, dim, heads, ffn, vocab,
                                                        sgd_lr, sgd_arena);
    const std::vector<ValuePtr> sgd_params = sgd_model.parameters();
    ttp::Store& sgd_store = sgd_arena.store();
    test::check(sgd_store.layout() == ttp::Layout::Sgd, "sgd_step's arena: the SGD layout");
    for (size_t k = 0; k < sgd_params.size(); ++k)
        sgd_params[k]->grad = grad_values(sgd_params[k]->numel(), 1e-3f, (uint32_t)k);
    uint64_t sgd_steps = 0;
    const Timing ts = time_steps(sgd_store, [&] { sgd_model.sgd_step(); }, settle_ms, warmup,
                                 iters, &sgd_steps);
    const double sgd_gps = (double)numel / (ts.ms_per_step * 1e-3) / 1e9;
    std::printf("sgd_step: %.4f ms/step, %.1f Gparams/s (%.0f GB/s at 12 B/param)\n",
                ts.ms_per_step, sgd_gps, sgd_gps * 12.0);
    {
        const ValuePtr& sp = sgd_model.layers[0].ln1.beta;
        const std::vector<float> w0 = sp->master(), g = sp->grad.value();
        sgd_model.sgd_step();
        std::vector<float> want(w0.size());
        for (size_t i = 0; i < w0.size(); ++i) {
            const float update = g[i] * sgd_lr;
            want[i] = w0[i] - update;
        }
        test::assert_bits(sp->master(), want, "sgd_step = w - lr*g");
    }

    // 4) the same sgd_step on the reference's own storage (a Bf16 arena: bf16 weights and
    // gradients, no master; each op rounded to bf16 as the reference's ttnn ops round theirs)
    ParamArena bf16_arena(ttp::Mode::Bf16);
    traced::TracedTransformerWithEmbedding<N> bf16_model(/*batch=*/8, seq, dim, heads, ffn, vocab,
                                                         sgd_lr, bf16_arena);
    const std::vector<ValuePtr> bf16_params = bf16_model.parameters();
    ttp::Store& bf16_store = bf16_arena.store();
    for (size_t k = 0; k < bf16_params.size(); ++k)
        bf16_params[k]->grad = grad_values(bf16_params[k]->numel(), 1e-3f, (uint32_t)k);
    uint64_t bf16_steps = 0;
    const Timing tb = time_steps(bf16_store, [&] { bf16_model.sgd_step(); }, settle_ms, warmup,
                                 iters, &bf16_steps);
    const double bf16_gps = (double)numel / (tb.ms_per_step * 1e-3) / 1e9;
    std::printf("sgd_step on bf16 storage: %.4f ms/step, %.1f Gparams/s (%.0f GB/s at 6 B/param)\n",
                tb.ms_per_step, bf16_gps, bf16_gps * 6.0);
    {
        const ValuePtr& sp = bf16_model.layers[0].ln1.beta;
        const std::vector<float> w0 = sp->data(), g = sp->grad.value();
        bf16_model.sgd_step();
        std::vector<float> want(w0.size());
        for (size_t i = 0; i < w0.size(); ++i)
            want[i] = test::bf16_round(w0[i] - test::bf16_round(g[i] * sgd_lr));
        test::assert_bits(sp->data(), want, "bf16 sgd_step = RNE(w - RNE(g*lr))");
    }

    std::printf("{\"bench\": \"gpt2_step_dropin\", \"layers\": %zu, \"tensors\": %zu, "
                "\"params\": %llu, \"adamw_ms_per_step\": %.5f, \"adamw_Gparams_per_s\": %.2f, "
                "\"adamw_settle_steps\": %d, \"sgd_ms_per_step\": %.5f, "
                "\"sgd_Gparams_per_s\": %.2f, \"sgd_settle_steps\": %d, \"sgd_layout\": \"sgd\", "
                "\"sgd_bf16_ms_per_step\": %.5f, \"sgd_bf16_Gparams_per_s\": %.2f, "
                "\"sgd_bf16_settle_steps\": %d, \"warmup\": %u, "
                "\"iters\": %u}\n",
                N, params.size(), (unsigned long long)numel, ta.ms_per_step, adam_gps,
                ta.settle_steps, ts.ms_per_step, sgd_gps, ts.settle_steps, tb.ms_per_step,
                bf16_gps, tb.settle_steps, warmup, iters);
    return test::finish("bench_gpt2_step");
}

}  // namespace

int main() {
    test::DeviceGuard dg;
    try {
        // GPT-2 small by default; the reference's bench defaults are the nano_gpt shapes
        const uint32_t seq = env_u32("BENCH_SEQ", 1024), dim = env_u32("BENCH_DIM", 768);
        const uint32_t heads = env_u32("BENCH_HEADS", 12), ffn = env_u32("BENCH_FFN_MULT", 4);
        const uint32_t vocab = env_u32("BENCH_VOCAB", 50257);
        const uint32_t layers = env_u32("BENCH_LAYERS", 12);
        if (!heads || dim % heads != 0) {
            std::printf("ERROR: dim (%u) must be divisible by heads (%u)\n", dim, heads);
            return 1;
        }
        if (!seq || !dim || !ffn || !vocab || !env_u32("BENCH_ITERS", 50)) {
            std::printf("ERROR: BENCH_SEQ, BENCH_DIM, BENCH_FFN_MULT, BENCH_VOCAB and "
                        "BENCH_ITERS must be positive\n");
            return 1;
        }
        switch (layers) {
            case 1: return run<1>(seq, dim, heads, ffn, vocab);
            case 2: return run<2>(seq, dim, heads, ffn, vocab);
            case 3: return run<3>(seq, dim, heads, ffn, vocab);
            case 6: return run<6>(seq, dim, heads, ffn, vocab);
            case 12: return run<12>(seq, dim, heads, ffn, vocab);
            default:
                std::printf("ERROR: supported layer counts: 1, 2, 3, 6, 12\n");
                return 1;
        }
    } catch (const std::exception& e) {
        std::printf("FAILED: %s\n", e.what());
        return 1;
    }
}
