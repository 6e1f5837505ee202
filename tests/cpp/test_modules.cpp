// test_modules.cpp — module-level optimizer surfaces: the static layers' sgd_step / zero_grad
// (autograd/static/nn.hpp:92-101,178-186,213-221,242-250,332-345) and the traced transformer's
// layer / stack / GPT sgd_step (autograd/traced/transformer_train.hpp:259-268,335-339,487-494)
// and TracedMLP<N>::sgd_step (autograd/traced/mlp.hpp:106-110).
// Each sgd_step must update exactly its module's tensors, bit-exact against `w - lr*dw`
// (one rounding per op, bf16 weights = RNE of the fp32 master; in a Bf16 arena each op
// rounded to bf16), in ONE update launch.
#include "autograd/optim.hpp"
#include "autograd/static.hpp"
#include "autograd/traced.hpp"
#include "common.hpp"

using autograd::ParamArena;
using autograd::ValuePtr;

static std::vector<float> ramp(size_t n, float a, float b) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = a + b * (float)((i * 7) % 113) - 0.4f * b * 113.0f;
    return v;
}

struct Ref {
    std::vector<std::vector<float>> w, g;
};

static Ref snapshot(const std::vector<ValuePtr>& ps, bool mixed, float seed) {
    Ref r;
    for (size_t k = 0; k < ps.size(); ++k) {
        r.w.push_back(ps[k]->master());
        auto g = ramp(ps[k]->numel(), 0.01f * seed, 0.003f * (float)(k + 1));
        ps[k]->grad = g;  // rounded to bf16 by the store in Mixed mode
        if (mixed)
            for (auto& x : g) x = test::bf16_round(x);
        r.g.push_back(g);
    }
    return r;
}

static void apply(Ref& r, size_t k, float lr) {
    for (size_t i = 0; i < r.w[k].size(); ++i) {
        const float update = r.g[k][i] * lr;
        r.w[k][i] = r.w[k][i] - update;
    }
}

static void check_all(const std::vector<ValuePtr>& ps, const Ref& r, bool mixed,
                      const std::string& what) {
    for (size_t k = 0; k < ps.size(); ++k) {
        test::assert_bits(ps[k]->master(), r.w[k], what + " master " + std::to_string(k));
        if (mixed) {
            std::vector<float> want(r.w[k].size());
            for (size_t i = 0; i < want.size(); ++i) want[i] = test::bf16_round(r.w[k][i]);
            test::assert_bits(ps[k]->data(), want, what + " bf16 " + std::to_string(k));
        }
    }
}

static uint64_t update_launches(ttp::Store& s) {
    double ms = 0;
    uint64_t n = 0;
    ttp::check(ttp_timing_collect(s.get(), TTP_KERNEL_UPDATE, &ms, &n));
    return n;
}

int main() {
    test::DeviceGuard dg;
    // ---- static layers ----------------------------------------------------------------
    {
        ParamArena arena(ttp::Mode::FP32);
        static_autograd::MLP mlp(32, 64, 128, 10, 0.01f, arena);
        auto ps = mlp.parameters();
        Ref r = snapshot(ps, false, 1.0f);
        mlp.sgd_step(0.1f);
        for (size_t k = 0; k < 4; ++k) apply(r, k, 0.1f);
        check_all(ps, r, false, "static MLP sgd_step");
        mlp.layer2.sgd_step(0.2f);  // only layer 2
        apply(r, 2, 0.2f);
        apply(r, 3, 0.2f);
        check_all(ps, r, false, "static Linear sgd_step");
        mlp.zero_grad();  // zeros_like: grads present and zero
        for (auto& p : ps) {
            test::check(p->grad.has_value(), "static zero_grad keeps the grad");
            test::assert_all_close(p->grad.value(), 0.0f, 0.0f, "static zero_grad zeros");
        }
        mlp.sgd_step(0.1f);  // w - 0.1*0 = w
        check_all(ps, r, false, "static sgd_step after zero_grad");
    }
    // ---- static PersistentMLP (autograd/static/nn.hpp:257-345): the train_step's update ---
    {
        ParamArena arena(ttp::Mode::FP32);
        static_autograd::PersistentMLP pm(32, 64, 0.05f, arena);
        auto ps = pm.parameters();
        test::assert_all_close(pm.layer2.weight->data(), 0.01f, 0.0f, "PersistentMLP init 0.01");
        Ref r = snapshot(ps, false, 4.0f);
        ttp::Store& store = arena.store();
        ttp::check(ttp_timing_enable(store.get(), 1));
        update_launches(store);
        pm.sgd_step();
        test::check(update_launches(store) == 1, "PersistentMLP sgd_step is one update launch");
        ttp::check(ttp_timing_enable(store.get(), 0));
        for (size_t k = 0; k < 4; ++k) apply(r, k, 0.05f);
        check_all(ps, r, false, "PersistentMLP sgd_step");
    }
    // ---- traced transformer: GPT with 2 blocks ----------------------------------------
    {
        ParamArena arena(ttp::Mode::Mixed);
        traced::TracedTransformerWithEmbedding<2> gpt(4, 32, 64, 4, 4, 65, 0.05f, arena);
        auto ps = gpt.parameters();
        test::check(ps.size() == 2 + 2 * 16 + 2, "GPT parameter count 36");
        Ref r = snapshot(ps, true, 2.0f);
        ttp::Store& store = arena.store();
        test::check(store.layout() == ttp::Layout::Sgd,
                    "a Mixed arena no Adam was declared over takes the SGD layout");
        ttp::check(ttp_timing_enable(store.get(), 1));
        update_launches(store);
        gpt.sgd_step();
        test::check(update_launches(store) == 1, "GPT sgd_step is one update launch");
        for (size_t k = 0; k < ps.size(); ++k) apply(r, k, 0.05f);
        check_all(ps, r, true, "GPT sgd_step");
        // one block's sgd_step touches its 16 tensors only (offset 2: after the embeddings)
        gpt.layers[1].sgd_step();
        test::check(update_launches(store) == 1, "block sgd_step is one update launch");
        for (size_t k = 2 + 16; k < 2 + 32; ++k) apply(r, k, 0.05f);
        check_all(ps, r, true, "block sgd_step");
        ttp::check(ttp_timing_enable(store.get(), 0));
    }
    // ---- traced MLP<4> (autograd/traced/mlp.hpp:106-110) -------------------------------
    {
        ParamArena arena(ttp::Mode::Mixed);
        traced::TracedMLP<4> tm(8, 48, 0.03f, arena);
        auto ps = tm.parameters();
        test::check(ps.size() == 8, "TracedMLP<4> parameter count 8");
        Ref r = snapshot(ps, true, 5.0f);
        ttp::Store& store = arena.store();
        ttp::check(ttp_timing_enable(store.get(), 1));
        update_launches(store);
        tm.sgd_step();
        test::check(update_launches(store) == 1, "TracedMLP sgd_step is one update launch");
        ttp::check(ttp_timing_enable(store.get(), 0));
        for (size_t k = 0; k < ps.size(); ++k) apply(r, k, 0.03f);
        check_all(ps, r, true, "TracedMLP sgd_step");
    }
    // ---- traced stack -----------------------------------------------------------------
    {
        ParamArena arena(ttp::Mode::FP32);
        traced::TracedTransformerStack<3> stack(2, 16, 32, 2, 4, 0.2f, arena);
        auto ps = stack.parameters();
        test::check(ps.size() == 3 * 16, "stack parameter count 48");
        Ref r = snapshot(ps, false, 3.0f);
        stack.sgd_step();
        for (size_t k = 0; k < ps.size(); ++k) apply(r, k, 0.2f);
        check_all(ps, r, false, "stack sgd_step");
    }
    // ---- the same GPT on the reference's own storage (a Bf16 arena: bf16 weights and
    // gradients, no master): each sgd_step is RNE(w - RNE(g*lr)) over its module's tensors,
    // the rounding of the reference's ttnn multiply and subtract, in one update launch ------
    {
        ParamArena arena(ttp::Mode::Bf16);
        traced::TracedTransformerWithEmbedding<2> gpt(4, 32, 64, 4, 4, 65, 0.05f, arena);
        auto ps = gpt.parameters();
        std::vector<std::vector<float>> w, g;
        for (size_t k = 0; k < ps.size(); ++k) {
            w.push_back(ps[k]->data());
            auto gk = ramp(ps[k]->numel(), 0.02f, 0.003f * (float)(k + 1));
            ps[k]->grad = gk;  // rounded to bf16 by the store
            for (auto& x : gk) x = test::bf16_round(x);
            g.push_back(gk);
        }
        auto step = [&](size_t k, float lr) {
            for (size_t i = 0; i < w[k].size(); ++i)
                w[k][i] = test::bf16_round(w[k][i] - test::bf16_round(g[k][i] * lr));
        };
        auto check = [&](const std::string& what) {
            for (size_t k = 0; k < ps.size(); ++k)
                test::assert_bits(ps[k]->data(), w[k], what + " " + std::to_string(k));
        };
        ttp::Store& store = arena.store();
        ttp::check(ttp_timing_enable(store.get(), 1));
        update_launches(store);
        gpt.sgd_step();
        test::check(update_launches(store) == 1, "bf16 GPT sgd_step is one update launch");
        for (size_t k = 0; k < ps.size(); ++k) step(k, 0.05f);
        check("bf16 GPT sgd_step");
        gpt.layers[0].sgd_step();  // block 0's 16 tensors only (after the 2 embeddings)
        test::check(update_launches(store) == 1, "bf16 block sgd_step is one update launch");
        for (size_t k = 2; k < 2 + 16; ++k) step(k, 0.05f);
        check("bf16 block sgd_step");
        ttp::check(ttp_timing_enable(store.get(), 0));
    }
    // ---- arena layouts: an Adam declared before first use gets Adam's layout; one declared
    // after converts the SGD layout at its first step, from the values SGD left ----------
    {
        ParamArena a(ttp::Mode::Mixed);
        auto w = a.parameter({300}, ramp(300, 0.1f, 0.001f), "w", true);
        autograd::AdamW opt({w}, 1e-3f);
        test::check(a.store().layout() == ttp::Layout::Default,
                    "an Adam declared before first use: the default layout");
        ParamArena b(ttp::Mode::Mixed);
        auto v = b.parameter({300}, ramp(300, 0.1f, 0.001f), "v", true);
        v->grad = ramp(300, 0.02f, 0.0005f);
        autograd::SGD sgd({v}, 0.1f);
        sgd.step();
        test::check(b.store().layout() == ttp::Layout::Sgd, "SGD alone: the SGD layout");
        const std::vector<float> before = v->master();
        autograd::AdamW late({v}, 1e-3f, {0.9, 0.95}, 1e-8f, 0.0f);
        late.step();
        test::check(b.store().layout() == ttp::Layout::Default,
                    "a later Adam step converts the store");
        // AdamW's first step with wd 0 moves each weight by lr * sign(g) (m_hat / sqrt(v_hat)
        // is g / |g| up to eps): check that it started from the SGD-updated master
        const std::vector<float> after = v->master(), g = v->grad.value();
        size_t bad = 0;
        for (size_t i = 0; i < after.size(); ++i) {
            const float moved = before[i] - after[i];
            const float want = g[i] > 0 ? 1e-3f : (g[i] < 0 ? -1e-3f : 0.0f);
            bad += std::fabs(moved - want) > 1e-6f;
        }
        test::check(bad == 0, "the converted store's first Adam step starts from SGD's master");
    }
    return test::finish("test_modules");
}
