// test_adam.cpp — autograd::Adam / AdamW over the flat store.  Adam follows py/optim.py:30-92
// (defaults lr 1e-3, betas (0.9, 0.999), eps 1e-8; t += 1 then bias corrections in host
// double, rounded to fp32 like full_like(fill_value=...)); the expected values below apply
// the same op order on the host with one rounding per op.  AdamW decays only the
// decay-flagged (2-D weight) tensors: p *= (float)(1 - lr*wd) before the Adam update.
#include <algorithm>
#include <cmath>

#include "autograd/nn.hpp"
#include "autograd/optim.hpp"
#include "common.hpp"

using namespace autograd;

struct Ref {
    std::vector<float> p, m, v;
};

static void adam_ref(Ref& r, const std::vector<float>& g, double lr, double b1, double b2,
                     double eps, uint64_t t, double wd, bool decay) {
    const float flr = (float)lr, fb1 = (float)b1, fb2 = (float)b2, fomb1 = (float)(1.0 - b1),
                fomb2 = (float)(1.0 - b2), feps = (float)eps;
    const float bias1 = (float)(1.0 - std::pow(b1, (double)t));
    const float bias2 = (float)(1.0 - std::pow(b2, (double)t));
    const float dmul = (float)(1.0 - lr * wd);
    for (size_t i = 0; i < g.size(); ++i) {
        float p = r.p[i];
        if (decay && wd != 0.0) p = p * dmul;
        const float m = fb1 * r.m[i] + fomb1 * g[i];
        const float gsq = g[i] * g[i];
        const float v = fb2 * r.v[i] + fomb2 * gsq;
        const float mh = m / bias1, vh = v / bias2;
        const float den = std::sqrt(vh) + feps;
        const float step = flr * (mh / den);
        r.p[i] = p - step;
        r.m[i] = m;
        r.v[i] = v;
    }
}

static std::vector<float> grad_of(size_t n, int seed) {
    std::vector<float> g(n);
    uint32_t x = 2463534242u + (uint32_t)seed * 7919u;
    for (size_t i = 0; i < n; ++i) {
        x ^= x << 13;
        x ^= x >> 17;
        x ^= x << 5;
        g[i] = ((float)(x & 0xFFFFFF) / 16777216.0f - 0.5f) * 0.02f;
    }
    return g;
}

static void run(bool decoupled) {
    const std::string tag = decoupled ? "AdamW" : "Adam";
    ParamArena arena(ttp::Mode::FP32);
    MLP model(64, 128, 10, arena);  // W1, b1, W2, b2 (decay on the weights)
    auto params = model.parameters();
    std::vector<Ref> ref;
    for (auto& p : params) {
        Ref r;
        r.p = p->master();
        r.m.assign(p->numel(), 0.0f);
        r.v.assign(p->numel(), 0.0f);
        ref.push_back(r);
    }
    const double lr = 1e-2, wd = decoupled ? 0.1 : 0.0;
    Adam* opt = decoupled ? new AdamW(params, (float)lr, {0.9, 0.95}, 1e-8f, (float)wd)
                          : new Adam(params, (float)lr, {0.9, 0.95}, 1e-8f);
    const double flr = (double)(float)lr, fwd = (double)(float)wd;
    for (uint64_t t = 1; t <= 5; ++t) {
        opt->zero_grad();
        for (size_t k = 0; k < params.size(); ++k) {
            auto g = grad_of(params[k]->numel(), (int)(t * 10 + k));
            params[k]->grad = g;
            adam_ref(ref[k], g, flr, 0.9, 0.95, (double)1e-8f, t, fwd, k % 2 == 0);
        }
        opt->step();
    }
    for (size_t k = 0; k < params.size(); ++k) {
        test::assert_bits(params[k]->master(), ref[k].p, tag + " param " + std::to_string(k));
        test::assert_bits(params[k]->store().state(TTP_BUF_EXP_AVG, params[k]->index), ref[k].m,
                          tag + " exp_avg " + std::to_string(k));
        test::assert_bits(params[k]->store().state(TTP_BUF_EXP_AVG_SQ, params[k]->index),
                          ref[k].v, tag + " exp_avg_sq " + std::to_string(k));
    }
    test::check(params[0]->store().step_count() == 5, tag + ": step count 5");
    delete opt;
}

// Two optimizers over two parameter groups of one arena, stepped in an uneven order: each
// group's bias corrections use its own optimizer's step count (py/optim.py:46,50 keeps `_step`
// per optimizer), and the arena's count reads as the last stepper's.
static void run_groups() {
    ParamArena arena(ttp::Mode::FP32);
    MLP model(64, 128, 10, arena);
    auto params = model.parameters();
    std::vector<Ref> ref;
    for (auto& p : params) {
        Ref r;
        r.p = p->master();
        r.m.assign(p->numel(), 0.0f);
        r.v.assign(p->numel(), 0.0f);
        ref.push_back(r);
    }
    const std::vector<size_t> ga = {0, 1}, gb = {2, 3};
    AdamW a({params[0], params[1]}, 1e-2f, {0.9, 0.95}, 1e-8f, 0.1f);
    Adam b({params[2], params[3]}, 3e-3f, {0.8, 0.999}, 1e-6f);
    uint64_t ta = 0, tb = 0;
    const char* order = "abbaab";
    for (int k = 0; order[k]; ++k) {
        const bool is_a = order[k] == 'a';
        const auto& members = is_a ? ga : gb;
        const uint64_t t = is_a ? ++ta : ++tb;
        for (size_t j : members) {
            auto g = grad_of(params[j]->numel(), 100 + k * 10 + (int)j);
            params[j]->grad = g;
            if (is_a)
                adam_ref(ref[j], g, (double)1e-2f, 0.9, 0.95, (double)1e-8f, t, (double)0.1f,
                         j == 0);
            else
                adam_ref(ref[j], g, (double)3e-3f, 0.8, 0.999, (double)1e-6f, t, 0.0, false);
        }
        if (is_a) a.step(); else b.step();
        test::check(params[0]->store().step_count() == t,
                    "groups: the arena holds the count of the optimizer that stepped last");
    }
    for (size_t k = 0; k < params.size(); ++k) {
        test::assert_bits(params[k]->master(), ref[k].p, "groups param " + std::to_string(k));
        test::assert_bits(params[k]->store().state(TTP_BUF_EXP_AVG, params[k]->index), ref[k].m,
                          "groups exp_avg " + std::to_string(k));
        test::assert_bits(params[k]->store().state(TTP_BUF_EXP_AVG_SQ, params[k]->index),
                          ref[k].v, "groups exp_avg_sq " + std::to_string(k));
    }
}

// Two AdamW optimizers over two groups of one loss-scaled arena, torch's GradScaler way: the
// first defers the scale update (opts.update_scale = false), the second updates it once per
// iteration from both overflows.  Each optimizer skips its own update on its own overflow.
// Scale 1024, growth 2 every 2 clean iterations, backoff 0.5; +inf in group a at iteration 2,
// in group b at 4, in both at 5: the scale goes 1024, 2048, 1024, 1024, 512, 256 (one backoff
// at 5), against 2048 at iteration 1 then a backoff per overflowing optimizer if each step
// updated it.
static void run_scaled_groups() {
    ParamArena arena(ttp::Mode::FP32);
    MLP model(64, 128, 10, arena);
    auto params = model.parameters();
    std::vector<Ref> ref;
    for (auto& p : params) {
        Ref r;
        r.p = p->master();
        r.m.assign(p->numel(), 0.0f);
        r.v.assign(p->numel(), 0.0f);
        ref.push_back(r);
    }
    ttp::Store& store = params[0]->store();
    store.configure_scaler(1024.0, 2.0, 0.5, 2, true);
    AdamW a({params[0], params[1]}, 1e-2f, {0.9, 0.95}, 1e-8f, 0.1f);
    AdamW b({params[2], params[3]}, 1e-2f, {0.9, 0.95}, 1e-8f, 0.1f);
    a.opts.update_scale = false;
    const float want_scale[6] = {1024.0f, 2048.0f, 1024.0f, 1024.0f, 512.0f, 256.0f};
    const bool inf_a[6] = {false, false, true, false, false, true};
    const bool inf_b[6] = {false, false, false, false, true, true};
    uint64_t ta = 0, tb = 0;
    float scale = 1024.0f;
    for (int k = 0; k < 6; ++k) {
        for (size_t j = 0; j < params.size(); ++j) {
            auto g = grad_of(params[j]->numel(), 300 + k * 10 + (int)j);
            std::vector<float> scaled(g.size());
            for (size_t i = 0; i < g.size(); ++i) scaled[i] = g[i] * scale;  // exact: 2^n
            const bool group_a = j < 2;
            if ((group_a ? inf_a[k] : inf_b[k]) && j % 2 == 0) scaled[3] = INFINITY;
            params[j]->grad = scaled;
            const bool skipped = group_a ? inf_a[k] : inf_b[k];
            if (!skipped) {
                const uint64_t t = (group_a ? ta : tb) + 1;
                adam_ref(ref[j], g, (double)1e-2f, 0.9, 0.95, (double)1e-8f, t, (double)0.1f,
                         j % 2 == 0);
            }
        }
        if (!inf_a[k]) ++ta;
        if (!inf_b[k]) ++tb;
        a.step();
        b.step();
        const auto st = store.scaler_state();
        scale = st.first;
        test::check(scale == want_scale[k],
                    "scaled groups: iteration " + std::to_string(k) + " scale " +
                        std::to_string(scale) + ", want " + std::to_string(want_scale[k]));
        test::check(store.step_count() == tb, "scaled groups: the arena holds b's count");
    }
    for (size_t k = 0; k < params.size(); ++k)
        test::assert_bits(params[k]->master(), ref[k].p, "scaled groups param " + std::to_string(k));
}

// A graph holding optimizer a's step, launched between optimizer b's eager steps: each launch
// hands the store's step count back to a (ttp::Graph::launch), so both keep their own.
static void run_graph_groups() {
    ParamArena arena(ttp::Mode::FP32);
    MLP model(64, 128, 10, arena);
    auto params = model.parameters();
    std::vector<Ref> ref;
    for (auto& p : params) {
        Ref r;
        r.p = p->master();
        r.m.assign(p->numel(), 0.0f);
        r.v.assign(p->numel(), 0.0f);
        ref.push_back(r);
    }
    const std::vector<size_t> ga = {0, 1}, gb = {2, 3};
    AdamW a({params[0], params[1]}, 1e-2f, {0.9, 0.95}, 1e-8f, 0.1f);
    Adam b({params[2], params[3]}, 3e-3f, {0.8, 0.999}, 1e-6f);
    ttp::Store& st = params[0]->store();
    ttp::Graph graph;
    uint64_t ta = 0, tb = 0;
    // lower case: an eager step; 'C': capture a's step (runs nothing); 'A': launch it
    const char* order = "abaCbAAbbA";
    for (int k = 0; order[k]; ++k) {
        const char ch = order[k];
        if (ch == 'C') {
            st.begin_capture();
            a.step();
            graph = st.end_capture();
            continue;
        }
        const bool is_a = ch == 'a' || ch == 'A';
        const auto& members = is_a ? ga : gb;
        const uint64_t t = is_a ? ++ta : ++tb;
        for (size_t j : members) {
            auto g = grad_of(params[j]->numel(), 300 + k * 10 + (int)j);
            params[j]->grad = g;
            if (is_a)
                adam_ref(ref[j], g, (double)1e-2f, 0.9, 0.95, (double)1e-8f, t, (double)0.1f,
                         j == 0);
            else
                adam_ref(ref[j], g, (double)3e-3f, 0.8, 0.999, (double)1e-6f, t, 0.0, false);
        }
        if (ch == 'A') graph.launch(); else if (is_a) a.step(); else b.step();
        test::check(st.step_count() == t,
                    "graph groups: the store holds the count of the optimizer that stepped last");
    }
    test::check(ta == 5 && tb == 4, "graph groups: 5 steps of a, 4 of b");
    for (size_t k = 0; k < params.size(); ++k) {
        test::assert_bits(params[k]->master(), ref[k].p, "graph groups param " + std::to_string(k));
        test::assert_bits(st.state(TTP_BUF_EXP_AVG, params[k]->index), ref[k].m,
                          "graph groups exp_avg " + std::to_string(k));
        test::assert_bits(st.state(TTP_BUF_EXP_AVG_SQ, params[k]->index), ref[k].v,
                          "graph groups exp_avg_sq " + std::to_string(k));
    }
}

// AdamW with clipping, its norm taken from per-tensor gradient sums (Store::grad_sumsq_tensors,
// AdamOptions::tensor_sums) against the same optimizer running the norm pass: the two add the
// same squares in different orders, so the weights agree within 2 ulp.
static void run_tensor_sums() {
    ParamArena a1(ttp::Mode::FP32), a2(ttp::Mode::FP32);
    MLP m1(64, 128, 10, a1), m2(64, 128, 10, a2);
    auto p1 = m1.parameters(), p2 = m2.parameters();
    for (size_t k = 0; k < p1.size(); ++k) p2[k]->set_data(p1[k]->master());
    AdamW o1(p1, 1e-2f, {0.9, 0.95}, 1e-8f, 0.1f, /*max_grad_norm*/ 0.05);
    AdamW o2(p2, 1e-2f, {0.9, 0.95}, 1e-8f, 0.1f, 0.05);
    o2.opts.tensor_sums = true;
    std::vector<uint32_t> all;
    for (auto& p : p2) all.push_back(p->index);
    for (int t = 1; t <= 4; ++t) {
        for (size_t k = 0; k < p1.size(); ++k) {
            auto g = grad_of(p1[k]->numel(), 500 + t * 10 + (int)k);
            p1[k]->grad = g;
            p2[k]->grad = g;
        }
        p2[0]->store().grad_sumsq_tensors(all);
        auto r1 = o1.step(true);
        auto r2 = o2.step(true);
        test::check(r1.clip_coef < 1.0f && r2.clip_coef == r1.clip_coef,
                    "tensor sums: the clip is active and has the same coefficient");
    }
    for (size_t k = 0; k < p1.size(); ++k) {
        const auto w1 = p1[k]->master(), w2 = p2[k]->master();
        uint32_t worst = 0;
        for (size_t i = 0; i < w1.size(); ++i) {
            const uint32_t u1 = test::bits(w1[i]), u2 = test::bits(w2[i]);
            worst = std::max(worst, u1 > u2 ? u1 - u2 : u2 - u1);
        }
        test::check(worst <= 2, "tensor sums: param " + std::to_string(k) + " within 2 ulp of the norm-pass step");
    }
    // a step with stale sums throws (nothing updated)
    p2[0]->grad = grad_of(p2[0]->numel(), 999);
    bool thrown = false;
    try { o2.step(); } catch (const std::runtime_error&) { thrown = true; }
    test::check(thrown, "tensor sums: a step after a gradient write without new sums throws");
}

// A backward's gradients in one bucket call (autograd::accumulate_grads_device over
// ttp_accumulate_grad_multi) against one accumulate_grad_device per parameter, both with sums
// and in reverse parameter order, from the same device sources (the grads of a third arena):
// AdamW steps from those sums give the same weights, bit for bit.
static void run_bucket_producer() {
    ParamArena a1(ttp::Mode::Mixed), a2(ttp::Mode::Mixed), as(ttp::Mode::FP32);
    MLP m1(64, 128, 10, a1), m2(64, 128, 10, a2), ms(64, 128, 10, as);
    auto p1 = m1.parameters(), p2 = m2.parameters(), ps = ms.parameters();
    AdamW o1(p1, 1e-2f, {0.9, 0.95}, 1e-8f, 0.1f, /*max_grad_norm*/ 0.05);
    AdamW o2(p2, 1e-2f, {0.9, 0.95}, 1e-8f, 0.1f, 0.05);
    o1.opts.tensor_sums = o2.opts.tensor_sums = true;
    for (size_t k = 0; k < p1.size(); ++k) p2[k]->set_data(p1[k]->master());
    for (int t = 1; t <= 3; ++t) {
        std::vector<ValuePtr> rev;
        std::vector<const void*> src;
        for (size_t k = ps.size(); k-- > 0;) {
            ps[k]->grad = grad_of(ps[k]->numel(), 700 + t * 10 + (int)k);
            rev.push_back(p2[k]);
            src.push_back(ps[k]->grad_ptr());
        }
        for (auto* p : {&p1, &p2})
            for (auto& v : *p) v->grad = std::nullopt;
        for (size_t k = p1.size(); k-- > 0;)
            p1[k]->accumulate_grad_device(ps[k]->grad_ptr(), TTP_DTYPE_F32, true);
        autograd::accumulate_grads_device(rev, src, TTP_DTYPE_F32, true);
        auto r1 = o1.step(true);
        auto r2 = o2.step(true);
        test::check(r1.grad_norm == r2.grad_norm && r1.clip_coef < 1.0f,
                    "bucket producer: the same norm from the sums, clip active");
    }
    for (size_t k = 0; k < p1.size(); ++k)
        test::assert_bits(p1[k]->master(), p2[k]->master(),
                          "bucket producer: param " + std::to_string(k));
    // parameters of two arenas in one call are refused
    bool thrown = false;
    try {
        autograd::accumulate_grads_device({p1[0], p2[1]}, {ps[0]->grad_ptr(), ps[1]->grad_ptr()},
                                          TTP_DTYPE_F32);
    } catch (const std::invalid_argument&) { thrown = true; }
    test::check(thrown, "bucket producer: parameters of two arenas are refused");
    // a parameter listed twice, or a null source, is refused before any launch
    const auto before = p2[0]->grad.value();
    for (int c = 0; c < 2; ++c) {
        thrown = false;
        try {
            if (c == 0)
                autograd::accumulate_grads_device({p2[0], p2[1], p2[0]},
                                                  {ps[0]->grad_ptr(), ps[1]->grad_ptr(),
                                                   ps[0]->grad_ptr()},
                                                  TTP_DTYPE_F32);
            else
                autograd::accumulate_grads_device({p2[0], p2[1]}, {ps[0]->grad_ptr(), nullptr},
                                                  TTP_DTYPE_F32);
        } catch (const std::invalid_argument&) { thrown = true; }
        test::check(thrown, c == 0 ? "bucket producer: a parameter listed twice is refused"
                                   : "bucket producer: a null source is refused");
        test::assert_bits(p2[0]->grad.value(), before,
                          "bucket producer: a refused list changes nothing");
    }
}

// Saved step counts belong to the store they were saved for: a store created after another
// was destroyed (here most likely at the same heap address) starts from its own count, not
// from what an optimizer saved for the destroyed one.
static void run_counts_outlive_store() {
    const std::vector<ttp::TensorSpec> specs = {{{256}, false, "w"}};
    auto a = std::make_shared<ttp::StepCounts>(), b = std::make_shared<ttp::StepCounts>();
    ttp::AdamOptions o;
    auto s1 = std::make_unique<ttp::Store>(specs, ttp::Mode::FP32);
    s1->set_grad(0, std::vector<float>(256, 0.5f));
    s1->claim_step_count(a);
    for (int k = 0; k < 3; ++k) s1->adam_step(o);
    s1->claim_step_count(b);  // a's count (3) saved for s1
    s1->adam_step(o);
    const void* where = s1.get();
    s1.reset();
    auto s2 = std::make_unique<ttp::Store>(specs, ttp::Mode::FP32);
    s2->set_grad(0, std::vector<float>(256, 0.5f));
    s2->claim_step_count(a);
    s2->adam_step(o);
    std::printf("counts: new store %s the destroyed one's address\n",
                (const void*)s2.get() == where ? "at" : "not at");
    test::check(s2->step_count() == 1, "a new store does not inherit a destroyed store's count");
}

int main() {
    test::DeviceGuard dg;
    run(false);
    run(true);
    run_groups();
    run_scaled_groups();
    run_graph_groups();
    run_tensor_sums();
    run_bucket_producer();
    run_counts_outlive_store();
    // py/optim.py:33-41 validation
    ParamArena arena;
    Linear l(4, 4, arena);
    int thrown = 0;
    try { Adam a(l.parameters(), 0.0f); } catch (const std::invalid_argument&) { ++thrown; }
    try { Adam a(l.parameters(), 1e-3f, {0.9, 0.999}, 0.0f); } catch (const std::invalid_argument&) { ++thrown; }
    try { Adam a(l.parameters(), 1e-3f, {1.1, 0.9}); } catch (const std::invalid_argument&) { ++thrown; }
    try { Adam a(l.parameters(), 1e-3f, {0.9, 1.0}); } catch (const std::invalid_argument&) { ++thrown; }
    test::check(thrown == 4, "Adam validation throws std::invalid_argument (" + std::to_string(thrown) + "/4)");
    return test::finish("test_adam");
}
