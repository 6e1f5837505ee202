// test_traced.cpp — the traced layers' optimizer surface: TracedSGD({layers}, lr).step()
// (autograd/traced/optim.hpp:15-29), per-module sgd_step(lr) (autograd/traced/nn.hpp:93-96,
// 272-275, 317-321), sgd_update (autograd/traced/ops.hpp:132-134) and the partitioned mesh
// layers (autograd/traced/mesh.hpp:167-170, 221-224, 270-274).  Each is
// `w - lr*dw` with one rounding per op; each call touches exactly its own tensors.
#include "autograd/traced.hpp"
#include "common.hpp"

using autograd::ParamArena;
using autograd::ValuePtr;

static std::vector<float> ramp(size_t n, float a, float b) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = a + b * (float)(i % 97);
    return v;
}

static std::vector<float> sgd_ref(const std::vector<float>& w, const std::vector<float>& g,
                                  float lr) {
    std::vector<float> out(w.size());
    for (size_t i = 0; i < w.size(); ++i) {
        const float update = g[i] * lr;
        out[i] = w[i] - update;
    }
    return out;
}

int main() {
    test::DeviceGuard dg;
    ParamArena arena(ttp::Mode::FP32);
    traced::TracedLinear l1(64, 32, 0.01f, arena), l2(32, 10, 0.01f, arena);
    traced::TracedLayerNorm ln(32, arena);
    traced::TracedEmbedding emb(65, 32, 0.02f, arena);

    // traced layers pre-allocate their grads: they exist (zero) before any backward
    test::check(l1.weight->grad.has_value(), "traced grads are pre-allocated");

    std::vector<ValuePtr> all = {l1.weight, l1.bias, l2.weight, l2.bias,
                                 ln.gamma,  ln.beta, emb.weight};
    std::vector<std::vector<float>> w, g;
    for (size_t k = 0; k < all.size(); ++k) {
        w.push_back(all[k]->master());
        g.push_back(ramp(all[k]->numel(), 0.5f + (float)k, 0.003f));
        all[k]->grad = g.back();  // what the backward pass writes into the grad buffers
    }

    // 1) TracedSGD over both linears: one launch, l1/l2 change, ln/emb do not
    traced::TracedSGD opt({&l1, &l2}, 0.05f);
    opt.step();
    for (size_t k = 0; k < 4; ++k) w[k] = sgd_ref(w[k], g[k], 0.05f);
    for (size_t k = 0; k < all.size(); ++k)
        test::assert_bits(all[k]->master(), w[k], "TracedSGD tensor " + std::to_string(k));

    // 2) per-module sgd_step: LayerNorm then Embedding
    ln.sgd_step(0.1f);
    w[4] = sgd_ref(w[4], g[4], 0.1f);
    w[5] = sgd_ref(w[5], g[5], 0.1f);
    emb.sgd_step(0.2f);
    w[6] = sgd_ref(w[6], g[6], 0.2f);
    l2.sgd_step(0.3f);
    w[2] = sgd_ref(w[2], g[2], 0.3f);
    w[3] = sgd_ref(w[3], g[3], 0.3f);
    for (size_t k = 0; k < all.size(); ++k)
        test::assert_bits(all[k]->master(), w[k], "sgd_step tensor " + std::to_string(k));

    // 3) free function sgd_update on one tensor
    traced::sgd_update(l1.bias, 0.7f);
    w[1] = sgd_ref(w[1], g[1], 0.7f);
    for (size_t k = 0; k < all.size(); ++k)
        test::assert_bits(all[k]->master(), w[k], "sgd_update tensor " + std::to_string(k));

    // layer init values of the reference's traced layers: LayerNorm gamma 1, beta 0
    ParamArena fresh(ttp::Mode::FP32);
    traced::TracedLayerNorm ln2(8, fresh);
    test::assert_all_close(ln2.gamma->data(), 1.0f, 0.0f, "LayerNorm gamma init");
    test::assert_all_close(ln2.beta->data(), 0.0f, 0.0f, "LayerNorm beta init");
    // TraceContext (autograd/traced/trace.hpp:21-88): the first run() captures the TracedSGD
    // step into a graph and executes it, later runs replay it; gradients change in between
    {
        ParamArena arena3(ttp::Mode::FP32);
        traced::TracedLinear a(16, 8, 0.01f, arena3), b(8, 4, 0.02f, arena3);
        traced::TracedSGD opt2({&a, &b}, 0.1f);
        std::vector<ValuePtr> ps = {a.weight, a.bias, b.weight, b.bias};
        std::vector<std::vector<float>> wr;
        for (auto& p : ps) wr.push_back(p->master());
        {
            traced::TraceContext trace(a.weight->store());
            for (int it = 0; it < 4; ++it) {
                std::vector<std::vector<float>> gr;
                for (size_t k = 0; k < ps.size(); ++k) {
                    gr.push_back(ramp(ps[k]->numel(), 0.25f * (float)(it + 1), 0.01f * (float)(k + 1)));
                    ps[k]->grad = gr.back();
                }
                if (it == 0)
                    opt2.step();  // eager once: the work tables exist before capture
                else
                    trace.run([&] { opt2.step(); });
                for (size_t k = 0; k < ps.size(); ++k) wr[k] = sgd_ref(wr[k], gr[k], 0.1f);
                for (size_t k = 0; k < ps.size(); ++k)
                    test::assert_bits(ps[k]->master(), wr[k],
                                      "TraceContext iteration " + std::to_string(it) + " tensor " +
                                          std::to_string(k));
                test::check(trace.is_captured() == (it >= 1), "TraceContext captured flag");
            }
        }  // the graph is released before the store
    }
    // the partitioned mesh layers (autograd/traced/mesh.hpp:119-290): three replicas in one
    // arena; a replica's sgd_step touches only its tensors, the mesh model's steps them all
    {
        ParamArena arena4(ttp::Mode::FP32);
        auto mesh = traced::TracedMeshModel<traced::TracedPartitionedMLP>::create_mlp(
            arena4, 3, /*batch*/ 32, 64, 32, 16);
        test::check(mesh.size() == 3 && mesh.models[2]->layer1.partition_id == 2,
                    "mesh: three replicas with their partition ids");
        auto ps = mesh.parameters();
        test::check(ps.size() == 12, "mesh: 4 tensors per replica");
        test::assert_all_close(mesh.models[1]->layer2.weight->data(), 0.01f, 0.0f,
                               "mesh: linears filled with 0.01");
        std::vector<std::vector<float>> wm, gm;
        for (size_t k = 0; k < ps.size(); ++k) {
            wm.push_back(ps[k]->master());
            gm.push_back(ramp(ps[k]->numel(), 0.1f * (float)(k + 1), 0.002f));
            ps[k]->grad = gm.back();
        }
        mesh.models[1]->sgd_step(0.05f);  // replica 1 only
        for (size_t k = 4; k < 8; ++k) wm[k] = sgd_ref(wm[k], gm[k], 0.05f);
        mesh.sgd_step(0.02f);  // every replica, one launch
        for (size_t k = 0; k < ps.size(); ++k) wm[k] = sgd_ref(wm[k], gm[k], 0.02f);
        for (size_t k = 0; k < ps.size(); ++k)
            test::assert_bits(ps[k]->master(), wm[k], "mesh tensor " + std::to_string(k));
        test::check(traced::MeshConfig::create(0).n_partitions == 8,
                    "mesh: n_partitions 0 is one per XCD");
    }
    return test::finish("test_traced");
}
