// traced.hpp — drop-in for the traced layers' optimizer surface (autograd/traced/*.hpp).
//
// The reference's traced layers own pre-allocated weight and gradient buffers that every
// backward overwrites (autograd/traced/nn.hpp:54-69), and update themselves with
// sgd_step(lr) = `w - lr*dw` per tensor (autograd/traced/nn.hpp:93-96, 272-275, 317-321).
// Here the buffers are tensors of one ParamArena whose grads always exist (zero until a
// backward writes them), and each sgd_step is one launch over that module's tensors.
// TracedSGD (autograd/traced/optim.hpp:15-29) steps all its layers in one launch.
#pragma once

#include <initializer_list>
#include <memory>
#include <vector>

#include "autograd/value.hpp"

namespace traced {

using autograd::ParamArena;
using autograd::ValuePtr;

namespace detail {
inline void sgd_on(const std::vector<ValuePtr>& ps, float lr) {
    if (ps.empty()) return;
    std::vector<uint32_t> idx;
    for (auto& p : ps) idx.push_back(p->index);
    ttp::SgdOptions o;
    o.lr = lr;
    ps.front()->store().sgd_step(o, &idx);
}
}  // namespace detail

// y = x @ weight.T + bias;  weight [out, in] filled with `init`, bias [1, out] zeros
// (autograd/traced/nn.hpp:61-68)
struct TracedLinear {
    ValuePtr weight, bias;  // d_weight / d_bias are weight->grad / bias->grad
    uint32_t in_features, out_features;

    TracedLinear(uint32_t in_f, uint32_t out_f, float init, ParamArena& arena)
        : weight(arena.parameter({out_f, in_f}, autograd::filled((uint64_t)out_f * in_f, init),
                                 "weight", true, /*grad_always=*/true)),
          bias(arena.parameter({1, out_f}, autograd::filled(out_f, 0.0f), "bias", false, true)),
          in_features(in_f),
          out_features(out_f) {}

    std::vector<ValuePtr> parameters() const { return {weight, bias}; }
    void sgd_step(float lr) { detail::sgd_on(parameters(), lr); }
};

// gamma ones, beta zeros (autograd/traced/nn.hpp LayerNorm)
struct TracedLayerNorm {
    ValuePtr gamma, beta;

    TracedLayerNorm(uint32_t dim, ParamArena& arena)
        : gamma(arena.parameter({1, dim}, autograd::filled(dim, 1.0f), "gamma", false, true)),
          beta(arena.parameter({1, dim}, autograd::filled(dim, 0.0f), "beta", false, true)) {}
    // the reference's (dim, eps, device) constructor; eps belongs to the forward pass
    TracedLayerNorm(uint32_t dim, float /*eps*/, ParamArena& arena) : TracedLayerNorm(dim, arena) {}

    std::vector<ValuePtr> parameters() const { return {gamma, beta}; }
    void sgd_step(float lr) { detail::sgd_on(parameters(), lr); }
};

// [vocab, dim] table filled with `init` (autograd/traced/nn.hpp:308-315).  The reference
// untilizes d_weight before its update (:317-321); the flat store has a single row-major
// layout, so there is nothing to convert.
struct TracedEmbedding {
    ValuePtr weight;

    TracedEmbedding(uint32_t vocab, uint32_t dim, float init, ParamArena& arena)
        : weight(arena.parameter({vocab, dim}, autograd::filled((uint64_t)vocab * dim, init),
                                 "embedding", true, true)) {}
    // the reference's (vocab, dim, batch, seq, init, device) constructor; batch and seq size
    // its forward buffers, which are not part of this engine
    TracedEmbedding(uint32_t vocab, uint32_t dim, uint32_t /*batch*/, uint32_t /*seq*/, float init,
                    ParamArena& arena)
        : TracedEmbedding(vocab, dim, init, arena) {}

    std::vector<ValuePtr> parameters() const { return {weight}; }
    void sgd_step(float lr) { detail::sgd_on(parameters(), lr); }
};

// autograd/traced/ops.hpp:132-134: param = param - lr * grad (one tensor)
inline void sgd_update(const ValuePtr& param, float lr) { detail::sgd_on({param}, lr); }

// N dim x dim linears filled with 0.01 (autograd/traced/mlp.hpp:18-70); sgd_step (:106-110)
// updates all N layers at the member lr, here in one launch.  The forward / backward buffers
// and train_step's passes are model compute, not part of this engine.
template <size_t N>
struct TracedMLP {
    std::vector<TracedLinear> layers;
    uint32_t batch, dim;
    float lr;

    TracedMLP(uint32_t b, uint32_t d, float learning_rate, ParamArena& arena)
        : batch(b), dim(d), lr(learning_rate) {
        layers.reserve(N);
        for (size_t i = 0; i < N; ++i) layers.emplace_back(d, d, 0.01f, arena);
    }

    std::vector<ValuePtr> parameters() const {
        std::vector<ValuePtr> ps;
        for (const auto& l : layers)
            for (auto& p : l.parameters()) ps.push_back(p);
        return ps;
    }
    void sgd_step() { detail::sgd_on(parameters(), lr); }
};

// One transformer block's parameters (autograd/traced/transformer_train.hpp:76-135): ln1,
// ln2 (gamma, beta), wq, wk, wv, wo [d, d], w1 [d, ffn], w2 [ffn, d] (weight, bias) = 16
// tensors, linears filled with 0.01.  sgd_step() (:259-268) is one launch over all 16.
struct TracedTransformerLayerTrainable {
    TracedLayerNorm ln1, ln2;
    TracedLinear wq, wk, wv, wo;
    TracedLinear w1, w2;
    uint32_t batch, seq, dim, heads, head_dim, ffn_dim;
    float lr;

    TracedTransformerLayerTrainable(uint32_t b, uint32_t s, uint32_t d, uint32_t h,
                                    uint32_t ffn_mult, float learning_rate, ParamArena& arena)
        : ln1(d, 1e-5f, arena),
          ln2(d, 1e-5f, arena),
          wq(d, d, 0.01f, arena),
          wk(d, d, 0.01f, arena),
          wv(d, d, 0.01f, arena),
          wo(d, d, 0.01f, arena),
          w1(d, d * ffn_mult, 0.01f, arena),
          w2(d * ffn_mult, d, 0.01f, arena),
          batch(b),
          seq(s),
          dim(d),
          heads(h),
          head_dim(d / h),
          ffn_dim(d * ffn_mult),
          lr(learning_rate) {}

    std::vector<ValuePtr> parameters() const {
        std::vector<ValuePtr> ps;
        for (auto* m : {&ln1, &ln2})
            for (auto& p : m->parameters()) ps.push_back(p);
        for (auto* m : {&wq, &wk, &wv, &wo, &w1, &w2})
            for (auto& p : m->parameters()) ps.push_back(p);
        return ps;
    }
    void sgd_step() { detail::sgd_on(parameters(), lr); }
};

// N blocks (transformer_train.hpp:275-345); sgd_step() (:335-339) is one launch over all.
template <size_t N>
struct TracedTransformerStack {
    static_assert(N >= 1, "Must have at least 1 layer");
    std::vector<TracedTransformerLayerTrainable> layers;
    float lr;

    TracedTransformerStack(uint32_t b, uint32_t s, uint32_t d, uint32_t h, uint32_t ffn_mult,
                           float learning_rate, ParamArena& arena)
        : lr(learning_rate) {
        layers.reserve(N);
        for (size_t i = 0; i < N; ++i) layers.emplace_back(b, s, d, h, ffn_mult, learning_rate, arena);
    }

    std::vector<ValuePtr> parameters() const {
        std::vector<ValuePtr> ps;
        for (auto& l : layers)
            for (auto& p : l.parameters()) ps.push_back(p);
        return ps;
    }
    void sgd_step() { detail::sgd_on(parameters(), lr); }
};

// The GPT model (transformer_train.hpp:363-501): token and position embeddings (0.02),
// N blocks, output projection [d, vocab] (0.02).  sgd_step() (:487-494) is one launch over
// every tensor of the model (the reference issues two programs per tensor plus an untilize
// per embedding).
template <size_t N>
struct TracedTransformerWithEmbedding {
    static_assert(N >= 1, "Must have at least 1 layer");
    TracedEmbedding tok_emb;
    TracedEmbedding pos_emb;
    std::vector<TracedTransformerLayerTrainable> layers;
    TracedLinear output_proj;
    uint32_t batch, seq, dim, vocab_size;
    float lr;

    TracedTransformerWithEmbedding(uint32_t b, uint32_t s, uint32_t d, uint32_t h,
                                   uint32_t ffn_mult, uint32_t vocab, float learning_rate,
                                   ParamArena& arena)
        : tok_emb(vocab, d, b, s, 0.02f, arena),
          pos_emb(s, d, b, s, 0.02f, arena),
          layers(make_layers(b, s, d, h, ffn_mult, learning_rate, arena)),
          output_proj(d, vocab, 0.02f, arena),
          batch(b),
          seq(s),
          dim(d),
          vocab_size(vocab),
          lr(learning_rate) {}

    std::vector<ValuePtr> parameters() const {
        std::vector<ValuePtr> ps = {tok_emb.weight, pos_emb.weight};
        for (auto& l : layers)
            for (auto& p : l.parameters()) ps.push_back(p);
        for (auto& p : output_proj.parameters()) ps.push_back(p);
        return ps;
    }
    void sgd_step() { detail::sgd_on(parameters(), lr); }

private:
    // declared in member order: embeddings, blocks, output projection (the flat layout)
    static std::vector<TracedTransformerLayerTrainable> make_layers(uint32_t b, uint32_t s,
                                                                    uint32_t d, uint32_t h,
                                                                    uint32_t ffn_mult, float lr,
                                                                    ParamArena& arena) {
        std::vector<TracedTransformerLayerTrainable> v;
        v.reserve(N);
        for (size_t i = 0; i < N; ++i) v.emplace_back(b, s, d, h, ffn_mult, lr, arena);
        return v;
    }
};

// traced::TraceContext (autograd/traced/trace.hpp:21-88) over a ttp::Store: the first
// run(fn) captures the work fn queues on the store's stream into a hipGraph and executes it;
// later calls replay it.  Step the captured tensor sets once eagerly before the first run.
// Release (or destroy) the TraceContext before the store.
class TraceContext {
public:
    explicit TraceContext(ttp::Store& store) : store_(&store) {}
    TraceContext(const TraceContext&) = delete;
    TraceContext& operator=(const TraceContext&) = delete;
    TraceContext(TraceContext&&) = default;
    TraceContext& operator=(TraceContext&&) = default;

    template <typename Fn>
    void run(Fn&& fn) {
        if (!graph_) {
            store_->begin_capture();
            try {
                fn();
            } catch (...) {
                store_->discard_capture();
                throw;
            }
            graph_ = store_->end_capture();
        }
        graph_.launch();
    }
    bool is_captured() const { return (bool)graph_; }
    void release() { graph_.reset(); }
    void reset() { release(); }

private:
    ttp::Store* store_;
    ttp::Graph graph_;
};

// The partitioned layers of autograd/traced/mesh.hpp:25-290: N model replicas, each pinned to
// its own partition of a Tenstorrent core grid, each updated by its own sgd_step.  On MI355X
// the hardware spreads every launch over all CUs, so a partition keeps only its id; the
// replicas' tensors share one ParamArena and TracedMeshModel::sgd_step is one launch over all
// of them (the reference issues two programs per tensor, four per layer, per replica).
struct PartitionConfig {
    uint32_t partition_id;
    explicit PartitionConfig(uint32_t id) : partition_id(id) {}
};

struct MeshConfig {
    uint32_t n_partitions = 0;
    std::vector<PartitionConfig> partitions;
    // mesh.hpp:42-53 defaults n_partitions = 0 to one partition per 8 Tensix cores; here it
    // is one per MI355X XCD (8)
    static MeshConfig create(uint32_t n_partitions) {
        MeshConfig c;
        c.n_partitions = n_partitions ? n_partitions : 8;
        for (uint32_t i = 0; i < c.n_partitions; ++i) c.partitions.emplace_back(i);
        return c;
    }
};

// weight [out, in] filled with `init`, bias [1, out] zeros (mesh.hpp:129-138); sgd_step
// (:167-170) is one launch over both
struct TracedPartitionedLinear : TracedLinear {
    uint32_t partition_id;
    TracedPartitionedLinear(uint32_t in_f, uint32_t out_f, float init, ParamArena& arena,
                            const PartitionConfig& config)
        : TracedLinear(in_f, out_f, init, arena), partition_id(config.partition_id) {}
};

// two layers filled with 0.01 (mesh.hpp:192-200); sgd_step (:221-224) is one launch over both
struct TracedPartitionedMLP {
    TracedPartitionedLinear layer1, layer2;
    uint32_t batch, dim;

    TracedPartitionedMLP(uint32_t b, uint32_t in_dim, uint32_t hidden_dim, uint32_t out_dim,
                         ParamArena& arena, const PartitionConfig& config)
        : layer1(in_dim, hidden_dim, 0.01f, arena, config),
          layer2(hidden_dim, out_dim, 0.01f, arena, config),
          batch(b),
          dim(hidden_dim) {}

    std::vector<ValuePtr> parameters() const {
        return {layer1.weight, layer1.bias, layer2.weight, layer2.bias};
    }
    void sgd_step(float lr) { detail::sgd_on(parameters(), lr); }
};

// N replicas (mesh.hpp:231-290); create_mlp builds N TracedPartitionedMLP in one arena
template <typename ModelType>
struct TracedMeshModel {
    std::vector<std::unique_ptr<ModelType>> models;
    MeshConfig config;

    static TracedMeshModel<TracedPartitionedMLP> create_mlp(ParamArena& arena,
                                                            uint32_t n_partitions, uint32_t batch,
                                                            uint32_t in_dim, uint32_t hidden_dim,
                                                            uint32_t out_dim) {
        TracedMeshModel<TracedPartitionedMLP> m;
        m.config = MeshConfig::create(n_partitions);
        for (const auto& part : m.config.partitions)
            m.models.push_back(std::make_unique<TracedPartitionedMLP>(batch, in_dim, hidden_dim,
                                                                      out_dim, arena, part));
        return m;
    }

    std::vector<ValuePtr> parameters() const {
        std::vector<ValuePtr> ps;
        for (const auto& model : models)
            for (auto& p : model->parameters()) ps.push_back(p);
        return ps;
    }
    // every replica's update in one launch (mesh.hpp:270-274 steps them one by one)
    void sgd_step(float lr) { detail::sgd_on(parameters(), lr); }
    size_t size() const { return models.size(); }
};

struct TracedSGD {
    std::vector<TracedLinear*> layers;
    float lr;

    TracedSGD(std::initializer_list<TracedLinear*> ls, float learning_rate)
        : layers(ls), lr(learning_rate) {}

    // one launch over every layer's weight and bias
    void step() {
        std::vector<ValuePtr> ps;
        for (auto* l : layers) {
            ps.push_back(l->weight);
            ps.push_back(l->bias);
        }
        detail::sgd_on(ps, lr);
    }
    // no zero_grad: gradients are overwritten each backward pass (autograd/traced/optim.hpp:28)
};

}  // namespace traced
