// ttperf.hpp — header-only C++ owner of a libttperf_hip context (include/ttperf/ttperf.h).
//
// ttp::Store is one flat parameter store on one GPU.  Errors from the C ABI become
// exceptions here (std::invalid_argument for the argument errors py/optim.py raises
// ValueError for, std::out_of_range for bad indices/sizes, std::runtime_error otherwise),
// the way TTNN errors surface as std::exception in the reference
// (bench/autograd/bench_gpt2_full.cpp:153-165).
#pragma once

#include <atomic>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "ttperf/ttperf.h"

namespace ttp {

inline void check(int rc) {
    if (rc == TTP_OK) return;
    std::string msg = std::string("libttperf_hip: ") + ttp_last_error();
    if (rc == TTP_ERR_INVALID) throw std::invalid_argument(msg);
    if (rc == TTP_ERR_RANGE) throw std::out_of_range(msg);
    throw std::runtime_error(msg);
}

// Bf16: the reference C++ autograd's own storage, bf16 weights and gradients and no fp32
// state; plain SGD only, each op rounded to bf16 as the reference's ttnn ops round theirs
// (TTP_MODE_BF16).
enum class Mode { FP32 = TTP_MODE_FP32, Mixed = TTP_MODE_MIXED, Bf16 = TTP_MODE_BF16 };
// Store layout of a Mixed store (TTP_STORE_SGD): Default keeps master, m and v in shared
// records (Adam's layout); Sgd keeps a contiguous master and no m / v, for stores that SGD
// steps (the first Adam step converts it to Default).  FP32 stores are laid out alike either
// way.
enum class Layout { Default = 0, Sgd = TTP_STORE_SGD };

struct TensorSpec {
    std::vector<uint64_t> shape;
    bool decay = false;
    std::string name;
    uint64_t numel() const {
        uint64_t n = 1;
        for (auto d : shape) n *= d;
        return n;
    }
};

struct AdamOptions {
    double lr = 1e-3, beta1 = 0.9, beta2 = 0.999, eps = 1e-8, weight_decay = 0.0;
    bool decoupled = true;
    double max_grad_norm = 0.0;
    bool tensor_sums = false;  // norm from Store::grad_sumsq_tensors (TTP_STEP_TENSOR_SUMS)
    // false: leave the loss scale to the iteration's last step or Store::scaler_update()
    // (TTP_STEP_DEFER_SCALE), for all but the last of several optimizers over one store
    bool update_scale = true;
    ttp_adam_hparams c() const {
        ttp_adam_hparams h{};
        h.flags = (tensor_sums ? TTP_STEP_TENSOR_SUMS : 0) | (update_scale ? 0 : TTP_STEP_DEFER_SCALE);
        h.lr = lr;
        h.beta1 = beta1;
        h.beta2 = beta2;
        h.eps = eps;
        h.weight_decay = weight_decay;
        h.decoupled = decoupled ? 1 : 0;
        h.max_grad_norm = max_grad_norm;
        return h;
    }
};

struct SgdOptions {
    double lr = 1e-2, momentum = 0.0, dampening = 0.0, weight_decay = 0.0;
    bool nesterov = false;
    double max_grad_norm = 0.0;
    bool tensor_sums = false;  // norm from Store::grad_sumsq_tensors (TTP_STEP_TENSOR_SUMS)
    bool update_scale = true;  // as AdamOptions::update_scale
    ttp_sgd_hparams c() const {
        ttp_sgd_hparams h{};
        h.flags = (tensor_sums ? TTP_STEP_TENSOR_SUMS : 0) | (update_scale ? 0 : TTP_STEP_DEFER_SCALE);
        h.lr = lr;
        h.momentum = momentum;
        h.dampening = dampening;
        h.weight_decay = weight_decay;
        h.nesterov = nesterov ? 1 : 0;
        h.max_grad_norm = max_grad_norm;
        return h;
    }
};

class Store;

// The step counts an optimizer keeps for the stores whose count another optimizer held when
// it last stepped them.  py/optim.py:46,50 keeps `_step` per optimizer; the count the
// kernels read lives in the store, so optimizers hand it over (Store::claim_step_count).
// Keyed by Store::uid(), never reused within a process, so a store allocated where a
// destroyed one lived does not inherit its count.
struct StepCounts {
    std::map<uint64_t, uint64_t> saved;
};

// A captured graph of a store's work (ttp_capture_begin .. ttp_capture_end); move-only.  It
// remembers which optimizer held the store's step count at capture, and hands the count back
// to it before each launch (a no-op unless another optimizer stepped the store since).
class Graph {
public:
    Graph() = default;
    explicit Graph(ttp_graph* g) : g_(g) {}
    Graph(ttp_graph* g, Store* store, std::weak_ptr<StepCounts> owner)
        : g_(g), store_(store), owner_(std::move(owner)) {}
    Graph(Graph&& o) noexcept : g_(o.g_), store_(o.store_), owner_(std::move(o.owner_)) {
        o.g_ = nullptr;
    }
    Graph& operator=(Graph&& o) noexcept {
        if (this != &o) {
            reset();
            g_ = o.g_;
            store_ = o.store_;
            owner_ = std::move(o.owner_);
            o.g_ = nullptr;
        }
        return *this;
    }
    Graph(const Graph&) = delete;
    Graph& operator=(const Graph&) = delete;
    ~Graph() { reset(); }
    inline void launch();
    void reset() {
        if (g_) ttp_graph_destroy(g_);
        g_ = nullptr;
    }
    explicit operator bool() const { return g_ != nullptr; }

private:
    ttp_graph* g_ = nullptr;
    Store* store_ = nullptr;
    std::weak_ptr<StepCounts> owner_;
};

class Store {
public:
    Store(const std::vector<TensorSpec>& specs, Mode mode, int device = 0,
          Layout layout = Layout::Default)
        : specs_(specs), mode_(mode) {
        // a library built against another ABI version would read these arguments differently
        if (ttp_abi_version() != TTP_ABI_VERSION)
            throw std::runtime_error("libttperf_hip implements ABI version " +
                                     std::to_string(ttp_abi_version()) + ", this header " +
                                     std::to_string(TTP_ABI_VERSION));
        std::vector<ttp_tensor_desc> d(specs.size());
        for (size_t i = 0; i < specs.size(); ++i) {
            d[i].numel = specs[i].numel();
            d[i].flags = specs[i].decay ? TTP_TENSOR_DECAY : 0u;
            d[i].reserved = 0;
        }
        ttp_ctx* c = nullptr;
        check(ttp_create(device, d.data(), (uint32_t)d.size(), (int)mode | (int)layout, &c));
        ctx_ = c;
    }
    ~Store() {
        if (ctx_) ttp_destroy(ctx_);
    }
    Store(const Store&) = delete;
    Store& operator=(const Store&) = delete;

    ttp_ctx* get() const { return ctx_; }
    uint64_t uid() const { return uid_; }
    Mode mode() const { return mode_; }
    // Sgd while a Mixed store keeps the SGD layout's contiguous master (until an Adam step)
    Layout layout() const {
        if (mode_ == Mode::Bf16) return Layout::Default;  // no master to lay out
        void* base = nullptr;
        uint32_t group = 0, stride = 0;
        check(ttp_buffer_layout(ctx_, TTP_BUF_MASTER, &base, &group, &stride));
        return mode_ == Mode::Mixed && stride == group ? Layout::Sgd : Layout::Default;
    }
    size_t size() const { return specs_.size(); }
    const TensorSpec& spec(uint32_t i) const { return specs_.at(i); }
    uint64_t numel(uint32_t i) const { return specs_.at(i).numel(); }

    // ---- data -------------------------------------------------------------------------------
    // fp32 weights of tensor i: the master copy (and its bf16 RNE copy in Mixed mode); in
    // Bf16 mode the bf16 weights, rounded to nearest even
    void set_weights(uint32_t i, const std::vector<float>& w) {
        if (mode_ == Mode::Bf16) {
            std::vector<uint16_t> h(w.size());
            for (size_t k = 0; k < w.size(); ++k) h[k] = to_bf16(w[k]);
            check(ttp_upload(ctx_, TTP_BUF_PARAM, i, h.data(), h.size(), TTP_HOST));
            return;
        }
        check(ttp_upload(ctx_, TTP_BUF_MASTER, i, w.data(), w.size(), TTP_HOST));
    }
    std::vector<float> master(uint32_t i) const { return download_f32(TTP_BUF_MASTER, i); }
    // model-facing weights widened to float (bf16 in Mixed and Bf16 mode)
    std::vector<float> weights(uint32_t i) const {
        if (mode_ == Mode::FP32) return download_f32(TTP_BUF_PARAM, i);
        return widen(download_u16(TTP_BUF_PARAM, i));
    }
    std::vector<uint16_t> weights_bf16(uint32_t i) const { return download_u16(TTP_BUF_PARAM, i); }
    std::vector<float> state(int which, uint32_t i) const { return download_f32(which, i); }

    // gradients: fp32 values (rounded to bf16 in Mixed and Bf16 mode, round-to-nearest-even)
    void set_grad(uint32_t i, const std::vector<float>& g) {
        if (mode_ == Mode::FP32) {
            check(ttp_upload(ctx_, TTP_BUF_GRAD, i, g.data(), g.size(), TTP_HOST));
        } else {
            std::vector<uint16_t> h(g.size());
            for (size_t k = 0; k < g.size(); ++k) h[k] = to_bf16(g[k]);
            check(ttp_upload(ctx_, TTP_BUF_GRAD, i, h.data(), h.size(), TTP_HOST));
        }
    }
    std::vector<float> grad(uint32_t i) const {
        if (mode_ == Mode::FP32) return download_f32(TTP_BUF_GRAD, i);
        return widen(download_u16(TTP_BUF_GRAD, i));
    }
    bool has_grad(uint32_t i) const {
        int h = 0;
        check(ttp_get_has_grad(ctx_, i, &h));
        return h != 0;
    }
    void set_has_grad(uint32_t i, bool h) { check(ttp_set_has_grad(ctx_, i, h ? 1 : 0)); }
    // fill = false (with set_to_none): flags only, the gradients keep their old contents
    // until written (TTP_ZERO_NO_FILL)
    void zero_grad(bool set_to_none = true, bool fill = true) {
        check(ttp_zero_grad(ctx_, (set_to_none ? 1 : 0) | (fill ? 0 : TTP_ZERO_NO_FILL)));
    }
    void zero_grad(const std::vector<uint32_t>& indices, bool set_to_none, bool fill = true) {
        check(ttp_zero_grad_subset(ctx_, indices.data(), (uint32_t)indices.size(),
                                   (set_to_none ? 1 : 0) | (fill ? 0 : TTP_ZERO_NO_FILL)));
    }
    // grad = g if tensor i has none, else grad + g (fp32 add, one rounding to the grad type);
    // sums: also store tensor i's gradient sum for a tensor_sums step (TTP_ACCUM_SUMSQ)
    void accumulate_grad(uint32_t i, const std::vector<float>& g, bool sums = false) {
        check(ttp_accumulate_grad(ctx_, i, g.data(), g.size(),
                                  TTP_DTYPE_F32 | (sums ? TTP_ACCUM_SUMSQ : 0), TTP_HOST));
    }
    // the same from device memory (fp32 or bf16 bits), e.g. a backward kernel's output
    void accumulate_grad_device(uint32_t i, const void* src, int dtype, bool sums = false) {
        check(ttp_accumulate_grad(ctx_, i, src, numel(i), dtype | (sums ? TTP_ACCUM_SUMSQ : 0),
                                  TTP_DEVICE));
    }
    // a backward's bucket in one launch: tensor idx[k] receives srcs[k] (device memory, all
    // of one dtype), as accumulate_grad_device(idx[k], srcs[k], dtype, sums) would
    void accumulate_grads_device(const std::vector<uint32_t>& idx,
                                 const std::vector<const void*>& srcs, int dtype,
                                 bool sums = false) {
        if (idx.size() != srcs.size())
            throw std::invalid_argument("accumulate_grads_device: one source per index");
        check(ttp_accumulate_grad_multi(ctx_, idx.data(), srcs.data(), (uint32_t)idx.size(),
                                        dtype | (sums ? TTP_ACCUM_SUMSQ : 0)));
    }
    void* device_ptr(int which, uint32_t i = TTP_ALL_TENSORS) {
        void* p = nullptr;
        check(ttp_buffer_ptr(ctx_, which, i, &p));
        return p;
    }

    // ---- steps --------------------------------------------------------------------------------
    ttp_step_report adam_step(const AdamOptions& o, const std::vector<uint32_t>* subset = nullptr,
                              bool want_report = false) {
        ttp_adam_hparams h = o.c();
        ttp_step_report r{};
        ttp_step_report* rp = want_report ? &r : nullptr;
        if (subset)
            check(ttp_adam_step_subset(ctx_, &h, subset->data(), (uint32_t)subset->size(), rp));
        else
            check(ttp_adam_step(ctx_, &h, rp));
        return r;
    }
    ttp_step_report sgd_step(const SgdOptions& o, const std::vector<uint32_t>* subset = nullptr,
                             bool want_report = false) {
        ttp_sgd_hparams h = o.c();
        ttp_step_report r{};
        ttp_step_report* rp = want_report ? &r : nullptr;
        if (subset)
            check(ttp_sgd_step_subset(ctx_, &h, subset->data(), (uint32_t)subset->size(), rp));
        else
            check(ttp_sgd_step(ctx_, &h, rp));
        return r;
    }
    // per-tensor gradient sums of the listed tensors, for a step with tensor_sums set
    void grad_sumsq_tensors(const std::vector<uint32_t>& indices) {
        check(ttp_grad_sumsq_tensors(ctx_, indices.data(), (uint32_t)indices.size()));
    }
    double grad_norm() {
        double n = 0;
        check(ttp_grad_norm(ctx_, &n));
        return n;
    }
    void configure_scaler(double init_scale = 65536.0, double growth = 2.0, double backoff = 0.5,
                          int interval = 2000, bool enabled = true) {
        ttp_scaler_config c{enabled ? 1 : 0, interval, init_scale, growth, backoff};
        check(ttp_scaler_configure(ctx_, &c));
    }
    // GradScaler.update() after steps that all had update_scale = false
    void scaler_update() { check(ttp_scaler_update(ctx_)); }
    std::pair<float, int32_t> scaler_state() {
        float s = 0;
        int32_t t = 0;
        check(ttp_scaler_get(ctx_, &s, &t));
        return {s, t};
    }
    uint64_t step_count() {
        uint64_t t = 0;
        check(ttp_get_step(ctx_, &t));
        return t;
    }
    void set_step_count(uint64_t t) { check(ttp_set_step(ctx_, t)); }
    void sync() { check(ttp_sync(ctx_)); }
    void save_state(const std::string& path) { check(ttp_save_state(ctx_, path.c_str())); }
    void load_state(const std::string& path) { check(ttp_load_state(ctx_, path.c_str())); }
    void begin_capture() {
        check(ttp_capture_begin(ctx_));
        capturing_ = true;
    }
    Graph end_capture() {
        capturing_ = false;
        ttp_graph* g = nullptr;
        check(ttp_capture_end(ctx_, &g));
        return Graph(g, this, t_owner_);
    }
    void discard_capture() {
        capturing_ = false;
        (void)ttp_capture_end(ctx_, nullptr);
    }

    // Make the step count `me`'s before the optimizer `me` steps this store.  A store that no
    // live optimizer stepped last keeps its count (a loaded checkpoint's, say); one that a
    // different live optimizer stepped last has that count saved for it and `me`'s restored
    // (0 if `me` never stepped the store): a synchronising read and a write, on a change of
    // owner only, which a graph capture cannot hold.
    void claim_step_count(const std::shared_ptr<StepCounts>& me) {
        std::shared_ptr<StepCounts> prev = t_owner_.lock();
        if (prev == me) return;
        auto it = me->saved.find(uid_);
        if (prev || it != me->saved.end()) {
            if (capturing_)
                throw std::runtime_error(
                    "libttperf_hip: a second optimizer steps this store inside a graph capture; "
                    "the step count hand-over reads the device and cannot be captured");
            if (prev) prev->saved[uid_] = step_count();
            uint64_t t = 0;
            if (it != me->saved.end()) {
                t = it->second;
                me->saved.erase(it);
            }
            set_step_count(t);
        }
        t_owner_ = me;
    }

    static uint16_t to_bf16(float x) {
        uint32_t u;
        std::memcpy(&u, &x, 4);
        if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
        u += 0x7FFFu + ((u >> 16) & 1u);
        return (uint16_t)(u >> 16);
    }

private:
    static std::vector<float> widen(const std::vector<uint16_t>& h) {
        std::vector<float> f(h.size());
        for (size_t k = 0; k < h.size(); ++k) {
            uint32_t u = (uint32_t)h[k] << 16;
            std::memcpy(&f[k], &u, 4);
        }
        return f;
    }
    std::vector<float> download_f32(int which, uint32_t i) const {
        std::vector<float> v(numel(i));
        check(ttp_download(ctx_, which, i, v.data(), v.size(), TTP_HOST));
        return v;
    }
    std::vector<uint16_t> download_u16(int which, uint32_t i) const {
        std::vector<uint16_t> v(numel(i));
        check(ttp_download(ctx_, which, i, v.data(), v.size(), TTP_HOST));
        return v;
    }

    static uint64_t next_uid() {
        static std::atomic<uint64_t> n{0};
        return ++n;
    }

    std::vector<TensorSpec> specs_;
    Mode mode_;
    uint64_t uid_ = next_uid();
    ttp_ctx* ctx_ = nullptr;
    bool capturing_ = false;
    std::weak_ptr<StepCounts> t_owner_;  // the optimizer whose step count the store holds
};

inline void Graph::launch() {
    if (store_)
        if (std::shared_ptr<StepCounts> o = owner_.lock()) store_->claim_step_count(o);
    check(ttp_graph_launch(g_));
}

}  // namespace ttp
