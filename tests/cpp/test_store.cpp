// test_store.cpp — the flat store's data paths through the C ABI: uploads and downloads of
// every buffer (host and device memory, per tensor and flat, longer than one staging piece),
// the state-record layout (ttp_buffer_layout, ttp_buffer_ptr refusals), a checkpoint round
// trip with rejection of a damaged file, and argument errors.  Also built with host-side
// AddressSanitizer/UBSan (make asan) to check the host code's memory handling.
//
// Device memory for the TTP_DEVICE transfers comes from a second context's flat grad buffer,
// so the test needs only the C ABI.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"

namespace {

uint32_t lcg(uint64_t& s) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(s >> 33);
}

std::vector<float> randn(size_t n, uint64_t seed) {  // small finite values, any sign
    std::vector<float> v(n);
    for (auto& x : v) x = ((float)(lcg(seed) & 0xFFFFFF) / 16777216.0f - 0.5f) * 0.02f;
    return v;
}

std::vector<float> download(ttp_ctx* c, int which, uint32_t i, uint64_t n) {
    std::vector<float> v(n);
    test::check(ttp_download(c, which, i, v.data(), n, TTP_HOST) == TTP_OK,
                std::string("download: ") + ttp_last_error());
    return v;
}

std::vector<uint16_t> download16(ttp_ctx* c, int which, uint32_t i, uint64_t n) {
    std::vector<uint16_t> v(n);
    test::check(ttp_download(c, which, i, v.data(), n, TTP_HOST) == TTP_OK,
                std::string("download: ") + ttp_last_error());
    return v;
}

uint16_t to_bf16(float x) {
    uint32_t u = test::bits(x);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

ttp_ctx* create(const std::vector<uint64_t>& numel, int mode) {
    std::vector<ttp_tensor_desc> d(numel.size());
    for (size_t i = 0; i < numel.size(); ++i) d[i] = {numel[i], (i % 2) ? TTP_TENSOR_DECAY : 0u, 0};
    ttp_ctx* c = nullptr;
    if (ttp_create(0, d.data(), (uint32_t)d.size(), mode, &c) != TTP_OK) {
        std::printf("FAIL: ttp_create: %s\n", ttp_last_error());
        std::exit(1);
    }
    return c;
}

void run_mode(int mode) {
    const bool mixed = mode == TTP_MODE_MIXED;
    const char* tag = mixed ? "mixed" : "fp32";
    // ragged sizes, and one tensor longer than a 16 Mi-element staging piece
    const std::vector<uint64_t> numel = {0, 1, 3, 63, 64, 65, 1000, 2049, (20ull << 20) + 7};
    ttp_ctx* c = create(numel, mode);
    uint64_t total = 0;
    test::check(ttp_flat_numel(c, &total) == TTP_OK, "flat_numel");
    std::vector<uint64_t> off(numel.size());
    for (uint32_t i = 0; i < numel.size(); ++i) ttp_tensor_info(c, i, &off[i], nullptr, nullptr);

    // weights and grads, then two Adam steps so every state buffer holds values
    for (uint32_t i = 0; i < numel.size(); ++i) {
        auto w = randn(numel[i], 100 + i);
        test::check(ttp_upload(c, TTP_BUF_MASTER, i, w.data(), w.size(), TTP_HOST) == TTP_OK,
                    std::string(tag) + " upload master: " + ttp_last_error());
        if (mixed) {
            auto p = download16(c, TTP_BUF_PARAM, i, numel[i]);
            size_t bad = 0;
            for (size_t k = 0; k < p.size(); ++k) bad += p[k] != to_bf16(w[k]);
            test::check(bad == 0, std::string(tag) + " bf16 copy of an uploaded master");
        }
        auto g = randn(numel[i], 200 + i);
        if (mixed) {
            std::vector<uint16_t> h(g.size());
            for (size_t k = 0; k < g.size(); ++k) h[k] = to_bf16(g[k]);
            ttp_upload(c, TTP_BUF_GRAD, i, h.data(), h.size(), TTP_HOST);
        } else {
            ttp_upload(c, TTP_BUF_GRAD, i, g.data(), g.size(), TTP_HOST);
        }
    }
    ttp_adam_hparams hp = {1e-3, 0.9, 0.95, 1e-8, 0.1, 1, 0, 1.0};
    for (int s = 0; s < 2; ++s)
        test::check(ttp_adam_step(c, &hp, nullptr) == TTP_OK, std::string("adam: ") + ttp_last_error());
    ttp_sgd_hparams sp = {1e-3, 0.9, 0.0, 0.0, 0, 0, 0.0};
    test::check(ttp_sgd_step(c, &sp, nullptr) == TTP_OK, std::string("sgd: ") + ttp_last_error());

    // layout: documented addressing, and pointers only for contiguous buffers
    const int state[3] = {TTP_BUF_MASTER, TTP_BUF_EXP_AVG, TTP_BUF_EXP_AVG_SQ};
    for (int which : state) {
        void* base = nullptr;
        uint32_t group = 0, stride = 0;
        test::check(ttp_buffer_layout(c, which, &base, &group, &stride) == TTP_OK, "layout");
        const uint32_t want = (which == TTP_BUF_MASTER) ? (mixed ? 192u : 64u) : (mixed ? 192u : 128u);
        test::check(group == 64 && stride == want,
                    std::string(tag) + " layout of buffer " + std::to_string(which));
        void* p = nullptr;
        const int rc = ttp_buffer_ptr(c, which, 3, &p);
        test::check(stride == 64 ? rc == TTP_OK : rc == TTP_ERR_STATE,
                    std::string(tag) + " buffer_ptr of buffer " + std::to_string(which));
    }
    for (int which : {TTP_BUF_PARAM, TTP_BUF_GRAD, TTP_BUF_MOMENTUM}) {
        void* p = nullptr;
        test::check(ttp_buffer_ptr(c, which, TTP_ALL_TENSORS, &p) == TTP_OK && p,
                    "buffer_ptr of a contiguous buffer");
    }

    // host round trips of each fp32 buffer: per tensor, then flat
    for (int which : {TTP_BUF_MASTER, TTP_BUF_EXP_AVG, TTP_BUF_EXP_AVG_SQ, TTP_BUF_MOMENTUM}) {
        const uint32_t k = 8;  // the long tensor: two staging pieces
        auto v = randn(numel[k], 300 + which);
        test::check(ttp_upload(c, which, k, v.data(), v.size(), TTP_HOST) == TTP_OK, "upload");
        test::assert_bits(download(c, which, k, numel[k]), v, std::string(tag) + " round trip");
        auto flat = download(c, which, TTP_ALL_TENSORS, total);
        std::vector<float> mid(flat.begin() + off[k], flat.begin() + off[k] + numel[k]);
        test::assert_bits(mid, v, std::string(tag) + " flat view of a tensor upload");
        auto f2 = randn(total, 400 + which);
        test::check(ttp_upload(c, which, TTP_ALL_TENSORS, f2.data(), total, TTP_HOST) == TTP_OK,
                    "flat upload");
        test::assert_bits(download(c, which, TTP_ALL_TENSORS, total), f2,
                          std::string(tag) + " flat round trip");
    }

    // device round trips through another context's flat grad buffer (fp32, `total` long)
    ttp_ctx* scratch = create({total}, TTP_MODE_FP32);
    void* dev = nullptr;
    test::check(ttp_buffer_ptr(scratch, TTP_BUF_GRAD, TTP_ALL_TENSORS, &dev) == TTP_OK && dev,
                "scratch device buffer");
    for (int which : state) {
        auto v = randn(total, 500 + which);
        ttp_upload(scratch, TTP_BUF_GRAD, TTP_ALL_TENSORS, v.data(), total, TTP_HOST);
        ttp_sync(scratch);
        test::check(ttp_upload(c, which, TTP_ALL_TENSORS, dev, total, TTP_DEVICE) == TTP_OK,
                    "device upload");
        ttp_sync(c);  // the upload reads `dev` on c's stream; the fill below is on scratch's
        ttp_zero_grad(scratch, 0);
        ttp_sync(scratch);
        test::check(ttp_download(c, which, TTP_ALL_TENSORS, dev, total, TTP_DEVICE) == TTP_OK,
                    "device download");
        ttp_sync(c);
        test::assert_bits(download(scratch, TTP_BUF_GRAD, TTP_ALL_TENSORS, total), v,
                          std::string(tag) + " device round trip");
    }
    ttp_destroy(scratch);

    // checkpoint: save, load into a fresh context, every buffer and the counters equal
    const std::string path = std::string("/tmp/ttp_test_store_") + tag + ".bin";
    test::check(ttp_adam_step(c, &hp, nullptr) == TTP_OK, "adam before save");
    test::check(ttp_save_state(c, path.c_str()) == TTP_OK, std::string("save: ") + ttp_last_error());
    ttp_ctx* d = create(numel, mode);
    test::check(ttp_load_state(d, path.c_str()) == TTP_OK, std::string("load: ") + ttp_last_error());
    for (int which : {TTP_BUF_MASTER, TTP_BUF_EXP_AVG, TTP_BUF_EXP_AVG_SQ, TTP_BUF_MOMENTUM})
        test::assert_bits(download(d, which, TTP_ALL_TENSORS, total),
                          download(c, which, TTP_ALL_TENSORS, total),
                          std::string(tag) + " checkpoint buffer " + std::to_string(which));
    if (mixed) {
        auto a = download16(c, TTP_BUF_PARAM, TTP_ALL_TENSORS, total);
        auto b = download16(d, TTP_BUF_PARAM, TTP_ALL_TENSORS, total);
        test::check(a == b, "checkpoint restores the bf16 copy");
    }
    uint64_t t1 = 0, t2 = 0;
    ttp_get_step(c, &t1);
    ttp_get_step(d, &t2);
    test::check(t1 == 4 && t2 == 4, "checkpoint step count (three Adam steps and one SGD step)");
    // a damaged file is rejected: flip one byte in the middle
    {
        FILE* f = std::fopen(path.c_str(), "r+b");
        std::fseek(f, 0, SEEK_END);
        const long size = std::ftell(f);
        std::fseek(f, size / 2, SEEK_SET);
        int ch = std::fgetc(f);
        std::fseek(f, size / 2, SEEK_SET);
        std::fputc(ch ^ 0x40, f);
        std::fclose(f);
    }
    test::check(ttp_load_state(d, path.c_str()) == TTP_ERR_INVALID, "damaged checkpoint rejected");
    std::remove(path.c_str());

    // argument errors
    std::vector<float> one(5);
    test::check(ttp_upload(c, TTP_BUF_MASTER, 2, one.data(), 5, TTP_HOST) == TTP_ERR_RANGE,
                "wrong element count");
    test::check(ttp_download(c, TTP_BUF_MASTER, 99, one.data(), 1, TTP_HOST) == TTP_ERR_RANGE,
                "tensor index out of range");
    test::check(ttp_buffer_layout(c, 17, nullptr, nullptr, nullptr) == TTP_ERR_INVALID,
                "unknown buffer id");
    ttp_destroy(d);
    ttp_destroy(c);
}

// The SGD layout of a MIXED store (TTP_STORE_SGD): a contiguous master and no m / v.  Master
// uploads keep the bf16 copy; plain and momentum SGD steps give w - lr*g and torch's first
// momentum step; the first use of m / v converts the store to the record layout with the
// master unchanged, and that conversion is refused while capturing and while graphs live.
void run_sgd_layout() {
    const std::vector<uint64_t> numel = {0, 1, 3, 63, 64, 65, 1000, 2049, 100003};
    ttp_ctx* c = create(numel, TTP_MODE_MIXED | TTP_STORE_SGD);
    int mode = -1;
    test::check(ttp_mode(c, &mode) == TTP_OK && mode == TTP_MODE_MIXED,
                "ttp_mode reports the precision mode of an SGD-layout store");
    uint64_t total = 0;
    ttp_flat_numel(c, &total);
    std::vector<uint64_t> off(numel.size());
    for (uint32_t i = 0; i < numel.size(); ++i) ttp_tensor_info(c, i, &off[i], nullptr, nullptr);
    void* base = nullptr;
    uint32_t group = 0, stride = 0;
    test::check(ttp_buffer_layout(c, TTP_BUF_MASTER, &base, &group, &stride) == TTP_OK &&
                    group == 64 && stride == 64,
                "SGD layout: the master is contiguous");
    void* p3 = nullptr;
    test::check(ttp_buffer_ptr(c, TTP_BUF_MASTER, 3, &p3) == TTP_OK &&
                    p3 == (char*)base + off[3] * 4,
                "SGD layout: master pointer of a tensor");
    std::vector<std::vector<float>> w(numel.size()), g(numel.size());
    for (uint32_t i = 0; i < numel.size(); ++i) {
        w[i] = randn(numel[i], 700 + i);
        g[i] = randn(numel[i], 800 + i);
        test::check(ttp_upload(c, TTP_BUF_MASTER, i, w[i].data(), w[i].size(), TTP_HOST) == TTP_OK,
                    std::string("sgd layout upload master: ") + ttp_last_error());
        auto p = download16(c, TTP_BUF_PARAM, i, numel[i]);
        size_t bad = 0;
        for (size_t k = 0; k < p.size(); ++k) bad += p[k] != to_bf16(w[i][k]);
        test::check(bad == 0, "SGD layout: bf16 copy of an uploaded master");
        std::vector<uint16_t> h(numel[i]);
        for (size_t k = 0; k < h.size(); ++k) {
            h[k] = to_bf16(g[i][k]);
            const uint32_t u = (uint32_t)h[k] << 16;
            std::memcpy(&g[i][k], &u, 4);  // the gradient value the store holds
        }
        ttp_upload(c, TTP_BUF_GRAD, i, h.data(), h.size(), TTP_HOST);
    }
    // plain SGD: w - (g*lr), rounded after the multiply and after the subtract
    const float lr = 0.01f;
    ttp_sgd_hparams plain = {lr, 0.0, 0.0, 0.0, 0, 0, 0.0};
    test::check(ttp_sgd_step(c, &plain, nullptr) == TTP_OK, std::string("sgd: ") + ttp_last_error());
    for (uint32_t i = 0; i < numel.size(); ++i)
        for (size_t k = 0; k < w[i].size(); ++k) {
            const float update = g[i][k] * lr;
            w[i][k] = w[i][k] - update;
        }
    for (uint32_t i = 0; i < numel.size(); ++i)
        test::assert_bits(download(c, TTP_BUF_MASTER, i, numel[i]), w[i],
                          "SGD layout: plain step, tensor " + std::to_string(i));
    // momentum 0.9: the first step stores buf = g and applies w - buf*lr
    ttp_sgd_hparams mom = {lr, 0.9, 0.0, 0.0, 0, 0, 0.0};
    test::check(ttp_sgd_step(c, &mom, nullptr) == TTP_OK, std::string("sgd m: ") + ttp_last_error());
    for (uint32_t i = 0; i < numel.size(); ++i) {
        for (size_t k = 0; k < w[i].size(); ++k) {
            const float update = g[i][k] * lr;
            w[i][k] = w[i][k] - update;
        }
        test::assert_bits(download(c, TTP_BUF_MASTER, i, numel[i]), w[i],
                          "SGD layout: first momentum step, tensor " + std::to_string(i));
        test::assert_bits(download(c, TTP_BUF_MOMENTUM, i, numel[i]), g[i],
                          "SGD layout: first momentum buffer, tensor " + std::to_string(i));
        auto p = download16(c, TTP_BUF_PARAM, i, numel[i]);
        size_t bad = 0;
        for (size_t k = 0; k < p.size(); ++k) bad += p[k] != to_bf16(w[i][k]);
        test::check(bad == 0, "SGD layout: bf16 weights after the steps");
    }

    // the conversion is refused while capturing and while a graph lives
    test::check(ttp_capture_begin(c) == TTP_OK, "capture begin");
    ttp_adam_hparams hp = {1e-3, 0.9, 0.95, 1e-8, 0.1, 1, 0, 0.0};
    test::check(ttp_adam_step(c, &hp, nullptr) == TTP_ERR_STATE, "no conversion while capturing");
    test::check(ttp_sgd_step(c, &plain, nullptr) == TTP_OK, "capture an SGD step");
    ttp_graph* graph = nullptr;
    test::check(ttp_capture_end(c, &graph) == TTP_OK && graph, "capture end");
    test::check(ttp_buffer_layout(c, TTP_BUF_EXP_AVG, nullptr, nullptr, nullptr) == TTP_ERR_STATE,
                "no conversion while a graph lives");
    test::check(ttp_adam_step_noalloc(c, &hp, nullptr, 0) == TTP_ERR_STATE,
                "the no-allocation step does not convert");
    test::check(ttp_graph_launch(graph) == TTP_OK, "graph launch");
    for (uint32_t i = 0; i < numel.size(); ++i)
        for (size_t k = 0; k < w[i].size(); ++k) {
            const float update = g[i][k] * lr;
            w[i][k] = w[i][k] - update;
        }
    test::check(ttp_graph_destroy(graph) == TTP_OK, "graph destroy");
    ttp_buffer_layout(c, TTP_BUF_MASTER, nullptr, &group, &stride);
    test::check(stride == 64, "a refused conversion leaves the SGD layout");

    // asking for m converts: master and bf16 weights unchanged, m and v zero
    const auto p16_before = download16(c, TTP_BUF_PARAM, TTP_ALL_TENSORS, total);
    test::check(ttp_buffer_layout(c, TTP_BUF_EXP_AVG, nullptr, &group, &stride) == TTP_OK &&
                    stride == 192,
                std::string("conversion on first use of m: ") + ttp_last_error());
    ttp_buffer_layout(c, TTP_BUF_MASTER, nullptr, &group, &stride);
    test::check(stride == 192, "after the conversion the master sits in the records");
    for (uint32_t i = 0; i < numel.size(); ++i)
        test::assert_bits(download(c, TTP_BUF_MASTER, i, numel[i]), w[i],
                          "conversion keeps the master, tensor " + std::to_string(i));
    test::check(download16(c, TTP_BUF_PARAM, TTP_ALL_TENSORS, total) == p16_before,
                "conversion keeps the bf16 weights");
    test::assert_bits(download(c, TTP_BUF_EXP_AVG_SQ, TTP_ALL_TENSORS, total),
                      std::vector<float>(total, 0.0f), "conversion: v starts at zero");
    test::check(ttp_adam_step(c, &hp, nullptr) == TTP_OK, std::string("adam: ") + ttp_last_error());
    ttp_destroy(c);
}

// ttp_accumulate_grad_multi against one ttp_accumulate_grad per tensor: an assign round, then
// an add round with sums, from fp32 device sources (the grads of an FP32 context of the same
// table), into a MIXED store and its twin; the gradients and flags match bit for bit, and
// the steps from the sums give the same state.  Duplicate indices and more than
// TTP_ACCUM_MULTI_MAX tensors are refused.
void run_multi_accumulate() {
    const std::vector<uint64_t> numel = {3000, 1, 2 * 8192 + 5, 0, 777, 8192};
    const uint64_t n = numel.size();
    ttp_ctx* src = create(numel, TTP_MODE_FP32);
    ttp_ctx* a = create(numel, TTP_MODE_MIXED);
    ttp_ctx* b = create(numel, TTP_MODE_MIXED);
    std::vector<uint32_t> idx;
    std::vector<const void*> ptr;
    for (uint32_t i = (uint32_t)n; i-- > 0;) {  // a backward's order
        idx.push_back(i);
        void* p = nullptr;
        test::check(ttp_buffer_ptr(src, TTP_BUF_GRAD, i, &p) == TTP_OK, "source pointer");
        ptr.push_back(p);
    }
    ttp_adam_hparams hp{};
    hp.lr = 1e-3;
    hp.beta1 = 0.9;
    hp.beta2 = 0.95;
    hp.eps = 1e-8;
    hp.weight_decay = 0.1;
    hp.decoupled = 1;
    hp.max_grad_norm = 0.5;
    hp.flags = TTP_STEP_TENSOR_SUMS;
    for (int round = 0; round < 2; ++round) {
        for (uint32_t i = 0; i < n; ++i) {
            auto v = randn(numel[i], 900 + 10 * round + i);
            if (numel[i])
                test::check(ttp_upload(src, TTP_BUF_GRAD, i, v.data(), v.size(), TTP_HOST) == TTP_OK,
                            "source upload");
        }
        const int dtype = TTP_DTYPE_F32 | (round ? TTP_ACCUM_SUMSQ : 0);
        test::check(ttp_accumulate_grad_multi(a, idx.data(), ptr.data(), (uint32_t)n, dtype) ==
                        TTP_OK,
                    std::string("multi accumulate: ") + ttp_last_error());
        for (uint32_t k = 0; k < n; ++k)
            test::check(ttp_accumulate_grad(b, idx[k], ptr[k], numel[idx[k]], dtype,
                                            TTP_DEVICE) == TTP_OK,
                        std::string("accumulate: ") + ttp_last_error());
        uint64_t total = 0;
        ttp_flat_numel(a, &total);
        test::check(download16(a, TTP_BUF_GRAD, TTP_ALL_TENSORS, total) ==
                        download16(b, TTP_BUF_GRAD, TTP_ALL_TENSORS, total),
                    "multi accumulate = per-tensor accumulates, round " + std::to_string(round));
        for (uint32_t i = 0; i < n; ++i) {
            int ha = 0, hb = 0;
            ttp_get_has_grad(a, i, &ha);
            ttp_get_has_grad(b, i, &hb);
            test::check(ha == 1 && hb == 1, "has-grad flags after the accumulates");
        }
    }
    ttp_step_report ra{}, rb{};
    test::check(ttp_adam_step(a, &hp, &ra) == TTP_OK && ttp_adam_step(b, &hp, &rb) == TTP_OK,
                std::string("steps from the sums: ") + ttp_last_error());
    test::check(ra.grad_norm == rb.grad_norm && ra.grad_norm > 0, "the same norm from the sums");
    uint64_t total = 0;
    ttp_flat_numel(a, &total);
    test::assert_bits(download(a, TTP_BUF_MASTER, TTP_ALL_TENSORS, total),
                      download(b, TTP_BUF_MASTER, TTP_ALL_TENSORS, total), "the same master");
    // zero_grad to None without the fill: the flags go, the memory stays, and the next
    // accumulates assign, as after the filling zero_grad
    const auto kept = download16(a, TTP_BUF_GRAD, TTP_ALL_TENSORS, total);
    test::check(ttp_zero_grad(a, 1 | TTP_ZERO_NO_FILL) == TTP_OK && ttp_zero_grad(b, 1) == TTP_OK,
                std::string("zero_grad: ") + ttp_last_error());
    test::check(download16(a, TTP_BUF_GRAD, TTP_ALL_TENSORS, total) == kept,
                "zero_grad without the fill leaves the gradients");
    for (uint32_t i = 0; i < n; ++i) {
        int ha = 1;
        ttp_get_has_grad(a, i, &ha);
        test::check(ha == 0, "zero_grad without the fill clears the has-grad flags");
    }
    test::check(ttp_zero_grad(a, TTP_ZERO_NO_FILL) == TTP_ERR_INVALID,
                "the fill is skipped only for gradients set to None");
    test::check(ttp_accumulate_grad_multi(a, idx.data(), ptr.data(), (uint32_t)n, TTP_DTYPE_F32) ==
                        TTP_OK &&
                    ttp_accumulate_grad_multi(b, idx.data(), ptr.data(), (uint32_t)n,
                                              TTP_DTYPE_F32) == TTP_OK,
                std::string("accumulates after zero_grad: ") + ttp_last_error());
    test::check(download16(a, TTP_BUF_GRAD, TTP_ALL_TENSORS, total) ==
                    download16(b, TTP_BUF_GRAD, TTP_ALL_TENSORS, total),
                "accumulates after zero_grad with and without the fill");
    // refusals
    std::vector<uint32_t> dup = {0, 2, 0};
    std::vector<const void*> dptr = {ptr[n - 1], ptr[n - 3], ptr[n - 1]};
    test::check(ttp_accumulate_grad_multi(a, dup.data(), dptr.data(), 3, TTP_DTYPE_F32) ==
                    TTP_ERR_INVALID,
                "an index listed twice is refused");
    std::vector<uint32_t> many(TTP_ACCUM_MULTI_MAX + 1, 0);
    std::vector<const void*> mptr(many.size(), ptr[0]);
    test::check(ttp_accumulate_grad_multi(a, many.data(), mptr.data(), (uint32_t)many.size(),
                                          TTP_DTYPE_F32) == TTP_ERR_RANGE,
                "more than TTP_ACCUM_MULTI_MAX tensors are refused");
    ttp_destroy(a);
    ttp_destroy(b);
    ttp_destroy(src);
}

}  // namespace

int main() {
    test::DeviceGuard guard;
    // first: the ASan build's allocator then ends the process in the same state as without
    // this section (device chunks it still holds at exit are freed after the HIP runtime)
    run_sgd_layout();
    run_mode(TTP_MODE_MIXED);
    run_mode(TTP_MODE_FP32);
    run_multi_accumulate();
    // a table past the 2^40-element bound is refused before any allocation
    ttp_tensor_desc big[2] = {{1ull << 40, 0, 0}, {64, 0, 0}};
    ttp_ctx* c = nullptr;
    test::check(ttp_create(0, big, 2, TTP_MODE_MIXED, &c) == TTP_ERR_INVALID && !c,
                "oversized table rejected");
    return test::finish("test_store");
}
