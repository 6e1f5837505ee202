// ttperf.hip — host side of libttperf_hip: the C ABI declared in include/ttperf/ttperf.h.
//
// A context is one flat parameter store on one device plus the state of one optimizer:
//   * layout: tensors in caller order, each starting on a 64-element boundary (256 B for
//     fp32, 128 B for bf16), so every lane's 4-element vector stays inside one tensor's
//     footprint; the padding is zero and never written by a step;
//   * optimizer state in records of 64-element slots (ttp::kRec): MIXED mode keeps master,
//     m and v of each 64-element group in one [master|m|v] record, allocated with the store
//     (in its SGD layout, TTP_STORE_SGD, a contiguous master and no m / v until the first
//     Adam step converts it); FP32 mode keeps its contiguous master (the model-facing
//     weights) and puts m and v in [m|v] records on first Adam use.  Momentum and the
//     model-facing buffers are contiguous.
//     Uploads, downloads and checkpoints convert between records and contiguous arrays;
//   * work table: chunks of <= kChunk (1024) elements of one tensor.  The table of all
//     tensors is built once; a second table is built only while some tensor has no grad
//     (py/optim.py:56-57 skip);
//   * step: [norm pass (partials + finalize) when clipping or loss scaling] + one fused
//     update pass, all on the context's stream, no host synchronisation (the skip decision
//     and, with loss scaling, the step count live on the device).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "ttperf/ttperf.h"
#include "kernels.hpp"

using ttp::Chunk;
using ttp::DevState;

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

// A failed HIP call returns TTP_ERR_OOM for an allocation that did not fit, else TTP_ERR_HIP.
// Its error is also left in HIP's per-thread "last error", which clear_hip_error() resets.
#define HIP_TRY(expr)                                                                  \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess) {                                                        \
            (void)hipGetLastError();                                                   \
            return fail(e_ == hipErrorOutOfMemory ? TTP_ERR_OOM : TTP_ERR_HIP,         \
                        std::string(#expr) + ": " + hipGetErrorString(e_));            \
        }                                                                              \
    } while (0)

// Kernel launches report their errors through hipGetLastError(), which returns the last
// error of any earlier HIP call on this thread (the caller's or torch's included).  It is
// reset before each launch, so that the check after it sees that launch's error only.
inline void clear_hip_error() { (void)hipGetLastError(); }

constexpr uint64_t kAlign = 64;  // elements
// Largest store: 2^40 elements (4 TiB of fp32 per buffer, far beyond one GPU's 288 GB), so the
// padded sizes and byte counts computed from it never wrap in 64 bits.
constexpr uint64_t kMaxElems = 1ull << 40;

uint64_t env_u64(const char* name, uint64_t dflt) {
    const char* s = std::getenv(name);
    if (!s || !*s) return dflt;
    char* end = nullptr;
    unsigned long long v = std::strtoull(s, &end, 10);
    return (end && *end == 0) ? (uint64_t)v : dflt;
}

struct TensorRec {
    uint64_t offset, numel;
    uint32_t flags;
    int has_grad;
};

struct EventPair {
    hipEvent_t a, b;
};

// Device work tables of one active tensor set: the update pass walks `chunks` (<= kChunk
// elements of one tensor each), the norm pass walks `tiles` (<= 16 KiB of gradients each).
struct WorkTables {
    Chunk* chunks = nullptr;
    uint32_t n_chunks = 0;
    Chunk* tiles = nullptr;
    uint32_t n_tiles = 0;
    uint64_t elems = 0;  // elements the chunks cover
    // the set's tensors in order, and where each one's tiles start (n_tensors + 1 entries):
    // per-tensor gradient sums (ttp_grad_sumsq_tensors, TTP_STEP_TENSOR_SUMS)
    uint32_t* tensor_ids = nullptr;
    uint32_t* tile_start = nullptr;
    uint32_t n_tensors = 0;
};

// Gradient bytes up to which MI355X's Infinity Cache (256 MB) still holds most of the
// gradients after the norm pass or the backward that wrote them.  The update's form is chosen
// on each side of it (see kLaneAdamMixed), and the norm pass reads about this many bytes of
// the last tiles with cached loads, the rest non-temporal (see NormSplit).
constexpr uint64_t kCachedGradBytes = 256ull << 20;

}  // namespace

// Norm-pass partials of ttp_adam_step_noalloc, the step entry point that allocates nothing: a
// fixed array of the library, one copy on each device, held until the process ends.  Host code
// never uses its name as an address: ttp_create looks up each device's copy once
// (hipGetSymbolAddress, with that device current) and the kernels take that pointer.  Every
// no-allocation step on a device shares the array, so such steps of different contexts must
// not overlap on one device.
constexpr uint32_t kNoAllocPartials = 8192;  // 64 KiB: one fp64 partial per norm-pass block
static __device__ __align__(256) double scratch[kNoAllocPartials];

namespace {

// Per device: its copy of `scratch`, and the stream and an event of the last eager
// no-allocation step, so that one on another stream (another context) waits for it instead
// of overwriting partials it has not consumed yet.  Both are made at ttp_create, so a step
// allocates nothing.
struct ScratchDev {
    double* ptr = nullptr;
    hipEvent_t done = nullptr;      // recorded after each eager no-allocation step
    hipStream_t last = nullptr;     // the stream it was recorded on
    bool used = false;
};
std::mutex g_scratch_mu;
std::map<int, ScratchDev> g_scratch;  // device -> its scratch array and ordering

// Called with `device` current: finds this device's copy of the scratch array once.
int ensure_scratch(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch.count(device)) return TTP_OK;
    ScratchDev d;
    HIP_TRY(hipGetSymbolAddress((void**)&d.ptr, HIP_SYMBOL(scratch)));
    HIP_TRY(hipEventCreateWithFlags(&d.done, hipEventDisableTiming));
    g_scratch[device] = d;
    return TTP_OK;
}

}  // namespace

struct ttp_ctx {
    int device = 0;
    int mode = TTP_MODE_FP32;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    int num_cus = 256;

    std::vector<TensorRec> tensors;
    uint64_t total = 0;

    void* param = nullptr;  // bf16 (MIXED) or == master (FP32)
    void* grad = nullptr;   // bf16 (MIXED) or fp32 (FP32)
    // slot bases (see buffer_stride): MIXED, the three slots of `records`; FP32 and the
    // MIXED SGD layout, the contiguous master and the two slots of `records` (null until the
    // first Adam use)
    float* master = nullptr;
    float* exp_avg = nullptr;
    float* exp_avg_sq = nullptr;
    float* records = nullptr;   // the state record array (the allocation)
    // MIXED store in the SGD layout (TTP_STORE_SGD): `master` is its own contiguous
    // allocation and `records` does not exist; cleared by the conversion of the first Adam use
    bool sgd_layout = false;
    float* momentum = nullptr;  // contiguous
    uint32_t* mom_init = nullptr;        // device, per tensor
    std::vector<uint8_t> host_mom_init;  // host view (exact while loss scaling is off)

    DevState* st = nullptr;
    double* partials = nullptr;
    uint32_t partials_cap = 0;

    uint32_t norm_grid_cap = 0;  // blocks of the norm pass (one partial each)
    uint32_t upd_lds = 0;        // dynamic LDS per update block (caps blocks per CU)
    uint64_t lane_launch_cap = 0;  // most blocks per lane-form launch (0: the grid limit)

    WorkTables all;  // every non-empty tensor
    uint32_t n_nonempty = 0;
    // tables of other active sets (a subset, or tensors without grad left out), keyed by
    // the sorted active tensor indices
    std::map<std::vector<uint32_t>, WorkTables> tables;

    void* staging = nullptr;  // device copy of a host gradient for ttp_accumulate_grad
    uint64_t staging_bytes = 0;

    // per-tensor sums of squares of the unscaled gradients (ttp_grad_sumsq_tensors) and
    // whether each is current (host view: cleared by any gradient write through the ABI, a
    // change of the loss scale, and every step)
    double* tsum = nullptr;
    std::vector<uint8_t> tsum_fresh;
    // while capturing: which per-tensor host flags the captured calls changed (kCapFresh,
    // kCapGrad bits), the flags at ttp_capture_begin, and the sums a captured step reads that
    // predate the capture
    std::vector<uint8_t> cap_touched, cap_fresh0, cap_grad0, cap_needs;
    double* tile_sums = nullptr;  // one per norm tile of a ttp_grad_sumsq_tensors call
    uint32_t tile_sums_cap = 0;
    // accumulates with their sums (TTP_ACCUM_SUMSQ): per norm tile of the store, one partial
    // per wave (tensor i's from kWaves x tile_base[i]), and per tensor whether they are still to be
    // combined into tsum (device flags; the next step from sums combines them).  acc_sums_used
    // is set by the first such accumulate: eager steps from sums combine from then on,
    // captured ones always
    double* acc_tiles = nullptr;
    uint32_t* tile_base = nullptr;
    std::vector<uint32_t> host_tile_base;
    uint32_t* tsum_pending = nullptr;
    bool acc_sums_used = false;
    std::vector<void*> retired;   // replaced buffers that live graphs may still write

    // bias-correction tables of every betas pair stepped with (kept, since captured graphs
    // and queued steps read them) and the current pair's
    std::map<std::pair<double, double>, std::pair<float*, uint32_t>> bias_tables;
    float* bias_tab = nullptr;
    uint32_t bias_len = 0;

    ttp_scaler_config scaler{0, 2000, 65536.0, 2.0, 0.5};
    uint64_t host_t = 0;     // step count while it lives on the host (see dev_t)
    bool device_t = false;   // set once the context has been captured: t stays on the device
    bool capturing = false;  // between ttp_capture_begin and ttp_capture_end
    uint32_t n_graphs = 0;   // live graphs; the buffers and tables they reference stay put

    bool timing = false;
    std::vector<EventPair> ev[2];
    std::vector<hipEvent_t> ev_pool;
};

struct ttp_graph {
    ttp_ctx* ctx;
    hipGraph_t graph;
    hipGraphExec_t exec;
    // what a launch does to the per-tensor host flags (whether a gradient exists, whether its
    // sum is current): the flags each tensor that a captured call changed ended the capture with
    struct FlagEffect {
        uint32_t tensor;
        uint8_t mask, fresh, has_grad;
    };
    std::vector<FlagEffect> effects;
    // tensors whose sums a captured step reads without a captured sums call before it: they
    // must be current at each launch
    std::vector<uint32_t> needs_fresh;
};

namespace {

// MIXED and BF16 stores hold bf16 gradients (and bf16 weights in PARAM); FP32 stores fp32
bool bf16_grads(const ttp_ctx* c) { return c->mode != TTP_MODE_FP32; }
size_t grad_esize(const ttp_ctx* c) { return bf16_grads(c) ? 2 : 4; }

// The step count (bias-correction t) lives on the device while loss scaling is on (the
// device decides whether a step is skipped) and once the context has been captured (a
// replayed graph cannot update host state); otherwise on the host.
bool t_on_device(const ttp_ctx* c) { return c->scaler.enabled || c->device_t; }

int no_capture(const ttp_ctx* c, const char* what) {
    if (!c->capturing) return TTP_OK;
    return fail(TTP_ERR_STATE, std::string(what) + " is not allowed while capturing a graph");
}
size_t param_esize(const ttp_ctx* c) { return bf16_grads(c) ? 2 : 4; }

uint32_t norm_tile(const ttp_ctx* c) {
    return bf16_grads(c) ? ttp::norm_tile_elems<uint16_t>() : ttp::norm_tile_elems<float>();
}

// A TTP_MODE_BF16 store holds its bf16 weights (PARAM) and gradients (GRAD) and no fp32
// state: the other buffers, and every call that would create them, are refused.
int bf16_store_refuses(const ttp_ctx* c, const char* what) {
    if (c->mode != TTP_MODE_BF16) return TTP_OK;
    return fail(TTP_ERR_INVALID, std::string(what) +
                                     ": a TTP_MODE_BF16 store holds bf16 weights and gradients "
                                     "only (no fp32 master, moments or momentum); create the "
                                     "store TTP_MODE_MIXED for fp32 optimizer state");
}

// pieces of <= `piece` elements of each listed non-empty tensor, in tensor order
void append_pieces(const ttp_ctx* c, const std::vector<uint32_t>& which, uint64_t piece,
                   std::vector<Chunk>& out) {
    for (uint32_t i : which) {
        const TensorRec& t = c->tensors[i];
        for (uint64_t b = 0; b < t.numel; b += piece) {
            Chunk ch;
            ch.begin = t.offset + b;
            ch.count = (uint32_t)std::min<uint64_t>(piece, t.numel - b);
            ch.meta = (t.flags & TTP_TENSOR_DECAY ? ttp::kChunkDecay : 0u) | ((uint32_t)i << 8);
            out.push_back(ch);
        }
    }
}

int upload_table(const std::vector<Chunk>& v, Chunk** d, uint32_t* n) {
    if (v.size() > 0xFFFFFFFFull) return fail(TTP_ERR_INVALID, "too many chunks");
    HIP_TRY(hipMalloc((void**)d, std::max<size_t>(v.size(), 1) * sizeof(Chunk)));
    if (!v.empty())
        HIP_TRY(hipMemcpy(*d, v.data(), v.size() * sizeof(Chunk), hipMemcpyHostToDevice));
    *n = (uint32_t)v.size();
    return TTP_OK;
}

int upload_u32(const std::vector<uint32_t>& v, uint32_t** d) {
    HIP_TRY(hipMalloc((void**)d, std::max<size_t>(v.size(), 1) * sizeof(uint32_t)));
    if (!v.empty())
        HIP_TRY(hipMemcpy(*d, v.data(), v.size() * sizeof(uint32_t), hipMemcpyHostToDevice));
    return TTP_OK;
}

int build_tables(const ttp_ctx* c, const std::vector<uint32_t>& which, WorkTables* w) {
    std::vector<Chunk> v;
    append_pieces(c, which, ttp::kChunk, v);
    w->elems = 0;
    for (const Chunk& ch : v) w->elems += ch.count;
    int rc = upload_table(v, &w->chunks, &w->n_chunks);
    if (rc) return rc;
    v.clear();
    append_pieces(c, which, norm_tile(c), v);
    if ((rc = upload_table(v, &w->tiles, &w->n_tiles))) return rc;
    // tiles are appended tensor by tensor, so each tensor's tiles are one run of the table
    std::vector<uint32_t> start(1, 0);
    for (uint32_t i : which) {
        const uint64_t tiles = (c->tensors[i].numel + norm_tile(c) - 1) / norm_tile(c);
        start.push_back(start.back() + (uint32_t)tiles);
    }
    w->n_tensors = (uint32_t)which.size();
    if ((rc = upload_u32(which, &w->tensor_ids))) return rc;
    return upload_u32(start, &w->tile_start);
}

void free_tables(WorkTables& w) {
    if (w.chunks) (void)hipFree(w.chunks);
    if (w.tiles) (void)hipFree(w.tiles);
    if (w.tensor_ids) (void)hipFree(w.tensor_ids);
    if (w.tile_start) (void)hipFree(w.tile_start);
    w = WorkTables{};
}

// The per-tensor host flags (a gradient exists; its sum is current) change only through these
// three, which also note, while a capture runs, what it changed: nothing captured runs before
// a launch, so ttp_capture_end restores the flags and each launch applies the change.
constexpr uint8_t kCapFresh = 1, kCapGrad = 2;
void stale_sums(ttp_ctx* c) {
    std::fill(c->tsum_fresh.begin(), c->tsum_fresh.end(), 0);
    if (c->capturing)
        for (uint8_t& m : c->cap_touched) m |= kCapFresh;
}
void set_fresh(ttp_ctx* c, uint32_t i, bool fresh) {
    c->tsum_fresh[i] = fresh ? 1 : 0;
    if (c->capturing) c->cap_touched[i] |= kCapFresh;
}
void set_grad_flag(ttp_ctx* c, uint32_t i, bool has) {
    c->tensors[i].has_grad = has ? 1 : 0;
    if (c->capturing) c->cap_touched[i] |= kCapGrad;
}

// TTP_STEP_TENSOR_SUMS: every tensor the step updates needs a current sum.  A step being
// captured notes the sums it reads from before the capture: each launch checks them.
int check_sums_current(ttp_ctx* c, const std::vector<uint32_t>& active) {
    for (uint32_t i : active)
        if (!c->tsum_fresh[i])
            return fail(TTP_ERR_STATE, "tensor " + std::to_string(i) +
                                           " has no current gradient sum: call "
                                           "ttp_grad_sumsq_tensors (or accumulate its gradient "
                                           "with TTP_ACCUM_SUMSQ) after its last gradient write, "
                                           "after the last step that updated it and after the "
                                           "last change of the loss scale");
    if (c->capturing)
        for (uint32_t i : active)
            if (!(c->cap_touched[i] & kCapFresh)) c->cap_needs[i] = 1;
    return TTP_OK;
}

// The per-tile sums buffer of ttp_grad_sumsq_tensors and of accumulates with their sums, grown
// to `tiles` entries (at least one); `what` names the call in the refusal while capturing.
int ensure_tile_sums(ttp_ctx* c, uint32_t tiles, const char* what) {
    tiles = std::max<uint32_t>(tiles, 1);
    if (tiles <= c->tile_sums_cap) return TTP_OK;
    int rc;
    if ((rc = no_capture(c, (std::string(what) + " (allocates)").c_str()))) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));  // queued calls may still use the old buffer
    if (c->tile_sums) {
        if (c->n_graphs)
            c->retired.push_back(c->tile_sums);  // a captured call may write it on replay
        else
            HIP_TRY(hipFree(c->tile_sums));
    }
    c->tile_sums = nullptr;
    c->tile_sums_cap = 0;
    HIP_TRY(hipMalloc((void**)&c->tile_sums, (size_t)tiles * sizeof(double)));
    c->tile_sums_cap = tiles;
    return TTP_OK;
}

// After a step: the stepped tensors' sums are spent (their gradients were consumed).  A step
// that updates the loss scale also makes every other sum stale, since those are of gradients
// unscaled by the old scale; a step that defers the update leaves the other tensors' sums
// current for the iteration's other optimizers.
void consume_sums(ttp_ctx* c, const std::vector<uint32_t>& active, bool scale_moves) {
    if (scale_moves) {
        stale_sums(c);
        return;
    }
    for (uint32_t i : active) set_fresh(c, i, false);
}

constexpr int32_t kStepFlags = TTP_STEP_TENSOR_SUMS | TTP_STEP_DEFER_SCALE;

int zero_device(ttp_ctx* c, void* p, uint64_t bytes) {
    // a fill kernel rather than a memset node, so the step sequence stays capturable
    if (!bytes) return TTP_OK;
    const uint64_t words = (bytes + 3) / 4;
    const uint32_t grid = (uint32_t)std::min<uint64_t>((words + ttp::kBlock - 1) / ttp::kBlock,
                                                       (uint64_t)c->num_cus * 16);
    clear_hip_error();
    hipLaunchKernelGGL(ttp::fill_zero_kernel, dim3(grid), dim3(ttp::kBlock), 0, c->stream,
                       (uint32_t*)p, words);
    HIP_TRY(hipGetLastError());
    return TTP_OK;
}

int alloc_zero(ttp_ctx* c, void** p, uint64_t bytes) {
    // padded to whole 4-byte words for the fill kernel
    HIP_TRY(hipMalloc(p, std::max<uint64_t>((bytes + 3) / 4 * 4, 4)));
    return zero_device(c, *p, bytes);
}

// blocks of a grid-stride elementwise kernel over n elements: at most 16 per CU
uint32_t elementwise_grid(const ttp_ctx* c, uint64_t n) {
    return (uint32_t)std::max<uint64_t>(
        1, std::min<uint64_t>((n + ttp::kBlock - 1) / ttp::kBlock, (uint64_t)c->num_cus * 16));
}

int ensure_adam_state(ttp_ctx* c) {
    // py/optim.py:58-71: m and v start as zeros on first use.  MIXED mode allocates them
    // (zero) with the master in its records at ttp_create; FP32 mode allocates the [m|v]
    // records here; a MIXED store in the SGD layout is converted to the [master|m|v] records
    // here (the master's values move unchanged, the bf16 weights stay as they are).
    if (c->exp_avg) return TTP_OK;
    int rc;
    if ((rc = bf16_store_refuses(c, "Adam's m and v"))) return rc;
    if ((rc = no_capture(c, "first Adam step (allocates m, v)"))) return rc;
    if (c->mode == TTP_MODE_MIXED && c->sgd_layout) {
        if (c->n_graphs)
            return fail(TTP_ERR_STATE, "the first Adam use of a store in the SGD layout moves "
                                       "its master into new state records, and live graphs "
                                       "of this context hold the old master's address: "
                                       "destroy them first");
        float* rec = nullptr;
        if ((rc = alloc_zero(c, (void**)&rec, c->total * 4 * 3))) {
            if (rec) (void)hipFree(rec);
            return rc;
        }
        clear_hip_error();
        hipLaunchKernelGGL(ttp::scatter_slot_kernel, dim3(elementwise_grid(c, c->total)),
                           dim3(ttp::kBlock), 0, c->stream, rec, ttp::kStrideMixed, (uint64_t)0,
                           c->total, (const float*)c->master, (uint16_t*)nullptr);
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(c->stream) != hipSuccess) {
            (void)hipFree(rec);
            return fail(TTP_ERR_HIP, "moving the master into state records failed");
        }
        HIP_TRY(hipFree(c->master));
        c->records = rec;
        c->master = rec;
        c->exp_avg = rec + ttp::kRec;
        c->exp_avg_sq = rec + 2 * ttp::kRec;
        c->sgd_layout = false;
        return TTP_OK;
    }
    if ((rc = alloc_zero(c, (void**)&c->records, c->total * 4 * 2))) return rc;
    c->exp_avg = c->records;
    c->exp_avg_sq = c->records + ttp::kRec;
    return TTP_OK;
}

int ensure_momentum(ttp_ctx* c) {
    int rc;
    if ((rc = bf16_store_refuses(c, "the momentum buffer"))) return rc;
    if (!c->momentum && (rc = no_capture(c, "first momentum step (allocates the buffer)"))) return rc;
    if (!c->momentum && (rc = alloc_zero(c, (void**)&c->momentum, c->total * 4))) return rc;
    return TTP_OK;
}

// Active set of a step: the listed tensors (all when `subset` is NULL) that have a grad
// and at least one element; returns its device work tables (built once per distinct set).
int select_tables(ttp_ctx* c, const uint32_t* subset, uint32_t nsub, const WorkTables** out,
                  std::vector<uint32_t>* active_out, bool require_grad = true,
                  bool may_build = true) {
    const uint32_t nt = (uint32_t)c->tensors.size();
    std::vector<uint32_t> active;
    if (subset) {
        std::vector<uint8_t> seen(nt, 0);
        for (uint32_t k = 0; k < nsub; ++k) {
            const uint32_t i = subset[k];
            if (i >= nt) return fail(TTP_ERR_RANGE, "tensor index " + std::to_string(i) + " out of range");
            if (seen[i]) return fail(TTP_ERR_INVALID, "tensor index " + std::to_string(i) + " listed twice");
            seen[i] = 1;
        }
        for (uint32_t i = 0; i < nt; ++i)
            if (seen[i] && (c->tensors[i].has_grad || !require_grad) && c->tensors[i].numel)
                active.push_back(i);
    } else {
        for (uint32_t i = 0; i < nt; ++i)
            if ((c->tensors[i].has_grad || !require_grad) && c->tensors[i].numel)
                active.push_back(i);
    }
    if (active.size() == c->n_nonempty) {
        *out = &c->all;
    } else {
        auto it = c->tables.find(active);
        if (it == c->tables.end()) {
            int rc;
            if (!may_build)
                return fail(TTP_ERR_STATE, "this tensor set has no work table yet and the "
                                           "no-allocation step builds none: step the same "
                                           "set once with ttp_adam_step[_subset] first");
            if ((rc = no_capture(c, "a step over a tensor set not stepped before (builds tables)")))
                return rc;
            if (c->tables.size() >= 64 && !c->n_graphs) {
                // queued work may still read the cached tables
                HIP_TRY(hipStreamSynchronize(c->stream));
                for (auto& kv : c->tables) free_tables(kv.second);
                c->tables.clear();
            }
            WorkTables w;
            rc = build_tables(c, active, &w);
            if (rc) {
                free_tables(w);
                return rc;
            }
            it = c->tables.emplace(active, w).first;
        }
        *out = &it->second;
    }
    if (active_out) *active_out = std::move(active);
    return TTP_OK;
}

// (float)(1 - beta^t) for t = 1.. until both round to exactly 1.0f (and stay there, since
// beta^t only shrinks); py/optim.py:51-52 evaluates the same host-double expression.  One
// table per betas pair, built on first use; optimizers with different betas over one store
// switch tables without a synchronisation.  Beyond kMaxBiasTables pairs (a betas schedule)
// the cache is emptied, after the queued work, unless graphs may read the tables.
constexpr size_t kMaxBiasTables = 16;

int ensure_bias_table(ttp_ctx* c, double b1, double b2, bool may_build = true) {
    const auto key = std::make_pair(b1, b2);
    auto it = c->bias_tables.find(key);
    if (it == c->bias_tables.end()) {
        int rc;
        if (!may_build)
            return fail(TTP_ERR_STATE, "no bias-correction table for these betas yet and the "
                                       "no-allocation step builds none: step once with "
                                       "ttp_adam_step[_subset] and the same betas first");
        if ((rc = no_capture(c, "a step with new betas (builds a table)"))) return rc;
        std::vector<float> tab;
        const uint64_t kMax = 1ull << 24;
        for (uint64_t t = 1;; ++t) {
            const float x1 = (float)(1.0 - std::pow(b1, (double)t));
            const float x2 = (float)(1.0 - std::pow(b2, (double)t));
            if (x1 == 1.0f && x2 == 1.0f) break;
            if (t > kMax)
                return fail(TTP_ERR_INVALID, "beta too close to 1: bias correction table too long");
            tab.push_back(x1);
            tab.push_back(x2);
        }
        if (c->bias_tables.size() >= kMaxBiasTables && !c->n_graphs) {
            HIP_TRY(hipStreamSynchronize(c->stream));  // queued steps may read them
            for (auto& kv : c->bias_tables) (void)hipFree(kv.second.first);
            c->bias_tables.clear();
            c->bias_tab = nullptr;
            c->bias_len = 0;
        }
        float* d = nullptr;
        HIP_TRY(hipMalloc((void**)&d, std::max<size_t>(tab.size(), 2) * sizeof(float)));
        // a synchronous copy into the new allocation, which no queued work reads
        if (!tab.empty() &&
            hipMemcpy(d, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipFree(d);
            return fail(TTP_ERR_HIP, "bias correction table upload failed");
        }
        it = c->bias_tables.emplace(key, std::make_pair(d, (uint32_t)(tab.size() / 2))).first;
    }
    c->bias_tab = it->second.first;
    c->bias_len = it->second.second;
    return TTP_OK;
}

hipEvent_t take_event(ttp_ctx* c) {
    if (!c->ev_pool.empty()) {
        hipEvent_t e = c->ev_pool.back();
        c->ev_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// RAII-free helpers: begin/end an event pair around one launch when timing is on
struct TimedLaunch {
    ttp_ctx* c;
    int kernel;
    hipEvent_t a = nullptr;
    TimedLaunch(ttp_ctx* ctx, int k, bool enabled = true) : c(ctx), kernel(k) {
        if (enabled && c->timing && !c->capturing && (a = take_event(c)))
            (void)hipEventRecord(a, c->stream);
    }
    void done() {
        if (!a) return;
        hipEvent_t b = take_event(c);
        if (!b) {
            c->ev_pool.push_back(a);  // no pair for it: back to the pool
            return;
        }
        (void)hipEventRecord(b, c->stream);
        c->ev[kernel].push_back({a, b});
    }
};

int check_ctx(const ttp_ctx* c) {
    if (!c) return fail(TTP_ERR_INVALID, "null context");
    return TTP_OK;
}

int set_dev(const ttp_ctx* c) {
    HIP_TRY(hipSetDevice(c->device));
    return TTP_OK;
}

// whether the gradients of an update over `w` fit the Infinity Cache (see kCachedGradBytes):
// MIXED SGD momentum then runs the four-element kernel, MIXED Adam its cached-gradient lane
// shape.
// The four-element kernel launches one 256-lane block per chunk in one launch, which holds
// at most 2^32 - 1 work-items; a set of that many chunks (millions of tiny tensors) counts as
// not cached and takes the lane forms, which split.
bool grads_cached(const ttp_ctx* c, const WorkTables* w) {
    return w->elems * grad_esize(c) <= kCachedGradBytes &&
           w->n_chunks <= 0xFFFFFFFFu / ttp::kUpdBlock;
}

// Largest grid of the grid-stride chunk kernels (gradient zeroing): 2^22 blocks of 256 lanes is
// 2^30 work-items, well inside the 2^32 a launch may hold; they loop over the rest.
constexpr uint32_t kMaxGridBlocks = 1u << 22;

// MIXED SGD momentum updates whose gradients fit the Infinity Cache run the four-element
// kernel, one block per chunk (at most 2^17 chunks); every other update runs a lane form: kE elements per
// lane in blocks of kLanes, each block walking kIt consecutive pieces of kLanes x kE
// elements, one block per 1/lane_parts<kE, kLanes, kIt>() of a chunk.
// MIXED Adam with cached gradients (GPT-2 124M; whole steps of bench.py after its settle
// phase, 5 warmup + 20 timed steps, three interleaved rounds on one box; four-element /
// 1 x 128 x 2 / 1 x 256 x 2):
//   back-to-back step       0.5589-0.5597 / 0.5519-0.5547 / 0.5602-0.5621 ms
//   update kernel alone     0.5222-0.5225 / 0.5123-0.5141 / 0.5195-0.5220 ms
//   249 MB gradient copy + step (a backward rewrites the gradients just before the step;
//   400 steps, 3 rounds, 2 processes)  0.660-0.662 / 0.631-0.632 / 0.633-0.634 ms
//   skipped step            0.069 / 0.148 / 0.096 ms (the early exit of every block)
//   nanoGPT-char (10.8M)    0.0543-0.0551 / 0.0544-0.0547 / 0.0556 ms
// The four-element form wins only the rare skipped step.  FP32 stores with cached gradients
// (8 GPT-2 blocks without wte, 57.5M params; four-element / lane form of the FP32 shapes
// below; 300 steps per event pair, 3 rounds, 2 processes): AdamW 0.2763-0.2768 / 0.2685-0.2687
// ms back to back, 0.3571-0.3577 / 0.3468-0.3474 ms with a gradient copy; SGD momentum
// 0.2124-0.2128 / 0.2068-0.2071 and 0.2938-0.2941 / 0.2858-0.2860 ms.  MIXED SGD momentum at
// GPT-2 124M keeps the four-element form (bench.py --optimizer sgdm, three rounds: 0.4365-0.4372
// against 0.4408-0.4423 ms for 1 x 256 x 2 back to back, 0.4424-0.4439 against 0.4562-0.4589
// with a cold cache).  Beyond the cache the shapes are the fastest measured at GPT-2 774M
// mixed / 1558M fp32 (interleaved rounds, x a 256-lane non-temporal copy of the same bytes;
// elements x lanes x pieces):
//   Adam MIXED  1 x 256 x 2: 1.014-1.016 (1x128x2 1.01, 1x256x1 0.96-0.98, four-element 0.91)
//   Adam FP32   1 x 128 x 2: 1.022-1.027 (1x256x2 1.01-1.02, 2x64x1 0.98, 2x64x2 0.89)
//   SGD MIXED   1 x 256 x 2: 0.923-0.926 (slower by: 2x128x1 0.4-1.1%, 1x128x2 0.4-0.6%,
//                            2x256x1 3.3%, 2x64x1 3.7%, 1x256x1 14%)
//   SGD FP32    2 x 64 x 1:  1.001-1.026 (slower by: 2x128x1 0.8-2.8%, 1x128x2 3.1-3.3%,
//                            1x64x2 3.6%, 1x256x2 3.7-5.6%, 2x64x2 9%, 1x64x1 27%)
// (SGD with momentum; each variant a build of its own, timed in turn on the same box, two
// boxes per mode.)  At 774M the 1 x 128 x 2 shape ties 1 x 256 x 2 on clean steps, back to
// back and after a gradient copy (3.476 against 3.472 ms, 4.095 against 4.089 ms), and
// dispatches twice the workgroups on a skipped step.
constexpr int kLaneAdamMixedCached = 1, kLanesAdamMixedCached = 128, kItAdamMixedCached = 2;
constexpr int kLaneAdamMixed = 1, kLanesAdamMixed = 256, kItAdamMixed = 2;
constexpr int kLaneAdamFp32 = 1, kLanesAdamFp32 = 128, kItAdamFp32 = 2;
constexpr int kLaneSgdMixed = 1, kLanesSgdMixed = 256, kItSgdMixed = 2;
constexpr int kLaneSgdFp32 = 2, kLanesSgdFp32 = 64, kItSgdFp32 = 1;
// MIXED SGD without momentum (the traced layers' sgd_step, autograd::SGD) moves 12 B per
// element, a third of them as bf16: two elements per lane make its gradient loads and bf16
// stores 4-byte words.  Step times, ms (back to back / after a device copy of the gradients,
// the copy excluded; 50 steps per event pair, two interleaved rounds on one box):
//   GPT-2 774M   2 x 256 x 1  1.611 / 1.593   (2 x 128 x 1 1.655 / 1.640, 1 x 256 x 2
//                2.074 / 2.062, the four-element form 1.635 / 1.618)
//   GPT-2 124M   2 x 256 x 1  0.268 / 0.261   (2 x 128 x 1 0.249 / 0.270, the four-element
//                form 0.274 / 0.269, 1 x 256 x 2 0.314 back to back)
// 5.76 TB/s at 774M, against 5.98 TB/s for the FP32 store's plain SGD (contiguous weights)
// and 4.48 TB/s for the 1 x 256 x 2 shape that momentum prefers.  One shape at every size:
// after a gradient rewrite, as in training, it is the fastest at both sizes.
constexpr int kLaneSgdPlainMixed = 2, kLanesSgdPlainMixed = 256, kItSgdPlainMixed = 1;
// The SGD layout of a MIXED store (TTP_STORE_SGD: contiguous master and momentum).  Measured
// with the product kernels in a timing-only program (GPT-2 tables and the C++ drop-in's
// 163M traced GPT, three rounds, medians, x a 64-lane non-temporal copy of the same bytes;
// back to back / after a device copy of the gradients):
//   plain    4 x 64 x 1:  124M 1.082 / 1.035, 163M 1.002 / 1.021, 774M 0.984 / 1.018
//                         (2x256x2 0.96-1.02, 4x128x1 0.94-1.04, 4x256x1 0.95-1.03,
//                         2x256x1 0.86-0.91, 1x256x2 0.69-0.73; the record master's
//                         2x256x1 0.82-0.89)
//   momentum 2 x 128 x 1: 124M 0.998 / 0.992, 163M 0.973 / 0.986, 774M 0.989 / 1.018
//                         (2x64x1 0.94-1.01, 4x64x1 0.94-1.04, 2x256x1 0.94-0.99,
//                         1x256x2 0.92-0.95; the record master's 1x256x2 0.88-0.92)
// Four elements per lane give the plain update 16-byte master loads and stores and 8-byte
// gradient and bf16 words, the copy's pattern; with its momentum stream the update does
// best with two.  One shape at every size (the gradients' place in the Infinity Cache made
// no difference to the ranking).
constexpr int kLaneSgdPlainContig = 4, kLanesSgdPlainContig = 64, kItSgdPlainContig = 1;
constexpr int kLaneSgdMomContig = 2, kLanesSgdMomContig = 128, kItSgdMomContig = 1;
// Plain SGD of a BF16 store (bf16 gradients and weights, 6 B per element): eight elements per
// lane, one 16-byte word per stream as the 64-lane copy moves them.  Step times in ms at
// GPT-2 124M / 774M, back to back / after a device copy of the gradients (one library build
// per shape, two interleaved rounds of three; x the 64-lane copy of the same 6 B/element):
//   8 x 64 x 1   0.113 / 0.111,  0.669 / 0.704   (774M: 1.044 / 0.992)
//   8 x 128 x 1  0.112 / 0.109,  0.695 / 0.716      8 x 64 x 2   0.107 / 0.112,  0.786 / 0.795
//   4 x 64 x 1   0.116 / 0.130,  0.801 / 0.796      4 x 128 x 1  0.119 / 0.131,  0.809 / 0.803
//   4 x 256 x 1  0.133 / 0.136,  0.865 / 0.856      8 x 32 x 1   0.152 / 0.160,  0.980 / 0.979
//   2 x 256 x 1  0.177 / 0.196,  1.175 / 1.171
constexpr int kLaneSgdBf16 = 8, kLanesSgdBf16 = 64, kItSgdBf16 = 1;
// FP32 SGD without momentum (fp32 gradients and weights, 12 B per element), the same program
// and method (124M / 774M / 1558M, x the 64-lane copy, back to back / after a gradient
// copy): 2 x 256 x 2 0.993 / 0.976, 1.003 / 1.013, 1.001 / 1.018 (4x256x1 0.97-0.99,
// 4x64x1 0.94-0.99, the momentum shape 2x64x1 0.86-0.88).  With momentum the 2 x 64 x 1 shape
// above stays: 0.976 / 0.959, 0.973 / 0.977, 0.986 / 0.992 (2x128x1 0.97-1.00, 4x64x1
// 0.91-0.97).
constexpr int kLaneSgdPlainFp32 = 2, kLanesSgdPlainFp32 = 256, kItSgdPlainFp32 = 2;

// One launch holds at most 2^32 - 1 work-items, so at most (2^32 - 1) / lanes blocks.  A
// lane-form update over more parts is split into launches at increasing part offsets
// (TTP_LANE_LAUNCH_BLOCKS lowers the per-launch limit, so tests reach the split on small
// stores).
template <typename Launch>
void launch_lanes(const ttp_ctx* c, uint64_t nparts, uint32_t lanes, Launch&& launch) {
    uint64_t max_blocks = 0xFFFFFFFFull / lanes;
    if (c->lane_launch_cap) max_blocks = std::min(max_blocks, c->lane_launch_cap);
    for (uint64_t p0 = 0; p0 < nparts; p0 += max_blocks)
        launch(dim3((uint32_t)std::min<uint64_t>(nparts - p0, max_blocks)), p0);
}

uint32_t norm_grid(const ttp_ctx* c, uint32_t nchunks) {
    return std::max<uint32_t>(1, std::min(nchunks, c->norm_grid_cap));
}

// The norm pass over n tiles as two launches (see norm_partials_kernel): non-temporal loads
// over tiles [0, split), cached loads over [split, n), the last kCachedGradBytes of gradients.
// Partials: g_nt of the first launch, then g_cached of the second.
struct NormSplit {
    uint32_t split, g_nt, g_cached;
    uint32_t partials() const { return g_nt + g_cached; }
};
NormSplit norm_split(const ttp_ctx* c, uint32_t n) {
    const uint32_t keep = (uint32_t)std::min<uint64_t>(
        n, kCachedGradBytes / ((uint64_t)norm_tile(c) * grad_esize(c)));
    NormSplit s;
    s.split = n - keep;
    s.g_nt = s.split ? norm_grid(c, s.split) : 0;
    s.g_cached = norm_grid(c, keep);
    return s;
}

template <typename GradT>
void launch_norm_pass(ttp_ctx* c, const WorkTables* w, const NormSplit& ns, int32_t scaler_on,
                      double* partials) {
    const GradT* g = (const GradT*)c->grad;
    const DevState* st = c->st;
    if (ns.g_nt)
        hipLaunchKernelGGL((ttp::norm_partials_kernel<GradT, true>), dim3(ns.g_nt),
                           dim3(ttp::kBlock), 0, c->stream, g, w->tiles, 0u, ns.split, st,
                           scaler_on, partials);
    hipLaunchKernelGGL((ttp::norm_partials_kernel<GradT, false>), dim3(ns.g_cached),
                       dim3(ttp::kBlock), 0, c->stream, g, w->tiles, ns.split, w->n_tiles, st,
                       scaler_on, partials + ns.g_nt);
}

// Step prologue on the device: the norm pass (partials, when `run_norm`) and the one-block
// finalize (norm, found_inf / skip, clip coefficient, loss scale, and the step count with its
// bias corrections when `count_t`); `probe` only computes the norm.
// `partials` (null: the context's own) holds one partial per norm-pass block; a caller-given
// array (the no-allocation step's) also turns the per-launch timing events off.
int launch_prologue(ttp_ctx* c, const WorkTables* w, bool run_norm, double max_norm, bool probe,
                    bool want_bias, bool count_t, bool from_sums = false,
                    bool defer_scale = false, double* partials = nullptr) {
    const NormSplit ns = norm_split(c, w->n_tiles);
    const int32_t scaler_on = c->scaler.enabled ? 1 : 0;
    TimedLaunch tl(c, TTP_KERNEL_NORM, partials == nullptr);
    if (!partials) partials = c->partials;
    if (run_norm && !from_sums) {
        clear_hip_error();
        if (bf16_grads(c))
            launch_norm_pass<uint16_t>(c, w, ns, scaler_on, partials);
        else
            launch_norm_pass<float>(c, w, ns, scaler_on, partials);
        HIP_TRY(hipGetLastError());
    }
    ttp::FinalizeArgs a{};
    a.partials = partials;
    a.npartials = run_norm ? ns.partials() : 0;
    if (run_norm && from_sums) {  // the step's tensors' sums, in tensor order
        // tile sums that accumulates with their sums left pending: combined first (a captured
        // step always launches this, since its replays may find them pending)
        if (w->n_tensors && (c->capturing || c->acc_sums_used)) {
            clear_hip_error();
            hipLaunchKernelGGL(ttp::combine_pending_sums_kernel, dim3(w->n_tensors),
                               dim3(ttp::kBlock), 0, c->stream, (const double*)c->acc_tiles,
                               (const uint32_t*)c->tile_base, (const uint32_t*)w->tile_start,
                               (const uint32_t*)w->tensor_ids, c->tsum_pending, c->tsum);
            HIP_TRY(hipGetLastError());
        }
        a.partials = c->tsum;
        a.idx = w->tensor_ids;
        a.npartials = w->n_tensors;
    }
    a.scaler_on = run_norm ? scaler_on : 0;
    a.defer_scale = defer_scale ? 1 : 0;
    a.count_t = count_t ? 1 : 0;
    a.probe = probe ? 1 : 0;
    a.growth_interval = c->scaler.growth_interval;
    a.growth_factor = c->scaler.growth_factor;
    a.backoff_factor = c->scaler.backoff_factor;
    a.max_norm = run_norm ? max_norm : 0.0;
    a.bias_tab = c->bias_tab;
    a.bias_len = c->bias_len;
    a.want_bias = want_bias ? 1 : 0;
    a.st = c->st;
    clear_hip_error();
    hipLaunchKernelGGL(ttp::norm_finalize_kernel, dim3(1), dim3(ttp::kBlock), 0, c->stream, a);
    HIP_TRY(hipGetLastError());
    tl.done();
    return TTP_OK;
}

// Whether two scaler configurations step alike: a captured graph holds `enabled` and the
// growth / backoff settings as launch arguments (the scale and tracker live on the device).
bool same_scaler_settings(const ttp_scaler_config& a, const ttp_scaler_config& b) {
    if ((a.enabled != 0) != (b.enabled != 0)) return false;
    return !a.enabled || (a.growth_interval == b.growth_interval &&
                          a.growth_factor == b.growth_factor &&
                          a.backoff_factor == b.backoff_factor);
}

int read_state(ttp_ctx* c, DevState* out) {
    HIP_TRY(hipMemcpyAsync(out, c->st, sizeof(DevState), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return TTP_OK;
}

int fill_report(ttp_ctx* c, bool norm_ran, ttp_step_report* r) {
    HIP_TRY(hipStreamSynchronize(c->stream));
    DevState s;
    int rc = read_state(c, &s);
    if (rc) return rc;
    std::memset(r, 0, sizeof(*r));
    r->found_inf = norm_ran ? s.found_inf : 0;
    r->skipped = (norm_ran && c->scaler.enabled) ? s.skip : 0;
    r->grad_norm = norm_ran ? s.norm : std::nan("");
    r->clip_coef = norm_ran ? s.clip_coef : 1.0f;
    r->scale = c->scaler.enabled ? s.scale : 1.0f;
    r->growth_tracker = c->scaler.enabled ? s.growth_tracker : 0;
    r->step = t_on_device(c) ? s.t : c->host_t;
    return TTP_OK;
}

// A caller's buffer that the GPU reads or writes directly (TTP_DEVICE transfers, device
// gradient sources): [p, p + bytes) must be device (or managed) memory of this context's
// device, inside one allocation.  A host pointer, another device's memory or a short buffer
// is refused here, before any launch or copy touches it.
int check_device_buffer(const ttp_ctx* c, const void* p, uint64_t bytes, const char* what) {
    if (!bytes) return TTP_OK;
    hipPointerAttribute_t at{};
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        clear_hip_error();
        return fail(TTP_ERR_INVALID, std::string(what) +
                                         " is not device memory (use TTP_HOST for host memory)");
    }
    if (at.type != hipMemoryTypeDevice && at.type != hipMemoryTypeManaged)
        return fail(TTP_ERR_INVALID, std::string(what) +
                                         " is not device memory (use TTP_HOST for host memory)");
    if (at.type == hipMemoryTypeDevice && at.device != c->device)
        return fail(TTP_ERR_INVALID, std::string(what) + " is on device " +
                                         std::to_string(at.device) + ", the context on device " +
                                         std::to_string(c->device));
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess) {
        clear_hip_error();
        return fail(TTP_ERR_INVALID, std::string(what) + " lies in no known device allocation");
    }
    const uintptr_t lo = (uintptr_t)p, end = (uintptr_t)base + size;
    if (lo < (uintptr_t)base || bytes > end - lo)
        return fail(TTP_ERR_RANGE, std::string(what) + ": " + std::to_string(bytes) +
                                       " bytes do not fit its allocation (" +
                                       std::to_string(end - lo) + " bytes from the pointer on)");
    return TTP_OK;
}

int check_index(const ttp_ctx* c, uint32_t i) {
    if (i >= c->tensors.size())
        return fail(TTP_ERR_RANGE, "tensor index " + std::to_string(i) + " out of range");
    return TTP_OK;
}

// Elements per record of buffer `which`: element e sits at base + (e / kRec) * stride +
// e % kRec; kRec means contiguous.
uint32_t buffer_stride(const ttp_ctx* c, int which) {
    const bool mixed = c->mode == TTP_MODE_MIXED;
    switch (which) {
        case TTP_BUF_MASTER: return mixed && !c->sgd_layout ? ttp::kStrideMixed : ttp::kRec;
        case TTP_BUF_EXP_AVG:
        case TTP_BUF_EXP_AVG_SQ: return mixed ? ttp::kStrideMixed : ttp::kStrideMV;
    }
    return ttp::kRec;
}

bool in_records(const ttp_ctx* c, int which) { return buffer_stride(c, which) != ttp::kRec; }

void* buffer_base(ttp_ctx* c, int which) {
    switch (which) {
        case TTP_BUF_PARAM: return c->param;
        case TTP_BUF_GRAD: return c->grad;
        case TTP_BUF_MASTER: return c->master;
        case TTP_BUF_EXP_AVG: return c->exp_avg;
        case TTP_BUF_EXP_AVG_SQ: return c->exp_avg_sq;
        case TTP_BUF_MOMENTUM: return c->momentum;
    }
    return nullptr;
}

size_t buffer_esize(const ttp_ctx* c, int which) {
    if (which == TTP_BUF_PARAM) return param_esize(c);
    if (which == TTP_BUF_GRAD) return grad_esize(c);
    return 4;
}

int check_buffer_id(int which) {
    if (which < TTP_BUF_PARAM || which > TTP_BUF_MOMENTUM)
        return fail(TTP_ERR_INVALID, "unknown buffer id " + std::to_string(which));
    return TTP_OK;
}

// a buffer id the context holds (or creates on first use): a BF16 store, PARAM and GRAD only
int check_buffer_in_mode(const ttp_ctx* c, int which) {
    int rc = check_buffer_id(which);
    if (rc) return rc;
    if (which != TTP_BUF_PARAM && which != TTP_BUF_GRAD)
        return bf16_store_refuses(c, ("buffer " + std::to_string(which)).c_str());
    return TTP_OK;
}

// Allocates the optimizer state a buffer id names (m, v or the momentum) on first use; in the
// SGD layout, m and v convert the store.  Callers validate everything else first, so that a
// refused call neither allocates nor converts.
int materialize(ttp_ctx* c, int which) {
    int rc = check_buffer_id(which);
    if (rc) return rc;
    if (which == TTP_BUF_EXP_AVG || which == TTP_BUF_EXP_AVG_SQ) return ensure_adam_state(c);
    if (which == TTP_BUF_MOMENTUM) return ensure_momentum(c);
    return TTP_OK;
}

int resolve_range(ttp_ctx* c, uint32_t index, uint64_t n, uint64_t* off, uint64_t* count) {
    if (index == TTP_ALL_TENSORS) {
        if (n != c->total)
            return fail(TTP_ERR_RANGE, "flat transfer must cover all " + std::to_string(c->total) +
                                           " elements, got " + std::to_string(n));
        *off = 0;
        *count = n;
        return TTP_OK;
    }
    int rc = check_index(c, index);
    if (rc) return rc;
    if (n != c->tensors[index].numel)
        return fail(TTP_ERR_RANGE, "tensor " + std::to_string(index) + " has " +
                                       std::to_string(c->tensors[index].numel) +
                                       " elements, got " + std::to_string(n));
    *off = c->tensors[index].offset;
    *count = n;
    return TTP_OK;
}

// Device staging buffer of at least `bytes` (host transfers pass through it).  Growing it
// waits for queued work, which may still read the old one.
int ensure_staging(ttp_ctx* c, uint64_t bytes) {
    if (c->staging_bytes >= bytes) return TTP_OK;
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (c->staging) HIP_TRY(hipFree(c->staging));
    c->staging = nullptr;
    c->staging_bytes = 0;
    HIP_TRY(hipMalloc(&c->staging, bytes));
    c->staging_bytes = bytes;
    return TTP_OK;
}

// Host transfers of record-stored buffers move through device staging in pieces of at most
// this many elements (64 MiB of fp32).
constexpr uint64_t kPieceElems = 16ull << 20;

// slot elements [first, first + n) of record-stored buffer `which` -> contiguous device array
// (a BF16 store's checkpoint master: its bf16 weights, widened exactly)
int gather_slot(ttp_ctx* c, int which, uint64_t first, uint64_t n, float* dst) {
    if (!n) return TTP_OK;
    clear_hip_error();
    if (c->mode == TTP_MODE_BF16 && which == TTP_BUF_MASTER) {
        hipLaunchKernelGGL(ttp::bf16_to_master_kernel, dim3(elementwise_grid(c, n)),
                           dim3(ttp::kBlock), 0, c->stream, (const uint16_t*)c->param + first,
                           dst, ttp::kRec, (uint64_t)0, n);
        HIP_TRY(hipGetLastError());
        return TTP_OK;
    }
    hipLaunchKernelGGL(ttp::gather_slot_kernel, dim3(elementwise_grid(c, n)), dim3(ttp::kBlock),
                       0, c->stream, (const float*)buffer_base(c, which),
                       buffer_stride(c, which), first, n, dst);
    HIP_TRY(hipGetLastError());
    return TTP_OK;
}

// contiguous device array (null: zeros) -> slot elements [first, first + n); an upload of
// MIXED-mode master weights also writes their bf16 copy
// (a BF16 store's checkpoint master: rounded to its bf16 weights, exactly for values that
// came from bf16)
int scatter_slot(ttp_ctx* c, int which, uint64_t first, uint64_t n, const float* src) {
    if (!n) return TTP_OK;
    if (c->mode == TTP_MODE_BF16 && which == TTP_BUF_MASTER) {
        if (!src) return fail(TTP_ERR_STATE, "a BF16 store's weights cannot be zeroed here");
        clear_hip_error();
        hipLaunchKernelGGL(ttp::master_to_bf16_kernel, dim3(elementwise_grid(c, n)),
                           dim3(ttp::kBlock), 0, c->stream, src, ttp::kRec,
                           (uint16_t*)c->param + first, (uint64_t)0, n);
        HIP_TRY(hipGetLastError());
        return TTP_OK;
    }
    uint16_t* p16 = (c->mode == TTP_MODE_MIXED && which == TTP_BUF_MASTER) ? (uint16_t*)c->param
                                                                          : nullptr;
    clear_hip_error();
    hipLaunchKernelGGL(ttp::scatter_slot_kernel, dim3(elementwise_grid(c, n)), dim3(ttp::kBlock),
                       0, c->stream, (float*)buffer_base(c, which), buffer_stride(c, which),
                       first, n, src, p16);
    HIP_TRY(hipGetLastError());
    return TTP_OK;
}

// upload/download of a record-stored buffer's elements [first, first + n)
int upload_slot(ttp_ctx* c, int which, uint64_t first, uint64_t n, const void* src, int kind) {
    if (kind == TTP_DEVICE) return scatter_slot(c, which, first, n, (const float*)src);
    int rc;
    const uint64_t piece = std::min(n, kPieceElems);
    if ((rc = ensure_staging(c, piece * 4))) return rc;
    for (uint64_t o = 0; o < n; o += piece) {
        const uint64_t k = std::min(piece, n - o);
        HIP_TRY(hipMemcpyAsync(c->staging, (const float*)src + o, k * 4, hipMemcpyHostToDevice,
                               c->stream));
        if ((rc = scatter_slot(c, which, first + o, k, (const float*)c->staging))) return rc;
        HIP_TRY(hipStreamSynchronize(c->stream));  // the staging buffer is refilled next
    }
    return TTP_OK;
}

int download_slot(ttp_ctx* c, int which, uint64_t first, uint64_t n, void* dst, int kind) {
    if (kind == TTP_DEVICE) return gather_slot(c, which, first, n, (float*)dst);
    int rc;
    const uint64_t piece = std::min(n, kPieceElems);
    if ((rc = ensure_staging(c, piece * 4))) return rc;
    for (uint64_t o = 0; o < n; o += piece) {
        const uint64_t k = std::min(piece, n - o);
        if ((rc = gather_slot(c, which, first + o, k, (float*)c->staging))) return rc;
        HIP_TRY(hipMemcpyAsync((float*)dst + o, c->staging, k * 4, hipMemcpyDeviceToHost,
                               c->stream));
        HIP_TRY(hipStreamSynchronize(c->stream));  // the staging buffer is refilled next
    }
    return TTP_OK;
}

void release(ttp_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (void* p : {(void*)c->grad, (void*)c->records, (void*)c->momentum, (void*)c->mom_init,
                    (void*)c->st, (void*)c->partials, c->staging, (void*)c->tsum,
                    (void*)c->tile_sums, (void*)c->acc_tiles, (void*)c->tile_base,
                    (void*)c->tsum_pending})
        if (p) (void)hipFree(p);
    for (auto& kv : c->bias_tables) (void)hipFree(kv.second.first);
    free_tables(c->all);
    for (auto& kv : c->tables) free_tables(kv.second);
    for (void* p : c->retired) (void)hipFree(p);
    // MIXED: param is the bf16 copy and master lives in `records` (in the SGD layout, in an
    // allocation of its own); FP32: param == master
    if (c->mode != TTP_MODE_FP32 && c->param) (void)hipFree(c->param);
    if ((c->mode == TTP_MODE_FP32 || c->sgd_layout) && c->master) (void)hipFree(c->master);
    for (auto& v : c->ev)
        for (auto& p : v) {
            (void)hipEventDestroy(p.a);
            (void)hipEventDestroy(p.b);
        }
    for (auto e : c->ev_pool) (void)hipEventDestroy(e);
    if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
    delete c;
}

}  // namespace

// =====================================================================================
// C ABI
// =====================================================================================
extern "C" {

const char* ttp_last_error(void) { return g_last_error.c_str(); }
int ttp_abi_version(void) { return TTP_ABI_VERSION; }

int ttp_device_count(int* count) {
    if (!count) return fail(TTP_ERR_INVALID, "null count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return TTP_OK;
}

int ttp_create(int device, const ttp_tensor_desc* descs, uint32_t n, int mode, ttp_ctx** out) {
    if (!out) return fail(TTP_ERR_INVALID, "null output pointer");
    *out = nullptr;
    if (n && !descs) return fail(TTP_ERR_INVALID, "null tensor table");
    const bool sgd_layout = (mode & TTP_STORE_SGD) != 0;
    mode &= ~TTP_STORE_SGD;
    if (mode != TTP_MODE_FP32 && mode != TTP_MODE_MIXED && mode != TTP_MODE_BF16)
        return fail(TTP_ERR_INVALID, "mode must be TTP_MODE_FP32, TTP_MODE_MIXED (optionally "
                                     "| TTP_STORE_SGD) or TTP_MODE_BF16");
    if (mode == TTP_MODE_BF16 && sgd_layout)
        return fail(TTP_ERR_INVALID, "TTP_STORE_SGD is a layout of a TTP_MODE_MIXED store's "
                                     "fp32 master; a TTP_MODE_BF16 store has none");
    // per-tensor kernels launch one 256-lane block per tensor: fewer than 2^32 work-items
    if (n >= (1u << 24)) return fail(TTP_ERR_INVALID, "too many tensors (max 2^24 - 1)");
    // the table must describe a store that fits one GPU: the padded footprint sum cannot
    // wrap, and every chunk index stays inside the buffers the kernels address
    uint64_t footprint = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (descs[i].flags & ~TTP_TENSOR_DECAY)
            return fail(TTP_ERR_INVALID, "unknown flags on tensor " + std::to_string(i));
        if (descs[i].reserved)
            return fail(TTP_ERR_INVALID, "tensor " + std::to_string(i) + ": reserved must be 0");
        if (descs[i].numel > kMaxElems)
            return fail(TTP_ERR_INVALID, "tensor " + std::to_string(i) + " has " +
                                             std::to_string(descs[i].numel) +
                                             " elements (max 2^40)");
        footprint += (descs[i].numel + kAlign - 1) / kAlign * kAlign;
        if (footprint > kMaxElems)
            return fail(TTP_ERR_INVALID, "the tensors total more than 2^40 elements");
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0)
        return fail(TTP_ERR_NO_DEVICE, "no HIP device available");
    if (device < 0 || device >= ndev)
        return fail(TTP_ERR_NO_DEVICE, "device " + std::to_string(device) + " out of range");

    ttp_ctx* c = new ttp_ctx();
    c->device = device;
    c->mode = mode;
    auto bail = [&](int rc) {
        release(c);
        return rc;
    };
    if (hipSetDevice(device) != hipSuccess) return bail(fail(TTP_ERR_HIP, "hipSetDevice failed"));
    int rc0 = ensure_scratch(device);  // this device's copy of the no-allocation scratch array
    if (rc0) return bail(rc0);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
        c->num_cus = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(TTP_ERR_HIP, "hipStreamCreate failed"));
    c->stream = c->own_stream;

    {
        // occupancy cap of the four-element update (MIXED SGD momentum, cached gradients):
        // LDS_per_CU / blocks_per_CU bytes of dynamic LDS per block
        int lds_cu = 0, lds_blk = 0;
        const uint64_t per_cu = env_u64("TTP_UPD_BLOCKS_PER_CU", ttp::kUpdBlocksPerCU);
        if (per_cu &&
            hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor,
                                  device) == hipSuccess &&
            hipDeviceGetAttribute(&lds_blk, hipDeviceAttributeMaxSharedMemoryPerBlock, device) ==
                hipSuccess &&
            lds_cu > 0 && lds_blk > 0) {
            uint64_t b = (uint64_t)lds_cu / per_cu / 512 * 512;
            c->upd_lds = (uint32_t)std::min<uint64_t>(b, (uint64_t)lds_blk);
        }
    }
    c->norm_grid_cap = (uint32_t)std::min<uint64_t>(
        65536, std::max<uint64_t>(1, env_u64("TTP_NORM_GRID", (uint64_t)c->num_cus * 8)));
    c->lane_launch_cap = env_u64("TTP_LANE_LAUNCH_BLOCKS", 0);

    // layout
    c->tensors.resize(n);
    uint64_t off = 0;
    for (uint32_t i = 0; i < n; ++i) {
        c->tensors[i] = {off, descs[i].numel, descs[i].flags, 0};
        off += (descs[i].numel + kAlign - 1) / kAlign * kAlign;
    }
    c->total = off;
    int rc;
    if (mode == TTP_MODE_MIXED && sgd_layout) {
        // the SGD layout: a contiguous master, no m / v (until the first Adam use), bf16 copy
        c->sgd_layout = true;
        if ((rc = alloc_zero(c, (void**)&c->master, c->total * 4))) return bail(rc);
        if ((rc = alloc_zero(c, &c->param, c->total * 2))) return bail(rc);
    } else if (mode == TTP_MODE_MIXED) {
        // [master|m|v] records (m, v zero until the first Adam step) and the bf16 copy
        if ((rc = alloc_zero(c, (void**)&c->records, c->total * 4 * 3))) return bail(rc);
        c->master = c->records;
        c->exp_avg = c->records + ttp::kRec;
        c->exp_avg_sq = c->records + 2 * ttp::kRec;
        if ((rc = alloc_zero(c, &c->param, c->total * 2))) return bail(rc);
    } else if (mode == TTP_MODE_BF16) {
        // the bf16 weights alone: no master, no records
        if ((rc = alloc_zero(c, &c->param, c->total * 2))) return bail(rc);
    } else {
        if ((rc = alloc_zero(c, (void**)&c->master, c->total * 4))) return bail(rc);
        c->param = c->master;
    }
    if ((rc = alloc_zero(c, &c->grad, c->total * grad_esize(c)))) return bail(rc);
    if ((rc = alloc_zero(c, (void**)&c->mom_init, std::max<uint64_t>(n, 1) * 4))) return bail(rc);
    c->host_mom_init.assign(n, 0);
    if ((rc = alloc_zero(c, (void**)&c->st, sizeof(DevState)))) return bail(rc);
    c->partials_cap = 2 * c->norm_grid_cap;  // the norm pass's two launches (NormSplit)
    if ((rc = alloc_zero(c, (void**)&c->partials, (uint64_t)c->partials_cap * 8))) return bail(rc);
    if ((rc = alloc_zero(c, (void**)&c->tsum, std::max<uint64_t>(n, 1) * 8))) return bail(rc);
    c->tsum_fresh.assign(n, 0);
    // the tile sums of accumulates with their sums: 32 B per 16 KiB of gradients
    {
        const uint64_t tile = norm_tile(c);
        uint64_t tiles = 0;
        c->host_tile_base.resize(std::max<uint32_t>(n, 1), 0);
        for (uint32_t i = 0; i < n; ++i) {
            c->host_tile_base[i] = (uint32_t)tiles;  // at most 2^40 / 4096 tiles
            tiles += (descs[i].numel + tile - 1) / tile;
        }
        if ((rc = alloc_zero(c, (void**)&c->acc_tiles,
                             std::max<uint64_t>(tiles, 1) * ttp::kWaves * 8)))
            return bail(rc);
        if ((rc = alloc_zero(c, (void**)&c->tsum_pending, std::max<uint64_t>(n, 1) * 4)))
            return bail(rc);
        if ((rc = alloc_zero(c, (void**)&c->tile_base, (uint64_t)c->host_tile_base.size() * 4)))
            return bail(rc);
    }

    std::vector<uint32_t> every;
    for (uint32_t i = 0; i < n; ++i)
        if (descs[i].numel) every.push_back(i);
    c->n_nonempty = (uint32_t)every.size();
    if ((rc = build_tables(c, every, &c->all))) return bail(rc);

    // the zero fills above run on the context's non-blocking stream, which the legacy-stream
    // hipMemcpy below does not wait for: finish them first
    if (hipStreamSynchronize(c->stream) != hipSuccess)
        return bail(fail(TTP_ERR_HIP, "stream synchronize failed"));
    DevState s{};
    s.scale = (float)c->scaler.init_scale;
    if (hipMemcpy(c->st, &s, sizeof(s), hipMemcpyHostToDevice) != hipSuccess)
        return bail(fail(TTP_ERR_HIP, "state upload failed"));
    if (hipMemcpy(c->tile_base, c->host_tile_base.data(), c->host_tile_base.size() * 4,
                  hipMemcpyHostToDevice) != hipSuccess)
        return bail(fail(TTP_ERR_HIP, "tile table upload failed"));
    *out = c;
    return TTP_OK;
}

int ttp_destroy(ttp_ctx* c) {
    if (!c) return TTP_OK;
    if (c->n_graphs)
        return fail(TTP_ERR_STATE, std::to_string(c->n_graphs) +
                                       " graph(s) of this context are alive; destroy them first");
    if (c->capturing) {
        hipGraph_t g = nullptr;
        if (hipStreamEndCapture(c->stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
        c->capturing = false;
    }
    release(c);
    return TTP_OK;
}

int ttp_set_stream(ttp_ctx* c, void* stream) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = no_capture(c, "ttp_set_stream"))) return rc;
    if ((rc = set_dev(c))) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->stream = (hipStream_t)stream;
    return TTP_OK;
}

int ttp_reset_stream(ttp_ctx* c) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = no_capture(c, "ttp_reset_stream"))) return rc;
    if ((rc = set_dev(c))) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->stream = c->own_stream;
    return TTP_OK;
}

int ttp_sync(ttp_ctx* c) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = no_capture(c, "ttp_sync"))) return rc;
    if ((rc = set_dev(c))) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    return TTP_OK;
}

int ttp_num_tensors(const ttp_ctx* c, uint32_t* n) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!n) return fail(TTP_ERR_INVALID, "null output");
    *n = (uint32_t)c->tensors.size();
    return TTP_OK;
}

int ttp_mode(const ttp_ctx* c, int* mode) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!mode) return fail(TTP_ERR_INVALID, "null output");
    *mode = c->mode;
    return TTP_OK;
}

int ttp_flat_numel(const ttp_ctx* c, uint64_t* total) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!total) return fail(TTP_ERR_INVALID, "null output");
    *total = c->total;
    return TTP_OK;
}

int ttp_tensor_info(const ttp_ctx* c, uint32_t i, uint64_t* offset, uint64_t* numel,
                    uint32_t* flags) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = check_index(c, i))) return rc;
    if (offset) *offset = c->tensors[i].offset;
    if (numel) *numel = c->tensors[i].numel;
    if (flags) *flags = c->tensors[i].flags;
    return TTP_OK;
}

int ttp_buffer_ptr(ttp_ctx* c, int which, uint32_t index, void** ptr) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!ptr) return fail(TTP_ERR_INVALID, "null output");
    if ((rc = check_buffer_in_mode(c, which))) return rc;
    // m and v live in records in both modes (and are refused before they would be allocated)
    if (which == TTP_BUF_EXP_AVG || which == TTP_BUF_EXP_AVG_SQ || in_records(c, which))
        return fail(TTP_ERR_STATE,
                    "buffer " + std::to_string(which) +
                        " is kept in interleaved state records in this precision mode; use "
                        "ttp_buffer_layout for its addressing, or ttp_upload / ttp_download");
    if (index != TTP_ALL_TENSORS && (rc = check_index(c, index))) return rc;
    if ((rc = set_dev(c))) return rc;
    if ((rc = materialize(c, which))) return rc;
    char* base = (char*)buffer_base(c, which);
    *ptr = index == TTP_ALL_TENSORS ? base
                                    : base + c->tensors[index].offset * buffer_esize(c, which);
    return TTP_OK;
}

int ttp_buffer_layout(ttp_ctx* c, int which, void** base, uint32_t* group, uint32_t* stride) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = check_buffer_in_mode(c, which))) return rc;
    if ((rc = set_dev(c))) return rc;
    if ((rc = materialize(c, which))) return rc;
    if (base) *base = buffer_base(c, which);
    if (group) *group = ttp::kRec;
    if (stride) *stride = buffer_stride(c, which);
    return TTP_OK;
}

int ttp_upload(ttp_ctx* c, int which, uint32_t index, const void* src, uint64_t n, int kind) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (kind == TTP_HOST && (rc = no_capture(c, "an upload from host memory"))) return rc;
    if (!src && n) return fail(TTP_ERR_INVALID, "null source");
    if (kind != TTP_HOST && kind != TTP_DEVICE) return fail(TTP_ERR_INVALID, "bad memory kind");
    if ((rc = check_buffer_in_mode(c, which))) return rc;
    if ((rc = set_dev(c))) return rc;
    uint64_t off, cnt;
    if ((rc = resolve_range(c, index, n, &off, &cnt))) return rc;
    const size_t es = buffer_esize(c, which);
    if (kind == TTP_DEVICE && (rc = check_device_buffer(c, src, cnt * es, "the upload source")))
        return rc;
    if ((rc = materialize(c, which))) return rc;  // after every check
    if (cnt && in_records(c, which)) {
        // record-stored state; a MIXED master upload also writes the bf16 copy
        if ((rc = upload_slot(c, which, off, cnt, src, kind))) return rc;
        if (kind == TTP_HOST) HIP_TRY(hipStreamSynchronize(c->stream));
    } else if (cnt) {
        char* dst = (char*)buffer_base(c, which) + off * es;
        HIP_TRY(hipMemcpyAsync(dst, src, cnt * es,
                               kind == TTP_HOST ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice,
                               c->stream));
        if (c->mode == TTP_MODE_MIXED && which == TTP_BUF_PARAM) {
            clear_hip_error();
            hipLaunchKernelGGL(ttp::bf16_to_master_kernel, dim3(elementwise_grid(c, cnt)),
                               dim3(ttp::kBlock), 0, c->stream, (const uint16_t*)c->param,
                               c->master, buffer_stride(c, TTP_BUF_MASTER), off, cnt);
            HIP_TRY(hipGetLastError());
        } else if (c->mode == TTP_MODE_MIXED && which == TTP_BUF_MASTER) {
            // the SGD layout's contiguous master: its bf16 copy follows, as for records
            clear_hip_error();
            hipLaunchKernelGGL(ttp::master_to_bf16_kernel, dim3(elementwise_grid(c, cnt)),
                               dim3(ttp::kBlock), 0, c->stream, (const float*)c->master,
                               ttp::kRec, (uint16_t*)c->param, off, cnt);
            HIP_TRY(hipGetLastError());
        }
        if (kind == TTP_HOST) HIP_TRY(hipStreamSynchronize(c->stream));
    }
    if (which == TTP_BUF_GRAD) {
        if (index == TTP_ALL_TENSORS) {
            for (uint32_t i = 0; i < (uint32_t)c->tensors.size(); ++i) set_grad_flag(c, i, true);
            stale_sums(c);
        } else {
            set_grad_flag(c, index, true);
            set_fresh(c, index, false);
        }
    }
    return TTP_OK;
}

int ttp_download(ttp_ctx* c, int which, uint32_t index, void* dst, uint64_t n, int kind) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (kind == TTP_HOST && (rc = no_capture(c, "a download to host memory"))) return rc;
    if (!dst && n) return fail(TTP_ERR_INVALID, "null destination");
    if (kind != TTP_HOST && kind != TTP_DEVICE) return fail(TTP_ERR_INVALID, "bad memory kind");
    if ((rc = check_buffer_in_mode(c, which))) return rc;
    if ((rc = set_dev(c))) return rc;
    uint64_t off, cnt;
    if ((rc = resolve_range(c, index, n, &off, &cnt))) return rc;
    const size_t es = buffer_esize(c, which);
    if (kind == TTP_DEVICE &&
        (rc = check_device_buffer(c, dst, cnt * es, "the download destination")))
        return rc;
    if ((rc = materialize(c, which))) return rc;  // after every check
    if (cnt && in_records(c, which)) {
        if ((rc = download_slot(c, which, off, cnt, dst, kind))) return rc;
        if (kind == TTP_HOST) HIP_TRY(hipStreamSynchronize(c->stream));
    } else if (cnt) {
        const char* src = (const char*)buffer_base(c, which) + off * es;
        HIP_TRY(hipMemcpyAsync(dst, src, cnt * es,
                               kind == TTP_HOST ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice,
                               c->stream));
        if (kind == TTP_HOST) HIP_TRY(hipStreamSynchronize(c->stream));
    }
    return TTP_OK;
}

int ttp_set_has_grad(ttp_ctx* c, uint32_t i, int has) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = check_index(c, i))) return rc;
    set_grad_flag(c, i, has != 0);
    set_fresh(c, i, false);  // marks grads written outside the ABI, or drops them
    return TTP_OK;
}

int ttp_get_has_grad(const ttp_ctx* c, uint32_t i, int* has) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = check_index(c, i))) return rc;
    if (!has) return fail(TTP_ERR_INVALID, "null output");
    *has = c->tensors[i].has_grad;
    return TTP_OK;
}

// set_to_none with TTP_ZERO_NO_FILL: flags only (the reference's grad = nullopt touches no
// memory); without set_to_none it would leave present gradients unzeroed, so it is refused
static int parse_zero_mode(int* set_to_none, bool* fill) {
    *fill = (*set_to_none & TTP_ZERO_NO_FILL) == 0;
    *set_to_none &= ~TTP_ZERO_NO_FILL;
    if (!*fill && !*set_to_none)
        return fail(TTP_ERR_INVALID, "TTP_ZERO_NO_FILL needs set_to_none: gradients that stay "
                                     "present must be zeroed");
    return TTP_OK;
}

int ttp_zero_grad(ttp_ctx* c, int set_to_none) {
    int rc = check_ctx(c);
    if (rc) return rc;
    bool fill;
    if ((rc = parse_zero_mode(&set_to_none, &fill))) return rc;
    if ((rc = set_dev(c))) return rc;
    if (fill && (rc = zero_device(c, c->grad, c->total * grad_esize(c)))) return rc;
    if (set_to_none) {
        for (uint32_t i = 0; i < (uint32_t)c->tensors.size(); ++i) set_grad_flag(c, i, false);
    }
    stale_sums(c);
    return TTP_OK;
}

int ttp_zero_grad_subset(ttp_ctx* c, const uint32_t* indices, uint32_t n, int set_to_none) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (n && !indices) return fail(TTP_ERR_INVALID, "null index list");
    bool fill;
    if ((rc = parse_zero_mode(&set_to_none, &fill))) return rc;
    if ((rc = set_dev(c))) return rc;
    if (!fill) {  // flags only: the indices are checked here, no work table is needed
        std::vector<uint8_t> seen(c->tensors.size(), 0);
        for (uint32_t k = 0; k < n; ++k) {
            if ((rc = check_index(c, indices[k]))) return rc;
            if (seen[indices[k]])
                return fail(TTP_ERR_INVALID,
                            "tensor index " + std::to_string(indices[k]) + " listed twice");
            seen[indices[k]] = 1;
        }
        for (uint32_t k = 0; k < n; ++k) {
            set_grad_flag(c, indices[k], false);
            set_fresh(c, indices[k], false);
        }
        return TTP_OK;
    }
    static const uint32_t none = 0;
    const WorkTables* w;
    std::vector<uint32_t> active;
    if ((rc = select_tables(c, indices ? indices : &none, n, &w, &active, false))) return rc;
    if (w->n_chunks) {
        const uint32_t grid = std::min(w->n_chunks, kMaxGridBlocks);  // grid-stride kernel
        clear_hip_error();
        if (bf16_grads(c))
            hipLaunchKernelGGL(ttp::zero_chunks_kernel<uint16_t>, dim3(grid), dim3(ttp::kUpdBlock),
                               0, c->stream, (uint16_t*)c->grad, w->chunks, w->n_chunks);
        else
            hipLaunchKernelGGL(ttp::zero_chunks_kernel<float>, dim3(grid), dim3(ttp::kUpdBlock),
                               0, c->stream, (float*)c->grad, w->chunks, w->n_chunks);
        HIP_TRY(hipGetLastError());
    }
    // set_to_none = 0 leaves the has-grad flags as they are, as ttp_zero_grad(ctx, 0) and
    // torch's zero_grad(set_to_none=False) do: a tensor without a grad stays without one
    for (uint32_t k = 0; k < n; ++k) {
        if (set_to_none) set_grad_flag(c, indices[k], false);
        set_fresh(c, indices[k], false);
    }
    return TTP_OK;
}

int ttp_accumulate_grad(ttp_ctx* c, uint32_t index, const void* src, uint64_t n, int dtype,
                        int kind) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = check_index(c, index))) return rc;
    const bool with_sums = (dtype & TTP_ACCUM_SUMSQ) != 0;
    dtype &= ~TTP_ACCUM_SUMSQ;
    if (dtype != TTP_DTYPE_F32 && dtype != TTP_DTYPE_BF16)
        return fail(TTP_ERR_INVALID, "src_dtype must be TTP_DTYPE_F32 or TTP_DTYPE_BF16, "
                                     "optionally | TTP_ACCUM_SUMSQ");
    if (kind != TTP_HOST && kind != TTP_DEVICE) return fail(TTP_ERR_INVALID, "bad memory kind");
    if (kind == TTP_HOST && (rc = no_capture(c, "accumulating a host gradient"))) return rc;
    // Whether the kernel assigns (no grad yet) or adds is fixed when the call is captured.
    // Every launch must therefore find the flag as the capture did: a call earlier in the same
    // capture must have set it (zero_grad with set_to_none, set_has_grad, a gradient upload
    // or an accumulate; zeroing to zeros leaves the flag as the launch finds it).
    if (c->capturing && !(c->cap_touched[index] & kCapGrad))
        return fail(TTP_ERR_STATE,
                    "a captured accumulate into tensor " + std::to_string(index) +
                        " must follow a call of the same capture that sets that tensor's "
                        "has-grad flag (zero_grad with set_to_none, set_has_grad, a gradient "
                        "upload or an accumulate): whether it assigns or adds is fixed when it "
                        "is captured");
    TensorRec& t = c->tensors[index];
    if (n != t.numel)
        return fail(TTP_ERR_RANGE, "tensor " + std::to_string(index) + " has " +
                                       std::to_string(t.numel) + " elements, got " +
                                       std::to_string(n));
    if (!src && n) return fail(TTP_ERR_INVALID, "null source");
    if ((rc = set_dev(c))) return rc;
    const size_t sbytes = dtype == TTP_DTYPE_BF16 ? 2 : 4;
    if (kind == TTP_DEVICE &&
        (rc = check_device_buffer(c, src, n * sbytes, "the incoming gradient")))
        return rc;
    // with its sum: one tile sum per 16 KiB norm tile of the tensor's gradients
    const uint64_t ntiles = with_sums ? (n + norm_tile(c) - 1) / norm_tile(c) : 0;
    if (with_sums) {
        if (ntiles >= (1u << 24))
            return fail(TTP_ERR_RANGE, "tensor " + std::to_string(index) + " has " +
                                           std::to_string(ntiles) +
                                           " tiles of 16 KiB of gradients; an accumulate with "
                                           "its sum takes at most 2^24 - 1");
    }
    if (n) {
        const void* dsrc = src;
        if (kind == TTP_HOST) {
            if ((rc = ensure_staging(c, n * sbytes))) return rc;
            HIP_TRY(hipMemcpyAsync(c->staging, src, n * sbytes, hipMemcpyHostToDevice, c->stream));
            dsrc = c->staging;
        }
        const int first = t.has_grad ? 0 : 1;
        const bool mixed = bf16_grads(c), bf16 = dtype == TTP_DTYPE_BF16;
        const uint64_t tiles = (n + norm_tile(c) - 1) / norm_tile(c);
        clear_hip_error();
        if (tiles < (1u << 24)) {
            // one-wave blocks, kAccBlocksPerTile per 16 KiB tile of the tensor's gradients
            // (with_sums: their sums too); fewer than 2^26 blocks of 64 lanes
            const int32_t scaler_on = c->scaler.enabled ? 1 : 0;
            const bool vec = ((uintptr_t)dsrc & 15u) == 0;
            const dim3 grid((uint32_t)tiles * ttp::kAccBlocksPerTile), block(ttp::kAccLanes);
            const DevState* st = c->st;
            double* ts = c->acc_tiles + (uint64_t)c->host_tile_base[index] * ttp::kWaves;
            uint32_t* pend = c->tsum_pending + index;
#define TTP_ACC_TILES(S, G, V, SUMS)                                                             \
    hipLaunchKernelGGL((ttp::accumulate_grad_tiles_kernel<S, G, V, SUMS>), grid, block, 0,       \
                       c->stream, (G*)c->grad + t.offset, (const S*)dsrc, n, first, st, scaler_on, \
                       ts, pend)
#define TTP_ACC_SRC(S, G)                                   \
    do {                                                    \
        if (vec && with_sums) TTP_ACC_TILES(S, G, true, true);   \
        else if (vec) TTP_ACC_TILES(S, G, true, false);          \
        else if (with_sums) TTP_ACC_TILES(S, G, false, true);    \
        else TTP_ACC_TILES(S, G, false, false);                  \
    } while (0)
            if (mixed && bf16)
                TTP_ACC_SRC(uint16_t, uint16_t);
            else if (mixed)
                TTP_ACC_SRC(float, uint16_t);
            else if (bf16)
                TTP_ACC_SRC(uint16_t, float);
            else
                TTP_ACC_SRC(float, float);
#undef TTP_ACC_SRC
#undef TTP_ACC_TILES
        } else {
            // beyond a launch's 2^32 work-items at one tile per block: the grid-stride kernel
            const uint32_t grid = elementwise_grid(c, n);
            if (mixed && bf16)
                hipLaunchKernelGGL((ttp::accumulate_grad_kernel<uint16_t, uint16_t>), dim3(grid),
                                   dim3(ttp::kBlock), 0, c->stream, (uint16_t*)c->grad + t.offset,
                                   (const uint16_t*)dsrc, n, first);
            else if (mixed)
                hipLaunchKernelGGL((ttp::accumulate_grad_kernel<float, uint16_t>), dim3(grid),
                                   dim3(ttp::kBlock), 0, c->stream, (uint16_t*)c->grad + t.offset,
                                   (const float*)dsrc, n, first);
            else if (bf16)
                hipLaunchKernelGGL((ttp::accumulate_grad_kernel<uint16_t, float>), dim3(grid),
                                   dim3(ttp::kBlock), 0, c->stream, (float*)c->grad + t.offset,
                                   (const uint16_t*)dsrc, n, first);
            else
                hipLaunchKernelGGL((ttp::accumulate_grad_kernel<float, float>), dim3(grid),
                                   dim3(ttp::kBlock), 0, c->stream, (float*)c->grad + t.offset,
                                   (const float*)dsrc, n, first);
        }
        HIP_TRY(hipGetLastError());
        if (kind == TTP_HOST) HIP_TRY(hipStreamSynchronize(c->stream));
    }
    // an empty tensor's sum is never read (no step updates it)
    if (with_sums) c->acc_sums_used = true;
    set_grad_flag(c, index, true);
    set_fresh(c, index, with_sums);
    return TTP_OK;
}

static_assert(ttp::kMultiMax == TTP_ACCUM_MULTI_MAX, "the header's limit is the kernel table's");

int ttp_accumulate_grad_multi(ttp_ctx* c, const uint32_t* indices, const void* const* srcs,
                              uint32_t n, int dtype) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (n > ttp::kMultiMax)
        return fail(TTP_ERR_RANGE, std::to_string(n) + " tensors in one call; at most " +
                                       std::to_string(ttp::kMultiMax));
    if (n && (!indices || !srcs)) return fail(TTP_ERR_INVALID, "null index or source list");
    const bool with_sums = (dtype & TTP_ACCUM_SUMSQ) != 0;
    dtype &= ~TTP_ACCUM_SUMSQ;
    if (dtype != TTP_DTYPE_F32 && dtype != TTP_DTYPE_BF16)
        return fail(TTP_ERR_INVALID, "src_dtype must be TTP_DTYPE_F32 or TTP_DTYPE_BF16, "
                                     "optionally | TTP_ACCUM_SUMSQ");
    if ((rc = set_dev(c))) return rc;
    const size_t sbytes = dtype == TTP_DTYPE_BF16 ? 2 : 4;
    const uint64_t tile = norm_tile(c);
    std::vector<uint8_t> seen(c->tensors.size(), 0);
    ttp::MultiAccArgs a{};
    uint64_t tiles = 0;
    bool vec = true;
    // every check first: a refused call changes nothing
    for (uint32_t k = 0; k < n; ++k) {
        const uint32_t i = indices[k];
        if ((rc = check_index(c, i))) return rc;
        if (seen[i]) return fail(TTP_ERR_INVALID, "tensor index " + std::to_string(i) +
                                                      " listed twice");
        seen[i] = 1;
        if (c->capturing && !(c->cap_touched[i] & kCapGrad))
            return fail(TTP_ERR_STATE,
                        "a captured accumulate into tensor " + std::to_string(i) +
                            " must follow a call of the same capture that sets that tensor's "
                            "has-grad flag (zero_grad with set_to_none, set_has_grad, a "
                            "gradient upload or an accumulate): whether it assigns or adds is "
                            "fixed when it is captured");
        const TensorRec& t = c->tensors[i];
        if (!t.numel) continue;
        if (!srcs[k]) return fail(TTP_ERR_INVALID, "null source for tensor " + std::to_string(i));
        if ((rc = check_device_buffer(c, srcs[k], t.numel * sbytes, "an incoming gradient")))
            return rc;
        vec = vec && ((uintptr_t)srcs[k] & 15u) == 0;
        tiles += (t.numel + tile - 1) / tile;
        if (tiles >= (1u << 24))
            return fail(TTP_ERR_RANGE, "the call covers " + std::to_string(tiles) +
                                           " or more tiles of 16 KiB of gradients; at most "
                                           "2^24 - 1 per call: split it");
        const uint32_t m = a.n++;
        if (!t.has_grad) a.first[m >> 5] |= 1u << (m & 31);
        a.tile_end[m] = (uint32_t)tiles;
        a.tile_base[m] = c->host_tile_base[i];
        a.tensor[m] = i;
        a.offset[m] = t.offset;
        a.numel[m] = t.numel;
        a.src[m] = srcs[k];
    }
    if (a.n) {
        const int32_t scaler_on = c->scaler.enabled ? 1 : 0;
        const bool mixed = bf16_grads(c), bf16 = dtype == TTP_DTYPE_BF16;
        const dim3 grid((uint32_t)tiles * ttp::kAccBlocksPerTile), block(ttp::kAccLanes);
        clear_hip_error();
#define TTP_ACC_MULTI(S, G, V, SUMS)                                                          \
    hipLaunchKernelGGL((ttp::accumulate_grads_multi_kernel<S, G, V, SUMS>), grid, block, 0,   \
                       c->stream, (G*)c->grad, a, (const DevState*)c->st, scaler_on,           \
                       c->acc_tiles, c->tsum_pending)
#define TTP_ACC_MULTI_SRC(S, G)                                   \
    do {                                                          \
        if (vec && with_sums) TTP_ACC_MULTI(S, G, true, true);    \
        else if (vec) TTP_ACC_MULTI(S, G, true, false);           \
        else if (with_sums) TTP_ACC_MULTI(S, G, false, true);     \
        else TTP_ACC_MULTI(S, G, false, false);                   \
    } while (0)
        if (mixed && bf16)
            TTP_ACC_MULTI_SRC(uint16_t, uint16_t);
        else if (mixed)
            TTP_ACC_MULTI_SRC(float, uint16_t);
        else if (bf16)
            TTP_ACC_MULTI_SRC(uint16_t, float);
        else
            TTP_ACC_MULTI_SRC(float, float);
#undef TTP_ACC_MULTI_SRC
#undef TTP_ACC_MULTI
        HIP_TRY(hipGetLastError());
    }
    if (with_sums) c->acc_sums_used = true;
    for (uint32_t k = 0; k < n; ++k) {
        set_grad_flag(c, indices[k], true);
        set_fresh(c, indices[k], with_sums);
    }
    return TTP_OK;
}

// `scratch_partials` non-null: the no-allocation step.  It builds no work or bias table and
// allocates no state (each missing one is refused with TTP_ERR_STATE), records no timing
// events, and its norm pass writes its partials there (at most kNoAllocPartials).
static int adam_step_impl(ttp_ctx* c, const ttp_adam_hparams* hp, const uint32_t* subset,
                          uint32_t nsub, ttp_step_report* report,
                          double* scratch_partials = nullptr) {
    const bool noalloc = scratch_partials != nullptr;
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = bf16_store_refuses(c, "an Adam step"))) return rc;
    if (!hp) return fail(TTP_ERR_INVALID, "null hyperparameters");
    // py/optim.py:33-41
    if (!(hp->lr > 0)) return fail(TTP_ERR_INVALID, "lr must be > 0");
    if (!(hp->eps > 0)) return fail(TTP_ERR_INVALID, "eps must be > 0");
    if (!(hp->beta1 > 0 && hp->beta1 < 1 && hp->beta2 > 0 && hp->beta2 < 1))
        return fail(TTP_ERR_INVALID, "betas must be in (0, 1)");
    if (!(hp->weight_decay >= 0)) return fail(TTP_ERR_INVALID, "weight_decay must be >= 0");
    if (hp->flags & ~kStepFlags) return fail(TTP_ERR_INVALID, "unknown step flags");
    if (report && (rc = no_capture(c, "a step report (synchronises)"))) return rc;
    if ((rc = set_dev(c))) return rc;
    if (noalloc && !c->exp_avg)
        return fail(TTP_ERR_STATE, "the first Adam step of an FP32 store, or of a MIXED store "
                                   "in the SGD layout, allocates m and v, which the "
                                   "no-allocation step does not: step once with "
                                   "ttp_adam_step[_subset] first");
    const WorkTables* w;
    std::vector<uint32_t> active;
    if ((rc = select_tables(c, subset, nsub, &w, &active, true, !noalloc))) return rc;
    const Chunk* chunks = w->chunks;
    const uint32_t n = w->n_chunks;

    const bool scaler = c->scaler.enabled != 0;
    const bool clip = hp->max_grad_norm > 0;
    const bool need_norm = scaler || clip;
    const bool devt = t_on_device(c);
    const bool from_sums = need_norm && (hp->flags & TTP_STEP_TENSOR_SUMS);
    const bool defer = scaler && (hp->flags & TTP_STEP_DEFER_SCALE);
    if (from_sums && (rc = check_sums_current(c, active))) return rc;
    if (noalloc && need_norm && !from_sums && norm_split(c, w->n_tiles).partials() > kNoAllocPartials)
        return fail(TTP_ERR_RANGE,
                    "the norm pass would write " +
                        std::to_string(norm_split(c, w->n_tiles).partials()) +
                        " partials; the no-allocation step holds at most " +
                        std::to_string(kNoAllocPartials) + " (lower TTP_NORM_GRID)");
    // the device table of bias corrections; built in host-count mode too (once per betas) so
    // that a later capture finds it, except when betas so close to 1 make it too long.  The
    // no-allocation step needs it only when the step count lives on the device.
    if ((!noalloc || devt) &&
        (rc = ensure_bias_table(c, hp->beta1, hp->beta2, !noalloc)) && (devt || noalloc))
        return rc;
    // m and v last, once nothing above can refuse the step: in the SGD layout this moves the
    // master into new records, which a refused call must not do
    if ((rc = ensure_adam_state(c))) return rc;
    if ((need_norm || devt) &&
        (rc = launch_prologue(c, w, need_norm, hp->max_grad_norm, false, devt, devt, from_sums,
                              defer, scratch_partials)))
        return rc;

    ttp::AdamArgs a{};
    a.chunks = chunks;
    a.nchunks = n;
    // py/optim.py:60-71: each hyperparameter is a full_like fill, i.e. rounded once to fp32
    a.lr = (float)hp->lr;
    a.b1 = (float)hp->beta1;
    a.omb1 = (float)(1.0 - hp->beta1);
    a.b2 = (float)hp->beta2;
    a.omb2 = (float)(1.0 - hp->beta2);
    a.eps = (float)hp->eps;
    a.decay_mul = (float)(1.0 - hp->lr * hp->weight_decay);
    a.wd = (float)hp->weight_decay;
    a.flags = (hp->decoupled ? ttp::kDecoupled : 0u) | (hp->weight_decay != 0.0 ? ttp::kWdOn : 0u);
    if (scaler) a.flags |= ttp::kUseInv | ttp::kCheckSkip;
    if (devt) a.flags |= ttp::kDevBias;
    if (clip) a.flags |= ttp::kUseClip;
    a.st = (need_norm || devt) ? c->st : nullptr;
    if (!devt) {
        c->host_t += 1;  // py/optim.py:50
        a.bias1 = (float)(1.0 - std::pow(hp->beta1, (double)c->host_t));
        a.bias2 = (float)(1.0 - std::pow(hp->beta2, (double)c->host_t));
    } else {
        a.bias1 = a.bias2 = 1.0f;  // replaced by the device values
    }
    if (n) {
        TimedLaunch tl(c, TTP_KERNEL_UPDATE, !noalloc);
        const uint16_t* g16 = (const uint16_t*)c->grad;
        const float* g32 = (const float*)c->grad;
        uint16_t* p16 = (uint16_t*)c->param;
        ttp::AdamArgs al = a;
        al.st = c->st;  // the lane forms read the device state unconditionally
        clear_hip_error();
        if (grads_cached(c, w) && c->mode == TTP_MODE_MIXED)
            launch_lanes(c,
                         (uint64_t)n * ttp::lane_parts<kLaneAdamMixedCached, kLanesAdamMixedCached,
                                                       kItAdamMixedCached>(),
                         kLanesAdamMixedCached, [&](dim3 g, uint64_t p0) {
                hipLaunchKernelGGL(
                    (ttp::adam_lane_kernel<uint16_t, true, kLaneAdamMixedCached,
                                           kLanesAdamMixedCached, kItAdamMixedCached>), g,
                    dim3(kLanesAdamMixedCached), 0, c->stream, g16, c->records, (float*)nullptr,
                    p16, al, p0);
            });
        else if (c->mode == TTP_MODE_MIXED)
            launch_lanes(c,
                         (uint64_t)n *
                             ttp::lane_parts<kLaneAdamMixed, kLanesAdamMixed, kItAdamMixed>(),
                         kLanesAdamMixed, [&](dim3 g, uint64_t p0) {
                hipLaunchKernelGGL(
                    (ttp::adam_lane_kernel<uint16_t, true, kLaneAdamMixed, kLanesAdamMixed,
                                           kItAdamMixed>), g,
                    dim3(kLanesAdamMixed), 0, c->stream, g16, c->records, (float*)nullptr, p16,
                    al, p0);
            });
        else
            launch_lanes(c,
                         (uint64_t)n *
                             ttp::lane_parts<kLaneAdamFp32, kLanesAdamFp32, kItAdamFp32>(),
                         kLanesAdamFp32, [&](dim3 g, uint64_t p0) {
                hipLaunchKernelGGL(
                    (ttp::adam_lane_kernel<float, false, kLaneAdamFp32, kLanesAdamFp32,
                                           kItAdamFp32>), g,
                    dim3(kLanesAdamFp32), 0, c->stream, g32, c->records, c->master,
                    (uint16_t*)nullptr, al, p0);
            });
        HIP_TRY(hipGetLastError());
        tl.done();
    }
    consume_sums(c, active, scaler && !defer);
    if (report) return fill_report(c, need_norm, report);
    return TTP_OK;
}

static int sgd_step_impl(ttp_ctx* c, const ttp_sgd_hparams* hp, const uint32_t* subset,
                         uint32_t nsub, ttp_step_report* report) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!hp) return fail(TTP_ERR_INVALID, "null hyperparameters");
    if (!(hp->lr > 0)) return fail(TTP_ERR_INVALID, "lr must be > 0");  // py/optim.py:9-10
    if (!(hp->momentum >= 0)) return fail(TTP_ERR_INVALID, "momentum must be >= 0");
    if (!(hp->weight_decay >= 0)) return fail(TTP_ERR_INVALID, "weight_decay must be >= 0");
    if (hp->nesterov && (hp->momentum <= 0 || hp->dampening != 0))
        return fail(TTP_ERR_INVALID, "nesterov needs momentum > 0 and zero dampening");
    if (hp->flags & ~kStepFlags) return fail(TTP_ERR_INVALID, "unknown step flags");
    if (c->mode == TTP_MODE_BF16 && (hp->momentum != 0.0 || hp->weight_decay != 0.0))
        return fail(TTP_ERR_INVALID, "a TTP_MODE_BF16 store steps plain SGD only (the "
                                     "reference's `data - lr * grad` in bf16): momentum and "
                                     "weight decay need fp32 state; create the store "
                                     "TTP_MODE_MIXED for them");
    if (report && (rc = no_capture(c, "a step report (synchronises)"))) return rc;
    if ((rc = set_dev(c))) return rc;
    const bool mom = hp->momentum != 0.0;
    const WorkTables* w;
    std::vector<uint32_t> active;
    if ((rc = select_tables(c, subset, nsub, &w, &active))) return rc;
    const Chunk* chunks = w->chunks;
    const uint32_t n = w->n_chunks;

    const bool scaler = c->scaler.enabled != 0;
    const bool clip = hp->max_grad_norm > 0;
    const bool need_norm = scaler || clip;
    const bool devt = t_on_device(c);
    const bool from_sums = need_norm && (hp->flags & TTP_STEP_TENSOR_SUMS);
    const bool defer = scaler && (hp->flags & TTP_STEP_DEFER_SCALE);
    if (from_sums && (rc = check_sums_current(c, active))) return rc;
    // the momentum buffer once nothing above can refuse the step (a refused call changes
    // nothing, not even what a checkpoint would hold)
    if (mom && (rc = ensure_momentum(c))) return rc;
    if ((need_norm || devt) &&
        (rc = launch_prologue(c, w, need_norm, hp->max_grad_norm, false, false, devt, from_sums,
                              defer)))
        return rc;
    if (!devt) c->host_t += 1;

    ttp::SgdArgs a{};
    a.chunks = chunks;
    a.nchunks = n;
    a.lr = (float)hp->lr;
    a.mu = (float)hp->momentum;
    a.omd = (float)(1.0 - hp->dampening);
    a.wd = (float)hp->weight_decay;
    a.mom_init = c->mom_init;
    a.flags = (hp->weight_decay != 0.0 ? ttp::kWdOn : 0u) | (mom ? ttp::kMomOn : 0u) |
              (hp->nesterov ? ttp::kNesterov : 0u);
    if (scaler) a.flags |= ttp::kUseInv | ttp::kCheckSkip;
    if (clip) a.flags |= ttp::kUseClip;
    a.st = (need_norm || devt) ? c->st : nullptr;
    if (n) {
        const dim3 block(ttp::kUpdBlock);
        TimedLaunch tl(c, TTP_KERNEL_UPDATE);
        const uint16_t* g16 = (const uint16_t*)c->grad;
        const float* g32 = (const float*)c->grad;
        uint16_t* p16 = (uint16_t*)c->param;
        ttp::SgdArgs al = a;
        al.st = c->st;  // the lane forms read the device state unconditionally
        clear_hip_error();
        // launches the lane-form kernel of shape <E, LN, IT> with master stride MS
#define TTP_SGD_LANES(GT, MIXED, MS, E, LN, IT, G, P16)                                        \
    launch_lanes(c, (uint64_t)n * ttp::lane_parts<E, LN, IT>(), LN, [&](dim3 g, uint64_t p0) { \
        hipLaunchKernelGGL((ttp::sgd_lane_kernel<GT, MIXED, MS, E, LN, IT>), g, dim3(LN), 0,  \
                           c->stream, G, c->master, c->momentum, P16, al, p0);                \
    })
        if (c->mode == TTP_MODE_BF16)
            launch_lanes(c, (uint64_t)n * ttp::lane_parts<kLaneSgdBf16, kLanesSgdBf16, kItSgdBf16>(),
                         kLanesSgdBf16, [&](dim3 g, uint64_t p0) {
                hipLaunchKernelGGL((ttp::sgd_bf16_lane_kernel<kLaneSgdBf16, kLanesSgdBf16,
                                                              kItSgdBf16>),
                                   g, dim3(kLanesSgdBf16), 0, c->stream, g16, p16, al, p0);
            });
        else if (c->mode == TTP_MODE_MIXED && c->sgd_layout && !mom)
            TTP_SGD_LANES(uint16_t, true, ttp::kRec, kLaneSgdPlainContig, kLanesSgdPlainContig,
                          kItSgdPlainContig, g16, p16);
        else if (c->mode == TTP_MODE_MIXED && c->sgd_layout)
            TTP_SGD_LANES(uint16_t, true, ttp::kRec, kLaneSgdMomContig, kLanesSgdMomContig,
                          kItSgdMomContig, g16, p16);
        else if (!mom && c->mode == TTP_MODE_MIXED)
            TTP_SGD_LANES(uint16_t, true, ttp::kStrideMixed, kLaneSgdPlainMixed,
                          kLanesSgdPlainMixed, kItSgdPlainMixed, g16, p16);
        else if (grads_cached(c, w) && c->mode == TTP_MODE_MIXED)
            hipLaunchKernelGGL((ttp::sgd_kernel<uint16_t, true, ttp::kStrideMixed>), dim3(n),
                               block, c->upd_lds, c->stream, g16, c->master, c->momentum, p16,
                               a);
        else if (c->mode == TTP_MODE_MIXED)
            TTP_SGD_LANES(uint16_t, true, ttp::kStrideMixed, kLaneSgdMixed, kLanesSgdMixed,
                          kItSgdMixed, g16, p16);
        else if (!mom)
            TTP_SGD_LANES(float, false, ttp::kRec, kLaneSgdPlainFp32, kLanesSgdPlainFp32,
                          kItSgdPlainFp32, g32, (uint16_t*)nullptr);
        else
            TTP_SGD_LANES(float, false, ttp::kRec, kLaneSgdFp32, kLanesSgdFp32, kItSgdFp32, g32,
                          (uint16_t*)nullptr);
#undef TTP_SGD_LANES
        HIP_TRY(hipGetLastError());
        tl.done();
        if (mom) {
            // the stepped tensors now hold a momentum buffer (torch: state created on first
            // use); with loss scaling the device decides, since the step may be skipped, and
            // once captured the marking is part of every replay
            bool needed = scaler || devt;
            for (uint32_t i : active)
                if (!c->host_mom_init[i]) needed = true;
            if (needed) {
                const uint32_t g =
                    std::max<uint32_t>(1, std::min<uint32_t>((n + ttp::kBlock - 1) / ttp::kBlock, 1024));
                clear_hip_error();
                hipLaunchKernelGGL(ttp::mark_mom_init_kernel, dim3(g), dim3(ttp::kBlock), 0,
                                   c->stream, chunks, n, c->mom_init, (const DevState*)c->st,
                                   scaler ? 1 : 0);
                HIP_TRY(hipGetLastError());
            }
            if (!scaler && !devt)
                for (uint32_t i : active) c->host_mom_init[i] = 1;
        }
    }
    consume_sums(c, active, scaler && !defer);
    if (report) return fill_report(c, need_norm, report);
    return TTP_OK;
}

}  // extern "C"

// (the step implementations above are static; their C entry points follow)
extern "C" {

int ttp_adam_step(ttp_ctx* c, const ttp_adam_hparams* hp, ttp_step_report* report) {
    return adam_step_impl(c, hp, nullptr, 0, report);
}

int ttp_adam_step_subset(ttp_ctx* c, const ttp_adam_hparams* hp, const uint32_t* indices,
                         uint32_t n, ttp_step_report* report) {
    if (n && !indices) return fail(TTP_ERR_INVALID, "null index list");
    static const uint32_t none = 0;
    return adam_step_impl(c, hp, indices ? indices : &none, n, report);
}

int ttp_adam_step_noalloc(ttp_ctx* c, const ttp_adam_hparams* hp, const uint32_t* indices,
                          uint32_t n) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (n && !indices) return fail(TTP_ERR_INVALID, "null index list");
    if ((rc = bf16_store_refuses(c, "an Adam step"))) return rc;
    if ((rc = set_dev(c))) return rc;
    // The device's scratch array is shared by every context: an eager step on another stream
    // than the last one's first waits for that step's event (host calls on one device are
    // serialised by the lock).  A captured step is ordered by its caller at each launch.
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    auto it = g_scratch.find(c->device);
    if (it == g_scratch.end() || !it->second.ptr)
        return fail(TTP_ERR_STATE, "no scratch array found for this device");
    ScratchDev& d = it->second;
    if (!c->capturing && d.used && d.last != c->stream)
        HIP_TRY(hipStreamWaitEvent(c->stream, d.done, 0));
    rc = adam_step_impl(c, hp, indices, n, nullptr, d.ptr);
    if (rc == TTP_OK && !c->capturing) {
        HIP_TRY(hipEventRecord(d.done, c->stream));
        d.last = c->stream;
        d.used = true;
    }
    return rc;
}

int ttp_sgd_step(ttp_ctx* c, const ttp_sgd_hparams* hp, ttp_step_report* report) {
    return sgd_step_impl(c, hp, nullptr, 0, report);
}

int ttp_sgd_step_subset(ttp_ctx* c, const ttp_sgd_hparams* hp, const uint32_t* indices,
                        uint32_t n, ttp_step_report* report) {
    if (n && !indices) return fail(TTP_ERR_INVALID, "null index list");
    static const uint32_t none = 0;
    return sgd_step_impl(c, hp, indices ? indices : &none, n, report);
}

int ttp_grad_norm(ttp_ctx* c, double* norm) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!norm) return fail(TTP_ERR_INVALID, "null output");
    if ((rc = no_capture(c, "ttp_grad_norm (synchronises)"))) return rc;
    if ((rc = set_dev(c))) return rc;
    const WorkTables* w;
    if ((rc = select_tables(c, nullptr, 0, &w, nullptr))) return rc;
    if ((rc = launch_prologue(c, w, true, 0.0, true, false, false))) return rc;
    DevState s;
    if ((rc = read_state(c, &s))) return rc;
    *norm = s.norm;
    return TTP_OK;
}

int ttp_grad_sumsq_tensors(ttp_ctx* c, const uint32_t* indices, uint32_t n) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (n && !indices) return fail(TTP_ERR_INVALID, "null index list");
    if ((rc = set_dev(c))) return rc;
    static const uint32_t none = 0;
    const WorkTables* w;
    std::vector<uint32_t> active;
    if ((rc = select_tables(c, indices ? indices : &none, n, &w, &active))) return rc;
    // one 256-lane block per tile, and a launch holds fewer than 2^32 work-items
    if (w->n_tiles >= (1u << 24))
        return fail(TTP_ERR_RANGE, "a gradient-sum call covers " + std::to_string(w->n_tiles) +
                                       " tiles of 16 KiB; at most 2^24 - 1 (256 GiB of "
                                       "gradients) per call: split the bucket");
    if ((rc = ensure_tile_sums(c, w->n_tiles, "a first gradient-sum call over this many tiles")))
        return rc;
    if (w->n_tiles) {
        // one norm-pass block per tile (each block's partial is its tile's sum), then one
        // block per tensor over its run of tiles
        const int32_t scaler_on = c->scaler.enabled ? 1 : 0;
        clear_hip_error();
        if (bf16_grads(c))
            hipLaunchKernelGGL((ttp::norm_partials_kernel<uint16_t, false>), dim3(w->n_tiles),
                               dim3(ttp::kBlock), 0, c->stream, (const uint16_t*)c->grad,
                               w->tiles, 0u, w->n_tiles, (const DevState*)c->st, scaler_on,
                               c->tile_sums);
        else
            hipLaunchKernelGGL((ttp::norm_partials_kernel<float, false>), dim3(w->n_tiles),
                               dim3(ttp::kBlock), 0, c->stream, (const float*)c->grad, w->tiles,
                               0u, w->n_tiles, (const DevState*)c->st, scaler_on, c->tile_sums);
        HIP_TRY(hipGetLastError());
        clear_hip_error();
        hipLaunchKernelGGL(ttp::tensor_sums_kernel, dim3(w->n_tensors), dim3(ttp::kBlock), 0,
                           c->stream, c->tile_sums, w->tile_start, w->tensor_ids, c->tsum,
                           c->tsum_pending);
        HIP_TRY(hipGetLastError());
    }
    for (uint32_t i : active) set_fresh(c, i, true);
    return TTP_OK;
}

int ttp_get_step(ttp_ctx* c, uint64_t* step) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!step) return fail(TTP_ERR_INVALID, "null output");
    if (!t_on_device(c)) {
        *step = c->host_t;
        return TTP_OK;
    }
    if ((rc = no_capture(c, "ttp_get_step (synchronises)"))) return rc;
    if ((rc = set_dev(c))) return rc;
    DevState s;
    if ((rc = read_state(c, &s))) return rc;
    *step = s.t;
    return TTP_OK;
}

int ttp_set_step(ttp_ctx* c, uint64_t step) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = no_capture(c, "ttp_set_step"))) return rc;
    if ((rc = set_dev(c))) return rc;
    c->host_t = step;
    HIP_TRY(hipStreamSynchronize(c->stream));
    HIP_TRY(hipMemcpy(&c->st->t, &step, sizeof(step), hipMemcpyHostToDevice));
    return TTP_OK;
}

int ttp_scaler_configure(ttp_ctx* c, const ttp_scaler_config* cfg) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!cfg) return fail(TTP_ERR_INVALID, "null scaler config");
    if (cfg->enabled) {
        if (!(cfg->init_scale > 0)) return fail(TTP_ERR_INVALID, "init_scale must be > 0");
        if (!(cfg->growth_factor > 1)) return fail(TTP_ERR_INVALID, "growth_factor must be > 1");
        if (!(cfg->backoff_factor > 0 && cfg->backoff_factor < 1))
            return fail(TTP_ERR_INVALID, "backoff_factor must be in (0, 1)");
        if (cfg->growth_interval <= 0) return fail(TTP_ERR_INVALID, "growth_interval must be > 0");
    }
    if ((rc = no_capture(c, "ttp_scaler_configure"))) return rc;
    if (c->n_graphs && !same_scaler_settings(c->scaler, *cfg))
        return fail(TTP_ERR_STATE, "the loss-scaler settings are part of this context's captured "
                                   "graphs; destroy them before changing the settings");
    if ((rc = set_dev(c))) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    DevState s;
    HIP_TRY(hipMemcpy(&s, c->st, sizeof(s), hipMemcpyDeviceToHost));
    const bool was = t_on_device(c), will = cfg->enabled || c->device_t;
    if (was && !will) c->host_t = s.t;  // device count -> host
    if (!was && will) s.t = c->host_t;  // host count -> device
    if (cfg->enabled) {
        s.scale = (float)cfg->init_scale;
        s.growth_tracker = 0;
    }
    s.pending = 0;
    HIP_TRY(hipMemcpy(c->st, &s, sizeof(s), hipMemcpyHostToDevice));
    c->scaler = *cfg;
    stale_sums(c);  // the sums are of gradients unscaled by the old scale
    return TTP_OK;
}

int ttp_scaler_get(ttp_ctx* c, float* scale, int32_t* tracker) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = no_capture(c, "ttp_scaler_get (synchronises)"))) return rc;
    if ((rc = set_dev(c))) return rc;
    DevState s;
    if ((rc = read_state(c, &s))) return rc;
    if (scale) *scale = s.scale;
    if (tracker) *tracker = s.growth_tracker;
    return TTP_OK;
}

int ttp_scaler_set(ttp_ctx* c, float scale, int32_t tracker) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!(scale > 0) || tracker < 0) return fail(TTP_ERR_INVALID, "scale must be > 0, tracker >= 0");
    if ((rc = no_capture(c, "ttp_scaler_set"))) return rc;
    if ((rc = set_dev(c))) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    DevState s;
    HIP_TRY(hipMemcpy(&s, c->st, sizeof(s), hipMemcpyDeviceToHost));
    s.scale = scale;
    s.growth_tracker = tracker;
    s.pending = 0;
    HIP_TRY(hipMemcpy(c->st, &s, sizeof(s), hipMemcpyHostToDevice));
    stale_sums(c);
    return TTP_OK;
}

int ttp_scaler_update(ttp_ctx* c) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!c->scaler.enabled) return TTP_OK;  // nothing to update, as GradScaler when disabled
    if ((rc = set_dev(c))) return rc;
    clear_hip_error();
    hipLaunchKernelGGL(ttp::scaler_update_kernel, dim3(1), dim3(64), 0, c->stream, c->st,
                       (int32_t)c->scaler.growth_interval, c->scaler.growth_factor,
                       c->scaler.backoff_factor);
    HIP_TRY(hipGetLastError());
    stale_sums(c);  // the scale may have moved
    return TTP_OK;
}

}  // extern "C"

namespace {

constexpr char kStateMagic[8] = {'T', 'T', 'P', 'S', 'T', 'A', 'T', 'E'};
constexpr uint32_t kStateVersion = 1;
constexpr size_t kStageBytes = 64ull << 20;

#pragma pack(push, 1)
struct StateHeader {
    char magic[8];
    uint32_t version, mode, n_tensors, buffers;
    uint64_t total, t;
    float scale;
    int32_t growth_tracker, scaler_enabled, growth_interval;
    double init_scale, growth_factor, backoff_factor;
};
struct StateTensor {
    uint64_t numel;
    uint32_t flags, mom_init;
};
#pragma pack(pop)

// 64-bit word hash (FNV-1a style multiply over 8-byte words, then a final avalanche)
struct Hash {
    uint64_t h = 0xcbf29ce484222325ull;
    void add(const void* p, size_t n) {
        const uint8_t* b = (const uint8_t*)p;
        size_t k = 0;
        for (; k + 8 <= n; k += 8) {
            uint64_t w;
            std::memcpy(&w, b + k, 8);
            h = (h ^ w) * 0x100000001b3ull;
            h ^= h >> 29;
        }
        for (; k < n; ++k) h = (h ^ b[k]) * 0x100000001b3ull;
    }
    uint64_t value() const {
        uint64_t x = h;
        x ^= x >> 33;
        x *= 0xff51afd7ed558ccdull;
        x ^= x >> 33;
        return x;
    }
};

struct File {
    FILE* f = nullptr;
    ~File() {
        if (f) std::fclose(f);
    }
};

struct Pinned {
    void* p = nullptr;
    ~Pinned() {
        if (p) (void)hipHostFree(p);
    }
};

// buffer id of a state-file buffer bit
int state_buffer_id(int bit) {
    switch (bit) {
        case 1: return TTP_BUF_MASTER;
        case 2: return TTP_BUF_EXP_AVG;
        case 4: return TTP_BUF_EXP_AVG_SQ;
    }
    return TTP_BUF_MOMENTUM;
}

}  // namespace

extern "C" {

int ttp_save_state(ttp_ctx* c, const char* path) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!path) return fail(TTP_ERR_INVALID, "null path");
    if ((rc = no_capture(c, "ttp_save_state"))) return rc;
    if ((rc = set_dev(c))) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    DevState ds;
    HIP_TRY(hipMemcpy(&ds, c->st, sizeof(ds), hipMemcpyDeviceToHost));
    std::vector<uint32_t> mom(std::max<size_t>(c->tensors.size(), 1), 0);
    HIP_TRY(hipMemcpy(mom.data(), c->mom_init, mom.size() * 4, hipMemcpyDeviceToHost));

    StateHeader h{};
    std::memcpy(h.magic, kStateMagic, 8);
    h.version = kStateVersion;
    h.mode = (uint32_t)c->mode;
    h.n_tensors = (uint32_t)c->tensors.size();
    h.buffers = 1u | (c->exp_avg ? 2u : 0u) | (c->exp_avg_sq ? 4u : 0u) | (c->momentum ? 8u : 0u);
    h.total = c->total;
    h.t = t_on_device(c) ? ds.t : c->host_t;
    h.scale = ds.scale;
    h.growth_tracker = ds.growth_tracker;
    h.scaler_enabled = c->scaler.enabled;
    h.growth_interval = c->scaler.growth_interval;
    h.init_scale = c->scaler.init_scale;
    h.growth_factor = c->scaler.growth_factor;
    h.backoff_factor = c->scaler.backoff_factor;

    // written to `path`.tmp and renamed over `path` once complete, so a failed save leaves an
    // earlier file at `path` intact
    const std::string tmp = std::string(path) + ".tmp";
    File f;
    f.f = std::fopen(tmp.c_str(), "wb");
    if (!f.f) return fail(TTP_ERR_INVALID, "cannot open " + tmp + " for writing");
    bool done = false;
    struct Cleanup {
        const std::string& p;
        const bool& done;
        ~Cleanup() {
            if (!done) (void)std::remove(p.c_str());
        }
    } cleanup{tmp, done};
    Hash hash;
    auto put = [&](const void* p, size_t n) {
        hash.add(p, n);
        return std::fwrite(p, 1, n, f.f) == n;
    };
    bool ok = put(&h, sizeof(h));
    for (size_t i = 0; ok && i < c->tensors.size(); ++i) {
        StateTensor t{c->tensors[i].numel, c->tensors[i].flags, mom[i]};
        ok = put(&t, sizeof(t));
    }
    // each buffer as one contiguous fp32 array, whatever its device layout: gathered into
    // device staging piece by piece, then through a pinned buffer to the file
    Pinned stage;
    HIP_TRY(hipHostMalloc(&stage.p, kStageBytes));
    if ((rc = ensure_staging(c, kStageBytes))) return rc;
    const uint64_t piece = kStageBytes / 4;
    for (int bit = 1; ok && bit <= 8; bit <<= 1) {
        if (!(h.buffers & (uint32_t)bit)) continue;
        const int which = state_buffer_id(bit);
        for (uint64_t o = 0; ok && o < c->total; o += piece) {
            const uint64_t n = std::min(piece, c->total - o);
            if ((rc = gather_slot(c, which, o, n, (float*)c->staging))) return rc;
            HIP_TRY(hipMemcpyAsync(stage.p, c->staging, n * 4, hipMemcpyDeviceToHost, c->stream));
            HIP_TRY(hipStreamSynchronize(c->stream));
            ok = put(stage.p, n * 4);
        }
    }
    const uint64_t sum = hash.value();
    ok = ok && std::fwrite(&sum, 1, 8, f.f) == 8;
    ok = ok && std::fflush(f.f) == 0;
    const int closed = std::fclose(f.f);
    f.f = nullptr;
    if (!ok || closed != 0) return fail(TTP_ERR_INVALID, "write to " + tmp + " failed");
    if (std::rename(tmp.c_str(), path) != 0)
        return fail(TTP_ERR_INVALID, "cannot rename " + tmp + " to " + path);
    done = true;
    return TTP_OK;
}

int ttp_load_state(ttp_ctx* c, const char* path) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!path) return fail(TTP_ERR_INVALID, "null path");
    if ((rc = no_capture(c, "ttp_load_state"))) return rc;
    if ((rc = set_dev(c))) return rc;
    File f;
    f.f = std::fopen(path, "rb");
    if (!f.f) return fail(TTP_ERR_INVALID, std::string("cannot open ") + path);
    Hash hash;
    auto get = [&](void* p, size_t n) {
        if (std::fread(p, 1, n, f.f) != n) return false;
        hash.add(p, n);
        return true;
    };
    StateHeader h;
    if (!get(&h, sizeof(h)) || std::memcmp(h.magic, kStateMagic, 8) != 0)
        return fail(TTP_ERR_INVALID, std::string(path) + " is not an optimizer-state file");
    if (h.version != kStateVersion)
        return fail(TTP_ERR_INVALID, "unsupported state file version " + std::to_string(h.version));
    if (h.mode != (uint32_t)c->mode)
        return fail(TTP_ERR_INVALID, "state file precision mode differs from the context's");
    if (h.n_tensors != c->tensors.size())
        return fail(TTP_ERR_INVALID, "state file has " + std::to_string(h.n_tensors) +
                                         " tensors, the context " +
                                         std::to_string(c->tensors.size()));
    if (!(h.buffers & 1u) || (h.buffers & ~15u))
        return fail(TTP_ERR_INVALID, "state file buffer mask is malformed");
    // the ranges ttp_scaler_configure and ttp_scaler_set accept
    if (h.scaler_enabled &&
        (!(h.init_scale > 0) || !(h.growth_factor > 1) ||
         !(h.backoff_factor > 0 && h.backoff_factor < 1) || h.growth_interval <= 0))
        return fail(TTP_ERR_INVALID, "state file loss-scaler settings are out of range");
    if (!(h.scale > 0) || h.growth_tracker < 0)
        return fail(TTP_ERR_INVALID, "state file loss scale or growth tracker is out of range");
    std::vector<uint32_t> mom(std::max<size_t>(c->tensors.size(), 1), 0);
    for (size_t i = 0; i < c->tensors.size(); ++i) {
        StateTensor t;
        if (!get(&t, sizeof(t))) return fail(TTP_ERR_INVALID, "state file is truncated");
        if (t.numel != c->tensors[i].numel || t.flags != c->tensors[i].flags)
            return fail(TTP_ERR_INVALID, "state file tensor " + std::to_string(i) +
                                             " differs from the context's (numel or flags)");
        mom[i] = t.mom_init ? 1u : 0u;
    }
    if (h.total != c->total)  // the layout follows from the table; this catches a bad header
        return fail(TTP_ERR_INVALID, "state file flat size differs from the context's");
    ttp_scaler_config file_scaler{h.scaler_enabled, h.growth_interval, h.init_scale,
                                  h.growth_factor, h.backoff_factor};
    if (c->n_graphs && !same_scaler_settings(c->scaler, file_scaler))
        return fail(TTP_ERR_STATE, "the state file's loss-scaler settings differ from those in "
                                   "this context's captured graphs; destroy them first");
    // The whole file is checked before the context is touched: its size, then its checksum
    // over every byte, so a damaged file leaves the context as it was.
    const int64_t data_pos = ftello(f.f);
    uint64_t nbuf = 0;
    for (int bit = 1; bit <= 8; bit <<= 1) nbuf += (h.buffers & (uint32_t)bit) ? 1 : 0;
    const uint64_t data_bytes = nbuf * c->total * 4;
    if (data_pos < 0 || fseeko(f.f, 0, SEEK_END) != 0)
        return fail(TTP_ERR_INVALID, std::string("cannot seek in ") + path);
    const int64_t end = ftello(f.f);
    if (end < data_pos || (uint64_t)(end - data_pos) < data_bytes + 8)
        return fail(TTP_ERR_INVALID, "state file is truncated");
    if ((uint64_t)(end - data_pos) > data_bytes + 8)
        return fail(TTP_ERR_INVALID, "state file has trailing bytes");
    if (fseeko(f.f, data_pos, SEEK_SET) != 0)
        return fail(TTP_ERR_INVALID, std::string("cannot seek in ") + path);
    Pinned stage;
    HIP_TRY(hipHostMalloc(&stage.p, kStageBytes));
    for (uint64_t o = 0; o < data_bytes; o += kStageBytes) {
        const uint64_t n = std::min<uint64_t>(kStageBytes, data_bytes - o);
        if (!get(stage.p, n)) return fail(TTP_ERR_INVALID, "state file is truncated");
    }
    const uint64_t want = hash.value();
    uint64_t sum = 0;
    if (std::fread(&sum, 1, 8, f.f) != 8) return fail(TTP_ERR_INVALID, "state file is truncated");
    if (sum != want) return fail(TTP_ERR_INVALID, "state file checksum mismatch");
    if (fseeko(f.f, data_pos, SEEK_SET) != 0)
        return fail(TTP_ERR_INVALID, std::string("cannot seek in ") + path);

    // allocate what the file holds; zero what the context holds and the file does not
    if ((h.buffers & 6u) && (rc = ensure_adam_state(c))) return rc;
    if ((h.buffers & 8u) && (rc = ensure_momentum(c))) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    if ((rc = ensure_staging(c, kStageBytes))) return rc;
    const uint64_t piece = kStageBytes / 4;
    for (int bit = 1; bit <= 8; bit <<= 1) {
        const int which = state_buffer_id(bit);
        if (!(h.buffers & (uint32_t)bit)) {
            // zeros (scatter with no source) into a buffer the context holds
            if (buffer_base(c, which) && (rc = scatter_slot(c, which, 0, c->total, nullptr)))
                return rc;
            continue;
        }
        // the master scatter also rewrites the MIXED-mode bf16 copy as RNE(master)
        for (uint64_t o = 0; o < c->total; o += piece) {
            const uint64_t n = std::min(piece, c->total - o);
            // the file was read whole above; a failure here is an I/O error or a file that
            // changed since, and leaves the context partly loaded
            if (std::fread(stage.p, 1, n * 4, f.f) != n * 4)
                return fail(TTP_ERR_INVALID, std::string("read from ") + path +
                                                 " failed after its checksum was verified");
            HIP_TRY(hipMemcpyAsync(c->staging, stage.p, n * 4, hipMemcpyHostToDevice, c->stream));
            if ((rc = scatter_slot(c, which, o, n, (const float*)c->staging))) return rc;
            HIP_TRY(hipStreamSynchronize(c->stream));  // stage.p is refilled next
        }
    }
    HIP_TRY(hipMemcpyAsync(c->mom_init, mom.data(), mom.size() * 4, hipMemcpyHostToDevice,
                           c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    for (size_t i = 0; i < c->tensors.size(); ++i) c->host_mom_init[i] = (uint8_t)mom[i];
    c->scaler.enabled = h.scaler_enabled;
    c->scaler.growth_interval = h.growth_interval;
    c->scaler.init_scale = h.init_scale;
    c->scaler.growth_factor = h.growth_factor;
    c->scaler.backoff_factor = h.backoff_factor;
    c->host_t = h.t;
    DevState ds;
    HIP_TRY(hipMemcpy(&ds, c->st, sizeof(ds), hipMemcpyDeviceToHost));
    ds.t = h.t;
    ds.scale = h.scale;
    ds.growth_tracker = h.growth_tracker;
    ds.pending = 0;
    HIP_TRY(hipMemcpy(c->st, &ds, sizeof(ds), hipMemcpyHostToDevice));
    stale_sums(c);
    return TTP_OK;
}

int ttp_capture_begin(ttp_ctx* c) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((rc = no_capture(c, "ttp_capture_begin"))) return rc;
    if (!c->stream)
        return fail(TTP_ERR_STATE, "the legacy default stream cannot be captured; use the "
                                   "context's own stream or a created stream");
    if ((rc = set_dev(c))) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (!t_on_device(c)) {  // from now on the step count lives on the device
        HIP_TRY(hipMemcpy(&c->st->t, &c->host_t, sizeof(c->host_t), hipMemcpyHostToDevice));
    }
    c->device_t = true;
    HIP_TRY(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = true;
    c->cap_touched.assign(c->tensors.size(), 0);
    c->cap_needs.assign(c->tensors.size(), 0);
    c->cap_fresh0 = c->tsum_fresh;
    c->cap_grad0.resize(c->tensors.size());
    for (size_t i = 0; i < c->tensors.size(); ++i) c->cap_grad0[i] = (uint8_t)c->tensors[i].has_grad;
    return TTP_OK;
}

int ttp_capture_end(ttp_ctx* c, ttp_graph** out) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (out) *out = nullptr;
    if (!c->capturing) return fail(TTP_ERR_STATE, "not capturing");
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(c->stream, &g);
    c->capturing = false;
    // nothing captured has run: the per-tensor flags return to their state at
    // ttp_capture_begin, and each launch applies the captured calls' effect on them
    std::vector<ttp_graph::FlagEffect> effects;
    std::vector<uint32_t> needs;
    for (uint32_t i = 0; i < (uint32_t)c->cap_touched.size(); ++i) {
        if (c->cap_touched[i])
            effects.push_back({i, c->cap_touched[i], c->tsum_fresh[i],
                               (uint8_t)c->tensors[i].has_grad});
        if (c->cap_needs[i]) needs.push_back(i);
        c->tsum_fresh[i] = c->cap_fresh0[i];
        c->tensors[i].has_grad = c->cap_grad0[i];
    }
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return fail(TTP_ERR_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
    }
    if (!out) {  // discard
        if (g) (void)hipGraphDestroy(g);
        return TTP_OK;
    }
    hipGraphExec_t ex = nullptr;
    const hipError_t e2 = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e2 != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(TTP_ERR_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e2));
    }
    *out = new ttp_graph{c, g, ex, std::move(effects), std::move(needs)};
    c->n_graphs += 1;
    return TTP_OK;
}

int ttp_graph_launch(ttp_graph* g) {
    if (!g) return fail(TTP_ERR_INVALID, "null graph");
    int rc;
    ttp_ctx* c = g->ctx;
    if ((rc = no_capture(c, "ttp_graph_launch"))) return rc;
    for (uint32_t i : g->needs_fresh)
        if (!c->tsum_fresh[i])
            return fail(TTP_ERR_STATE, "the graph steps with per-tensor sums taken before it, and "
                                       "tensor " + std::to_string(i) + " has no current gradient "
                                       "sum: call ttp_grad_sumsq_tensors before launching it");
    if ((rc = set_dev(c))) return rc;
    HIP_TRY(hipGraphLaunch(g->exec, c->stream));
    // as the captured calls do eagerly: a step consumes the sums, a sums call renews them,
    // gradient writes and zero_grad set or clear the has-grad flags
    for (const auto& f : g->effects) {
        if (f.mask & kCapFresh) c->tsum_fresh[f.tensor] = f.fresh;
        if (f.mask & kCapGrad) c->tensors[f.tensor].has_grad = f.has_grad;
    }
    return TTP_OK;
}

int ttp_graph_destroy(ttp_graph* g) {
    if (!g) return TTP_OK;
    (void)hipSetDevice(g->ctx->device);
    if (g->ctx->stream) (void)hipStreamSynchronize(g->ctx->stream);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    g->ctx->n_graphs -= 1;
    delete g;
    return TTP_OK;
}

int ttp_timing_enable(ttp_ctx* c, int on) {
    int rc = check_ctx(c);
    if (rc) return rc;
    c->timing = on != 0;
    return TTP_OK;
}

int ttp_timing_collect(ttp_ctx* c, int kernel, double* total_ms, uint64_t* launches) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (kernel != TTP_KERNEL_NORM && kernel != TTP_KERNEL_UPDATE)
        return fail(TTP_ERR_INVALID, "unknown kernel id");
    if ((rc = set_dev(c))) return rc;
    double sum = 0.0;
    uint64_t cnt = 0;
    auto& v = c->ev[kernel];
    // every pair goes back to the pool, also after a failure, so no event is listed twice
    hipError_t e = hipSuccess;
    for (auto& p : v) {
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventSynchronize(p.b);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, p.a, p.b);
        if (e == hipSuccess) {
            sum += ms;
            ++cnt;
        }
        c->ev_pool.push_back(p.a);
        c->ev_pool.push_back(p.b);
    }
    v.clear();
    HIP_TRY(e);
    if (total_ms) *total_ms = sum;
    if (launches) *launches = cnt;
    return TTP_OK;
}

}  // extern "C"
