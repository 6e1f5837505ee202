// kernels.hpp — gfx950 device code of libttperf_hip.
//
// One optimizer step over the flat store is at most four launches on one stream:
//   norm_partials_kernel  reads only the gradients (2 B/param bf16, 4 B/param fp32) in 16 KiB
//                         tiles: fp64 sum of squares of the unscaled grads, one partial per
//                         block; no atomics and no fences (a per-block device-scope fence +
//                         ticket costs ~50 ns per block on MI355X, serialised, which tripled
//                         the pass's time).  Two launches above 256 MiB of gradients:
//                         non-temporal loads, then cached loads for the last 256 MiB;
//   norm_finalize_kernel  one block: sums the partials in index order (deterministic),
//                         decides found_inf / skip and the clip coefficient, advances the step
//                         count and the loss scale;
//   adam_lane_kernel /    one fused pass per element: grad transform (unscale, clip), weight
//   sgd_lane_kernel       decay, the optimizer update and the bf16 copy, one or two elements
//                         per lane; sgd_kernel does the same with four elements per lane
//                         (16-byte fp32 and 8-byte bf16 vectors) for MIXED SGD momentum
//                         updates whose gradients fit the Infinity Cache.  Each element is touched once.
// Optimizer state is stored in records (see kRec): in MIXED mode each 64-element group of the
// flat store keeps its fp32 master, m and v side by side in one 768-byte record; in FP32 mode
// (where the fp32 master is the model-facing weight and stays contiguous) m and v share
// 512-byte records.  The update then streams grad, state records and the bf16 copy instead of
// nine separate arrays: the state read and write of a group hit the same DRAM pages, and the
// step no longer depends on where the allocator happened to place five large buffers
// relative to each other (GPT-2 124M, fresh allocations, 6 rounds: 571-617 us per step with
// separate buffers, 570-580 us with records).
// Work is a table of chunks of kChunk elements (the last chunk of a tensor is shorter; every
// chunk starts on a 64-element boundary).  Update blocks are dispatched in (reverse) chunk
// order, so the resident blocks sweep a narrow window of each buffer, which keeps DRAM pages
// open.  The four-element update (MIXED SGD momentum, cached gradients) runs one 256-thread block
// per chunk, one vector per lane, at most kUpdBlocksPerCU blocks per CU; for it 16K-element
// chunks, a persistent grid, two or four vectors per lane, 512-thread blocks and unlimited
// occupancy each measured 3-12% slower (as a four-element Adam update, which the lane forms
// have replaced).  No MFMA: nothing here is a contraction.
//
// Arithmetic matches the oracle bit for bit: no contraction (-ffp-contract=off), IEEE
// division and square root (HIP's correctly rounded fp32 div/sqrt), denormals kept.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ttp {

constexpr int kBlock = 256;     // 4 wave64s: norm pass, finalize and helper kernels
constexpr int kUpdBlock = 256;  // 4 wave64s: the four-element update
constexpr int kVec = 4;         // elements per lane per vector
constexpr uint32_t kChunk = kUpdBlock * kVec;  // 1024 elements: one vector per lane
// Resident blocks per CU of the four-element update.  The host reserves LDS_per_CU /
// kUpdBlocksPerCU bytes of (unused) dynamic LDS per block so that no more than this many are
// resident: 16 waves per CU sweep the HBM pages of the streams with fewer row conflicts than
// the 32+ waves that registers alone would allow (measured on the four-element Adam update
// that the lane forms have replaced: separate state arrays, GPT-2 124M, same box,
// interleaved repeats: 568 us vs 588 us for 512-thread blocks at 3 per CU, 622 us uncapped;
// GPT-2 XL fp32: 7.36 ms vs 7.63 ms).  With state records, 4, 5, 6 and 8 blocks per CU
// measure alike and 3 is 27% slower.
constexpr int kUpdBlocksPerCU = 4;
constexpr uint32_t kChunkDecay = 1u;

// State records.  Element i of a record-stored buffer sits at
//   slot_base + (i / kRec) * stride + i % kRec
// where slot_base is the record array's base plus slot * kRec.  Tensors start on kRec
// boundaries, so a tensor's state is whole records and a lane's 4-element vector never
// straddles two.  A contiguous buffer is the case stride == kRec.
constexpr uint32_t kRec = 64;
constexpr uint32_t kStrideMixed = 3 * kRec;  // MIXED: [master | m | v]
constexpr uint32_t kStrideMV = 2 * kRec;     // FP32:  [m | v]

__host__ __device__ __forceinline__ uint64_t rec_index(uint64_t i, uint32_t stride) {
    return (i / kRec) * stride + (i % kRec);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct Chunk {
    uint64_t begin;  // first element (flat index)
    uint32_t count;  // elements in this chunk (exact, not padded)
    uint32_t meta;   // bit 0: decay; bits 8..31: tensor index
};

// chunk k of a table as one 16-byte load (a field-wise read compiles to two dependent loads:
// the count first, then begin and meta)
__device__ __forceinline__ Chunk load_chunk(const Chunk* t, uint64_t k) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(t + k);
    return Chunk{(uint64_t)w.x | ((uint64_t)w.y << 32), w.z, w.w};
}

// Device-resident step state.  Written only by norm_finalize_kernel (and by the host between
// steps); read by the update pass that follows it on the same stream.
struct DevState {
    float scale;             // loss scale (persistent)
    int32_t growth_tracker;  // clean steps since the last scale change (persistent)
    uint64_t t;              // applied steps while loss scaling is on (persistent)
    double sumsq;            // last pass: sum of squares of the unscaled grads
    double norm;             // last pass: sqrt(sumsq)
    float inv_scale;         // last pass: 1/scale used to unscale
    float clip_coef;         // last pass: clip multiplier (1 when not clipping)
    float bias1, bias2;      // last pass: Adam bias corrections for the new t
    int32_t found_inf;       // last pass: a non-finite gradient was seen
    int32_t skip;            // last pass: the update must not run
    // steps that deferred the scale update since the last one (several optimizers over one
    // store: torch's GradScaler.step per optimizer, then one update): kPendingStep once such a
    // step ran, | kPendingInf if one of them saw an overflow.  The next scale update combines
    // it with its own and clears it (persistent).
    int32_t pending;
    int32_t reserved;
};
static_assert(sizeof(DevState) == 64, "DevState is one 64-byte block");
constexpr int32_t kPendingInf = 1, kPendingStep = 2;

// ------------------------------------------------------------------------------------
// bf16
// ------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// round-to-nearest-even; NaN -> canonical 0x7FC0
__device__ __forceinline__ uint32_t bf16_rne(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    return ((u & 0x7FFFFFFFu) > 0x7F800000u) ? 0x7FC0u : r;
}

__device__ __forceinline__ uint32_t bf16_pack(float a, float b) {
    return bf16_rne(a) | (bf16_rne(b) << 16);
}

// ------------------------------------------------------------------------------------
// vector memory helpers (all addresses 16-byte / 8-byte aligned by construction)
// ------------------------------------------------------------------------------------
__device__ __forceinline__ f32x4 ld4(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
}
__device__ __forceinline__ void st4(float* p, f32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
}

// 4 gradients as fp32 from either storage type, with ordinary (temporal) loads: the
// four-element update runs only on gradients that fit the 256 MB Infinity Cache, where the
// norm pass or the backward left them
__device__ __forceinline__ f32x4 ld_grad4(const float* g, uint64_t i) {
    return *reinterpret_cast<const f32x4*>(g + i);
}
__device__ __forceinline__ f32x4 ld_grad4(const uint16_t* g, uint64_t i) {
    const u32x2 w = *reinterpret_cast<const u32x2*>(g + i);
    f32x4 r;
    r.x = bf16_lo(w.x);
    r.y = bf16_hi(w.x);
    r.z = bf16_lo(w.y);
    r.w = bf16_hi(w.y);
    return r;
}

__device__ __forceinline__ void st_bf16x4(uint16_t* p, uint64_t i, f32x4 v) {
    u32x2 w;
    w.x = bf16_pack(v.x, v.y);
    w.y = bf16_pack(v.z, v.w);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(p + i));
}

// partial vector (the last one of a tensor): element-wise stores of the first n lanes
__device__ __forceinline__ void st4_partial(float* p, f32x4 v, int n) {
    p[0] = v.x;
    if (n > 1) p[1] = v.y;
    if (n > 2) p[2] = v.z;
}
__device__ __forceinline__ void st_bf16x4_partial(uint16_t* p, f32x4 v, int n) {
    p[0] = (uint16_t)bf16_rne(v.x);
    if (n > 1) p[1] = (uint16_t)bf16_rne(v.y);
    if (n > 2) p[2] = (uint16_t)bf16_rne(v.z);
}

// ------------------------------------------------------------------------------------
// block reduction of a double (fixed shape: deterministic)
// ------------------------------------------------------------------------------------
__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

__device__ __forceinline__ double block_sum(double x, double* lds) {
    x = wave_sum(x);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) lds[wave] = x;
    __syncthreads();
    double r = 0.0;
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 0; w < kBlock / 64; ++w) r += lds[w];
    }
    __syncthreads();
    return r;  // valid in thread 0
}

// ------------------------------------------------------------------------------------
// norm pass, part 1: per-block partial sums of squares of the unscaled gradients
// ------------------------------------------------------------------------------------
// 16-byte loads: 8 bf16 or 4 fp32 gradients per lane
template <typename GradT>
struct GradVec;
template <>
struct GradVec<uint16_t> {
    static constexpr int kElems = 8;
    typedef uint32_t raw __attribute__((ext_vector_type(4)));
    static __device__ __forceinline__ float at(const raw& w, int j) {
        return (j & 1) ? bf16_hi(w[j >> 1]) : bf16_lo(w[j >> 1]);
    }
    // element j of a vector that starts as zeros
    static __device__ __forceinline__ void put(raw& w, int j, uint16_t h) {
        w[j >> 1] |= (j & 1) ? ((uint32_t)h << 16) : (uint32_t)h;
    }
};
template <>
struct GradVec<float> {
    static constexpr int kElems = 4;
    typedef f32x4 raw;
    static __device__ __forceinline__ float at(const raw& w, int j) { return w[j]; }
    static __device__ __forceinline__ void put(raw& w, int j, float x) { w[j] = x; }
};

// Norm tiles: kNormLoads 16-byte loads per lane, so a tile is 16 KiB of gradients (8192 bf16
// or 4096 fp32); the pass has its own tile table (same tensors, bigger pieces than the update's
// chunks) so each descriptor fetch is amortised over 4 loads per lane.
constexpr int kNormLoads = 4;
template <typename GradT>
constexpr uint32_t norm_tile_elems() {
    return (uint32_t)(kBlock * kNormLoads * 16 / sizeof(GradT));
}

// Grid-stride over the norm tiles t0 .. t1-1, one partial per block.  A whole tile (every tile
// but a tensor's last) is four unconditional 16-byte loads per lane, all issued before the
// arithmetic (the scheduling barrier keeps the compiler from interleaving them with it, which
// left one or two loads in flight: 6.0-6.3 TB/s against 6.7-6.9 at GPT-2 774M / 1558M).
// kNT selects non-temporal loads.  The host runs the pass as two launches: non-temporal over
// all but the last kCachedGradBytes of gradients, then cached loads over those, which the
// update, walking the chunks in reverse, reads first and so finds in the 256 MB Infinity
// Cache (measured on GPT-2 124M: update 531 us after this pass vs 559 us alone; at 774M and
// 1558M fp32 the split pass runs 232 and 931 us against 246-260 and 978-1030 us with cached
// loads throughout, the update unchanged).  No atomics and no fences: each block writes one
// partial and norm_finalize_kernel (next on the stream) combines them.  Squares of fp32
// values are exact in fp64, and any inf/NaN gradient makes the sum non-finite.
template <typename GradT, bool kNT>
__global__ __launch_bounds__(kBlock) void norm_partials_kernel(const GradT* __restrict__ g,
                                                               const Chunk* __restrict__ tiles,
                                                               uint32_t t0, uint32_t t1,
                                                               const DevState* __restrict__ st,
                                                               int32_t scaler_on,
                                                               double* __restrict__ partials) {
    typedef GradVec<GradT> GV;
    typedef typename GV::raw R;
    constexpr int E = GV::kElems;
    constexpr uint32_t kTile = norm_tile_elems<GradT>();
    __shared__ double lds[kBlock / 64];
    const float inv = scaler_on ? (float)(1.0 / (double)st->scale) : 1.0f;
    // two accumulators (element j of a vector goes to acc[j & 1]): a fixed order, so the
    // sum stays deterministic, with half the dependent-add chain.  The square of an fp32 value
    // is exact in fp64, so fma(x, x, acc) rounds exactly as acc + x*x does (one rounding, of
    // the add) with one instruction instead of two.
    double acc[2] = {0.0, 0.0};
    for (uint32_t c = t0 + blockIdx.x; c < t1; c += gridDim.x) {
        const Chunk ch = load_chunk(tiles, c);
        const R* q = reinterpret_cast<const R*>(g + ch.begin) + threadIdx.x;
        if (ch.count == kTile) {
            R w[kNormLoads];
#pragma unroll
            for (int l = 0; l < kNormLoads; ++l)
                w[l] = kNT ? __builtin_nontemporal_load(q + l * kBlock) : q[l * kBlock];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int l = 0; l < kNormLoads; ++l) {
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    const double x = (double)(GV::at(w[l], j) * inv);
                    acc[j & 1] = __builtin_fma(x, x, acc[j & 1]);
                }
            }
        } else {  // a tensor's last tile: only the vectors (and elements) below its count
#pragma unroll
            for (int l = 0; l < kNormLoads; ++l) {
                const uint32_t off = (uint32_t)(l * kBlock + threadIdx.x) * E;
                const uint32_t nv = off < ch.count ? min(ch.count - off, (uint32_t)E) : 0u;
                if (nv) {
                    const R w = q[l * kBlock];
#pragma unroll
                    for (int j = 0; j < E; ++j) {
                        const double x = (uint32_t)j < nv ? (double)(GV::at(w, j) * inv) : 0.0;
                        acc[j & 1] = __builtin_fma(x, x, acc[j & 1]);
                    }
                }
            }
        }
    }
    const double b = block_sum(acc[0] + acc[1], lds);
    if (threadIdx.x == 0) partials[blockIdx.x] = b;
}

// ------------------------------------------------------------------------------------
// norm pass, part 2 (one block): combine the partials in index order (deterministic), then
// decide found_inf / skip, the clip coefficient, the step count and the loss scale
// ------------------------------------------------------------------------------------
struct FinalizeArgs {
    const double* partials;
    const uint32_t* idx;    // non-null: partial k is partials[idx[k]] (per-tensor sums)
    uint32_t npartials;     // 0: no norm pass ran (step counting only)
    int32_t scaler_on;      // unscale by 1/scale, skip on inf, update the scale
    int32_t defer_scale;    // with scaler_on: note the step and its overflow in `pending`;
                            // leave the scale as it is
    int32_t count_t;        // the step count lives on the device: advance it (unless skipped)
    int32_t probe;          // only compute sumsq/norm (ttp_grad_norm); touch nothing else
    int32_t growth_interval;
    double growth_factor;
    double backoff_factor;
    double max_norm;        // > 0: clip
    const float* bias_tab;  // [2*bias_len]: (1-beta1^t, 1-beta2^t) for t = 1..bias_len
    uint32_t bias_len;      // t > bias_len: both corrections are exactly 1.0f
    int32_t want_bias;
    DevState* st;
};

// torch _amp_update_scale_ semantics, over this step's overflow and the pending overflow of
// the steps that deferred their update since the last one (found_inf summed over optimizers,
// as GradScaler.update does): the new scale and growth tracker (the pending flag is cleared)
struct ScaleUpdate {
    float scale;
    int32_t tracker;
};
__device__ __forceinline__ ScaleUpdate next_scale(float scale, int32_t tracker, int32_t pending,
                                                  int32_t found, int32_t growth_interval,
                                                  double growth_factor, double backoff_factor) {
    if (found || (pending & kPendingInf)) return {(float)((double)scale * backoff_factor), 0};
    const int32_t ok = tracker + 1;
    if (ok == growth_interval) {
        const float ns = (float)((double)scale * growth_factor);
        return {ns - ns == 0.0f ? ns : scale, 0};  // grows only to a finite scale
    }
    return {scale, ok};
}

// (float)(1 - beta^t) for t = 1 .. bias_len from the host-built table; 1.0f beyond (and for
// t = 0, which no applied step has)
__device__ __forceinline__ float bias_entry(const float* tab, uint32_t len, uint64_t t, int j) {
    return (t >= 1 && t <= len) ? tab[2 * (t - 1) + j] : 1.0f;
}

__global__ __launch_bounds__(kBlock) void norm_finalize_kernel(FinalizeArgs a) {
    __shared__ double lds[kBlock / 64];
    DevState* st = a.st;
    // Every load is issued before thread 0 decides: the first round of partials, then the
    // whole step state (one 64-byte block, uniform, so scalar loads) and the bias corrections
    // of both outcomes (t + 1 if the step applies, t if it is skipped), whose latency overlaps
    // the partials' and their sum.  Read one after another, as the decisions need them, they
    // were six dependent round trips on thread 0 after the sum.
    // Partials: all loads of a round issued before the adds, each thread's order fixed
    // (deterministic); with an index list (per-tensor sums), a round's indices load first.
    // Loads past the end read the last entry and count as 0 in the adds (a branch or a select
    // at each load made the compiler wait for it there).
    constexpr int kPer = 8;
    const uint32_t n = a.npartials;
    double v[kPer];
    auto load_round = [&](uint32_t base) {  // base < n
        uint32_t at[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) at[k] = min(base + (uint32_t)k * kBlock + threadIdx.x, n - 1);
        if (a.idx) {
#pragma unroll
            for (int k = 0; k < kPer; ++k) at[k] = a.idx[at[k]];
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) v[k] = a.partials[at[k]];
    };
    if (n) {
        load_round(0);
    } else {
#pragma unroll
        for (int k = 0; k < kPer; ++k) v[k] = 0.0;
    }
    const DevState s0 = *st;
    float b1n = 1.0f, b2n = 1.0f, b1s = 1.0f, b2s = 1.0f;
    if (a.count_t && a.want_bias) {
        b1n = bias_entry(a.bias_tab, a.bias_len, s0.t + 1, 0);
        b2n = bias_entry(a.bias_tab, a.bias_len, s0.t + 1, 1);
        b1s = bias_entry(a.bias_tab, a.bias_len, s0.t, 0);
        b2s = bias_entry(a.bias_tab, a.bias_len, s0.t, 1);
    }
    // keeps the compiler from moving the first round's adds (which wait for the partials)
    // ahead of the state loads
    __builtin_amdgcn_sched_barrier(0);
    double s = 0.0;
    for (uint32_t base = 0;;) {
#pragma unroll
        for (int k = 0; k < kPer; ++k)
            s += base + (uint32_t)k * kBlock + threadIdx.x < n ? v[k] : 0.0;
        base += kBlock * kPer;
        if (base >= n) break;
        load_round(base);
    }
    s = block_sum(s, lds);
    if (threadIdx.x != 0) return;

    const float inv = a.scaler_on ? (float)(1.0 / (double)s0.scale) : 1.0f;
    const double norm = sqrt(s);
    st->sumsq = s;
    st->norm = norm;
    if (a.probe) return;
    const int found = !(s <= 1.7976931348623157e308);  // inf or NaN
    const int skip = a.scaler_on && found;
    float coef = 1.0f;
    if (a.max_norm > 0.0) {
        double cd = a.max_norm / (norm + 1e-6);
        if (cd > 1.0) cd = 1.0;
        coef = (float)cd;
    }
    st->found_inf = found;
    st->skip = skip;
    st->inv_scale = inv;
    st->clip_coef = coef;
    if (a.count_t) {
        st->t = skip ? s0.t : s0.t + 1;
        if (a.want_bias) {
            st->bias1 = skip ? b1s : b1n;
            st->bias2 = skip ? b2s : b2n;
        }
    }
    if (a.scaler_on) {
        if (a.defer_scale) {
            st->pending = s0.pending | kPendingStep | (found ? kPendingInf : 0);
        } else {
            const ScaleUpdate u = next_scale(s0.scale, s0.growth_tracker, s0.pending, found,
                                             a.growth_interval, a.growth_factor,
                                             a.backoff_factor);
            st->scale = u.scale;
            st->growth_tracker = u.tracker;
            st->pending = 0;
        }
    }
}

// ttp_scaler_update: the scale update of an iteration whose steps all deferred it; nothing
// when no step deferred it since the last update, so an iteration's scale never moves twice
__global__ void scaler_update_kernel(DevState* st, int32_t growth_interval, double growth_factor,
                                     double backoff_factor) {
    if (threadIdx.x == 0 && blockIdx.x == 0 && (st->pending & kPendingStep)) {
        const ScaleUpdate u = next_scale(st->scale, st->growth_tracker, st->pending, 0,
                                         growth_interval, growth_factor, backoff_factor);
        st->scale = u.scale;
        st->growth_tracker = u.tracker;
        st->pending = 0;
    }
}

// Per-tensor sums of squares (ttp_grad_sumsq_tensors), from one norm_partials_kernel block per
// tile: block t adds the tile sums of the t-th listed tensor, tiles tile_start[t] ..
// tile_start[t+1]-1, each lane in tile order, then the fixed block reduction, into
// sums[tensor_ids[t]].
// the sum of tile_sums[b .. e-1] in a fixed order (valid in thread 0): lane l adds tiles
// b + l, b + l + kBlock, b + l + 2 kBlock, ... in that order, a round of kSumRound of them
// loaded before their adds (as norm_finalize_kernel), then the fixed block reduction.  One
// order for every caller, so a tensor's sum does not depend on which call computed its tiles.
// The round size sets only how many loads are in flight, not the order (tiles past the end
// add +0.0 to a sum of squares, which leaves it as it is).  A round's loads are unconditional
// (an index past the end reads tile e-1, whose value the add then replaces by +0.0), so all of
// them are in flight at once: with a bounds check at each load, the compiler waited for each
// one before the next (GPT-2 124M's largest tensor, 4,712 tiles of four wave partials,
// combined in 8.6 us).
constexpr int kSumRound = 16;
__device__ __forceinline__ double sum_tiles(const double* __restrict__ tile_sums, uint32_t b,
                                            uint32_t e, double* lds) {
    constexpr int kPer = kSumRound;
    double s = 0.0;
    for (uint32_t base = b; base < e; base += kBlock * kPer) {
        double v[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k)
            v[k] = tile_sums[min(base + (uint32_t)k * kBlock + threadIdx.x, e - 1)];
#pragma unroll
        for (int k = 0; k < kPer; ++k) s += base + (uint32_t)k * kBlock + threadIdx.x < e ? v[k] : 0.0;
    }
    return block_sum(s, lds);
}

// A tensor's sum supersedes tile sums an earlier accumulate with sums left pending for it.
__global__ __launch_bounds__(kBlock) void tensor_sums_kernel(const double* __restrict__ tile_sums,
                                                             const uint32_t* __restrict__ tile_start,
                                                             const uint32_t* __restrict__ tensor_ids,
                                                             double* __restrict__ sums,
                                                             uint32_t* __restrict__ pending) {
    __shared__ double lds[kBlock / 64];
    const uint32_t t = blockIdx.x;
    const double s = sum_tiles(tile_sums, tile_start[t], tile_start[t + 1], lds);
    if (threadIdx.x == 0) {
        sums[tensor_ids[t]] = s;
        pending[tensor_ids[t]] = 0u;
    }
}

// The wave partials an accumulate with sums leaves per 16 KiB tile (kWaves of them, in wave
// order; see accumulate_grad_tiles_kernel): tile k's sum is their total added as block_sum
// adds its waves' sums, (((0 + w0) + w1) + w2) + w3, so it equals the norm pass's partial of
// that tile bit for bit.
constexpr int kWaves = kBlock / 64;
__device__ __forceinline__ double tile_from_waves(const double* __restrict__ w, uint32_t k) {
    double r = 0.0;
#pragma unroll
    for (int j = 0; j < kWaves; ++j) r += w[(uint64_t)k * kWaves + j];
    return r;
}

// Before a step that takes its norm from per-tensor sums: block t combines the t-th stepped
// tensor's tile sums that accumulates with their sums left in the store-wide array (the wave
// partials of its tiles, from kWaves x tile_base[tensor]), if it has any pending: each tile
// from its waves, then the tiles in sum_tiles' order, so the tensor's sum equals what
// ttp_grad_sumsq_tensors gives for the same gradients.  One launch per step instead of one
// per accumulate.
__global__ __launch_bounds__(kBlock) void combine_pending_sums_kernel(
    const double* __restrict__ acc_waves, const uint32_t* __restrict__ tile_base,
    const uint32_t* __restrict__ tile_start, const uint32_t* __restrict__ tensor_ids,
    uint32_t* __restrict__ pending, double* __restrict__ sums) {
    __shared__ double lds[kBlock / 64];
    const uint32_t t = blockIdx.x, i = tensor_ids[t];
    if (!pending[i]) return;  // uniform over the block
    const double* w = acc_waves + (uint64_t)tile_base[i] * kWaves;
    const uint32_t e = tile_start[t + 1] - tile_start[t];
    // sum_tiles' order, rounds and unconditional loads, over tile values formed from the wave
    // partials
    constexpr int kPer = kSumRound;
    double s = 0.0;
    for (uint32_t base = 0; base < e; base += kBlock * kPer) {
        double v[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k)
            v[k] = tile_from_waves(w, min(base + (uint32_t)k * kBlock + threadIdx.x, e - 1));
#pragma unroll
        for (int k = 0; k < kPer; ++k) s += base + (uint32_t)k * kBlock + threadIdx.x < e ? v[k] : 0.0;
    }
    s = block_sum(s, lds);
    if (threadIdx.x == 0) {
        sums[i] = s;
        pending[i] = 0u;
    }
}

// ------------------------------------------------------------------------------------
// fused Adam / AdamW update
// ------------------------------------------------------------------------------------
constexpr uint32_t kUseInv = 1u;    // multiply grads by st->inv_scale
constexpr uint32_t kUseClip = 2u;   // multiply grads by st->clip_coef
constexpr uint32_t kDevBias = 4u;   // take bias1/bias2 from st (step count on device)
constexpr uint32_t kCheckSkip = 8u; // return if st->skip
constexpr uint32_t kDecoupled = 16u;
constexpr uint32_t kWdOn = 32u;

struct AdamArgs {
    const Chunk* chunks;
    uint32_t nchunks;
    uint32_t flags;
    float lr, b1, omb1, b2, omb2, eps, bias1, bias2, decay_mul, wd;
    const DevState* st;
};

struct Coefs {
    float inv, clip, bias1, bias2;
};

// One element in the op order of py/optim.py:76-86 after the grad transforms and decay.
__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v,
                                          const AdamArgs& a, const Coefs& k, bool use_inv,
                                          bool use_clip, bool decay) {
    if (use_inv) g = g * k.inv;
    if (use_clip) g = g * k.clip;
    if (decay) {
        if (a.flags & kDecoupled) p = p * a.decay_mul;
        else g = g + a.wd * p;
    }
    m = a.b1 * m + a.omb1 * g;
    const float gsq = g * g;
    v = a.b2 * v + a.omb2 * gsq;
    const float m_hat = m / k.bias1;
    const float v_hat = v / k.bias2;
    const float denom = __builtin_sqrtf(v_hat) + a.eps;
    const float step = a.lr * (m_hat / denom);
    p = p - step;
}

// Stores of one vector: whole (16 B / 8 B) or the first n elements (a tensor's last vector).
// a, b, c point at the vector's first element in their buffers; the bf16 copy of va goes to
// p16[i].
template <bool kMixed>
__device__ __forceinline__ void store_vec(float* a, float* b, float* c, uint16_t* p16, uint64_t i,
                                          const f32x4& va, const f32x4& vb, const f32x4& vc,
                                          int n) {
    if (n >= kVec) {
        st4(a, va);
        if (b) st4(b, vb);
        if (c) st4(c, vc);
        if (kMixed) st_bf16x4(p16, i, va);
    } else {
        st4_partial(a, va, n);
        if (b) st4_partial(b, vb, n);
        if (c) st4_partial(c, vc, n);
        if (kMixed) st_bf16x4_partial(p16 + i, va, n);
    }
}

// ------------------------------------------------------------------------------------
// lane forms: one or two elements per lane, for stores whose gradients exceed the Infinity
// Cache
// ------------------------------------------------------------------------------------
// Each block of kLanes lanes takes 1/lane_parts<kE, kLanes, kIt>() of a chunk (the last chunks
// first): kIt consecutive pieces of kLanes x kE elements, each lane kE consecutive elements of
// each piece, with no occupancy cap.  A lane holds 14-32 B of loads in flight instead of the
// four-element form's 56-64 B (one 4-element vector per stream), and full occupancy
// (registers allow 32 waves per CU) hides the
// arithmetic.  The state is addressed from the record base alone (one 64-bit address per
// lane, the other slots at immediate offsets), and the chunk descriptor is one 16-byte scalar
// load issued together with the device-state loads, so two dependent scalar round trips
// (arguments, then descriptor and state) precede the data loads.  The host picks the shape
// per optimizer and mode (see kLaneAdamMixed in ttperf.hip).  Measured (interleaved rounds,
// x a plain 256-lane non-temporal copy of the same bytes): GPT-2 774M mixed AdamW, one element
// per lane, 256 lanes, two pieces: 1.014-1.018 against 0.96-0.98 with one piece and
// 0.91-0.93 for a four-element Adam form; GPT-2 1558M fp32 AdamW, one element, 128 lanes, two
// pieces: 1.018-1.027 against 0.977 for two elements in one piece and 0.905-0.927.  Below
// the Infinity Cache bound, GPT-2 124M mixed AdamW with 128-lane blocks of two pieces runs its
// update in 0.512-0.514 ms against 0.522 ms for the four-element Adam form, and 5% faster when
// a backward has just rewritten the gradients; FP32 AdamW and SGD momentum at 57.5M params run
// their steps 2-3% faster than in four-element forms.  A four-element form dispatched half the
// grid for a skipped step's early exit.
template <int kE, int kLanes, int kIt>
constexpr uint32_t lane_parts() {
    return kChunk / (kLanes * kE * kIt);
}

// kE (1, 2 or 4) gradients as fp32 (ordinary loads: faster here than non-temporal ones at
// 774M).  A lane's kE elements start at a multiple of kE and tensors start on 64-element
// boundaries, so a lane whose tensor ends inside it still reads inside the tensor's footprint.
template <int kE>
__device__ __forceinline__ void ld_grad_lane(const uint16_t* g, uint64_t i, float* out) {
    static_assert(kE == 1 || kE == 2 || kE == 4, "1, 2 or 4 elements per lane");
    if constexpr (kE == 1) {
        out[0] = __uint_as_float((uint32_t)g[i] << 16);
    } else if constexpr (kE == 2) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(g + i);
        out[0] = bf16_lo(w);
        out[1] = bf16_hi(w);
    } else {
        const u32x2 w = *reinterpret_cast<const u32x2*>(g + i);
        out[0] = bf16_lo(w.x);
        out[1] = bf16_hi(w.x);
        out[2] = bf16_lo(w.y);
        out[3] = bf16_hi(w.y);
    }
}
template <int kE>
__device__ __forceinline__ void ld_grad_lane(const float* g, uint64_t i, float* out) {
    static_assert(kE == 1 || kE == 2 || kE == 4, "1, 2 or 4 elements per lane");
    if constexpr (kE == 1) {
        out[0] = g[i];
    } else if constexpr (kE == 2) {
        const f32x2 w = *reinterpret_cast<const f32x2*>(g + i);
        out[0] = w.x;
        out[1] = w.y;
    } else {
        const f32x4 w = *reinterpret_cast<const f32x4*>(g + i);
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = w[j];
    }
}
// kE fp32 values, non-temporal
template <int kE>
__device__ __forceinline__ void ld_lane(const float* p, float* out) {
    if constexpr (kE == 1) {
        out[0] = __builtin_nontemporal_load(p);
    } else if constexpr (kE == 2) {
        const f32x2 w = __builtin_nontemporal_load(reinterpret_cast<const f32x2*>(p));
        out[0] = w.x;
        out[1] = w.y;
    } else {
        const f32x4 w = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = w[j];
    }
}
// the first n (1..kE) of kE fp32 values, non-temporal: one vector store when n == kE
template <int kE>
__device__ __forceinline__ void st_lane(float* p, const float* v, int n) {
    if constexpr (kE == 1) {
        __builtin_nontemporal_store(v[0], p);
    } else if constexpr (kE == 2) {
        if (n == 2)
            __builtin_nontemporal_store(f32x2{v[0], v[1]}, reinterpret_cast<f32x2*>(p));
        else
            __builtin_nontemporal_store(v[0], p);
    } else {
        if (n == 4) {
            __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]},
                                        reinterpret_cast<f32x4*>(p));
        } else {
#pragma unroll
            for (int j = 0; j < 3; ++j)
                if (j < n) __builtin_nontemporal_store(v[j], p + j);
        }
    }
}
template <int kE>
__device__ __forceinline__ void st_bf16_lane(uint16_t* p, const float* v, int n) {
    if constexpr (kE == 1) {
        __builtin_nontemporal_store((uint16_t)bf16_rne(v[0]), p);
    } else if constexpr (kE == 2) {
        if (n == 2)
            __builtin_nontemporal_store(bf16_pack(v[0], v[1]), reinterpret_cast<uint32_t*>(p));
        else
            __builtin_nontemporal_store((uint16_t)bf16_rne(v[0]), p);
    } else {
        if (n == 4) {
            __builtin_nontemporal_store(u32x2{bf16_pack(v[0], v[1]), bf16_pack(v[2], v[3])},
                                        reinterpret_cast<u32x2*>(p));
        } else {
#pragma unroll
            for (int j = 0; j < 3; ++j)
                if (j < n) __builtin_nontemporal_store((uint16_t)bf16_rne(v[j]), p + j);
        }
    }
}

// One piece of the lane-form Adam update: this lane's kE elements at flat index i (the first
// n of them stored: a tensor's last piece may end inside the lane).
template <typename GradT, bool kMixed, int kE>
__device__ __forceinline__ void adam_piece(const GradT* __restrict__ grad,
                                           float* __restrict__ records, float* __restrict__ master,
                                           uint16_t* __restrict__ param16, const AdamArgs& a,
                                           const Coefs& k, bool use_inv, bool use_clip,
                                           bool decay, uint64_t i, int n) {
    constexpr uint32_t kStateStride = kMixed ? kStrideMixed : kStrideMV;
    const uint64_t s = rec_index(i, kStateStride);
    float* pp = kMixed ? records + s : master + i;
    float* mp = kMixed ? records + s + kRec : records + s;
    float* vp = mp + kRec;
    float g[kE], p[kE], m[kE], v[kE];
    ld_grad_lane<kE>(grad, i, g);
    ld_lane<kE>(pp, p);
    ld_lane<kE>(mp, m);
    ld_lane<kE>(vp, v);
#pragma unroll
    for (int j = 0; j < kE; ++j) adam_elem(p[j], g[j], m[j], v[j], a, k, use_inv, use_clip, decay);
    st_lane<kE>(pp, p, n);
    st_lane<kE>(mp, m, n);
    st_lane<kE>(vp, v, n);
    if (kMixed) st_bf16_lane<kE>(param16 + i, p, n);
}

// The lane-form Adam update: one block per part of kIt consecutive pieces of kLanes x kE
// elements, r = nparts - 1 - (part0 + blockIdx.x) (the last chunks first, as the norm pass);
// the host splits stores beyond one launch's 2^32 - 1 work-items into launches at increasing
// part0.  With kIt = 2 each lane walks its two pieces in turn (a loop the compiler keeps
// rolled): at GPT-2 774M mixed that measured 1.01x the copy against 0.96-0.98x for one piece
// per block, and halves the grid a skipped step dispatches.  records is the record array's
// base ([master|m|v] in MIXED, [m|v] in FP32), master the contiguous FP32 weights (unused in
// MIXED).  a.st must be valid: its fields are read unconditionally and used as a.flags say.
// The arithmetic is adam_elem's, so every shape gives the same results bit for bit.
template <typename GradT, bool kMixed, int kE, int kLanes, int kIt>
__global__ __launch_bounds__(kLanes) void adam_lane_kernel(const GradT* __restrict__ grad,
                                                           float* __restrict__ records,
                                                           float* __restrict__ master,
                                                           uint16_t* __restrict__ param16,
                                                           AdamArgs a, uint64_t part0) {
    constexpr uint32_t kPiece = kLanes * kE;
    constexpr uint32_t kP = lane_parts<kE, kLanes, kIt>();
    const uint64_t r = (uint64_t)a.nchunks * kP - 1 - (part0 + blockIdx.x);
    const Chunk ch = load_chunk(a.chunks, r / kP);
    const DevState* st = a.st;
    // `|` and `&`, not `||` and `&&`: the skip flag and the descriptor are both needed before
    // the first branch, so their loads issue together
    const bool run = ((a.flags & kCheckSkip) == 0) | (st->skip == 0);
    const uint32_t off = (uint32_t)(r % kP) * (kPiece * kIt) + threadIdx.x * kE;
    if (!(run & (off < ch.count))) return;
    const bool dev_bias = a.flags & kDevBias;
    const Coefs k{st->inv_scale, st->clip_coef, dev_bias ? st->bias1 : a.bias1,
                  dev_bias ? st->bias2 : a.bias2};
    const bool use_inv = a.flags & kUseInv, use_clip = a.flags & kUseClip;
    const bool decay = (ch.meta & kChunkDecay) && (a.flags & kWdOn);
    if constexpr (kIt == 1) {
        adam_piece<GradT, kMixed, kE>(grad, records, master, param16, a, k, use_inv, use_clip,
                                      decay, ch.begin + off,
                                      (int)min(ch.count - off, (uint32_t)kE));
    } else {
#pragma unroll 1
        for (int q = 0; q < kIt; ++q) {
            const uint32_t o = off + q * kPiece;
            if (o >= ch.count) break;
            adam_piece<GradT, kMixed, kE>(grad, records, master, param16, a, k, use_inv,
                                          use_clip, decay, ch.begin + o,
                                          (int)min(ch.count - o, (uint32_t)kE));
        }
    }
}

// ------------------------------------------------------------------------------------
// fused SGD (+ momentum / dampening / nesterov / L2)
// ------------------------------------------------------------------------------------
constexpr uint32_t kMomOn = 64u;
constexpr uint32_t kNesterov = 128u;

struct SgdArgs {
    const Chunk* chunks;
    uint32_t nchunks;
    uint32_t flags;
    float lr, mu, omd, wd;
    const uint32_t* mom_init;  // per tensor: 1 once the momentum buffer holds a value
    const DevState* st;
};

// One element of SGD: grad transforms, L2 decay, momentum / dampening / nesterov, then
// `p - g*lr` rounded after the multiply and after the subtract.
__device__ __forceinline__ void sgd_elem(float& p, float g, float& b, const SgdArgs& a, float inv,
                                         float clip, bool use_inv, bool use_clip, bool decay,
                                         bool mom_on, bool first, bool nesterov) {
    if (use_inv) g = g * inv;
    if (use_clip) g = g * clip;
    if (decay) g = g + a.wd * p;
    if (mom_on) {
        const float bj = first ? g : a.mu * b + a.omd * g;
        b = bj;
        g = nesterov ? g + a.mu * bj : bj;
    }
    const float update = g * a.lr;  // autograd/dynamic/optim.hpp:24
    p = p - update;                 // autograd/dynamic/optim.hpp:25
}

// Flat element i of a master slot with kMStride elements per record: kRec is a contiguous
// master (FP32 mode, and the SGD layout of a MIXED store), kStrideMixed slot 0 of the
// [master|m|v] records.
template <uint32_t kMStride>
__device__ __forceinline__ uint64_t master_index(uint64_t i) {
    if constexpr (kMStride == kRec) return i;
    else return rec_index(i, kMStride);
}

// The four-element SGD update: one block per chunk (grid == nchunks), blocks in reverse chunk
// order, one 4-element vector per lane, for MIXED momentum steps whose gradients fit the
// Infinity Cache (at most 2^17 chunks), at most kUpdBlocksPerCU blocks per CU.  master is
// the master slot base (see master_index); momentum is contiguous.
template <typename GradT, bool kMixed, uint32_t kMStride>
__global__ __launch_bounds__(kUpdBlock) void sgd_kernel(const GradT* __restrict__ grad,
                                                        float* __restrict__ master,
                                                        float* __restrict__ momentum,
                                                        uint16_t* __restrict__ param16,
                                                        SgdArgs a) {
    float inv = 1.0f, clip = 1.0f;
    if (a.st) {
        if ((a.flags & kCheckSkip) && a.st->skip) return;
        inv = a.st->inv_scale;
        clip = a.st->clip_coef;
    }
    const bool use_inv = a.flags & kUseInv, use_clip = a.flags & kUseClip;
    const bool mom_on = a.flags & kMomOn, nesterov = a.flags & kNesterov;
    const Chunk ch = a.chunks[a.nchunks - 1 - blockIdx.x];  // last chunks first (see norm pass)
    const uint32_t off = threadIdx.x * kVec;
    if (off >= ch.count) return;
    const int n = (int)min(ch.count - off, (uint32_t)kVec);
    const bool decay = (ch.meta & kChunkDecay) && (a.flags & kWdOn);
    const bool first = mom_on && a.mom_init[ch.meta >> 8] == 0u;
    const uint64_t i = ch.begin + off;
    float* pp = master + master_index<kMStride>(i);
    f32x4 g = ld_grad4(grad, i);
    f32x4 p = ld4(pp);
    f32x4 b = {0.0f, 0.0f, 0.0f, 0.0f};
    if (mom_on && !first) b = ld4(momentum + i);
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
        float pj = p[j], bj = b[j];
        sgd_elem(pj, g[j], bj, a, inv, clip, use_inv, use_clip, decay, mom_on, first, nesterov);
        p[j] = pj;
        b[j] = bj;
    }
    store_vec<kMixed>(pp, mom_on ? momentum + i : nullptr, nullptr, param16, i, p, b, b, n);
}

// One piece of the lane-form SGD update (see adam_piece).
template <typename GradT, bool kMixed, uint32_t kMStride, int kE>
__device__ __forceinline__ void sgd_piece(const GradT* __restrict__ grad,
                                          float* __restrict__ master,
                                          float* __restrict__ momentum,
                                          uint16_t* __restrict__ param16, const SgdArgs& a,
                                          float inv, float clip, bool use_inv, bool use_clip,
                                          bool decay, bool mom_on, bool first, bool nesterov,
                                          uint64_t i, int n) {
    float* pp = master + master_index<kMStride>(i);
    float g[kE], p[kE], bm[kE];
    ld_grad_lane<kE>(grad, i, g);
    ld_lane<kE>(pp, p);
    if (mom_on && !first) {
        ld_lane<kE>(momentum + i, bm);
    } else {
#pragma unroll
        for (int j = 0; j < kE; ++j) bm[j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kE; ++j)
        sgd_elem(p[j], g[j], bm[j], a, inv, clip, use_inv, use_clip, decay, mom_on, first,
                 nesterov);
    st_lane<kE>(pp, p, n);
    if (mom_on) st_lane<kE>(momentum + i, bm, n);
    if (kMixed) st_bf16_lane<kE>(param16 + i, p, n);
}

// The lane-form SGD update, launched and shaped as adam_lane_kernel.  master is the master
// slot base (see master_index); momentum is contiguous.  a.st must be valid.
template <typename GradT, bool kMixed, uint32_t kMStride, int kE, int kLanes, int kIt>
__global__ __launch_bounds__(kLanes) void sgd_lane_kernel(const GradT* __restrict__ grad,
                                                          float* __restrict__ master,
                                                          float* __restrict__ momentum,
                                                          uint16_t* __restrict__ param16,
                                                          SgdArgs a, uint64_t part0) {
    constexpr uint32_t kPiece = kLanes * kE;
    constexpr uint32_t kP = lane_parts<kE, kLanes, kIt>();
    const uint64_t r = (uint64_t)a.nchunks * kP - 1 - (part0 + blockIdx.x);
    const Chunk ch = load_chunk(a.chunks, r / kP);
    const DevState* st = a.st;
    const bool run = ((a.flags & kCheckSkip) == 0) | (st->skip == 0);  // see adam_lane_kernel
    const uint32_t off = (uint32_t)(r % kP) * (kPiece * kIt) + threadIdx.x * kE;
    if (!(run & (off < ch.count))) return;
    const bool use_inv = a.flags & kUseInv, use_clip = a.flags & kUseClip;
    const bool mom_on = a.flags & kMomOn, nesterov = a.flags & kNesterov;
    const bool decay = (ch.meta & kChunkDecay) && (a.flags & kWdOn);
    const bool first = mom_on && a.mom_init[ch.meta >> 8] == 0u;
    const float inv = st->inv_scale, clip = st->clip_coef;
    if constexpr (kIt == 1) {
        sgd_piece<GradT, kMixed, kMStride, kE>(grad, master, momentum, param16, a, inv, clip,
                                               use_inv, use_clip, decay, mom_on, first, nesterov,
                                               ch.begin + off,
                                               (int)min(ch.count - off, (uint32_t)kE));
    } else {
#pragma unroll 1
        for (int q = 0; q < kIt; ++q) {
            const uint32_t o = off + q * kPiece;
            if (o >= ch.count) break;
            sgd_piece<GradT, kMixed, kMStride, kE>(grad, master, momentum, param16, a, inv, clip,
                                                   use_inv, use_clip, decay, mom_on, first,
                                                   nesterov, ch.begin + o,
                                                   (int)min(ch.count - o, (uint32_t)kE));
        }
    }
}

// ------------------------------------------------------------------------------------
// plain SGD of a TTP_MODE_BF16 store: bf16 weights updated in place, no fp32 state
// ------------------------------------------------------------------------------------
// The value of x rounded to bf16 (round to nearest even; NaN -> the quiet NaN 0x7FC0).
__device__ __forceinline__ float bf16_round(float x) {
    return __uint_as_float(bf16_rne(x) << 16);
}

// One element: the grad transforms, then autograd/dynamic/optim.hpp:24-25 on bf16 tensors,
// each ttnn op's result rounded to bf16: update = multiply(grad, lr), data = subtract(data,
// update).  Product and difference are formed in fp32 and rounded from there.
__device__ __forceinline__ float sgd_bf16_elem(float p, float g, float lr, float inv, float clip,
                                               bool use_inv, bool use_clip) {
    if (use_inv) g = g * inv;
    if (use_clip) g = g * clip;
    const float update = bf16_round(g * lr);  // autograd/dynamic/optim.hpp:24
    return bf16_round(p - update);            // autograd/dynamic/optim.hpp:25
}

// kE (2, 4 or 8) bf16 values at p as fp32: one 4-, 8- or 16-byte word (non-temporal: the
// weights are read once and rewritten)
template <int kE>
__device__ __forceinline__ void ld_bf16_lane(const uint16_t* p, float* out) {
    static_assert(kE == 2 || kE == 4 || kE == 8, "2, 4 or 8 elements per lane");
    if constexpr (kE == 2) {
        const uint32_t w = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
        out[0] = bf16_lo(w);
        out[1] = bf16_hi(w);
    } else if constexpr (kE == 4) {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        out[0] = bf16_lo(w.x);
        out[1] = bf16_hi(w.x);
        out[2] = bf16_lo(w.y);
        out[3] = bf16_hi(w.y);
    } else {
        const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            out[2 * j] = bf16_lo(w[j]);
            out[2 * j + 1] = bf16_hi(w[j]);
        }
    }
}
// kE gradients as fp32 (ordinary loads, as ld_grad_lane)
template <int kE>
__device__ __forceinline__ void ld_grad_bf16_lane(const uint16_t* g, float* out) {
    if constexpr (kE <= 4) {
        ld_grad_lane<kE>(g, 0, out);
    } else {
        const u32x4 w = *reinterpret_cast<const u32x4*>(g);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            out[2 * j] = bf16_lo(w[j]);
            out[2 * j + 1] = bf16_hi(w[j]);
        }
    }
}
// the first n (1..kE) of kE values already rounded to bf16: one word when n == kE
template <int kE>
__device__ __forceinline__ void st_bf16_rounded_lane(uint16_t* p, const float* v, int n) {
    if (n == kE) {
        if constexpr (kE == 2) {
            __builtin_nontemporal_store(bf16_pack(v[0], v[1]), reinterpret_cast<uint32_t*>(p));
        } else if constexpr (kE == 4) {
            __builtin_nontemporal_store(u32x2{bf16_pack(v[0], v[1]), bf16_pack(v[2], v[3])},
                                        reinterpret_cast<u32x2*>(p));
        } else {
            __builtin_nontemporal_store(u32x4{bf16_pack(v[0], v[1]), bf16_pack(v[2], v[3]),
                                              bf16_pack(v[4], v[5]), bf16_pack(v[6], v[7])},
                                        reinterpret_cast<u32x4*>(p));
        }
    } else {
#pragma unroll
        for (int j = 0; j < kE - 1; ++j)
            if (j < n) p[j] = (uint16_t)bf16_rne(v[j]);
    }
}

// The plain SGD update of a BF16 store, launched and shaped as the other lane forms (one
// block per 1/lane_parts of a chunk, the last chunks first): 6 B per element (gradient and
// weight read, weight written).  A lane's kE elements start at a multiple of kE and tensors
// start on 64-element boundaries, so the whole-word loads of a tensor's last lane stay inside
// its footprint; only its first n values are stored.  a.st must be valid.
template <int kE, int kLanes, int kIt>
__global__ __launch_bounds__(kLanes) void sgd_bf16_lane_kernel(const uint16_t* __restrict__ grad,
                                                               uint16_t* __restrict__ param,
                                                               SgdArgs a, uint64_t part0) {
    constexpr uint32_t kPiece = kLanes * kE;
    constexpr uint32_t kP = lane_parts<kE, kLanes, kIt>();
    const uint64_t r = (uint64_t)a.nchunks * kP - 1 - (part0 + blockIdx.x);
    const Chunk ch = load_chunk(a.chunks, r / kP);
    const DevState* st = a.st;
    const bool run = ((a.flags & kCheckSkip) == 0) | (st->skip == 0);  // see adam_lane_kernel
    const uint32_t off = (uint32_t)(r % kP) * (kPiece * kIt) + threadIdx.x * kE;
    if (!(run & (off < ch.count))) return;
    const bool use_inv = a.flags & kUseInv, use_clip = a.flags & kUseClip;
    const float inv = st->inv_scale, clip = st->clip_coef;
#pragma unroll 1
    for (int q = 0; q < kIt; ++q) {
        const uint32_t o = off + q * kPiece;
        if (o >= ch.count) break;
        const uint64_t i = ch.begin + o;
        float g[kE], p[kE];
        ld_grad_bf16_lane<kE>(grad + i, g);
        ld_bf16_lane<kE>(param + i, p);
#pragma unroll
        for (int j = 0; j < kE; ++j)
            p[j] = sgd_bf16_elem(p[j], g[j], a.lr, inv, clip, use_inv, use_clip);
        st_bf16_rounded_lane<kE>(param + i, p, (int)min(ch.count - o, (uint32_t)kE));
    }
}

// after a momentum step: mark the stepped tensors' buffers as initialised (unless skipped)
__global__ __launch_bounds__(kBlock) void mark_mom_init_kernel(const Chunk* chunks, uint32_t n,
                                                               uint32_t* mom_init,
                                                               const DevState* st,
                                                               int check_skip) {
    if (check_skip && st->skip) return;
    for (uint32_t c = blockIdx.x * kBlock + threadIdx.x; c < n; c += gridDim.x * kBlock)
        mom_init[chunks[c].meta >> 8] = 1u;
}

// ------------------------------------------------------------------------------------
// gradient accumulation into the flat grad buffer (the backward side of the store)
// ------------------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ void from_f32(float x, float* out) { *out = x; }
__device__ __forceinline__ void from_f32(float x, uint16_t* out) { *out = (uint16_t)bf16_rne(x); }

// first: grad = incoming (converted); else grad = grad + incoming (fp32 add, one rounding)
template <typename SrcT, typename GradT>
__global__ __launch_bounds__(kBlock) void accumulate_grad_kernel(GradT* __restrict__ grad,
                                                                 const SrcT* __restrict__ src,
                                                                 uint64_t n, int first) {
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * kBlock) {
        const float in = to_f32(src[i]);
        const float r = first ? in : to_f32(grad[i]) + in;
        from_f32(r, grad + i);
    }
}

// zero the grads of the chunks' tensors (a module's zero_grad): one vector per lane
__device__ __forceinline__ void zero_vec(float* g, uint64_t i, int n) {
    if (n >= kVec) {
        st4(g + i, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
    } else {
        for (int j = 0; j < n; ++j) g[i + j] = 0.0f;
    }
}
__device__ __forceinline__ void zero_vec(uint16_t* g, uint64_t i, int n) {
    if (n >= kVec) {
        __builtin_nontemporal_store(u32x2{0u, 0u}, reinterpret_cast<u32x2*>(g + i));
    } else {
        for (int j = 0; j < n; ++j) g[i + j] = 0;
    }
}

// The same accumulation over one tensor of n elements in 16 KiB norm tiles, one 64-lane block
// per wave-share of a tile (kAccBlocksPerTile blocks per tile), all of a lane's loads of a whole
// tile issued before its arithmetic (the grid-stride kernel above, one element per lane per
// iteration, serves tensors of 2^24 or more tiles only).
// kSums: it also computes the sum of squares of the resulting (stored) gradients, unscaled by
// 1/scale when scaler_on: tile t of the tensor (tiles start at its first element, as the norm
// pass's tiles do) is split over kAccBlocksPerTile one-wave blocks, and each lane takes the
// elements that lane `lane` (0..kBlock-1) of the norm pass takes in that tile (kNormLoads
// vectors of GradVec<GradT>::kElems); the squares go into the two accumulators in the norm
// pass's order, and each wave's total (wave_sum, block_sum's first stage) is stored as that
// tile's partial of that wave.  tile_from_waves then adds a tile's wave partials as block_sum
// does, so the tile sums are bit-identical to norm_partials_kernel's over the same gradients.
// A wave's partial needs no LDS and no barrier (a block reduction lengthened each launch by
// 0.6-2.4 us).  The first wave of tile 0 marks the tensor's partials pending.  The squares come
// from values already in registers, so the sums add no memory traffic.
// Measured on MI355X over GPT-2 124M's seven 25 MB buckets of bf16 gradients (assigned; each
// source written just before its call, as a backward leaves it, or long before): one-wave
// blocks against 256-lane ones 92-101 against 98-108 us with the sums (within 2% without);
// non-temporal source loads against cached ones 83-97 against 94-110 us without the sums
// (added onto the stored gradients: 126 against 132-154 us).  The source is read once.
// kVecSrc: the source is 16-byte aligned and read in non-temporal vectors (else element by
// element).
constexpr uint32_t kAccLanes = 64;
constexpr uint32_t kAccBlocksPerTile = kBlock / kAccLanes;
template <int E, bool kVecSrc>
__device__ __forceinline__ void ld_src(const uint16_t* p, float* out) {
    if constexpr (kVecSrc && E == 8) {
        const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            out[2 * j] = bf16_lo(w[j]);
            out[2 * j + 1] = bf16_hi(w[j]);
        }
    } else if constexpr (kVecSrc && E == 4) {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        out[0] = bf16_lo(w.x);
        out[1] = bf16_hi(w.x);
        out[2] = bf16_lo(w.y);
        out[3] = bf16_hi(w.y);
    } else {
#pragma unroll
        for (int j = 0; j < E; ++j) out[j] = to_f32(p[j]);
    }
}
template <int E, bool kVecSrc>
__device__ __forceinline__ void ld_src(const float* p, float* out) {
    if constexpr (kVecSrc) {
#pragma unroll
        for (int h = 0; h < E / 4; ++h) {
            const f32x4 w = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4 * h));
#pragma unroll
            for (int j = 0; j < 4; ++j) out[4 * h + j] = w[j];
        }
    } else {
#pragma unroll
        for (int j = 0; j < E; ++j) out[j] = p[j];
    }
}

// Tile `tile` of one tensor's gradients (grad, n elements) from src, as the lanes
// wave * 64 .. wave * 64 + 63 of a 256-lane tile: a one-wave block's work in both accumulate
// kernels.  inv: 1/scale for the sums; wave_sums: the tensor's run of the store-wide wave
// partials; pending: its flag, which the first wave of its first tile sets.
template <typename SrcT, typename GradT, bool kVecSrc, bool kSums>
__device__ __forceinline__ void accumulate_tile(GradT* __restrict__ grad,
                                                const SrcT* __restrict__ src, uint64_t n,
                                                int first, float inv, uint32_t tile,
                                                uint32_t wave, double* __restrict__ wave_sums,
                                                uint32_t* __restrict__ pending) {
    const uint32_t lane = wave * kAccLanes + threadIdx.x;  // the lane of a 256-lane tile
    typedef GradVec<GradT> GV;
    typedef typename GV::raw R;
    constexpr int E = GV::kElems;
    constexpr uint32_t kTile = norm_tile_elems<GradT>();
    const uint64_t t0 = (uint64_t)tile * kTile;
    // Elements from this tile's start to the tensor's end; below kTile, the last tile's count.
    // No min() of the two ahead of the branch: hipcc (ROCm 7.2, gfx950) has built such a
    // min as a scalar select at the top of the last-tile branch that read the condition code
    // of another compare (of `first`), so that an assign into a last tile took the whole tile
    // and wrote past the tensor's end (tests/test_isa_cpu.py scans for that form).
    const uint64_t left = n - t0;
    double acc[2] = {0.0, 0.0};
    // the squares of a vector's stored values, in the norm pass's order
    auto add_squares = [&](const float* v, uint32_t nv) {
        if constexpr (kSums) {
#pragma unroll
            for (int j = 0; j < E; ++j) {
                const double x = (uint32_t)j < nv ? (double)(v[j] * inv) : 0.0;
                acc[j & 1] = __builtin_fma(x, x, acc[j & 1]);
            }
        }
    };
    // a whole vector's new values from the incoming ones (and the old gradient vector w),
    // stored as one 16-byte word; v receives the stored values
    auto store_vec = [&](uint64_t i, const float* in, const R& w, float* v) {
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const float r = first ? in[j] : GV::at(w, j) + in[j];
            GradT h;
            from_f32(r, &h);
            v[j] = to_f32(h);
        }
        if constexpr (E == 8) {
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = bf16_pack(v[2 * j], v[2 * j + 1]);
            *reinterpret_cast<u32x4*>(grad + i) = o;
        } else {
            *reinterpret_cast<f32x4*>(grad + i) = f32x4{v[0], v[1], v[2], v[3]};
        }
    };
    if (left >= kTile) {
        // a whole tile: every load of the lane issued before the arithmetic (the scheduling
        // barrier keeps them ahead of it, as in the norm pass: with one vector in flight at a
        // time the call ran at a fraction of the copy rate)
        float in[kNormLoads][E];
        R w[kNormLoads];
#pragma unroll
        for (int l = 0; l < kNormLoads; ++l) {
            const uint64_t i = t0 + (uint32_t)(l * kBlock + lane) * E;
            ld_src<E, kVecSrc>(src + i, in[l]);
            if (!first) w[l] = *reinterpret_cast<const R*>(grad + i);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int l = 0; l < kNormLoads; ++l) {
            float v[E];
            store_vec(t0 + (uint32_t)(l * kBlock + lane) * E, in[l], w[l], v);
            add_squares(v, (uint32_t)E);
        }
    } else {  // a tensor's last tile: the vectors (and elements) below its count
        const uint32_t count = (uint32_t)left;
#pragma unroll
        for (int l = 0; l < kNormLoads; ++l) {
            const uint32_t off = (uint32_t)(l * kBlock + lane) * E;
            const uint32_t nv = off < count ? min(count - off, (uint32_t)E) : 0u;
            if (!nv) continue;
            const uint64_t i = t0 + off;
            float v[E];
            if (nv == (uint32_t)E) {
                float in[E];
                ld_src<E, kVecSrc>(src + i, in);
                R w;
                if (!first) w = *reinterpret_cast<const R*>(grad + i);
                store_vec(i, in, w, v);
            } else {  // the tensor's last, partial vector
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    v[j] = 0.0f;
                    if ((uint32_t)j < nv) {
                        const float x = to_f32(src[i + j]);
                        const float r = first ? x : to_f32(grad[i + j]) + x;
                        GradT h;
                        from_f32(r, &h);
                        grad[i + j] = h;
                        v[j] = to_f32(h);
                    }
                }
            }
            add_squares(v, nv);
        }
    }
    if constexpr (kSums) {
        // each wave's total, the first stage of block_sum, with no LDS or barrier after it
        const double part = wave_sum(acc[0] + acc[1]);
        if (threadIdx.x == 0) wave_sums[(uint64_t)tile * kWaves + wave] = part;
        if (tile == 0 && lane == 0) *pending = 1u;
    }
}

// one tensor per launch, kAccBlocksPerTile one-wave blocks per tile
template <typename SrcT, typename GradT, bool kVecSrc, bool kSums>
__global__ __launch_bounds__(kAccLanes) void accumulate_grad_tiles_kernel(
    GradT* __restrict__ grad, const SrcT* __restrict__ src, uint64_t n, int first,
    const DevState* __restrict__ st, int32_t scaler_on, double* __restrict__ wave_sums,
    uint32_t* __restrict__ pending) {
    const float inv = (kSums && scaler_on) ? (float)(1.0 / (double)st->scale) : 1.0f;
    accumulate_tile<SrcT, GradT, kVecSrc, kSums>(grad, src, n, first, inv,
                                                 blockIdx.x / kAccBlocksPerTile,
                                                 blockIdx.x % kAccBlocksPerTile, wave_sums,
                                                 pending);
}

// Several tensors per launch (a backward's bucket): the table travels in the kernel
// arguments, so a call allocates and copies nothing and can be captured.  Tensor k takes
// tiles [tile_end[k-1], tile_end[k]) of the launch, kAccBlocksPerTile one-wave blocks each;
// its fields as in accumulate_grad_tiles_kernel.
constexpr uint32_t kMultiMax = 64;
struct MultiAccArgs {
    uint32_t n;                      // tensors in the table (each with at least one element)
    uint32_t first[kMultiMax / 32];  // bit k: tensor k has no grad yet (its values assign)
    uint32_t tile_end[kMultiMax];    // tiles of tensors 0..k
    uint32_t tile_base[kMultiMax];   // its first tile in the store-wide wave partials
    uint32_t tensor[kMultiMax];      // its index in the tensor table (its pending flag)
    uint64_t offset[kMultiMax];      // its first element in the flat grad buffer
    uint64_t numel[kMultiMax];
    const void* src[kMultiMax];
};

template <typename SrcT, typename GradT, bool kVecSrc, bool kSums>
__global__ __launch_bounds__(kAccLanes) void accumulate_grads_multi_kernel(
    GradT* __restrict__ grad, const MultiAccArgs a, const DevState* __restrict__ st,
    int32_t scaler_on, double* __restrict__ wave_sums, uint32_t* __restrict__ pending) {
    // the block's tensor: the first k with its tile g < tile_end[k] (uniform in the block)
    const uint32_t g = blockIdx.x / kAccBlocksPerTile;
    uint32_t lo = 0, hi = a.n - 1;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (g < a.tile_end[mid])
            hi = mid;
        else
            lo = mid + 1;
    }
    const uint32_t k = lo;
    const uint32_t tile = g - (k ? a.tile_end[k - 1] : 0u);
    const float inv = (kSums && scaler_on) ? (float)(1.0 / (double)st->scale) : 1.0f;
    accumulate_tile<SrcT, GradT, kVecSrc, kSums>(
        grad + a.offset[k], static_cast<const SrcT*>(a.src[k]), a.numel[k],
        (int)((a.first[k >> 5] >> (k & 31)) & 1u), inv, tile, blockIdx.x % kAccBlocksPerTile,
        wave_sums + (uint64_t)a.tile_base[k] * kWaves, pending + a.tensor[k]);
}

template <typename GradT>
__global__ __launch_bounds__(kUpdBlock) void zero_chunks_kernel(GradT* __restrict__ grad,
                                                                const Chunk* __restrict__ chunks,
                                                                uint32_t nchunks) {
    for (uint32_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
        const Chunk ch = chunks[c];
        const uint32_t off = threadIdx.x * kVec;
        if (off >= ch.count) continue;
        zero_vec(grad, ch.begin + off, (int)min(ch.count - off, (uint32_t)kVec));
    }
}

// ------------------------------------------------------------------------------------
// small elementwise helpers
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void fill_zero_kernel(uint32_t* p, uint64_t n_words) {
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n_words;
         i += (uint64_t)gridDim.x * kBlock)
        p[i] = 0u;
}

// The kernels below address a state slot (base, stride) over the flat elements
// [first, first + n); stride == kRec is a contiguous buffer.

// bf16 copy of the master weights: p16[i] = RNE(master[i])
__global__ __launch_bounds__(kBlock) void master_to_bf16_kernel(const float* master,
                                                                uint32_t stride, uint16_t* p16,
                                                                uint64_t first, uint64_t n) {
    for (uint64_t k = (uint64_t)blockIdx.x * kBlock + threadIdx.x; k < n;
         k += (uint64_t)gridDim.x * kBlock) {
        const uint64_t i = first + k;
        p16[i] = (uint16_t)bf16_rne(master[rec_index(i, stride)]);
    }
}

// master[i] = float(p16[i]) (exact widening)
__global__ __launch_bounds__(kBlock) void bf16_to_master_kernel(const uint16_t* p16,
                                                                float* master, uint32_t stride,
                                                                uint64_t first, uint64_t n) {
    for (uint64_t k = (uint64_t)blockIdx.x * kBlock + threadIdx.x; k < n;
         k += (uint64_t)gridDim.x * kBlock) {
        const uint64_t i = first + k;
        master[rec_index(i, stride)] = __uint_as_float((uint32_t)p16[i] << 16);
    }
}

// dst[k] = slot[first + k]: a slot's elements as one contiguous array (downloads, checkpoints)
__global__ __launch_bounds__(kBlock) void gather_slot_kernel(const float* slot, uint32_t stride,
                                                             uint64_t first, uint64_t n,
                                                             float* dst) {
    for (uint64_t k = (uint64_t)blockIdx.x * kBlock + threadIdx.x; k < n;
         k += (uint64_t)gridDim.x * kBlock)
        dst[k] = slot[rec_index(first + k, stride)];
}

// slot[first + k] = src[k] (0 when src is null); with p16, also p16[first + k] = RNE(value)
// (an upload of MIXED-mode master weights keeps the bf16 copy consistent)
__global__ __launch_bounds__(kBlock) void scatter_slot_kernel(float* slot, uint32_t stride,
                                                              uint64_t first, uint64_t n,
                                                              const float* src, uint16_t* p16) {
    for (uint64_t k = (uint64_t)blockIdx.x * kBlock + threadIdx.x; k < n;
         k += (uint64_t)gridDim.x * kBlock) {
        const uint64_t i = first + k;
        const float x = src ? src[k] : 0.0f;
        slot[rec_index(i, stride)] = x;
        if (p16) p16[i] = (uint16_t)bf16_rne(x);
    }
}

}  // namespace ttp
