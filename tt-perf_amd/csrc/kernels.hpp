// kernels.hpp — gfx950 device code of libttperf_hip.
//
// Two passes make one optimizer step over the flat store:
//   norm_kernel    reads only the gradients (2 B/param bf16, 4 B/param fp32): fp64 sum of
//                  squares of the unscaled grads, wave shuffle + LDS block tree, one partial
//                  per block, and a last-block finalize (atomic ticket) that sums the partials
//                  in index order (deterministic), decides found_inf / skip, the clip
//                  coefficient, advances the step count and the loss scale.
//   adam_kernel /  one fused pass per element: grad transform (unscale, clip), weight decay,
//   sgd_kernel     the optimizer update and the bf16 copy.  Each element is touched once;
//                  loads/stores are 16-byte (fp32 x4) and 8-byte (bf16 x4) per lane, so every
//                  wave instruction covers a contiguous 1 KiB / 512 B span.
// Work is a table of chunks (<= chunk_elems elements of one tensor, 64-element aligned
// start); block b takes chunks b, b+grid, ...  No MFMA: nothing here is a contraction.
//
// Arithmetic matches the oracle bit for bit: no contraction (-ffp-contract=off), IEEE
// division and square root (HIP's correctly rounded fp32 div/sqrt), denormals kept.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ttp {

constexpr int kBlock = 256;   // 4 wave64s
constexpr int kVec = 4;       // elements per lane per vector
constexpr uint32_t kChunkDecay = 1u;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct Chunk {
    uint64_t begin;  // first element (flat index)
    uint32_t count;  // elements in this chunk (exact, not padded)
    uint32_t meta;   // bit 0: decay; bits 8..31: tensor index
};

// Device-resident step state.  Written only by the norm pass's last block (and by the
// host between steps); read by the update pass that follows it on the same stream.
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
    uint32_t ticket;         // blocks finished; the last block puts it back to 0
    uint32_t pad;
};

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

// 4 gradients as fp32 from either storage type
__device__ __forceinline__ f32x4 ld_grad4(const float* g, uint64_t i) { return ld4(g + i); }
__device__ __forceinline__ f32x4 ld_grad4(const uint16_t* g, uint64_t i) {
    const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(g + i));
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
// norm / inf-check / finalize pass
// ------------------------------------------------------------------------------------
struct NormArgs {
    const Chunk* chunks;
    uint32_t nchunks;
    int32_t scaler_on;      // unscale by 1/scale, skip on inf, update the scale, own t
    int32_t probe;          // only compute sumsq/norm (ttp_grad_norm); touch nothing else
    int32_t growth_interval;
    double growth_factor;
    double backoff_factor;
    double max_norm;        // > 0: clip
    const float* bias_tab;  // [2*bias_len]: (1-beta1^t, 1-beta2^t) for t = 1..bias_len
    uint32_t bias_len;      // t > bias_len: both corrections are exactly 1.0f
    int32_t want_bias;
    double* partials;       // [gridDim.x]
    DevState* st;
};

template <typename GradT>
__global__ __launch_bounds__(kBlock) void norm_kernel(const GradT* __restrict__ g, NormArgs a) {
    __shared__ double lds[kBlock / 64];
    __shared__ int last;
    const float inv = a.scaler_on ? (float)(1.0 / (double)a.st->scale) : 1.0f;
    double acc = 0.0;
    for (uint32_t c = blockIdx.x; c < a.nchunks; c += gridDim.x) {
        const Chunk ch = a.chunks[c];
        const uint64_t end = ch.begin + ch.count;
        for (uint64_t i = ch.begin + (uint64_t)threadIdx.x * kVec; i < end;
             i += (uint64_t)kBlock * kVec) {
            f32x4 v = ld_grad4(g, i);
            const int n = (int)min<uint64_t>(end - i, kVec);
            v.x = v.x * inv;
            v.y = n > 1 ? v.y * inv : 0.0f;
            v.z = n > 2 ? v.z * inv : 0.0f;
            v.w = n > 3 ? v.w * inv : 0.0f;
            // squares of fp32 values are exact in fp64; any inf/NaN makes the sum non-finite
            acc += (double)v.x * (double)v.x;
            acc += (double)v.y * (double)v.y;
            acc += (double)v.z * (double)v.z;
            acc += (double)v.w * (double)v.w;
        }
    }
    const double bsum = block_sum(acc, lds);
    if (threadIdx.x == 0) {
        a.partials[blockIdx.x] = bsum;
        __threadfence();
        const uint32_t prev = atomicAdd(&a.st->ticket, 1u);
        last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    double s = 0.0;
    for (uint32_t b = threadIdx.x; b < gridDim.x; b += kBlock) s += a.partials[b];
    s = block_sum(s, lds);
    if (threadIdx.x != 0) return;

    DevState* st = a.st;
    st->ticket = 0;
    st->sumsq = s;
    st->norm = sqrt(s);
    if (a.probe) return;
    const int found = !(s <= 1.7976931348623157e308);  // inf or NaN
    const int skip = a.scaler_on && found;
    float coef = 1.0f;
    if (a.max_norm > 0.0) {
        double cd = a.max_norm / (st->norm + 1e-6);
        if (cd > 1.0) cd = 1.0;
        coef = (float)cd;
    }
    st->found_inf = found;
    st->skip = skip;
    st->inv_scale = inv;
    st->clip_coef = coef;
    if (a.scaler_on) {
        if (!skip) st->t += 1;
        if (a.want_bias) {
            const uint64_t t = st->t;
            st->bias1 = (t >= 1 && t <= a.bias_len) ? a.bias_tab[2 * (t - 1)] : 1.0f;
            st->bias2 = (t >= 1 && t <= a.bias_len) ? a.bias_tab[2 * (t - 1) + 1] : 1.0f;
        }
        // torch _amp_update_scale_ semantics
        if (found) {
            st->scale = (float)((double)st->scale * a.backoff_factor);
            st->growth_tracker = 0;
        } else {
            const int32_t ok = st->growth_tracker + 1;
            if (ok == a.growth_interval) {
                const float ns = (float)((double)st->scale * a.growth_factor);
                if (ns - ns == 0.0f) st->scale = ns;  // finite
                st->growth_tracker = 0;
            } else {
                st->growth_tracker = ok;
            }
        }
    }
    __threadfence();
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

template <typename GradT, bool kMixed>
__global__ __launch_bounds__(kBlock) void adam_kernel(const GradT* __restrict__ grad,
                                                      float* __restrict__ master,
                                                      float* __restrict__ exp_avg,
                                                      float* __restrict__ exp_avg_sq,
                                                      uint16_t* __restrict__ param16,
                                                      AdamArgs a) {
    Coefs k{1.0f, 1.0f, a.bias1, a.bias2};
    if (a.st) {
        if ((a.flags & kCheckSkip) && a.st->skip) return;
        k.inv = a.st->inv_scale;
        k.clip = a.st->clip_coef;
        if (a.flags & kDevBias) {
            k.bias1 = a.st->bias1;
            k.bias2 = a.st->bias2;
        }
    }
    const bool use_inv = a.flags & kUseInv, use_clip = a.flags & kUseClip;
    for (uint32_t c = blockIdx.x; c < a.nchunks; c += gridDim.x) {
        const Chunk ch = a.chunks[c];
        const bool decay = (ch.meta & kChunkDecay) && (a.flags & kWdOn);
        const uint64_t end = ch.begin + ch.count;
        for (uint64_t i = ch.begin + (uint64_t)threadIdx.x * kVec; i < end;
             i += (uint64_t)kBlock * kVec) {
            const f32x4 g = ld_grad4(grad, i);
            f32x4 p = ld4(master + i);
            f32x4 m = ld4(exp_avg + i);
            f32x4 v = ld4(exp_avg_sq + i);
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                float pj = p[j], mj = m[j], vj = v[j];
                adam_elem(pj, g[j], mj, vj, a, k, use_inv, use_clip, decay);
                p[j] = pj;
                m[j] = mj;
                v[j] = vj;
            }
            if (i + kVec <= end) {
                st4(master + i, p);
                st4(exp_avg + i, m);
                st4(exp_avg_sq + i, v);
                if (kMixed) st_bf16x4(param16, i, p);
            } else {
                const int n = (int)(end - i);
                st4_partial(master + i, p, n);
                st4_partial(exp_avg + i, m, n);
                st4_partial(exp_avg_sq + i, v, n);
                if (kMixed) st_bf16x4_partial(param16 + i, p, n);
            }
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

template <typename GradT, bool kMixed>
__global__ __launch_bounds__(kBlock) void sgd_kernel(const GradT* __restrict__ grad,
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
    for (uint32_t c = blockIdx.x; c < a.nchunks; c += gridDim.x) {
        const Chunk ch = a.chunks[c];
        const bool decay = (ch.meta & kChunkDecay) && (a.flags & kWdOn);
        const bool first = mom_on && a.mom_init[ch.meta >> 8] == 0u;
        const uint64_t end = ch.begin + ch.count;
        for (uint64_t i = ch.begin + (uint64_t)threadIdx.x * kVec; i < end;
             i += (uint64_t)kBlock * kVec) {
            f32x4 g = ld_grad4(grad, i);
            f32x4 p = ld4(master + i);
            f32x4 b = {0.0f, 0.0f, 0.0f, 0.0f};
            if (mom_on && !first) b = ld4(momentum + i);
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                float gj = g[j];
                if (use_inv) gj = gj * inv;
                if (use_clip) gj = gj * clip;
                if (decay) gj = gj + a.wd * p[j];
                if (mom_on) {
                    const float bj = first ? gj : a.mu * b[j] + a.omd * gj;
                    b[j] = bj;
                    gj = nesterov ? gj + a.mu * bj : bj;
                }
                const float update = gj * a.lr;  // autograd/dynamic/optim.hpp:24
                p[j] = p[j] - update;             // autograd/dynamic/optim.hpp:25
            }
            if (i + kVec <= end) {
                st4(master + i, p);
                if (mom_on) st4(momentum + i, b);
                if (kMixed) st_bf16x4(param16, i, p);
            } else {
                const int n = (int)(end - i);
                st4_partial(master + i, p, n);
                if (mom_on) st4_partial(momentum + i, b, n);
                if (kMixed) st_bf16x4_partial(param16 + i, p, n);
            }
        }
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
// small elementwise helpers
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void fill_zero_kernel(uint32_t* p, uint64_t n_words) {
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n_words;
         i += (uint64_t)gridDim.x * kBlock)
        p[i] = 0u;
}

__global__ __launch_bounds__(kBlock) void master_to_bf16_kernel(const float* src, uint16_t* dst,
                                                                uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * kBlock)
        dst[i] = (uint16_t)bf16_rne(src[i]);
}

__global__ __launch_bounds__(kBlock) void bf16_to_master_kernel(const uint16_t* src, float* dst,
                                                                uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * kBlock)
        dst[i] = __uint_as_float((uint32_t)src[i] << 16);
}

}  // namespace ttp
