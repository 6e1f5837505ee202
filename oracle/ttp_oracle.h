/*
 * ttp_oracle.h — CPU restatement of csirak/tt-perf's optimizer step, used ONLY as the
 * checker by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.  It is test
 * infrastructure: no product code links, loads or calls it.
 *
 * What it restates (reference file:line):
 *   Adam op order ............ py/optim.py:49-87 (t += 1; bias1/bias2 in host double; m, v,
 *                              m_hat, v_hat, denom, step, p as separate fp32-rounded ops)
 *   SGD ...................... autograd/dynamic/optim.hpp:21-27, autograd/traced/ops.hpp:132-134,
 *                              py/optim.py:13-22 (p - lr*g: multiply, then subtract; no FMA)
 *   None-grad skip ........... py/optim.py:56-57, autograd/dynamic/optim.hpp:23
 *   zero_grad ................ py/optim.py:89-92, autograd/dynamic/optim.hpp:30-34
 * What the reference lacks and is restated from library semantics (torch 2.x):
 *   decoupled weight decay (torch.optim.AdamW: p *= 1 - lr*wd before the Adam update),
 *   L2 weight decay and momentum/dampening/nesterov (torch.optim.SGD, torch.optim.Adam),
 *   loss scaling (torch.amp.GradScaler: unscale by 1/scale, skip on inf/nan, update scale),
 *   global-norm clipping (torch.nn.utils.clip_grad_norm_: coef = max/(norm+1e-6) <= 1),
 *   bf16 round-to-nearest-even of the fp32 master (c10::BFloat16 conversion).
 *
 * Pins (each checked in tests/): reference known answers (autograd/tests/test_sgd.cpp:45-70,
 * verify/verify_autograd.py:119-162, tests/adam_optimizer.py:15-92), torch library goldens in
 * tests/golden/, an exhaustive 2^32 bf16 rounding check against an independent method,
 * brute-force fp64/fsum norms, and the closed-form loss-scale sequence.
 *
 * Arithmetic: fp32 IEEE, round-to-nearest, no contraction (built with -ffp-contract=off),
 * no flush-to-zero; norms accumulate in fp64 in a fixed blocked order (deterministic for any
 * thread count).
 */
#ifndef TTP_ORACLE_H
#define TTP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_MODE_FP32 0
#define ORC_MODE_MIXED 1
/* bf16 weights (param) and bf16 grads only, the reference C++ autograd's BFLOAT16 tensors
 * (autograd/dynamic/autograd.hpp:72): master, moments and momentum are not used; the only
 * step is plain SGD with each ttnn op rounded to bf16 (see orc_sgd_step) */
#define ORC_MODE_BF16 2
#define ORC_DECAY 1u

typedef struct orc_tensor {
    uint64_t offset;
    uint64_t numel;
    uint32_t flags;    /* ORC_DECAY */
    int32_t has_grad;  /* 0 = grad is None */
} orc_tensor;

typedef struct orc_store {
    int32_t mode;
    uint32_t n_tensors;
    const orc_tensor* tensors;
    uint64_t total;        /* elements per flat buffer */
    void* param;           /* float* (FP32) or uint16_t* bf16 bits (MIXED, BF16) */
    void* grad;            /* float* (FP32) or uint16_t* bf16 bits (MIXED, BF16) */
    float* master;         /* == param in FP32 mode */
    float* exp_avg;
    float* exp_avg_sq;
    float* momentum;
    uint8_t* mom_init;     /* per tensor: momentum buffer initialised */
    int32_t scaler_enabled;
    int32_t growth_interval;
    double growth_factor;
    double backoff_factor;
    float scale;
    int32_t growth_tracker;
    uint64_t t;            /* applied steps */
    int32_t nthreads;
    int32_t pending;       /* steps that deferred the scale update since the last one:
                              ORC_PENDING_STEP once one ran, | ORC_PENDING_INF on overflow */
} orc_store;

/* step flag: with loss scaling on, skip this step's own update on overflow but leave the
 * scale update to the iteration's last step or orc_scaler_update_pending (torch's
 * GradScaler.step for one of several optimizers, then one GradScaler.update) */
#define ORC_STEP_DEFER_SCALE 2
#define ORC_PENDING_INF 1
#define ORC_PENDING_STEP 2

typedef struct orc_adam_hp {
    double lr, beta1, beta2, eps, weight_decay;
    int32_t decoupled, flags;
    double max_grad_norm;
} orc_adam_hp;

typedef struct orc_sgd_hp {
    double lr, momentum, dampening, weight_decay;
    int32_t nesterov, flags;
    double max_grad_norm;
} orc_sgd_hp;

typedef struct orc_report {
    int32_t found_inf;
    int32_t skipped;
    double grad_norm;
    float clip_coef;
    float scale;
    int32_t growth_tracker;
    int32_t reserved;
    uint64_t step;
} orc_report;

/* bf16 */
uint16_t orc_bf16_rne(float x);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_array(const float* x, uint16_t* out, uint64_t n);
void orc_bf16_to_f32_array(const uint16_t* x, float* out, uint64_t n);
/* Compares orc_bf16_rne against an independent nearest-even search for every fp32 bit
 * pattern in [lo, hi); returns the number of disagreements. */
uint64_t orc_bf16_check_range(uint64_t lo, uint64_t hi, int nthreads);

/* host-side constant rounding shared by both optimizers */
float orc_bias_correction(double beta, uint64_t t);
float orc_clip_coef(double norm, double max_norm);
void orc_scaler_update(float* scale, int32_t* tracker, int found_inf, double growth_factor,
                       double backoff_factor, int32_t growth_interval);
/* GradScaler.update after deferred steps: the scale update over their pending overflow;
 * nothing if no step deferred it since the last update */
void orc_scaler_update_pending(orc_store* s);

/* layout: offsets of n tensors, each aligned up to `align` elements; returns total */
uint64_t orc_layout(const uint64_t* numel, uint32_t n, uint64_t align, uint64_t* offsets);

/* norm pass: sum of squares (fp64) of the unscaled grads of tensors with has_grad,
 * and whether any of them is non-finite. */
double orc_grad_sumsq(const orc_store* s, float inv_scale, int32_t* found_inf);

/* Value::accumulate_grad (autograd/dynamic/autograd.hpp:78-83, py/engine.py:149-156): the
 * tensor's grad becomes src when it has none, else grad + src (fp32 add, one rounding to the
 * grad type); src is float (src_bf16 = 0) or bf16 bits (src_bf16 = 1). */
void orc_accumulate_grad(orc_store* s, uint32_t index, const void* src, int src_bf16);

/* one optimizer step over the store (fused: one pass per element).  A BF16 store takes plain
 * SGD only (momentum and weight decay 0; Adam returns -1): param = RNE_bf16(param -
 * RNE_bf16(g * lr)), the two bf16 roundings of `subtract(data, multiply(grad, lr))`. */
int orc_adam_step(orc_store* s, const orc_adam_hp* hp, orc_report* rep);
int orc_sgd_step(orc_store* s, const orc_sgd_hp* hp, orc_report* rep);
/* the same Adam step executed op by op as py/optim.py:76-86 issues it: every op is a
 * separate full pass over the tensor into a freshly allocated temporary */
int orc_adam_step_opbyop(orc_store* s, const orc_adam_hp* hp, orc_report* rep);

#ifdef __cplusplus
}
#endif

#endif
