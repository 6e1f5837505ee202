/*
 * ttperf.h — C ABI of libttperf_hip, the MI355X (gfx950) optimizer-step engine.
 *
 * One context owns a flat parameter store on one GPU: every tensor of a model is a
 * {offset, numel, flags} view into flat HBM buffers (param, grad, fp32 master, exp_avg,
 * exp_avg_sq, momentum); the optimizer-private fp32 state is interleaved in records of
 * 64-element slots (see ttp_buffer_layout).  A step over all tensors is one multi-tensor update
 * launch (split in several only beyond 2^32 work-items), plus, when clipping or loss scaling
 * is on, a grad-norm/inf-check pass (one launch, two above 256 MiB of gradients) and a
 * one-block finalize.
 *
 * Reference interfaces each group of entry points replaces (csirak/tt-perf):
 *   ttp_create / ttp_destroy / ttp_tensor_*  — per-parameter storage owned by
 *       autograd::Value (autograd/dynamic/autograd.hpp:38-84), static_autograd::Value
 *       (autograd/static/value.hpp:27-48) and the per-layer tensors of the traced layers
 *       (autograd/traced/nn.hpp:54-69); parameters() lists (autograd/dynamic/nn.hpp:35,52-54).
 *   ttp_set_has_grad / ttp_zero_grad         — `grad = std::nullopt` / `p.grad = None`
 *       (autograd/dynamic/optim.hpp:30-34, py/optim.py:89-92, py/engine.py:141-142) and
 *       static zero_grad (autograd/static/nn.hpp:98-101).
 *   ttp_adam_step                            — Adam.step (py/optim.py:49-87), extended with
 *       decoupled weight decay, fp32 master weights, loss scaling and global-norm clipping.
 *   ttp_sgd_step                             — SGD::step (autograd/dynamic/optim.hpp:21-27),
 *       SGD.step (py/optim.py:13-22), TracedSGD::step / sgd_update
 *       (autograd/traced/optim.hpp:22-26, autograd/traced/ops.hpp:132-134) and every
 *       per-module sgd_step (autograd/traced/nn.hpp:93-96,272-275,317-321), extended with
 *       momentum, dampening, nesterov and L2 weight decay.
 *   ttp_last_error                           — the ValueError / std::exception paths
 *       (py/optim.py:9-16,33-41,54-55); no exception crosses this ABI.
 *
 * Conventions: every function returns TTP_OK (0) or a negative TTP_ERR_* code and leaves
 * a message for ttp_last_error() (thread-local).  All work is ordered on the context's
 * stream and is asynchronous, except ttp_download to host memory, ttp_sync, ttp_scaler_get,
 * ttp_get_step, ttp_grad_norm and any step call given a non-NULL report, which wait for
 * the stream.  A context is used by one host thread at a time.
 *
 * Environment, read at ttp_create (tuning only):
 *   TTP_UPD_BLOCKS_PER_CU  resident update blocks per CU of the four-element update (MIXED SGD
 *                          with momentum up to 256 MiB of gradients; default 4; 0: no cap); every other
 *                          update runs uncapped.  Results do not depend on it.
 *   TTP_NORM_GRID          blocks of each gradient-norm launch (default 8 x CUs, at most
 *                          65536; the pass is two launches above 256 MiB of gradients).  It
 *                          fixes the fp64 summation order of the norm: deterministic for a
 *                          given value, last bits may differ between values.
 *   TTP_LANE_LAUNCH_BLOCKS most blocks per launch of the lane-form updates (all but MIXED SGD
 *                          with momentum up to 256 MiB of gradients; default: what 2^32 - 1 work-items
 *                          allow); a larger update is split into several launches.  Results
 *                          do not depend on it.
 */
#ifndef TTPERF_TTPERF_H
#define TTPERF_TTPERF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version, returned by ttp_abi_version().  Changes:
 *   3  TTP_MODE_BF16 (the reference's own storage: bf16 weights and gradients, no fp32
 *      state; plain SGD with its two bf16 roundings).  Nothing else changes.
 *   2  TTP_STORE_SGD (the SGD layout of a MIXED store, OR'd into ttp_create's mode);
 *      TTP_ACCUM_SUMSQ (ttp_accumulate_grad also stores the tensor's gradient sum);
 *      ttp_accumulate_grad_multi (several tensors' gradients in one launch);
 *      TTP_ZERO_NO_FILL (ttp_zero_grad[_subset] to None without the fill).
 *      Behaviour changes of existing entry points, which a caller written against version 1
 *      must follow: ttp_zero_grad_subset with set_to_none = 0 leaves the has-grad flags as
 *      they were (version 1 marked the listed tensors as having a grad); a captured
 *      ttp_accumulate_grad is refused unless an earlier call of the same capture set that
 *      tensor's has-grad flag.
 *   1  first version. */
#define TTP_ABI_VERSION 3

/* ---- status codes ---------------------------------------------------------------- */
#define TTP_OK 0
#define TTP_ERR_INVALID (-1)   /* bad argument: the cases py/optim.py raises ValueError for */
#define TTP_ERR_NO_DEVICE (-2) /* no HIP device, or device index out of range            */
#define TTP_ERR_HIP (-3)       /* a HIP runtime call failed                               */
#define TTP_ERR_OOM (-4)       /* device or pinned-host allocation failed                 */
#define TTP_ERR_STATE (-5)     /* call not valid in the context's current state/mode      */
#define TTP_ERR_RANGE (-6)     /* tensor index or element count out of range              */

/* ---- precision modes -------------------------------------------------------------- */
#define TTP_MODE_FP32 0  /* fp32 params/grads; the param buffer is the master copy    */
#define TTP_MODE_MIXED 1 /* bf16 params/grads + fp32 master; bf16 param = RNE(master) */
/* TTP_MODE_BF16: bf16 weights (PARAM) and bf16 gradients (GRAD) and nothing else, the storage
 * of the reference's C++ autograd, whose parameters and gradients are BFLOAT16 ttnn tensors
 * (autograd/dynamic/autograd.hpp:72,88-99, autograd/traced/nn.hpp:24-35).  No fp32 master,
 * moments or momentum: 4 B/param in all.  Its one update is the reference's plain SGD,
 * `data = subtract(data, multiply(grad, lr))` (autograd/dynamic/optim.hpp:21-27,
 * autograd/traced/ops.hpp:132-134, autograd/traced/nn.hpp:93-96), with the rounding of each
 * ttnn op to bf16: update = RNE_bf16(g * lr), param = RNE_bf16(param - update), each product
 * and difference formed in fp32 first (6 B/param moved per step, against 12 for MIXED SGD).
 * Loss scaling and clipping apply to g before the product, as in the other modes.  Adam
 * (every entry point), and SGD with momentum, dampening, nesterov or weight decay, need fp32
 * state and are refused (TTP_ERR_INVALID, nothing changed); so are MASTER, EXP_AVG,
 * EXP_AVG_SQ and MOMENTUM in ttp_buffer_ptr, ttp_buffer_layout, ttp_upload and ttp_download,
 * and TTP_STORE_SGD.  A checkpoint holds the weights in its master buffer (each bf16 value
 * widened to fp32, exactly), and loading it rounds them back. */
#define TTP_MODE_BF16 2

/* ---- store layout flags, OR'd into ttp_create's mode -------------------------------- */
/* TTP_STORE_SGD: the SGD layout of a MIXED store.  By default a MIXED store keeps each
 * 64-element group's fp32 master, m and v side by side in one [master|m|v] record (Adam reads
 * and writes all three in one pass).  A store stepped only by SGD never touches m and v, and
 * its update would read the master as one 256-byte slot of every 768-byte record.  With this
 * flag the fp32 master is one contiguous buffer and no m / v exist (4 B/param instead of
 * 12 B/param of optimizer state), which lets the SGD update stream its four buffers (bf16
 * grad, master read and write, bf16 weights) like a copy.  The first Adam step, or any call
 * that asks for EXP_AVG / EXP_AVG_SQ (ttp_buffer_layout, ttp_upload, ttp_download,
 * ttp_load_state of a file holding them), converts the store to the default layout once: it
 * allocates the records, moves the master into them (values unchanged) and frees the
 * contiguous copy, waiting for the queued work.  A call that is refused for any other reason
 * converts nothing (the conversion comes after its checks).  That conversion is refused
 * (TTP_ERR_STATE, nothing changed) while capturing, while graphs of the context are alive
 * (they hold the old master's address) and by ttp_adam_step_noalloc.  A master pointer from
 * ttp_buffer_ptr is invalid after it.  ttp_mode reports the precision mode only; the layout
 * shows in ttp_buffer_layout (MASTER: stride 64 in the SGD layout, 192 in the default one).
 * In FP32 mode the master is the contiguous model-facing weight and m, v are allocated on
 * first Adam use anyway, so the flag changes nothing there.  Checkpoint files do not depend
 * on the layout.  No counterpart in the reference, whose SGD updates each parameter's own
 * tensor (autograd/dynamic/optim.hpp:21-27, autograd/traced/nn.hpp:93-96). */
#define TTP_STORE_SGD 0x100

/* ---- buffers of the flat store ---------------------------------------------------- */
#define TTP_BUF_PARAM 0      /* model-facing weights: fp32 (FP32) or bf16 (MIXED, BF16) */
#define TTP_BUF_GRAD 1       /* gradients: fp32 (FP32) or bf16 (MIXED, BF16)            */
#define TTP_BUF_MASTER 2     /* fp32 master weights (same memory as PARAM in FP32 mode) */
#define TTP_BUF_EXP_AVG 3    /* Adam first moment m, fp32                               */
#define TTP_BUF_EXP_AVG_SQ 4 /* Adam second moment v, fp32                              */
#define TTP_BUF_MOMENTUM 5   /* SGD momentum buffer, fp32                               */

/* Pass as `index` to address the whole flat buffer (in layout order, padding included). */
#define TTP_ALL_TENSORS 0xFFFFFFFFu

/* ---- per-tensor flags -------------------------------------------------------------- */
#define TTP_TENSOR_DECAY 1u /* weight decay applies to this tensor (e.g. 2-D weights) */

/* Memory kinds for upload/download. */
#define TTP_HOST 0
#define TTP_DEVICE 1

/* Element types of incoming gradients (ttp_accumulate_grad). */
#define TTP_DTYPE_F32 0
#define TTP_DTYPE_BF16 1
/* OR'd into ttp_accumulate_grad's src_dtype: also store the tensor's sum of squares of its
 * resulting gradients for a TTP_STEP_TENSOR_SUMS step (see ttp_accumulate_grad). */
#define TTP_ACCUM_SUMSQ 0x100

typedef struct ttp_ctx ttp_ctx;
typedef struct ttp_graph ttp_graph;

typedef struct ttp_tensor_desc {
    uint64_t numel;  /* elements; 0 is allowed (the tensor is then never touched); the
                        64-element-padded sizes of a table total at most 2^40; at most
                        2^24 - 1 tensors */
    uint32_t flags;  /* TTP_TENSOR_* */
    uint32_t reserved; /* must be 0 */
} ttp_tensor_desc;

/* Adam / AdamW.  Hyperparameters are host doubles (Python floats in py/optim.py:31-47);
 * the engine rounds lr, betas, 1-beta, eps and the bias corrections to fp32 exactly as
 * py/optim.py's full_like(fill_value=...) does. */
typedef struct ttp_adam_hparams {
    double lr;            /* > 0 */
    double beta1, beta2;  /* in (0, 1) */
    double eps;           /* > 0 */
    double weight_decay;  /* >= 0; applied only to TTP_TENSOR_DECAY tensors */
    int32_t decoupled;    /* 1: AdamW (p *= 1 - lr*wd first); 0: L2 (g += wd*p)   */
    int32_t flags;        /* TTP_STEP_* (0: none) */
    double max_grad_norm; /* > 0: clip the global L2 norm to this; <= 0: no clipping */
} ttp_adam_hparams;

/* SGD with optional momentum, dampening, nesterov and L2 weight decay.
 * momentum = dampening = weight_decay = 0 is exactly `p - lr*g` (two roundings, no FMA)
 * as autograd/dynamic/optim.hpp:24-25. */
typedef struct ttp_sgd_hparams {
    double lr;            /* > 0 */
    double momentum;      /* >= 0 */
    double dampening;     /* any; torch semantics */
    double weight_decay;  /* >= 0 */
    int32_t nesterov;     /* requires momentum > 0 and dampening == 0 */
    int32_t flags;        /* TTP_STEP_* (0: none) */
    double max_grad_norm; /* > 0: clip; <= 0: off */
} ttp_sgd_hparams;

/* Step flags.
 * TTP_STEP_TENSOR_SUMS: take the gradient norm (and the inf/NaN check) from the per-tensor
 *   sums of squares that ttp_grad_sumsq_tensors stored for the step's tensors, instead of a
 *   norm pass over all their gradients.  Every tensor the step updates needs a current sum:
 *   one computed after its last gradient write through this ABI (upload, accumulate, zero,
 *   set_has_grad), after the last step that updated that tensor, and after the last change
 *   of the loss scale (a step that updates it, ttp_scaler_update, configure, set or a loaded
 *   state); otherwise the step fails with TTP_ERR_STATE before any work is queued.
 *   Gradients written through a device pointer after their sum was taken are the caller's
 *   to avoid.  The norm is the same sum of the same squares, added
 *   in another order: it can differ from the norm pass's in the last bits.
 *   Captured calls count when their graph is launched, not when they are captured: each
 *   launch consumes or renews sums as its captured steps and sums calls do eagerly, and a
 *   graph whose step reads sums taken before the capture is refused at launch (TTP_ERR_STATE,
 *   nothing queued) unless those sums are current. */
#define TTP_STEP_TENSOR_SUMS 1
/* TTP_STEP_DEFER_SCALE: with loss scaling on, the step unscales, checks its own tensors for
 *   inf/NaN and skips its own update on overflow, but leaves the loss scale and the growth
 *   tracker as they are and notes the overflow instead.  This is torch's GradScaler.step for
 *   one of several optimizers of an iteration: give it to every step of the iteration but
 *   the last, or to all of them and then call ttp_scaler_update.  The next step without the
 *   flag (or ttp_scaler_update) updates the scale once, backing off if that step or any
 *   deferred step since the last update saw an overflow (GradScaler.update).  Without the
 *   flag every step updates the scale itself, which is right for one optimizer per store:
 *   several optimizers over disjoint tensor groups of one store that each update it would
 *   unscale later groups by a moved scale and advance the tracker once per optimizer.
 *   Ignored while loss scaling is off. */
#define TTP_STEP_DEFER_SCALE 2

/* Dynamic loss scaling (torch.amp.GradScaler semantics).  While enabled, every step
 * unscales the gradients by 1/scale, skips the whole update when any gradient is
 * non-finite (params, moments and the step count stay bit-unchanged), and then updates
 * the scale: x backoff on overflow, x growth after growth_interval clean steps. */
typedef struct ttp_scaler_config {
    int32_t enabled;
    int32_t growth_interval; /* > 0 */
    double init_scale;       /* > 0 */
    double growth_factor;    /* > 1 */
    double backoff_factor;   /* in (0, 1) */
} ttp_scaler_config;

typedef struct ttp_step_report {
    int32_t found_inf;      /* non-finite gradient seen (only checked when a norm pass ran) */
    int32_t skipped;        /* the update was skipped (loss scaling on and found_inf)       */
    double grad_norm;       /* global L2 norm of the unscaled gradients; NaN if not computed */
    float clip_coef;        /* multiplier applied to the gradients (1 when not clipping)    */
    float scale;            /* loss scale after this step's update                          */
    int32_t growth_tracker; /* clean steps since the last scale change                      */
    int32_t reserved;
    uint64_t step;          /* optimizer steps applied so far (bias-correction t)           */
} ttp_step_report;

/* ---- context lifetime --------------------------------------------------------------- */
int ttp_device_count(int* count);
/* mode: TTP_MODE_FP32, TTP_MODE_MIXED (optionally | TTP_STORE_SGD) or TTP_MODE_BF16. */
int ttp_create(int device, const ttp_tensor_desc* descs, uint32_t n_tensors, int mode,
               ttp_ctx** out);
int ttp_destroy(ttp_ctx* ctx);
/* Order all further work on an existing HIP stream (hipStream_t passed as void*; NULL is
 * the legacy default stream, e.g. torch's default stream).  Waits for work already queued.
 * The stream stays the caller's: it must remain valid until the context moves to another
 * stream (ttp_set_stream, ttp_reset_stream) or is destroyed, since ttp_destroy and
 * ttp_graph_destroy wait on it. */
int ttp_set_stream(ttp_ctx* ctx, void* hip_stream);
/* Back to the context's own (non-blocking) stream. */
int ttp_reset_stream(ttp_ctx* ctx);
int ttp_sync(ttp_ctx* ctx);

/* ---- layout ------------------------------------------------------------------------- */
int ttp_num_tensors(const ttp_ctx* ctx, uint32_t* n);
int ttp_mode(const ttp_ctx* ctx, int* mode);
/* total elements of each flat buffer (tensor footprints are 64-element aligned) */
int ttp_flat_numel(const ttp_ctx* ctx, uint64_t* total);
int ttp_tensor_info(const ttp_ctx* ctx, uint32_t index, uint64_t* offset, uint64_t* numel,
                    uint32_t* flags);
/* Device address of buffer `which` for tensor `index` (or the flat base for
 * TTP_ALL_TENSORS), for the buffers stored contiguously: PARAM, GRAD and MOMENTUM always,
 * MASTER in FP32 mode (where it is PARAM) and in a MIXED store's SGD layout.  The
 * optimizer-private fp32 state is otherwise kept in
 * interleaved records (MIXED: master, m and v of each 64-element group side by side; FP32:
 * m and v), for which this returns TTP_ERR_STATE; use ttp_buffer_layout, or ttp_upload /
 * ttp_download, which convert.  Moment/momentum buffers are allocated on first use; asking
 * for one allocates it (zero-filled).  Replaces direct access to a Value's data/grad
 * tensors (autograd/dynamic/autograd.hpp:38-84, autograd/static/value.hpp:27-48). */
int ttp_buffer_ptr(ttp_ctx* ctx, int which, uint32_t index, void** ptr);
/* Addressing of any buffer: flat element e of `which` sits at
 *   base + (e / group) * stride + e % group   (in elements of the buffer's type).
 * group == stride for a contiguous buffer; MIXED-mode MASTER/EXP_AVG/EXP_AVG_SQ have
 * group 64, stride 192 (slots 0, 1, 2 of one record), except MASTER in the SGD layout
 * (TTP_STORE_SGD: contiguous); FP32-mode EXP_AVG/EXP_AVG_SQ group 64, stride 128.  Each
 * tensor starts on a record boundary.  Allocates like ttp_buffer_ptr.
 * No counterpart in the reference, whose optimizer state is private per-tensor ttnn
 * tensors (py/optim.py:58-71). */
int ttp_buffer_layout(ttp_ctx* ctx, int which, void** base, uint32_t* group, uint32_t* stride);

/* ---- data movement ------------------------------------------------------------------ */
/* Copy n elements (exactly the tensor's numel, or the flat total for TTP_ALL_TENSORS)
 * in the buffer's element type.  Uploading GRAD marks the tensor(s) as having a grad.
 * MIXED mode keeps the two weight copies consistent: uploading MASTER also writes
 * PARAM = RNE_bf16(MASTER), uploading PARAM also writes MASTER = float(PARAM).
 * A TTP_DEVICE pointer (here and in ttp_accumulate_grad) must be device or managed memory of
 * the context's device, with all n elements inside one allocation: other pointers are refused
 * with TTP_ERR_INVALID, a buffer too short with TTP_ERR_RANGE, before any work is queued. */
int ttp_upload(ttp_ctx* ctx, int which, uint32_t index, const void* src, uint64_t n,
               int src_kind);
int ttp_download(ttp_ctx* ctx, int which, uint32_t index, void* dst, uint64_t n,
                 int dst_kind);

/* ---- gradients ---------------------------------------------------------------------- */
/* has_grad = 0 is `grad = None`: the tensor is skipped by every step (its param and
 * optimizer state are not touched) and left out of the grad norm. */
int ttp_set_has_grad(ttp_ctx* ctx, uint32_t index, int has_grad);
int ttp_get_has_grad(const ttp_ctx* ctx, uint32_t index, int* has_grad);
/* Zero the whole grad buffer; set_to_none = 1 also clears every has_grad flag.
 * One fill over the flat buffer replaces the per-tensor zeros_like allocations of
 * autograd/static/nn.hpp:98-101 and the nullopt loop of autograd/dynamic/optim.hpp:30-34.
 * set_to_none = 1 | TTP_ZERO_NO_FILL clears the flags without the fill, as the reference's
 * `grad = std::nullopt` touches no memory.  The gradients then keep their old contents until
 * written.  Nothing of the library reads them: the next accumulate into a tensor assigns its
 * whole gradient, and steps, norms and sums skip tensors without a grad.  A flat download or
 * a view shows the old values, and a caller that writes gradients through ttp_buffer_ptr and
 * marks them with ttp_set_has_grad must write every element.  For a backward that delivers
 * every gradient by accumulate, it saves one write of the whole buffer per iteration.
 * Without set_to_none it is refused (TTP_ERR_INVALID).  The same holds for
 * ttp_zero_grad_subset. */
#define TTP_ZERO_NO_FILL 0x100
int ttp_zero_grad(ttp_ctx* ctx, int set_to_none);
/* A module's zero_grad: the listed tensors' grads (each index at most once) become zeros
 * (set_to_none = 0: the static layers' zeros_like, autograd/static/nn.hpp:98-101, 183-186)
 * or become None (set_to_none = 1).  As with ttp_zero_grad, set_to_none = 0 leaves the
 * has-grad flags as they are (a tensor without a grad stays without one, as in torch's
 * zero_grad(set_to_none=False)); a caller whose zeroed grads count as present, like the
 * static layers, marks them with ttp_set_has_grad.  One launch over the listed tensors. */
int ttp_zero_grad_subset(ttp_ctx* ctx, const uint32_t* indices, uint32_t n_indices,
                         int set_to_none);
/* Value::accumulate_grad (autograd/dynamic/autograd.hpp:78-83; static_autograd::Value,
 * autograd/static/value.hpp:39-47) on the flat grad buffer: when tensor `index` has no grad,
 * its grad becomes the incoming gradient; otherwise grad = grad + incoming, added in fp32 and
 * rounded once (round-to-nearest-even) to the grad buffer's type.  `src` holds exactly numel
 * values of `src_dtype` (TTP_DTYPE_*) in host or device memory (`src_kind`).  Marks the
 * tensor as having a grad.  Stream-ordered; a host source is consumed before returning.
 * Captured, the call's choice between assigning and adding is fixed at capture time, so it
 * is refused (TTP_ERR_STATE) unless an earlier call of the same capture set that tensor's
 * has-grad flag (ttp_zero_grad[_subset] with set_to_none = 1, ttp_set_has_grad, a gradient
 * upload or an accumulate): every launch then finds the flag as the capture did.
 * src_dtype | TTP_ACCUM_SUMSQ: the same launch also computes the sum of squares of the
 * tensor's resulting gradients (unscaled by the current loss scale, as
 * ttp_grad_sumsq_tensors does, tile for tile in the same order, so bit-identical to it) and
 * stores it as the tensor's current sum: a backward that accumulates every parameter's last
 * gradient this way leaves a TTP_STEP_TENSOR_SUMS step nothing to read twice (no norm pass, no
 * bucket call).  It adds no launch and no memory traffic to the accumulate: the launch writes
 * one partial per wave of each 16 KiB tile into a store-wide array (32 B per 16 KiB of
 * gradients, allocated with the store), and the next step from sums combines the pending
 * partials of all its tensors in one launch.  The loss scale must not change between this call and the step (as
 * for any sum).  A tensor of 2^24 or more 16 KiB tiles of gradients is refused with
 * TTP_ERR_RANGE. */
int ttp_accumulate_grad(ttp_ctx* ctx, uint32_t index, const void* src, uint64_t n,
                        int src_dtype, int src_kind);
/* Several tensors' incoming gradients in one launch, as a backward hands over a bucket of
 * them: for k < n, tensor indices[k] receives srcs[k] (its numel values of src_dtype, in
 * device memory) exactly as ttp_accumulate_grad(ctx, indices[k], srcs[k], numel, src_dtype,
 * TTP_DEVICE) would, bit for bit, TTP_ACCUM_SUMSQ included; same capture rule.  Each index
 * at most once, at most TTP_ACCUM_MULTI_MAX per call, and fewer than 2^24 tiles of 16 KiB of
 * gradients in all.  The call's table travels in the kernel's arguments: it allocates and
 * copies nothing.  A refused call changes nothing.  It extends Value::accumulate_grad
 * (autograd/dynamic/autograd.hpp:78-83) to a bucket: one launch instead of n, which for a
 * backward's many small tensors is mostly launch latency saved. */
#define TTP_ACCUM_MULTI_MAX 64
int ttp_accumulate_grad_multi(ttp_ctx* ctx, const uint32_t* indices, const void* const* srcs,
                              uint32_t n, int src_dtype);

/* ---- optimizer steps ------------------------------------------------------------------ */
int ttp_adam_step(ttp_ctx* ctx, const ttp_adam_hparams* hp, ttp_step_report* report);
int ttp_sgd_step(ttp_ctx* ctx, const ttp_sgd_hparams* hp, ttp_step_report* report);
/* The same steps restricted to the listed tensors (each index at most once): what one
 * module's sgd_step(lr) touches (autograd/traced/nn.hpp:93-96,272-275,317-321,
 * autograd/static/nn.hpp:92-95) or one optimizer's parameter list (py/optim.py:7,31).
 * Tensors outside the list, or without a grad, are not touched; the grad norm used for
 * clipping and the inf check cover the listed tensors only.  The step count and loss
 * scale are per context. */
int ttp_adam_step_subset(ttp_ctx* ctx, const ttp_adam_hparams* hp, const uint32_t* indices,
                         uint32_t n_indices, ttp_step_report* report);
int ttp_sgd_step_subset(ttp_ctx* ctx, const ttp_sgd_hparams* hp, const uint32_t* indices,
                        uint32_t n_indices, ttp_step_report* report);
/* The Adam step of ttp_adam_step (indices NULL: every tensor) or ttp_adam_step_subset (the
 * listed tensors), with the same arithmetic and results, allocating nothing: no device or
 * pinned memory, no work or bias-correction table, no timing event.  No counterpart in the
 * reference; it is for callers that cannot allocate: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Its norm pass writes its per-block
 * partials into a fixed 64 KiB array of the library on each device (8192 fp64 partials,
 * held until the process ends) instead of the context's own buffer; a step whose norm pass
 * would write more (one per block: up to TTP_NORM_GRID, twice that above 256 MiB of
 * gradients) fails with TTP_ERR_RANGE.  Every
 * no-allocation step on one device shares that array.  Eager calls are ordered by the
 * library: a call on another stream than the previous call's waits for that call's work
 * (an event made at ttp_create; no allocation).  Captured calls are not: graph launches of
 * such steps on different streams of one device race unless the caller orders them.
 * Whatever the step would have to allocate is refused with TTP_ERR_STATE before any work is
 * queued: a tensor set, or (with loss scaling or after a capture) betas, not stepped before,
 * and the m and v of the first Adam step of an FP32 store or of a MIXED store in the SGD
 * layout.  Step once with ttp_adam_step[_subset] first.  In host-count mode (no loss
 * scaling, never captured) the step needs no bias-correction table and builds none: a later
 * capture of Adam steps with those betas needs one allocating step with them first (the
 * capture refuses them otherwise).  A TTP_MODE_BF16 store refuses it (TTP_ERR_INVALID), as
 * it refuses every Adam step.  There is no report: ttp_scaler_get and ttp_get_step read the
 * results. */
int ttp_adam_step_noalloc(ttp_ctx* ctx, const ttp_adam_hparams* hp, const uint32_t* indices,
                          uint32_t n_indices);
/* Global L2 norm of the gradients that exist, unscaled by the current loss scale when
 * scaling is on (synchronous; does not change any state). */
int ttp_grad_norm(ttp_ctx* ctx, double* norm);
/* Per-tensor sums of squares of the listed tensors' gradients (those that have one),
 * unscaled by the current loss scale, kept on the device for a following step with
 * TTP_STEP_TENSOR_SUMS.  Meant for buckets of tensors whose gradients became final during the
 * backward: each call is a memory-bound pass over the bucket's gradients that can run on a
 * stream beside the backward's compute (ttp_set_stream, with the caller's events ordering it
 * after the bucket's producers), taking the norm pass off the step.  Asynchronous on the
 * context's stream; each tensor's sum adds its 16 KiB tiles' sums in tile order.  No
 * counterpart in the reference, whose optimizer has no gradient norm. */
int ttp_grad_sumsq_tensors(ttp_ctx* ctx, const uint32_t* indices, uint32_t n);

/* ---- step counter and loss scaler ------------------------------------------------------- */
int ttp_get_step(ttp_ctx* ctx, uint64_t* step);
int ttp_set_step(ttp_ctx* ctx, uint64_t step);
/* ttp_scaler_configure also resets the scale to init_scale and the tracker to 0.  Captured
 * graphs hold `enabled` and the growth / backoff settings as launch arguments: while graphs
 * of the context are alive, a configuration that changes them fails with TTP_ERR_STATE (the
 * same settings, to reset the scale, are accepted). */
int ttp_scaler_configure(ttp_ctx* ctx, const ttp_scaler_config* cfg);
int ttp_scaler_get(ttp_ctx* ctx, float* scale, int32_t* growth_tracker);
int ttp_scaler_set(ttp_ctx* ctx, float scale, int32_t growth_tracker);
/* The scale update of an iteration whose steps all passed TTP_STEP_DEFER_SCALE
 * (torch.amp.GradScaler.update after several GradScaler.step calls): back off if any of them
 * saw an overflow, else count one clean step toward growth.  Stream-ordered, capturable; a
 * no-op while loss scaling is off, and when no step deferred the update since the last one
 * (torch raises there), so an iteration's scale never moves twice.  ttp_scaler_configure, ttp_scaler_set and ttp_load_state
 * drop a pending overflow; ttp_save_state does not record one (save between iterations). */
int ttp_scaler_update(ttp_ctx* ctx);

/* ---- optimizer-state checkpoint ------------------------------------------------------------
 * The reference has no optimizer checkpoint (its TTNN tensors live only in device memory).
 * ttp_save_state writes what a resumed run needs to continue bit for bit: the fp32 master
 * weights, the Adam moments and the momentum buffer that exist, the per-tensor momentum
 * initialisation flags, the step count t and the loss scaler (config, scale, tracker), with
 * the tensor table they belong to and a trailing checksum.  Gradients are not saved.
 * Layout (little-endian): "TTPSTATE", u32 version 1, u32 mode, u32 n_tensors, u32 buffer
 * mask (1 master, 2 exp_avg, 4 exp_avg_sq, 8 momentum), u64 total, u64 t, f32 scale,
 * i32 growth_tracker, i32 scaler enabled, i32 growth_interval, f64 init_scale,
 * f64 growth_factor, f64 backoff_factor; n_tensors x {u64 numel, u32 flags, u32 momentum
 * initialised}; each present buffer as total fp32 values (padding included); u64 checksum
 * of all preceding bytes.  Both calls are synchronous and stream through a 64 MiB pinned
 * buffer.  ttp_save_state writes `path`.tmp and renames it over `path` when complete, so a
 * failed save leaves an earlier file at `path` as it was.  ttp_load_state requires the same
 * mode and tensor table (numel and flags), and loss-scaler values in the ranges that
 * ttp_scaler_configure and ttp_scaler_set accept; a buffer the file lacks is zeroed; the bf16
 * weights are recomputed from the master (a TTP_MODE_BF16 store saves its bf16 weights as the
 * master, widened exactly, and loads them back).  It reads the whole file and checks its size and
 * checksum before it changes the context, so a damaged, truncated or mismatched file is
 * rejected with the context unchanged (only an I/O error on the second read, or a file
 * replaced during the call, can leave it partly loaded).  While graphs of the context are
 * alive, a file whose loss-scaler settings differ from the context's is refused
 * (TTP_ERR_STATE), as ttp_scaler_configure refuses them. */
int ttp_save_state(ttp_ctx* ctx, const char* path);
int ttp_load_state(ttp_ctx* ctx, const char* path);

/* ---- graph capture and replay -------------------------------------------------------------
 * The counterpart of traced::TraceContext (autograd/traced/trace.hpp:21-88: capture once,
 * then replay): everything queued on the context's stream between ttp_capture_begin and
 * ttp_capture_end (the engine's steps, zero_grad and device-side transfers, and the caller's
 * own kernels when the context uses the caller's stream) becomes one hipGraph, replayed by
 * ttp_graph_launch.  From ttp_capture_begin on, the context keeps the Adam step count and its
 * bias corrections on the device, so each replay advances t exactly as an eager step does.
 * While capturing, calls that would allocate, build a work table or synchronise fail with
 * TTP_ERR_STATE: step each tensor set (and each optimizer, for its state) eagerly once before
 * capturing, pass no step report, and use no host transfers.  The legacy default stream
 * cannot be captured.  A graph replays the tensor sets, hyperparameters and flags seen at
 * capture time.  Captured calls change the per-tensor host flags (whether a gradient exists,
 * whether its sum is current) when the graph is launched: ttp_capture_end restores them to
 * their state at ttp_capture_begin, and each launch applies what the captured calls did to
 * them.  Destroy a context's graphs before the context (ttp_destroy refuses). */
int ttp_capture_begin(ttp_ctx* ctx);
/* out == NULL discards the capture. */
int ttp_capture_end(ttp_ctx* ctx, ttp_graph** out);
int ttp_graph_launch(ttp_graph* graph);
int ttp_graph_destroy(ttp_graph* graph);

/* ---- per-kernel timing (HIP events on the context's stream) ------------------------------ */
#define TTP_KERNEL_NORM 0   /* grad-norm / inf-check / scaler finalize pass */
#define TTP_KERNEL_UPDATE 1 /* fused multi-tensor update pass               */
/* on = 1 starts recording an event pair around every launch of every kernel. */
int ttp_timing_enable(ttp_ctx* ctx, int on);
/* Waits for the recorded events, returns the summed milliseconds and the count of `kernel`
 * passes since the last reset (an event pair spans each pass: a norm pass with its finalize,
 * an update with all its launches), then forgets them. */
int ttp_timing_collect(ttp_ctx* ctx, int kernel, double* total_ms, uint64_t* launches);

const char* ttp_last_error(void);
int ttp_abi_version(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* TTPERF_TTPERF_H */
