/*
 * ttp_oracle.c — CPU restatement of csirak/tt-perf's optimizer step (test infrastructure;
 * see ttp_oracle.h for the reference lines each part follows and how each part is pinned).
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off).  Every fp32 expression below
 * rounds after each operation (FLT_EVAL_METHOD 0 on x86-64, contraction off), which is the
 * op-at-a-time rounding of the reference's TTNN programs.
 */
#include "ttp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------ */
/* bf16                                                                                 */
/* ------------------------------------------------------------------------------------ */

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* Round-to-nearest-even to bf16 by the carry trick; NaN becomes the canonical quiet NaN
 * 0x7FC0 (what torch's float->bfloat16 conversion returns for every NaN). */
uint16_t orc_bf16_rne(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void orc_f32_to_bf16_array(const float* x, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = orc_bf16_rne(x[i]);
}

void orc_bf16_to_f32_array(const uint16_t* x, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(x[i]);
}

/* Independent method: take the two bf16 neighbours of x (truncation and the next pattern
 * away from zero), measure both distances exactly in double, pick the nearer, ties to the
 * even pattern.  The pattern past the largest finite bf16 is +-inf, whose "value" for the
 * rounding decision is 2^128 (IEEE overflow threshold). */
static uint16_t bf16_nearest_search(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    if ((u & 0x7FFFFFFFu) == 0x7F800000u) return (uint16_t)(u >> 16);
    uint16_t lo = (uint16_t)(u >> 16);
    uint16_t hi = (uint16_t)(lo + 1u);
    double xv = fabs((double)x);
    double lv = fabs((double)orc_bf16_to_f32(lo));
    double hv = ((hi & 0x7FFFu) == 0x7F80u) ? ldexp(1.0, 128) : fabs((double)orc_bf16_to_f32(hi));
    double dl = xv - lv, dh = hv - xv;
    if (dl < dh) return lo;
    if (dh < dl) return hi;
    return (lo & 1u) ? hi : lo;
}

uint64_t orc_bf16_check_range(uint64_t lo, uint64_t hi, int nthreads) {
    uint64_t bad = 0;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static) reduction(+ : bad)
    for (int64_t i = (int64_t)lo; i < (int64_t)hi; ++i) {
        float x = u2f((uint32_t)i);
        if (orc_bf16_rne(x) != bf16_nearest_search(x)) ++bad;
    }
    return bad;
}

/* ------------------------------------------------------------------------------------ */
/* host constants                                                                       */
/* ------------------------------------------------------------------------------------ */

/* py/optim.py:50-52: bias = 1 - beta ** step in host double; the ttnn full_like fill then
 * rounds it to the tensor dtype (fp32 here). */
float orc_bias_correction(double beta, uint64_t t) {
    return (float)(1.0 - pow(beta, (double)t));
}

/* clip_grad_norm_: coef = max_norm / (total_norm + 1e-6), clamped to at most 1.  Evaluated
 * in double and rounded once; NaN propagates (torch's clamp keeps NaN). */
float orc_clip_coef(double norm, double max_norm) {
    double c = max_norm / (norm + 1e-6);
    if (c > 1.0) c = 1.0;
    return (float)c;
}

/* torch _amp_update_scale_: backoff on overflow, grow after growth_interval clean steps
 * (only if the grown scale is finite); products in double, stored as fp32. */
void orc_scaler_update(float* scale, int32_t* tracker, int found_inf, double growth_factor,
                       double backoff_factor, int32_t growth_interval) {
    if (found_inf) {
        *scale = (float)((double)*scale * backoff_factor);
        *tracker = 0;
    } else {
        int32_t ok = *tracker + 1;
        if (ok == growth_interval) {
            float ns = (float)((double)*scale * growth_factor);
            if (isfinite(ns)) *scale = ns;
            *tracker = 0;
        } else {
            *tracker = ok;
        }
    }
}

uint64_t orc_layout(const uint64_t* numel, uint32_t n, uint64_t align, uint64_t* offsets) {
    uint64_t off = 0;
    for (uint32_t i = 0; i < n; ++i) {
        offsets[i] = off;
        off += (numel[i] + align - 1) / align * align;
    }
    return off;
}

/* ------------------------------------------------------------------------------------ */
/* work decomposition: fixed 64K-element chunks of tensors that have a grad              */
/* ------------------------------------------------------------------------------------ */

#define ORC_CHUNK 65536u

typedef struct {
    uint64_t begin, end;
    uint32_t tensor, flags;
} chunk_t;

static chunk_t* build_chunks(const orc_store* s, uint64_t* nc_out) {
    uint64_t nc = 0;
    for (uint32_t i = 0; i < s->n_tensors; ++i)
        if (s->tensors[i].has_grad && s->tensors[i].numel)
            nc += (s->tensors[i].numel + ORC_CHUNK - 1) / ORC_CHUNK;
    chunk_t* c = (chunk_t*)malloc(sizeof(chunk_t) * (nc ? nc : 1));
    uint64_t k = 0;
    for (uint32_t i = 0; i < s->n_tensors; ++i) {
        const orc_tensor* t = &s->tensors[i];
        if (!t->has_grad || !t->numel) continue;
        for (uint64_t b = 0; b < t->numel; b += ORC_CHUNK) {
            c[k].begin = t->offset + b;
            c[k].end = t->offset + (b + ORC_CHUNK < t->numel ? b + ORC_CHUNK : t->numel);
            c[k].tensor = i;
            c[k].flags = t->flags;
            ++k;
        }
    }
    *nc_out = nc;
    return c;
}

static inline float load_grad(const orc_store* s, uint64_t i) {
    return s->mode != ORC_MODE_FP32 ? orc_bf16_to_f32(((const uint16_t*)s->grad)[i])
                                     : ((const float*)s->grad)[i];
}

double orc_grad_sumsq(const orc_store* s, float inv_scale, int32_t* found_inf) {
    uint64_t nc = 0;
    chunk_t* ch = build_chunks(s, &nc);
    double* part = (double*)calloc(nc ? nc : 1, sizeof(double));
    int* bad = (int*)calloc(nc ? nc : 1, sizeof(int));
    int nt = s->nthreads > 0 ? s->nthreads : 1;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
    for (int64_t k = 0; k < (int64_t)nc; ++k) {
        double acc = 0.0;
        int b = 0;
        for (uint64_t i = ch[k].begin; i < ch[k].end; ++i) {
            float g = load_grad(s, i) * inv_scale;
            if (!isfinite(g)) b = 1;
            acc += (double)g * (double)g;
        }
        part[k] = acc;
        bad[k] = b;
    }
    double sum = 0.0;
    int any = 0;
    for (uint64_t k = 0; k < nc; ++k) { sum += part[k]; any |= bad[k]; }
    free(part); free(bad); free(ch);
    if (found_inf) *found_inf = any;
    return sum;
}

void orc_accumulate_grad(orc_store* s, uint32_t index, const void* src, int src_bf16) {
    orc_tensor* t = (orc_tensor*)&s->tensors[index];
    const int first = !t->has_grad;
    for (uint64_t k = 0; k < t->numel; ++k) {
        const float in = src_bf16 ? orc_bf16_to_f32(((const uint16_t*)src)[k]) : ((const float*)src)[k];
        const uint64_t i = t->offset + k;
        if (s->mode != ORC_MODE_FP32) {
            uint16_t* g = (uint16_t*)s->grad;
            g[i] = orc_bf16_rne(first ? in : orc_bf16_to_f32(g[i]) + in);
        } else {
            float* g = (float*)s->grad;
            g[i] = first ? in : g[i] + in;
        }
    }
    t->has_grad = 1;
}

/* ------------------------------------------------------------------------------------ */
/* Adam / AdamW                                                                         */
/* ------------------------------------------------------------------------------------ */

typedef struct {
    float lr, b1, omb1, b2, omb2, eps, bias1, bias2;
    float decay_mul;  /* (float)(1 - lr*wd): decoupled decay factor */
    float wd;         /* (float)wd: L2 coefficient */
    float inv_scale, clip;
    int use_inv, use_clip, decoupled, wd_on;
} adam_coefs;

static void adam_make_coefs(const orc_adam_hp* hp, uint64_t t, adam_coefs* c) {
    /* py/optim.py:60-71 fills lr, beta1, beta2, 1-beta1, 1-beta2, eps with full_like:
     * the Python double rounded once to fp32. */
    c->lr = (float)hp->lr;
    c->b1 = (float)hp->beta1;
    c->omb1 = (float)(1.0 - hp->beta1);
    c->b2 = (float)hp->beta2;
    c->omb2 = (float)(1.0 - hp->beta2);
    c->eps = (float)hp->eps;
    c->bias1 = orc_bias_correction(hp->beta1, t);
    c->bias2 = orc_bias_correction(hp->beta2, t);
    c->decay_mul = (float)(1.0 - hp->lr * hp->weight_decay);
    c->wd = (float)hp->weight_decay;
    c->decoupled = hp->decoupled;
    c->wd_on = hp->weight_decay != 0.0;
}

/* One element of Adam in the op order of py/optim.py:76-86, preceded by the gradient
 * transforms (unscale, clip) and the weight decay of the tensor. */
static inline void adam_elem(float* pp, float g, float* mp, float* vp, const adam_coefs* c,
                             int decay) {
    float p = *pp;
    if (c->use_inv) g = g * c->inv_scale;
    if (c->use_clip) g = g * c->clip;
    if (decay && c->wd_on) {
        if (c->decoupled) p = p * c->decay_mul;      /* AdamW: param.mul_(1 - lr*wd) */
        else g = g + c->wd * p;                       /* Adam L2: grad.add(param, alpha=wd) */
    }
    float m = c->b1 * *mp + c->omb1 * g;             /* py/optim.py:76 */
    float gsq = g * g;                                /* :77 */
    float v = c->b2 * *vp + c->omb2 * gsq;           /* :78 */
    float m_hat = m / c->bias1;                       /* :82 */
    float v_hat = v / c->bias2;                       /* :83 */
    float denom = sqrtf(v_hat) + c->eps;              /* :84 */
    float step = c->lr * (m_hat / denom);             /* :85 */
    p = p - step;                                     /* :86 */
    *pp = p;
    *mp = m;
    *vp = v;
}

static int adam_validate(const orc_adam_hp* hp) {
    /* py/optim.py:33-41 */
    if (!(hp->lr > 0) || !(hp->eps > 0)) return -1;
    if (!(hp->beta1 > 0 && hp->beta1 < 1 && hp->beta2 > 0 && hp->beta2 < 1)) return -1;
    if (!(hp->weight_decay >= 0)) return -1;
    return 0;
}

/* shared prologue: norm pass, skip decision, clip coefficient */
static void step_prologue(orc_store* s, double max_norm, float* inv_scale, float* clip,
                          int* use_clip, int* skip, orc_report* rep) {
    int need_norm = s->scaler_enabled || max_norm > 0;
    *inv_scale = s->scaler_enabled ? (float)(1.0 / (double)s->scale) : 1.0f;
    int32_t found = 0;
    double norm = NAN;
    if (need_norm) norm = sqrt(orc_grad_sumsq(s, *inv_scale, &found));
    *skip = s->scaler_enabled && found;
    *use_clip = max_norm > 0;
    *clip = *use_clip ? orc_clip_coef(norm, max_norm) : 1.0f;
    if (rep) {
        memset(rep, 0, sizeof(*rep));
        rep->found_inf = found;
        rep->skipped = *skip;
        rep->grad_norm = norm;
        rep->clip_coef = *clip;
    }
}

/* torch GradScaler: each optimizer's step checks and skips on its own overflow; update()
 * then moves the scale once, on the overflow found by any optimizer since the last update
 * (found_inf summed over optimizers, torch/amp/grad_scaler.py update) */
void orc_scaler_update_pending(orc_store* s) {
    if (!s->scaler_enabled || !(s->pending & ORC_PENDING_STEP)) return;
    orc_scaler_update(&s->scale, &s->growth_tracker, s->pending & ORC_PENDING_INF,
                      s->growth_factor, s->backoff_factor, s->growth_interval);
    s->pending = 0;
}

static void step_epilogue(orc_store* s, int found_inf, int defer, orc_report* rep) {
    if (s->scaler_enabled) {
        s->pending |= ORC_PENDING_STEP | (found_inf ? ORC_PENDING_INF : 0);
        if (!defer) orc_scaler_update_pending(s);
    }
    if (rep) {
        /* without loss scaling the report carries scale 1 and tracker 0 */
        rep->scale = s->scaler_enabled ? s->scale : 1.0f;
        rep->growth_tracker = s->scaler_enabled ? s->growth_tracker : 0;
        rep->step = s->t;
    }
}

int orc_adam_step(orc_store* s, const orc_adam_hp* hp, orc_report* rep) {
    if (adam_validate(hp) || s->mode == ORC_MODE_BF16) return -1;
    if (!s->exp_avg || !s->exp_avg_sq) return -5;
    orc_report local;
    orc_report* r = rep ? rep : &local;
    float inv, clip;
    int use_clip, skip;
    step_prologue(s, hp->max_grad_norm, &inv, &clip, &use_clip, &skip, r);
    if (!skip) {
        s->t += 1; /* py/optim.py:50 */
        adam_coefs c;
        adam_make_coefs(hp, s->t, &c);
        c.inv_scale = inv;
        c.use_inv = s->scaler_enabled;
        c.clip = clip;
        c.use_clip = use_clip;
        uint64_t nc = 0;
        chunk_t* ch = build_chunks(s, &nc);
        int nt = s->nthreads > 0 ? s->nthreads : 1;
        const int mixed = s->mode == ORC_MODE_MIXED;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
        for (int64_t k = 0; k < (int64_t)nc; ++k) {
            const int decay = (ch[k].flags & ORC_DECAY) != 0;
            for (uint64_t i = ch[k].begin; i < ch[k].end; ++i) {
                adam_elem(&s->master[i], load_grad(s, i), &s->exp_avg[i], &s->exp_avg_sq[i],
                          &c, decay);
                if (mixed) ((uint16_t*)s->param)[i] = orc_bf16_rne(s->master[i]);
            }
        }
        free(ch);
    }
    step_epilogue(s, r->found_inf, hp->flags & ORC_STEP_DEFER_SCALE, r);
    return 0;
}

/* ---- op-by-op Adam: one full pass per ttnn op, each into a new temporary ------------- */

static float* tmp_alloc(uint64_t n) { return (float*)malloc(sizeof(float) * (n ? n : 1)); }

#define PASS(nt, n, expr)                                              \
    do {                                                                \
        _Pragma("omp parallel for num_threads(nt) schedule(static)")   \
        for (int64_t i = 0; i < (int64_t)(n); ++i) { expr; }           \
    } while (0)

int orc_adam_step_opbyop(orc_store* s, const orc_adam_hp* hp, orc_report* rep) {
    if (adam_validate(hp) || s->mode == ORC_MODE_BF16) return -1;
    if (!s->exp_avg || !s->exp_avg_sq) return -5;
    orc_report local;
    orc_report* r = rep ? rep : &local;
    float inv, clip;
    int use_clip, skip;
    step_prologue(s, hp->max_grad_norm, &inv, &clip, &use_clip, &skip, r);
    if (!skip) {
        s->t += 1;
        adam_coefs c;
        adam_make_coefs(hp, s->t, &c);
        int nt = s->nthreads > 0 ? s->nthreads : 1;
        for (uint32_t ti = 0; ti < s->n_tensors; ++ti) {
            const orc_tensor* T = &s->tensors[ti];
            if (!T->has_grad || !T->numel) continue; /* py/optim.py:56-57 */
            const uint64_t n = T->numel, o = T->offset;
            float* p = s->master + o;
            float* m0 = s->exp_avg + o;
            float* v0 = s->exp_avg_sq + o;
            float* g = tmp_alloc(n);
            if (s->mode == ORC_MODE_MIXED) {
                const uint16_t* gb = (const uint16_t*)s->grad + o;
                PASS(nt, n, g[i] = orc_bf16_to_f32(gb[i]));
            } else {
                const float* gf = (const float*)s->grad + o;
                PASS(nt, n, g[i] = gf[i]);
            }
            if (s->scaler_enabled) PASS(nt, n, g[i] = g[i] * inv);
            if (use_clip) PASS(nt, n, g[i] = g[i] * clip);
            if ((T->flags & ORC_DECAY) && c.wd_on) {
                if (c.decoupled) {
                    PASS(nt, n, p[i] = p[i] * c.decay_mul);
                } else {
                    float* wp = tmp_alloc(n);
                    PASS(nt, n, wp[i] = c.wd * p[i]);
                    PASS(nt, n, g[i] = g[i] + wp[i]);
                    free(wp);
                }
            }
            float *a = tmp_alloc(n), *b = tmp_alloc(n), *m = tmp_alloc(n);
            PASS(nt, n, a[i] = c.b1 * m0[i]);            /* mul(beta1, m)          :76 */
            PASS(nt, n, b[i] = c.omb1 * g[i]);           /* mul(1-beta1, grad)     :76 */
            PASS(nt, n, m[i] = a[i] + b[i]);             /* add                    :76 */
            float *gsq = tmp_alloc(n), *v = tmp_alloc(n);
            PASS(nt, n, gsq[i] = g[i] * g[i]);           /* grad_sq                :77 */
            PASS(nt, n, a[i] = c.b2 * v0[i]);            /* mul(beta2, v)          :78 */
            PASS(nt, n, b[i] = c.omb2 * gsq[i]);         /* mul(1-beta2, grad_sq)  :78 */
            PASS(nt, n, v[i] = a[i] + b[i]);             /* add                    :78 */
            float *mh = tmp_alloc(n), *vh = tmp_alloc(n), *den = tmp_alloc(n);
            PASS(nt, n, mh[i] = m[i] / c.bias1);          /* m_hat                  :82 */
            PASS(nt, n, vh[i] = v[i] / c.bias2);          /* v_hat                  :83 */
            PASS(nt, n, den[i] = sqrtf(vh[i]));           /* sqrt                   :84 */
            PASS(nt, n, den[i] = den[i] + c.eps);         /* + eps                  :84 */
            PASS(nt, n, a[i] = mh[i] / den[i]);           /* div(m_hat, denom)      :85 */
            PASS(nt, n, b[i] = c.lr * a[i]);              /* mul(lr, .)             :85 */
            PASS(nt, n, p[i] = p[i] - b[i]);              /* sub                    :86 */
            memcpy(m0, m, n * sizeof(float));             /* state["m"] = m         :79 */
            memcpy(v0, v, n * sizeof(float));             /* state["v"] = v         :80 */
            if (s->mode == ORC_MODE_MIXED) {
                uint16_t* pb = (uint16_t*)s->param + o;
                PASS(nt, n, pb[i] = orc_bf16_rne(p[i]));
            }
            free(g); free(a); free(b); free(m); free(gsq); free(v);
            free(mh); free(vh); free(den);
        }
    }
    step_epilogue(s, r->found_inf, hp->flags & ORC_STEP_DEFER_SCALE, r);
    return 0;
}

/* ------------------------------------------------------------------------------------ */
/* SGD (+ momentum, dampening, nesterov, L2 weight decay)                               */
/* ------------------------------------------------------------------------------------ */

typedef struct {
    float lr, mu, omd, wd, inv_scale, clip;
    int use_inv, use_clip, wd_on, mom_on, nesterov;
} sgd_coefs;

static inline void sgd_elem(float* pp, float g, float* bp, const sgd_coefs* c, int decay,
                            int first) {
    float p = *pp;
    if (c->use_inv) g = g * c->inv_scale;
    if (c->use_clip) g = g * c->clip;
    if (decay && c->wd_on) g = g + c->wd * p;        /* d_p.add(param, alpha=wd) */
    if (c->mom_on) {
        float buf = first ? g : c->mu * *bp + c->omd * g; /* buf.mul_(mu).add_(d_p, 1-damp) */
        *bp = buf;
        g = c->nesterov ? g + c->mu * buf : buf;
    }
    /* autograd/dynamic/optim.hpp:24-25: update = multiply(grad, lr); data - update */
    float update = g * c->lr;
    *pp = p - update;
}

/* autograd/dynamic/optim.hpp:24-25 on the reference's BFLOAT16 tensors
 * (autograd/dynamic/autograd.hpp:72, autograd/traced/nn.hpp:24-35): each ttnn op writes a
 * bf16 tensor, so multiply(grad, lr) and subtract(data, update) each round their fp32 result
 * to bf16 (round to nearest even) */
static inline uint16_t sgd_bf16_elem(uint16_t p, float g, const sgd_coefs* c) {
    if (c->use_inv) g = g * c->inv_scale;
    if (c->use_clip) g = g * c->clip;
    const float update = orc_bf16_to_f32(orc_bf16_rne(g * c->lr)); /* multiply(grad, lr) */
    return orc_bf16_rne(orc_bf16_to_f32(p) - update);               /* subtract(data, .) */
}

int orc_sgd_step(orc_store* s, const orc_sgd_hp* hp, orc_report* rep) {
    /* py/optim.py:9-10 (lr > 0); torch.optim.SGD for the rest */
    if (!(hp->lr > 0) || !(hp->momentum >= 0) || !(hp->weight_decay >= 0)) return -1;
    if (s->mode == ORC_MODE_BF16 && (hp->momentum != 0.0 || hp->weight_decay != 0.0)) return -1;
    if (hp->nesterov && (hp->momentum <= 0 || hp->dampening != 0)) return -1;
    const int mom_on = hp->momentum != 0.0;
    if (mom_on && (!s->momentum || !s->mom_init)) return -5;
    orc_report local;
    orc_report* r = rep ? rep : &local;
    float inv, clip;
    int use_clip, skip;
    step_prologue(s, hp->max_grad_norm, &inv, &clip, &use_clip, &skip, r);
    if (!skip) {
        s->t += 1;
        sgd_coefs c;
        c.lr = (float)hp->lr;
        c.mu = (float)hp->momentum;
        c.omd = (float)(1.0 - hp->dampening);
        c.wd = (float)hp->weight_decay;
        c.wd_on = hp->weight_decay != 0.0;
        c.mom_on = mom_on;
        c.nesterov = hp->nesterov;
        c.inv_scale = inv;
        c.use_inv = s->scaler_enabled;
        c.clip = clip;
        c.use_clip = use_clip;
        uint64_t nc = 0;
        chunk_t* ch = build_chunks(s, &nc);
        int nt = s->nthreads > 0 ? s->nthreads : 1;
        const int mixed = s->mode == ORC_MODE_MIXED;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
        for (int64_t k = 0; k < (int64_t)nc; ++k) {
            const int decay = (ch[k].flags & ORC_DECAY) != 0;
            const int first = mom_on ? !s->mom_init[ch[k].tensor] : 0;
            for (uint64_t i = ch[k].begin; i < ch[k].end; ++i) {
                if (s->mode == ORC_MODE_BF16) {
                    uint16_t* pb = (uint16_t*)s->param;
                    pb[i] = sgd_bf16_elem(pb[i], load_grad(s, i), &c);
                    continue;
                }
                sgd_elem(&s->master[i], load_grad(s, i), mom_on ? &s->momentum[i] : NULL, &c,
                         decay, first);
                if (mixed) ((uint16_t*)s->param)[i] = orc_bf16_rne(s->master[i]);
            }
        }
        if (mom_on)
            for (uint64_t k = 0; k < nc; ++k) s->mom_init[ch[k].tensor] = 1;
        free(ch);
    }
    step_epilogue(s, r->found_inf, hp->flags & ORC_STEP_DEFER_SCALE, r);
    return 0;
}
