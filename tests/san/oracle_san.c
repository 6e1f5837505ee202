/*
 * oracle_san.c — drives every entry point of the CPU oracle (oracle/ttp_oracle.c) on ragged
 * tensor tables, with every flat buffer allocated at its exact size, so that a build under
 * AddressSanitizer/UBSan (tests/test_oracle_sanitizers.py) catches any out-of-bounds access or
 * undefined behaviour in the checker itself.  It also re-checks two invariants on the way:
 * the op-by-op Adam (py/optim.py:76-86 as separate passes) equals the fused step bit for bit,
 * and a step skipped on a non-finite gradient leaves the state untouched.  A BF16 store runs with
 * no fp32 state allocated at all.
 * Prints "oracle_san: PASS" and exits 0 when every check holds.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ttp_oracle.h"

static int failures = 0;
#define CHECK(cond, msg)                                  \
    do {                                                  \
        if (!(cond)) {                                    \
            printf("FAIL: %s (line %d)\n", msg, __LINE__); \
            ++failures;                                   \
        }                                                 \
    } while (0)

static uint64_t rng = 88172645463325252ull;
static float frand(float scale) {
    rng ^= rng << 13;
    rng ^= rng >> 7;
    rng ^= rng << 17;
    return ((float)(rng >> 40) / 16777216.0f - 0.5f) * scale;
}

typedef struct {
    orc_store s;
    orc_tensor* t;
    uint64_t* numel;
} Store;

static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) {
        printf("out of memory\n");
        exit(3);
    }
    return p;
}

static Store make(const uint64_t* numel, uint32_t n, int mode, int nthreads) {
    Store st;
    memset(&st, 0, sizeof st);
    uint64_t* off = xmalloc(n * sizeof(uint64_t));
    const uint64_t total = orc_layout(numel, n, 64, off);
    st.t = xmalloc(n * sizeof(orc_tensor));
    for (uint32_t i = 0; i < n; ++i) {
        st.t[i].offset = off[i];
        st.t[i].numel = numel[i];
        st.t[i].flags = (i % 2) ? ORC_DECAY : 0u;
        st.t[i].has_grad = 1;
    }
    free(off);
    orc_store* s = &st.s;
    s->mode = mode;
    s->n_tensors = n;
    s->tensors = st.t;
    s->total = total;
    const size_t gsz = mode == ORC_MODE_MIXED ? 2 : 4;
    s->grad = xmalloc(total * gsz);
    s->master = xmalloc(total * 4);
    s->param = mode == ORC_MODE_MIXED ? xmalloc(total * 2) : (void*)s->master;
    s->exp_avg = xmalloc(total * 4);
    s->exp_avg_sq = xmalloc(total * 4);
    s->momentum = xmalloc(total * 4);
    s->mom_init = xmalloc(n ? n : 1);
    memset(s->mom_init, 0, n ? n : 1);
    memset(s->exp_avg, 0, total * 4);
    memset(s->exp_avg_sq, 0, total * 4);
    memset(s->momentum, 0, total * 4);
    for (uint64_t k = 0; k < total; ++k) s->master[k] = frand(0.04f);
    if (mode == ORC_MODE_MIXED) orc_f32_to_bf16_array(s->master, (uint16_t*)s->param, total);
    s->growth_interval = 3;
    s->growth_factor = 2.0;
    s->backoff_factor = 0.5;
    s->scale = 1024.0f;
    s->nthreads = nthreads;
    return st;
}

static void fill_grads(Store* st, float scale) {
    orc_store* s = &st->s;
    for (uint64_t k = 0; k < s->total; ++k) {
        const float g = frand(2e-3f) * scale;
        if (s->mode == ORC_MODE_MIXED)
            ((uint16_t*)s->grad)[k] = orc_bf16_rne(g);
        else
            ((float*)s->grad)[k] = g;
    }
}

static void copy_state(Store* dst, const Store* src) {
    const uint64_t total = src->s.total;
    memcpy(dst->s.master, src->s.master, total * 4);
    memcpy(dst->s.exp_avg, src->s.exp_avg, total * 4);
    memcpy(dst->s.exp_avg_sq, src->s.exp_avg_sq, total * 4);
    memcpy(dst->s.grad, src->s.grad, total * (src->s.mode == ORC_MODE_MIXED ? 2 : 4));
    if (src->s.mode == ORC_MODE_MIXED) memcpy(dst->s.param, src->s.param, total * 2);
    dst->s.t = src->s.t;
    dst->s.scale = src->s.scale;
    dst->s.growth_tracker = src->s.growth_tracker;
    dst->s.scaler_enabled = src->s.scaler_enabled;
}

static void release(Store* st) {
    orc_store* s = &st->s;
    free(s->grad);
    if (s->mode == ORC_MODE_MIXED) free(s->param);
    free(s->master);
    free(s->exp_avg);
    free(s->exp_avg_sq);
    free(s->momentum);
    free(s->mom_init);
    free(st->t);
}

static void run_mode(int mode) {
    const uint64_t numel[] = {0, 1, 3, 63, 64, 65, 1000, 2049, 4097, 10};
    const uint32_t n = sizeof numel / sizeof numel[0];
    Store a = make(numel, n, mode, 4), b = make(numel, n, mode, 1);
    orc_report r;
    const int mixed = mode == ORC_MODE_MIXED;
    a.s.scaler_enabled = b.s.scaler_enabled = mixed;

    // fused vs op-by-op Adam (AdamW, clip) on identical inputs, thread counts 4 and 1
    orc_adam_hp hp = {1e-2, 0.9, 0.95, 1e-8, 0.1, 1, 0, 0.5};
    a.t[4].has_grad = b.t[4].has_grad = 0;  // a None grad
    for (int step = 0; step < 4; ++step) {
        fill_grads(&a, mixed ? a.s.scale : 1.0f);
        copy_state(&b, &a);
        CHECK(orc_adam_step(&a.s, &hp, &r) == 0, "orc_adam_step");
        CHECK(orc_adam_step_opbyop(&b.s, &hp, NULL) == 0, "orc_adam_step_opbyop");
        CHECK(memcmp(a.s.master, b.s.master, a.s.total * 4) == 0, "fused == op-by-op: master");
        CHECK(memcmp(a.s.exp_avg, b.s.exp_avg, a.s.total * 4) == 0, "fused == op-by-op: m");
        CHECK(memcmp(a.s.exp_avg_sq, b.s.exp_avg_sq, a.s.total * 4) == 0, "fused == op-by-op: v");
        CHECK(a.s.t == b.s.t && a.s.scale == b.s.scale, "fused == op-by-op: counters");
    }
    // a non-finite gradient: with loss scaling the step is skipped and nothing moves
    if (mixed) {
        fill_grads(&a, a.s.scale);
        ((uint16_t*)a.s.grad)[a.t[7].offset + 5] = 0x7F80;  // +inf
        copy_state(&b, &a);
        const float scale = a.s.scale;
        CHECK(orc_adam_step(&a.s, &hp, &r) == 0, "orc_adam_step (inf)");
        CHECK(r.found_inf && r.skipped, "inf found and step skipped");
        CHECK(a.s.scale == scale * 0.5f && a.s.growth_tracker == 0, "scale backed off");
        CHECK(memcmp(a.s.master, b.s.master, a.s.total * 4) == 0, "skipped step: master");
        CHECK(memcmp(a.s.exp_avg_sq, b.s.exp_avg_sq, a.s.total * 4) == 0, "skipped step: v");
        CHECK(a.s.t == b.s.t, "skipped step: t");
    }
    // SGD family: momentum 0 equals plain SGD bitwise; momentum, nesterov, dampening + L2
    orc_sgd_hp plain = {1e-2, 0.0, 0.0, 0.0, 0, 0, 0.0};
    fill_grads(&a, mixed ? a.s.scale : 1.0f);
    copy_state(&b, &a);
    orc_sgd_hp zero_mom = plain;
    zero_mom.momentum = 0.0;
    CHECK(orc_sgd_step(&a.s, &plain, NULL) == 0 && orc_sgd_step(&b.s, &zero_mom, NULL) == 0, "sgd");
    CHECK(memcmp(a.s.master, b.s.master, a.s.total * 4) == 0, "sgd momentum 0 == plain");
    orc_sgd_hp variants[3] = {{1e-2, 0.9, 0.0, 0.0, 0, 0, 1.0}, {1e-2, 0.9, 0.0, 0.0, 1, 0, 0.0},
                              {1e-2, 0.9, 0.1, 1e-2, 0, 0, 0.5}};
    for (int v = 0; v < 3; ++v)
        for (int step = 0; step < 2; ++step) {
            fill_grads(&a, mixed ? a.s.scale : 1.0f);
            CHECK(orc_sgd_step(&a.s, &variants[v], &r) == 0, "sgd variant");
        }
    // gradient accumulation (fp32 and bf16 sources), norm pass
    for (uint32_t i = 0; i < n; ++i) {
        float* f = xmalloc((numel[i] ? numel[i] : 1) * 4);
        uint16_t* h = xmalloc((numel[i] ? numel[i] : 1) * 2);
        for (uint64_t k = 0; k < numel[i]; ++k) f[k] = frand(1e-2f);
        orc_f32_to_bf16_array(f, h, numel[i]);
        a.t[i].has_grad = 0;
        orc_accumulate_grad(&a.s, i, f, 0);
        orc_accumulate_grad(&a.s, i, h, 1);
        CHECK(a.t[i].has_grad == 1, "accumulate marks the grad present");
        free(f);
        free(h);
    }
    int32_t inf = 0;
    const double ss = orc_grad_sumsq(&a.s, 1.0f, &inf);
    CHECK(ss >= 0.0 && !inf, "grad_sumsq");
    release(&a);
    release(&b);
}

/* A BF16 store holds only bf16 weights and bf16 gradients: its fp32 state pointers stay NULL,
 * so any read or write of them in this mode faults here.  Adam and SGD with momentum or decay
 * are refused with nothing changed; plain SGD runs the same with 4 threads as with 1; a
 * non-finite gradient under loss scaling skips the step. */
static void run_bf16(void) {
    const uint64_t numel[] = {0, 1, 3, 63, 64, 65, 1000, 2049, 4097, 10};
    const uint32_t n = sizeof numel / sizeof numel[0];
    orc_tensor ta[sizeof numel / sizeof numel[0]], tb[sizeof numel / sizeof numel[0]];
    uint64_t off[sizeof numel / sizeof numel[0]];
    const uint64_t total = orc_layout(numel, n, 64, off);
    for (uint32_t i = 0; i < n; ++i) {
        ta[i].offset = off[i];
        ta[i].numel = numel[i];
        ta[i].flags = (i % 2) ? ORC_DECAY : 0u;
        ta[i].has_grad = 1;
    }
    memcpy(tb, ta, sizeof ta);
    orc_store a, b;
    memset(&a, 0, sizeof a);
    a.mode = ORC_MODE_BF16;
    a.n_tensors = n;
    a.tensors = ta;
    a.total = total;
    a.param = xmalloc(total * 2);
    a.grad = xmalloc(total * 2);
    a.growth_interval = 3;
    a.growth_factor = 2.0;
    a.backoff_factor = 0.5;
    a.scale = 1024.0f;
    a.nthreads = 4;
    b = a;
    b.tensors = tb;
    b.param = xmalloc(total * 2);
    b.grad = xmalloc(total * 2);
    b.nthreads = 1;
    uint16_t* pa = a.param;
    uint16_t* ga = a.grad;
    uint16_t* keep = xmalloc(total * 2);
    for (uint64_t k = 0; k < total; ++k) {
        pa[k] = orc_bf16_rne(frand(0.5f));
        ga[k] = orc_bf16_rne(frand(0.1f));
    }
    orc_report r;
    memcpy(keep, pa, total * 2);
    orc_adam_hp adam = {1e-3, 0.9, 0.999, 1e-8, 0.0, 1, 0, 0.0};
    CHECK(orc_adam_step(&a, &adam, &r) == -1, "BF16 store refuses Adam");
    CHECK(orc_adam_step_opbyop(&a, &adam, NULL) == -1, "BF16 store refuses op-by-op Adam");
    orc_sgd_hp refused[2] = {{1e-2, 0.9, 0.0, 0.0, 0, 0, 0.0}, {1e-2, 0.0, 0.0, 1e-2, 0, 0, 0.0}};
    for (int v = 0; v < 2; ++v)
        CHECK(orc_sgd_step(&a, &refused[v], &r) == -1, "BF16 store refuses momentum and decay");
    CHECK(memcmp(pa, keep, total * 2) == 0 && a.t == 0, "refusals change nothing");

    // plain SGD, with and without clipping, a None grad: 4 threads against 1, bit for bit
    ta[4].has_grad = tb[4].has_grad = 0;
    orc_sgd_hp plain[2] = {{1e-2, 0.0, 0.0, 0.0, 0, 0, 0.0}, {5e-2, 0.0, 0.0, 0.0, 0, 0, 0.25}};
    for (int step = 0; step < 4; ++step) {
        for (uint64_t k = 0; k < total; ++k) ga[k] = orc_bf16_rne(frand(0.1f));
        memcpy(b.param, a.param, total * 2);
        memcpy(b.grad, a.grad, total * 2);
        memcpy(keep, pa, total * 2);
        CHECK(orc_sgd_step(&a, &plain[step % 2], &r) == 0 &&
                  orc_sgd_step(&b, &plain[step % 2], NULL) == 0, "BF16 sgd");
        CHECK(memcmp(a.param, b.param, total * 2) == 0, "BF16 sgd: 4 threads == 1 thread");
        CHECK(memcmp(pa + ta[4].offset, keep + ta[4].offset, numel[4] * 2) == 0,
              "BF16 sgd: a None grad leaves its weights");
        CHECK(a.t == (uint64_t)step + 1 && b.t == (uint64_t)step + 1, "BF16 sgd: step count");
    }
    // one element by hand: 1.0 - bf16(1.0 * 0.5) = 0.5, exact in bf16
    pa[ta[1].offset] = 0x3F80;
    ga[ta[1].offset] = 0x3F80;
    orc_sgd_hp half = {0.5, 0.0, 0.0, 0.0, 0, 0, 0.0};
    CHECK(orc_sgd_step(&a, &half, NULL) == 0 && pa[ta[1].offset] == 0x3F00, "BF16 sgd: 1 - 0.5");

    // loss scaling: a +inf gradient skips the step and backs the scale off
    a.scaler_enabled = 1;
    for (uint64_t k = 0; k < total; ++k) ga[k] = orc_bf16_rne(frand(0.1f) * a.scale);
    ga[ta[7].offset + 5] = 0x7F80;
    memcpy(keep, pa, total * 2);
    const uint64_t t0 = a.t;
    const float scale = a.scale;
    CHECK(orc_sgd_step(&a, &plain[1], &r) == 0, "BF16 sgd (inf)");
    CHECK(r.found_inf && r.skipped && a.t == t0, "BF16 sgd: inf found and step skipped");
    CHECK(a.scale == scale * 0.5f && memcmp(pa, keep, total * 2) == 0, "BF16 skipped step");

    // accumulation into bf16 gradients from fp32 and bf16 sources, then the norm pass
    for (uint32_t i = 0; i < n; ++i) {
        float* f = xmalloc((numel[i] ? numel[i] : 1) * 4);
        uint16_t* h = xmalloc((numel[i] ? numel[i] : 1) * 2);
        for (uint64_t k = 0; k < numel[i]; ++k) f[k] = frand(1e-2f);
        orc_f32_to_bf16_array(f, h, numel[i]);
        ta[i].has_grad = 0;
        orc_accumulate_grad(&a, i, f, 0);
        orc_accumulate_grad(&a, i, h, 1);
        CHECK(ta[i].has_grad == 1, "BF16 accumulate marks the grad present");
        for (uint64_t k = 0; k < numel[i]; ++k)  // h + h with h exact in bf16: exactly 2h
            CHECK(ga[ta[i].offset + k] == orc_bf16_rne(2.0f * orc_bf16_to_f32(h[k])),
                  "BF16 accumulate: h + h");
        free(f);
        free(h);
    }
    int32_t inf = 0;
    CHECK(orc_grad_sumsq(&a, 1.0f, &inf) >= 0.0 && !inf, "BF16 grad_sumsq");
    free(keep);
    free(a.param);
    free(a.grad);
    free(b.param);
    free(b.grad);
}

int main(void) {
    run_mode(ORC_MODE_FP32);
    run_mode(ORC_MODE_MIXED);
    run_bf16();
    // bf16 helpers: a slice of the exhaustive rounding check, special values, array forms
    CHECK(orc_bf16_check_range(0x7F7F0000ull, 0x7F810000ull, 2) == 0, "bf16 near overflow/inf/NaN");
    CHECK(orc_bf16_check_range(0x00000000ull, 0x00020000ull, 2) == 0, "bf16 denormals");
    float x[5] = {0.0f, -0.0f, INFINITY, NAN, 1.00390625f};
    uint16_t h[5];
    float y[5];
    orc_f32_to_bf16_array(x, h, 5);
    orc_bf16_to_f32_array(h, y, 5);
    CHECK(h[2] == 0x7F80 && h[3] == 0x7FC0 && y[4] == 1.0f, "bf16 specials and ties to even");
    CHECK(orc_clip_coef(0.5, 1.0) == 1.0f && orc_clip_coef(4.0, 1.0) < 0.26f, "clip coefficient");
    CHECK(orc_bias_correction(0.9, 1) == (float)(1.0 - 0.9), "bias correction");
    float scale = 8.0f;
    int32_t tracker = 2;
    orc_scaler_update(&scale, &tracker, 0, 2.0, 0.5, 3);
    CHECK(scale == 16.0f && tracker == 0, "scaler growth");
    if (failures) {
        printf("oracle_san: %d check(s) failed\n", failures);
        return 1;
    }
    printf("oracle_san: PASS\n");
    return 0;
}
