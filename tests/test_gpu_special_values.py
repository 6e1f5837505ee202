"""Parity at IEEE special values: libttperf_hip against the CPU oracle when weights, gradients
and moments hold the values that ordinary random inputs never reach.

Seeded random inputs (N(0, 1e-3) gradients and the like) exercise neither subnormals, nor
squares that overflow or underflow fp32, nor bf16 rounding ties, nor non-finite values.  These
cases fill every buffer with such values, mixed with ordinary ones:
- fp32: +-0, the smallest and largest subnormals, the smallest normal, 2^-64 and 2^-66 (whose
  squares are subnormal), 2^64 (whose square overflows, so Adam's v becomes inf), FLT_MAX, and
  patterns on and around the bf16 rounding ties (0x3F808000 rounds to even, 0x3F818000 up,
  0x7F7F8000 and FLT_MAX to bf16 inf, 0x00008000 a subnormal tie);
- bf16 gradients of a mixed store: +-0, subnormals 0x0001 .. 0x007F, the bf16 maximum;
- non-finite values (+-inf, quiet and signalling NaNs of either sign) in gradients and
  weights, without loss scaling (they propagate through the update, as in the reference) and
  with it (the step is skipped and the scale backs off).
Weights, m and v are uploaded with these values too (v as magnitudes), so the update's
division and square root see subnormal and infinite operands.

Every store mode (fp32, mixed in the default layout, mixed in the SGD layout) and optimizer
form (AdamW, Adam with L2 decay and eps = 1e-30, the reference's plain SGD, Nesterov SGD with
decay) runs three steps with and without clipping at 1.0; so does a BF16 store (bf16 weights
and gradients only) with the reference's plain SGD, each op rounded to bf16.  After every step the weights, the
bf16 copies and the optimizer state must equal the oracle's bit for bit, except that two NaNs
count as equal whatever their sign and payload (x86 and the GPU produce different default
NaNs; the bf16 conversion maps every NaN to 0x7FC0 on both).  The step reports must agree
exactly: skip, overflow, step count, loss scale, and the clip coefficient (both NaN counts as
equal); the norm to 1e-12 relative, or in the same non-finite class.
"""
import numpy as np
import pytest

import oracle as O
from gpu_util import make_pair, pad_mask

pytestmark = pytest.mark.gpu

SHAPES = [(300,), (17, 5), (1,), (4096,), (64,)]
DECAY = [True, False, False, True, True]

F32_FINITE = np.array([
    0x00000000, 0x80000000,              # +-0
    0x00000001, 0x80000001,              # smallest subnormals
    0x00000100, 0x00400000, 0x807FFFFF,  # subnormals, largest subnormal
    0x00800000, 0x80800000,              # smallest normals
    0x1F800000, 0x9E800000,              # 2^-64, -2^-66: squares subnormal in fp32
    0x0C000000,                          # ~9.9e-32: square underflows to 0
    0x5F800000, 0xDF800000,              # 2^64: square overflows fp32
    0x7F7FFFFF, 0xFF7FFFFF,              # FLT_MAX: bf16 rounds it to inf
    0x3F800000, 0xBF800000,              # +-1
    0x3F808000, 0x3F818000, 0x3F808001,  # bf16 tie to even, tie up, above the tie
    0xBF818000, 0x00008000, 0x80018000,  # negative tie, subnormal ties
    0x7F7F8000, 0xFF7F7FFF,              # tie to bf16 inf; just below it
    0x4B000001, 0x3A83126F,              # ordinary values
], dtype=np.uint32).view(np.float32)
F32_NONFINITE = np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x7F800001,
                          0xFFA00000], dtype=np.uint32).view(np.float32)
BF16_FINITE = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x007F, 0x807F, 0x0040, 0x0080, 0x8080,
                        0x1F80, 0x9E80, 0x5F80, 0xDF80, 0x7F7F, 0xFF7F, 0x3F80, 0x3A83, 0xBB44],
                       dtype=np.uint16)
BF16_NONFINITE = np.array([0x7F80, 0xFF80, 0x7FC0, 0xFFC1, 0x7F81], dtype=np.uint16)

OPTS = {
    "adamw": ("adam", dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1,
                           decoupled=True)),
    "adam_l2_tiny_eps": ("adam", dict(lr=1e-2, betas=(0.8, 0.99), eps=1e-30, weight_decay=0.05,
                                      decoupled=False)),
    "sgd": ("sgd", dict(lr=1e-2)),
    "sgd_nesterov_wd": ("sgd", dict(lr=1e-2, momentum=0.9, nesterov=True, weight_decay=0.01)),
}
VARIANTS = ["finite", "finite_clip", "nonfinite", "nonfinite_clip", "scaled", "scaled_overflow"]
MODES = ["fp32", "mixed", "mixed_sgd_layout"]
CASES = [(m, o, v) for m in MODES for o in OPTS for v in VARIANTS
         if m != "fp32" or not v.startswith("scaled")]
# a BF16 store (bf16 weights and grads only) steps plain SGD, each op rounded to bf16
CASES += [("bf16", "sgd", v) for v in VARIANTS]
STORE_MODE = {"fp32": O.MODE_FP32, "mixed": O.MODE_MIXED, "mixed_sgd_layout": O.MODE_MIXED,
              "bf16": O.MODE_BF16}


def _mix(rng, total, mask, specials, ordinary):
    """`total` values: at tensor elements, a seeded draw of about half `specials` (each many
    times over in the larger tensors) and half `ordinary` values; zeros in the padding."""
    n = int(mask.sum())
    reps = -(-n // len(specials))
    pool = np.concatenate([np.tile(specials, reps), ordinary(rng, reps * len(specials))])
    rng.shuffle(pool)
    pool = pool[:n]
    out = np.zeros(total, dtype=specials.dtype)
    out[mask] = pool
    return out


def _normal_f32(std):
    return lambda rng, n: rng.normal(0.0, std, n).astype(np.float32)


def _normal_bf16(std):
    return lambda rng, n: O.bf16_rne(rng.normal(0.0, std, n).astype(np.float32))


def _check_bits(name, got, want, mask):
    g, w = got[mask], want[mask]
    if g.dtype == np.uint16:
        bad = g != w
        gb, wb = g, w
    else:
        gb, wb = g.view(np.uint32), w.view(np.uint32)
        bad = (gb != wb) & ~(np.isnan(g) & np.isnan(w))
    n = int(np.count_nonzero(bad))
    print(f"  {name}: {n} of {g.size} differ", flush=True)
    if n:
        at = np.flatnonzero(bad)[:6]
        raise AssertionError(f"{name}: {n} values differ; first at {at.tolist()}: got "
                             f"{[hex(int(x)) for x in gb[at]]} want {[hex(int(x)) for x in wb[at]]}")


def _check_report(r, e, scaler, norm_ran):
    assert (r["skipped"], r["found_inf"], r["step"]) == (e["skipped"], e["found_inf"], e["step"])
    if scaler:
        assert (r["scale"], r["growth_tracker"]) == (e["scale"], e["growth_tracker"])
    rc, ec = np.float32(r["clip_coef"]), np.float32(e["clip_coef"])
    assert rc.view(np.uint32) == ec.view(np.uint32) or (np.isnan(rc) and np.isnan(ec)), (rc, ec)
    if norm_ran:
        rn, en = r["grad_norm"], e["grad_norm"]
        if np.isfinite(en):
            assert abs(rn - en) <= 1e-12 * en, (rn, en)
        else:
            assert np.isnan(rn) == np.isnan(en) and not np.isfinite(rn), (rn, en)


@pytest.mark.parametrize("mode,opt,variant", CASES)
def test_special_values_match_the_oracle(mode, opt, variant, tmp_path):
    import ttperf
    from ttperf import _lib as L
    kind, hp = OPTS[opt]
    mixed = mode != "fp32"
    seed = 7000 + CASES.index((mode, opt, variant))
    print(f"case {mode} {opt} {variant} seed {seed}", flush=True)
    store, ref = make_pair(SHAPES, DECAY, STORE_MODE[mode], seed=seed,
                           layout="sgd" if mode == "mixed_sgd_layout" else "default")
    rng = np.random.default_rng(seed)
    mask = pad_mask(store)
    total = store.total
    nonfinite = variant.startswith("nonfinite")
    clip = 1.0 if variant.endswith("clip") else None
    scaler = variant.startswith("scaled")

    # weights (non-finite ones too in the non-finite variants), m and v
    wspec = np.concatenate([F32_FINITE, F32_NONFINITE]) if nonfinite else F32_FINITE
    master = _mix(rng, total, mask, wspec, _normal_f32(0.02))
    if mode == "bf16":  # the weights themselves are bf16: the values rounded, ties included
        store.upload(L.BUF_PARAM, L.ALL_TENSORS, O.bf16_rne(master))
        ref.param[:total] = O.bf16_rne(master)
        which = ["param"]
    else:
        store.upload(L.BUF_MASTER, L.ALL_TENSORS, master)
        ref.master[:total] = master
        if mixed:
            ref.param[:total] = O.bf16_rne(master)
        which = ["master"] + (["param"] if mixed else [])
    if kind == "adam":
        m = _mix(rng, total, mask, F32_FINITE, _normal_f32(1e-3))
        v = np.abs(_mix(rng, total, mask, F32_FINITE, _normal_f32(1e-3)))
        store.upload(L.BUF_EXP_AVG, L.ALL_TENSORS, m)
        store.upload(L.BUF_EXP_AVG_SQ, L.ALL_TENSORS, v)
        ref.exp_avg[:total] = m
        ref.exp_avg_sq[:total] = v
        which += ["exp_avg", "exp_avg_sq"]
    elif hp.get("momentum"):
        which += ["momentum"]
    if scaler:
        store.configure_scaler(True, init_scale=65536.0, growth_interval=2)
        ref.configure_scaler(True, 65536.0, growth_interval=2)

    for step in range(3):
        bad_grads = nonfinite or (variant == "scaled_overflow" and step == 1)
        if mixed:
            gspec = np.concatenate([BF16_FINITE, BF16_NONFINITE]) if bad_grads else BF16_FINITE
            g = _mix(rng, total, mask, gspec, _normal_bf16(1e-3 * (ref.scale if scaler else 1.0)))
        else:
            gspec = np.concatenate([F32_FINITE, F32_NONFINITE]) if bad_grads else F32_FINITE
            g = _mix(rng, total, mask, gspec, _normal_f32(1e-3))
        store.upload(L.BUF_GRAD, L.ALL_TENSORS, g)
        ref.grad[:total] = g
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        if kind == "adam":
            r = store.adam_step(report=True, max_grad_norm=clip, **hp)
            e = ref.adam_step(max_grad_norm=clip or 0.0, **hp)
        else:
            r = store.sgd_step(report=True, max_grad_norm=clip, **hp)
            e = ref.sgd_step(max_grad_norm=clip or 0.0, **hp)
        print(f" step {step}: skipped {e['skipped']} found_inf {e['found_inf']} "
              f"norm {e['grad_norm']:.6g} coef {e['clip_coef']:.6g}", flush=True)
        _check_report(r, e, scaler, norm_ran=bool(clip) or scaler)
        if variant == "scaled_overflow":
            assert e["skipped"] == (step == 1)
        for name in which:
            _check_bits(name, store.download(getattr(L, {
                "master": "BUF_MASTER", "param": "BUF_PARAM", "exp_avg": "BUF_EXP_AVG",
                "exp_avg_sq": "BUF_EXP_AVG_SQ", "momentum": "BUF_MOMENTUM"}[name])),
                getattr(ref, name)[:total], mask)
    # a checkpoint keeps every bit, NaN payloads included
    path = tmp_path / "special.ttp"
    store.save_state(path)
    fresh = ttperf.ParamStore(SHAPES, mode={"mixed_sgd_layout": "mixed"}.get(mode, mode),
                              decay=DECAY,
                              layout="sgd" if mode == "mixed_sgd_layout" else "default")
    fresh.load_state(path)
    assert fresh.step_count == store.step_count
    if scaler:
        assert fresh.scaler_state() == store.scaler_state()
    for name in which:
        buf = getattr(L, {"master": "BUF_MASTER", "param": "BUF_PARAM", "exp_avg": "BUF_EXP_AVG",
                          "exp_avg_sq": "BUF_EXP_AVG_SQ", "momentum": "BUF_MOMENTUM"}[name])
        a, b = store.download(buf)[mask], fresh.download(buf)[mask]
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{name} after save / load"
    fresh.close()
    got = store.download(L.BUF_PARAM if mode == "bf16" else L.BUF_MASTER)[mask]
    if mode == "bf16":
        got = O.bf16_to_f32(got)
    print(f"  final weights: {int(np.count_nonzero((got != 0) & (np.abs(got) < np.finfo(np.float32).tiny)))} "
          f"subnormal, {int(np.count_nonzero(~np.isfinite(got)))} non-finite", flush=True)
    store.close()


# incoming values whose pairwise sums stay finite (the finite iteration of the accumulate test)
F32_SUMMABLE = F32_FINITE[np.abs(F32_FINITE) < 1e38]
BF16_SUMMABLE = BF16_FINITE[np.abs(O.bf16_to_f32(BF16_FINITE)) < 1e38]

ACC_CASES = [(mode, src, multi, sums) for mode in ("fp32", "mixed", "bf16")
             for src in ("f32", "bf16") for multi in (False, True) for sums in (False, True)]


@pytest.mark.parametrize("mode,src,multi,sums", ACC_CASES)
def test_special_values_accumulate_match_the_oracle(mode, src, multi, sums):
    """Gradient accumulation at special values: each tensor receives two incoming gradients
    (the first assigns, the second adds: subnormal + subnormal, FLT_MAX + FLT_MAX = inf,
    inf + -inf = NaN, ...), one call per tensor or one bucket call, with or without the tiles'
    sums; the gradients must equal the oracle's bit for bit after each call.  Then an AdamW
    step with clipping (and loss scaling in a mixed store) takes its norm from the sums, or
    from its norm pass, and must match the oracle's step; a BF16 store takes the reference's
    plain SGD there, with clipping and loss scaling.  Two iterations: finite incoming
    values whose sums stay finite, then the largest and the non-finite ones too."""
    import torch
    from ttperf import _lib as L
    mixed = mode != "fp32"  # bf16 gradients (and loss scaling below)
    seed = 7500 + ACC_CASES.index((mode, src, multi, sums))
    print(f"case {mode} src {src} multi {multi} sums {sums} seed {seed}", flush=True)
    store, ref = make_pair(SHAPES, DECAY, STORE_MODE[mode], seed=seed)
    rng = np.random.default_rng(seed)
    mask = pad_mask(store)
    total = store.total
    if mixed:
        store.configure_scaler(True, init_scale=65536.0, growth_interval=2)
        ref.configure_scaler(True, 65536.0, growth_interval=2)
    hp = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, decoupled=True)
    which = ["master", "exp_avg", "exp_avg_sq"] + (["param"] if mixed else [])
    if mode == "bf16":
        hp, which = dict(lr=1e-2), ["param"]
    n = len(SHAPES)
    numels = [t.numel for t in store.tensors]
    for it, bad in enumerate((False, True)):
        store.zero_grad(set_to_none=True)
        ref.zero_grad(set_to_none=True)
        for rnd in range(2):
            vals = []
            for i in range(n):
                if src == "bf16":
                    spec = np.concatenate([BF16_FINITE, BF16_NONFINITE]) if bad else BF16_SUMMABLE
                    v = _mix(rng, numels[i], np.ones(numels[i], bool), spec,
                             _normal_bf16(1e-3 * ref.scale if mixed else 1e-3))
                else:
                    spec = np.concatenate([F32_FINITE, F32_NONFINITE]) if bad else F32_SUMMABLE
                    v = _mix(rng, numels[i], np.ones(numels[i], bool), spec,
                             _normal_f32(1e-3 * ref.scale if mixed else 1e-3))
                vals.append(v)
                ref.accumulate_grad(i, v)
            if multi:
                dev = [torch.from_numpy(v.view(np.int16)).cuda().view(torch.bfloat16)
                       if v.dtype == np.uint16 else torch.from_numpy(v).cuda() for v in vals]
                store.accumulate_grads(list(range(n)), dev, sums=sums)
            else:
                for i in range(n):
                    store.accumulate_grad(i, vals[i], sums=sums)
            _check_bits(f"grad after round {rnd}", store.download(L.BUF_GRAD), ref.grad[:total],
                        mask)
        if mode == "bf16":
            r = store.sgd_step(report=True, max_grad_norm=1.0, tensor_sums=sums, **hp)
            e = ref.sgd_step(max_grad_norm=1.0, **hp)
        else:
            r = store.adam_step(report=True, max_grad_norm=1.0, tensor_sums=sums, **hp)
            e = ref.adam_step(max_grad_norm=1.0, **hp)
        print(f" iteration {it}: skipped {e['skipped']} found_inf {e['found_inf']} "
              f"norm {e['grad_norm']:.6g} coef {e['clip_coef']:.6g}", flush=True)
        _check_report(r, e, mixed, norm_ran=True)
        assert e["found_inf"] == bad
        for name in which:
            _check_bits(name, store.download(getattr(L, {
                "master": "BUF_MASTER", "param": "BUF_PARAM", "exp_avg": "BUF_EXP_AVG",
                "exp_avg_sq": "BUF_EXP_AVG_SQ"}[name])), getattr(ref, name)[:total], mask)
    store.close()
