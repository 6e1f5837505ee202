"""Pins the CPU oracle (oracle/ttp_oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible slip in the restatement (a dropped term, a wrong
sign, decay applied after the update, bias correction on the wrong moment, a clip applied
before the unscale, a scale that grows on the wrong step) fails it:
  * the reference's own known answers (autograd/tests/test_sgd.cpp:45-70,
    verify/verify_autograd.py:119-162, tests/adam_optimizer.py:15-92, tests/sgd_optimizer.py:15-39);
  * torch library goldens for what the reference lacks (tests/golden/make_golden.py);
  * an exhaustive 2^32 check of the bf16 rounding against an independent method;
  * fp64 / math.fsum brute force for the norm; closed forms and invariants.
"""
import math

import numpy as np
import pytest

import oracle as O
from conftest import f32_ulp_diff, golden


# ---------------------------------------------------------------------------- helpers
def split(flat, numels):
    out, o = [], 0
    for n in numels:
        out.append(flat[o:o + n])
        o += n
    return out


def gather(st, which):
    return np.concatenate([st.view(which, i) for i in range(st.n)])


def run_torch_fixture(d, step_fn, mode=O.MODE_FP32, state_keys=("exp_avg", "exp_avg_sq")):
    numels = [int(n) for n in d["shapes_numel"]]
    st = O.OracleStore(numels, flags=[int(x) for x in d["decay"]], mode=mode)
    for i, x in enumerate(split(d["init"], numels)):
        st.set_master(i, x)
    hist = {"param": []}
    for k in state_keys:
        hist[k] = []
    for s in range(d["grads"].shape[0]):
        for i, g in enumerate(split(d["grads"][s], numels)):
            st.set_grad(i, g if mode == O.MODE_FP32 else O.bf16_rne(g))
        step_fn(st)
        hist["param"].append(gather(st, "master"))
        for k in state_keys:
            hist[k].append(gather(st, k))
    return st, {k: np.stack(v) for k, v in hist.items()}


def assert_close_rel(a, b, rtol, atol, what):
    err = np.abs(a.astype(np.float64) - b.astype(np.float64))
    lim = rtol * np.abs(b.astype(np.float64)) + atol
    worst = np.max(err - lim)
    assert worst <= 0, f"{what}: max excess {worst:g} (max err {err.max():g})"


# ---------------------------------------------------------------------------- bf16
def test_bf16_exhaustive_against_independent_rounding():
    # every fp32 bit pattern: carry-trick RNE vs nearest-even search in exact double
    assert O.lib().orc_bf16_check_range(0, 1 << 32, 8) == 0


def test_bf16_matches_torch_conversion():
    d = golden("bf16_torch.npz")
    x = d["x_bits"].view(np.float32)
    got = O.bf16_rne(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], d["bf16"][~nan])
    # NaN: canonical 0x7FC0 (c10::BFloat16's scalar conversion); torch's vectorised CPU
    # path writes 0xFFFF instead, so only NaN-ness is compared against the fixture.
    assert np.all(got[nan] == 0x7FC0)
    assert np.all((d["bf16"][nan] & 0x7F80) == 0x7F80) and np.all(d["bf16"][nan] & 0x7F)


def test_bf16_round_trip_is_identity():
    h = np.arange(1 << 16, dtype=np.uint16)
    f = O.bf16_to_f32(h)
    back = O.bf16_rne(f)
    finite_or_inf = ~np.isnan(f)
    assert np.array_equal(back[finite_or_inf], h[finite_or_inf])


# ---------------------------------------------------------------------------- reference known answers
@pytest.mark.parametrize("mode", [O.MODE_FP32, O.MODE_MIXED])
def test_sgd_bias_known_answer(mode):
    # autograd/tests/test_sgd.cpp:45-70 and verify/verify_autograd.py:119-162: a bias of
    # zeros with grad 32 (batch of ones) at lr 0.01 goes to -0.32, then -0.64.
    st = O.OracleStore([32], mode=mode)
    st.set_master(0, np.zeros(32, np.float32))
    g = np.full(32, 32.0, np.float32)
    expect = []
    for _ in range(2):
        st.set_grad(0, g if mode == O.MODE_FP32 else O.bf16_rne(g))
        st.sgd_step(lr=0.01)
        expect.append(st.view("master", 0).copy())
    np.testing.assert_allclose(expect[0], -0.32, atol=1e-6)
    np.testing.assert_allclose(expect[1], -0.64, atol=1e-6)
    # exact fp32 values of two rounded ops per step (multiply, then subtract)
    u = np.float32(32.0) * np.float32(0.01)
    assert np.all(expect[0] == np.float32(0) - u)
    assert np.all(expect[1] == (np.float32(0) - u) - u)
    if mode == O.MODE_MIXED:
        assert np.array_equal(st.view("param", 0), O.bf16_rne(expect[1]))


def test_adam_one_step_known_answer():
    # tests/adam_optimizer.py:25-50: Linear(32,32) from seed 31, grad = x^T @ ones, lr 0.1,
    # compared with the closed form _adam_step_ref (the reference asserts 1e-1; the fp32
    # restatement lands within a few ulp of the closed form).
    d = golden("reference_known_answers.npz")
    st = O.OracleStore([1024])
    st.set_master(0, d["adam1_w0"])
    st.set_grad(0, d["adam1_grad"])
    st.adam_step(lr=0.1, betas=(0.9, 0.999), eps=1e-8)
    got = st.view("master", 0).reshape(32, 32)
    np.testing.assert_allclose(got, d["adam1_w1"], atol=1e-1, rtol=1e-1)
    # the closed form divides lr*m_hat by the denominator, py/optim.py:85 multiplies lr by
    # m_hat/denom: both within a few ulp of the step size lr (w - lr*sign(g) can cancel, so
    # the bound is absolute)
    assert np.abs(got.astype(np.float64) - d["adam1_w1"]).max() <= 8 * np.spacing(np.float32(0.1))


def test_adam_two_steps_known_answer():
    # tests/adam_optimizer.py:53-92: two steps through tanh with grads from the current weights
    d = golden("reference_known_answers.npz")
    x = d["adam2_x"].astype(np.float32)
    st = O.OracleStore([1024])
    st.set_master(0, d["adam2_w0"])
    for _ in range(2):
        w = st.view("master", 0).reshape(32, 32)
        z = np.tanh(x @ w)
        st.set_grad(0, (x.T @ (1 - z * z)).astype(np.float32))
        st.adam_step(lr=0.1, betas=(0.9, 0.999), eps=1e-8)
        st.zero_grad()
    got = st.view("master", 0).reshape(32, 32)
    np.testing.assert_allclose(got, d["adam2_w2"], atol=1e-1, rtol=1e-1)
    np.testing.assert_allclose(got, d["adam2_w2"], atol=1e-5, rtol=1e-5)


def test_sgd_bf16_known_answer():
    # tests/sgd_optimizer.py:15-39: bf16 w0 - 0.1 * grad (reference tolerance 5e-2)
    d = golden("reference_known_answers.npz")
    st = O.OracleStore([1024], mode=O.MODE_MIXED)
    st.set_master(0, O.bf16_to_f32(d["sgd1_w0"]))
    st.set_grad(0, d["sgd1_grad"])
    st.sgd_step(lr=0.1)
    got = O.bf16_to_f32(st.view("param", 0))
    np.testing.assert_allclose(got, O.bf16_to_f32(d["sgd1_w1"]).ravel(), atol=5e-2, rtol=5e-2)


# ---------------------------------------------------------------------------- BF16 stores
def test_sgd_bf16_store_reproduces_the_reference_test_formulas_exactly():
    # tests/sgd_optimizer.py:15-39 and :42-78 compute their expected weights with torch on
    # bf16 tensors, `w - 0.1 * grad`: the product and the difference each rounded to bf16.
    # A BF16 store reproduces them bit for bit (its grads are the fixtures' own), over one
    # step and over two steps of the tanh model; the fp32-master store only within tolerance.
    d = golden("reference_known_answers.npz")
    st = O.OracleStore([1024], mode=O.MODE_BF16)
    st.param[:1024] = d["sgd1_w0"].ravel()
    st.set_grad(0, d["sgd1_grad"].ravel())
    st.sgd_step(lr=0.1)
    assert np.array_equal(st.view("param", 0), d["sgd1_w1"].ravel())
    st = O.OracleStore([1024], mode=O.MODE_BF16)
    st.param[:1024] = d["sgd2_w0"].ravel()
    for g, w in (("sgd2_g1", "sgd2_w1"), ("sgd2_g2", "sgd2_w2")):
        st.set_grad(0, d[g].ravel())
        st.sgd_step(lr=0.1)
        assert np.array_equal(st.view("param", 0), d[w].ravel()), w
    # py/optim.py:19-21 itself on bf16 tensors fills lr into a bf16 tensor (full_like), so its
    # product uses lr = RNE_bf16(0.1): a BF16 store stepped with that lr equals torch's run of
    # the same three ops on bf16 tensors, which differs from the fp32-lr formula above
    st = O.OracleStore([1024], mode=O.MODE_BF16)
    st.param[:1024] = d["sgd1_w0"].ravel()
    st.set_grad(0, d["sgd1_grad"].ravel())
    lr16 = float(O.bf16_to_f32(O.bf16_rne(np.array([0.1], np.float32)))[0])
    assert lr16 == 0.10009765625
    st.sgd_step(lr=lr16)
    assert np.array_equal(st.view("param", 0), d["sgd_pyopt_w1"].ravel())
    assert not np.array_equal(d["sgd_pyopt_w1"], d["sgd1_w1"])
    mixed = O.OracleStore([1024], mode=O.MODE_MIXED)
    mixed.set_master(0, O.bf16_to_f32(d["sgd1_w0"].ravel()))
    mixed.set_grad(0, d["sgd1_grad"].ravel())
    mixed.sgd_step(lr=0.1)
    assert not np.array_equal(mixed.view("param", 0), d["sgd1_w1"].ravel())


def test_sgd_bf16_store_bias_known_answer():
    # autograd/tests/test_sgd.cpp:45-70 on the reference's bf16 tensors: grad 32 at lr 0.01
    # gives the update RNE_bf16(0.32) = 0.3203125, so the bias goes to -0.3203125, then to
    # RNE_bf16(-0.640625) = -0.640625 (within the test's 0.1 of -0.32 and -0.64)
    st = O.OracleStore([32], mode=O.MODE_BF16)
    for want in (-0.3203125, -0.640625):
        st.set_grad(0, O.bf16_rne(np.full(32, 32.0, np.float32)))
        st.sgd_step(lr=0.01)
        assert np.all(O.bf16_to_f32(st.view("param", 0)) == np.float32(want))


def _rne_rational(x, neg, sig_bits):
    """x (a Fraction, exact) rounded to nearest, ties to even, in a binary format with
    `sig_bits` significant bits and fp32's exponent range below (subnormals from 2^-126 down;
    no overflow in the cases used).  Returns (value, negative) so that zeros keep a sign."""
    from fractions import Fraction
    if x == 0:
        return Fraction(0), neg
    negative = x < 0
    a = -x if negative else x
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    q = Fraction(2) ** (max(e, -126) - (sig_bits - 1))
    n, rem = divmod(a, q)
    if 2 * rem > q or (2 * rem == q and n % 2 == 1):
        n += 1
    r = n * q
    return (-r if negative else r), negative


def _bf16_of(v):
    value, negative = v
    f = np.float32(float(value)) if value != 0 else np.float32(-0.0 if negative else 0.0)
    return int(f.view(np.uint32) >> 16)


def test_sgd_bf16_store_against_exact_rational_rounding():
    # Every finite bf16 weight below 2^126 in magnitude, stepped with a few (grad, lr) pairs,
    # against exact rational arithmetic rounded by an independent nearest-even routine: the
    # product g*lr rounded to fp32, then to bf16 (multiply's result), the difference rounded
    # to fp32, then to bf16 (subtract's).  The signs of zero follow IEEE: an exact zero
    # difference is +0 unless both operands are -0 and +0; an underflowing product or
    # difference keeps its sign.
    from fractions import Fraction
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = O.bf16_to_f32(bits)
    keep = np.isfinite(vals) & (np.abs(vals) < 2.0 ** 126)
    bits, vals = bits[keep], vals[keep]
    for g_f, lr in ((32.0, 0.01), (-3.140625, 1e-3), (2.0 ** -100, 0.1), (0.0078125, 3e-5)):
        g_bits = int(O.bf16_rne(np.array([g_f], np.float32))[0])
        st = O.OracleStore([len(bits)], mode=O.MODE_BF16, nthreads=8)
        st.param[:len(bits)] = bits
        st.set_grad(0, np.full(len(bits), g_bits, np.uint16))
        st.sgd_step(lr=lr)
        got = st.view("param", 0)
        g = Fraction(float(O.bf16_to_f32(np.array([g_bits], np.uint16))[0]))
        lr32 = Fraction(float(np.float32(lr)))
        prod_neg = (g < 0) != (lr32 < 0)
        u = _rne_rational(*_rne_rational(g * lr32, prod_neg, 24), 8)
        u_val, u_neg = u
        want = np.empty(len(bits), np.uint16)
        for k, (b, v) in enumerate(zip(bits, vals)):
            p_neg = bool(int(b) >> 15)
            d = Fraction(float(v)) - u_val
            # exact zero: -0 - (+0) is -0, every other zero difference +0
            d_neg = (d < 0) or (d == 0 and p_neg and not u_neg and v == 0 and u_val == 0)
            want[k] = _bf16_of(_rne_rational(*_rne_rational(d, d_neg, 24), 8))
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, (g_f, lr, [(hex(int(bits[i])), hex(int(got[i])), hex(int(want[i])))
                                         for i in bad[:5]])


# ---------------------------------------------------------------------------- torch goldens
def _adam_run(d, **hp):
    return run_torch_fixture(d, lambda st: st.adam_step(**hp))[1]


@pytest.mark.parametrize("name,hp", [
    ("torch_adam", dict(lr=0.1, betas=(0.9, 0.999), eps=1e-8)),
    ("torch_adamw", dict(lr=0.05, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.3,
                         decoupled=True)),
    ("torch_adam_l2", dict(lr=0.05, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.3,
                           decoupled=False)),
])
def test_adam_family_matches_torch(name, hp):
    d = golden(name + ".npz")
    got = _adam_run(d, **hp)
    # torch evaluates lr/bc1 * m / (sqrt(v)/sqrt(bc2) + eps) and lerps m; the restatement
    # keeps py/optim.py's op order, so they agree to a few fp32 roundings per step.
    assert_close_rel(got["exp_avg"], d["exp_avg"], 2e-6, 1e-7, name + " m")
    assert_close_rel(got["exp_avg_sq"], d["exp_avg_sq"], 2e-6, 1e-8, name + " v")
    assert_close_rel(got["param"], d["param"], 2e-6, 2e-7, name + " p")


def test_adamw_decay_placement_is_visible():
    # decay applied after the update instead of before must fail the torch comparison
    d = golden("torch_adamw.npz")
    got = _adam_run(d, lr=0.05, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0)
    with pytest.raises(AssertionError):
        assert_close_rel(got["param"], d["param"], 2e-6, 2e-7, "no-decay")


@pytest.mark.parametrize("name", ["torch_sgd_plain", "torch_sgd_momentum", "torch_sgd_damp_wd",
                                  "torch_sgd_nesterov"])
def test_sgd_family_matches_torch(name):
    d = golden(name + ".npz")
    lr, mu, damp, wd, nest = d["hp"]
    keys = ("momentum",) if mu else ()
    _, got = run_torch_fixture(
        d, lambda st: st.sgd_step(lr=lr, momentum=mu, dampening=damp, weight_decay=wd,
                                  nesterov=bool(nest)), state_keys=keys)
    assert_close_rel(got["param"], d["param"], 1e-6, 1e-7, name + " p")
    if mu:
        assert_close_rel(got["momentum"], d["momentum_buffer"], 1e-6, 1e-7, name + " buf")


def test_scaler_sequences_match_torch():
    d = golden("torch_scaler.npz")

    def run(steps, inf_steps, interval, tracker0=0):
        st = O.OracleStore([4], mode=O.MODE_MIXED)
        st.configure_scaler(True, 65536.0, 2.0, 0.5, interval)
        if tracker0:
            st.set_scaler_state(65536.0, tracker0)
        scales, trackers, skipped = [], [], []
        for s in range(1, steps + 1):
            g = np.ones(4, np.float32) * st.scale
            if s in inf_steps:
                g[1] = np.inf
            st.set_grad(0, O.bf16_rne(g))
            r = st.sgd_step(lr=1e-3)
            scales.append(r["scale"])
            trackers.append(r["growth_tracker"])
            skipped.append(r["skipped"])
        return np.array(scales), np.array(trackers), np.array(skipped)

    s, t, k = run(200, {50, 100, 150, 200}, 2000)
    assert np.array_equal(s, d["cfg3_scale"]) and np.array_equal(t, d["cfg3_tracker"])
    assert np.array_equal(k, d["cfg3_skipped"])
    # closed form of the config-3 schedule: skips at 50/100/150/200, 65536 -> 4096
    assert list(np.nonzero(k)[0] + 1) == [50, 100, 150, 200] and s[-1] == 4096.0
    s, t, k = run(14, set(d["short_inf"].tolist()), 3)
    assert np.array_equal(s, d["short_scale"]) and np.array_equal(t, d["short_tracker"])
    assert np.array_equal(k, d["short_skipped"])
    s, t, _ = run(3, set(), 2000, tracker0=1999)
    assert np.array_equal(s, d["forced_scale"]) and np.array_equal(t, d["forced_tracker"])


def _two_optimizer_scaler_run(d, defer_first=True, call_update=False):
    """Two parameter groups of one loss-scaled oracle store stepped as two optimizers per
    iteration (group 0 = tensor 0, group 1 = tensor 1), as tests/golden's
    torch_scaler_two_opt fixture steps two torch optimizers under one GradScaler."""
    st = O.OracleStore([4, 3], mode=O.MODE_MIXED)
    st.configure_scaler(True, 65536.0, 2.0, 0.5, int(d["interval"]))
    inf1, inf2 = set(d["inf1"].tolist()), set(d["inf2"].tolist())
    scales, trackers, skip1, skip2 = [], [], [], []
    for s in range(1, len(d["scale"]) + 1):
        g0 = np.ones(4, np.float32) * st.scale
        g1 = np.ones(3, np.float32) * st.scale
        if s in inf1:
            g0[2] = np.inf
        if s in inf2:
            g1[0] = np.inf
        st.set_grad(0, O.bf16_rne(g0))
        st.set_grad(1, O.bf16_rne(g1))
        st.set_has_grad(1, False)  # optimizer 1 owns tensor 0
        r1 = st.sgd_step(lr=1e-3, update_scale=not defer_first)
        st.set_has_grad(0, False)
        st.set_has_grad(1, True)   # optimizer 2 owns tensor 1
        r2 = st.sgd_step(lr=1e-3, update_scale=not call_update)
        if call_update:
            st.scaler_update()
        scales.append(st.scale)
        trackers.append(st.growth_tracker)
        skip1.append(r1["skipped"])
        skip2.append(r2["skipped"])
    return np.array(scales), np.array(trackers), np.array(skip1), np.array(skip2)


def test_scaler_with_two_optimizers_matches_torch():
    """Each optimizer skips on its own overflow and the scale moves once per iteration, on
    the overflow of either: torch's GradScaler.step per optimizer and one update().  The
    deferred first step plus an updating second step, and two deferred steps plus
    scaler_update, both give torch's sequence; updating the scale in each step does not."""
    d = golden("torch_scaler_two_opt.npz")
    for call_update in (False, True):
        s, t, k1, k2 = _two_optimizer_scaler_run(d, call_update=call_update)
        assert np.array_equal(s, d["scale"]) and np.array_equal(t, d["tracker"])
        assert np.array_equal(k1, d["skip1"]) and np.array_equal(k2, d["skip2"])
    # both overflowing in one iteration backs off once (65536 -> 32768 at step 9, not 16384)
    assert d["scale"][8] == d["scale"][7] / 2 and d["skip1"][8] and d["skip2"][8]
    s, t, _, _ = _two_optimizer_scaler_run(d, defer_first=False)
    assert not (np.array_equal(s, d["scale"]) and np.array_equal(t, d["tracker"]))


def test_scaler_update_moves_the_scale_once_per_iteration():
    """scaler_update applies only after a step that deferred the update: after an updating
    step, or a second time, it changes nothing; after deferred steps it counts one clean
    step, or backs off once however many of them overflowed."""
    st = O.OracleStore([4, 3], mode=O.MODE_MIXED)
    st.configure_scaler(True, 1024.0, 2.0, 0.5, 3)

    def step(update_scale, inf=False):
        g = np.ones(4, np.float32) * st.scale
        if inf:
            g[0] = np.inf
        st.set_grad(0, O.bf16_rne(g))
        return st.sgd_step(lr=1e-3, update_scale=update_scale)

    step(True)
    assert (st.scale, st.growth_tracker) == (1024.0, 1)
    st.scaler_update()  # no deferred step since the last update: nothing
    assert (st.scale, st.growth_tracker) == (1024.0, 1)
    step(False)
    step(False)
    st.scaler_update()  # two clean deferred steps: one clean iteration
    assert (st.scale, st.growth_tracker) == (1024.0, 2)
    st.scaler_update()
    assert (st.scale, st.growth_tracker) == (1024.0, 2)
    r = step(False, inf=True)
    assert r["skipped"] and r["scale"] == 1024.0  # deferred: the scale waits
    step(False, inf=True)
    step(False)
    st.scaler_update()  # two overflows in the iteration: one backoff
    assert (st.scale, st.growth_tracker) == (512.0, 0)
    step(False)
    step(True)  # the updating step closes the iteration ...
    assert (st.scale, st.growth_tracker) == (512.0, 1)
    st.scaler_update()  # ... so this changes nothing
    assert (st.scale, st.growth_tracker) == (512.0, 1)


@pytest.mark.parametrize("case", ["big", "small", "mid"])
def test_clip_matches_torch(case):
    d = golden("torch_clip.npz")
    g = d[f"{case}_grads"]
    st = O.OracleStore([g.size])
    st.set_grad(0, g)
    sumsq, bad = st.grad_sumsq()
    norm = math.sqrt(sumsq)
    assert not bad
    assert abs(norm - float(d[f"{case}_fsum_norm"])) <= 1e-12 * norm
    assert abs(norm - float(d[f"{case}_norm"])) <= 1e-5 * norm  # torch norms in fp32
    coef = O.lib().orc_clip_coef(norm, float(d[f"{case}_max"]))
    clipped = (g * np.float32(coef)).astype(np.float32)
    assert f32_ulp_diff(clipped, d[f"{case}_clipped"]).max() <= 2
    if case == "small":
        assert coef == 1.0


# ---------------------------------------------------------------------------- invariants
def _random_store(rng, mode, numels=(257, 64, 1000, 3), decay=(1, 0, 1, 0)):
    st = O.OracleStore(list(numels), flags=list(decay), mode=mode)
    for i, n in enumerate(numels):
        st.set_master(i, rng.normal(0, 0.5, n).astype(np.float32))
    return st


def _set_random_grads(st, rng, scale=1.0):
    for i, n in enumerate(st.numels):
        g = (rng.normal(0, 1e-2, n) * scale).astype(np.float32)
        st.set_grad(i, g if st.mode == O.MODE_FP32 else O.bf16_rne(g))


@pytest.mark.parametrize("mode", [O.MODE_FP32, O.MODE_MIXED])
def test_opbyop_equals_fused_bitwise(rng, mode):
    a = _random_store(np.random.default_rng(5), mode)
    b = _random_store(np.random.default_rng(5), mode)
    for st in (a, b):
        st.configure_scaler(True, 1024.0)
    for s in range(4):
        r1 = np.random.default_rng(100 + s)
        r2 = np.random.default_rng(100 + s)
        _set_random_grads(a, r1, 1024.0)
        _set_random_grads(b, r2, 1024.0)
        hp = dict(lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.05)
        a.adam_step(**hp)
        b.adam_step(opbyop=True, **hp)
    for k in ("master", "exp_avg", "exp_avg_sq", "param"):
        assert np.array_equal(getattr(a, k), getattr(b, k)), k


def test_adamw_wd0_is_adam_bitwise(rng):
    a = _random_store(np.random.default_rng(9), O.MODE_FP32, decay=(0, 0, 0, 0))
    b = _random_store(np.random.default_rng(9), O.MODE_FP32, decay=(1, 1, 1, 1))
    for s in range(3):
        _set_random_grads(a, np.random.default_rng(s))
        _set_random_grads(b, np.random.default_rng(s))
        a.adam_step(lr=1e-3)
        b.adam_step(lr=1e-3, weight_decay=0.0)
    assert np.array_equal(a.master, b.master)


def test_sgd_momentum0_is_plain_sgd(rng):
    a = _random_store(np.random.default_rng(3), O.MODE_FP32)
    p0 = a.master.copy()
    _set_random_grads(a, np.random.default_rng(4))
    g = a.grad.copy()
    a.sgd_step(lr=0.05)
    expect = (p0 - (g * np.float32(0.05))).astype(np.float32)
    assert np.array_equal(a.master, expect)


def test_mixed_param_is_rne_of_master(rng):
    st = _random_store(rng, O.MODE_MIXED)
    for s in range(3):
        _set_random_grads(st, rng)
        st.adam_step(lr=1e-2, weight_decay=0.1)
    for i in range(st.n):
        assert np.array_equal(st.view("param", i), O.bf16_rne(st.view("master", i)))


def test_skipped_step_leaves_state_bit_unchanged(rng):
    st = _random_store(rng, O.MODE_MIXED)
    st.configure_scaler(True, 65536.0)
    _set_random_grads(st, rng, 65536.0)
    st.adam_step(lr=1e-3, weight_decay=0.1, max_grad_norm=1.0)
    snap = {k: getattr(st, k).copy() for k in ("master", "param", "exp_avg", "exp_avg_sq")}
    t0 = st.t
    _set_random_grads(st, rng, 65536.0)
    st.view("grad", 2)[17] = 0x7F80  # +inf in bf16
    r = st.adam_step(lr=1e-3, weight_decay=0.1, max_grad_norm=1.0)
    assert r["found_inf"] and r["skipped"] and st.t == t0 and st.scale == 32768.0
    for k, v in snap.items():
        assert np.array_equal(getattr(st, k), v), k


def test_none_grad_tensor_untouched(rng):
    # py/optim.py:56-57 / autograd/dynamic/optim.hpp:23: params without grad are skipped
    st = _random_store(rng, O.MODE_FP32)
    _set_random_grads(st, rng)
    st.set_has_grad(1, False)
    before = st.view("master", 1).copy()
    st.adam_step(lr=1e-2, weight_decay=0.5)
    assert np.array_equal(st.view("master", 1), before)
    assert not st.view("exp_avg", 1).any()
    st.zero_grad()
    assert not any(st.has_grad(i) for i in range(st.n))


def test_norm_brute_force_and_scaling(rng):
    g = rng.normal(0, 1, 37).astype(np.float32)
    st = O.OracleStore([37])
    st.set_grad(0, g)
    s1, _ = st.grad_sumsq()
    assert s1 == pytest.approx(math.fsum(float(x) ** 2 for x in g), rel=1e-15)
    s2, _ = st.grad_sumsq(inv_scale=0.25)  # power of two: exact scaling of every square
    assert s2 == s1 / 16
    for bad in (np.inf, -np.inf, np.nan):
        h = g.copy()
        h[5] = bad
        st.set_grad(0, h)
        assert st.grad_sumsq()[1]
    h = g.copy()
    h[5] = 3e38  # huge but finite: no overflow flag
    st.set_grad(0, h)
    assert not st.grad_sumsq()[1]


def test_bias_correction_host_double():
    # py/optim.py:51-52 in host double, rounded once to fp32
    for beta in (0.9, 0.95, 0.999):
        for t in (1, 2, 7, 100, 5000):
            assert O.lib().orc_bias_correction(beta, t) == np.float32(1.0 - beta ** t)


def test_validation_rejects_reference_cases():
    # tests/adam_optimizer.py:126-151 and tests/sgd_optimizer.py:112-122
    st = O.OracleStore([4])
    st.set_grad(0, np.ones(4, np.float32))
    for hp in (dict(lr=0.0), dict(lr=-1.0), dict(eps=0.0), dict(betas=(1.1, 0.9)),
               dict(betas=(0.9, 0.0))):
        with pytest.raises(ValueError):
            st.adam_step(**hp)
    for lr in (0.0, -1.0):
        with pytest.raises(ValueError):
            st.sgd_step(lr=lr)


def test_accumulate_grad_matches_torch_bf16_and_fp32_addition(rng):
    """orc_accumulate_grad: first call assigns, later calls add in fp32 with one rounding to
    the grad type; pinned on torch's own bf16 / fp32 tensor addition (a library, not the
    reference) on values chosen to exercise bf16 rounding and ties."""
    import torch
    n = 4096
    a = (rng.standard_normal(n) * 3).astype(np.float32)
    b = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    b[:64] = np.ldexp(1.0, -9) * np.sign(a[:64])  # near-tie increments relative to |a|~1
    for mode in (O.MODE_MIXED, O.MODE_FP32):
        st = O.OracleStore([n], mode=mode, nthreads=1)
        for src_kind in ("f32", "bf16"):
            st.zero_grad()
            ga = O.bf16_rne(a) if src_kind == "bf16" else a
            gb = O.bf16_rne(b) if src_kind == "bf16" else b
            st.accumulate_grad(0, ga)
            st.accumulate_grad(0, gb)
            ta = torch.from_numpy(O.bf16_to_f32(ga) if src_kind == "bf16" else a)
            tb = torch.from_numpy(O.bf16_to_f32(gb) if src_kind == "bf16" else b)
            if mode == O.MODE_MIXED:
                g = ta.to(torch.bfloat16)          # first assignment rounds to the grad type
                g.add_(tb if src_kind == "f32" else tb.to(torch.bfloat16))
                want = g.view(torch.int16).numpy().view(np.uint16)
                assert np.array_equal(st.grad[:n], want), (mode, src_kind)
            else:
                want = (ta + tb).numpy()
                assert np.array_equal(st.grad[:n].view(np.uint32), want.view(np.uint32))
            assert st.has_grad(0)


def test_layout_invariants(rng):
    """orc_layout (the flat store's tensor placement): every tensor starts on a 64-element
    boundary (16-byte vectors never straddle tensors, 128-byte lines for bf16), tensors do not
    overlap and keep caller order, and the padding per tensor is < 64 elements."""
    for trial in range(50):
        n = int(rng.integers(0, 40))
        numels = [int(x) for x in rng.integers(0, 5000, n)]
        if trial % 5 == 0 and n:
            numels[0] = 0  # empty tensors are allowed
        offs, total = O.layout(numels)
        assert len(offs) == n
        end = 0
        for o, k in zip(offs, numels):
            assert o % O.ALIGN == 0
            assert o >= end  # caller order, no overlap
            assert o - end < O.ALIGN  # padding below one alignment unit
            end = int(o) + k
        assert total % O.ALIGN == 0 and end <= total < end + O.ALIGN
        assert total <= sum(numels) + O.ALIGN * n
    offs, total = O.layout([])
    assert total == 0
