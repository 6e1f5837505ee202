"""Writes the small golden fixtures under tests/golden/ (run from the repo root:
`python tests/golden/make_golden.py`).

Sources of truth, none of them the reference's code (which needs ttnn and cannot run here):
  * torch library semantics for what the reference lacks: torch.optim.AdamW / Adam / SGD
    (foreach=False, single-tensor path), torch.amp.GradScaler on CPU,
    torch.nn.utils.clip_grad_norm_, torch's float32 -> bfloat16 conversion;
  * the reference tests' own known-answer setups, recomputed with their closed forms:
    tests/adam_optimizer.py:15-92 (seeds 31 and 32, _adam_step_ref) and
    tests/sgd_optimizer.py:15-78 (seeds 21 and 22, bf16 `w - 0.1*grad`).
Every fixture is data: inputs and expected outputs in .npz (no pickles).
"""
import math
import os

import numpy as np
import torch

OUT = os.path.dirname(os.path.abspath(__file__))


def f32(t):
    return t.detach().to(torch.float32).cpu().numpy().astype(np.float32)


def bf16_bits(t):
    return t.detach().to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)


# ------------------------------------------------------------------------------------------
def gen_bf16_special():
    vals = [0.0, -0.0, 1.0, -1.0, 1.00390625, 1.005859375, 1.0078125, 3.4028234663852886e38,
            -3.4028234663852886e38, 3.3895313892515355e38, 3.3961775292e38, 1e-45, -1e-45,
            1.1754942e-38, 1.17549435e-38, 9.1835e-41, float("inf"), float("-inf"),
            float("nan"), 65504.0, 1e-8, 0.1, 1.0 / 3.0, 2.0 ** -133, 2.0 ** -126]
    bits = [0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F817FFF, 0x7F7F8000, 0x7F7FFFFF,
            0xFF7FFFFF, 0x7FC00001, 0xFF800001, 0x7F800001, 0x00008000, 0x00018000,
            0x80008000, 0x0000FFFF, 0x7F7F7FFF, 0x3F7FFFFF, 0x00007FFF]
    x = np.concatenate([np.array(vals, np.float32),
                        np.array(bits, np.uint32).view(np.float32)])
    rng = np.random.default_rng(7)
    r = rng.integers(0, 2 ** 32, size=4096, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, r])
    y = bf16_bits(torch.from_numpy(x.copy()))
    np.savez(os.path.join(OUT, "bf16_torch.npz"), x_bits=x.view(np.uint32), bf16=y)


# ------------------------------------------------------------------------------------------
SHAPES = [(7, 5), (5,), (3, 4), (13,)]
DECAY = [1, 0, 1, 0]


def _init_params(seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g) * 0.5 for s in SHAPES]


def _grads(seed, steps):
    g = torch.Generator().manual_seed(seed)
    return [[torch.randn(*s, generator=g) for s in SHAPES] for _ in range(steps)]


def _run_torch_opt(make_opt, seed, steps, state_keys):
    params = [torch.nn.Parameter(p.clone()) for p in _init_params(seed)]
    opt = make_opt(params)
    grads = _grads(seed + 1000, steps)
    hist = {k: [] for k in ["param"] + state_keys}
    for s in range(steps):
        for p, g in zip(params, grads[s]):
            p.grad = g.clone()
        opt.step()
        hist["param"].append(np.concatenate([f32(p).ravel() for p in params]))
        for k in state_keys:
            hist[k].append(np.concatenate([f32(opt.state[p][k]).ravel() for p in params]))
    out = {"init": np.concatenate([f32(p).ravel() for p in _init_params(seed)]),
           "grads": np.stack([np.concatenate([f32(g).ravel() for g in gs]) for gs in grads]),
           "shapes_numel": np.array([int(np.prod(s)) for s in SHAPES], np.int64),
           "decay": np.array(DECAY, np.int32)}
    for k, v in hist.items():
        out[k] = np.stack(v)
    return out


def gen_adam_family():
    steps = 6
    # AdamW with decay only on the decayed tensors (two param groups), aggressive lr/wd so a
    # misplaced decay or bias correction shows far above fp32 rounding.
    hp = dict(lr=0.05, betas=(0.9, 0.95), eps=1e-8)

    def adamw(ps):
        return torch.optim.AdamW(
            [{"params": [p for p, d in zip(ps, DECAY) if d], "weight_decay": 0.3},
             {"params": [p for p, d in zip(ps, DECAY) if not d], "weight_decay": 0.0}],
            foreach=False, **hp)

    def adam_l2(ps):
        return torch.optim.Adam(
            [{"params": [p for p, d in zip(ps, DECAY) if d], "weight_decay": 0.3},
             {"params": [p for p, d in zip(ps, DECAY) if not d], "weight_decay": 0.0}],
            foreach=False, **hp)

    def adam(ps):
        return torch.optim.Adam(ps, foreach=False, lr=0.1, betas=(0.9, 0.999), eps=1e-8)

    for name, fn in (("adamw", adamw), ("adam_l2", adam_l2), ("adam", adam)):
        d = _run_torch_opt(fn, 11, steps, ["exp_avg", "exp_avg_sq"])
        np.savez(os.path.join(OUT, f"torch_{name}.npz"), **d)


def gen_sgd_family():
    steps = 5
    variants = {
        "sgd_plain": dict(momentum=0.0, dampening=0.0, nesterov=False, wd=0.0),
        "sgd_momentum": dict(momentum=0.9, dampening=0.0, nesterov=False, wd=0.0),
        "sgd_damp_wd": dict(momentum=0.9, dampening=0.1, nesterov=False, wd=0.01),
        "sgd_nesterov": dict(momentum=0.9, dampening=0.0, nesterov=True, wd=0.01),
    }
    for name, v in variants.items():
        def mk(ps, v=v):
            return torch.optim.SGD(
                [{"params": [p for p, d in zip(ps, DECAY) if d], "weight_decay": v["wd"]},
                 {"params": [p for p, d in zip(ps, DECAY) if not d], "weight_decay": 0.0}],
                lr=0.05, momentum=v["momentum"], dampening=v["dampening"],
                nesterov=v["nesterov"], foreach=False)
        keys = ["momentum_buffer"] if v["momentum"] else []
        d = _run_torch_opt(mk, 21, steps, keys)
        d["hp"] = np.array([0.05, v["momentum"], v["dampening"], v["wd"], float(v["nesterov"])])
        np.savez(os.path.join(OUT, f"torch_{name}.npz"), **d)


# ------------------------------------------------------------------------------------------
def _scaler_run(steps, inf_steps, growth_interval, init_scale=2.0 ** 16, tracker0=0):
    p = torch.nn.Parameter(torch.ones(4))
    opt = torch.optim.SGD([p], lr=0.0)
    sc = torch.amp.GradScaler("cpu", init_scale=init_scale, growth_factor=2.0,
                              backoff_factor=0.5, growth_interval=growth_interval)
    scales, trackers, skipped = [], [], []
    for s in range(1, steps + 1):
        loss = (p * 1.0).sum()
        sc.scale(loss).backward()
        if s == 1 and tracker0:
            sc._growth_tracker.fill_(tracker0)  # initialised by sc.scale() above
        if s in inf_steps:
            p.grad[1] = float("inf")
        sc.unscale_(opt)
        found = sum(v.item() for v in sc._found_inf_per_device(opt).values())
        sc.step(opt)
        sc.update()
        opt.zero_grad()
        scales.append(sc.get_scale())
        trackers.append(int(sc._growth_tracker.item()))
        skipped.append(int(found > 0))
    return (np.array(scales, np.float64), np.array(trackers, np.int32),
            np.array(skipped, np.int32))


def gen_scaler():
    out = {}
    # config-3 pattern: 200 steps, +inf on every 50th, growth every 2000 clean steps
    s, t, k = _scaler_run(200, {50, 100, 150, 200}, 2000)
    out.update(cfg3_scale=s, cfg3_tracker=t, cfg3_skipped=k)
    # growth and backoff interleaved with a short interval
    s, t, k = _scaler_run(14, {4, 5, 11}, 3)
    out.update(short_scale=s, short_tracker=t, short_skipped=k, short_inf=np.array([4, 5, 11]))
    # growth event forced by setting the tracker to 1999 (the ABI setter case)
    s, t, k = _scaler_run(3, set(), 2000, tracker0=1999)
    out.update(forced_scale=s, forced_tracker=t)
    np.savez(os.path.join(OUT, "torch_scaler.npz"), **out)


def gen_scaler_two_optimizers(steps=14, inf1=(4, 9), inf2=(5, 9, 12), interval=3):
    """GradScaler with two optimizers over two parameters: GradScaler.step(opt) for each,
    then one GradScaler.update() per iteration.  Each optimizer skips on its own overflow;
    the scale moves once, on the overflow of either (and grows after `interval` iterations
    in which neither overflowed)."""
    p1 = torch.nn.Parameter(torch.ones(4))
    p2 = torch.nn.Parameter(torch.ones(3))
    o1 = torch.optim.SGD([p1], lr=0.0)
    o2 = torch.optim.SGD([p2], lr=0.0)
    sc = torch.amp.GradScaler("cpu", init_scale=2.0 ** 16, growth_factor=2.0,
                              backoff_factor=0.5, growth_interval=interval)
    scales, trackers, skip1, skip2 = [], [], [], []
    for s in range(1, steps + 1):
        sc.scale(p1.sum() + p2.sum()).backward()
        if s in inf1:
            p1.grad[2] = float("inf")
        if s in inf2:
            p2.grad[0] = float("inf")
        sc.unscale_(o1)
        sc.unscale_(o2)
        f1 = sum(v.item() for v in sc._found_inf_per_device(o1).values())
        f2 = sum(v.item() for v in sc._found_inf_per_device(o2).values())
        sc.step(o1)
        sc.step(o2)
        sc.update()
        o1.zero_grad()
        o2.zero_grad()
        scales.append(sc.get_scale())
        trackers.append(int(sc._growth_tracker.item()))
        skip1.append(int(f1 > 0))
        skip2.append(int(f2 > 0))
    np.savez(os.path.join(OUT, "torch_scaler_two_opt.npz"),
             scale=np.array(scales, np.float64), tracker=np.array(trackers, np.int32),
             skip1=np.array(skip1, np.int32), skip2=np.array(skip2, np.int32),
             inf1=np.array(inf1), inf2=np.array(inf2), interval=np.array(interval))


def gen_clip():
    out = {}
    g = torch.Generator().manual_seed(5)
    for name, scale_, max_norm in (("big", 3.0, 1.0), ("small", 0.01, 1.0), ("mid", 1.0, 2.5)):
        grads = [torch.randn(*s, generator=g) * scale_ for s in SHAPES]
        ps = [torch.nn.Parameter(torch.zeros(*s)) for s in SHAPES]
        for p, gg in zip(ps, grads):
            p.grad = gg.clone()
        total = torch.nn.utils.clip_grad_norm_(ps, max_norm, foreach=False)
        out[f"{name}_grads"] = np.concatenate([f32(x).ravel() for x in grads])
        out[f"{name}_clipped"] = np.concatenate([f32(p.grad).ravel() for p in ps])
        out[f"{name}_norm"] = np.array(float(total), np.float64)
        out[f"{name}_max"] = np.array(max_norm, np.float64)
        out[f"{name}_fsum_norm"] = np.array(
            math.sqrt(math.fsum(float(v) ** 2 for x in grads for v in x.ravel().tolist())))
    np.savez(os.path.join(OUT, "torch_clip.npz"), **out)


# ------------------------------------------------------------------------------------------
def _adam_step_ref(weight, grad, lr, betas, eps, step, m, v):
    # closed form of tests/adam_optimizer.py:15-22
    beta1, beta2 = betas
    m = beta1 * m + (1.0 - beta1) * grad
    v = beta2 * v + (1.0 - beta2) * (grad * grad)
    m_hat = m / (1.0 - (beta1 ** step))
    v_hat = v / (1.0 - (beta2 ** step))
    weight = weight - lr * m_hat / (torch.sqrt(v_hat) + eps)
    return weight, m, v


def _linear_init(seed, n_in, n_out):
    # py/nn.py:_init_weight: torch.randn(in, out, dtype=bf16) * (1/sqrt(in)), after the test's
    # manual_seed and its x = torch.randn(32, 32)
    torch.manual_seed(seed)
    x = torch.randn(32, 32)
    w = torch.randn(n_in, n_out, dtype=torch.bfloat16) * (1.0 / math.sqrt(n_in))
    return x, w


def gen_reference_known_answers():
    out = {}
    # tests/adam_optimizer.py:25-50 — one step, grad_w = x^T @ ones
    x, w = _linear_init(31, 32, 32)
    w0 = w.to(torch.float32)
    grad = x.to(torch.float32).t() @ torch.ones(32, 32)
    w1, _, _ = _adam_step_ref(w0, grad, 0.1, (0.9, 0.999), 1e-8, 1,
                              torch.zeros_like(grad), torch.zeros_like(grad))
    out.update(adam1_w0=f32(w0), adam1_grad=f32(grad), adam1_w1=f32(w1))
    # tests/adam_optimizer.py:53-92 — two steps through tanh, grads recomputed from weights
    x, w = _linear_init(32, 32, 32)
    w_t = w.to(torch.float32)
    xf = x.to(torch.float32)

    def tanh_grad(weight):
        z = torch.tanh(xf @ weight)
        return xf.t() @ (torch.ones_like(z) * (1 - z * z))

    m = torch.zeros_like(w_t)
    v = torch.zeros_like(w_t)
    w1, m, v = _adam_step_ref(w_t, tanh_grad(w_t), 0.1, (0.9, 0.999), 1e-8, 1, m, v)
    w2, _, _ = _adam_step_ref(w1, tanh_grad(w1), 0.1, (0.9, 0.999), 1e-8, 2, m, v)
    out.update(adam2_x=f32(x), adam2_w0=f32(w_t), adam2_w2=f32(w2))
    # tests/sgd_optimizer.py:15-39 — bf16 `w0 - 0.1 * (x_b^T @ ones_b)`
    x, w = _linear_init(21, 32, 32)
    xb = x.to(torch.bfloat16)
    grad_b = xb.t() @ torch.ones(32, 32, dtype=torch.bfloat16)
    w_ref = w - 0.1 * grad_b
    out.update(sgd1_w0=bf16_bits(w), sgd1_grad=bf16_bits(grad_b), sgd1_w1=bf16_bits(w_ref))
    # tests/sgd_optimizer.py:42-78 — two bf16 steps through tanh, each `weight - 0.1 * grad_w`
    # with grad_w from the current weights; the gradients of both steps are kept so that a
    # step can be checked on its own inputs
    x, w = _linear_init(22, 32, 32)
    xb = x.to(torch.bfloat16)

    def bf16_tanh_grad(weight):
        z = torch.tanh(xb @ weight)
        return xb.transpose(-2, -1) @ (torch.ones_like(z) * (1 - z * z))

    g1 = bf16_tanh_grad(w)
    w1 = w - 0.1 * g1
    g2 = bf16_tanh_grad(w1)
    w2 = w1 - 0.1 * g2
    out.update(sgd2_w0=bf16_bits(w), sgd2_g1=bf16_bits(g1), sgd2_w1=bf16_bits(w1),
               sgd2_g2=bf16_bits(g2), sgd2_w2=bf16_bits(w2))
    # py/optim.py:19-21 itself on bf16 tensors: lr filled into a tensor of the gradient's dtype
    # (full_like, so lr rounds to bf16), then mul and sub, each result a bf16 tensor; on the
    # one-step fixture's weights and gradients
    w0 = torch.from_numpy(out["sgd1_w0"].view(np.int16)).view(torch.bfloat16)
    gb = torch.from_numpy(out["sgd1_grad"].view(np.int16)).view(torch.bfloat16)
    lr_tt = torch.full_like(gb, 0.1)
    out.update(sgd_pyopt_w1=bf16_bits(w0 - gb * lr_tt))
    np.savez(os.path.join(OUT, "reference_known_answers.npz"), **out)


if __name__ == "__main__":
    gen_bf16_special()
    gen_adam_family()
    gen_sgd_family()
    gen_scaler()
    gen_scaler_two_optimizers()
    gen_clip()
    gen_reference_known_answers()
    print("fixtures written to", OUT)
