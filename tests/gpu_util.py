"""Helpers of the GPU parity tests: a libttperf_hip store and an oracle store with the same
layout and the same seeded inputs, gradients generated on the device by torch and copied to
the host for the oracle, and bit-level comparisons."""
import os
import sys

import numpy as np

import oracle as O
from conftest import REPO, f32_ulp_diff

sys.path.insert(0, os.path.join(REPO, "tt-perf_amd"))


def torch_mod():
    import torch
    return torch


def make_pair(shapes, decay, mode, init_std=0.02, seed=0, init="normal", layout="default"):
    """GPU store + oracle store holding identical fp32 master weights (a BF16 store: identical
    bf16 weights, the seeded values rounded to nearest even).  layout="sgd": a mixed store in
    the SGD layout (contiguous master, no m / v until an Adam step converts it)."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    store = ttperf.ParamStore(shapes, mode={O.MODE_MIXED: "mixed", O.MODE_FP32: "fp32",
                                            O.MODE_BF16: "bf16"}[mode],
                              decay=decay, layout=layout)
    store.set_stream(torch.cuda.current_stream())
    numels = [t.numel for t in store.tensors]
    ref = O.OracleStore(numels, flags=[1 if d else 0 for d in decay], mode=mode,
                        nthreads=min(16, os.cpu_count() or 1))
    assert [int(o) for o in ref.offsets] == list(store.offsets)
    assert ref.total == store.total
    g = torch.Generator(device="cuda").manual_seed(seed)
    flat = torch.zeros(store.total, dtype=torch.float32, device="cuda")
    for i, (t, s) in enumerate(zip(store.tensors, shapes)):
        o = store.offsets[i]
        if init == "uniform":  # U(-1/sqrt(fan_in), 1/sqrt(fan_in)), fan_in = first dim
            b = 1.0 / np.sqrt(s[0])
            flat[o:o + t.numel].uniform_(-b, b, generator=g)
        elif len(s) >= 2:
            flat[o:o + t.numel].normal_(0.0, init_std, generator=g)
        elif "ln" in t.name and t.name.endswith("weight"):
            flat[o:o + t.numel].fill_(1.0)
        else:
            flat[o:o + t.numel].normal_(0.0, init_std, generator=g)
    if mode == O.MODE_BF16:
        w = flat.to(torch.bfloat16)
        store.upload(L.BUF_PARAM, L.ALL_TENSORS, w)
        ref.param[:store.total] = w.view(torch.int16).cpu().numpy().view(np.uint16)
        return store, ref
    store.upload(L.BUF_MASTER, L.ALL_TENSORS, flat)
    # the oracle's arrays hold at least one element (an all-empty table has total 0)
    ref.master[:store.total] = flat.cpu().numpy()
    if mode == O.MODE_MIXED:
        ref.param[:] = O.bf16_rne(ref.master)
    return store, ref


def pad_mask(store):
    m = np.zeros(store.total, dtype=bool)
    for i, t in enumerate(store.tensors):
        m[store.offsets[i]:store.offsets[i] + t.numel] = True
    return m


def device_grads(store, gen, std, scale=1.0, heavy_frac=0.0, heavy_std=1.0, inf_at=None,
                 into=None):
    """Seeded N(0, std) * scale grads on the device (bf16 in MIXED and BF16), written into the store;
    returns the host copy (uint16 bits or float32) for the oracle.  into: an oracle's grad
    array, which receives the copy directly (no host temporary of the store's size, which at
    billions of elements costs more than the step under test); its first store.total elements
    are returned."""
    torch = torch_mod()
    g = torch.randn(store.total, generator=gen, device="cuda", dtype=torch.float32) * std
    if heavy_frac:
        pick = torch.rand(store.total, generator=gen, device="cuda") < heavy_frac
        g = torch.where(pick, torch.randn(store.total, generator=gen, device="cuda") * heavy_std, g)
    if scale != 1.0:
        g = g * scale
    if inf_at is not None:
        g[inf_at] = float("inf")
    from ttperf import _lib as L
    if store.mode != L.MODE_FP32:
        g = g.to(torch.bfloat16)
    store.upload(L.BUF_GRAD, L.ALL_TENSORS, g)
    if into is not None:
        bits = store.mode != L.MODE_FP32
        assert into.dtype == (np.uint16 if bits else np.float32) and len(into) >= store.total
        dst = torch.from_numpy(into.view(np.int16) if bits else into)[:store.total]
        dst.copy_(g.view(torch.int16) if bits else g)
        return into[:store.total]
    host = g.cpu()
    if store.mode != L.MODE_FP32:
        return host.view(torch.int16).numpy().view(np.uint16)
    return host.numpy()


def compare_state(store, ref, which=("master", "exp_avg", "exp_avg_sq", "param"), max_ulp=0,
                  mask=None, slice_elems=1 << 25):
    """Max ulp difference per buffer (padding excluded), compared in slices so that
    billion-element stores do not need several full-size temporaries; asserts <= max_ulp,
    and bf16 params bit-exact."""
    from ttperf import _lib as L
    bufs = {"master": L.BUF_MASTER, "exp_avg": L.BUF_EXP_AVG, "exp_avg_sq": L.BUF_EXP_AVG_SQ,
            "param": L.BUF_PARAM, "momentum": L.BUF_MOMENTUM}
    out = {}
    if mask is None:
        mask = pad_mask(store)
    for name in which:
        got = store.download(bufs[name])
        want = getattr(ref, name)
        worst, nbad = 0, 0
        for a in range(0, store.total, slice_elems):
            b = min(store.total, a + slice_elems)
            # a bit-identical slice (padding included) has no difference to count: the ulp
            # arithmetic below costs about 100 times more and runs only where bits differ
            if np.array_equal(got[a:b].view(np.uint8), want[a:b].view(np.uint8)):
                continue
            m = mask[a:b]
            if got.dtype == np.uint16:
                nbad += int(np.count_nonzero((got[a:b] != want[a:b]) & m))
            else:
                d = f32_ulp_diff(got[a:b][m], want[a:b][m])
                if d.size:
                    worst = max(worst, int(d.max()))
                    nbad += int(np.count_nonzero(d))
        out[name] = nbad if got.dtype == np.uint16 else worst
        print(f"  compare {name} ({store.total} elements): "
              + (f"{nbad} bf16 values differ" if got.dtype == np.uint16
                 else f"max {worst} ulp, {nbad} values differ"), flush=True)
        if got.dtype == np.uint16:
            assert nbad == 0, f"{name}: {nbad} bf16 values differ"
        else:
            assert worst <= max_ulp, f"{name}: max {worst} ulp (> {max_ulp}), {nbad} values differ"
        del got
    return out
