"""GPU tests of the state-record layout: the fp32 optimizer state (MIXED: master, m, v; FP32:
m, v) is stored in records of 64-element slots, and the C ABI converts on upload, download and
checkpoint.

The addressing that ttp_buffer_layout documents is checked against raw device memory read
with hipMemcpy (HIP runtime, not engine code), so a wrong record index in the engine cannot
cancel out between the update kernel and the engine's own gather.  Round trips cover per-tensor
and flat transfers, host and device memory, ragged tensors, and host transfers longer than one
staging piece (16 Mi elements).
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from gpu_util import compare_state, device_grads, make_pair, torch_mod

pytestmark = pytest.mark.gpu

SHAPES = [(1,), (63,), (65,), (7, 9), (130,), (64, 64), (3,)]
DECAY = [False, False, False, True, False, True, False]


def _hip():
    torch_mod()  # torch first: one HIP runtime per process (the one torch loaded)
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.restype = C.c_int
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    return hip


def _raw_f32(addr, count):
    """count fp32 values at device address addr, copied by hipMemcpy (device to host)."""
    torch = torch_mod()
    torch.cuda.synchronize()
    out = np.empty(count, np.float32)
    assert _hip().hipMemcpy(out.ctypes.data, addr, count * 4, 2) == 0
    return out


def _stepped_pair(mode, seed):
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, mode, seed=seed)
    gen = torch.Generator(device="cuda").manual_seed(seed + 1)
    hp = dict(lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    for _ in range(2):
        g = device_grads(store, gen, 1e-2)
        ref.grad[:] = g
        for i in range(len(SHAPES)):
            ref.set_has_grad(i, True)
        store.adam_step(**hp)
        ref.adam_step(**hp)
    return store, ref


@pytest.mark.parametrize("mode", [O.MODE_MIXED, O.MODE_FP32])
def test_layout_matches_raw_device_memory(mode):
    from ttperf import _lib as L
    store, ref = _stepped_pair(mode, seed=11)
    compare_state(store, ref, max_ulp=0)
    mixed = mode == O.MODE_MIXED
    want = {L.BUF_MASTER: (64, 192) if mixed else (64, 64),
            L.BUF_EXP_AVG: (64, 192) if mixed else (64, 128),
            L.BUF_EXP_AVG_SQ: (64, 192) if mixed else (64, 128)}
    bases = {}
    for which, (group, stride) in want.items():
        base, g, s = store.layout(which)
        assert (g, s) == (group, stride), (which, g, s)
        bases[which] = base
        nrec = store.total // group
        raw = _raw_f32(base, (nrec - 1) * stride + group)
        e = np.arange(store.total)
        laid = raw[(e // group) * stride + e % group]
        got = store.download(which)
        assert np.array_equal(laid.view(np.uint32), got.view(np.uint32)), which
        print(f"  layout of buffer {which}: group {g}, stride {s}, {store.total} elements "
              "match raw device memory", flush=True)
    # the slots of one record array: m follows master (MIXED) by one slot, v follows m
    if mixed:
        assert bases[L.BUF_EXP_AVG] - bases[L.BUF_MASTER] == 64 * 4
    assert bases[L.BUF_EXP_AVG_SQ] - bases[L.BUF_EXP_AVG] == 64 * 4
    # contiguous buffers keep their pointers; interleaved ones refuse
    import ttperf
    for which in (L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ) + ((L.BUF_MASTER,) if mixed else ()):
        with pytest.raises(ttperf.TTPError) as e:
            store.ptr(which, 0)
        assert e.value.code == L.ERR_STATE and "ttp_buffer_layout" in str(e.value)
    for which in (L.BUF_PARAM, L.BUF_GRAD, L.BUF_MOMENTUM):
        base, g, s = store.layout(which)
        assert g == s == 64 and store.ptr(which) == base
        assert store.ptr(which, 3) == base + store.offsets[3] * store._esize(which)
    if not mixed:
        assert store.ptr(L.BUF_MASTER) == store.ptr(L.BUF_PARAM)
    store.close()


@pytest.mark.parametrize("mode", [O.MODE_MIXED, O.MODE_FP32])
def test_state_round_trips(mode):
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = _stepped_pair(mode, seed=12)
    rng = np.random.default_rng(5)
    before = {w: store.download(w) for w in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ,
                                             L.BUF_PARAM)}
    # per tensor, host source: only that tensor's slots change
    for which in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ):
        k = 4
        n = store.tensors[k].numel
        vals = rng.normal(0, 1, n).astype(np.float32)
        store.upload(which, k, vals)
        assert np.array_equal(store.download(which, k).view(np.uint32), vals.view(np.uint32))
        flat = store.download(which)
        o = store.offsets[k]
        expect = before[which].copy()
        expect[o:o + n] = vals
        assert np.array_equal(flat.view(np.uint32), expect.view(np.uint32)), which
        before[which] = flat
        if which == L.BUF_MASTER and mode == O.MODE_MIXED:
            p16 = store.download(L.BUF_PARAM, k)
            assert np.array_equal(p16, O.bf16_rne(vals))
    # flat, device source and device destination
    for which in (L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ, L.BUF_MASTER):
        src = torch.randn(store.total, device="cuda")
        store.upload(which, L.ALL_TENSORS, src)
        back = torch.empty(store.total, device="cuda")
        store.download(which, L.ALL_TENSORS, out=back)
        torch.cuda.synchronize()
        assert torch.equal(back.view(torch.int32), src.view(torch.int32)), which
    if mode == O.MODE_MIXED:
        # a bf16 PARAM upload widens into the master slots
        p = torch.randn(store.total, device="cuda").to(torch.bfloat16)
        store.upload(L.BUF_PARAM, L.ALL_TENSORS, p)
        m = store.download(L.BUF_MASTER)
        want = (p.float().cpu().numpy())
        assert np.array_equal(m.view(np.uint32), want.view(np.uint32))
    store.close()


def test_host_transfers_longer_than_one_staging_piece():
    """20.5 Mi elements: host uploads and downloads of record-stored state run in two pieces."""
    import ttperf
    from ttperf import _lib as L
    shapes = [(5000, 4100), (77,)]
    store = ttperf.ParamStore(shapes, mode="mixed", decay=[True, False])
    rng = np.random.default_rng(9)
    for which in (L.BUF_MASTER, L.BUF_EXP_AVG_SQ):
        vals = rng.normal(0, 1, store.total).astype(np.float32)
        store.upload(which, L.ALL_TENSORS, vals)
        got = store.download(which)
        assert np.array_equal(got.view(np.uint32), vals.view(np.uint32)), which
        one = store.download(which, 0)
        assert np.array_equal(one.view(np.uint32), vals[:5000 * 4100].view(np.uint32))
    assert np.array_equal(store.download(L.BUF_PARAM),
                          O.bf16_rne(store.download(L.BUF_MASTER)))
    store.close()
