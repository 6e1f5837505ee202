"""GPU tests of the optimizer-state checkpoint (ttp_save_state / ttp_load_state): a run that
is saved, loaded into a fresh context and continued matches the oracle at every step (the
oracle restored from its own snapshot at the save) and ends bit-identical to the
uninterrupted run; the saved buffers, parsed at the offsets the format documents, equal the
store's; files move between the SGD and the default layout of a mixed store; malformed,
mismatched and corrupted files are rejected."""
import struct

import numpy as np
import pytest

import oracle as O
from gpu_util import compare_state, make_pair, torch_mod

pytestmark = pytest.mark.gpu

SHAPES = [(300, 7), (64,), (129, 33), (5,), (2048,), (1, 2049), (4097,)]
DECAY = [True, False, True, False, False, True, False]


def _grads(store, gen, std, scale=1.0, inf_at=None):
    import torch
    from ttperf import _lib as L
    g = torch.randn(store.total, generator=gen, device="cuda") * std * scale
    if inf_at is not None:
        g[inf_at] = float("inf")
    if store.mode == L.MODE_MIXED:
        g = g.to(torch.bfloat16)
    return g


def _all_state(store):
    from ttperf import _lib as L
    out = {}
    for name, buf in (("master", L.BUF_MASTER), ("exp_avg", L.BUF_EXP_AVG),
                      ("exp_avg_sq", L.BUF_EXP_AVG_SQ), ("param", L.BUF_PARAM),
                      ("momentum", L.BUF_MOMENTUM)):
        a = store.download(buf)
        out[name] = a.view(np.uint32) if a.dtype == np.float32 else a
    return out


def _host(g):
    """The host copy of device gradients, in the oracle's types (bf16 bits or float32)."""
    import torch
    if g.dtype == torch.bfloat16:
        return g.cpu().view(torch.int16).numpy().view(np.uint16)
    return g.cpu().numpy()


ORACLE_STATE = ("master", "param", "exp_avg", "exp_avg_sq", "momentum", "mom_init")


def _snapshot(ref):
    return dict({k: getattr(ref, k).copy() for k in ORACLE_STATE}, t=ref.t, scale=ref.scale,
                tracker=ref.growth_tracker)


def _restore(ref, snap):
    for k in ORACLE_STATE:
        getattr(ref, k)[:] = snap[k]
    ref.t = snap["t"]
    ref.set_scaler_state(snap["scale"], snap["tracker"])


def _file_buffers(path, n_tensors, total):
    """The fp32 buffers of a state file, read at the offsets the format in ttperf.h gives: an
    80-byte header (buffer mask at byte 20, total at 24, t at 32), n_tensors 16-byte tensor
    records, then each present buffer (bit 1 master, 2 exp_avg, 4 exp_avg_sq, 8 momentum, in
    that order) as `total` fp32 values, then the 8-byte checksum."""
    raw = path.read_bytes()
    mask, = struct.unpack_from("<I", raw, 20)
    assert struct.unpack_from("<I", raw, 16)[0] == n_tensors
    assert struct.unpack_from("<Q", raw, 24)[0] == total
    t, = struct.unpack_from("<Q", raw, 32)
    off = 80 + 16 * n_tensors
    out = {}
    for bit, name in ((1, "master"), (2, "exp_avg"), (4, "exp_avg_sq"), (8, "momentum")):
        if mask & bit:
            out[name] = np.frombuffer(raw, np.uint32, total, off)
            off += 4 * total
    assert off + 8 == len(raw)
    return out, t


def _check_file_against_store(path, store):
    """Every buffer of the file equals the store's download of it, bit for bit: a swapped
    buffer order in save or load cannot pass."""
    from ttperf import _lib as L
    bufs, t = _file_buffers(path, len(store.tensors), store.total)
    ids = {"master": L.BUF_MASTER, "exp_avg": L.BUF_EXP_AVG, "exp_avg_sq": L.BUF_EXP_AVG_SQ,
           "momentum": L.BUF_MOMENTUM}
    for name, data in bufs.items():
        assert np.array_equal(data, store.download(ids[name]).view(np.uint32)), name
    assert t == store.step_count
    return set(bufs)


def test_adamw_mixed_scaler_resume_matches_the_oracle(tmp_path):
    """Mixed AdamW with loss scaling (an overflow at step 5) and clipping, saved after step 3:
    every step of the run and of its resumed continuation in a fresh context is compared with
    the oracle (the resumed oracle restored from its own snapshot at the save), and the saved
    file's buffers, parsed at their documented offsets, equal the store's."""
    from ttperf import _lib as L
    torch = torch_mod()
    a, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=100)
    a.configure_scaler(True, init_scale=4096.0, growth_interval=3)
    ref.configure_scaler(True, 4096.0, growth_interval=3)
    gen = torch.Generator(device="cuda").manual_seed(101)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.05)
    grads, reports_a = [], []
    for k in range(8):
        g = _grads(a, gen, 1e-2, scale=ref.scale, inf_at=a.offsets[0] + 5 if k == 5 else None)
        grads.append(g)
        a.upload(L.BUF_GRAD, L.ALL_TENSORS, g)
        ref.grad[:] = _host(g)
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        r = a.adam_step(report=True, **hp)
        e = ref.adam_step(**hp)
        for key in ("found_inf", "skipped", "scale", "growth_tracker", "step"):
            assert r[key] == e[key], (k, key)
        compare_state(a, ref, max_ulp=2)
        reports_a.append(r)
        if k == 3:
            a.save_state(tmp_path / "state.bin")
            saved = _snapshot(ref)
            assert _check_file_against_store(tmp_path / "state.bin", a) == \
                {"master", "exp_avg", "exp_avg_sq"}
    assert reports_a[5]["skipped"] == 1
    b, ref_b = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=999)  # different weights: replaced
    b.load_state(tmp_path / "state.bin")
    ref_b.configure_scaler(True, 4096.0, growth_interval=3)
    _restore(ref_b, saved)
    compare_state(b, ref_b, max_ulp=0)
    assert b.step_count == ref_b.t == reports_a[3]["step"]
    assert b.scaler_state() == (np.float32(ref_b.scale), ref_b.growth_tracker)
    for k in range(4, 8):
        b.upload(L.BUF_GRAD, L.ALL_TENSORS, grads[k])
        ref_b.grad[:] = _host(grads[k])
        for i in range(ref_b.n):
            ref_b.set_has_grad(i, True)
        r = b.adam_step(report=True, **hp)
        e = ref_b.adam_step(**hp)
        for key in ("found_inf", "skipped", "scale", "growth_tracker", "step", "clip_coef"):
            assert r[key] == reports_a[k][key], (k, key)
            assert key == "clip_coef" or r[key] == e[key], (k, key)
        compare_state(b, ref_b, max_ulp=2)
    fa, fb = _all_state(a), _all_state(b)
    for name in ("master", "exp_avg", "exp_avg_sq", "param"):
        assert np.array_equal(fa[name], fb[name]), name


def test_sgd_momentum_fp32_resume_keeps_momentum_init(tmp_path):
    """Tensor 3 never had a grad before the save: its momentum buffer is still
    uninitialised, and after the load its first momentum step must start from the gradient.
    The run and its continuation are compared with the oracle at every step."""
    from ttperf import _lib as L
    torch = torch_mod()
    a, ref = make_pair(SHAPES, DECAY, O.MODE_FP32, seed=102)
    gen = torch.Generator(device="cuda").manual_seed(103)
    hp = dict(lr=1e-2, momentum=0.9, dampening=0.1, weight_decay=0.01)
    grads = [_grads(a, gen, 1e-1) for _ in range(6)]

    def step(store, oracle, k):
        store.upload(L.BUF_GRAD, L.ALL_TENSORS, grads[k])
        oracle.grad[:] = _host(grads[k])
        for i in range(oracle.n):
            oracle.set_has_grad(i, True)
        if k < 3:
            store.tensors[3].grad = None
            oracle.set_has_grad(3, False)
        store.sgd_step(**hp)
        oracle.sgd_step(**hp)
        compare_state(store, oracle, which=("master", "momentum"), max_ulp=0)

    for k in range(3):
        step(a, ref, k)
    a.save_state(tmp_path / "sgd.bin")
    saved = _snapshot(ref)
    assert _check_file_against_store(tmp_path / "sgd.bin", a) == {"master", "momentum"}
    for k in range(3, 6):
        step(a, ref, k)
    b, ref_b = make_pair(SHAPES, DECAY, O.MODE_FP32, seed=7)
    b.load_state(tmp_path / "sgd.bin")
    _restore(ref_b, saved)
    assert not ref_b.mom_init[3]
    for k in range(3, 6):
        step(b, ref_b, k)
    fa, fb = _all_state(a), _all_state(b)
    for name in ("master", "momentum"):
        assert np.array_equal(fa[name], fb[name]), name
    assert a.step_count == b.step_count == 6


def test_sgd_layout_checkpoints_load_into_either_layout(tmp_path):
    """The file format does not depend on the layout.  A mixed store in the SGD layout,
    stepped by SGD with momentum and loss scaling, saves master and momentum only; the file
    loads into a store in the SGD layout and into one in the default layout, and both continue
    with the oracle.  A default-layout store's Adam file (master, m, v) loads into an
    SGD-layout store by converting it first."""
    from ttperf import _lib as L
    torch = torch_mod()
    a, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=110, layout="sgd")
    a.configure_scaler(True, init_scale=1024.0, growth_interval=2)
    ref.configure_scaler(True, 1024.0, growth_interval=2)
    gen = torch.Generator(device="cuda").manual_seed(111)
    hp = dict(lr=1e-2, momentum=0.9, nesterov=True, max_grad_norm=1.0)

    def step(store, oracle, g):
        store.upload(L.BUF_GRAD, L.ALL_TENSORS, g)
        oracle.grad[:] = _host(g)
        for i in range(oracle.n):
            oracle.set_has_grad(i, True)
        r = store.sgd_step(report=True, **hp)
        e = oracle.sgd_step(**hp)
        assert (r["skipped"], r["scale"], r["step"]) == (e["skipped"], e["scale"], e["step"])
        compare_state(store, oracle, which=("master", "param", "momentum"), max_ulp=2)

    for k in range(4):
        step(a, ref, _grads(a, gen, 1e-2, scale=ref.scale, inf_at=7 if k == 2 else None))
    assert a.sgd_layout
    a.save_state(tmp_path / "sgd_layout.bin")
    saved = _snapshot(ref)
    assert _check_file_against_store(tmp_path / "sgd_layout.bin", a) == {"master", "momentum"}
    later = [_grads(a, gen, 1e-2, scale=ref.scale) for _ in range(2)]
    for layout in ("sgd", "default"):
        b, ref_b = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=5, layout=layout)
        b.load_state(tmp_path / "sgd_layout.bin")
        ref_b.configure_scaler(True, 1024.0, growth_interval=2)
        _restore(ref_b, saved)
        assert b.sgd_layout == (layout == "sgd")
        which = ("master", "param", "momentum") + (("exp_avg", "exp_avg_sq") if layout ==
                                                   "default" else ())
        compare_state(b, ref_b, which=which, max_ulp=0)
        for g in later:
            step(b, ref_b, g)
        b.close()
    # an Adam file into an SGD-layout store: the load converts it (m and v from the file)
    c, ref_c = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=112)
    adam = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    for _ in range(2):
        g = _grads(c, gen, 1e-2)
        c.upload(L.BUF_GRAD, L.ALL_TENSORS, g)
        ref_c.grad[:] = _host(g)
        for i in range(ref_c.n):
            ref_c.set_has_grad(i, True)
        c.adam_step(**adam)
        ref_c.adam_step(**adam)
    c.save_state(tmp_path / "adam.bin")
    d, _ = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=6, layout="sgd")
    d.load_state(tmp_path / "adam.bin")
    assert not d.sgd_layout
    compare_state(d, ref_c, max_ulp=0)
    g = _grads(c, gen, 1e-2)
    d.upload(L.BUF_GRAD, L.ALL_TENSORS, g)
    ref_c.grad[:] = _host(g)
    d.adam_step(**adam)
    ref_c.adam_step(**adam)
    compare_state(d, ref_c, max_ulp=2)


def test_load_rejects_mismatch_and_corruption(tmp_path):
    import ttperf
    from ttperf import _lib as L
    a = ttperf.ParamStore([(100,), (64, 8)], mode="mixed")
    a.tensors[0].grad = np.zeros(100, np.uint16)
    a.adam_step(lr=1e-3)
    path = tmp_path / "s.bin"
    a.save_state(path)
    raw = path.read_bytes()
    master = a.download(L.BUF_MASTER).view(np.uint32).copy()

    def snapshot(store):
        bufs = [L.BUF_MASTER, L.BUF_PARAM, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ]
        return ([store.download(b).tobytes() for b in bufs], store.step_count,
                store.scaler_state())

    def expect_invalid(store, p, what):
        before = snapshot(store)
        with pytest.raises(ttperf.TTPValueError) as e:
            store.load_state(p)
        assert what in str(e.value), str(e.value)
        # the whole file is checked before the store is touched
        assert snapshot(store) == before, f"a rejected load ({what}) changed the store"

    expect_invalid(ttperf.ParamStore([(100,), (64, 9)], mode="mixed"), path, "tensor")
    expect_invalid(ttperf.ParamStore([(100,), (64, 8)], mode="fp32"), path, "mode")
    expect_invalid(ttperf.ParamStore([(100,), (64, 8)], mode="mixed", decay=[True, True]),
                   path, "flags")
    bad = bytearray(raw)
    bad[len(bad) // 2] ^= 0x40
    (tmp_path / "bad.bin").write_bytes(bytes(bad))
    expect_invalid(a, tmp_path / "bad.bin", "checksum")
    bad = bytearray(raw)
    bad[-9] ^= 0x01  # the last data byte, read after every buffer before it
    (tmp_path / "bad_end.bin").write_bytes(bytes(bad))
    expect_invalid(a, tmp_path / "bad_end.bin", "checksum")
    (tmp_path / "short.bin").write_bytes(raw[:-100])
    expect_invalid(a, tmp_path / "short.bin", "truncated")
    (tmp_path / "long.bin").write_bytes(raw + b"\0" * 8)
    expect_invalid(a, tmp_path / "long.bin", "trailing")
    (tmp_path / "junk.bin").write_bytes(b"not a state file at all" * 4)
    expect_invalid(a, tmp_path / "junk.bin", "not an optimizer-state file")
    expect_invalid(a, tmp_path / "missing.bin", "cannot open")
    # a well-formed file whose loss-scaler fields are out of range is refused, before the
    # store is touched.  The file is re-signed with the format's checksum: a 64-bit
    # multiply-xor hash over the 8-byte little-endian words of everything before it (for a
    # store this small every hashed piece is whole words), then a final avalanche.
    def resign(body):
        m = (1 << 64) - 1
        h = 0xcbf29ce484222325
        for (w,) in struct.iter_unpack("<Q", body):
            h = ((h ^ w) * 0x100000001b3) & m
            h ^= h >> 29
        h ^= h >> 33
        h = (h * 0xff51afd7ed558ccd) & m
        h ^= h >> 33
        return body + struct.pack("<Q", h)

    assert len(raw) % 8 == 0 and resign(raw[:-8]) == raw, "the checksum restatement"
    scaled = ttperf.ParamStore([(100,), (64, 8)], mode="mixed")
    scaled.configure_scaler(True, init_scale=1024.0, growth_interval=3)
    scaled.save_state(tmp_path / "scaled.bin")
    good = (tmp_path / "scaled.bin").read_bytes()
    assert resign(good[:-8]) == good
    # header: magic[8], u32 version/mode/n_tensors/buffers, u64 total/t, f32 scale,
    # i32 growth_tracker/scaler_enabled/growth_interval, f64 init_scale/growth/backoff
    for off, fmt, value, what in ((52, "<i", 0, "loss-scaler settings"),
                                  (72, "<d", 1.5, "loss-scaler settings"),
                                  (40, "<f", -1.0, "loss scale"),
                                  (44, "<i", -2, "growth tracker")):
        bad = bytearray(good[:-8])
        struct.pack_into(fmt, bad, off, value)
        (tmp_path / "bad_scaler.bin").write_bytes(resign(bytes(bad)))
        expect_invalid(a, tmp_path / "bad_scaler.bin", what)
    scaled.close()
    # a save goes through path.tmp: none is left behind, and a failed rename removes it
    assert not (tmp_path / "s.bin.tmp").exists()
    (tmp_path / "adir").mkdir()
    with pytest.raises(ttperf.TTPValueError) as e:
        a.save_state(tmp_path / "adir")
    assert "rename" in str(e.value)
    assert not (tmp_path / "adir.tmp").exists() and (tmp_path / "adir").is_dir()
    # a good load after the failures restores a consistent state
    fresh = ttperf.ParamStore([(100,), (64, 8)], mode="mixed")
    fresh.load_state(path)
    assert np.array_equal(fresh.download(L.BUF_MASTER).view(np.uint32), master)
    assert fresh.step_count == 1
