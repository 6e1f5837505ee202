"""GPU tests of the optimizer-state checkpoint (ttp_save_state / ttp_load_state): a run that
is saved, loaded into a fresh context and continued ends bit-identical to the uninterrupted
run; malformed, mismatched and corrupted files are rejected."""
import struct

import numpy as np
import pytest

import oracle as O
from gpu_util import make_pair, torch_mod

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


def test_adamw_mixed_scaler_resume_is_bit_exact(tmp_path):
    from ttperf import _lib as L
    torch = torch_mod()
    a, _ = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=100)
    a.configure_scaler(True, init_scale=4096.0, growth_interval=3)
    gen = torch.Generator(device="cuda").manual_seed(101)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.05)
    grads = []
    scale = 4096.0
    reports_a = []
    for k in range(8):
        g = _grads(a, gen, 1e-2, scale=scale, inf_at=a.offsets[0] + 5 if k == 5 else None)
        grads.append(g)
        a.upload(L.BUF_GRAD, L.ALL_TENSORS, g)
        r = a.adam_step(report=True, **hp)
        reports_a.append(r)
        scale = r["scale"]
        if k == 3:
            a.save_state(tmp_path / "state.bin")
            saved = _all_state(a)
    b, _ = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=999)  # different weights: all replaced
    b.load_state(tmp_path / "state.bin")
    got = _all_state(b)
    for name in ("master", "exp_avg", "exp_avg_sq", "param"):
        assert np.array_equal(got[name], saved[name]), name
    assert b.step_count == reports_a[3]["step"]
    assert b.scaler_state() == (reports_a[3]["scale"], reports_a[3]["growth_tracker"])
    for k in range(4, 8):
        b.upload(L.BUF_GRAD, L.ALL_TENSORS, grads[k])
        r = b.adam_step(report=True, **hp)
        for key in ("found_inf", "skipped", "scale", "growth_tracker", "step", "clip_coef"):
            assert r[key] == reports_a[k][key], (k, key)
    fa, fb = _all_state(a), _all_state(b)
    for name in ("master", "exp_avg", "exp_avg_sq", "param"):
        assert np.array_equal(fa[name], fb[name]), name


def test_sgd_momentum_fp32_resume_keeps_momentum_init(tmp_path):
    """Tensor 3 never had a grad before the save: its momentum buffer is still
    uninitialised, and after the load its first momentum step must start from the gradient."""
    from ttperf import _lib as L
    torch = torch_mod()
    a, _ = make_pair(SHAPES, DECAY, O.MODE_FP32, seed=102)
    gen = torch.Generator(device="cuda").manual_seed(103)
    hp = dict(lr=1e-2, momentum=0.9, dampening=0.1, weight_decay=0.01)
    grads = [_grads(a, gen, 1e-1) for _ in range(6)]
    for k in range(6):
        a.upload(L.BUF_GRAD, L.ALL_TENSORS, grads[k])
        if k < 3:
            a.tensors[3].grad = None
        a.sgd_step(**hp)
        if k == 2:
            a.save_state(tmp_path / "sgd.bin")
    b, _ = make_pair(SHAPES, DECAY, O.MODE_FP32, seed=7)
    b.load_state(tmp_path / "sgd.bin")
    for k in range(3, 6):
        b.upload(L.BUF_GRAD, L.ALL_TENSORS, grads[k])
        b.sgd_step(**hp)
    fa, fb = _all_state(a), _all_state(b)
    for name in ("master", "momentum"):
        assert np.array_equal(fa[name], fb[name]), name
    assert a.step_count == b.step_count == 6


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
