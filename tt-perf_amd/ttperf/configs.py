"""Parameter tables of the benchmark configurations (tensor names, shapes, decay flags).

GPT-2 layout (tied LM head): wte, wpe, then per block ln_1 (w, b), attn.c_attn (w, b),
attn.c_proj (w, b), ln_2 (w, b), mlp.c_fc (w, b), mlp.c_proj (w, b), then ln_f (w, b).
Weight decay applies to the 2-D tensors only.
"""
from __future__ import annotations

import math


def gpt2_params(n_layer, d_model, vocab, ctx):
    d = d_model
    t = [("wte", (vocab, d)), ("wpe", (ctx, d))]
    for i in range(n_layer):
        h = f"h.{i}."
        t += [(h + "ln_1.weight", (d,)), (h + "ln_1.bias", (d,)),
              (h + "attn.c_attn.weight", (d, 3 * d)), (h + "attn.c_attn.bias", (3 * d,)),
              (h + "attn.c_proj.weight", (d, d)), (h + "attn.c_proj.bias", (d,)),
              (h + "ln_2.weight", (d,)), (h + "ln_2.bias", (d,)),
              (h + "mlp.c_fc.weight", (d, 4 * d)), (h + "mlp.c_fc.bias", (4 * d,)),
              (h + "mlp.c_proj.weight", (4 * d, d)), (h + "mlp.c_proj.bias", (d,))]
    t += [("ln_f.weight", (d,)), ("ln_f.bias", (d,))]
    return t


def mlp_params():
    # config 1: W1[64,128], b1[128], W2[128,10], b2[10] (the [in, out] layout of py/nn.py:36)
    return [("W1", (64, 128)), ("b1", (128,)), ("W2", (128, 10)), ("b2", (10,))]


CONFIGS = {
    "mlp": dict(params=mlp_params, mode="fp32"),
    "nanogpt_char": dict(params=lambda: gpt2_params(6, 384, 65, 256), mode="mixed"),
    "gpt2_124m": dict(params=lambda: gpt2_params(12, 768, 50257, 1024), mode="mixed"),
    "gpt2_774m": dict(params=lambda: gpt2_params(36, 1280, 50257, 1024), mode="mixed"),
    "gpt2_1558m": dict(params=lambda: gpt2_params(48, 1600, 50257, 1024), mode="fp32"),
}


# one GPU's share of a data-parallel, ZeRO-1-sharded step: (configuration, shards, index).
# The last of 8 GPT-2 124M shards: 28 ragged pieces of the last three blocks and ln_f.
SHARDS = {"gpt2_124m_shard8": ("gpt2_124m", 8, 7)}


def mode(name):
    """Precision mode of a configuration (a shard has its configuration's)."""
    return CONFIGS[SHARDS[name][0] if name in SHARDS else name]["mode"]


def table(name):
    """(names, shapes, decay flags, numels) of a configuration."""
    if name in SHARDS:
        return shard_table(*SHARDS[name])
    entries = CONFIGS[name]["params"]()
    names = [n for n, _ in entries]
    shapes = [s for _, s in entries]
    decay = [len(s) >= 2 for s in shapes]
    numels = [int(math.prod(s)) for s in shapes]
    return names, shapes, decay, numels


def shard_table(name, n_shards, k, align=64):
    """Shard k of n_shards of a configuration's flat store, as a ZeRO-1 optimizer shard would
    own it: the contiguous element range [k*S, (k+1)*S) of the 64-element-aligned flat layout
    (S rounded up to a multiple of `align`, so state records stay whole), expressed as a table
    of 1-D pieces of the tensors it covers, each keeping its tensor's decay flag."""
    names, _, decay, numels = table(name)
    offsets, total = [], 0
    for n in numels:
        offsets.append(total)
        total += (n + align - 1) // align * align
    per = (total + n_shards - 1) // n_shards
    per = (per + align - 1) // align * align
    lo, hi = k * per, min(total, (k + 1) * per)
    out_names, out_shapes, out_decay, out_numels = [], [], [], []
    for nm, d, o, n in zip(names, decay, offsets, numels):
        a, b = max(o, lo), min(o + n, hi)
        if a < b:
            out_names.append(f"{nm}[{a - o}:{b - o}]")
            out_shapes.append((b - a,))
            out_decay.append(d)
            out_numels.append(b - a)
    return out_names, out_shapes, out_decay, out_numels
