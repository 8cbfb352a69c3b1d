"""The reference's engine test idiom (tests/test_hybrid_rust.py:103-226, op list of main.rs:745-776):
drive the stack with a list of feed / snapshot / crop operations of mixed sizes — single tokens,
odd prefill lengths, a feed that crosses the 64-token chunk boundary, decode after a crop — and
compare every position's output with the oracle composite fed the same operations (its cache
restored from a copy at the snapshot). Same reduced shape as test_stack_gpu.py.

Bar: as in test_stack_gpu.py, twice the floor that bf16 rounding directions put under the
comparison, measured per feed by running the oracle a second time (its own cache and snapshots)
on inputs moved by at most 2^-20 of themselves. Measured: floor ~1e-3 to 3e-3, the GPU's distance
1.3e-3 to 4.3e-3; a single-token feed right after the first short prefill sits near 1e-3."""
import copy

import pytest
import torch

from conftest import perturb, rel_err, rms_err
from oracle import mixer_ref as R

from aegist_mixer import ops

from test_stack_gpu import CFG, KINDS, check_stack_feed, make_layers

pytestmark = pytest.mark.gpu

OPS = [("feed", 5), ("feed", 30), ("snapshot",), ("feed", 100), ("feed", 1), ("feed", 1), ("crop", 50),
       ("feed", 64), ("feed", 1), ("snapshot",), ("feed", 3), ("crop", 120), ("feed", 1)]


def _fresh_cache(B, cap):
    c = CFG
    C = 2 * c["hk"] * 128 + c["hv"] * 128
    nd, na = KINDS.count("delta"), KINDS.count("attn")
    return {"length": 0,
            "conv": [torch.zeros(B, C, 3) for _ in range(nd)],
            "state": [torch.zeros(B, c["hv"], 128, 128) for _ in range(nd)],
            "k": [torch.zeros(B, c["n_kv"], cap, 256, dtype=torch.bfloat16) for _ in range(na)],
            "v": [torch.zeros(B, c["n_kv"], cap, 256, dtype=torch.bfloat16) for _ in range(na)]}


@pytest.mark.parametrize("B", [1, 2])
def test_stack_op_list_every_position(dev, B):
    cap = 256
    layers, dl = make_layers(3, dev)
    stack = ops.HybridStack(CFG, KINDS, dl, max_batch=B, max_tokens=B * 128, max_context=cap)
    cache, cache_p = _fresh_cache(B, cap), _fresh_cache(B, cap)
    snaps = []  # oracle copies (plain, perturbed) at each snapshot, newest last (the stack keeps two slots)
    g_ = torch.Generator().manual_seed(11)
    for i, op in enumerate(OPS):
        print(f"op {i}: {op}", flush=True)
        if op[0] == "feed":
            x = torch.randn(B, op[1], CFG["d_model"], generator=g_)
            ref = R.hybrid_stack_forward(x.clone(), layers, KINDS, cache, CFG)
            xp = perturb(x, 300 + i)
            ref_p = R.hybrid_stack_forward(xp.clone(), layers, KINDS, cache_p, CFG)
            xd = x.to(dev)
            stack.forward(xd)
            torch.cuda.synchronize()
            check_stack_feed(xd.cpu() - x, ref - x, ref_p - xp, f"op {i} feed {op[1]}")
        elif op[0] == "snapshot":
            stack.snapshot()
            snaps.append((copy.deepcopy(cache), copy.deepcopy(cache_p)))
            snaps = snaps[-2:]
        else:  # crop to the newest snapshot at or before n
            kept = stack.crop(op[1])
            cands = [s for s in snaps if s[0]["length"] <= op[1]]
            want = cands[-1][0]["length"] if cands else 0
            if op[1] >= cache["length"]:
                want = cache["length"]
            assert kept == want, (i, op, kept, want)
            if kept < cache["length"]:
                if cands:
                    cache, cache_p = copy.deepcopy(cands[-1][0]), copy.deepcopy(cands[-1][1])
                else:
                    cache, cache_p = _fresh_cache(B, cap), _fresh_cache(B, cap)
        assert stack.length == cache["length"], (i, op)
    stack.close()
