"""GPU parity of the hybrid mixer stack (config 4 composite: x = x + mixer(znorm(x)) per
layer, MoE as identity) against the oracle composite, on a reduced shape: d_model 256, 2 QK /
4 V DeltaNet heads, 4 / 2 attention heads (head_dim 256), 8 layers (3 DeltaNet + 1 attention,
twice). Prefill of 100 tokens then 3 decode steps at batch 2. Both sides round the projection
inputs to bf16; the bar for the 8-layer composite is 5e-3 (per-op bars: 1e-3 / 2e-3)."""
import pytest
import torch

from conftest import rel_err
from oracle import mixer_ref as R

from aegist_mixer import ops

pytestmark = pytest.mark.gpu

CFG = dict(d_model=256, hk=2, hv=4, n_heads=4, n_kv=2, head_dim=256, rotary_dim=64, rope_theta=1e7, eps=1e-6)
KINDS = (["delta"] * 3 + ["attn"]) * 2


def make_layers(seed, dev):
    g_ = torch.Generator().manual_seed(seed)
    c = CFG
    C = 2 * c["hk"] * 128 + c["hv"] * 128
    dm, hv, H, KV, HD = c["d_model"], c["hv"], c["n_heads"], c["n_kv"], c["head_dim"]

    def w(*shape, std=0.02):
        return (torch.randn(*shape, generator=g_) * std).to(torch.bfloat16)
    layers = []
    for kind in KINDS:
        W = {"norm1": w(dm, std=0.1)}
        if kind == "delta":
            W.update(w_qkv=w(C, dm, std=0.06), w_z=w(hv * 128, dm, std=0.06), w_b=w(hv, dm, std=0.06),
                     w_a=w(hv, dm, std=0.06), conv_w=w(C, 4, std=0.3), a_log=w(hv, std=0.5), dt_bias=w(hv, std=0.5),
                     gnorm_w=(1 + 0.1 * torch.randn(128, generator=g_)).to(torch.bfloat16),
                     w_out=w(dm, hv * 128, std=0.02))
        else:
            W.update(w_q=w(2 * H * HD, dm, std=0.06), w_k=w(KV * HD, dm, std=0.06), w_v=w(KV * HD, dm, std=0.06),
                     w_o=w(dm, H * HD, std=0.02), q_norm=w(HD, std=0.1), k_norm=w(HD, std=0.1))
        layers.append(W)
    dev_layers = [{k: v.to(dev) for k, v in W.items()} for W in layers]
    return layers, dev_layers


def test_stack_prefill_then_decode(dev):
    B, T, steps, cap = 2, 100, 3, 128
    layers, dl = make_layers(0, dev)
    c = CFG
    C = 2 * c["hk"] * 128 + c["hv"] * 128
    nd, na = KINDS.count("delta"), KINDS.count("attn")
    cache = {"length": 0,
             "conv": [torch.zeros(B, C, 3) for _ in range(nd)],
             "state": [torch.zeros(B, c["hv"], 128, 128) for _ in range(nd)],
             "k": [torch.zeros(B, c["n_kv"], cap, 256, dtype=torch.bfloat16) for _ in range(na)],
             "v": [torch.zeros(B, c["n_kv"], cap, 256, dtype=torch.bfloat16) for _ in range(na)]}
    stack = ops.HybridStack(c, KINDS, dl, max_batch=B, max_tokens=B * T, max_context=cap)
    g_ = torch.Generator().manual_seed(1)
    x = torch.randn(B, T, c["d_model"], generator=g_)
    ref = R.hybrid_stack_forward(x.clone(), layers, KINDS, cache, c)
    xd = x.to(dev)
    stack.forward(xd)
    torch.cuda.synchronize()
    assert rel_err(xd - x.to(dev), ref - x) < 5e-3, rel_err(xd - x.to(dev), ref - x)
    for s in range(steps):
        xt = torch.randn(B, 1, c["d_model"], generator=g_)
        ref = R.hybrid_stack_forward(xt.clone(), layers, KINDS, cache, c)
        xdt = xt.to(dev)
        stack.forward(xdt)
        torch.cuda.synchronize()
        assert rel_err(xdt - xt.to(dev), ref - xt) < 5e-3, (s, rel_err(xdt - xt.to(dev), ref - xt))
    assert stack.length == T + steps
    stack.close()


def test_stack_rejects_overflow(dev):
    layers, dl = make_layers(2, dev)
    stack = ops.HybridStack(CFG, KINDS, dl, max_batch=1, max_tokens=8, max_context=10)
    x = torch.zeros(1, 8, CFG["d_model"], device=dev)
    stack.forward(x)
    with pytest.raises(ops.AegistError, match="max_context"):
        stack.forward(torch.zeros(1, 4, CFG["d_model"], device=dev))
    with pytest.raises(ops.AegistError, match="max_tokens"):
        stack.forward(torch.zeros(1, 9, CFG["d_model"], device=dev))
    stack.reset()
    assert stack.length == 0
    stack.close()


@pytest.mark.parametrize("hk,hv", [(2, 2), (1, 4)])
def test_stack_head_ratios(dev, hk, hv):
    """The stack's fused decode core is built per value-to-QK head ratio (1, 2, 4): a 70-token
    prefill (chunked path) and 3 decode steps at batch 2 against the oracle, for ratios 1 and 4."""
    global CFG
    saved = CFG
    CFG = dict(saved, hk=hk, hv=hv)
    try:
        B, T, steps, cap = 2, 70, 3, 96
        layers, dl = make_layers(5, dev)
        c = CFG
        C = 2 * hk * 128 + hv * 128
        nd, na = KINDS.count("delta"), KINDS.count("attn")
        cache = {"length": 0,
                 "conv": [torch.zeros(B, C, 3) for _ in range(nd)],
                 "state": [torch.zeros(B, hv, 128, 128) for _ in range(nd)],
                 "k": [torch.zeros(B, c["n_kv"], cap, 256, dtype=torch.bfloat16) for _ in range(na)],
                 "v": [torch.zeros(B, c["n_kv"], cap, 256, dtype=torch.bfloat16) for _ in range(na)]}
        stack = ops.HybridStack(c, KINDS, dl, max_batch=B, max_tokens=B * T, max_context=cap)
        g_ = torch.Generator().manual_seed(6)
        for n in [T] + [1] * steps:
            x = torch.randn(B, n, c["d_model"], generator=g_)
            ref = R.hybrid_stack_forward(x.clone(), layers, KINDS, cache, c)
            xd = x.to(dev)
            stack.forward(xd)
            torch.cuda.synchronize()
            err = rel_err(xd - x.to(dev), ref - x)
            assert err < 1e-2, (n, err)
        stack.close()
    finally:
        CFG = saved
