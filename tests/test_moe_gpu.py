"""GPU parity of the mixture-of-experts block (router top-k, device-side grouping, 4-bit SwiGLU
experts on MFMA, combine with the gated shared expert) against the CPU oracle in fp64.

The experts' 4-bit codes enter the MFMA exactly, the fp32 activations as bf16 hi + lo (~16
significant bits), and the scale / min of every 64-group is applied in fp32, so the routed
output matches an fp32 evaluation of q4_dequantize + SwiGLU (hybrid.py:463-469, 608-628): the
bar is 5e-5 norm-wise max relative error. Router indices must match exactly, except where two
experts' probabilities are within fp32 rounding of each other (then the swap is checked to be
such a near-tie); the router weights within 1e-5."""
import pytest
import torch

from conftest import rel_err
from oracle import mixer_ref as R

from aegist_mixer import ops
from aegist_mixer._lib import AegistError

pytestmark = pytest.mark.gpu

TOL_MOE = 5e-5
TOL_WTS = 1e-5


def _experts(E, D, I, seed):
    """E random 4-bit expert rows: random codes, scales in [0.002, 0.01], mins in [-0.06, -0.01]."""
    g = torch.Generator().manual_seed(seed)
    rb = R.expert_row_bytes(D, I)
    rows = torch.randint(0, 256, (E, rb), generator=g, dtype=torch.uint8)
    gu_q, gu_s = 2 * I * D // 2, 2 * I * (D // 64) * 2
    dn_q, dn_s = D * I // 2, D * (I // 64) * 2
    sec = [(gu_q, gu_s, 0), (gu_q + gu_s, gu_s, 1), (gu_q + 2 * gu_s + dn_q, dn_s, 0),
           (gu_q + 2 * gu_s + dn_q + dn_s, dn_s, 1)]
    for off, nb, is_min in sec:
        n = nb // 2
        v = torch.rand(E, n, generator=g)
        v = -(0.01 + 0.05 * v) if is_min else 0.002 + 0.008 * v
        rows[:, off:off + nb] = v.half().view(torch.uint8).reshape(E, nb)
    rows[:, gu_q + 2 * gu_s + dn_q + 2 * dn_s:] = 0
    return rows


def _route_ok(idx_gpu, wts_gpu, h, W, K):
    ridx, rwts = R.route(h, W, K)
    p = torch.softmax(h.double() @ W.double().t(), -1)
    gi = idx_gpu.cpu().long()
    for t in range(h.shape[0]):
        if not torch.equal(gi[t], ridx[t]):
            # only near-ties may swap: the probabilities at each differing rank agree to fp32
            pa, pb = p[t, gi[t]], p[t, ridx[t]]
            assert torch.allclose(pa, pb, rtol=1e-6, atol=0), (t, gi[t].tolist(), ridx[t].tolist())
    assert rel_err(wts_gpu, rwts) < TOL_WTS
    return gi


@pytest.mark.parametrize("T,D,E,K", [(1, 2048, 256, 8), (37, 2048, 256, 8), (16, 512, 64, 4), (5, 2048, 300, 16)])
def test_router_topk(dev, T, D, E, K):
    print(f"router T={T} D={D} E={E} K={K}", flush=True)
    g = torch.Generator().manual_seed(T + E)
    h = torch.randn(T, D, generator=g)
    W = (torch.randn(E, D, generator=g) * 0.02).bfloat16()
    idx, wts = ops.router_topk(h.to(dev), W.to(dev), K)
    torch.cuda.synchronize()
    _route_ok(idx, wts, h, W, K)


def test_router_ties_to_lower_expert(dev):
    h = torch.randn(3, 256)
    W = torch.ones(40, 256, dtype=torch.bfloat16)
    idx, wts = ops.router_topk(h.to(dev), W.to(dev), 8)
    assert idx.cpu().tolist() == [list(range(8))] * 3
    assert torch.allclose(wts.cpu(), torch.full((3, 8), 0.125))


def _run_experts(dev, T, D, I, E, K, seed, x0=None, shared=False, eptr_perm=None, bad_ids=False):
    g = torch.Generator().manual_seed(seed)
    rows = _experts(E, D, I, seed)
    h = torch.randn(T, D, generator=g)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).int()
    if bad_ids:
        idx[::3, 0] = E + 5
        idx[1::4, -1] = -1
    wts = torch.rand(T, K, generator=g)
    wts = wts / wts.sum(-1, keepdim=True)
    x = torch.zeros(T, D) if x0 is None else x0.clone()
    ysh = torch.randn(T, D, generator=g) if shared else None
    wg = (torch.randn(D, generator=g) * 0.05).bfloat16() if shared else None
    rows_d = rows.to(dev)
    eptr = None
    if eptr_perm is not None:
        # a non-contiguous placement: expert e lives at slot perm[e] of a shuffled copy
        perm = eptr_perm(E)
        slots = torch.empty_like(rows_d)
        slots[perm] = rows_d
        rb = rows.shape[1]
        eptr = torch.tensor([slots.data_ptr() + int(perm[e]) * rb for e in range(E)], dtype=torch.int64, device=dev)
    xd = x.to(dev)
    ops.moe_experts(h.to(dev), None if eptr is not None else rows_d, idx.to(dev), wts.to(dev), xd, I,
                    ysh=ysh.to(dev) if shared else None, wg=wg.to(dev) if shared else None, eptr=eptr)
    torch.cuda.synchronize()
    ref = R.moe_experts(h, rows, idx.long(), wts, D, I)
    if shared:
        ref = ref + torch.sigmoid(h.double() @ wg.double()).unsqueeze(-1) * ysh.double()
    return xd.cpu().double() - x.double(), ref


@pytest.mark.parametrize("T,E,K", [(1, 256, 8), (16, 256, 8), (4, 8, 8), (300, 16, 8), (200, 16, 8), (130, 8, 4),
                                   (512, 64, 8), (100, 24, 8)])
def test_moe_experts(dev, T, E, K):
    """Decode and prefill batches: in batches of 16 or more picks per expert on average, experts
    with more than 32 picks take balanced tiles of up to 64 (300 x 8 / 16: 150 each = 3 x 50;
    200 x 8 / 16: 2 x 50; 130 x 4 / 8: 65 = 33 + 32; 512 x 8 / 64: ~64 each, one or two tiles;
    100 x 8 / 24: ~33 each, so some experts stay on the <= 32-pick tiles)."""
    print(f"moe experts T={T} E={E} K={K}", flush=True)
    got, ref = _run_experts(dev, T, 2048, 512, E, K, seed=T * 7 + E)
    err = rel_err(got, ref)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < TOL_MOE


def test_moe_experts_shapes_and_shared(dev):
    got, ref = _run_experts(dev, 33, 256, 128, 12, 3, seed=11, shared=True)
    assert rel_err(got, ref) < TOL_MOE


def test_moe_experts_accumulates_into_residual(dev):
    x0 = torch.randn(9, 512)
    got, ref = _run_experts(dev, 9, 512, 192, 20, 4, seed=12, x0=x0)
    assert rel_err(got, ref) < 1e-4  # the difference of two fp32 residuals carries their rounding


def test_moe_experts_out_of_range_ids_add_nothing(dev):
    got, ref = _run_experts(dev, 24, 512, 128, 10, 4, seed=13, bad_ids=True)
    assert rel_err(got, ref) < TOL_MOE


def test_moe_experts_pointer_table_placement(dev):
    got, ref = _run_experts(dev, 20, 512, 128, 16, 4, seed=14, eptr_perm=lambda E: torch.randperm(E))
    assert rel_err(got, ref) < TOL_MOE


def test_moe_forward_end_to_end(dev):
    """Router -> experts -> gated shared expert (int8 QLinear SwiGLU) against the oracle, with the
    oracle routing on the GPU's picks where they are near-ties."""
    T, D, I, E, K, SH = 12, 1024, 256, 32, 8, 256
    g = torch.Generator().manual_seed(15)
    rows = _experts(E, D, I, 15)
    h = torch.randn(T, D, generator=g)
    W = (torch.randn(E, D, generator=g) * 0.02).bfloat16()
    wq = [R.qlinear_quantize(torch.randn(n, k, generator=g) * 0.02) for n, k in ((SH, D), (SH, D), (D, SH))]
    wg = (torch.randn(D, generator=g) * 0.05).bfloat16()
    x = torch.zeros(T, D, device=dev)
    shared = tuple((q.to(dev), s.to(dev)) for q, s in wq)
    idx, wts = ops.moe_forward(h.to(dev), x, W.to(dev), rows.to(dev), I, K, shared=shared, shared_gate=wg.to(dev))
    torch.cuda.synchronize()
    gi = _route_ok(idx, wts, h, W, K)
    gsh = R.qlinear_engine(h, *wq[0])
    ush = R.qlinear_engine(h, *wq[1])
    act = (torch.nn.functional.silu(gsh.double()) * ush.double()).float()
    ysh = R.qlinear_engine(act, *wq[2])
    ref = R.moe_experts(h, rows, gi, wts.cpu(), D, I)
    ref = ref + torch.sigmoid(h.double() @ wg.double()).unsqueeze(-1) * ysh.double()
    assert rel_err(x, ref) < 1e-4


def test_silu_mul_and_shared_gate_add(dev):
    g = torch.Generator().manual_seed(16)
    a, b = torch.randn(1000, generator=g), torch.randn(1000, generator=g)
    out = ops.silu_mul(a.to(dev), b.to(dev))
    assert rel_err(out, torch.nn.functional.silu(a.double()) * b.double()) < 1e-6
    x, y, h = torch.randn(5, 320, generator=g), torch.randn(5, 320, generator=g), torch.randn(5, 320, generator=g)
    wg = torch.randn(320, generator=g).bfloat16()
    xd = x.to(dev)
    ops.shared_gate_add(xd, y.to(dev), h.to(dev), wg.to(dev))
    ref = x.double() + torch.sigmoid(h.double() @ wg.double()).unsqueeze(-1) * y.double()
    assert rel_err(xd, ref) < 1e-6


def test_moe_rejects_bad_shapes(dev):
    h = torch.zeros(2, 100, device=dev)
    with pytest.raises(AegistError):
        ops.router_topk(h, torch.zeros(8, 100, dtype=torch.bfloat16, device=dev), 2)  # D % 8
    rows = torch.zeros(4, R.expert_row_bytes(128, 64), dtype=torch.uint8, device=dev)
    with pytest.raises(AegistError):
        ops.moe_experts(torch.zeros(2, 128, device=dev), rows, torch.zeros(2, 2, dtype=torch.int32, device=dev),
                        torch.zeros(2, 2, device=dev), torch.zeros(2, 128, device=dev), 96)  # I % 64


def test_moe_experts_big_tiles_match_small(dev):
    """The 64-pick big-tile kernels against the <= 32-pick kernels (AEGIST_MOE_BIG=0) on the
    same prefill batch: both within the oracle bar, and within fp32 rounding of each other."""
    import os
    T, E, K, D, I = 256, 16, 8, 2048, 512
    got_big, ref = _run_experts(dev, T, D, I, E, K, seed=21)
    old = os.environ.get("AEGIST_MOE_BIG")
    os.environ["AEGIST_MOE_BIG"] = "0"
    try:
        got_small, _ = _run_experts(dev, T, D, I, E, K, seed=21)
    finally:
        if old is None:
            del os.environ["AEGIST_MOE_BIG"]
        else:
            os.environ["AEGIST_MOE_BIG"] = old
    assert rel_err(got_big, ref) < TOL_MOE
    assert rel_err(got_small, ref) < TOL_MOE
    assert rel_err(got_big, got_small) < 1e-5
