"""GPU parity of the gated DeltaNet kernels against the CPU oracle (bar: 1e-3 norm-wise max
relative error on fp32 outputs and final state; bf16 outputs within one bf16 rounding)."""
import math

import pytest
import torch
import torch.nn.functional as F

from conftest import DELTA_TOL, rel_err
from oracle import mixer_ref as R

from aegist_mixer import ops

pytestmark = pytest.mark.gpu

D = 128


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _bf(x):
    return x.to(torch.bfloat16)


def decode_inputs(B, HK, HV, seed=0, state_std=0.02):
    g_ = _gen(seed)
    C = 2 * HK * D + HV * D
    qkv = _bf(torch.randn(B, C, generator=g_))
    conv_w = _bf(torch.randn(C, 4, generator=g_) * 0.05)
    conv_state = torch.randn(B, C, 3, generator=g_)
    g = -F.softplus(torch.randn(B, HV, generator=g_))
    beta = torch.sigmoid(torch.randn(B, HV, generator=g_))
    state = torch.randn(B, HV, D, D, generator=g_) * state_std
    return qkv, conv_w, conv_state, g, beta, state


@pytest.mark.parametrize("B,HK,HV", [(1, 16, 32), (3, 2, 4), (2, 4, 4), (2, 2, 8), (64, 16, 32)])
def test_decode_step_fused_matches_oracle(dev, B, HK, HV):
    print(f"decode_step B={B} HK={HK} HV={HV}", flush=True)
    qkv, w, cs, g, beta, S = decode_inputs(B, HK, HV, seed=B + HK)
    S_ref = S.clone()
    o_ref, cs_ref = R.delta_decode_fused(qkv, w, cs, g, beta, S_ref, HK, HV, D)
    cs_d, S_d = cs.to(dev), S.to(dev)
    o = ops.delta_decode_step(qkv.to(dev), w.to(dev), cs_d, g.to(dev), beta.to(dev), S_d, HK, HV)
    torch.cuda.synchronize()
    assert rel_err(o, o_ref) < DELTA_TOL
    assert rel_err(S_d, S_ref) < DELTA_TOL
    assert torch.equal(cs_d.cpu(), cs_ref)  # the conv state is a copy of inputs: exact


def test_decode_step_bf16_out_and_fp32_in(dev):
    B, HK, HV = 4, 16, 32
    qkv, w, cs, g, beta, S = decode_inputs(B, HK, HV, seed=11)
    S_ref = S.clone()
    o_ref, _ = R.delta_decode_fused(qkv, w, cs, g, beta, S_ref, HK, HV, D)
    o = ops.delta_decode_step(qkv.float().to(dev), w.to(dev), cs.to(dev), g.to(dev), beta.to(dev), S.to(dev), HK, HV,
                              out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    # bf16 output: within one bf16 rounding of the fp32 reference
    assert (o.float().cpu() - o_ref).abs().max() <= o_ref.abs().max() * 2 ** -8


def test_decode_steps_chain_equals_oracle(dev):
    """16 consecutive decode steps: state and conv state carry across calls."""
    B, HK, HV = 2, 16, 32
    qkv, w, cs, g, beta, S = decode_inputs(B, HK, HV, seed=5, state_std=0.0)
    S_ref, cs_ref = S.clone(), cs.clone()
    S_d, cs_d, w_d = S.to(dev), cs.to(dev), w.to(dev)
    g_ = _gen(99)
    for step in range(16):
        x = _bf(torch.randn(B, qkv.shape[1], generator=g_))
        gg = -F.softplus(torch.randn(B, HV, generator=g_))
        bb = torch.sigmoid(torch.randn(B, HV, generator=g_))
        o_ref, cs_ref = R.delta_decode_fused(x, w, cs_ref, gg, bb, S_ref, HK, HV, D)
        o = ops.delta_decode_step(x.to(dev), w_d, cs_d, gg.to(dev), bb.to(dev), S_d, HK, HV)
        assert rel_err(o, o_ref) < DELTA_TOL, step
    assert rel_err(S_d, S_ref) < DELTA_TOL


def seq_inputs(B, HK, HV, T, seed):
    g_ = _gen(seed)
    q = _bf(torch.randn(B, HK, T, D, generator=g_))
    k = _bf(torch.randn(B, HK, T, D, generator=g_))
    v = _bf(torch.randn(B, HV, T, D, generator=g_))
    beta = torch.sigmoid(torch.randn(B, HV, T, generator=g_))
    g = -F.softplus(torch.randn(B, HV, T, generator=g_))
    return q, k, v, g, beta


def oracle_seq(q, k, v, g, beta, S0=None, chunked=True):
    r = v.shape[1] // q.shape[1]
    qf = R.l2norm(q.float().repeat_interleave(r, 1)) * D ** -0.5
    kf = R.l2norm(k.float().repeat_interleave(r, 1))
    fn = R.delta_rule_chunked if chunked else R.delta_rule_recurrent
    return fn(qf, kf, v.float(), g, beta, S0)


def test_config0_recurrent_256_steps(dev):
    """Config 0: B=1, 16 QK / 32 V heads, 256 sequential steps from a zero state."""
    q, k, v, g, beta = seq_inputs(1, 16, 32, 256, seed=0)
    o_ref, S_ref = oracle_seq(q, k, v, g, beta)
    S = torch.zeros(1, 32, D, D, device=dev)
    o = ops.delta_rule_recurrent(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), S, normalize=True,
                                 qscale=D ** -0.5)
    torch.cuda.synchronize()
    assert rel_err(o, o_ref) < DELTA_TOL
    assert rel_err(S, S_ref) < DELTA_TOL


@pytest.mark.parametrize("T", [1, 3, 37])
def test_recurrent_with_state_and_fp32(dev, T):
    q, k, v, g, beta = seq_inputs(2, 2, 4, T, seed=T)
    S0 = torch.randn(2, 4, D, D, generator=_gen(3)) * 0.02
    o_ref, S_ref = oracle_seq(q, k, v, g, beta, S0.clone(), chunked=False)
    qf = (R.l2norm(q.float()) * D ** -0.5).to(dev)
    kf = R.l2norm(k.float()).to(dev)
    S = S0.to(dev)
    o = ops.delta_rule_recurrent(qf, kf, v.float().to(dev), g.to(dev), beta.to(dev), S)
    torch.cuda.synchronize()
    assert rel_err(o, o_ref) < DELTA_TOL and rel_err(S, S_ref) < DELTA_TOL


def test_delta_rule_step_mirror(dev):
    B, H = 3, 4
    g_ = _gen(7)
    q = R.l2norm(torch.randn(B, H, D, generator=g_)) * D ** -0.5
    k = R.l2norm(torch.randn(B, H, D, generator=g_))
    v = torch.randn(B, H, D, generator=g_)
    g = -F.softplus(torch.randn(B, H, generator=g_))
    beta = torch.sigmoid(torch.randn(B, H, generator=g_))
    S0 = torch.randn(B, H, D, D, generator=g_) * 0.05
    S_ref = S0.clone()
    o_ref = R.delta_rule_step(q, k, v, g, beta, S_ref)
    S = S0.to(dev)
    o = ops.delta_rule_step(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), S)
    torch.cuda.synchronize()
    assert rel_err(o, o_ref) < DELTA_TOL and rel_err(S, S_ref) < DELTA_TOL


# --- engine-ABI mirrors (batch 1, fp32, engine layouts) ----------------------------------------

def test_engine_delta_pipeline(dev):
    """conv_silu -> l2norm_heads -> delta_scan on y [T, C], as hybrid.rs:835-852, T = 5 then 1."""
    HK, HV, T = 16, 32, 5
    C = 2 * HK * D + HV * D
    g_ = _gen(21)
    x = torch.randn(T + 1, C, generator=g_)
    w = _bf(torch.randn(C, 4, generator=g_) * 0.05)
    cs0 = torch.randn(1, C, 3, generator=g_)
    gg = -F.softplus(torch.randn(T + 1, HV, generator=g_))
    bb = torch.sigmoid(torch.randn(T + 1, HV, generator=g_))
    gb = torch.cat([gg, bb], -1)
    S0 = torch.randn(1, HV, D, D, generator=g_) * 0.02
    # oracle over all T+1 tokens at once
    y_ref, cs_ref = R.conv_silu(x.unsqueeze(0), w.float(), cs0)
    qr, kr, vr = R.delta_prep(y_ref, HK, HV, D, D)
    o_ref, S_ref = R.delta_rule_recurrent(qr, kr, vr, gg.t().unsqueeze(0), bb.t().unsqueeze(0), S0.clone())
    # GPU: feed T then 1 token
    cs, S, wd = cs0[0].clone().to(dev), S0[0].clone().to(dev), w.to(dev)
    outs = []
    for a, b_ in [(0, T), (T, T + 1)]:
        y = ops.engine_conv_silu(x[a:b_].to(dev), wd, cs)
        ops.engine_l2norm_heads(y, HK)
        outs.append(ops.engine_delta_scan(y, gb[a:b_].contiguous().to(dev), S, HK, HV))
    torch.cuda.synchronize()
    o = torch.cat(outs, 0)  # [T+1, HV, D]
    assert rel_err(o, o_ref[0].transpose(0, 1)) < DELTA_TOL
    assert rel_err(S, S_ref[0]) < DELTA_TOL
    assert torch.equal(cs.cpu(), cs_ref[0])


def test_engine_gates_and_gated_norm(dev):
    T, Dm, HV = 7, 2048, 32
    g_ = _gen(3)
    h = torch.randn(T, Dm, generator=g_)
    wb, wa = _bf(torch.randn(HV, Dm, generator=g_) * 0.02), _bf(torch.randn(HV, Dm, generator=g_) * 0.02)
    a_log, dt = _bf(torch.randn(HV, generator=g_)), _bf(torch.randn(HV, generator=g_))
    gg, bb = R.delta_gates(h, wb, wa, a_log, dt)
    gb = ops.engine_delta_gates(h.to(dev), wb.to(dev), wa.to(dev), a_log.to(dev), dt.to(dev))
    torch.cuda.synchronize()
    assert rel_err(gb[:, :HV], gg) < 1e-5 and rel_err(gb[:, HV:], bb) < 1e-5
    o = torch.randn(T, HV, D, generator=g_)
    z = torch.randn(T, HV, D, generator=g_)
    wn = _bf(1 + 0.1 * torch.randn(D, generator=g_))
    ref = R.gated_norm(o, z, wn.float())
    got = ops.engine_gated_norm(o.to(dev), z.to(dev), wn.to(dev))
    torch.cuda.synchronize()
    assert rel_err(got, ref) < 1e-5


def test_engine_znorm(dev):
    x = torch.randn(9, 2048, generator=_gen(1))
    w = _bf(torch.randn(2048, generator=_gen(2)) * 0.1)
    got = ops.engine_znorm(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert rel_err(got, R.znorm(x, w.float())) < 1e-5


# --- chunked WY prefill (MFMA) ----------------------------------------------------------------

@pytest.mark.parametrize("T,with_state", [(1, False), (37, True), (64, False), (100, True), (130, False),
                                          (512, True), (2100, True)])
def test_chunked_matches_recurrent_oracle(dev, T, with_state):
    print(f"chunked T={T} state={with_state}", flush=True)
    q, k, v, g, beta = seq_inputs(1, 4, 8, T, seed=T)
    S0 = torch.randn(1, 8, D, D, generator=_gen(T)) * 0.02 if with_state else None
    o_ref, S_ref = oracle_seq(q, k, v, g, beta, None if S0 is None else S0.clone(), chunked=False)
    S = S0.to(dev) if with_state else None
    o, S_out = ops.delta_rule_chunked(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), S, normalize=True,
                                      qscale=D ** -0.5)
    torch.cuda.synchronize()
    assert rel_err(o, o_ref) < DELTA_TOL
    assert rel_err(S_out, S_ref) < DELTA_TOL


def test_chunked_batch_and_layout(dev):
    """B = 3, HV/HK = 2, engine-style row layout (q | k | v packed per token), fp32 inputs."""
    B, HK, HV, T = 3, 2, 4, 150
    g_ = _gen(8)
    y = torch.randn(B, T, 2 * HK * D + HV * D, generator=g_)
    qv = y[..., :HK * D].reshape(B, T, HK, D).transpose(1, 2)
    kv = y[..., HK * D:2 * HK * D].reshape(B, T, HK, D).transpose(1, 2)
    vv = y[..., 2 * HK * D:].reshape(B, T, HV, D).transpose(1, 2)
    beta = torch.sigmoid(torch.randn(B, HV, T, generator=g_))
    g = -F.softplus(torch.randn(B, HV, T, generator=g_))
    o_ref, S_ref = oracle_seq(qv, kv, vv, g, beta, None)
    yd = y.to(dev)
    qd = yd[..., :HK * D].reshape(B, T, HK, D).transpose(1, 2)
    kd = yd[..., HK * D:2 * HK * D].reshape(B, T, HK, D).transpose(1, 2)
    vd = yd[..., 2 * HK * D:].reshape(B, T, HV, D).transpose(1, 2)
    o, S = ops.delta_rule_chunked(qd, kd, vd, g.to(dev), beta.to(dev), None, normalize=True, qscale=D ** -0.5)
    torch.cuda.synchronize()
    assert rel_err(o, o_ref) < DELTA_TOL and rel_err(S, S_ref) < DELTA_TOL


def test_config2_prefill_8k(dev):
    """Config 2: B=1, T=8192, 16 QK / 32 V heads, zero initial state; against the CPU chunked
    oracle on the full sequence and the recurrent form on the first 512 tokens."""
    T = 8192
    q, k, v, g, beta = seq_inputs(1, 16, 32, T, seed=2)
    qd, kd, vd, gd, bd = (t.to(dev) for t in (q, k, v, g, beta))
    o, S = ops.delta_rule_chunked(qd, kd, vd, gd, bd, None, normalize=True, qscale=D ** -0.5)
    o512, S512 = ops.delta_rule_chunked(qd[:, :, :512], kd[:, :, :512], vd[:, :, :512], gd[:, :, :512],
                                        bd[:, :, :512], None, normalize=True, qscale=D ** -0.5)
    torch.cuda.synchronize()
    o_ref, S_ref = oracle_seq(q, k, v, g, beta, None, chunked=True)
    assert rel_err(o, o_ref) < DELTA_TOL, rel_err(o, o_ref)
    assert rel_err(S, S_ref) < DELTA_TOL, rel_err(S, S_ref)
    r_ref, rS_ref = oracle_seq(q[:, :, :512], k[:, :, :512], v[:, :, :512], g[:, :, :512], beta[:, :, :512], None,
                               chunked=False)
    assert rel_err(o512, r_ref) < DELTA_TOL and rel_err(S512, rS_ref) < DELTA_TOL
    assert torch.equal(o[:, :, :512].cpu(), o512.cpu()) or rel_err(o[:, :, :512], o512) < 1e-6


def test_engine_delta_scan_long_prompt(dev):
    """delta_scan mirror at T = 200 takes the chunked path; equals the recurrent oracle."""
    HK, HV, T = 16, 32, 200
    C = 2 * HK * D + HV * D
    g_ = _gen(31)
    y = torch.randn(T, C, generator=g_)
    gg = -F.softplus(torch.randn(T, HV, generator=g_))
    bb = torch.sigmoid(torch.randn(T, HV, generator=g_))
    S0 = torch.randn(1, HV, D, D, generator=g_) * 0.02
    qr, kr, vr = R.delta_prep(y.unsqueeze(0), HK, HV, D, D)
    yn = torch.cat([qr[0, ::2].transpose(0, 1).reshape(T, -1), kr[0, ::2].transpose(0, 1).reshape(T, -1),
                    vr[0].transpose(0, 1).reshape(T, -1)], -1).contiguous()
    o_ref, S_ref = R.delta_rule_recurrent(qr, kr, vr, gg.t().unsqueeze(0), bb.t().unsqueeze(0), S0.clone())
    S = S0[0].clone().to(dev)
    o = ops.engine_delta_scan(yn.to(dev), torch.cat([gg, bb], -1).to(dev), S, HK, HV)
    torch.cuda.synchronize()
    assert rel_err(o, o_ref[0].transpose(0, 1)) < DELTA_TOL
    assert rel_err(S, S_ref[0]) < DELTA_TOL


def test_chunked_multi_segment_on_side_stream(dev):
    """Two 5000-token calls (3 segments each, so the fused K2 + next-segment K1 launches run) on a
    non-default stream, the second continuing from the first's state: equals the oracle over
    the 10000-token sequence. Small heads keep the CPU oracle quick."""
    HK, HV, T = 2, 4, 5000
    q, k, v, g, beta = seq_inputs(1, HK, HV, 2 * T, seed=77)
    o_ref, S_ref = oracle_seq(q, k, v, g, beta, None, chunked=True)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        qd, kd, vd, gd, bd = (t.to(dev) for t in (q, k, v, g, beta))
        S = torch.zeros(1, HV, D, D, device=dev)
        o1, _ = ops.delta_rule_chunked(qd[:, :, :T], kd[:, :, :T], vd[:, :, :T], gd[:, :, :T], bd[:, :, :T], S,
                                       normalize=True, qscale=D ** -0.5)
        o2, _ = ops.delta_rule_chunked(qd[:, :, T:], kd[:, :, T:], vd[:, :, T:], gd[:, :, T:], bd[:, :, T:], S,
                                       normalize=True, qscale=D ** -0.5)
        o = torch.cat([o1, o2], 2)
    side.synchronize()
    assert rel_err(o, o_ref) < DELTA_TOL
    assert rel_err(S, S_ref) < DELTA_TOL
