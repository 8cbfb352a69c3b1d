"""GPU parity of the gated GQA attention kernels against the CPU oracle (bar: 2e-3 norm-wise
max relative error on fp32 outputs; the cache rows written must equal the oracle's bf16)."""
import pytest
import torch

from conftest import ATTN_TOL, rel_err
from oracle import mixer_ref as R

from aegist_mixer import ops

pytestmark = pytest.mark.gpu

HD, RD, THETA = 256, 64, 1e7


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def decode_case(B, H, KV, L, cap, seed, dtype=torch.bfloat16):
    g_ = _gen(seed)
    qg = torch.randn(B, H, 2 * HD, generator=g_).to(dtype)
    kn = torch.randn(B, KV, HD, generator=g_).to(dtype)
    vn = torch.randn(B, KV, HD, generator=g_).to(dtype)
    qw = (torch.randn(HD, generator=g_) * 0.1).to(torch.bfloat16)
    kw = (torch.randn(HD, generator=g_) * 0.1).to(torch.bfloat16)
    kc = torch.randn(B, KV, cap, HD, generator=g_).to(torch.bfloat16)
    vc = torch.randn(B, KV, cap, HD, generator=g_).to(torch.bfloat16)
    return qg, kn, vn, qw, kw, kc, vc


@pytest.mark.parametrize("B,H,KV,L", [(1, 16, 2, 0), (1, 16, 2, 1), (2, 16, 2, 100), (1, 16, 2, 4096),
                                      (3, 8, 2, 777), (2, 4, 4, 300), (8, 16, 2, 4096), (1, 16, 2, 32768)])
def test_attention_decode_matches_oracle(dev, B, H, KV, L):
    print(f"attention_decode B={B} H={H} KV={KV} L={L}", flush=True)
    cap = L + 5
    qg, kn, vn, qw, kw, kc, vc = decode_case(B, H, KV, L, cap, seed=L + B)
    kc_r, vc_r = kc.clone(), vc.clone()
    ref = R.attention_decode(qg.float(), kn.float(), vn.float(), qw.float(), kw.float(), kc_r, vc_r, L, RD, THETA)
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    out = ops.attention_decode(qg.to(dev), kn.to(dev), vn.to(dev), qw.to(dev), kw.to(dev), kc_d, vc_d, L, RD, THETA)
    torch.cuda.synchronize()
    assert rel_err(out, ref) < ATTN_TOL
    # the appended row: k roped then rounded to bf16, v copied; allow 1 bf16 ulp on k
    assert torch.equal(vc_d[:, :, L].cpu(), vc_r[:, :, L])
    dk = (kc_d[:, :, L].float().cpu() - kc_r[:, :, L].float()).abs()
    assert (dk <= kc_r[:, :, L].float().abs() * 2 ** -7 + 1e-6).all()


@pytest.mark.slow
@pytest.mark.parametrize("B,L", [(1, 131072), (32, 4096)])
def test_attention_decode_long(dev, B, L):
    print(f"attention_decode long B={B} L={L}", flush=True)
    qg, kn, vn, qw, kw, kc, vc = decode_case(B, 16, 2, L, L + 1, seed=3)
    kc_r, vc_r = kc.clone(), vc.clone()
    ref = R.attention_decode(qg.float(), kn.float(), vn.float(), qw.float(), kw.float(), kc_r, vc_r, L, RD, THETA)
    out = ops.attention_decode(qg.to(dev), kn.to(dev), vn.to(dev), qw.to(dev), kw.to(dev), kc.to(dev), vc.to(dev), L,
                               RD, THETA)
    torch.cuda.synchronize()
    assert rel_err(out, ref) < ATTN_TOL


def test_attention_prefill_saturates_beyond_fp16(dev):
    """The prefill stages K / V as fp16: cache values beyond +-65504 saturate there (a V column
    around 1e5 gives a finite output equal to the reference on the clamped cache), where a plain
    conversion would make them infinite and the output NaN."""
    B, H, KV, T, pos = 1, 8, 2, 150, 10
    g_ = _gen(77)
    q = torch.randn(B, H, T, HD, generator=g_) * 0.5
    kc = torch.randn(B, KV, pos + T, HD, generator=g_).to(torch.bfloat16)
    vc = torch.randn(B, KV, pos + T, HD, generator=g_)
    vc[..., 5] = 1e5 * torch.sign(vc[..., 5])
    vc = vc.to(torch.bfloat16)
    out = ops.attention_core(q.to(dev), kc.to(dev), vc.to(dev), None, pos)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = R.attention_core(q, kc, vc.float().clamp(-65504, 65504).to(torch.bfloat16), pos, KV).transpose(1, 2)
    assert rel_err(out, ref) < ATTN_TOL


def test_attention_decode_bf16_out(dev):
    qg, kn, vn, qw, kw, kc, vc = decode_case(2, 16, 2, 500, 505, seed=9)
    ref = R.attention_decode(qg.float(), kn.float(), vn.float(), qw.float(), kw.float(), kc.clone(), vc.clone(),
                             500, RD, THETA)
    out = ops.attention_decode(qg.to(dev), kn.to(dev), vn.to(dev), qw.to(dev), kw.to(dev), kc.to(dev), vc.to(dev), 500,
                               RD, THETA, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert (out.float().cpu() - ref).abs().max() <= ref.abs().max() * 2 ** -8 + 1e-3 * ref.abs().max()


@pytest.mark.parametrize("B,H,KV,T,pos,qs,vs", [(1, 16, 2, 2, 0, 0.5, 1), (1, 16, 2, 17, 30, 0.5, 1),
                                                (2, 8, 2, 64, 0, 0.5, 1), (1, 16, 2, 130, 5, 0.5, 1),
                                                (1, 16, 2, 1000, 0, 0.5, 1), (2, 16, 2, 300, 500, 0.5, 1),
                                                (1, 4, 4, 77, 3, 0.5, 1),
                                                # (sequence, KV head) pairs a multiple of 8: the
                                                # persistent schedule's per-XCD pair ownership
                                                (4, 16, 2, 300, 0, 0.5, 1), (8, 8, 2, 256, 20, 0.5, 1),
                                                # sharp softmax (scores ~ +-30) and large / small V
                                                (1, 16, 2, 260, 0, 3.0, 1), (1, 8, 2, 200, 40, 0.5, 300),
                                                (1, 8, 2, 200, 40, 0.5, 1e-3),
                                                # 128 (sequence, KV head) pairs and 9 query blocks
                                                # each: several rounds per workgroup
                                                (8, 16, 2, 1100, 64, 0.5, 1)])
def test_attention_core_prefill(dev, B, H, KV, T, pos, qs, vs):
    """The MFMA prefill takes K / V as fp16 (exact for bf16 values in fp16's range; converted once
    into the workspace, or per tile without it) and q and P as fp16: ~11 significant bits against
    the fp64 loop."""
    print(f"attention_core prefill B={B} H={H} KV={KV} T={T} pos={pos} q*{qs} v*{vs}", flush=True)
    g_ = _gen(T)
    q = torch.randn(B, H, T, HD, generator=g_) * qs
    kc = torch.randn(B, KV, pos + T + 3, HD, generator=g_).to(torch.bfloat16)
    vc = (torch.randn(B, KV, pos + T + 3, HD, generator=g_) * vs).to(torch.bfloat16)
    gate = torch.randn(B, T, H * HD, generator=g_)
    ref = R.gated_attention_out(R.attention_core(q, kc, vc, pos, KV), gate).reshape(B, T, H, HD)
    out = ops.attention_core(q.to(dev), kc.to(dev), vc.to(dev), gate.to(dev), pos)
    # without the fp16-copy workspace the kernel converts its tiles itself: same values, same
    # order of operations, so the same bits
    out2 = ops.attention_core(q.to(dev), kc.to(dev), vc.to(dev), gate.to(dev), pos, f16_copy=False)
    torch.cuda.synchronize()
    err = rel_err(out, ref)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < ATTN_TOL
    assert torch.equal(out, out2)


def test_engine_attention_pipeline(dev):
    """attn_prep -> attention_gated with engine layouts, prefill of 9 tokens then 1 decode."""
    H, KV, cap = 16, 2, 64
    g_ = _gen(4)
    T = 10
    qg = torch.randn(T, H, 2 * HD, generator=g_)
    k = torch.randn(T, KV, HD, generator=g_)
    v = torch.randn(T, KV, HD, generator=g_)
    qw = (torch.randn(HD, generator=g_) * 0.1).to(torch.bfloat16)
    kw = (torch.randn(HD, generator=g_) * 0.1).to(torch.bfloat16)
    kc_r = torch.zeros(1, KV, cap, HD, dtype=torch.bfloat16)
    vc_r = torch.zeros(1, KV, cap, HD, dtype=torch.bfloat16)
    q_r, gate_r = R.attn_prep(qg.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), qw.float(), kw.float(), kc_r, vc_r, 0,
                              RD, THETA)
    ref = R.gated_attention_out(R.attention_core(q_r, kc_r, vc_r, 0, KV), gate_r).reshape(T, H, HD)
    kc = torch.zeros(KV, cap, HD, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros(KV, cap, HD, dtype=torch.bfloat16, device=dev)
    outs = []
    for a, b_ in [(0, 9), (9, 10)]:
        qgd = qg[a:b_].contiguous().to(dev)
        qn = ops.engine_attn_prep(qgd, k[a:b_].contiguous().to(dev), v[a:b_].contiguous().to(dev), qw.to(dev),
                                  kw.to(dev), kc, vc, a, RD, THETA)
        assert rel_err(qn, q_r[0, :, a:b_].transpose(0, 1)) < 1e-5
        outs.append(ops.engine_attention_gated(qn, kc, vc, qgd, a))
    torch.cuda.synchronize()
    assert rel_err(torch.cat(outs, 0), ref) < ATTN_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,L", [(3, 0), (3, 37), (2, 4096), (1, 4159)])
def test_attention_decode_fused_prep(dev, B, L, dtype):
    """The decode launch that does its own prep (rotary dim 64): the rows it appends equal the
    separate prep kernel's bit for bit, and the cache's old contents at row L and past it never
    reach the output (they are set to NaN first; the last split stages the new row in their place).
    L = 0 has no cached rows at all; 37 and 4159 put row L mid-tile of the last split."""
    print(f"attention_decode fused prep B={B} L={L} {dtype}", flush=True)
    H, KV, cap = 16, 2, L + 8
    qg, kn, vn, qw, kw, kc, vc = decode_case(B, H, KV, L, cap, 300 + L, dtype)
    kc[:, :, L:] = float("nan")
    vc[:, :, L:] = float("nan")
    ref = R.attention_decode(qg.float(), kn.float(), vn.float(), qw.float(), kw.float(), kc.clone(), vc.clone(), L, RD,
                             THETA)
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    out = ops.attention_decode(qg.to(dev), kn.to(dev), vn.to(dev), qw.to(dev), kw.to(dev), kc_d, vc_d, L, RD, THETA)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert rel_err(out, ref) < ATTN_TOL
    for b in range(B):
        kp = kc[b].clone().to(dev)
        vp = vc[b].clone().to(dev)
        ops.engine_attn_prep(qg[b:b + 1].float().to(dev), kn[b:b + 1].float().to(dev), vn[b:b + 1].float().to(dev),
                             qw.to(dev), kw.to(dev), kp, vp, L, RD, THETA)
        torch.cuda.synchronize()
        assert torch.equal(kc_d[b, :, L].view(torch.int16), kp[:, L].view(torch.int16)), b
        assert torch.equal(vc_d[b, :, L].view(torch.int16), vp[:, L].view(torch.int16)), b


@pytest.mark.slow
@pytest.mark.parametrize("B,L", [(8, 32768), (32, 32768), (8, 131072), (32, 131072), (64, 32768)])
def test_attention_decode_config3_points(dev, B, L):
    """Config 3's large points at full size (16 query / 2 KV heads, head_dim 256, bf16 caches
    ~N(0, 1) filled on the device): two of the B sequences against the CPU oracle, and the same two
    run alone (B = 1, so a different split of the context and a different merge) against the batch
    result. The B = 64 point is the north star's batch-64 decode."""
    print(f"attention_decode config3 B={B} L={L}", flush=True)
    H, KV, cap = 16, 2, L + 1
    kc = ops.fill_normal(torch.empty(B, KV, cap, HD, dtype=torch.bfloat16, device=dev), 1000 + B)
    vc = ops.fill_normal(torch.empty(B, KV, cap, HD, dtype=torch.bfloat16, device=dev), 2000 + B)
    g_ = _gen(B + L)
    qg = torch.randn(B, H, 2 * HD, generator=g_).to(torch.bfloat16)
    kn = torch.randn(B, KV, HD, generator=g_).to(torch.bfloat16)
    vn = torch.randn(B, KV, HD, generator=g_).to(torch.bfloat16)
    qw = (torch.randn(HD, generator=g_) * 0.1).to(torch.bfloat16)
    kw = (torch.randn(HD, generator=g_) * 0.1).to(torch.bfloat16)
    rows = (0, B - 1)
    kc_rows = [kc[b:b + 1].cpu() for b in rows]
    vc_rows = [vc[b:b + 1].cpu() for b in rows]
    out = ops.attention_decode(qg.to(dev), kn.to(dev), vn.to(dev), qw.to(dev), kw.to(dev), kc, vc, L, RD, THETA)
    torch.cuda.synchronize()
    for i, b in enumerate(rows):
        ref = R.attention_decode(qg[b:b + 1].float(), kn[b:b + 1].float(), vn[b:b + 1].float(), qw.float(), kw.float(),
                                 kc_rows[i], vc_rows[i], L, RD, THETA)
        err = rel_err(out[b:b + 1], ref)
        print(f"  row {b}: rel err vs oracle {err:.2e}", flush=True)
        assert err < ATTN_TOL
        # the same sequence alone: its own split of the context and merge
        kc1, vc1 = kc_rows[i].to(dev), vc_rows[i].to(dev)
        alone = ops.attention_decode(qg[b:b + 1].to(dev), kn[b:b + 1].to(dev), vn[b:b + 1].to(dev), qw.to(dev),
                                     kw.to(dev), kc1, vc1, L, RD, THETA)
        torch.cuda.synchronize()
        err1 = rel_err(alone, out[b:b + 1])
        print(f"  row {b}: batch vs alone {err1:.2e}", flush=True)
        assert err1 < 1e-5
    del kc, vc
    torch.cuda.empty_cache()
