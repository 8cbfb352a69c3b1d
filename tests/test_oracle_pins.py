"""Pins for the CPU oracle (oracle/mixer_ref.py), independent of its own formulas.

The reference ships no golden vectors for the mixer ops (its only parity test is the
end-to-end logits test tests/test_hybrid_rust.py, which needs the 21 GB brain and CUDA), so
each oracle function is pinned here by fp64 brute force, closed-form special cases,
equivalences between the recurrent and chunked forms, and algebraic identities, chosen so a
dropped term, a wrong sign or index, or a transposed operand fails at least one of them."""
import math

import pytest
import torch
import torch.nn.functional as F

from conftest import rel_err
from oracle import mixer_ref as R

torch.manual_seed(0)


def _unit(x):
    return x / x.norm(dim=-1, keepdim=True)


def _delta_inputs(B=2, H=3, T=7, d=8, dtype=torch.float64, seed=0):
    g_ = torch.Generator().manual_seed(seed)
    q = _unit(torch.randn(B, H, T, d, generator=g_, dtype=dtype)) * d ** -0.5
    k = _unit(torch.randn(B, H, T, d, generator=g_, dtype=dtype))
    v = torch.randn(B, H, T, d, generator=g_, dtype=dtype)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=g_, dtype=dtype))
    g = -F.softplus(torch.randn(B, H, T, generator=g_, dtype=dtype))
    return q, k, v, g, beta


def _brute_delta(q, k, v, g, beta, S0=None):
    """Scalar loops in fp64: the gated delta rule written element by element."""
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    S = torch.zeros(B, H, dk, dv, dtype=torch.float64) if S0 is None else S0.double().clone()
    o = torch.zeros(B, H, T, dv, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            for t in range(T):
                a = math.exp(g[b, h, t].item())
                for i in range(dk):
                    for j in range(dv):
                        S[b, h, i, j] *= a
                for j in range(dv):
                    kv = sum(S[b, h, i, j].item() * k[b, h, t, i].item() for i in range(dk))
                    dl = (v[b, h, t, j].item() - kv) * beta[b, h, t].item()
                    for i in range(dk):
                        S[b, h, i, j] += k[b, h, t, i].item() * dl
                for j in range(dv):
                    o[b, h, t, j] = sum(S[b, h, i, j].item() * q[b, h, t, i].item() for i in range(dk))
    return o, S


def test_delta_step_matches_brute_force():
    q, k, v, g, beta = _delta_inputs(B=1, H=2, T=5, d=6)
    S0 = torch.randn(1, 2, 6, 6, dtype=torch.float64) * 0.1
    o, S = R.delta_rule_recurrent(q, k, v, g, beta, S0)
    ob, Sb = _brute_delta(q, k, v, g, beta, S0)
    assert rel_err(o, ob) < 1e-12 and rel_err(S, Sb) < 1e-12


def test_delta_step_special_cases():
    d = 8
    S0 = torch.randn(1, 1, d, d, dtype=torch.float64)
    q = torch.randn(1, 1, d, dtype=torch.float64)
    k = _unit(torch.randn(1, 1, d, dtype=torch.float64))
    v = torch.randn(1, 1, d, dtype=torch.float64)
    # beta = 0: the state only decays, o = (e^g S)^T q
    g = torch.tensor([[-0.7]], dtype=torch.float64)
    S = S0.clone()
    o = R.delta_rule_step(q, k, v, g, torch.zeros(1, 1, dtype=torch.float64), S)
    assert torch.allclose(S, S0 * math.exp(-0.7))
    assert torch.allclose(o[0, 0], (S0[0, 0] * math.exp(-0.7)).t() @ q[0, 0])
    # g = 0, beta = 1, k = e_i: row i of S becomes v, other rows unchanged
    i = 3
    e = torch.zeros(1, 1, d, dtype=torch.float64)
    e[0, 0, i] = 1
    S = S0.clone()
    R.delta_rule_step(q, e, v, torch.zeros(1, 1, dtype=torch.float64), torch.ones(1, 1, dtype=torch.float64), S)
    expect = S0.clone()
    expect[0, 0, i] = v[0, 0]
    assert torch.allclose(S, expect)
    # S0 = 0, one token: o = (q . k) beta v
    S = torch.zeros(1, 1, d, d, dtype=torch.float64)
    bt = torch.tensor([[0.37]], dtype=torch.float64)
    o = R.delta_rule_step(q, k, v, g, bt, S)
    assert torch.allclose(o[0, 0], (q[0, 0] @ k[0, 0]) * 0.37 * v[0, 0])


@pytest.mark.parametrize("T", [1, 5, 63, 64, 100, 130])
@pytest.mark.parametrize("with_state", [False, True])
def test_chunked_equals_recurrent(T, with_state):
    q, k, v, g, beta = _delta_inputs(B=2, H=2, T=T, d=16, seed=T)
    S0 = torch.randn(2, 2, 16, 16, dtype=torch.float64) * 0.05 if with_state else None
    o1, S1 = R.delta_rule_recurrent(q, k, v, g, beta, S0)
    o2, S2 = R.delta_rule_chunked(q, k, v, g, beta, S0, chunk=64)
    assert rel_err(o2, o1) < 1e-10 and rel_err(S2, S1) < 1e-10


def test_chunked_chunk_size_invariance():
    q, k, v, g, beta = _delta_inputs(B=1, H=2, T=96, d=16, seed=3)
    o1, S1 = R.delta_rule_chunked(q, k, v, g, beta, None, chunk=16)
    o2, S2 = R.delta_rule_chunked(q, k, v, g, beta, None, chunk=64)
    assert rel_err(o1, o2) < 1e-10 and rel_err(S1, S2) < 1e-10


def test_chunked_fp32_vs_fp64_at_scale():
    """The fp32 oracle itself stays far inside the 1e-3 bar at d = 128, T = 512."""
    q, k, v, g, beta = _delta_inputs(B=1, H=2, T=512, d=128, seed=5)
    o64, S64 = R.delta_rule_chunked(q, k, v, g, beta)
    o32, S32 = R.delta_rule_chunked(*(t.float() for t in (q, k, v, g, beta)))
    assert rel_err(o32, o64) < 1e-5 and rel_err(S32, S64) < 1e-5


def test_conv_silu_brute_force_and_streaming():
    B, T, C, K = 2, 9, 5, 4
    x = torch.randn(B, T, C, dtype=torch.float64)
    w = torch.randn(C, K, dtype=torch.float64)
    st = torch.randn(B, C, K - 1, dtype=torch.float64)
    y, ns = R.conv_silu(x, w, st)
    full = torch.cat([st.transpose(1, 2), x], 1)  # [B, K-1+T, C], oldest first
    yb = torch.zeros_like(x)
    for b in range(B):
        for t in range(T):
            for c in range(C):
                acc = sum(w[c, j].item() * full[b, t + j, c].item() for j in range(K))
                yb[b, t, c] = acc / (1 + math.exp(-acc))
    assert rel_err(y, yb) < 1e-12
    assert torch.equal(ns, full[:, -(K - 1):].transpose(1, 2))
    # feeding one token at a time gives the same outputs and state
    s = st.clone()
    ys = []
    for t in range(T):
        yt, s = R.conv_silu(x[:, t:t + 1], w, s)
        ys.append(yt)
    assert rel_err(torch.cat(ys, 1), y) < 1e-12 and torch.equal(s, ns)


def test_norms_closed_form():
    x = torch.randn(3, 16, dtype=torch.float64)
    w = torch.randn(16, dtype=torch.float64) * 0.1
    rms = (x.pow(2).mean(-1, keepdim=True) + 1e-6).sqrt()
    # znorm / gated_norm compute in fp32 by definition (hybrid.py:127, 143): fp32-level bar
    assert rel_err(R.znorm(x, w), x / rms * (1 + w)) < 1e-6
    z = torch.randn(3, 16, dtype=torch.float64)
    wg = torch.randn(16, dtype=torch.float64)
    assert rel_err(R.gated_norm(x, z, wg), wg * x / rms * z * torch.sigmoid(z)) < 1e-6
    assert rel_err(R.gated_norm(x, z, wg, act="sigmoid"), wg * x / rms * torch.sigmoid(z)) < 1e-6
    l2 = R.l2norm(x)
    assert rel_err(l2.norm(dim=-1), torch.ones(3, dtype=torch.float64)) < 1e-6


def test_delta_gates_closed_form():
    h = torch.randn(4, 32, dtype=torch.float64)
    wb, wa = torch.randn(3, 32, dtype=torch.float64), torch.randn(3, 32, dtype=torch.float64)
    a_log, dt = torch.randn(3, dtype=torch.float64), torch.randn(3, dtype=torch.float64)
    g, beta = R.delta_gates(h, wb, wa, a_log, dt)
    for t in range(4):
        for j in range(3):
            b_ = 1 / (1 + math.exp(-(h[t] @ wb[j]).item()))
            xx = (h[t] @ wa[j]).item() + dt[j].item()
            sp = xx if xx > 20 else math.log1p(math.exp(xx))
            # computed in fp32 by definition (hybrid.py:403-404 take .float())
            assert abs(beta[t, j].item() - b_) < 1e-6
            assert abs(g[t, j].item() + math.exp(a_log[j].item()) * sp) < 1e-5 * (1 + abs(sp))


def test_delta_prep_head_mapping():
    hk, hv, d = 2, 4, 8
    y = torch.randn(1, 1, 2 * hk * d + hv * d, dtype=torch.float64)
    q, k, v = R.delta_prep(y, hk, hv, d, d)
    for h in range(hv):
        kh = h // (hv // hk)
        qraw = y[0, 0, kh * d:(kh + 1) * d]
        kraw = y[0, 0, hk * d + kh * d: hk * d + (kh + 1) * d]
        # heads are cast to fp32 before the norm (hybrid.py:408): fp32-level bar
        assert rel_err(q[0, h, 0], qraw / (qraw.pow(2).sum() + 1e-6).sqrt() / math.sqrt(d)) < 1e-6
        assert rel_err(k[0, h, 0], kraw / (kraw.pow(2).sum() + 1e-6).sqrt()) < 1e-6
        assert torch.equal(v[0, h, 0], y[0, 0, 2 * hk * d + h * d: 2 * hk * d + (h + 1) * d].float())


def test_rope_identities():
    rd, theta = 64, 1e7
    inv = R.rope_inv_freq(rd, theta)
    assert inv[0].item() == 1.0
    # against the closed form evaluated in fp64
    for j in range(rd // 2):
        assert abs(inv[j].item() - theta ** (-2 * j / rd)) <= 1e-7 * theta ** (-2 * j / rd)
    x = torch.randn(5, 256, dtype=torch.float64)
    c0, s0 = R.rope_tables(rd, theta, torch.tensor([0]))
    assert torch.equal(R.apply_partial_rope(x, c0.double(), s0.double()), x)  # position 0 = identity
    pos = torch.tensor([7, 1000, 131072])
    c, s = R.rope_tables(rd, theta, pos)
    for p_i in range(3):
        y = R.apply_partial_rope(x[:1], c[p_i:p_i + 1].double(), s[p_i:p_i + 1].double())
        # pairs (j, j + rd/2) rotate by angle pos * inv_j; the rest pass through
        for j in (0, 5, 31):
            ang = float(pos[p_i]) * float(inv[j])
            a, b = x[0, j].item(), x[0, j + rd // 2].item()
            assert abs(y[0, j].item() - (a * math.cos(ang) - b * math.sin(ang))) < 1e-4
            assert abs(y[0, j + rd // 2].item() - (b * math.cos(ang) + a * math.sin(ang))) < 1e-4
        assert torch.equal(y[0, rd:], x[0, rd:])
        assert abs(y[0, :rd].norm().item() - x[0, :rd].norm().item()) < 1e-5


def _brute_attention(q, k, v, pos, G):
    """fp64 loops: softmax(q k^T / sqrt(HD)) v with causal offset and GQA h // G."""
    B, H, T, HD = q.shape
    out = torch.zeros(B, H, T, HD, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            for t in range(T):
                L = pos + t + 1
                s = [(q[b, h, t] @ k[b, h // G, l]).item() / math.sqrt(HD) for l in range(L)]
                m = max(s)
                p = [math.exp(x - m) for x in s]
                Z = sum(p)
                out[b, h, t] = sum(p[l] / Z * v[b, h // G, l] for l in range(L))
    return out


@pytest.mark.parametrize("T,pos", [(1, 0), (1, 9), (3, 0), (4, 5)])
def test_attention_core_brute_force(T, pos):
    B, H, KV, HD = 2, 4, 2, 16
    q = torch.randn(B, H, T, HD, dtype=torch.float64)
    kc = torch.randn(B, KV, pos + T + 3, HD, dtype=torch.float64)
    vc = torch.randn(B, KV, pos + T + 3, HD, dtype=torch.float64)
    y = R.attention_core(q, kc, vc, pos, KV)
    yb = _brute_attention(q, kc, vc, pos, H // KV)
    assert rel_err(y, yb) < 1e-6  # the oracle runs SDPA in fp32, as hybrid.py:300-309


def test_attention_single_key_is_gated_value():
    B, H, KV, HD = 1, 4, 2, 8
    qg = torch.randn(B, 1, H, 2 * HD, dtype=torch.float64)
    k = torch.randn(B, 1, KV, HD, dtype=torch.float64)
    v = torch.randn(B, 1, KV, HD, dtype=torch.float64)
    kc = torch.zeros(B, KV, 4, HD, dtype=torch.float64)
    vc = torch.zeros(B, KV, 4, HD, dtype=torch.float64)
    w = torch.zeros(HD, dtype=torch.float64)
    y = R.attention_decode(qg[:, 0], k[:, 0], v[:, 0], w, w, kc, vc, 0, 4, 1e7)
    gate = qg[:, 0, :, HD:]
    for h in range(H):
        assert rel_err(y[0, h], v[0, 0, h // 2] * torch.sigmoid(gate[0, h])) < 1e-6


# --- QLinear (model.py:78-93) and the engine matvec (aegist.cu:52-172) -------------------------

def test_qlinear_quantize_known_answer():
    """Rows chosen so the fp32 scale is exact: s = 1 and s = 2; q rounds half to even."""
    w = torch.tensor([[127.0, -63.5, 31.5, 0.49, -0.5],
                      [-254.0, 1.0, 3.0, 5.0, 253.0],
                      [0.0, 0.0, 0.0, 0.0, 0.0]])
    q, s = R.qlinear_quantize(w)
    assert q.dtype == torch.int8 and s.dtype == torch.bfloat16
    assert q[0].tolist() == [127, -64, 32, 0, 0]
    assert q[1].tolist() == [-127, 0, 2, 2, 126]  # 0.5 -> 0, 1.5 -> 2, 2.5 -> 2, 126.5 -> 126
    assert q[2].tolist() == [0, 0, 0, 0, 0]
    assert s[0].item() == 1.0 and s[1].item() == 2.0
    assert s[2].item() == torch.tensor(1e-8 / 127.0).to(torch.bfloat16).item()


def test_qlinear_quantize_round_trip_bound():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(64, 300, generator=g) * 0.02
    q, s = R.qlinear_quantize(w)
    s32 = w.abs().amax(1, keepdim=True) / 127.0
    assert (q.abs() <= 127).all() and (q.abs().amax(1) == 127).all()
    # with the fp32 scale the error is at most half a step
    assert ((q.float() * s32 - w).abs() <= s32 / 2 * (1 + 1e-5)).all()


def test_qlinear_engine_brute_force_and_identity():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 5, generator=g)
    q = torch.randint(-127, 128, (3, 5), generator=g, dtype=torch.int8)
    s = torch.rand(3, generator=g).to(torch.bfloat16)
    y = R.qlinear_engine(x, q, s)
    for m in range(2):
        for n in range(3):
            ref = sum(float(x[m, k]) * int(q[n, k]) for k in range(5)) * float(s[n])
            assert abs(float(y[m, n]) - ref) <= 1e-6 * (1 + abs(ref))
    # identity weight: q = 127 I, s = bf16(1/127) -> y = x * 127 * bf16(1/127)
    qi, si = R.qlinear_quantize(torch.eye(5))
    assert (qi == 127 * torch.eye(5, dtype=torch.int8)).all()
    yi = R.qlinear_engine(x, qi, si)
    assert torch.allclose(yi, x * (127 * float(si[0])), rtol=1e-6, atol=0)
    # accumulate adds; no scale means 1; linearity in x
    y0 = torch.randn(2, 3, generator=g)
    assert torch.allclose(R.qlinear_engine(x, q, s, y0, accumulate=True), y0 + y, atol=1e-6)
    assert torch.allclose(R.qlinear_engine(x, q, None), x @ q.float().t(), rtol=1e-6, atol=1e-5)
    x2 = torch.randn(2, 5, generator=g)
    assert torch.allclose(R.qlinear_engine(x + x2, q, s), y + R.qlinear_engine(x2, q, s), rtol=1e-5, atol=1e-4)


def test_qlinear_torch_module_form_matches_engine_form():
    """QLinear.forward dequantises first; in fp32 that differs from the engine's scale-after-dot
    form by rounding only."""
    g = torch.Generator().manual_seed(2)
    w = torch.randn(40, 256, generator=g) * 0.02
    x = torch.randn(7, 256, generator=g)
    q, s = R.qlinear_quantize(w)
    assert rel_err(R.qlinear_torch(x, q, s), R.qlinear_engine(x, q, s)) < 1e-5
    # and both approximate the unquantised linear to the int8 step size
    assert rel_err(R.qlinear_engine(x, q, s), x @ w.t()) < 2e-2


# --- QSA indexer (hc.py:237-283; next.cu:488-705) -------------------------------------------

def test_idx_select_known_answers():
    sc = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0, 0.0, 0.0, 0.0]])
    # position 7 with R = 1: 8 complete blocks; top 2 of {3, 3, 3} go to the lower blocks
    assert R.idx_select(sc, top=2, R=1, pos0=7) == [[1, 2]]
    assert R.idx_select(sc, top=4, R=1, pos0=7) == [[1, 2, 3, 4]]
    # at most `top` complete blocks: all of them, whatever the scores
    assert R.idx_select(sc, top=8, R=1, pos0=7) == [[0, 1, 2, 3, 4, 5, 6, 7]]
    # R = 2, position 4: (4 + 1) // 2 = 2 complete blocks <= top 3
    assert R.idx_select(sc, top=3, R=2, pos0=4) == [[0, 1]]
    # all-zero scores (every head's dot product negative): the lowest blocks
    assert R.idx_select(torch.zeros(1, 10), top=3, R=1, pos0=9) == [[0, 1, 2]]


def test_idx_scores_and_blocks_brute_force():
    g = torch.Generator().manual_seed(3)
    T, H, HD, RB, pos0 = 2, 3, 8, 2, 5
    qi = torch.randn(T, H, HD, generator=g)
    bk = torch.randn(4, HD, generator=g)
    sc = R.idx_scores(qi, bk, pos0, RB)
    for t in range(T):
        for b in range(4):
            if b >= (pos0 + t + 1) // RB:
                assert sc[t, b] == float("-inf")
                continue
            want = sum(max(0.0, sum(float(qi[t, h, i]) * float(bk[b, i]) for i in range(HD))) for h in range(H))
            assert abs(float(sc[t, b]) - want / math.sqrt(HD)) < 1e-5 * (1 + abs(want))
    # block keys: R = 1 is rope(znorm(key)) at the key's own position; R = 2 averages pairs
    kraw = torch.randn(8, 128, generator=g)
    kw = torch.randn(128, generator=g) * 0.1
    one = R.idx_blocks(kraw, kw, 1, 0, 8, 64, 1e7)
    cos, sin = R.rope_tables(64, 1e7, torch.arange(8))
    assert torch.allclose(one, R.apply_partial_rope(R.znorm(kraw, kw), cos, sin), atol=1e-6)
    two = R.idx_blocks(kraw, kw, 2, 1, 3, 64, 1e7)
    mean = (kraw[2:8:2] + kraw[3:8:2]) / 2
    cos, sin = R.rope_tables(64, 1e7, torch.tensor([2, 4, 6]))
    assert torch.allclose(two, R.apply_partial_rope(R.znorm(mean, kw), cos, sin), atol=1e-6)


def test_engine_list_form_equals_hc_mask_form():
    """The engine's block lists + tail select exactly the keys of hc.py's mask, and attention
    over them equals SDPA with that mask (hc.py:298-299)."""
    g = torch.Generator().manual_seed(4)
    T, H, KV, HD, RB, top, pos0 = 6, 4, 2, 32, 4, 5, 60
    L = pos0 + T
    nb = L // RB
    sc = torch.rand(T, nb, generator=g)  # continuous: no ties
    vis = (torch.arange(pos0, L) + 1) // RB
    sc = sc.masked_fill(torch.arange(nb).view(1, -1) >= vis.view(-1, 1), float("-inf"))
    lists = R.idx_select(sc, top, RB, pos0)
    mask = R.qsa_mask(sc, top, RB, pos0, L)
    for t in range(T):
        p = pos0 + t
        keys = {b * RB + j for b in lists[t] for j in range(RB)} | set(range((p + 1) // RB * RB, p + 1))
        assert set(torch.nonzero(mask[t]).flatten().tolist()) == keys
    q = torch.randn(T, H, HD, generator=g)
    kc = torch.randn(KV, L, HD, generator=g)
    vc = torch.randn(KV, L, HD, generator=g)
    qg = torch.randn(T, H, 2 * HD, generator=g)
    got = R.attention_list(q, kc, vc, qg, pos0, lists, RB)
    k = kc.repeat_interleave(H // KV, 0).unsqueeze(0)
    v = vc.repeat_interleave(H // KV, 0).unsqueeze(0)
    y = F.scaled_dot_product_attention(q.transpose(0, 1).unsqueeze(0), k, v, attn_mask=mask)[0].transpose(0, 1)
    assert torch.allclose(got, y * torch.sigmoid(qg[..., HD:]), atol=1e-5)


def test_gated_norm_sigmoid_gate_closed_form():
    g = torch.Generator().manual_seed(5)
    o, z, w = torch.randn(3, 16, generator=g), torch.randn(3, 16, generator=g), torch.randn(16, generator=g)
    rms = torch.sqrt((o.double() ** 2).mean(-1, keepdim=True) + 1e-6)
    want = w.double() * (o.double() / rms) / (1 + torch.exp(-z.double()))
    assert torch.allclose(R.gated_norm(o, z, w, act="sigmoid").double(), want, atol=1e-6)


# --- mixture of experts -----------------------------------------------------------------------

def test_q4_dequantize_known_answers():
    # byte 0x21 holds codes (1, 2): the even element in the low nibble; 0xF0 holds (0, 15)
    packed = torch.zeros(1, 32, dtype=torch.uint8)
    packed[0, 0], packed[0, 1] = 0x21, 0xF0
    scale = torch.tensor([[0.5]], dtype=torch.float16)
    mn = torch.tensor([[-1.0]], dtype=torch.float16)
    w = R.q4_dequantize(packed, scale, mn, 64)
    assert w.shape == (1, 64)
    assert w[0, :4].tolist() == [-0.5, 0.0, -1.0, 6.5]
    assert torch.all(w[0, 4:] == -1.0)


def test_expert_row_layout_by_hand():
    # D = 128, I = 64, group 64: place single codes by hand-computed byte offsets and read them
    # back through unpack_expert (gate rows first, then up rows, then the down matrix)
    D, I = 128, 64
    gu_q, gu_s = 2 * I * D // 2, 2 * I * (D // 64) * 2
    dn_q, dn_s = D * I // 2, D * (I // 64) * 2
    assert R.expert_row_bytes(D, I) == -(-(gu_q + 2 * gu_s + dn_q + 2 * dn_s) // 64) * 64
    row = torch.zeros(R.expert_row_bytes(D, I), dtype=torch.uint8)
    one = torch.tensor([1.0], dtype=torch.float16).view(torch.uint8)  # f16 1.0 = bytes 00 3c
    row[gu_q:gu_q + gu_s].view(torch.float16)[:] = 1.0     # every gate/up scale 1, min 0
    row[gu_q + 2 * gu_s + dn_q:gu_q + 2 * gu_s + dn_q + dn_s].view(torch.float16)[:] = 1.0
    row[(I + 5) * (D // 2) + 7] = 0x30                     # up row 5, input 15 -> code 3
    row[gu_q + 2 * gu_s + 9 * (I // 2) + 2] = 0x07         # down row 9, input 4 -> code 7
    assert one.tolist() == [0, 60]
    gu, dn = R.unpack_expert(row, D, I)
    nz = gu.nonzero().tolist()
    assert nz == [[I + 5, 15]] and gu[I + 5, 15] == 3.0
    assert dn.nonzero().tolist() == [[9, 4]] and dn[9, 4] == 7.0


def test_route_ties_and_brute_force():
    # equal logits: the lower experts first, equal weights
    h = torch.ones(2, 8)
    W = torch.ones(6, 8, dtype=torch.bfloat16)
    idx, wts = R.route(h, W, 3)
    assert idx.tolist() == [[0, 1, 2], [0, 1, 2]]
    assert torch.allclose(wts, torch.full((2, 3), 1 / 3, dtype=torch.float64))
    g = torch.Generator().manual_seed(7)
    h = torch.randn(5, 16, generator=g)
    W = torch.randn(12, 16, generator=g).bfloat16()
    idx, wts = R.route(h, W, 4)
    for t in range(5):
        lg = [sum(float(h[t, d]) * float(W[e, d]) for d in range(16)) for e in range(12)]
        m = max(lg)
        p = [math.exp(v - m) for v in lg]
        p = [v / sum(p) for v in p]
        best = sorted(range(12), key=lambda e: (-p[e], e))[:4]
        assert idx[t].tolist() == best
        s = sum(p[e] for e in best)
        assert all(abs(float(wts[t, i]) - p[e] / s) < 1e-12 for i, e in enumerate(best))


def test_expert_ffn_and_bank_brute_force():
    g = torch.Generator().manual_seed(8)
    D, I, E = 64, 64, 3
    rows = []
    for _ in range(E):
        rows.append(R.pack_expert(torch.randint(0, 16, (2 * I, D), generator=g),
                                  (torch.rand(2 * I, 1, generator=g) * 0.01).half(),
                                  (-torch.rand(2 * I, 1, generator=g) * 0.05).half(),
                                  torch.randint(0, 16, (D, I), generator=g),
                                  (torch.rand(D, 1, generator=g) * 0.01).half(),
                                  (-torch.rand(D, 1, generator=g) * 0.05).half()))
    rows = torch.stack(rows)
    h = torch.randn(4, D, generator=g)
    idx = torch.tensor([[0, 2], [1, 1], [2, 0], [9, 1]])  # expert 9 is out of range: adds nothing
    wts = torch.tensor([[0.75, 0.25], [0.5, 0.5], [0.9, 0.1], [0.3, 0.7]])
    got = R.moe_experts(h, rows, idx, wts, D, I)
    for t in range(4):
        want = [0.0] * D
        for k in range(2):
            e = int(idx[t, k])
            if e >= E:
                continue
            gu, dn = R.unpack_expert(rows[e], D, I)
            a = []
            for r in range(I):
                gate = sum(float(gu[r, c]) * float(h[t, c]) for c in range(D))
                up = sum(float(gu[I + r, c]) * float(h[t, c]) for c in range(D))
                a.append(gate / (1 + math.exp(-gate)) * up)
            for o in range(D):
                want[o] += float(wts[t, k]) * sum(float(dn[o, r]) * a[r] for r in range(I))
        assert torch.allclose(got[t], torch.tensor(want, dtype=torch.float64), rtol=1e-9, atol=1e-9)


def test_moe_forward_shared_gate():
    g = torch.Generator().manual_seed(9)
    D, I, E = 64, 64, 4
    rows = torch.stack([R.pack_expert(torch.randint(0, 16, (2 * I, D), generator=g), torch.full((2 * I, 1), 0.01),
                                      torch.full((2 * I, 1), -0.05), torch.randint(0, 16, (D, I), generator=g),
                                      torch.full((D, 1), 0.01), torch.full((D, 1), -0.05)) for _ in range(E)])
    h = torch.randn(3, D, generator=g)
    W = torch.randn(E, D, generator=g).bfloat16()
    ysh = torch.randn(3, D, generator=g)
    wg = torch.randn(D, generator=g).bfloat16()
    out, idx, wts = R.moe_forward(h, W, rows, D, I, 2, ysh=ysh, shared_gate=wg)
    routed = R.moe_experts(h, rows, idx, wts, D, I)
    for t in range(3):
        s = sum(float(h[t, d]) * float(wg[d]) for d in range(D))
        gate = 1 / (1 + math.exp(-s))
        assert torch.allclose(out[t], routed[t] + gate * ysh[t].double(), atol=1e-12)
