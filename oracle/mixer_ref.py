"""CPU restatement of the Aegist token-mixer ops (torch-CPU, fp32 unless stated).

TEST INFRASTRUCTURE ONLY. This module is the checker that the HIP kernels are compared
against; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
it. The product path (the HIP library and its bindings) never calls into it.

Every function restates one op of the reference's torch model, written from the equations
in /root/reference/aegist-fast-35b/aegist/hybrid.py (cited per function as
``hybrid.py:<lines>``) and the engine conventions of aegist_rs/kernels/hybrid.cu. Layouts
follow the reference: DeltaNet tensors heads-first ``[B, H, T, d]``; attention caches
``[B, KV, cap, HD]``.

Pinning (how each function is checked independently of its own formula) lives in
tests/test_oracle_pins.py: fp64 brute force, closed-form special cases, chunked-vs-recurrent
equivalence, one-at-a-time-vs-all-at-once conv, RoPE identities and norm preservation.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


# --- norms (hybrid.py:119-147) --------------------------------------------------------------

def znorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Zero-centred RMSNorm ``(1 + w) * x / rms(x)`` in fp32 (hybrid.py:119-130)."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * (1.0 + w.float())).to(x.dtype)


def gated_norm(x: torch.Tensor, z: torch.Tensor, w: torch.Tensor, eps: float = 1e-6,
               act: str = "silu") -> torch.Tensor:
    """``w * rmsnorm(x) * act(z)`` per value head (hybrid.py:133-147).

    The normalised x is cast back to x.dtype before the weight multiply (hybrid.py:145) and
    the gate is computed in fp32 (hybrid.py:146)."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    y = w * xf.to(x.dtype)
    g = torch.sigmoid(z.float()) if act == "sigmoid" else F.silu(z.float())
    return (y * g).to(x.dtype)


# --- position (hybrid.py:152-166) ------------------------------------------------------------

def rope_inv_freq(rotary_dim: int, theta: float) -> torch.Tensor:
    """``1 / theta^(2j / rd)`` for j < rd/2, as fp32.

    hybrid.py:154 evaluates this with torch's fp32 ``pow``. This build evaluates it in fp64
    and rounds once to fp32, and the HIP library is handed the identical table (computed the
    same way on the host), so CPU and GPU angles agree to the last bit of ``pos * inv``."""
    j = torch.arange(0, rotary_dim, 2, dtype=torch.float64)
    return (1.0 / (theta ** (j / rotary_dim))).to(torch.float32)


def rope_tables(rotary_dim: int, theta: float, positions: torch.Tensor):
    """cos/sin tables ``[len(positions), rd]`` with ``emb = cat(f, f)`` (hybrid.py:152-157)."""
    inv = rope_inv_freq(rotary_dim, theta)
    f = torch.outer(positions.to(torch.float32), inv)  # fp32 product, as hybrid.py:155
    emb = torch.cat([f, f], -1)
    return emb.cos(), emb.sin()


def apply_partial_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE on the first ``cos.shape[-1]`` dims; pass the rest (hybrid.py:160-166)."""
    rd = cos.shape[-1]
    xr, xp = x[..., :rd], x[..., rd:]
    h = rd // 2
    rot = torch.cat([-xr[..., h:], xr[..., :h]], -1)
    return torch.cat([xr * cos.to(x.dtype) + rot * sin.to(x.dtype), xp], -1)


# --- gated DeltaNet (hybrid.py:314-421) ------------------------------------------------------

def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``x * rsqrt(sum(x^2) + eps)`` over the last dim (hybrid.py:314-315)."""
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def delta_rule_step(q, k, v, g, beta, state):
    """One token of the gated delta rule (hybrid.py:318-324).

    q, k ``[B,H,dk]``; v ``[B,H,dv]``; g, beta ``[B,H]``; state ``[B,H,dk,dv]`` fp32, updated
    in place. Returns o ``[B,H,dv]``."""
    state.mul_(g.exp()[..., None, None])
    kv_mem = (state * k.unsqueeze(-1)).sum(-2)
    delta = (v - kv_mem) * beta.unsqueeze(-1)
    state.add_(k.unsqueeze(-1) * delta.unsqueeze(-2))
    return (state * q.unsqueeze(-1)).sum(-2)


def delta_rule_recurrent(q, k, v, g, beta, state=None):
    """``delta_rule_step`` looped over T (the form hybrid.py:411-413 takes one token at a time).

    q, k ``[B,H,T,dk]``; v ``[B,H,T,dv]``; g, beta ``[B,H,T]``. Returns (o, final state)."""
    B, H, T, dk = k.shape
    dv = v.shape[-1]
    S = torch.zeros(B, H, dk, dv, dtype=q.dtype) if state is None else state.clone().to(q.dtype)
    outs = [delta_rule_step(q[:, :, t], k[:, :, t], v[:, :, t], g[:, :, t], beta[:, :, t], S) for t in range(T)]
    o = torch.stack(outs, 2) if outs else torch.zeros(B, H, 0, dv, dtype=q.dtype)
    return o, S


def delta_rule_chunked(q, k, v, g, beta, state=None, chunk: int = 64):
    """Chunked WY/UT form of the gated delta rule (hybrid.py:327-361).

    Pads T to a multiple of ``chunk`` (hybrid.py:336-339); per chunk with ``cum = cumsum(g)``:
    ``A = (kb k^T) o decay`` solved as a unit lower-triangular system (diagonal ignored) for
    ``u = A^-1 vb`` and ``w = A^-1 (kb e^cum)``; ``intra = (q k^T) o decay`` (diagonal kept);
    then sequentially ``v_new = u - w S; o = (q e^cum) S + intra v_new;
    S = S e^{cum_last} + (k e^{cum_last - cum})^T v_new``."""
    B, H, T, dk = k.shape
    dv = v.shape[-1]
    pad = (chunk - T % chunk) % chunk
    if pad:
        q, k, v = (F.pad(t, (0, 0, 0, pad)) for t in (q, k, v))
        g, beta = (F.pad(t, (0, pad)) for t in (g, beta))
    n = (T + pad) // chunk
    kb = (k * beta.unsqueeze(-1)).view(B, H, n, chunk, dk)
    vb = (v * beta.unsqueeze(-1)).view(B, H, n, chunk, dv)
    q, k = q.reshape(B, H, n, chunk, dk), k.reshape(B, H, n, chunk, dk)
    cum = g.reshape(B, H, n, chunk).cumsum(-1)
    upper = torch.ones(chunk, chunk, dtype=torch.bool).triu(1)
    decay = (cum.unsqueeze(-1) - cum.unsqueeze(-2)).masked_fill(upper, float("-inf")).exp()
    system = (kb @ k.transpose(-1, -2)) * decay
    u = torch.linalg.solve_triangular(system, vb, upper=False, unitriangular=True)
    w = torch.linalg.solve_triangular(system, kb * cum.exp().unsqueeze(-1), upper=False, unitriangular=True)
    intra = (q @ k.transpose(-1, -2)) * decay
    q_dec = q * cum.exp().unsqueeze(-1)
    k_dec = k * (cum[..., -1:] - cum).exp().unsqueeze(-1)
    chunk_decay = cum[..., -1].exp()[..., None, None]
    S = torch.zeros(B, H, dk, dv, dtype=q.dtype) if state is None else state.to(q.dtype).clone()
    outs = []
    for i in range(n):
        v_new = u[:, :, i] - w[:, :, i] @ S
        outs.append(q_dec[:, :, i] @ S + intra[:, :, i] @ v_new)
        S = S * chunk_decay[:, :, i] + k_dec[:, :, i].transpose(-1, -2) @ v_new
    out = torch.stack(outs, 2).reshape(B, H, n * chunk, dv)[:, :, :T]
    return out, S


def conv_silu(x: torch.Tensor, w: torch.Tensor, state: torch.Tensor | None):
    """Depthwise causal conv (kernel K) continuing from the K-1 previous inputs, then SiLU.

    x ``[B,T,C]``; w ``[C,K]`` (w[:, K-1] multiplies the newest input); state ``[B,C,K-1]``
    oldest first, or None for zeros. Returns (y ``[B,T,C]``, new state ``[B,C,K-1]``) — the
    new state is the last K-1 inputs of ``cat(state, x)`` (hybrid.py:393-398; the engine's
    conv_silu in hybrid.cu:205-221 has the same contract)."""
    B, T, C = x.shape
    K = w.shape[1]
    prev = torch.zeros(B, C, K - 1, dtype=x.dtype) if state is None else state.to(x.dtype)
    xp = torch.cat([prev, x.transpose(1, 2)], -1)
    new_state = xp[..., -(K - 1):].clone()
    y = F.silu(F.conv1d(xp, w.to(x.dtype).unsqueeze(1), groups=C)).transpose(1, 2)
    return y, new_state


def delta_gates(h, wb, wa, a_log, dt_bias):
    """``beta = sigmoid(h Wb^T)``, ``g = -exp(A_log) softplus(h Wa^T + dt_bias)`` (hybrid.py:403-404;
    F.softplus has threshold 20, as hybrid.cu:195). h ``[..., D]``; wb, wa ``[HV, D]``."""
    beta = (h.float() @ wb.float().t()).sigmoid()
    g = -a_log.float().exp() * F.softplus(h.float() @ wa.float().t() + dt_bias.float())
    return g, beta


def delta_prep(y: torch.Tensor, hk: int, hv: int, dk: int, dv: int, eps: float = 1e-6):
    """Split post-conv rows ``y [B,T,2*hk*dk + hv*dv]`` into heads-first q, k, v
    ``[B,HV,T,d]`` with the QK heads repeated ``hv/hk`` times, q and k L2-normalised and q
    scaled by ``dk^-1/2`` (hybrid.py:399-410)."""
    B, T, _ = y.shape
    q, k, v = y.split([hk * dk, hk * dk, hv * dv], -1)
    q, k, v = q.reshape(B, T, hk, dk), k.reshape(B, T, hk, dk), v.reshape(B, T, hv, dv)
    r = hv // hk
    if r > 1:
        q, k = q.repeat_interleave(r, 2), k.repeat_interleave(r, 2)
    q, k, v = (t.transpose(1, 2).float() for t in (q, k, v))
    q, k = l2norm(q, eps), l2norm(k, eps)
    return q * dk ** -0.5, k, v


def delta_decode_fused(qkv, conv_w, conv_state, g, beta, state, hk: int, hv: int, d: int = 128):
    """One decode token of a gated DeltaNet layer from the pre-conv projection onwards:
    conv state update + depthwise conv + SiLU + split + L2-norm + q-scale + delta step
    (hybrid.py:390-413 with T == 1 and history).

    qkv ``[B,C]``; conv_w ``[C,4]``; conv_state ``[B,C,3]`` (returned updated, new tensor);
    g, beta ``[B,HV]``; state ``[B,HV,d,d]`` (updated in place). Returns (o ``[B,HV,d]``,
    new conv state)."""
    y, new_conv = conv_silu(qkv.float().unsqueeze(1), conv_w.float(), conv_state.float())
    q, k, v = delta_prep(y, hk, hv, d, d)
    o = delta_rule_step(q[:, :, 0], k[:, :, 0], v[:, :, 0], g.float(), beta.float(), state)
    return o, new_conv


# --- gated attention (hybrid.py:265-311) ----------------------------------------------------

def attn_prep(qg, k, v, q_norm_w, k_norm_w, kc, vc, pos: int, rotary_dim: int, theta: float,
              eps: float = 1e-6):
    """ZNorm of q (first HD of each head's ``[query | gate]``) and of k, partial RoPE at
    positions ``pos..pos+T-1``, and the k/v append into the cache (hybrid.py:284-296).

    qg ``[B,T,H,2HD]``; k, v ``[B,T,KV,HD]``; kc, vc ``[B,KV,cap,HD]`` (written in their own
    dtype, e.g. bf16, at ``pos:pos+T``). Returns (q ``[B,H,T,HD]`` fp32, gate ``[B,T,H*HD]``)."""
    B, T, H, HD2 = qg.shape
    HD = HD2 // 2
    KV = k.shape[2]
    q, gate = qg.float().chunk(2, -1)
    gate = gate.reshape(B, T, H * HD)
    q = znorm(q, q_norm_w, eps).transpose(1, 2)
    kk = znorm(k.float(), k_norm_w, eps).transpose(1, 2)
    vv = v.float().transpose(1, 2)
    cos, sin = rope_tables(rotary_dim, theta, torch.arange(pos, pos + T))
    q, kk = apply_partial_rope(q, cos, sin), apply_partial_rope(kk, cos, sin)
    kc[:, :, pos:pos + T] = kk.to(kc.dtype)
    vc[:, :, pos:pos + T] = vv.to(vc.dtype)
    return q, gate


def attention_core(q, kc, vc, pos: int, n_kv: int):
    """Causal GQA softmax attention of T queries at positions ``pos..pos+T-1`` over cache
    rows ``[0, pos+T)`` (hybrid.py:297-309: grouped SDPA at T == 1, causal / ``tril(pos)``
    mask otherwise). q ``[B,H,T,HD]``; kc, vc ``[B,KV,cap,HD]``. Query head h reads KV head
    ``h // (H/KV)``. Returns ``[B,H,T,HD]`` fp32."""
    B, H, T, HD = q.shape
    g = H // n_kv
    k = kc[:, :, :pos + T].float().repeat_interleave(g, 1)
    v = vc[:, :, :pos + T].float().repeat_interleave(g, 1)
    mask = torch.ones(T, pos + T, dtype=torch.bool).tril(pos)
    return F.scaled_dot_product_attention(q.float(), k, v, attn_mask=mask)


def gated_attention_out(y, gate):
    """``y * sigmoid(gate)`` with y ``[B,H,T,HD]`` -> ``[B,T,H*HD]`` (hybrid.py:310)."""
    B, H, T, HD = y.shape
    return y.transpose(1, 2).reshape(B, T, H * HD) * torch.sigmoid(gate.float())


def attention_decode(qg, k_new, v_new, q_norm_w, k_norm_w, kc, vc, pos: int, rotary_dim: int,
                     theta: float, eps: float = 1e-6):
    """One query token per sequence: attn_prep at ``pos`` then attention over ``pos+1`` keys
    and the sigmoid gate (hybrid.py:280-310 with T == 1). qg ``[B,H,2HD]``; k_new, v_new
    ``[B,KV,HD]``. Returns ``[B,H,HD]`` fp32; writes the new k/v into the caches."""
    B, H, HD2 = qg.shape
    KV = k_new.shape[1]
    q, gate = attn_prep(qg.unsqueeze(1), k_new.unsqueeze(1), v_new.unsqueeze(1), q_norm_w, k_norm_w,
                        kc, vc, pos, rotary_dim, theta, eps)
    y = attention_core(q, kc, vc, pos, KV)
    return gated_attention_out(y, gate).reshape(B, H, HD2 // 2)


# --- QSA sparse-attention indexer of the second core (hc.py:237-283; next.cu:488-705) ------

def idx_prep(qk, qw, pos0: int, rotary_dim: int, theta: float, eps: float = 1e-6):
    """qk ``[T, (H+1), HD]`` (H index query heads, then the index key). Returns
    (qi ``[T, H, HD]`` = rope(znorm_qw(q)) at positions pos0.., kraw ``[T, HD]`` the raw keys)
    (hc.py:255, 264; next.cu:488-503)."""
    T = qk.shape[0]
    q, k = qk[:, :-1].float(), qk[:, -1].float()
    cos, sin = rope_tables(rotary_dim, theta, torch.arange(pos0, pos0 + T))
    qi = apply_partial_rope(znorm(q, qw.float(), eps), cos.unsqueeze(1), sin.unsqueeze(1))
    return qi, k


def idx_blocks(kraw, kw, R: int, b0: int, n: int, rotary_dim: int, theta: float, eps: float = 1e-6):
    """Block keys b0 .. b0+n-1: the mean of R raw keys, znorm_kw, rope at the block's first
    position b R (hc.py:265-268 with fp32 keys, as the engine keeps them; next.cu:505-520).
    kraw ``[>= (b0+n) R, HD]`` fp32. Returns ``[n, HD]``."""
    HD = kraw.shape[-1]
    blocks = kraw[b0 * R:(b0 + n) * R].float().view(n, R, HD)
    m = blocks[:, 0].clone()
    for j in range(1, R):  # summed in order, then divided, as the engine does
        m = m + blocks[:, j]
    m = m / R
    cos, sin = rope_tables(rotary_dim, theta, torch.arange(b0, b0 + n) * R)
    return apply_partial_rope(znorm(m, kw.float(), eps), cos, sin)


def idx_scores(qi, bk, pos0: int, R: int):
    """``sc[t, b] = sum_h relu(qi[t, h] . bk[b]) / sqrt(HD)`` for the blocks complete at the
    query's position, -inf elsewhere (hc.py:269-273; next.cu:522-541). Returns ``[T, nb]``."""
    T, H, HD = qi.shape
    nb = bk.shape[0]
    d = torch.einsum("thd,nd->thn", qi.double(), bk.double())
    sc = (torch.relu(d).sum(1) / math.sqrt(HD)).float()
    vis = (torch.arange(pos0, pos0 + T) + 1) // R
    return sc.masked_fill(torch.arange(nb).view(1, -1) >= vis.view(-1, 1), float("-inf"))


def idx_select(sc, top: int, R: int, pos0: int):
    """Per query: every complete block when there are at most ``top`` of them, else the ``top``
    highest scores with ties going to the lower block, listed in block order (next.cu:543-625;
    hc.py:274-278 leaves the tie order to torch.topk). Returns a list of block-index lists."""
    out = []
    for t in range(sc.shape[0]):
        n = (pos0 + t + 1) // R
        if n <= top:
            out.append(list(range(n)))
            continue
        s = sc[t, :n].tolist()
        order = sorted(range(n), key=lambda b: (-s[b], b))
        out.append(sorted(order[:top]))
    return out


def attention_list(q, kc, vc, qg, pos0: int, lists, R: int):
    """attention_gated over each query's listed blocks plus its own incomplete block
    (next.cu:627-705; hc.py:279-283 as a mask). q ``[T, H, HD]`` (normed, roped), kc / vc
    ``[KV, cap, HD]``, qg ``[T, H, 2 HD]`` (gate = second half). Returns ``[T, H, HD]`` fp32."""
    T, H, HD = q.shape
    KV = kc.shape[0]
    g = H // KV
    out = torch.empty(T, H, HD)
    for t in range(T):
        p = pos0 + t
        complete = (p + 1) // R
        keys = [b * R + j for b in lists[t] for j in range(R)] + list(range(complete * R, p + 1))
        idx = torch.tensor(keys, dtype=torch.long)
        for h in range(H):
            k = kc[h // g, idx].double()
            v = vc[h // g, idx].double()
            a = torch.softmax(k @ q[t, h].double() / math.sqrt(HD), 0)
            out[t, h] = ((a @ v) * torch.sigmoid(qg[t, h, HD:].double())).float()
    return out


def qsa_mask(sc, top: int, R: int, pos0: int, L: int):
    """The indexer's output in hc.py's form (hc.py:270-283): a bool mask ``[T, L]`` of the keys
    each query attends to (chosen blocks' tokens, its own incomplete block, causal). Picks with
    torch.topk, so ties are resolved however torch resolves them."""
    T, nb = sc.shape
    p = torch.arange(pos0, pos0 + T)
    complete = (p + 1) // R
    k_top = min(top, nb)
    chosen = torch.zeros(T, nb, dtype=torch.bool)
    chosen.scatter_(-1, sc.topk(k_top, -1).indices, True)
    chosen &= torch.isfinite(sc)
    tok = chosen.repeat_interleave(R, -1)
    tail = torch.arange(L).view(1, -1) >= (complete * R).view(-1, 1)
    causal = torch.arange(L).view(1, -1) <= p.view(-1, 1)
    return (F.pad(tok, (0, L - nb * R)) | tail) & causal


# --- projections: QLinear (model.py:78-93) and the engine matvecs (aegist.cu:52-172) --------

def qlinear_quantize(weight: torch.Tensor):
    """QLinear.__init__ (model.py:84-90): per-output-row absmax scale
    s = max|w_row| (clamped at 1e-8) / 127; q = round(w / s) as int8 (round half to even);
    the scale is kept in bf16 (after q was computed with the fp32 scale)."""
    w = weight.float()
    s = w.abs().amax(1, keepdim=True).clamp(min=1e-8) / 127.0
    q = torch.round(w / s).to(torch.int8)
    return q, s.to(torch.bfloat16).reshape(-1)


def qlinear_engine(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor | None, y: torch.Tensor | None = None,
                   accumulate: bool = False) -> torch.Tensor:
    """The engine's int8 / bf16 matvec and matmul (aegist.cu:52-63 row_dot_i8, :85-91 gemv_i8,
    :108-124 gemv_bf16, :126-172 gemm_i8): fp32 dot of the fp32 activation row with the weight
    row (int8 or bf16 values taken exactly), times the row scale, optionally added into y.
    Summed in fp64 here so the restatement carries no rounding of its own."""
    acc = x.double() @ q.double().t()
    if scale is not None:
        acc = acc * scale.double()
    acc = acc.float()
    if accumulate:
        return y.float() + acc
    return acc


def qlinear_torch(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """QLinear.forward (model.py:92-93): F.linear(x, q.to(x.dtype) * scale.to(x.dtype)) - the
    weight is dequantised in the activation dtype (bf16 rounding of q*s in a bf16 model)."""
    w = q.to(x.dtype) * scale.to(x.dtype).reshape(-1, 1)
    return F.linear(x, w)


# --- mixture of experts (hybrid.py:424-652; engine hybrid.cu:313-577) ------------------------
# Computed in fp64 from the exact stored values (fp32 activations, bf16 router, f16 scales).

def q4_dequantize(packed: torch.Tensor, scale: torch.Tensor, mn: torch.Tensor, group: int = 64) -> torch.Tensor:
    """hybrid.py:463-469: two 4-bit codes per byte, the even element in the low nibble;
    w = code * scale + min per `group` consecutive inputs. Returns fp64 [..., 2 * packed.shape[-1]]."""
    lo = (packed & 0xF).double()
    hi = (packed >> 4).double()
    code = torch.stack([lo, hi], -1).flatten(-2)
    *lead, n = code.shape
    code = code.view(*lead, n // group, group)
    return (code * scale.double().unsqueeze(-1) + mn.double().unsqueeze(-1)).reshape(*lead, n)


def expert_layout(D: int, I: int, group: int = 64):
    """hybrid.py:472-482: the sections of one 4-bit expert row, in order: (name, shape, dtype)."""
    return [("gu_q", (2 * I, D // 2), torch.uint8), ("gu_s", (2 * I, D // group), torch.float16),
            ("gu_m", (2 * I, D // group), torch.float16), ("dn_q", (D, I // 2), torch.uint8),
            ("dn_s", (D, I // group), torch.float16), ("dn_m", (D, I // group), torch.float16)]


def expert_row_bytes(D: int, I: int, group: int = 64) -> int:
    """hybrid.py:485-487: the section bytes, rounded up to 64."""
    n = sum(math.prod(shape) * torch.tensor([], dtype=dt).element_size() for _, shape, dt in expert_layout(D, I, group))
    return -(-n // 64) * 64


def pack_codes(codes: torch.Tensor) -> torch.Tensor:
    """uint8 codes [..., n] in 0..15 -> [..., n / 2], the even element in the low nibble (hybrid.py:460)."""
    c = codes.to(torch.uint8)
    return c[..., 0::2] | (c[..., 1::2] << 4)


def pack_expert(gu_codes, gu_s, gu_m, dn_codes, dn_s, dn_m) -> torch.Tensor:
    """One expert row (uint8 [expert_row_bytes]) from codes [2I, D] / [D, I] and f16 scales and mins."""
    D = gu_codes.shape[1]
    I = dn_codes.shape[1]
    parts = [pack_codes(gu_codes), gu_s.half(), gu_m.half(), pack_codes(dn_codes), dn_s.half(), dn_m.half()]
    row = torch.cat([p.contiguous().view(torch.uint8).reshape(-1) for p in parts])
    return F.pad(row, (0, expert_row_bytes(D, I) - row.numel()))


def unpack_expert(row: torch.Tensor, D: int, I: int, group: int = 64):
    """hybrid.py:536-548 (4-bit branch): one row -> (gate_up [2I, D], down [D, I]) in fp64."""
    out, off = {}, 0
    for name, shape, dt in expert_layout(D, I, group):
        nb = math.prod(shape) * torch.tensor([], dtype=dt).element_size()
        out[name] = row[off:off + nb].view(dt).view(shape)
        off += nb
    return (q4_dequantize(out["gu_q"], out["gu_s"], out["gu_m"], group),
            q4_dequantize(out["dn_q"], out["dn_s"], out["dn_m"], group))


def route(h: torch.Tensor, W: torch.Tensor, K: int):
    """MoE.route (hybrid.py:637-641) with the engine's tie rule (equal probabilities: the lower
    expert first, hybrid.cu:30-39): p = softmax(h W^T), the K largest in descending order,
    weights p / sum(top p). h fp32 [T, D], W bf16 [E, D]. Returns (idx int64 [T, K], wts fp64)."""
    logits = h.double() @ W.double().t()
    p = torch.softmax(logits, -1)
    order = torch.sort(-p, dim=-1, stable=True).indices[:, :K]
    top = torch.gather(p, 1, order)
    return order, top / top.sum(-1, keepdim=True)


def expert_ffn(x: torch.Tensor, gu: torch.Tensor, dn: torch.Tensor) -> torch.Tensor:
    """One SwiGLU expert (hybrid.py:624-626): gate | up = x gu^T; down(silu(gate) * up). fp64."""
    gate, up = (x.double() @ gu.t()).chunk(2, -1)
    return (F.silu(gate) * up) @ dn.t()


def moe_experts(h: torch.Tensor, rows: torch.Tensor, idx: torch.Tensor, wts: torch.Tensor, D: int, I: int):
    """ExpertBank.forward (hybrid.py:608-628): out[t] = sum_k wts[t, k] * expert_idx[t,k](h[t]).
    rows: uint8 [E, row_bytes]. Picks with an id outside [0, E) add nothing. fp64 [T, D]."""
    out = torch.zeros(h.shape[0], D, dtype=torch.float64)
    E = rows.shape[0]
    for e in sorted(set(int(v) for v in idx.reshape(-1).tolist())):
        if not 0 <= e < E:
            continue
        tok, kk = (idx == e).nonzero(as_tuple=True)
        gu, dn = unpack_expert(rows[e], D, I)
        out.index_add_(0, tok, expert_ffn(h[tok], gu, dn) * wts[tok, kk].double().unsqueeze(-1))
    return out


def swiglu(x: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, wd: torch.Tensor) -> torch.Tensor:
    """SwiGLU (model.py:188-196): down(silu(gate x) * up x), fp64 from the given weights."""
    x = x.double()
    return (F.silu(x @ wg.double().t()) * (x @ wu.double().t())) @ wd.double().t()


def moe_forward(h, router_w, rows, D: int, I: int, K: int, ysh=None, shared_gate=None):
    """MoE.forward (hybrid.py:647-652): routed experts + sigmoid(h . shared_gate) * shared(h).
    ysh: the shared expert's output [T, D] (or None). Returns (out fp64 [T, D], idx, wts)."""
    idx, wts = route(h, router_w, K)
    out = moe_experts(h, rows, idx, wts, D, I)
    if ysh is not None:
        out = out + torch.sigmoid(h.double() @ shared_gate.double()).unsqueeze(-1) * ysh.double()
    return out, idx, wts


# --- composites: the mixers and the layer stack (config 4) ---------------------------------

def _lin(x, w, round_in: bool):
    """x @ w^T with w a bf16 nn.Linear weight [out, in]; with round_in the activation is
    rounded to bf16 first, as a bf16 model feeds its projections (the HIP stack does the same)."""
    xin = x.to(torch.bfloat16).float() if round_in else x.float()
    return xin @ w.float().t()


def gated_deltanet_mixer(h, W: dict, conv_state, state, length: int, hk: int, hv: int, eps: float = 1e-6,
                         round_in: bool = True):
    """GatedDeltaNet.forward (hybrid.py:388-421). h [B,T,d]; conv_state [B,C,3] (returned
    updated as a new tensor); state [B,HV,128,128] updated in place. Returns (out [B,T,d],
    new conv state)."""
    B, T, _ = h.shape
    d = 128
    qkv = _lin(h, W["w_qkv"], round_in)
    z = _lin(h, W["w_z"], round_in).view(B, T, hv, d)
    b = _lin(h, W["w_b"], round_in)
    a = _lin(h, W["w_a"], round_in)
    y, new_conv = conv_silu(qkv, W["conv_w"].float(), conv_state)
    q, k, v = delta_prep(y, hk, hv, d, d)
    beta = b.sigmoid().transpose(1, 2)
    g = (-W["a_log"].float().exp() * F.softplus(a + W["dt_bias"].float())).transpose(1, 2)
    if T == 1 and length > 0:
        out = delta_rule_step(q[:, :, 0], k[:, :, 0], v[:, :, 0], g[:, :, 0], beta[:, :, 0], state).unsqueeze(2)
    else:
        out, S = delta_rule_chunked(q, k, v, g, beta, state if length > 0 else None)
        state.copy_(S)
    out = out.transpose(1, 2)
    o = gated_norm(out, z, W["gnorm_w"].float(), eps)
    return _lin(o.reshape(B, T, hv * d), W["w_out"], round_in), new_conv


def gated_attention_mixer(h, W: dict, kc, vc, pos: int, H: int, KV: int, HD: int = 256, rotary_dim: int = 64,
                          theta: float = 1e7, eps: float = 1e-6, round_in: bool = True):
    """GatedAttention.forward (hybrid.py:280-311) with the cache rows written at pos..pos+T-1."""
    B, T, _ = h.shape
    qg = _lin(h, W["w_q"], round_in).view(B, T, H, 2 * HD)
    k = _lin(h, W["w_k"], round_in).view(B, T, KV, HD)
    v = _lin(h, W["w_v"], round_in).view(B, T, KV, HD)
    q, gate = attn_prep(qg, k, v, W["q_norm"].float(), W["k_norm"].float(), kc, vc, pos, rotary_dim, theta, eps)
    y = gated_attention_out(attention_core(q, kc, vc, pos, KV), gate)
    return _lin(y, W["w_o"], round_in)


def hybrid_stack_forward(x, layers: list, kinds: list, cache: dict, cfg: dict, round_in: bool = True):
    """HybridBlock.forward with the MoE FFN as identity (hybrid.py:812-843): per layer
    x = x + mixer(znorm(x)). cache: {'length', 'conv': [..], 'state': [..], 'k': [..], 'v': [..]}
    per-kind lists, updated. Returns the new x."""
    delta_i = attn_i = 0
    for W, kind in zip(layers, kinds):
        h = znorm(x, W["norm1"].float(), cfg["eps"])
        if kind == "attn":
            y = gated_attention_mixer(h, W, cache["k"][attn_i], cache["v"][attn_i], cache["length"], cfg["n_heads"],
                                      cfg["n_kv"], cfg["head_dim"], cfg["rotary_dim"], cfg["rope_theta"], cfg["eps"],
                                      round_in)
            attn_i += 1
        else:
            y, cache["conv"][delta_i] = gated_deltanet_mixer(h, W, cache["conv"][delta_i], cache["state"][delta_i],
                                                             cache["length"], cfg["hk"], cfg["hv"], cfg["eps"],
                                                             round_in)
            delta_i += 1
        x = x + y
    cache["length"] += x.shape[1]
    return x
