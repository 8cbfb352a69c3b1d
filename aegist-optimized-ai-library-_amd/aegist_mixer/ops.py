"""Host API over libaegist_mixer for torch device tensors.

Names and argument meanings follow the reference's torch model
(/root/reference/aegist-fast-35b/aegist/hybrid.py): ``delta_rule_step`` (:318-324),
``delta_rule_chunked`` (:327-361), the GatedDeltaNet decode path (:388-421) and
GatedAttention (:265-311); the ``engine_*`` functions wrap the engine-ABI mirrors of
aegist_rs/kernels/hybrid.cu one to one. Every function launches HIP kernels on the current
torch stream and returns without synchronising. torch is only the allocator and stream
provider here: no op computes anything in torch.
"""
from __future__ import annotations

import torch

from ._lib import BF16, F32, I8, AegistError, call, lib

_DT = {torch.float32: F32, torch.bfloat16: BF16}


def _dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise AegistError("dtype", -3, f"tensor dtype {t.dtype} not supported (fp32 or bf16)") from None


def _p(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise AegistError("device", -1, "tensor is not on a GPU device")
    return t.data_ptr()


def _need_contig(*ts):
    for t in ts:
        if t is not None and not t.is_contiguous():
            raise AegistError("layout", -1, "tensor must be contiguous")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


_ws_cache: dict[tuple, torch.Tensor] = {}


def _workspace(nbytes: int, device) -> torch.Tensor:
    """Workspace tensor of at least nbytes (kept per device and stream, grown on demand). The
    library never allocates: this caller-side buffer is what the *_ws entry points receive.
    One buffer per (device, current stream), so calls on different streams never share scratch
    bytes, and reuse on one stream is ordered by that stream; a replaced buffer is released
    through torch's stream-ordered caching allocator."""
    key = (str(device), torch.cuda.current_stream(device).cuda_stream)
    ws = _ws_cache.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _ws_cache[key] = ws
    return ws


# --- synthetic inputs ------------------------------------------------------------------------

def fill_normal(t: torch.Tensor, seed: int, mean: float = 0.0, std: float = 1.0) -> torch.Tensor:
    """Fill t (fp32 or bf16, contiguous) from the counter-based N(mean, std) generator."""
    _need_contig(t)
    call("aegist_fill_normal", _p(t), t.numel(), _dt(t), seed & ((1 << 64) - 1), mean, std, _stream())
    return t


def rope_inv_freq(rotary_dim: int, theta: float) -> torch.Tensor:
    """The library's RoPE table (CPU fp32), 1 / theta^(2j/rd) rounded once from double."""
    out = torch.empty(rotary_dim // 2, dtype=torch.float32)
    call("aegist_rope_inv_freq", out.data_ptr(), rotary_dim, theta)
    return out


# --- gated DeltaNet -----------------------------------------------------------------------------

def delta_decode_step(qkv, conv_w, conv_state, g, beta, state, hk: int, hv: int,
                      out_dtype=torch.float32, eps: float = 1e-6):
    """One decode token per sequence (hybrid.py:390-413 at T == 1 with history): conv-state
    update + conv + SiLU + split + L2-norm + q/sqrt(128) + gated delta step, fused.

    qkv [B, C] (fp32/bf16, pre-conv); conv_w [C, 4] bf16; conv_state [B, C, 3] fp32 and
    state [B, HV, 128, 128] fp32 are updated in place; g, beta [B, HV] fp32.
    Returns o [B, HV, 128] in out_dtype."""
    B = qkv.shape[0]
    _need_contig(qkv, conv_w, conv_state, g, beta, state)
    out = torch.empty(B, hv, 128, dtype=out_dtype, device=qkv.device)
    call("aegist_delta_decode_step", _p(qkv), _dt(qkv), _p(conv_w), _p(conv_state), _p(g), _p(beta), _p(state),
         _p(out), _dt(out), B, hk, hv, 128 ** -0.5, eps, _stream())
    return out


def _seq_strides(t: torch.Tensor):
    """(batch, token, head) element strides of a heads-first [B, H, T, d] tensor."""
    if t.stride(-1) != 1:
        raise AegistError("layout", -1, "the head dim must be contiguous")
    return t.stride(0), t.stride(2), t.stride(1)


def delta_rule_recurrent(q, k, v, g, beta, state=None, normalize: bool = False, qscale: float = 1.0,
                         eps: float = 1e-6, out_dtype=torch.float32):
    """The gated delta rule token by token (hybrid.py:318-324 looped).

    q, k [B, HK, T, d]; v [B, HV, T, d] (heads-first, fp32 or bf16, any strides with the
    head dim contiguous); g, beta [B, HV, T] fp32; state [B, HV, d, d] fp32 updated in place,
    or None for a zero initial state. With normalize the kernel applies hybrid.py:408-410
    (L2-norm of q and k, q * qscale). Returns o [B, HV, T, d]."""
    B, HK, T, d = q.shape
    HV = v.shape[1]
    if d != 128 or v.shape[-1] != 128:
        raise AegistError("delta_rule_recurrent", -1, "dk = dv = 128 required")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise AegistError("delta_rule_recurrent", -3, "q, k, v must share a dtype")
    if k.stride() != q.stride():
        raise AegistError("delta_rule_recurrent", -1, "q and k must have the same strides")
    gt = g.transpose(1, 2).contiguous()   # [B, T, HV]
    bt = beta.transpose(1, 2).contiguous()
    out = torch.empty(B, HV, T, d, dtype=out_dtype, device=q.device)
    sq, sv, so = _seq_strides(q), _seq_strides(v), _seq_strides(out)
    if state is not None:
        _need_contig(state)
    call("aegist_delta_recurrent", _p(q), _p(k), _p(v), _dt(q), *sq, *sv, _p(gt), _p(bt), _p(state), _p(out),
         _dt(out), *so, B, T, HK, HV, int(normalize), qscale, eps, _stream())
    return out


def delta_rule_step(q, k, v, g, beta, state):
    """One token (hybrid.py:318-324). q, k [B, H, dk]; v [B, H, dv]; g, beta [B, H];
    state [B, H, dk, dv] fp32 updated in place. Returns o [B, H, dv] fp32."""
    o = delta_rule_recurrent(q.unsqueeze(2), k.unsqueeze(2), v.unsqueeze(2), g.unsqueeze(2), beta.unsqueeze(2),
                             state)
    return o[:, :, 0]


def delta_rule_chunked(q, k, v, g, beta, state=None, chunk: int = 64, normalize: bool = False,
                       qscale: float = 1.0, eps: float = 1e-6, out_dtype=torch.float32):
    """Chunked WY form (hybrid.py:327-361), on MFMA. Same tensors as delta_rule_recurrent;
    returns (o [B, HV, T, d], final state [B, HV, d, d] fp32). A given state is updated in
    place and also returned."""
    if chunk != 64:
        raise AegistError("delta_rule_chunked", -1, "chunk size 64 only")
    B, HK, T, d = q.shape
    HV = v.shape[1]
    if d != 128 or v.shape[-1] != 128:
        raise AegistError("delta_rule_chunked", -1, "dk = dv = 128 required")
    if k.stride() != q.stride() or k.dtype != q.dtype or v.dtype != q.dtype:
        raise AegistError("delta_rule_chunked", -1, "q and k must share strides; q, k, v a dtype")
    gt = g.transpose(1, 2).contiguous()
    bt = beta.transpose(1, 2).contiguous()
    out = torch.empty(B, HV, T, d, dtype=out_dtype, device=q.device)
    S = torch.zeros(B, HV, d, d, dtype=torch.float32, device=q.device) if state is None else state
    _need_contig(S)
    nbytes = lib().aegist_delta_chunked_workspace_bytes(B, T, HV)
    ws = _workspace(nbytes, q.device)
    sq, sv, so = _seq_strides(q), _seq_strides(v), _seq_strides(out)
    call("aegist_delta_chunked", _p(q), _p(k), _p(v), _dt(q), *sq, *sv, _p(gt), _p(bt), _p(S), _p(out), _dt(out),
         *so, B, T, HK, HV, int(normalize), qscale, eps, _p(ws), ws.numel(), _stream())
    return out, S


# --- gated attention --------------------------------------------------------------------------

def attention_decode(qg, k_new, v_new, q_norm_w, k_norm_w, kc, vc, pos: int, rotary_dim: int = 64,
                     theta: float = 1e7, eps: float = 1e-6, out_dtype=torch.float32):
    """One query token per sequence at position ``pos`` (hybrid.py:280-310 at T == 1):
    ZNorm + partial RoPE of q and the new k, cache append, split-K attention over rows
    [0, pos], sigmoid gate. qg [B, H, 2*HD]; k_new, v_new [B, KV, HD]; caches
    [B, KV, cap, HD] bf16. Returns [B, H, HD] in out_dtype."""
    B, H, HD2 = qg.shape
    KV, HD, cap = kc.shape[1], kc.shape[3], kc.shape[2]
    _need_contig(qg, k_new, v_new, kc, vc, q_norm_w, k_norm_w)
    if k_new.dtype != qg.dtype or v_new.dtype != qg.dtype:
        raise AegistError("attention_decode", -3, "qg, k_new, v_new must share a dtype")
    out = torch.empty(B, H, HD, dtype=out_dtype, device=qg.device)
    nbytes = lib().aegist_attention_decode_workspace_bytes(B, H, KV, pos + 1)
    ws = _workspace(nbytes, qg.device)
    call("aegist_attention_decode", _p(qg), _p(k_new), _p(v_new), _dt(qg), _p(q_norm_w), _p(k_norm_w), _p(kc),
         _p(vc), _p(out), _dt(out), B, H, KV, HD, rotary_dim, pos, cap, eps, theta, _p(ws), ws.numel(), _stream())
    return out


def attention_core(q, kc, vc, gate, pos: int, scale: float | None = None, f16_copy: bool = True):
    """Causal GQA attention core (hybrid.py:297-310). q [B, H, T, HD] fp32 (normed and roped);
    caches [B, KV, cap, HD] bf16 holding rows [0, pos + T); gate [B, T, H*HD] fp32 or None.
    Returns [B, T, H, HD] fp32 (gated when gate is given). For T > 1, f16_copy=False withholds
    the workspace of the fp16 cache copy (the kernel then converts its tiles as it stages them)."""
    B, H, T, HD = q.shape
    KV, cap = kc.shape[1], kc.shape[2]
    _need_contig(q, kc, vc, gate)
    out = torch.empty(B, T, H, HD, dtype=torch.float32, device=q.device)
    nbytes = lib().aegist_attention_decode_workspace_bytes(B, H, KV, pos + 1)
    if T > 1 and f16_copy:
        nbytes = max(nbytes, lib().aegist_attention_core_workspace_bytes(B, H, KV, T, pos))
    ws = _workspace(nbytes, q.device)
    sc = HD ** -0.5 if scale is None else scale
    call("aegist_attention_core", _p(q), _p(kc), _p(vc), _p(gate), _p(out), B, H, KV, T, pos, cap, sc, _p(ws),
         ws.numel(), _stream())
    return out


# --- engine-ABI mirrors (batch 1, fp32 activations; aegist_rs/kernels/hybrid.cu) ---------------

def engine_znorm(x, w, eps=1e-6):
    rows, D = x.shape
    out = torch.empty_like(x)
    call("aegist_znorm", _p(x), _p(w), _p(out), rows, D, eps, _stream())
    return out


def engine_attn_prep(qg, k, v, qw, kw, kc, vc, pos0, rotary_dim=64, theta=1e7, eps=1e-6):
    """qg [T, H, 2HD]; k, v [T, KV, HD]; kc, vc [KV, cap, HD] bf16. Returns qn [T, H, HD]."""
    T, H, HD2 = qg.shape
    KV, cap, HD = kc.shape
    qn = torch.empty(T, H, HD, dtype=torch.float32, device=qg.device)
    call("aegist_attn_prep", _p(qg), _p(k), _p(v), _p(qw), _p(kw), _p(qn), _p(kc), _p(vc), T, H, KV, HD, rotary_dim,
         pos0, cap, eps, theta, _stream())
    return qn


def engine_attention_gated(qn, kc, vc, qg, pos0):
    T, H, HD = qn.shape
    KV, cap, _ = kc.shape
    out = torch.empty(T, H, HD, dtype=torch.float32, device=qn.device)
    need = lib().aegist_attention_gated_workspace_bytes(T, H, KV, pos0)
    ws = _workspace(need, qn.device)
    call("aegist_attention_gated_ws", _p(qn), _p(kc), _p(vc), _p(qg), _p(out), T, H, KV, pos0, cap, HD ** -0.5,
         _p(ws), ws.numel(),
         _stream())
    return out


def engine_delta_gates(h, wb, wa, a_log, dt_bias):
    T, D = h.shape
    HV = wb.shape[0]
    gb = torch.empty(T, 2 * HV, dtype=torch.float32, device=h.device)
    call("aegist_delta_gates", _p(h), _p(wb), _p(wa), _p(a_log), _p(dt_bias), _p(gb), T, D, HV, _stream())
    return gb


def engine_conv_silu(x, w, state):
    T, Cc = x.shape
    y = torch.empty_like(x)
    call("aegist_conv_silu", _p(x), _p(y), _p(w), _p(state), T, Cc, _stream())
    return y


def engine_l2norm_heads(y, nq, dk=128, qscale=128 ** -0.5, eps=1e-6):
    T, Cc = y.shape
    call("aegist_l2norm_heads", _p(y), T, Cc, nq, dk, qscale, eps, _stream())
    return y


def engine_delta_scan(y, gb, state, hk, hv):
    T, Cc = y.shape
    o = torch.empty(T, hv, 128, dtype=torch.float32, device=y.device)
    ws = _workspace(lib().aegist_delta_scan_workspace_bytes(T, hk, hv), y.device)
    call("aegist_delta_scan_ws", _p(y), _p(gb), _p(state), _p(o), T, Cc, hk, hv, _p(ws), ws.numel(), _stream())
    return o


def engine_gated_norm(o, z, w, eps=1e-6):
    T, HV, DV = o.shape
    out = torch.empty_like(o)
    call("aegist_gated_norm", _p(o), _p(z), _p(w), _p(out), T, HV, DV, eps, _stream())
    return out


# --- the hybrid mixer stack (config 4) ----------------------------------------------------------

# --- second core: QSA indexer and gated norm with a choice of gate (engine ABI, batch 1) -----

def engine_idx_prep(qk, qw, qi, kraw, pos0: int, rotary_dim: int = 64, theta: float = 1e7, eps: float = 1e-6):
    """qk [T, H+1, 128] -> qi [T, H, 128] (normed, roped) and kraw[pos0:pos0+T] (raw keys)."""
    _need_contig(qk, qw, qi, kraw)
    T, H1, HD = qk.shape
    call("aegist_idx_prep", _p(qk), _p(qw), _p(qi), _p(kraw), T, H1 - 1, HD, rotary_dim, pos0, eps, theta, _stream())
    return qi


def engine_idx_blocks(kraw, kw, bk, b0: int, n: int, R: int, rotary_dim: int = 64, theta: float = 1e7,
                      eps: float = 1e-6):
    _need_contig(kraw, kw, bk)
    call("aegist_idx_blocks", _p(kraw), _p(kw), _p(bk), b0, n, R, kraw.shape[-1], rotary_dim, eps, theta, _stream())
    return bk


def engine_idx_scores(qi, bk, sc, pos0: int, R: int):
    _need_contig(qi, bk, sc)
    T, H, HD = qi.shape
    call("aegist_idx_scores", _p(qi), _p(bk), _p(sc), T, H, HD, pos0, R, sc.shape[1], _stream())
    return sc


def engine_idx_select(sc, blist, nsel, top: int, R: int, pos0: int):
    _need_contig(sc, blist, nsel)
    ws = _workspace(lib().aegist_idx_select_workspace_bytes(sc.shape[0], top, R, pos0), sc.device)
    call("aegist_idx_select_ws", _p(sc), _p(blist), _p(nsel), sc.shape[0], top, R, pos0, sc.shape[1], _p(ws),
         ws.numel(), _stream())
    return blist, nsel


def engine_attention_gated_list(q, kc, vc, qg, pos0: int, blist, nsel, top: int, R: int, scale: float | None = None):
    """q [T, H, 256] normed + roped; kc, vc [KV, cap, 256] bf16; qg [T, H, 512]; -> out [T, H, 256]."""
    _need_contig(q, kc, vc, qg, blist, nsel)
    T, H, HD = q.shape
    KV, cap = kc.shape[0], kc.shape[1]
    out = torch.empty(T, H, HD, dtype=torch.float32, device=q.device)
    ws = _workspace(lib().aegist_attention_gated_list_workspace_bytes(T, H, KV, pos0, top, R), q.device)
    call("aegist_attention_gated_list_ws", _p(q), _p(kc), _p(vc), _p(qg), _p(out), T, H, KV, pos0, cap,
         HD ** -0.5 if scale is None else scale, _p(blist), _p(nsel), top, R, _p(ws), ws.numel(), _stream())
    return out


def engine_gated_norm2(o, z, w, sig: bool, eps: float = 1e-6):
    _need_contig(o, z, w)
    T, HV, DV = o.shape
    out = torch.empty_like(o)
    call("aegist_gated_norm2", _p(o), _p(z), _p(w), _p(out), T, HV, DV, eps, int(sig), _stream())
    return out


# --- projections (QLinear, aegist/model.py:78-93; engine gemv_i8 / gemm_i8 / gemv_bf16) -------

def linear(x, weight, scale=None, out=None, accumulate: bool = False):
    """out[..., n] (+)= scale[n] * sum_k x[..., k] weight[n, k] in fp32.

    x: [..., K] fp32 or bf16 (rows contiguous); weight: [N, K] int8 (QLinear.qweight) or bf16;
    scale: [N] bf16 (QLinear.scale) or None; out: fp32 [..., N] (allocated if None; with
    accumulate=True the product is added into it, the engine's fused residual add)."""
    K = x.shape[-1]
    N = weight.shape[0]
    if weight.dim() != 2 or weight.shape[1] != K:
        raise AegistError("shape", -1, f"weight {tuple(weight.shape)} does not match x [..., {K}]")
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1:
        raise AegistError("layout", -1, "x rows must be contiguous")
    _need_contig(weight, scale)
    M = x2.shape[0]
    if out is None:
        if accumulate:
            raise AegistError("shape", -1, "accumulate needs out")
        out = torch.empty(*x.shape[:-1], N, dtype=torch.float32, device=x.device)
    _need_contig(out)
    if out.dtype != torch.float32 or out.numel() != M * N:
        raise AegistError("shape", -1, "out must be fp32 [..., N]")
    if weight.dtype == torch.int8:
        wdt = I8
    elif weight.dtype == torch.bfloat16:
        wdt = BF16
    else:
        raise AegistError("dtype", -3, "weight must be int8 or bf16")
    if scale is not None and (scale.dtype != torch.bfloat16 or scale.numel() != N):
        raise AegistError("shape", -1, "scale must be bf16 [N]")
    call("aegist_linear", _p(x2), _dt(x2), x2.stride(0), _p(weight), wdt, _p(scale), _p(out), N, M, N, K,
         int(accumulate), _stream())
    return out


def linear_multi(x, weights, scales=None, outs=None):
    """One launch for up to four weight matrices sharing the input x [M, K]: returns
    [x @ (w_i * s_i)^T] as fp32 [M, N_i] (a layer's input projections, e.g. in_qkv | in_z |
    in_b | in_a). All weights share one dtype (int8 or bf16); scales: list of bf16 [N_i] or None."""
    import ctypes as C
    n = len(weights)
    if not 1 <= n <= 4:
        raise AegistError("shape", -1, "1 to 4 weight matrices")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    wdt = {torch.int8: I8, torch.bfloat16: BF16}.get(weights[0].dtype)
    if wdt is None or any(w.dtype != weights[0].dtype for w in weights):
        raise AegistError("dtype", -3, "weights must all be int8 or all bf16")
    for w in weights:
        _need_contig(w)
        if w.dim() != 2 or w.shape[1] != K:
            raise AegistError("shape", -1, "weight shape does not match x")
    if outs is None:
        outs = [torch.empty(M, w.shape[0], dtype=torch.float32, device=x.device) for w in weights]
    Wa = (C.c_void_p * n)(*[w.data_ptr() for w in weights])
    Sa = None if scales is None else (C.c_void_p * n)(*[None if sc is None else sc.data_ptr() for sc in scales])
    Ya = (C.c_void_p * n)(*[o.data_ptr() for o in outs])
    La = (C.c_longlong * n)(*[o.stride(0) for o in outs])
    Na = (C.c_int * n)(*[w.shape[0] for w in weights])
    call("aegist_linear_multi", _p(x2), _dt(x2), x2.stride(0), wdt, n, C.cast(Wa, C.c_void_p),
         None if Sa is None else C.cast(Sa, C.c_void_p), C.cast(Ya, C.c_void_p), C.cast(La, C.c_void_p),
         C.cast(Na, C.c_void_p), M, K, 0, _stream())
    return outs


def gemv_i8(x, qweight, scale, y=None, accumulate: bool = False):
    """Engine gemv_i8 (aegist.cu:85-91): y[n] (+)= scale[n] * (qweight[n] . x), x fp32 [K]."""
    _need_contig(x, qweight, scale)
    N, K = qweight.shape
    if y is None:
        y = torch.empty(N, dtype=torch.float32, device=x.device)
    call("aegist_gemv_i8", _p(x), _p(qweight), _p(scale), _p(y), N, K, int(accumulate), _stream())
    return y


def gemm_i8(x, qweight, scale, y=None, accumulate: bool = False):
    """Engine gemm_i8 (aegist.cu:126-172): Y[m, n] (+)= scale[n] * (qweight[n] . X[m]), X fp32 [M, K]."""
    _need_contig(x, qweight, scale)
    M, K = x.shape
    N = qweight.shape[0]
    if y is None:
        y = torch.empty(M, N, dtype=torch.float32, device=x.device)
    call("aegist_gemm_i8", _p(x), _p(qweight), _p(scale), _p(y), M, N, K, int(accumulate), _stream())
    return y


def gemv_bf16(x, weight, y=None):
    """Engine gemv_bf16 (aegist.cu:108-124): y[n] = weight[n] . x, x fp32 [K], weight bf16 [N, K]."""
    _need_contig(x, weight)
    N, K = weight.shape
    if y is None:
        y = torch.empty(N, dtype=torch.float32, device=x.device)
    call("aegist_gemv_bf16", _p(x), _p(weight), _p(y), N, K, _stream())
    return y


# --- mixture of experts (MoE, aegist/hybrid.py:631-652; HybridEngine::moe, hybrid.rs:863-955) -----

def router_topk(h, W, K: int):
    """router_topk (hybrid.cu:317-362): h fp32 [T, D], W bf16 [E, D] -> (idx int32 [T, K], wts fp32
    [T, K]): the K most probable experts of softmax(h W^T) in descending order (ties to the lower
    expert), weights renormalised over the picks."""
    _need_contig(h, W)
    T, D = h.shape
    E = W.shape[0]
    idx = torch.empty(T, K, dtype=torch.int32, device=h.device)
    wts = torch.empty(T, K, dtype=torch.float32, device=h.device)
    ws = _workspace(lib().aegist_router_topk_workspace_bytes(T, E), h.device)
    call("aegist_router_topk_ws", _p(h), _p(W), _p(idx), _p(wts), T, D, E, K, _p(ws), ws.numel(), _stream())
    return idx, wts


def expert_pointers(experts):
    """Device array of expert-row addresses for a contiguous uint8 [E, row_bytes] expert tensor."""
    E, rb = experts.shape
    base = experts.data_ptr()
    return torch.tensor([base + e * rb for e in range(E)], dtype=torch.int64, device=experts.device)


def moe_experts(h, experts, idx, wts, x, I: int, ysh=None, wg=None, eptr=None):
    """x[t] += sum_k wts[t, k] * expert_idx[t, k](h[t]) (+ sigmoid(h[t] . wg) * ysh[t]); in place.

    h, x: fp32 [T, D]; experts: uint8 [E, row] in the expert_layout of hybrid.py:472-482 (or pass
    eptr, an int64 device array of E row addresses, with experts=None and E = eptr.numel());
    idx int32 / wts fp32 [T, K]; ysh fp32 [T, D] and wg bf16 [D] for the gated shared expert."""
    _need_contig(h, idx, wts, x, ysh, wg)
    T, D = h.shape
    K = idx.shape[1]
    if eptr is None:
        eptr = expert_pointers(experts)
    E = eptr.numel()
    need = lib().aegist_moe_workspace_bytes(T, K, D, I, E)
    ws = torch.empty(need, dtype=torch.uint8, device=h.device)
    call("aegist_moe_experts", _p(h), _p(eptr), _p(idx), _p(wts), _p(x), T, D, I, E, K, _p(ysh), _p(wg), _p(ws),
         need, _stream())
    return x


def shared_gate_add(x, y, h, wg):
    """shared_gate_add (hybrid.cu:569-577): x[t] += sigmoid(h[t] . wg) * y[t], in place."""
    _need_contig(x, y, h, wg)
    T, D = x.shape
    call("aegist_shared_gate_add", _p(x), _p(y), _p(h), _p(wg), T, D, _stream())
    return x


def silu_mul(g, u, out=None):
    """silu_mul (aegist.cu:174-178): out = silu(g) * u."""
    _need_contig(g, u)
    if out is None:
        out = torch.empty_like(g)
    call("aegist_silu_mul", _p(g), _p(u), _p(out), g.numel(), _stream())
    return out


def moe_forward(h, x, router_w, experts, I: int, K: int, shared=None, shared_gate=None):
    """The MoE block of one layer on the residual x (MoE.forward, hybrid.py:647-652; the engine's
    moe(), hybrid.rs:863-955, without its expert paging): route, the routed experts, and the
    shared SwiGLU expert gated by sigmoid(h . shared_gate). shared: ((w_gate, s_gate), (w_up,
    s_up), (w_down, s_down)) QLinear int8 weights with bf16 scales (or bf16 weights with None).
    Returns (idx, wts)."""
    idx, wts = router_topk(h, router_w, K)
    ysh = None
    if shared is not None:
        (wgt, sg), (wup, su), (wdn, sd) = shared
        g = linear(h, wgt, sg)
        u = linear(h, wup, su)
        ysh = linear(silu_mul(g, u), wdn, sd)
    moe_experts(h, experts, idx, wts, x, I, ysh=ysh, wg=shared_gate if shared is not None else None)
    return idx, wts


class HybridStack:
    """Batched mixer stack on the device (aegist_stack_* of the C ABI): per layer
    x = x + mixer(znorm(x)), DeltaNet or gated attention, MoE FFN as identity
    (hybrid.py:812-843; hybrid.rs:760-861). `layers` is a list of dicts of bf16 device tensors
    named as AegistLayerWeights; the stack keeps pointers to them (they must stay alive)."""

    _DELTA = ("norm1", "w_qkv", "w_z", "w_b", "w_a", "conv_w", "a_log", "dt_bias", "gnorm_w", "w_out")
    _ATTN = ("norm1", "w_q", "w_k", "w_v", "w_o", "q_norm", "k_norm")

    def __init__(self, cfg: dict, kinds: list, layers: list, max_batch: int, max_tokens: int, max_context: int):
        import ctypes as C
        from ._lib import LayerWeights, StackConfig
        c = StackConfig()
        c.n_layers, c.d_model, c.hk, c.hv = len(kinds), cfg["d_model"], cfg["hk"], cfg["hv"]
        c.n_heads, c.n_kv, c.head_dim, c.rotary_dim = cfg["n_heads"], cfg["n_kv"], cfg["head_dim"], cfg["rotary_dim"]
        c.rope_theta, c.eps = cfg["rope_theta"], cfg["eps"]
        c.max_batch, c.max_tokens, c.max_context = max_batch, max_tokens, max_context
        for i, k in enumerate(kinds):
            c.layer_is_attn[i] = 1 if k == "attn" else 0
        self._h = C.c_void_p()
        call("aegist_stack_create", C.byref(c), C.byref(self._h))
        self.layers = layers  # keep the weights alive
        for i, (W, kind) in enumerate(zip(layers, kinds)):
            lw = LayerWeights()
            for name in (self._ATTN if kind == "attn" else self._DELTA):
                t = W[name]
                if t.dtype != torch.bfloat16 or not t.is_contiguous():
                    raise AegistError("HybridStack", -3, f"layer {i} {name}: contiguous bf16 expected")
                setattr(lw, name, _p(t))
            call("aegist_stack_set_layer", self._h, i, C.byref(lw))

    def forward(self, x):
        """x [B, T, d] fp32 contiguous device tensor, updated in place and returned."""
        _need_contig(x)
        B, T, _ = x.shape
        call("aegist_stack_forward", self._h, _p(x), B, T, _stream())
        return x

    def reset(self):
        call("aegist_stack_reset", self._h, _stream())

    def snapshot(self):
        """Remember the recurrent state at the current length (Lm::snapshot)."""
        call("aegist_stack_snapshot", self._h, _stream())

    def crop(self, n: int) -> int:
        """Go back to at most n tokens (Lm::crop); returns the length kept: the latest snapshot
        at or before n, 0 if there is none (the stack is reset), the length if n >= length."""
        r = lib().aegist_stack_crop(self._h, int(n), _stream())
        if r < 0:
            raise AegistError("aegist_stack_crop", r, lib().aegist_last_error().decode(errors="replace"))
        return r

    def state_bytes(self, n: int | None = None) -> int:
        return lib().aegist_stack_state_bytes(self._h, self.length if n is None else int(n))

    def save_state(self, path, toks, key: str | None = None, b: int = 0):
        """Write sequence b's state after len(toks) == length tokens to `path` in the engine's
        saved-state format (Lm::save_state)."""
        import ctypes as C
        from . import state_file
        n = self.length
        if len(toks) != n:
            raise AegistError("save_state", -1, f"{len(toks)} token ids for a length of {n}")
        buf = C.create_string_buffer(max(1, self.state_bytes(n)))
        call("aegist_stack_save_state", self._h, b, buf, len(buf), _stream())
        state_file.write(path, key, list(toks), buf.raw[:self.state_bytes(n)])

    def load_state(self, path, key: str | None = None, b: int = 0) -> list:
        """Read a state written by save_state (same key) into sequence b; returns its token ids
        (Lm::load_state). On an error the stack is left empty and the error is raised."""
        from . import state_file
        try:
            toks, payload = state_file.read(path, key)
        except state_file.StateFileError:
            self.reset()
            raise
        call("aegist_stack_load_state", self._h, b, len(toks), payload, len(payload), _stream())
        return toks

    @property
    def length(self) -> int:
        return lib().aegist_stack_length(self._h)

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().aegist_stack_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def embed(table, ids):
    """fp32 rows of a bf16 embedding table [V, d] for int32 ids [n] (device tensors)."""
    n, D = ids.numel(), table.shape[1]
    out = torch.empty(n, D, dtype=torch.float32, device=table.device)
    call("aegist_embed_bf16", _p(table), _p(ids), _p(out), n, D, _stream())
    return out
