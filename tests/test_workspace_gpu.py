"""The engine-ABI mirrors with their reference signatures (no workspace argument) run on the
caller's bound workspace: 100 calls leave the device's free memory unchanged (no hidden
allocation, no growth), the results equal the explicit *_ws form's, and unbinding makes the
next call fail with AEGIST_ERR_WORKSPACE instead of allocating."""
import ctypes as C

import pytest
import torch

from aegist_mixer import _lib, ops

pytestmark = pytest.mark.gpu


def _free_bytes():
    f, t = C.c_size_t(), C.c_size_t()
    _lib.call("aegist_mem_info", C.byref(f), C.byref(t))
    return f.value


def test_mirrors_allocate_nothing(dev):
    L = _lib.lib()
    g_ = torch.Generator(device="cpu").manual_seed(0)
    H, KV, HD, cap, pos = 16, 2, 256, 8192, 4095
    HK, HV, T = 16, 32, 130
    Cc = 2 * HK * 128 + HV * 128
    q = torch.randn(1, H, HD, generator=g_).to(dev)
    qg = torch.randn(1, H, 2 * HD, generator=g_).to(dev)
    kc = torch.randn(KV, cap, HD, generator=g_).to(torch.bfloat16).to(dev)
    vc = torch.randn(KV, cap, HD, generator=g_).to(torch.bfloat16).to(dev)
    out = torch.empty(1, H, HD, device=dev)
    out_ws = torch.empty_like(out)
    y = torch.randn(T, Cc, generator=g_)
    y[:, : 2 * HK * 128] = torch.nn.functional.normalize(y[:, : 2 * HK * 128].view(T, 2 * HK, 128), dim=-1).view(T, -1)
    y = y.to(dev)
    gb = torch.cat([-torch.nn.functional.softplus(torch.randn(T, HV, generator=g_)),
                    torch.sigmoid(torch.randn(T, HV, generator=g_))], 1).to(dev)
    state = torch.zeros(HV, 128, 128, device=dev)
    state_ws = torch.zeros_like(state)
    o = torch.empty(T, HV, 128, device=dev)
    o_ws = torch.empty_like(o)
    need = max(L.aegist_attention_gated_workspace_bytes(1, H, KV, pos), L.aegist_delta_scan_workspace_bytes(T, HK, HV))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    ws2 = torch.empty(need, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    # explicit-workspace results first
    _lib.call("aegist_attention_gated_ws", q.data_ptr(), kc.data_ptr(), vc.data_ptr(), qg.data_ptr(),
              out_ws.data_ptr(), 1, H, KV, pos, cap, HD ** -0.5, ws2.data_ptr(), need, st)
    _lib.call("aegist_delta_scan_ws", y.data_ptr(), gb.data_ptr(), state_ws.data_ptr(), o_ws.data_ptr(), T, Cc, HK,
              HV, ws2.data_ptr(), need, st)
    torch.cuda.synchronize()
    _lib.call("aegist_bind_workspace", ws.data_ptr(), need)
    try:
        before = _free_bytes()
        for i in range(100):
            _lib.call("aegist_attention_gated", q.data_ptr(), kc.data_ptr(), vc.data_ptr(), qg.data_ptr(),
                      out.data_ptr(), 1, H, KV, pos, cap, HD ** -0.5, st)
            state.zero_()
            _lib.call("aegist_delta_scan", y.data_ptr(), gb.data_ptr(), state.data_ptr(), o.data_ptr(), T, Cc, HK, HV,
                      st)
        torch.cuda.synchronize()
        after = _free_bytes()
        assert after == before, (before, after)
        assert torch.equal(out, out_ws)
        assert torch.equal(o, o_ws) and torch.equal(state, state_ws)
    finally:
        _lib.call("aegist_bind_workspace", None, 0)
    rc = L.aegist_attention_gated(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), qg.data_ptr(), out.data_ptr(), 1, H, KV,
                                  pos, cap, HD ** -0.5, st)
    assert rc == -2 and "aegist_bind_workspace" in _lib.last_error()


def test_python_mirrors_use_caller_workspace(dev):
    """ops.engine_* pass a torch-owned workspace to the *_ws forms: they work with nothing bound."""
    H, KV, HD, cap = 16, 2, 256, 1024
    qn = torch.randn(1, H, HD, device=dev)
    qg = torch.randn(1, H, 2 * HD, device=dev)
    kc = torch.randn(KV, cap, HD, device=dev).to(torch.bfloat16)
    vc = torch.randn(KV, cap, HD, device=dev).to(torch.bfloat16)
    out = ops.engine_attention_gated(qn, kc, vc, qg, 700)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
