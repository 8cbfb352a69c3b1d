"""aegist_attention_decode_noalloc (fixed in-library scratch, no allocation) against
aegist_attention_decode with a caller workspace, through the C ABI: two calls in a row, the
second with a smaller input (fewer sequences, shorter context), each bit-identical to the
workspace form on the same inputs (both run the same kernels). Also: a shape whose scratch
exceeds the fixed size is refused before any launch."""
import pytest
import torch

from aegist_mixer import _lib, ops

pytestmark = pytest.mark.gpu


def _inputs(B, H, KV, HD, cap, L, seed, dev):
    g_ = torch.Generator().manual_seed(seed)
    qg = torch.randn(B, H, 2 * HD, generator=g_).to(torch.bfloat16).to(dev)
    kn = torch.randn(B, KV, HD, generator=g_).to(torch.bfloat16).to(dev)
    vn = torch.randn(B, KV, HD, generator=g_).to(torch.bfloat16).to(dev)
    qw = (0.1 * torch.randn(HD, generator=g_)).to(torch.bfloat16).to(dev)
    kw = (0.1 * torch.randn(HD, generator=g_)).to(torch.bfloat16).to(dev)
    kc = torch.randn(B, KV, cap, HD, generator=g_).to(torch.bfloat16).to(dev)
    vc = torch.randn(B, KV, cap, HD, generator=g_).to(torch.bfloat16).to(dev)
    return qg, kn, vn, qw, kw, kc, vc


def _call(name, qg, kn, vn, qw, kw, kc, vc, out, pos, ws=None):
    B, H, HD2 = qg.shape
    KV, cap, HD = kc.shape[1], kc.shape[2], kc.shape[3]
    st = torch.cuda.current_stream().cuda_stream
    args = [qg.data_ptr(), kn.data_ptr(), vn.data_ptr(), _lib.BF16, qw.data_ptr(), kw.data_ptr(), kc.data_ptr(),
            vc.data_ptr(), out.data_ptr(), _lib.F32, B, H, KV, HD, 64, pos, cap, 1e-6, 1e7]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    _lib.call(name, *args, st)


@pytest.mark.parametrize("shapes", [((8, 4096, 4000), (2, 1024, 700)), ((32, 32768, 30000), (1, 4096, 100))])
def test_noalloc_matches_workspace_form(dev, shapes):
    H, KV, HD = 16, 2, 256
    for i, (B, cap, pos) in enumerate(shapes):
        print(f"noalloc call {i}: B={B} cap={cap} pos={pos}", flush=True)
        a = _inputs(B, H, KV, HD, cap, pos, 10 + i, dev)
        b = tuple(t.clone() for t in a)
        out_n = torch.empty(B, H, HD, device=dev)
        out_w = torch.empty_like(out_n)
        _call("aegist_attention_decode_noalloc", *a, out_n, pos)
        need = _lib.lib().aegist_attention_decode_workspace_bytes(B, H, KV, pos + 1)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        _call("aegist_attention_decode", *b, out_w, pos, ws)
        torch.cuda.synchronize()
        assert torch.equal(out_n, out_w), (i, (out_n - out_w).abs().max().item())
        assert torch.equal(a[5], b[5]) and torch.equal(a[6], b[6])  # the appended cache rows too
        assert torch.isfinite(out_n).all()


def test_noalloc_refuses_oversized_scratch(dev):
    L = _lib.lib()
    B, H, KV, pos = 2048, 16, 2, 1000
    assert L.aegist_attention_decode_workspace_bytes(B, H, KV, pos + 1) > 32 << 20
    rc = L.aegist_attention_decode_noalloc(None, None, None, _lib.BF16, None, None, None, None, None, _lib.F32, B, H,
                                           KV, 256, 64, pos, pos + 1, 1e-6, 1e7, None)
    assert rc == -2 and "32" in _lib.last_error()
