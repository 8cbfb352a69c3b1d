"""GPU parity of the projection kernels (QLinear int8 / bf16 weights) against the CPU oracle's
engine formula (aegist.cu gemv_i8 / gemm_i8 / gemv_bf16). The kernel splits an fp32 activation
into bf16 hi + lo, so the bar is fp32-level: 2e-5 norm-wise max relative error (1e-5 for
bf16 activations, whose products are exact)."""
import pytest
import torch

from conftest import rel_err
from oracle import mixer_ref as R

from aegist_mixer import ops
from aegist_mixer._lib import AegistError

pytestmark = pytest.mark.gpu

TOL_F32X = 2e-5
TOL_BF16X = 1e-5


def _case(M, N, K, seed, xdtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    q, s = R.qlinear_quantize(w)
    x = torch.randn(M, K, generator=g).to(xdtype)
    return x, q, s, w


@pytest.mark.parametrize("M,N,K", [(1, 32, 16), (1, 2048, 4096), (1, 8192, 2048), (5, 100, 48), (16, 4096, 2048),
                                   (17, 300, 2048), (33, 2048, 4096), (64, 8192, 2048), (100, 520, 1024),
                                   (300, 64, 256)])
def test_linear_int8_fp32x(dev, M, N, K):
    print(f"linear int8 fp32x M={M} N={N} K={K}", flush=True)
    x, q, s, _ = _case(M, N, K, seed=M + N + K)
    ref = R.qlinear_engine(x, q, s)
    out = ops.linear(x.to(dev), q.to(dev), s.to(dev))
    torch.cuda.synchronize()
    assert rel_err(out, ref) < TOL_F32X


@pytest.mark.parametrize("M,N,K", [(1, 4096, 2048), (16, 8192, 2048), (48, 2048, 4096), (64, 32, 2048),
                                   (130, 256, 512)])
def test_linear_bf16_weight_bf16x(dev, M, N, K):
    print(f"linear bf16 bf16x M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    ref = R.qlinear_engine(x.float(), w.float(), None)
    out = ops.linear(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert rel_err(out, ref) < TOL_BF16X


@pytest.mark.parametrize("M,N,K,xdt,acc", [(16, 12352, 2048, torch.bfloat16, False),
                                            (1, 9216, 2048, torch.bfloat16, True),
                                            (7, 8224, 512, torch.bfloat16, False),
                                            (16, 8320, 768, torch.float32, True),
                                            (3, 8200, 256, torch.float32, False)])
def test_linear_bf16_weight_streamed(dev, M, N, K, xdt, acc):
    """bf16 weights at M <= 16 over more than 8192 rows (K a multiple of 256) take the
    LDS-staged stream kernel: ragged last row tiles (N not a multiple of 32), bf16 and fp32
    activations, the residual accumulate."""
    print(f"linear streamed M={M} N={N} K={K} x={xdt} acc={acc}", flush=True)
    g = torch.Generator().manual_seed(M * 11 + N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, K, generator=g).to(xdt)
    y0 = torch.randn(M, N, generator=g)
    ref = R.qlinear_engine(x.float(), w.float(), None, y0.clone() if acc else None, accumulate=acc)
    out = y0.to(dev) if acc else None
    out = ops.linear(x.to(dev), w.to(dev), out=out, accumulate=acc)
    torch.cuda.synchronize()
    assert rel_err(out, ref) < (TOL_BF16X if xdt == torch.bfloat16 else TOL_F32X)


def test_linear_accumulate_and_strides(dev):
    """Residual add into a strided Y (ldy > N) from a strided X (ldx > K), bf16 weights, fp32 X."""
    M, N, K = 9, 96, 640
    g = torch.Generator().manual_seed(5)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    xbig = torch.randn(M, K + 64, generator=g)
    ybig = torch.randn(M, N + 32, generator=g)
    ref = ybig.clone()
    ref[:, :N] = R.qlinear_engine(xbig[:, :K], w.float(), None, ybig[:, :N], accumulate=True)
    xd, yd = xbig.to(dev), ybig.to(dev)
    from aegist_mixer._lib import BF16, F32, call
    wd = w.to(dev)  # held: a temporary's memory could be reused before the kernel reads it
    call("aegist_linear", xd.data_ptr(), F32, K + 64, wd.data_ptr(), BF16, None, yd.data_ptr(), N + 32, M, N, K,
         1, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rel_err(yd, ref) < TOL_F32X
    assert torch.equal(yd[:, N:].cpu(), ybig[:, N:])  # the columns past N are untouched


def test_engine_entry_points(dev):
    """gemv_i8 (with and without accumulate), gemm_i8 and gemv_bf16 with the engine argument lists."""
    x, q, s, w = _case(1, 2048, 4096, seed=11)
    y0 = torch.randn(2048)
    yd = y0.to(dev)
    ops.gemv_i8(x[0].to(dev), q.to(dev), s.to(dev), yd, accumulate=True)
    out1 = ops.gemv_i8(x[0].to(dev), q.to(dev), s.to(dev))
    X, q2, s2, _ = _case(40, 1024, 2048, seed=12)
    out2 = ops.gemm_i8(X.to(dev), q2.to(dev), s2.to(dev))
    wb = w.to(torch.bfloat16)
    out3 = ops.gemv_bf16(x[0].to(dev), wb.to(dev))
    torch.cuda.synchronize()
    assert rel_err(yd, R.qlinear_engine(x, q, s, y0.unsqueeze(0), accumulate=True)[0]) < TOL_F32X
    assert rel_err(out1, R.qlinear_engine(x, q, s)[0]) < TOL_F32X
    assert rel_err(out2, R.qlinear_engine(X, q2, s2)) < TOL_F32X
    assert rel_err(out3, R.qlinear_engine(x, wb.float(), None)[0]) < TOL_F32X


def test_linear_shape_errors(dev):
    x = torch.randn(2, 24, device=dev)
    w = torch.zeros(8, 24, dtype=torch.int8, device=dev)
    with pytest.raises(AegistError):
        ops.linear(x, w)  # K % 16 != 0


@pytest.mark.parametrize("M", [1, 16, 40])
def test_linear_multi_matches_separate(dev, M):
    """One grouped launch over a layer's input projections (sizes of in_qkv, in_z, in_b, in_a
    scaled down, plus an empty one) equals the oracle per weight."""
    print(f"linear_multi M={M}", flush=True)
    g = torch.Generator().manual_seed(M)
    K = 512
    Ns = [1024, 512, 32, 0]
    ws = [torch.randn(n, K, generator=g) * 0.02 for n in Ns]
    qs = [R.qlinear_quantize(w) for w in ws]
    x = torch.randn(M, K, generator=g)
    outs = ops.linear_multi(x.to(dev), [q.to(dev) for q, _ in qs], [s.to(dev) for _, s in qs])
    wb = [w.to(torch.bfloat16) for w in ws[:3]]
    xb = x.to(torch.bfloat16)
    outs_b = ops.linear_multi(xb.to(dev), [w.to(dev) for w in wb])
    torch.cuda.synchronize()
    for (q, s), o in zip(qs[:3], outs[:3]):
        assert rel_err(o, R.qlinear_engine(x, q, s)) < TOL_F32X
    assert outs[3].numel() == 0
    for w, o in zip(wb, outs_b):
        assert rel_err(o, R.qlinear_engine(xb.float(), w.float(), None)) < TOL_BF16X


@pytest.mark.parametrize("Ns", [[264, 40, 302], [100, 64], [8, 8, 1000]])
def test_linear_multi_stacked_gemm(dev, Ns):
    """Past 64 rows, bf16 weights sharing X run as one tiled-GEMM launch stacked along N when every
    weight but the last has a multiple of 8 rows (segment boundaries inside a 256-column tile, a
    ragged last segment, three segments in one tile), else one launch per weight: each output
    equal to the oracle per weight."""
    print(f"linear_multi stacked GEMM Ns={Ns}", flush=True)
    g = torch.Generator().manual_seed(sum(Ns))
    K, M = 512, 300
    wb = [(torch.randn(n, K, generator=g) * 0.02).to(torch.bfloat16) for n in Ns]
    xb = torch.randn(M, K, generator=g).to(torch.bfloat16)
    outs = ops.linear_multi(xb.to(dev), [w.to(dev) for w in wb])
    torch.cuda.synchronize()
    for w, o in zip(wb, outs):
        assert rel_err(o, R.qlinear_engine(xb.float(), w.float(), None)) < TOL_BF16X


def test_linear_multi_streamed_layer_group(dev):
    """A DeltaNet layer's input group at config-4 width (in_qkv 8192, in_z 4096, in_b 32,
    in_a 32 rows over K 2048, bf16 weights and activations, M = 16): one stream-kernel launch,
    each output equal to the oracle per weight."""
    print("linear_multi streamed group", flush=True)
    g = torch.Generator().manual_seed(99)
    K, M = 2048, 16
    Ns = [8192, 4096, 32, 32]
    wb = [(torch.randn(n, K, generator=g) * 0.02).to(torch.bfloat16) for n in Ns]
    xb = torch.randn(M, K, generator=g).to(torch.bfloat16)
    outs = ops.linear_multi(xb.to(dev), [w.to(dev) for w in wb])
    torch.cuda.synchronize()
    for w, o in zip(wb, outs):
        assert rel_err(o, R.qlinear_engine(xb.float(), w.float(), None)) < TOL_BF16X


@pytest.mark.parametrize("M,N,K,acc", [(64, 2048, 4096, False), (64, 2048, 4096, True), (33, 1000, 2048, True),
                                       (17, 2048, 512, False), (40, 4096, 768, False)])
def test_linear_bf16_splitk_bound_workspace(dev, M, N, K, acc):
    """17..64 rows of bf16 X against one bf16 weight of few rows split K over the calling thread's
    bound workspace (fp32 partials added in slice order by a second launch): same bar against the
    oracle, deterministic from call to call, and the same as the unbound path to fp32 rounding."""
    from aegist_mixer._lib import call
    print(f"linear bf16 split-K M={M} N={N} K={K} acc={acc}", flush=True)
    g = torch.Generator().manual_seed(M * 13 + N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    y0 = torch.randn(M, N, generator=g)
    ref = R.qlinear_engine(x.float(), w.float(), None) + (y0 if acc else 0)
    xd, wd = x.to(dev), w.to(dev)
    plain = y0.to(dev)
    ops.linear(xd, wd, out=plain, accumulate=acc)
    ws = torch.empty(16 << 20, device=dev, dtype=torch.uint8)
    call("aegist_bind_workspace", ws.data_ptr(), ws.numel())
    try:
        outs = []
        for _ in range(2):
            out = y0.to(dev)
            ops.linear(xd, wd, out=out, accumulate=acc)
            outs.append(out)
        torch.cuda.synchronize()
    finally:
        call("aegist_bind_workspace", None, 0)
    assert torch.equal(outs[0], outs[1])
    assert rel_err(outs[0], ref) < TOL_BF16X
    assert rel_err(outs[0], plain) < 1e-6
