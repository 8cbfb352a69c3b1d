"""GPU parity of the tiled MFMA GEMMs that `aegist_linear` uses past 64 rows - bf16 weights and
activations (the prefill-sized projections of the layer stack) and int8 QLinear weights with
fp32 activations (the engine's gemm_i8) - against the oracle's engine formula (fp64 dot products
of the exact weight values). bf16 x bf16 products are exact and the kernel sums in fp32, so the
bar is the fp32-level 1e-5 norm-wise relative error; the fp32 activations of the int8 path enter
as bf16 hi + lo (within 2^-16 of fp32), bar 2e-5 as for the weight-streaming kernel. Shapes cover
M just past the decode range, ragged M / N / K tails against the 256 x 256 x 64 tiles, the
residual accumulate into a strided Y, and the stack's full prefill shape (M = 16 x 2048),
checked on a sample of rows."""
import pytest
import torch

from conftest import rel_err
from oracle import mixer_ref as R

from aegist_mixer import ops
from aegist_mixer._lib import BF16, call

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _mats(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    return x, w


@pytest.mark.parametrize("M,N,K", [(65, 256, 64), (256, 2048, 2048), (300, 1000, 128), (1024, 8192, 2048),
                                   (777, 4096, 4096), (513, 48, 320)])
def test_gemm_matches_oracle(dev, M, N, K):
    print(f"gemm M={M} N={N} K={K}", flush=True)
    x, w = _mats(M, N, K, seed=M + N + K)
    ref = R.qlinear_engine(x.float(), w.float(), None)
    out = ops.linear(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    err = rel_err(out, ref)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < TOL


def test_gemm_accumulate_strided(dev):
    """Residual add into Y with ldy > N from X with ldx > K; the columns past N stay untouched."""
    M, N, K = 400, 640, 256
    x, w = _mats(M, N, K + 64, seed=3)
    w = w[:, :K].contiguous()
    y0 = torch.randn(M, N + 32)
    ref = y0.clone()
    ref[:, :N] = R.qlinear_engine(x[:, :K].float(), w.float(), None, y0[:, :N], accumulate=True)
    # device tensors held in names: a temporary's memory could be reused by the next copy before
    # the kernel reads it
    xd, yd, wd = x.to(dev), y0.to(dev), w.to(dev)
    call("aegist_linear", xd.data_ptr(), BF16, K + 64, wd.data_ptr(), BF16, None, yd.data_ptr(), N + 32, M, N, K,
         1, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rel_err(yd, ref) < TOL
    assert torch.equal(yd[:, N:].cpu(), y0[:, N:])


@pytest.mark.parametrize("N,K,acc", [(2048, 4096, True), (8192, 2048, False)])
def test_gemm_stack_prefill_shape(dev, N, K, acc):
    """M = 16 x 2048 rows (config 4's prefill), checked on 96 rows spread over the tiles."""
    M = 16 * 2048
    print(f"gemm stack shape M={M} N={N} K={K} acc={acc}", flush=True)
    g = torch.Generator().manual_seed(N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    xd = (torch.randn(M, K, generator=g)).to(torch.bfloat16).to(dev)
    y0 = torch.randn(M, N, generator=g) if acc else None
    out = ops.linear(xd, w.to(dev), out=y0.to(dev) if acc else None, accumulate=acc)
    torch.cuda.synchronize()
    rows = torch.cat([torch.arange(0, 32), torch.randint(32, M - 32, (32,), generator=g), torch.arange(M - 32, M)])
    xs = xd[rows].float().cpu()
    ref = R.qlinear_engine(xs, w.float(), None, y0[rows] if acc else None, accumulate=acc)
    err = rel_err(out[rows.to(dev)], ref)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("M,N,K,acc", [(65, 256, 64, False), (300, 1000, 128, True), (1024, 8192, 2048, False),
                                       (777, 2048, 4096, True)])
def test_gemm_i8_matches_oracle(dev, M, N, K, acc):
    """The engine's gemm_i8 (aegist.cu:126-172): int8 W, bf16 row scales, fp32 X, fused residual."""
    print(f"gemm_i8 M={M} N={N} K={K} acc={acc}", flush=True)
    g = torch.Generator().manual_seed(M * 3 + N + K)
    q, sc = R.qlinear_quantize(torch.randn(N, K, generator=g) * 0.02)
    x = torch.randn(M, K, generator=g)
    y0 = torch.randn(M, N, generator=g)
    ref = R.qlinear_engine(x, q, sc, y0.clone() if acc else None, accumulate=acc)
    yd, xd, qd, sd = y0.to(dev), x.to(dev), q.to(dev), sc.to(dev)
    call("aegist_gemm_i8", xd.data_ptr(), qd.data_ptr(), sd.data_ptr(), yd.data_ptr(), M, N, K, int(acc),
         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    err = rel_err(yd, ref)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < 2e-5


def test_gemm_i8_hi_lo_bound(dev):
    """gemm_i8 past 64 rows splits each fp32 X value into bf16 hi + lo (|x - hi - lo| <=
    2^-16 |x|), so each output is within 2^-16 sum_k |x_k w_k s| (plus fp32 accumulation) of the
    exact dot product; checked with X around 1e3 of mixed signs, where the lo term carries bits
    that bf16 alone would drop. (The engine kernel sums in plain fp32: results are not
    bit-compatible with it, only within this bound.)"""
    M, N, K = 96, 512, 2048
    g = torch.Generator().manual_seed(5)
    q, sc = R.qlinear_quantize(torch.randn(N, K, generator=g) * 0.02)
    x = torch.randn(M, K, generator=g) * 1e3
    yd = torch.empty(M, N, device=dev)
    xd, qd, sd = x.to(dev), q.to(dev), sc.to(dev)
    call("aegist_gemm_i8", xd.data_ptr(), qd.data_ptr(), sd.data_ptr(), yd.data_ptr(), M, N, K, 0,
         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    w = q.double() * sc.double()[:, None]
    exact = x.double() @ w.t()
    mag = x.double().abs() @ w.abs().t()
    bound = (2.0 ** -16 + K * 2.0 ** -24) * mag
    diff = (yd.double().cpu() - exact).abs()
    print(f"  max diff / bound {(diff / bound).max().item():.3f}", flush=True)
    assert (diff <= bound).all()
    # a bf16-only X would miss the bound: the lo term is doing work here
    xb = x.to(torch.bfloat16).double()
    assert ((xb @ w.t() - exact).abs() > bound).any()
