"""Benchmark of the token-mixer hot path on one MI355X.

Headline (`value`): gated DeltaNet decode throughput at batch 64 over the 30 DeltaNet layers
of the Qwen3.6-35B-A3B stack: one step = 30 launches of the fused
conv + L2-norm + delta-step kernel, each on its own layer's 128 MiB fp32 state (3.84 GiB in
total, so the 256 MB MALL cannot hold the working set), inputs resident in HBM. tok/s =
64 tokens per step / step time. `roofline` prices the kernel against 8 TB/s HBM with the
algorithmic bytes of one launch; `cpu_baseline` times the CPU oracle on one layer.

Extra fields carry the other BASELINE configs measured in the same run.
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "aegist-optimized-ai-library-_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

B, HK, HV, D, LAYERS = 64, 16, 32, 128, 30
C = 2 * HK * D + HV * D


def decode_bytes_per_launch() -> int:
    """Algorithmic HBM bytes of one layer's decode step at batch B: state read + write,
    conv state read + write, bf16 qkv in, bf16 o out, fp32 g and beta, bf16 conv weights."""
    per_seq = 2 * HV * D * D * 4 + 2 * C * 3 * 4 + C * 2 + HV * D * 2 + 2 * HV * 4
    return B * per_seq + C * 4 * 2


def cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def _errs(torch, x, ref):
    """Norm-wise max relative error max|x - ref| / max|ref| and the element-wise
    max |x - ref| / (|ref| + 1e-3 max|ref|), on fp32 (pre-rounding) outputs."""
    x, ref = x.detach().double().cpu(), ref.detach().double().cpu()
    d, m = (x - ref).abs(), ref.abs().max().item()
    return {"norm": float(d.max().item() / m), "elem": float((d / (ref.abs() + 1e-3 * m)).max().item())}


def cpu_baseline_decode(torch, ops=None, dev=None):
    """The oracle's fused decode step (torch-CPU fp32) on one layer at batch 64; 2 warm-ups,
    median of 5; scaled to 30 layers. With a device it is also the checker: the first (untimed)
    call's outputs are compared with the HIP kernel's on the same inputs (config 1's layer), and
    config 2's full 8k chunked prefill is compared with the oracle's chunked form."""
    from oracle import mixer_ref as R
    torch.set_num_threads(cpu_threads())
    g_ = torch.Generator().manual_seed(0)
    qkv = torch.randn(B, C, generator=g_).to(torch.bfloat16)
    w = (torch.randn(C, 4, generator=g_) * 0.05).to(torch.bfloat16)
    cs = torch.randn(B, C, 3, generator=g_)
    g = -torch.nn.functional.softplus(torch.randn(B, HV, generator=g_))
    beta = torch.sigmoid(torch.randn(B, HV, generator=g_))
    S = torch.randn(B, HV, D, D, generator=g_) * 0.02
    parity = None
    if dev is not None:
        Sd, csd = S.to(dev), cs.to(dev)
        od = ops.delta_decode_step(qkv.to(dev), w.to(dev), csd, g.to(dev), beta.to(dev), Sd, HK, HV)
        S0 = S.clone()
        o0, cs0 = R.delta_decode_fused(qkv, w, cs, g, beta, S0, HK, HV, D)
        parity = {"config1_decode": {"o": _errs(torch, od, o0), "state": _errs(torch, Sd, S0),
                                     "conv_state_exact": bool(torch.equal(csd.cpu(), cs0))}}
    times = []
    for i in range(7):
        t0 = time.perf_counter()
        R.delta_decode_fused(qkv, w, cs, g, beta, S, HK, HV, D)
        if i >= 2:
            times.append(time.perf_counter() - t0)
    per_layer = statistics.median(times)
    out = {"value": B / (per_layer * LAYERS), "unit": "tok/s", "cores": cpu_threads(), "cpu_model": cpu_model(),
           "kind": "port",
           "sample": f"1 of {LAYERS} layers at B={B} (oracle.mixer_ref.delta_decode_fused, torch-CPU fp32), "
                     f"median of 5 after 2 warm-ups, scaled x{LAYERS}; {per_layer * 1e3:.1f} ms per layer"}
    if dev is not None:
        parity["config2_prefill"] = prefill_parity(torch, ops, dev, R)
        out["parity"] = parity
    return out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _median_time(fn, warm=2, n=5):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(n):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline_configs(torch):
    """The oracle (torch-CPU fp32, all host cores) on bounded samples of configs 0, 2, 3 and 4,
    each reported in the unit of the matching GPU leg. Samples: config 0 in full (256 steps,
    B = 1); config 2 on the first 1024 of 8192 tokens (the chunked form is linear in T);
    config 3 at one point (B = 1, L = 32768); config 4 as one DeltaNet and one attention layer at
    full shape (decode at B = 16 with 2048 cached tokens; prefill on 256 of 2048 tokens of one
    sequence) scaled to 30 + 10 layers. Every figure is the median of 5 timed runs after 2
    untimed warm-ups."""
    from oracle import mixer_ref as R
    torch.set_num_threads(cpu_threads())
    F = torch.nn.functional
    g_ = torch.Generator().manual_seed(1)
    out = {}

    def qkvgb(Bt, T, hv=HV):
        q = R.l2norm(torch.randn(Bt, hv, T, D, generator=g_).to(torch.bfloat16).float()) * D ** -0.5
        k = R.l2norm(torch.randn(Bt, hv, T, D, generator=g_).to(torch.bfloat16).float())
        v = torch.randn(Bt, hv, T, D, generator=g_).to(torch.bfloat16).float()
        g = -F.softplus(torch.randn(Bt, hv, T, generator=g_))
        beta = torch.sigmoid(torch.randn(Bt, hv, T, generator=g_))
        return q, k, v, g, beta

    # config 0: 256 sequential steps, B = 1
    q, k, v, g, beta = qkvgb(1, 256)
    t = _median_time(lambda: R.delta_rule_recurrent(q, k, v, g, beta, None))
    out["config0_recurrent"] = {"value": round(256 / t, 1), "unit": "tok/s", "sample": "full: B=1, 256 steps, 32 heads"}
    # config 2: chunked prefill on a 1024-token sample
    Ts = 1024
    q, k, v, g, beta = qkvgb(1, Ts)
    t = _median_time(lambda: R.delta_rule_chunked(q, k, v, g, beta, None))
    out["config2_prefill"] = {"value": round(Ts / t, 1), "unit": "tok/s",
                              "sample": f"first {Ts} of {PREFILL_T} tokens, B=1, 32 heads (linear in T)"}
    # config 3: one decode point
    L, Bt = 32768, 1
    kc = torch.randn(Bt, ATTN_KV, L + 1, ATTN_HD, generator=g_).to(torch.bfloat16)
    vc = torch.randn(Bt, ATTN_KV, L + 1, ATTN_HD, generator=g_).to(torch.bfloat16)
    qg = torch.randn(Bt, ATTN_H, 2 * ATTN_HD, generator=g_).to(torch.bfloat16)
    kn = torch.randn(Bt, ATTN_KV, ATTN_HD, generator=g_).to(torch.bfloat16)
    vn = torch.randn(Bt, ATTN_KV, ATTN_HD, generator=g_).to(torch.bfloat16)
    zw = torch.zeros(ATTN_HD)
    t = _median_time(lambda: R.attention_decode(qg, kn, vn, zw, zw, kc, vc, L, ATTN_RD, ATTN_THETA))
    out["config3_decode"] = {"value": round(Bt / t, 1), "unit": "tok/s", "sample": f"B={Bt}, L={L} (one of nine points)"}
    del kc, vc
    # config 4: one layer of each kind at full shape
    Cc = 2 * HK * D + HV * D

    def w(*shape, std=0.02):
        return (torch.randn(*shape, generator=g_) * std).to(torch.bfloat16)
    Wd = {"norm1": w(2048), "w_qkv": w(Cc, 2048), "w_z": w(4096, 2048), "w_b": w(32, 2048), "w_a": w(32, 2048),
          "conv_w": w(Cc, 4, std=0.05), "a_log": w(32, std=0.5), "dt_bias": w(32, std=0.5),
          "gnorm_w": w(128, std=0.1) + 1, "w_out": w(2048, 4096)}
    Wa = {"norm1": w(2048), "w_q": w(8192, 2048), "w_k": w(512, 2048), "w_v": w(512, 2048), "w_o": w(2048, 4096),
          "q_norm": w(256, std=0.1), "k_norm": w(256, std=0.1)}
    B4, T4, Tp = 16, 2048, 256
    conv, st = torch.zeros(B4, Cc, 3), torch.zeros(B4, HV, D, D)
    kc4 = torch.zeros(B4, ATTN_KV, T4 + 1, ATTN_HD, dtype=torch.bfloat16)
    vc4 = torch.zeros_like(kc4)
    h1 = torch.randn(B4, 1, 2048, generator=g_)
    td = _median_time(lambda: R.gated_deltanet_mixer(h1, Wd, conv, st.clone(), 1, HK, HV))
    ta = _median_time(lambda: R.gated_attention_mixer(h1, Wa, kc4, vc4, T4, ATTN_H, ATTN_KV))
    hp = torch.randn(1, Tp, 2048, generator=g_)
    tdp = _median_time(lambda: R.gated_deltanet_mixer(hp, Wd, torch.zeros(1, Cc, 3), torch.zeros(1, HV, D, D), 0,
                                                      HK, HV))
    tap = _median_time(lambda: R.gated_attention_mixer(hp, Wa, kc4[:1], vc4[:1], 0, ATTN_H, ATTN_KV))
    step = 30 * td + 10 * ta
    # prefill: per-token cost of the 256-token sample (attention's quadratic part is a small
    # share of its layer at T = 2048; the sample understates it, so the CPU figure is generous)
    pre_tok_s = Tp / (30 * tdp + 10 * tap)
    out["config4_stack"] = {"decode_tok_s": round(B4 / step, 2), "prefill_tok_s": round(pre_tok_s, 1),
                            "unit": "tok/s",
                            "sample": f"one DeltaNet + one attention layer at d 2048: decode at B={B4} over "
                                      f"{T4} cached tokens, prefill on {Tp} tokens of one sequence; scaled to 30 + 10 "
                                      f"layers"}
    return out


def prefill_parity(torch, ops, dev, R):
    """Config 2 at full size (B=1, T=8192, bf16 q/k/v normalised in-kernel, zero state): the HIP
    chunked prefill (fp32 output) against the oracle's chunked form on the same values."""
    bf = torch.bfloat16
    q = ops.fill_normal(torch.empty(1, PREFILL_T, HK, D, device=dev, dtype=bf), 7101).transpose(1, 2)
    k = ops.fill_normal(torch.empty(1, PREFILL_T, HK, D, device=dev, dtype=bf), 7102).transpose(1, 2)
    v = ops.fill_normal(torch.empty(1, PREFILL_T, HV, D, device=dev, dtype=bf), 7103).transpose(1, 2)
    g = -torch.nn.functional.softplus(ops.fill_normal(torch.empty(1, HV, PREFILL_T, device=dev), 7104))
    beta = torch.sigmoid(ops.fill_normal(torch.empty(1, HV, PREFILL_T, device=dev), 7105))
    od, Sd = ops.delta_rule_chunked(q, k, v, g, beta, None, normalize=True, qscale=D ** -0.5)
    rep = HV // HK
    qc = R.l2norm(q.float().cpu().repeat_interleave(rep, 1), 1e-6) * D ** -0.5
    kc = R.l2norm(k.float().cpu().repeat_interleave(rep, 1), 1e-6)
    oc, Sc = R.delta_rule_chunked(qc, kc, v.float().cpu(), g.cpu(), beta.cpu(), None)
    return {"o": _errs(torch, od, oc), "state": _errs(torch, Sd, Sc)}


PREFILL_T = 8192
# algorithmic FLOPs per (value head, 64-token chunk): kb k^T, two unit-triangular solves,
# q k^T, w S, q S, k^T v_new, intra v_new (C = 64, d = 128)
FLOP_PER_HEAD_CHUNK = 2 * 64 * 64 * 128 + 2 * (64 * 63 // 2) * 128 * 2 + 2 * 64 * 64 * 128 + 3 * 2 * 64 * 128 * 128 \
    + 2 * 64 * 64 * 128


def bench_prefill(torch, ops, dev, reps=40):
    """Config 2: chunked DeltaNet prefill, B=1, T=8192, 16 QK / 32 V heads, bf16 q/k/v
    (normalised in-kernel), fp32 state; one layer per call."""
    bf = torch.bfloat16
    q = ops.fill_normal(torch.empty(1, PREFILL_T, HK, D, device=dev, dtype=bf), 7001).transpose(1, 2)
    k = ops.fill_normal(torch.empty(1, PREFILL_T, HK, D, device=dev, dtype=bf), 7002).transpose(1, 2)
    v = ops.fill_normal(torch.empty(1, PREFILL_T, HV, D, device=dev, dtype=bf), 7003).transpose(1, 2)
    # g / beta generated token-major ([B, T, HV], the engine's gb layout) and passed as [B, HV, T]
    # views, so the binding's layout change is a no-op and the timed call is the kernels alone
    g = -torch.nn.functional.softplus(ops.fill_normal(torch.empty(1, PREFILL_T, HV, device=dev), 7004)).transpose(1, 2)
    beta = torch.sigmoid(ops.fill_normal(torch.empty(1, PREFILL_T, HV, device=dev), 7005)).transpose(1, 2)
    S = torch.zeros(1, HV, D, D, device=dev)
    run = lambda: ops.delta_rule_chunked(q, k, v, g, beta, S, normalize=True, qscale=D ** -0.5, out_dtype=bf)
    # ~100 ms of warm-up: after the CPU-side legs the GPU clocks need that long to ramp back up
    t_end = time.perf_counter() + 0.1
    while time.perf_counter() < t_end:
        for _ in range(20):
            run()
        torch.cuda.synchronize()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    flops = FLOP_PER_HEAD_CHUNK * HV * (PREFILL_T // 64)
    tflops = flops / (ms * 1e-3) / 1e12
    return {"workload": "config2: chunked WY prefill, B=1, T=8192, 32 V heads, one layer", "ms": round(ms, 4),
            "tok_s": round(PREFILL_T / (ms * 1e-3), 1), "tflops": round(tflops, 2),
            "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "flop_per_call": flops}


ATTN_H, ATTN_KV, ATTN_HD, ATTN_RD, ATTN_THETA = 16, 2, 256, 64, 1e7


def attn_decode_bytes(Bt, L):
    """Algorithmic bytes of one gated attention decode call over L cached rows (+ the new one):
    bf16 K and V rows read, q and gate in, new k / v in and appended, output out."""
    return 2048 * Bt * (L + 1) + Bt * ATTN_H * ATTN_HD * 2 * 3 + Bt * ATTN_KV * ATTN_HD * 2 * 2


def bench_decode_step(torch, ops, dev, L=4096, reps=10):
    """The north-star decode step at batch 64: the 30 DeltaNet layers (config 1's fused decode
    launch, each on its own state) and the 10 gated-attention layers (config 3's decode at
    L = 4096, each on its own K / V cache), interleaved 3 : 1 as in the stack, inputs resident
    in HBM. Roofline: the sum of both kinds' algorithmic bytes over the step time."""
    from aegist_mixer._lib import BF16, call, lib
    bf = torch.bfloat16
    stream = torch.cuda.current_stream().cuda_stream
    delta, attn = [], []
    for l in range(LAYERS):
        st = ops.fill_normal(torch.empty(B, HV, D, D, device=dev), 1000 + l, 0.0, 0.02)
        qkv = ops.fill_normal(torch.empty(B, C, device=dev, dtype=bf), 2000 + l)
        cs = ops.fill_normal(torch.empty(B, C, 3, device=dev), 3000 + l)
        w = ops.fill_normal(torch.empty(C, 4, device=dev, dtype=bf), 4000 + l, 0.0, 0.05)
        g = -torch.nn.functional.softplus(ops.fill_normal(torch.empty(B, HV, device=dev), 5000 + l))
        beta = torch.sigmoid(ops.fill_normal(torch.empty(B, HV, device=dev), 6000 + l))
        delta.append((qkv, w, cs, g, beta, st, torch.empty(B, HV, D, device=dev, dtype=bf)))
    cap = L + 1
    nbytes = lib().aegist_attention_decode_workspace_bytes(B, ATTN_H, ATTN_KV, cap)
    ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    for l in range(LAYERS // 3):
        kc = ops.fill_normal(torch.empty(B, ATTN_KV, cap, ATTN_HD, device=dev, dtype=bf), 8001 + 10 * l)
        vc = ops.fill_normal(torch.empty(B, ATTN_KV, cap, ATTN_HD, device=dev, dtype=bf), 8002 + 10 * l)
        qg = ops.fill_normal(torch.empty(B, ATTN_H, 2 * ATTN_HD, device=dev, dtype=bf), 8003 + 10 * l)
        kn = ops.fill_normal(torch.empty(B, ATTN_KV, ATTN_HD, device=dev, dtype=bf), 8004 + 10 * l)
        vn = ops.fill_normal(torch.empty(B, ATTN_KV, ATTN_HD, device=dev, dtype=bf), 8005 + 10 * l)
        nw = ops.fill_normal(torch.empty(2, ATTN_HD, device=dev, dtype=bf), 8006 + 10 * l, 0.0, 0.1)
        attn.append((qg, kn, vn, nw, kc, vc, torch.empty(B, ATTN_H, ATTN_HD, device=dev, dtype=bf)))
    torch.cuda.synchronize()

    def run_delta(t):
        qkv, w, cs, g, beta, st, out = t
        call("aegist_delta_decode_step", qkv.data_ptr(), BF16, w.data_ptr(), cs.data_ptr(), g.data_ptr(),
             beta.data_ptr(), st.data_ptr(), out.data_ptr(), BF16, B, HK, HV, D ** -0.5, 1e-6, stream)

    def run_attn(t):
        qg, kn, vn, nw, kc, vc, o = t
        # position L: the new row is written at L (the same slot every step) and attended with the L before it
        call("aegist_attention_decode", qg.data_ptr(), kn.data_ptr(), vn.data_ptr(), BF16, nw[0].data_ptr(),
             nw[1].data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(), BF16, B, ATTN_H, ATTN_KV, ATTN_HD,
             ATTN_RD, L, cap, 1e-6, ATTN_THETA, ws.data_ptr(), nbytes, stream)

    def step():
        for l in range(LAYERS // 3):
            for j in range(3):
                run_delta(delta[3 * l + j])
            run_attn(attn[l])

    def timed(fn, n):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n
    ms = timed(step, reps)
    ms_attn = timed(lambda: [run_attn(t) for t in attn], reps)
    byt_d = LAYERS * decode_bytes_per_launch()
    byt_a = (LAYERS // 3) * attn_decode_bytes(B, L)
    gbs = (byt_d + byt_a) / (ms * 1e-3) / 1e9
    a_gbs = byt_a / (ms_attn * 1e-3) / 1e9
    del delta, attn, ws
    torch.cuda.empty_cache()
    return {"workload": f"batch-{B} decode step: 30 DeltaNet layers (config 1) + 10 gated GQA layers "
                        f"(16 q / 2 KV heads, HD 256, L={L} cached rows each, distinct caches)",
            "ms_per_step": round(ms, 4), "tok_s": round(B / (ms * 1e-3), 1),
            "bytes_per_step": byt_d + byt_a,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)},
            "attention_only": {"ms_10_layers": round(ms_attn, 4), "GB_s": round(a_gbs, 1),
                               "hbm_frac": round(a_gbs / HBM_PEAK_GBS, 4)}}


def bench_attention_decode(torch, ops, dev, reps=20):
    """Config 3: gated GQA decode (ZNorm + RoPE of q and the new k, cache append, split-K
    attention over L+1 rows, sigmoid gate) at L in {4k, 32k, 128k} x B in {1, 8, 32}.
    Bytes per call = 2048 B L (bf16 K and V) + q/gate/new k, v/out."""
    from aegist_mixer._lib import BF16, call, lib
    out = []
    bf = torch.bfloat16
    stream = torch.cuda.current_stream().cuda_stream
    for L in (4096, 32768, 131072):
        for Bt in (1, 8, 32, 64):
            cap = L + 1
            kc = ops.fill_normal(torch.empty(Bt, ATTN_KV, cap, ATTN_HD, device=dev, dtype=bf), 8001)
            vc = ops.fill_normal(torch.empty(Bt, ATTN_KV, cap, ATTN_HD, device=dev, dtype=bf), 8002)
            qg = ops.fill_normal(torch.empty(Bt, ATTN_H, 2 * ATTN_HD, device=dev, dtype=bf), 8003)
            kn = ops.fill_normal(torch.empty(Bt, ATTN_KV, ATTN_HD, device=dev, dtype=bf), 8004)
            vn = ops.fill_normal(torch.empty(Bt, ATTN_KV, ATTN_HD, device=dev, dtype=bf), 8005)
            qw = torch.zeros(ATTN_HD, device=dev, dtype=bf)
            kw = torch.zeros(ATTN_HD, device=dev, dtype=bf)
            o = torch.empty(Bt, ATTN_H, ATTN_HD, device=dev, dtype=bf)
            nbytes = lib().aegist_attention_decode_workspace_bytes(Bt, ATTN_H, ATTN_KV, L + 1)
            ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)

            def run():
                call("aegist_attention_decode", qg.data_ptr(), kn.data_ptr(), vn.data_ptr(), BF16, qw.data_ptr(),
                     kw.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(), BF16, Bt, ATTN_H, ATTN_KV, ATTN_HD,
                     ATTN_RD, L, cap, 1e-6, ATTN_THETA, ws.data_ptr(), nbytes, stream)
            for _ in range(3):
                run()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                run()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            byt = attn_decode_bytes(Bt, L)
            gbs = byt / (us * 1e-6) / 1e9
            out.append({"L": L, "B": Bt, "us": round(us, 2), "tok_s": round(Bt / (us * 1e-6), 1),
                        "GB_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
            del kc, vc, ws
            torch.cuda.empty_cache()
    return {"workload": "config3: gated GQA decode, 16 q heads / 2 KV heads, HD 256, bf16 cache", "points": out,
            "note": "L=4096 at B=1 (8 MB) is MALL-resident and launch-bound"}


def bench_attention_prefill(torch, ops, dev, T=2048, reps=40):
    """Causal gated GQA prefill (config 4's attention layers): T=2048, 16 q heads, 2 KV heads,
    HD 256, cache rows [0, T), at config 4's B=16 (the headline fields) and at B=1 (`points`).
    FLOPs = 4 * B * H * HD * T (T + 1) / 2 (QK^T and PV)."""
    from aegist_mixer._lib import call, lib
    bf = torch.bfloat16
    stream = torch.cuda.current_stream().cuda_stream
    points = []
    for B in (1, 16):
        q = ops.fill_normal(torch.empty(B, ATTN_H, T, ATTN_HD, device=dev), 9001)
        kc = ops.fill_normal(torch.empty(B, ATTN_KV, T, ATTN_HD, device=dev, dtype=bf), 9002)
        vc = ops.fill_normal(torch.empty(B, ATTN_KV, T, ATTN_HD, device=dev, dtype=bf), 9003)
        gate = ops.fill_normal(torch.empty(B, T, ATTN_H * ATTN_HD, device=dev), 9004)
        out = torch.empty(B, T, ATTN_H, ATTN_HD, device=dev)
        # the fp16 copy of the cache rows the kernel reads (allocated outside the timing; its
        # conversion pass runs inside every timed call)
        nws = lib().aegist_attention_core_workspace_bytes(B, ATTN_H, ATTN_KV, T, 0)
        ws = torch.empty(nws, dtype=torch.uint8, device=dev)

        def run():
            call("aegist_attention_core", q.data_ptr(), kc.data_ptr(), vc.data_ptr(), gate.data_ptr(), out.data_ptr(),
                 B, ATTN_H, ATTN_KV, T, 0, T, ATTN_HD ** -0.5, ws.data_ptr(), nws, stream)
        for _ in range(2):
            run()
        torch.cuda.synchronize()
        n = reps if B == 1 else max(2, reps // 4)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            run()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / n
        tf = 4 * B * ATTN_H * ATTN_HD * T * (T + 1) / 2 / (us * 1e-6) / 1e12
        points.append({"B": B, "us": round(us, 2), "tflops": round(tf, 2), "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)})
        del q, kc, vc, gate, out, ws
    p16 = points[-1]
    return {"workload": f"causal gated GQA prefill, T={T}, 16/2 heads, HD 256 (headline fields: config 4's B=16; "
                        f"B=1 in points)",
            "us": p16["us"], "tflops": p16["tflops"], "mfma_frac": p16["mfma_frac"], "points": points}


def bench_gemm(torch, ops, dev, reps=10):
    """Prefill-sized projections of config 4 (M = 16 x 2048 tokens, bf16 weights and activations,
    fp32 out): the library's tiled MFMA GEMM through `aegist_linear`, and torch's bf16 matmul
    (hipBLASLt / rocBLAS, bf16 out) on the same operands as a library reference. FLOPs = 2 M N K."""
    M = 16 * 2048
    shapes = [(8192, 2048, False, "in_qkv / attention q|gate"), (4096, 2048, False, "in_z"),
              (2048, 4096, True, "out projection (+= residual)")]
    points = []
    for N, K, acc, what in shapes:
        x = ops.fill_normal(torch.empty(M, K, device=dev, dtype=torch.bfloat16), 7001)
        w = ops.fill_normal(torch.empty(N, K, device=dev, dtype=torch.bfloat16), 7002, std=0.02)
        y = torch.zeros(M, N, device=dev)

        def ours():
            ops.linear(x, w, out=y, accumulate=acc)

        def lib_ref():
            torch.matmul(x, w.t())

        row = {"N": N, "K": K, "what": what}
        for name, fn in (("ours", ours), ("torch_bf16_out", lib_ref)):
            for _ in range(2):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
            row[name + "_us"] = round(us, 1)
            row[name + "_tflops"] = round(tf, 1)
        row["mfma_frac"] = round(row["ours_tflops"] / MFMA_BF16_PEAK_TFLOPS, 4)
        points.append(row)
        del x, w, y
    # the engine's QLinear GEMM (int8 weights, bf16 row scales, fp32 activations) on a 1024-token
    # prefill chunk
    from aegist_mixer._lib import call
    Mi, Ni, Ki = 1024, 8192, 2048
    xi = ops.fill_normal(torch.empty(Mi, Ki, device=dev), 7003)
    qi = torch.randint(-127, 128, (Ni, Ki), device=dev, dtype=torch.int8)
    si = ops.fill_normal(torch.empty(Ni, device=dev, dtype=torch.bfloat16), 7004, mean=0.01, std=0.001)
    yi = torch.zeros(Mi, Ni, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def gi8():
        call("aegist_gemm_i8", xi.data_ptr(), qi.data_ptr(), si.data_ptr(), yi.data_ptr(), Mi, Ni, Ki, 0, stream)
    for _ in range(2):
        gi8()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        gi8()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    i8 = {"M": Mi, "N": Ni, "K": Ki, "us": round(us, 1), "tflops": round(2.0 * Mi * Ni * Ki / (us * 1e-6) / 1e12, 1)}
    del xi, qi, si, yi
    return {"workload": f"config4 prefill projections, M={M}, bf16 x bf16 -> fp32", "points": points,
            "gemm_i8": i8}


def bench_proj(torch, ops, dev, reps=3):
    """Decode-sized projections (QLinear int8 + bf16 scale with fp32 activations, as the engine
    ships them; bf16 weights with bf16 activations, as config 4 runs them). The timed loop walks
    a ring of distinct weight matrices totalling > 1 GB so that every launch streams its weights
    from HBM, as a 40-layer decode step does (a single 17-67 MB matrix would sit in the MALL).
    Bytes per launch = W + X + Y. A workspace is bound on the calling thread (as the engine binds
    its scratch), which lets 17..64 rows against a weight of few rows split K."""
    from aegist_mixer._lib import BF16, F32, I8, call
    stream = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(16 << 20, device=dev, dtype=torch.uint8)
    call("aegist_bind_workspace", ws.data_ptr(), ws.numel())
    out = []
    for wdt, xdt, N, K in [(I8, F32, 8192, 2048), (BF16, BF16, 8192, 2048), (BF16, BF16, 2048, 4096)]:
        wbytes = N * K * (1 if wdt == I8 else 2)
        ncopy = max(2, (1 << 30) // wbytes + 1)
        if wdt == I8:
            Ws = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev) for _ in range(ncopy)]
            sc = ops.fill_normal(torch.empty(N, device=dev, dtype=torch.bfloat16), 77, 1e-3, 0.0)
        else:
            Ws = [ops.fill_normal(torch.empty(N, K, device=dev, dtype=torch.bfloat16), 80 + i, 0.0, 0.02)
                  for i in range(ncopy)]
            sc = None
        for M in (1, 16, 64):
            X = ops.fill_normal(torch.empty(M, K, device=dev, dtype=torch.float32 if xdt == F32 else torch.bfloat16), 5)
            Y = torch.empty(M, N, device=dev)

            def run(Wm):
                call("aegist_linear", X.data_ptr(), xdt, K, Wm.data_ptr(), wdt, None if sc is None else sc.data_ptr(),
                     Y.data_ptr(), N, M, N, K, 0, stream)
            for Wm in Ws[:2]:
                run(Wm)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                for Wm in Ws:
                    run(Wm)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (reps * ncopy)
            nbytes = wbytes + M * K * X.element_size() + M * N * 4
            gbs = nbytes / (us * 1e-6) / 1e9
            out.append({"w": "int8" if wdt == I8 else "bf16", "x": "fp32" if xdt == F32 else "bf16", "M": M, "N": N,
                        "K": K, "us": round(us, 2), "GB_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
        del Ws
        torch.cuda.empty_cache()
    call("aegist_bind_workspace", None, 0)
    del ws
    return {"workload": "decode projections Y[M,N] = X[M,K] W[N,K]^T (x scale), weights streamed from HBM "
                        "(16 MB workspace bound)", "points": out}


def bench_moe(torch, ops, dev, reps=3):
    """MoE block after the mixer (hybrid.py:631-652): router top-8 of 256 experts, then the 4-bit
    SwiGLU experts (D 2048, I 512, 64-groups: 1,769,472 bytes per expert) added into the residual.
    Decode points stream a ring of 6 layers' experts (2.7 GB, beyond the MALL) and are priced
    against HBM: bytes = unique experts touched x expert bytes + router weights + activations.
    The prefill point (T = 2048, one layer) is priced in algorithmic FLOPs, 2 T K (2 I D + D I)."""
    from aegist_mixer._lib import call, lib
    E, K, D, I, NL = 256, 8, 2048, 512, 6
    rb = 1769472
    gu_q, gu_s = 2 * I * D // 2, 2 * I * (D // 64) * 2
    dn_q, dn_s = D * I // 2, D * (I // 64) * 2
    layers = []
    for li in range(NL):
        rows = torch.randint(0, 256, (E, rb), dtype=torch.uint8, device=dev)
        for off, nb, v in ((gu_q, gu_s, 0.005), (gu_q + gu_s, gu_s, -0.03), (gu_q + 2 * gu_s + dn_q, dn_s, 0.005),
                           (gu_q + 2 * gu_s + dn_q + dn_s, dn_s, -0.03)):
            rows[:, off:off + nb].view(torch.float16).fill_(v)
        eptr = torch.arange(E, dtype=torch.int64, device=dev) * rb + rows.data_ptr()
        W = (torch.randn(E, D, device=dev) * 0.02).to(torch.bfloat16)
        layers.append((rows, eptr, W))
    stream = torch.cuda.current_stream().cuda_stream
    points = []
    for T in (1, 16, 64, 2048):
        h = torch.randn(T, D, device=dev)
        x = torch.zeros(T, D, device=dev)
        idx = torch.empty(T, K, dtype=torch.int32, device=dev)
        wts = torch.empty(T, K, device=dev)
        need = lib().aegist_moe_workspace_bytes(T, K, D, I, E)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        rneed = lib().aegist_router_topk_workspace_bytes(T, E)
        rws = torch.empty(max(rneed, 1), dtype=torch.uint8, device=dev)
        uniq = []

        def run(li):
            rows, eptr, W = layers[li]
            call("aegist_router_topk_ws", h.data_ptr(), W.data_ptr(), idx.data_ptr(), wts.data_ptr(), T, D, E, K,
                 rws.data_ptr(), rneed, stream)
            call("aegist_moe_experts", h.data_ptr(), eptr.data_ptr(), idx.data_ptr(), wts.data_ptr(), x.data_ptr(),
                 T, D, I, E, K, None, None, ws.data_ptr(), need, stream)
        for li in range(NL):
            run(li)
            uniq.append(int(torch.unique(idx).numel()))
        torch.cuda.synchronize()
        n = NL * (reps if T < 2048 else 1)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            run(i % NL)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / n
        u = sum(uniq) / len(uniq)
        pt = {"T": T, "us": round(us, 2), "unique_experts": round(u, 1)}
        if T < 2048:
            byts = u * rb + E * D * 2 + T * D * 4 * 3
            pt.update({"GB_s": round(byts / us / 1e3, 1), "hbm_frac": round(byts / us / 1e3 / HBM_PEAK_GBS, 4)})
        else:
            tf = 2 * T * K * (2 * I * D + D * I) / (us * 1e-6) / 1e12
            pt.update({"tflops": round(tf, 2), "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)})
        points.append(pt)
        del h, x, idx, wts, ws
    del layers
    return {"workload": "MoE block: router top-8 of 256, 4-bit SwiGLU experts D 2048 / I 512 (group 64), residual add",
            "points": points}


def bench_qsa(torch, ops, dev, reps=20):
    """Second core's sparse decode step at long context: one query at position L - 1 with
    L = 131072, R = 4 (32768 blocks), top = 512 (budget 2048), 16 index heads of 128 (an assumed
    head count: the released config is not in the reference tree), then attention over the 512
    listed blocks + tail with 16 / 2 heads of 256. Times each kernel of the decode-time path
    (block scores, top-k select, listed attention) with HIP events."""
    from aegist_mixer._lib import call, lib
    stream = torch.cuda.current_stream().cuda_stream
    L, RB, top, H, KV, HD, IH = 131072, 4, 512, 16, 2, 256, 16
    nb = L // RB
    pos0 = L - 1
    qi = ops.fill_normal(torch.empty(1, IH, 128, device=dev), 71)
    bk = ops.fill_normal(torch.empty(nb, 128, device=dev), 72)
    sc = torch.empty(1, nb, device=dev)
    blist = torch.empty(1, top, dtype=torch.int32, device=dev)
    nsel = torch.empty(1, dtype=torch.int32, device=dev)
    q = ops.fill_normal(torch.empty(1, H, HD, device=dev), 73)
    kc = ops.fill_normal(torch.empty(KV, L, HD, device=dev, dtype=torch.bfloat16), 74)
    vc = ops.fill_normal(torch.empty(KV, L, HD, device=dev, dtype=torch.bfloat16), 75)
    qg = ops.fill_normal(torch.empty(1, H, 2 * HD, device=dev), 76)
    out = torch.empty(1, H, HD, device=dev)
    sel_need = lib().aegist_idx_select_workspace_bytes(1, top, RB, pos0)
    sel_ws = torch.empty(max(sel_need, 1), dtype=torch.uint8, device=dev)
    lst_need = lib().aegist_attention_gated_list_workspace_bytes(1, H, KV, pos0, top, RB)
    lst_ws = torch.empty(max(lst_need, 1), dtype=torch.uint8, device=dev)
    steps = {
        "scores": lambda: call("aegist_idx_scores", qi.data_ptr(), bk.data_ptr(), sc.data_ptr(), 1, IH, 128, pos0, RB,
                               nb, stream),
        "select": lambda: call("aegist_idx_select_ws", sc.data_ptr(), blist.data_ptr(), nsel.data_ptr(), 1, top, RB,
                               pos0, nb, sel_ws.data_ptr(), sel_need, stream),
        "attention_list": lambda: call("aegist_attention_gated_list_ws", q.data_ptr(), kc.data_ptr(),
                                       vc.data_ptr(), qg.data_ptr(), out.data_ptr(), 1, H, KV, pos0, L, HD ** -0.5,
                                       blist.data_ptr(), nsel.data_ptr(), top, RB, lst_ws.data_ptr(), lst_need, stream),
    }
    res = {"workload": f"QSA sparse decode, L={L}, R={RB}, top={top}, 16 index heads x 128, 16/2 heads x 256",
           "note": "16 index heads is an assumption (the released head count is not in the reference tree)"}
    for name, fn in steps.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name + "_us"] = round(e0.elapsed_time(e1) * 1e3 / reps, 2)
    # bytes: block keys for the scores; 2 KV heads x (top R + tail) rows of K and V for the attention
    res["scores_GB_s"] = round(nb * 128 * 4 / (res["scores_us"] * 1e-6) / 1e9, 1)
    res["attention_list_GB_s"] = round(KV * (top * RB + RB) * HD * 2 * 2 / (res["attention_list_us"] * 1e-6) / 1e9, 1)
    return res


def bench_stack(torch, ops, dev, B=16, T=2048, steps=256):
    """Config 4: 40-layer hybrid mixer stack (3 DeltaNet + 1 attention, x10; d 2048), bf16
    projection weights ~N(0, 0.02) (random init), MoE FFN as identity, bf16 embedding table
    ~N(0, 0.02) with random token ids. Prefill B x T tokens, then `steps` decode steps at B."""
    bf = torch.bfloat16
    cfg = dict(d_model=2048, hk=16, hv=32, n_heads=16, n_kv=2, head_dim=256, rotary_dim=64, rope_theta=1e7, eps=1e-6)
    kinds = (["delta"] * 3 + ["attn"]) * 10
    C = 2 * 16 * 128 + 32 * 128
    seed = [100]

    def w(*shape, std=0.02):
        seed[0] += 1
        return ops.fill_normal(torch.empty(*shape, device=dev, dtype=bf), seed[0], 0.0, std)
    layers = []
    for kind in kinds:
        W = {"norm1": w(2048, std=0.0)}
        if kind == "delta":
            W.update(w_qkv=w(C, 2048), w_z=w(4096, 2048), w_b=w(32, 2048), w_a=w(32, 2048), conv_w=w(C, 4, std=0.05),
                     a_log=w(32, std=0.0), dt_bias=w(32, std=0.0), gnorm_w=w(128, std=0.0), w_out=w(2048, 4096))
            W["dt_bias"].fill_(1.0)
            W["gnorm_w"].fill_(1.0)
        else:
            W.update(w_q=w(8192, 2048), w_k=w(512, 2048), w_v=w(512, 2048), w_o=w(2048, 4096), q_norm=w(256, std=0.0),
                     k_norm=w(256, std=0.0))
        layers.append(W)
    table = w(4096, 2048)
    stack = ops.HybridStack(cfg, kinds, layers, max_batch=B, max_tokens=B * T, max_context=T + steps)
    ids = torch.randint(0, 4096, (B, T + steps), generator=torch.Generator().manual_seed(5), dtype=torch.int32).to(dev)
    e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    # warm-up pass, then the timed run from a reset state
    x = ops.embed(table, ids[:, :T].reshape(-1)).view(B, T, 2048)
    stack.forward(x)
    stack.reset()
    torch.cuda.synchronize()
    e[0].record()
    x = ops.embed(table, ids[:, :T].reshape(-1)).view(B, T, 2048)
    stack.forward(x)
    e[1].record()
    for s in range(steps):
        xt = ops.embed(table, ids[:, T + s].contiguous()).view(B, 1, 2048)
        stack.forward(xt)
    e[2].record()
    torch.cuda.synchronize()
    pre_ms, dec_ms = e[0].elapsed_time(e[1]), e[1].elapsed_time(e[2])
    stack.close()
    # decode roofline: algorithmic HBM bytes of one B-token step = every projection weight once,
    # each DeltaNet layer's recurrent state read + written and conv state read + written, each
    # attention layer's K and V rows read (mean context over the timed steps), the new K / V rows
    nd, na = kinds.count("delta"), kinds.count("attn")
    w_delta = (C + 4096 + 32 + 32) * 2048 * 2 + 2048 * 4096 * 2
    w_attn = (8192 + 512 + 512) * 2048 * 2 + 2048 * 4096 * 2
    st_bytes = B * (2 * 32 * 128 * 128 * 4 + 2 * C * 3 * 4)
    mean_L = T + (steps + 1) / 2
    kv_bytes = B * 2 * mean_L * 256 * 2 * 2
    step_bytes = nd * (w_delta + st_bytes) + na * (w_attn + kv_bytes)
    gbs = step_bytes / (dec_ms / steps * 1e-3) / 1e9
    return {"workload": f"config4: 40-layer mixer stack, d 2048, prefill {B}x{T} then {steps} decode steps at B={B}",
            "prefill_ms": round(pre_ms, 3), "prefill_tok_s": round(B * T / (pre_ms * 1e-3), 1),
            "decode_ms_per_step": round(dec_ms / steps, 4), "decode_tok_s": round(B * steps / (dec_ms * 1e-3), 1),
            "total_tok_s": round(B * (T + steps) / ((pre_ms + dec_ms) * 1e-3), 1),
            "decode_roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_step": int(step_bytes)},
            "finite": bool(torch.isfinite(xt).all().item())}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a 1 GiB device copy (calibrates rocprof FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--legs", type=str, default="prefill,decode_step,attention_decode,attention_prefill,gemm,proj,qsa,moe,stack",
                    help="comma list of the extra legs to run after the decode headline (default: all); "
                         "'none' for the headline only")
    ap.add_argument("--traffic", type=str, default=str(ROOT / "profiles" / "delta_decode_traffic.json"),
                    help="JSON file with measured HBM bytes per decode launch (from rocprof --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the mixer path is not "
              f"sharded in this build", file=sys.stderr)
        sys.exit(2)

    import torch
    from aegist_mixer import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bf = torch.bfloat16
    # per-layer resident inputs, filled on the device by the counter-based generator
    layers = []
    for l in range(LAYERS):
        st = torch.empty(B, HV, D, D, device=dev)
        ops.fill_normal(st, 1000 + l, 0.0, 0.02)
        qkv = ops.fill_normal(torch.empty(B, C, device=dev, dtype=bf), 2000 + l)
        cs = ops.fill_normal(torch.empty(B, C, 3, device=dev), 3000 + l)
        w = ops.fill_normal(torch.empty(C, 4, device=dev, dtype=bf), 4000 + l, 0.0, 0.05)
        g = -torch.nn.functional.softplus(ops.fill_normal(torch.empty(B, HV, device=dev), 5000 + l))
        beta = torch.sigmoid(ops.fill_normal(torch.empty(B, HV, device=dev), 6000 + l))
        out = torch.empty(B, HV, D, device=dev, dtype=bf)
        layers.append((qkv, w, cs, g, beta, st, out))
    torch.cuda.synchronize()

    from aegist_mixer._lib import BF16, call
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        for (qkv, w, cs, g, beta, st, out) in layers:
            call("aegist_delta_decode_step", qkv.data_ptr(), BF16, w.data_ptr(), cs.data_ptr(), g.data_ptr(),
                 beta.data_ptr(), st.data_ptr(), out.data_ptr(), BF16, B, HK, HV, D ** -0.5, 1e-6, stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / args.steps
    value = B / (ms_step * 1e-3)
    # the headline's 3.84 GB of layer states are not needed by the legs below
    del layers
    torch.cuda.empty_cache()
    launch_ms = ms_step / LAYERS
    nbytes = decode_bytes_per_launch()
    achieved = nbytes / (launch_ms * 1e-3) / 1e9

    res = {
        "metric": "mixer decode tok/s @bs64 + % HBM roofline; DeltaNet prefill tok/s @8k",
        "value": round(value, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 state, bf16 I/O",
        "data": "synthetic (device counter-based N(0,1) generator; state N(0,0.02))",
        "config": {"workload": "config1: gated DeltaNet decode step, B=64, 16 QK / 32 V heads, d=128, "
                               "conv k=4 over 8192 channels, 30 layers (distinct states)",
                   "batch": B, "layers": LAYERS, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "delta_decode_kernel", "bytes_per_launch": nbytes,
                     "launch_us": round(launch_ms * 1e3, 2)},
        "wall_s": round(wall, 3),
    }
    if args.traffic and os.path.exists(args.traffic):
        with open(args.traffic) as f:
            res["roofline"]["traffic"] = json.load(f).get("bytes_per_launch")
    legs = {"prefill": bench_prefill, "decode_step": bench_decode_step, "attention_decode": bench_attention_decode,
            "attention_prefill": bench_attention_prefill, "proj": bench_proj, "qsa": bench_qsa,
            "moe": bench_moe, "stack": bench_stack, "gemm": bench_gemm}
    want = [] if args.legs.strip() == "none" else [x.strip() for x in args.legs.split(",") if x.strip()]
    unknown = [x for x in want if x not in legs]
    if unknown:
        print(f"unknown --legs {unknown}; choose from {sorted(legs)}", file=sys.stderr)
        sys.exit(2)
    for name in want:
        res[name] = legs[name](torch, ops, dev)
    if args.calib_copy:
        src = torch.empty(1 << 28, device=dev)  # 1 GiB fp32
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline_decode(torch, ops, dev)
        res["cpu_baseline"]["configs"] = cpu_baseline_configs(torch)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
