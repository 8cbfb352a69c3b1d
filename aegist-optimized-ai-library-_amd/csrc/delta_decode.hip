// Gated DeltaNet decode step, batched and fused, for gfx950.
//
// One workgroup per (sequence b, QK head kh) serves the R = HV/HK value heads that share that
// QK head, with 256 threads per value head. The workgroup
//   1. runs the causal conv (kernel 4) + SiLU for its 256 + 128R channels and writes the new
//      conv state (each channel is owned by exactly one workgroup, so the in-place update is
//      race-free),
//   2. L2-normalises q and k (q also times qscale) in fp32 through LDS,
//   3. streams each value head's 128x128 fp32 state HBM -> VGPRs -> HBM exactly once, in
//      four 32-column slices with two slices in flight (columns of S are independent): the
//      first two slices are requested before the conv even starts; per slice every thread
//      holds 4 rows x 4 columns, the column dot products S^T k and S^T q are reduced over
//      rows (three xor shuffles + LDS across 4 waves), then S' = e^g S + k delta^T is
//      written with delta = (v - e^g S^T k) beta, o = e^g S^T q + (k.q) delta is emitted,
//      and slice j+2 is requested. Loads and stores are nontemporal (streamed once).
// The o formula is S'^T q expanded, so the state is read once and written once: the kernel
// is HBM-bound at 2 x 64 KiB of state per (b, value head) plus ~2 KiB of conv traffic.
//
// Semantics: hybrid.py:390-413 (conv, split, l2norm, q scale, delta_rule_step :318-324);
// the engine's T == 1 path conv_silu -> l2norm_heads -> delta_scan (hybrid.cu:205-300).
#include "common.h"

using namespace aegist;

namespace {

constexpr int D = 128;  // dk = dv

// State traffic is streamed: nontemporal loads and stores keep the 128 MiB-per-layer state
// from displacing reusable lines in L2 / MALL.
__device__ __forceinline__ float4 ld_stream(const float* p) {
    float4 r;
    r.x = __builtin_nontemporal_load(p);
    r.y = __builtin_nontemporal_load(p + 1);
    r.z = __builtin_nontemporal_load(p + 2);
    r.w = __builtin_nontemporal_load(p + 3);
    return r;
}
__device__ __forceinline__ void st_stream(float* p, float4 v) {
    __builtin_nontemporal_store(v.x, p);
    __builtin_nontemporal_store(v.y, p + 1);
    __builtin_nontemporal_store(v.z, p + 2);
    __builtin_nontemporal_store(v.w, p + 3);
}

// Layer-stack form (kStack): the gates come from the b / a projection rows instead of g / beta
// arrays (beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias), as gates_from_proj), and the
// output row of each value head goes through the gated norm w * rmsnorm(o) * silu(z) into bf16
// (as gated_norm_bf16) inside the kernel: three launches of the stack's decode step become one.
struct StackGates {
    const float* ba;          // [B, 2 HV]: b, then a
    const uint16_t* a_log;    // [HV] bf16
    const uint16_t* dt_bias;  // [HV] bf16
    const float* z;           // [B, HV * D]
    const uint16_t* gnorm_w;  // [D] bf16
    float gnorm_eps;
};

template <int R, typename Tin, typename Tout, bool kStack = false>
__global__ void __launch_bounds__(256 * R) delta_decode_kernel(
    const Tin* __restrict__ qkv, const uint16_t* __restrict__ conv_w, float* __restrict__ conv_state,
    const float* __restrict__ g, const float* __restrict__ beta, float* __restrict__ state, Tout* __restrict__ out,
    int HK, int HV, float qscale, float eps, StackGates sg) {
    constexpr int NT = 256 * R;
    constexpr int NCH = 2 * D + R * D;
    __shared__ float sq[D], sk[D], sv[R][D];
    __shared__ float red[8];
    __shared__ float4 part[2][R][4][2][8];
    __shared__ float so[kStack ? R : 1][kStack ? D : 1];

    const int kh = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int C = 2 * HK * D + HV * D;
    const int wave = tid / WAVE, lane = tid % WAVE;
    // state mapping: per value head 256 threads; lane = (column group cg of 4 columns within a
    // 32-column slice, row group rr); thread rows rbase + 32 i, i < 4
    const int hl = tid / 256, lt = tid % 256, w4 = lt / WAVE, cg = lane % 8, rr = lane / 8;
    const int hv = kh * R + hl;
    float* S = state + ((size_t)b * HV + hv) * D * D;
    const int rbase = w4 * 8 + rr;

    // ---- 0. the inputs of this thread's first conv channel are requested first (the prologue
    // needs them first, and vector-memory loads return in order), then the state column slices
    // (independent of the conv): two in flight (4 workgroups' worth of state per CU at batch 64),
    // all four in the stack form, whose batch-16 grid is a single round of one workgroup per CU
    auto chan = [&](int ch) {
        return ch < D ? kh * D + ch : ch < 2 * D ? HK * D + kh * D + (ch - D) : 2 * HK * D + kh * R * D + (ch - 2 * D);
    };
    float xv0 = 0.f, c0s0 = 0.f, c0s1 = 0.f, c0s2 = 0.f;
    uint2 wp0 = {0u, 0u};
    if (tid < NCH) {
        const int c = chan(tid);
        xv0 = Act<Tin>::ld(qkv, (size_t)b * C + c);
        const float* st = conv_state + ((size_t)b * C + c) * 3;
        c0s0 = st[0];
        c0s1 = st[1];
        c0s2 = st[2];
        wp0 = *(const uint2*)(conv_w + (size_t)c * 4);
    }
    __builtin_amdgcn_sched_barrier(0);
    constexpr int NSF = kStack ? 4 : 2;
    float4 s[NSF][4];
#pragma unroll
    for (int j = 0; j < NSF; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) s[j][i] = ld_stream(S + (size_t)(rbase + 32 * i) * D + 32 * j + cg * 4);

    // ---- 1. conv + SiLU + conv-state update for this workgroup's channels
    float ymine = 0.f;
    for (int ch = tid; ch < NCH; ch += NT) {
        const int c = chan(ch);
        float* st = conv_state + ((size_t)b * C + c) * 3;
        float xv, s0, s1, s2;
        uint2 wp;
        if (ch == tid) {
            xv = xv0; s0 = c0s0; s1 = c0s1; s2 = c0s2; wp = wp0;
        } else {
            xv = Act<Tin>::ld(qkv, (size_t)b * C + c);
            s0 = st[0]; s1 = st[1]; s2 = st[2];
            wp = *(const uint2*)(conv_w + (size_t)c * 4);
        }
        const float acc = bf_lo(wp.x) * s0 + bf_hi(wp.x) * s1 + bf_lo(wp.y) * s2 + bf_hi(wp.y) * xv;
        const float y = silu_f(acc);
        st[0] = s1;
        st[1] = s2;
        st[2] = xv;
        if (ch < 2 * D) ymine = y;  // threads 0..255 keep their q/k channel for the norms
        else sv[(ch - 2 * D) / D][(ch - 2 * D) % D] = y;
    }

    // ---- 2. L2 norms: q lives in waves 0-1, k in waves 2-3
    if (tid < 2 * D) {
        float ss = wave_sum(ymine * ymine);
        if (lane == 0) red[wave] = ss;
    }
    __syncthreads();
    if (tid < D) {
        sq[tid] = (ymine * rsqrtf(red[0] + red[1] + eps)) * qscale;
    } else if (tid < 2 * D) {
        sk[tid - D] = ymine * rsqrtf(red[2] + red[3] + eps);
    }
    __syncthreads();
    if (tid < D) {
        float p = wave_sum(sq[tid] * sk[tid]);
        if (lane == 0) red[4 + wave] = p;
    }
    __syncthreads();
    const float kq = red[4] + red[5];
    float decay, bt;
    if constexpr (kStack) {
        const float bb = sg.ba[(size_t)b * 2 * HV + hv], aa = sg.ba[(size_t)b * 2 * HV + HV + hv];
        bt = 1.f / (1.f + expf(-bb));
        const float xx = aa + bf2f(sg.dt_bias[hv]);
        const float sp = xx > 20.f ? xx : log1pf(expf(xx));
        decay = expf(-expf(bf2f(sg.a_log[hv])) * sp);
    } else {
        decay = expf(g[(size_t)b * HV + hv]);
        bt = beta[(size_t)b * HV + hv];
    }
    float kr[4], qr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        kr[i] = sk[rbase + 32 * i];
        qr[i] = sq[rbase + 32 * i];
    }

    // ---- 3. four 32-column slices, two in flight: reduce, update, store, prefetch
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float4 pk = {0.f, 0.f, 0.f, 0.f}, pq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 x = s[j % NSF][i];
            pk.x += x.x * kr[i]; pk.y += x.y * kr[i]; pk.z += x.z * kr[i]; pk.w += x.w * kr[i];
            pq.x += x.x * qr[i]; pq.y += x.y * qr[i]; pq.z += x.z * qr[i]; pq.w += x.w * qr[i];
        }
        // sums over the lanes l ^ 8, l ^ 16, l ^ 32 (DPP and lane swaps, no LDS permutes)
        auto red = [](float x) { return pair_sum32(pair_sum16(x + lane_xor<8>(x))); };
        pk.x = red(pk.x); pk.y = red(pk.y); pk.z = red(pk.z); pk.w = red(pk.w);
        pq.x = red(pq.x); pq.y = red(pq.y); pq.z = red(pq.z); pq.w = red(pq.w);
        if (rr == 0) {
            part[j & 1][hl][w4][0][cg] = pk;
            part[j & 1][hl][w4][1][cg] = pq;
        }
        __syncthreads();
        float4 SK = part[j & 1][hl][0][0][cg], SQ = part[j & 1][hl][0][1][cg];
#pragma unroll
        for (int w = 1; w < 4; w++) {
            const float4 a = part[j & 1][hl][w][0][cg], c = part[j & 1][hl][w][1][cg];
            SK.x += a.x; SK.y += a.y; SK.z += a.z; SK.w += a.w;
            SQ.x += c.x; SQ.y += c.y; SQ.z += c.z; SQ.w += c.w;
        }
        const float* vv = sv[hl] + 32 * j + cg * 4;
        float4 dl;
        dl.x = (vv[0] - decay * SK.x) * bt;
        dl.y = (vv[1] - decay * SK.y) * bt;
        dl.z = (vv[2] - decay * SK.z) * bt;
        dl.w = (vv[3] - decay * SK.w) * bt;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 x = s[j % NSF][i];
            float4 n;
            n.x = decay * x.x + kr[i] * dl.x;
            n.y = decay * x.y + kr[i] * dl.y;
            n.z = decay * x.z + kr[i] * dl.z;
            n.w = decay * x.w + kr[i] * dl.w;
            st_stream(S + (size_t)(rbase + 32 * i) * D + 32 * j + cg * 4, n);
        }
        if (j + NSF < 4) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                s[j % NSF][i] = ld_stream(S + (size_t)(rbase + 32 * i) * D + 32 * (j + NSF) + cg * 4);
        }
        if (w4 == 0 && rr == 0) {
            if constexpr (kStack) {
                float* o = so[hl] + 32 * j + cg * 4;
                o[0] = decay * SQ.x + kq * dl.x;
                o[1] = decay * SQ.y + kq * dl.y;
                o[2] = decay * SQ.z + kq * dl.z;
                o[3] = decay * SQ.w + kq * dl.w;
            } else {
                Tout* o = out + ((size_t)b * HV + hv) * D + 32 * j + cg * 4;
                Act<Tout>::st(o, 0, decay * SQ.x + kq * dl.x);
                Act<Tout>::st(o, 1, decay * SQ.y + kq * dl.y);
                Act<Tout>::st(o, 2, decay * SQ.z + kq * dl.z);
                Act<Tout>::st(o, 3, decay * SQ.w + kq * dl.w);
            }
        }
    }
    if constexpr (kStack) {
        // gated norm of this head's output row by the head's first wave, in gated_norm_bf16's
        // order (lane sums elements lane and lane + 64, then the wave sum)
        __syncthreads();
        if (w4 == 0) {
            const float* o = so[hl];
            float ss = 0.f;
            for (int i = lane; i < D; i += WAVE) ss += o[i] * o[i];
            ss = wave_sum(ss);
            const float r = rsqrtf(ss / (float)D + sg.gnorm_eps);
            const size_t base = ((size_t)b * HV + hv) * D;
            for (int i = lane; i < D; i += WAVE) {
                const float zz = sg.z[base + i];
                Act<Tout>::st(out, base + i, bf2f(sg.gnorm_w[i]) * (o[i] * r) * (zz / (1.f + expf(-zz))));
            }
        }
    }
}

template <int R, typename Tin>
int launch_out(const void* qkv, const uint16_t* w, float* cs, const float* g, const float* beta, float* state,
               void* out, int out_dtype, int B, int HK, int HV, float qscale, float eps, hipStream_t st) {
    dim3 grid(HK, B);
    if (out_dtype == AEGIST_F32)
        delta_decode_kernel<R, Tin, float><<<grid, 256 * R, 0, st>>>((const Tin*)qkv, w, cs, g, beta, state,
                                                                    (float*)out, HK, HV, qscale, eps, StackGates{});
    else if (out_dtype == AEGIST_BF16)
        delta_decode_kernel<R, Tin, uint16_t><<<grid, 256 * R, 0, st>>>((const Tin*)qkv, w, cs, g, beta, state,
                                                                       (uint16_t*)out, HK, HV, qscale, eps,
                                                                       StackGates{});
    else
        return fail(AEGIST_ERR_DTYPE, "delta_decode_step: out dtype must be AEGIST_F32 or AEGIST_BF16");
    return after_launch("delta_decode_step");
}

template <int R>
int launch_in(const void* qkv, int in_dtype, const uint16_t* w, float* cs, const float* g, const float* beta,
              float* state, void* out, int out_dtype, int B, int HK, int HV, float qscale, float eps, hipStream_t st) {
    if (in_dtype == AEGIST_F32)
        return launch_out<R, float>(qkv, w, cs, g, beta, state, out, out_dtype, B, HK, HV, qscale, eps, st);
    if (in_dtype == AEGIST_BF16)
        return launch_out<R, uint16_t>(qkv, w, cs, g, beta, state, out, out_dtype, B, HK, HV, qscale, eps, st);
    return fail(AEGIST_ERR_DTYPE, "delta_decode_step: qkv dtype must be AEGIST_F32 or AEGIST_BF16");
}

}  // namespace

namespace aegist {
// The layer stack's decode step: fp32 qkv projection rows, gates from the b / a projection rows,
// gated norm into the bf16 input of the out projection (ob [B, HV * 128]).
int launch_delta_decode_stack(const float* qkv, const uint16_t* conv_w, float* conv_state, const float* ba,
                              const uint16_t* a_log, const uint16_t* dt_bias, const float* z, const uint16_t* gnorm_w,
                              float gnorm_eps, float* state, uint16_t* ob, int B, int HK, int HV, float qscale,
                              float eps, hipStream_t st) {
    if (B < 0 || HK <= 0 || HV <= 0 || HV % HK) return fail(AEGIST_ERR_SHAPE, "stack decode: need HV % HK == 0");
    if (B == 0) return 0;
    const StackGates sg{ba, a_log, dt_bias, z, gnorm_w, gnorm_eps};
    const dim3 grid(HK, B);
    switch (HV / HK) {
        case 1:
            delta_decode_kernel<1, float, uint16_t, true><<<grid, 256, 0, st>>>(qkv, conv_w, conv_state, nullptr, nullptr,
                                                                                state, ob, HK, HV, qscale, eps, sg);
            break;
        case 2:
            delta_decode_kernel<2, float, uint16_t, true><<<grid, 512, 0, st>>>(qkv, conv_w, conv_state, nullptr, nullptr,
                                                                                state, ob, HK, HV, qscale, eps, sg);
            break;
        case 4:
            delta_decode_kernel<4, float, uint16_t, true><<<grid, 1024, 0, st>>>(qkv, conv_w, conv_state, nullptr,
                                                                                 nullptr, state, ob, HK, HV, qscale, eps,
                                                                                 sg);
            break;
        default: return fail(AEGIST_ERR_SHAPE, "stack decode: HV / HK must be 1, 2 or 4");
    }
    return after_launch("delta_decode_stack");
}

int launch_delta_decode(const void* qkv, int in_dtype, const uint16_t* conv_w, float* conv_state, const float* g,
                        const float* beta, float* state, void* out, int out_dtype, int B, int HK, int HV,
                        float qscale, float eps, hipStream_t st) {
    if (B < 0 || HK <= 0 || HV <= 0 || HV % HK) return fail(AEGIST_ERR_SHAPE, "delta_decode_step: need HV % HK == 0");
    if (B == 0) return 0;
    switch (HV / HK) {
        case 1: return launch_in<1>(qkv, in_dtype, conv_w, conv_state, g, beta, state, out, out_dtype, B, HK, HV, qscale, eps, st);
        case 2: return launch_in<2>(qkv, in_dtype, conv_w, conv_state, g, beta, state, out, out_dtype, B, HK, HV, qscale, eps, st);
        case 4: return launch_in<4>(qkv, in_dtype, conv_w, conv_state, g, beta, state, out, out_dtype, B, HK, HV, qscale, eps, st);
        default: return fail(AEGIST_ERR_SHAPE, "delta_decode_step: HV / HK must be 1, 2 or 4");
    }
}
}  // namespace aegist

extern "C" int aegist_delta_decode_step(const void* qkv, int qkv_dtype, const uint16_t* conv_w, float* conv_state,
                                        const float* g, const float* beta, float* state, void* out, int out_dtype,
                                        int B, int HK, int HV, float qscale, float eps, void* stream) {
    return launch_delta_decode(qkv, qkv_dtype, conv_w, conv_state, g, beta, state, out, out_dtype, B, HK, HV, qscale,
                               eps, AEG_STREAM(stream));
}
