// Bandwidth-light ops around the mixer: norms, gates, conv + SiLU, L2-norm, gated norm and
// the attention prep (ZNorm + partial RoPE + bf16 cache append). One wave64 per head or row
// segment, reductions by wave butterflies, no block-wide barriers where a wave suffices.
// Engine-ABI mirrors of aegist_rs/kernels/hybrid.cu (cited per entry point).
#include "common.h"

#include <algorithm>

using namespace aegist;

// ---------------------------------------------------------------------------------------------
// ZNorm: out = (1 + w) * x * rsqrt(mean(x^2) + eps). One block of 256 per row.
// Semantics: hybrid.py:119-130 / hybrid.cu:69-78.
__global__ void __launch_bounds__(256) znorm_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                    float* __restrict__ out, int D, float eps) {
    __shared__ float red[4];
    const float* xr = x + (size_t)blockIdx.x * D;
    float* orow = out + (size_t)blockIdx.x * D;
    float ss = 0.f;
    for (int i = threadIdx.x; i < D; i += 256) ss += xr[i] * xr[i];
    ss = block_sum(ss, red);
    float inv = rsqrtf(ss / (float)D + eps);
    for (int i = threadIdx.x; i < D; i += 256) orow[i] = (xr[i] * inv) * (1.f + bf2f(w[i]));
}

extern "C" int aegist_znorm(const float* x, const uint16_t* w, float* out, int rows, int D, float eps, void* stream) {
    AEG_REQUIRE(rows >= 0 && D > 0, "znorm: rows >= 0 and D > 0 required");
    if (rows == 0) return 0;
    znorm_kernel<<<rows, 256, 0, AEG_STREAM(stream)>>>(x, w, out, D, eps);
    return after_launch("znorm");
}

// ---------------------------------------------------------------------------------------------
// Attention prep. One wave per (token, head): heads [0, H) are queries (read from the first HD
// of each head's 2*HD row of qg), heads [H, H+KV) are keys (k rows) whose values (v rows) are
// copied alongside. HD <= 256 (4 elements per lane); RoPE partners are exchanged through LDS.
struct RopeTable {
    float inv[128];
};

template <typename Tin>
__global__ void __launch_bounds__(256) attn_prep_kernel(
    const Tin* __restrict__ qg, const Tin* __restrict__ k, const Tin* __restrict__ v, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, float* __restrict__ qn, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    int B, int T, int H, int KV, int HD, int RD, int pos0, int cap, float eps, RopeTable rope) {
    __shared__ float buf[4][256];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int item = blockIdx.x * 4 + wave;  // (b, t, head) flattened
    const int heads = H + KV;
    const bool valid = item < B * T * heads;
    const int it = valid ? item : 0;
    const int hh = it % heads, t = (it / heads) % T, b = it / (heads * T);
    const bool isq = hh < H;
    const int h = isq ? hh : hh - H;
    const Tin* src = isq ? qg + (((size_t)b * T + t) * H + h) * 2 * HD : k + (((size_t)b * T + t) * KV + h) * HD;
    const uint16_t* nw = isq ? qw : kw;
    const Tin* vs = v + (((size_t)b * T + t) * KV + (isq ? 0 : h)) * HD;
    // the row, its norm weights and (key heads) the value row are all loaded up front
    float x[4], wn[4], vv[4], ss = 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        int i = lane + r * WAVE;
        x[r] = i < HD ? Act<Tin>::ld(src, i) : 0.f;
        wn[r] = i < HD ? bf2f(nw[i]) : 0.f;
        vv[r] = i < HD && !isq ? Act<Tin>::ld(vs, i) : 0.f;
    }
#pragma unroll
    for (int r = 0; r < 4; r++) ss += x[r] * x[r];
    ss = wave_sum(ss);
    const float inv = rsqrtf(ss / (float)HD + eps);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        int i = lane + r * WAVE;
        x[r] = i < HD ? (x[r] * inv) * (1.f + wn[r]) : 0.f;
        buf[wave][i] = x[r];
    }
    __syncthreads();
    if (!valid) return;
    const int half = RD / 2, pos = pos0 + t;
    float outv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        int i = lane + r * WAVE;
        outv[r] = x[r];
        if (i < RD) {
            int j = i < half ? i : i - half;
            float ang = (float)pos * rope.inv[j];
            float s, c;
            sincosf(ang, &s, &c);
            float rot = i < half ? -buf[wave][i + half] : buf[wave][i - half];
            outv[r] = x[r] * c + rot * s;
        }
    }
    if (isq) {
        float* dst = qn + (((size_t)b * T + t) * H + h) * HD;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            int i = lane + r * WAVE;
            if (i < HD) dst[i] = outv[r];
        }
    } else {
        size_t o = (((size_t)b * KV + h) * cap + pos) * HD;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            int i = lane + r * WAVE;
            if (i < HD) {
                kc[o + i] = f2bf(outv[r]);
                vc[o + i] = f2bf(vv[r]);
            }
        }
    }
}

// 4 consecutive activations as fp32 (one 16-byte load for fp32, one 8-byte load for bf16)
template <typename T> __device__ __forceinline__ void ld4(const T* p, float* o);
template <> __device__ __forceinline__ void ld4<float>(const float* p, float* o) {
    const float4 a = *(const float4*)p;
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
}
template <> __device__ __forceinline__ void ld4<uint16_t>(const uint16_t* p, float* o) {
    const uint2 a = *(const uint2*)p;
    o[0] = bf_lo(a.x); o[1] = bf_hi(a.x); o[2] = bf_lo(a.y); o[3] = bf_hi(a.y);
}

// The same per (token, head) wave with 4 consecutive elements per lane (16-byte loads and
// stores) and the RoPE partner - element e +- RD/2, which sits RD/8 lanes away with the same
// slot - taken by lane shuffle, so there is no LDS exchange or workgroup barrier. For HD a
// multiple of 4 up to 256 and RD a multiple of 8.
template <typename Tin>
__global__ void __launch_bounds__(256) attn_prep_vec_kernel(
    const Tin* __restrict__ qg, const Tin* __restrict__ k, const Tin* __restrict__ v, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, float* __restrict__ qn, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    int B, int T, int H, int KV, int HD, int RD, int pos0, int cap, float eps, RopeTable rope) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int item = blockIdx.x * 4 + wave;  // (b, t, head) flattened
    const int heads = H + KV;
    if (item >= B * T * heads) return;
    const int hh = item % heads, t = (item / heads) % T, b = item / (heads * T);
    const bool isq = hh < H;
    const int h = isq ? hh : hh - H;
    const Tin* src = isq ? qg + (((size_t)b * T + t) * H + h) * 2 * HD : k + (((size_t)b * T + t) * KV + h) * HD;
    const Tin* vs = v + (((size_t)b * T + t) * KV + (isq ? 0 : h)) * HD;
    const uint16_t* nw = isq ? qw : kw;
    const int e0 = 4 * lane;
    const bool act = e0 < HD;
    // the row, its norm weights and (key heads) the value row, all requested up front
    float x[4] = {0.f, 0.f, 0.f, 0.f}, vv[4] = {0.f, 0.f, 0.f, 0.f}, wn[4] = {0.f, 0.f, 0.f, 0.f};
    if (act) {
        ld4<Tin>(src + e0, x);
        const uint2 wp = *(const uint2*)(nw + e0);
        wn[0] = bf_lo(wp.x); wn[1] = bf_hi(wp.x); wn[2] = bf_lo(wp.y); wn[3] = bf_hi(wp.y);
        if (!isq) ld4<Tin>(vs + e0, vv);
    }
    float ss = (x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3]);
    ss = wave_sum(ss);
    const float inv = rsqrtf(ss / (float)HD + eps);
    float y[4];
#pragma unroll
    for (int r = 0; r < 4; r++) y[r] = (x[r] * inv) * (1.f + wn[r]);
    const int half = RD / 2, pos = pos0 + t;
    const int plane = e0 < half ? lane + half / 4 : lane - half / 4;  // partner lane (RoPE dims)
    float outv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float yp = __shfl(y[r], plane < 0 ? 0 : (plane > 63 ? 63 : plane), WAVE);
        const int i = e0 + r;
        outv[r] = y[r];
        if (i < RD) {
            const int j = i < half ? i : i - half;
            float sn, c;
            sincosf((float)pos * rope.inv[j], &sn, &c);
            outv[r] = y[r] * c + (i < half ? -yp : yp) * sn;
        }
    }
    if (!act) return;
    if (isq) {
        *(float4*)(qn + (((size_t)b * T + t) * H + h) * HD + e0) = float4{outv[0], outv[1], outv[2], outv[3]};
    } else {
        const size_t o = (((size_t)b * KV + h) * cap + pos) * HD + e0;
        *(uint2*)(kc + o) = uint2{f2bf2(outv[0], outv[1]), f2bf2(outv[2], outv[3])};
        *(uint2*)(vc + o) = uint2{f2bf2(vv[0], vv[1]), f2bf2(vv[2], vv[3])};
    }
}

namespace aegist {
int make_rope_table(RopeTable* tab, int RD, float theta) {
    if (RD <= 0 || (RD & 1) || RD > 256) return fail(AEGIST_ERR_SHAPE, "rope: rotary dim must be even and in [2, 256]");
    return aegist_rope_inv_freq(tab->inv, RD, theta);
}

// Batched prep used by the engine mirror and by the batched decode entry point.
// qn [B, T, H, HD] fp32 (the engine layout); caches [B, KV, cap, HD].
int launch_attn_prep(const void* qg, const void* k, const void* v, int in_dtype, const uint16_t* qw,
                     const uint16_t* kw, float* qn, uint16_t* kc, uint16_t* vc, int B, int T, int H, int KV, int HD,
                     int RD, int pos0, int cap, float eps, float theta, hipStream_t stream) {
    if (HD <= 0 || HD > 256 || RD > HD) return fail(AEGIST_ERR_SHAPE, "attn_prep: need 0 < HD <= 256 and RD <= HD");
    if (pos0 < 0 || pos0 + T > cap) return fail(AEGIST_ERR_SHAPE, "attn_prep: positions exceed the cache capacity");
    RopeTable tab;
    int rc = make_rope_table(&tab, RD, theta);
    if (rc) return rc;
    int items = B * T * (H + KV);
    if (items == 0) return 0;
    dim3 grid((items + 3) / 4);
    // 16-byte (fp32) or 8-byte (bf16) element runs: every row start and the bases aligned so
    const size_t es = in_dtype == AEGIST_F32 ? 4 : 2;
    const bool vec = HD % 4 == 0 && RD % 8 == 0 && (uintptr_t)qg % (4 * es) == 0 && (uintptr_t)k % (4 * es) == 0 &&
                     (uintptr_t)v % (4 * es) == 0 && (uintptr_t)qn % 16 == 0 && (uintptr_t)kc % 8 == 0 &&
                     (uintptr_t)vc % 8 == 0 && (uintptr_t)qw % 8 == 0 && (uintptr_t)kw % 8 == 0;
    if (vec && in_dtype == AEGIST_F32) {
        attn_prep_vec_kernel<float><<<grid, 256, 0, stream>>>((const float*)qg, (const float*)k, (const float*)v, qw, kw,
                                                              qn, kc, vc, B, T, H, KV, HD, RD, pos0, cap, eps, tab);
        return after_launch("attn_prep");
    }
    if (vec && in_dtype == AEGIST_BF16) {
        attn_prep_vec_kernel<uint16_t><<<grid, 256, 0, stream>>>((const uint16_t*)qg, (const uint16_t*)k,
                                                                 (const uint16_t*)v, qw, kw, qn, kc, vc, B, T, H, KV,
                                                                 HD, RD, pos0, cap, eps, tab);
        return after_launch("attn_prep");
    }
    if (in_dtype == AEGIST_F32)
        attn_prep_kernel<float><<<grid, 256, 0, stream>>>((const float*)qg, (const float*)k, (const float*)v, qw, kw, qn,
                                                          kc, vc, B, T, H, KV, HD, RD, pos0, cap, eps, tab);
    else if (in_dtype == AEGIST_BF16)
        attn_prep_kernel<uint16_t><<<grid, 256, 0, stream>>>((const uint16_t*)qg, (const uint16_t*)k,
                                                             (const uint16_t*)v, qw, kw, qn, kc, vc, B, T, H, KV, HD,
                                                             RD, pos0, cap, eps, tab);
    else
        return fail(AEGIST_ERR_DTYPE, "attn_prep: dtype must be AEGIST_F32 or AEGIST_BF16");
    return after_launch("attn_prep");
}
}  // namespace aegist

extern "C" int aegist_attn_prep(const float* qg, const float* k, const float* v, const uint16_t* qw, const uint16_t* kw,
                                float* qn, uint16_t* kc, uint16_t* vc, int T, int H, int KV, int HD, int RD, int pos0,
                                int cap, float eps, float theta, void* stream) {
    return launch_attn_prep(qg, k, v, AEGIST_F32, qw, kw, qn, kc, vc, 1, T, H, KV, HD, RD, pos0, cap, eps, theta,
                            AEG_STREAM(stream));
}

// ---------------------------------------------------------------------------------------------
// DeltaNet gates: one wave per (token, output j); j < HV -> beta_j, else g_{j-HV}.
// gb [T, 2HV]: g first, then beta (hybrid.cu:179-200; hybrid.py:403-404, softplus threshold 20).
__global__ void __launch_bounds__(256) delta_gates_kernel(const float* __restrict__ h, const uint16_t* __restrict__ wb,
                                                          const uint16_t* __restrict__ wa,
                                                          const uint16_t* __restrict__ a_log,
                                                          const uint16_t* __restrict__ dt_bias, float* __restrict__ gb,
                                                          int T, int D, int HV) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int item = blockIdx.x * 4 + wave;
    if (item >= T * 2 * HV) return;
    const int t = item / (2 * HV), j = item % (2 * HV);
    const float* hr = h + (size_t)t * D;
    const uint16_t* wr = j < HV ? wb + (size_t)j * D : wa + (size_t)(j - HV) * D;
    float acc = 0.f;
    for (int i = lane; i < D; i += WAVE) acc += hr[i] * bf2f(wr[i]);
    acc = wave_sum(acc);
    if (lane == 0) {
        if (j < HV) {
            gb[(size_t)t * 2 * HV + HV + j] = 1.f / (1.f + expf(-acc));
        } else {
            int jj = j - HV;
            float xx = acc + bf2f(dt_bias[jj]);
            float sp = xx > 20.f ? xx : log1pf(expf(xx));
            gb[(size_t)t * 2 * HV + jj] = -expf(bf2f(a_log[jj])) * sp;
        }
    }
}

extern "C" int aegist_delta_gates(const float* h, const uint16_t* wb, const uint16_t* wa, const uint16_t* a_log,
                                  const uint16_t* dt_bias, float* gb, int T, int D, int HV, void* stream) {
    AEG_REQUIRE(T >= 0 && D > 0 && HV > 0, "delta_gates: bad shape");
    if (T == 0) return 0;
    int items = T * 2 * HV;
    delta_gates_kernel<<<(items + 3) / 4, 256, 0, AEG_STREAM(stream)>>>(h, wb, wa, a_log, dt_bias, gb, T, D, HV);
    return after_launch("delta_gates");
}

// ---------------------------------------------------------------------------------------------
// Depthwise causal conv (kernel 4) + SiLU over T rows, continuing from state [C,3] (oldest
// first). One block owns 64 channels for the whole sequence, so the in-place state update is
// ordered after every read of the old state by the block barrier. Threads: 64 channels x 4
// token lanes. (hybrid.cu:205-221; hybrid.py:390-398.)
__global__ void __launch_bounds__(256) conv_silu_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                        const uint16_t* __restrict__ w, float* __restrict__ state,
                                                        int T, int C) {
    const int c = blockIdx.x * 64 + (threadIdx.x % 64), tl = threadIdx.x / 64;
    const bool ok = c < C;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, w0 = 0.f, w1 = 0.f, w2 = 0.f, w3 = 0.f;
    if (ok) {
        s0 = state[(size_t)c * 3];
        s1 = state[(size_t)c * 3 + 1];
        s2 = state[(size_t)c * 3 + 2];
        w0 = bf2f(w[(size_t)c * 4]);
        w1 = bf2f(w[(size_t)c * 4 + 1]);
        w2 = bf2f(w[(size_t)c * 4 + 2]);
        w3 = bf2f(w[(size_t)c * 4 + 3]);
        for (int t = tl; t < T; t += 4) {
            float xm3 = t >= 3 ? x[(size_t)(t - 3) * C + c] : (t == 0 ? s0 : (t == 1 ? s1 : s2));
            float xm2 = t >= 2 ? x[(size_t)(t - 2) * C + c] : (t == 0 ? s1 : s2);
            float xm1 = t >= 1 ? x[(size_t)(t - 1) * C + c] : s2;
            float x0 = x[(size_t)t * C + c];
            y[(size_t)t * C + c] = conv4_silu(w0, w1, w2, w3, xm3, xm2, xm1, x0);
        }
    }
    __syncthreads();
    if (ok && tl == 0) {
        // new state = last three of [s0, s1, s2, x_0 .. x_{T-1}]
        float h0 = T >= 3 ? x[(size_t)(T - 3) * C + c] : (T == 2 ? s2 : (T == 1 ? s1 : s0));
        float h1 = T >= 2 ? x[(size_t)(T - 2) * C + c] : (T == 1 ? s2 : s1);
        float h2 = T >= 1 ? x[(size_t)(T - 1) * C + c] : s2;
        state[(size_t)c * 3] = h0;
        state[(size_t)c * 3 + 1] = h1;
        state[(size_t)c * 3 + 2] = h2;
    }
}

namespace aegist {
int launch_conv_silu_batched(const float* x, float* y, const uint16_t* w, float* state, int B, int T, int C,
                             hipStream_t st);
}
extern "C" int aegist_conv_silu(const float* x, float* y, const uint16_t* w, float* state, int T, int C, void* stream) {
    AEG_REQUIRE(T >= 0 && C > 0, "conv_silu: bad shape");
    if (T == 0) return 0;
    if (C % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 && (uintptr_t)w % 8 == 0)
        return launch_conv_silu_batched(x, y, w, state, 1, T, C, AEG_STREAM(stream));
    conv_silu_kernel<<<(C + 63) / 64, 256, 0, AEG_STREAM(stream)>>>(x, y, w, state, T, C);
    return after_launch("conv_silu");
}

// ---------------------------------------------------------------------------------------------
// L2-norm of the first 2*nq heads of each row (queries scaled by qscale). One wave per
// (row, head). (hybrid.cu:225-232; hybrid.py:314-315, 408-410.)
__global__ void __launch_bounds__(256) l2norm_heads_kernel(float* __restrict__ y, int T, int C, int nq, int dk,
                                                           float qscale, float eps) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int item = blockIdx.x * 4 + wave;
    if (item >= T * 2 * nq) return;
    const int t = item / (2 * nq), hh = item % (2 * nq);
    float* p = y + (size_t)t * C + (size_t)hh * dk;
    float ss = 0.f;
    for (int i = lane; i < dk; i += WAVE) ss += p[i] * p[i];
    ss = wave_sum(ss);
    const float r = rsqrtf(ss + eps), s = hh < nq ? qscale : 1.f;
    for (int i = lane; i < dk; i += WAVE) p[i] = (p[i] * r) * s;
}

extern "C" int aegist_l2norm_heads(float* y, int T, int C, int nq, int dk, float qscale, float eps, void* stream) {
    AEG_REQUIRE(T >= 0 && nq > 0 && dk > 0 && 2 * nq * dk <= C, "l2norm_heads: bad shape");
    if (T == 0) return 0;
    int items = T * 2 * nq;
    l2norm_heads_kernel<<<(items + 3) / 4, 256, 0, AEG_STREAM(stream)>>>(y, T, C, nq, dk, qscale, eps);
    return after_launch("l2norm_heads");
}

// ---------------------------------------------------------------------------------------------
// Gated norm: out = w * rmsnorm(o) * silu(z) per value head; one wave per (row, head).
// (hybrid.cu:303-311; hybrid.py:133-147 with act = silu.)
__global__ void __launch_bounds__(256) gated_norm_kernel(const float* __restrict__ o, const float* __restrict__ z,
                                                         const uint16_t* __restrict__ w, float* __restrict__ out,
                                                         int rows, int DV, float eps) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int item = blockIdx.x * 4 + wave;
    if (item >= rows) return;
    const size_t base = (size_t)item * DV;
    float ss = 0.f;
    for (int i = lane; i < DV; i += WAVE) ss += o[base + i] * o[base + i];
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / (float)DV + eps);
    for (int i = lane; i < DV; i += WAVE) {
        float zz = z[base + i];
        out[base + i] = bf2f(w[i]) * (o[base + i] * r) * (zz / (1.f + expf(-zz)));
    }
}

extern "C" int aegist_gated_norm(const float* o, const float* z, const uint16_t* w, float* out, int T, int HV, int DV,
                                 float eps, void* stream) {
    AEG_REQUIRE(T >= 0 && HV > 0 && DV > 0, "gated_norm: bad shape");
    int rows = T * HV;
    if (rows == 0) return 0;
    gated_norm_kernel<<<(rows + 3) / 4, 256, 0, AEG_STREAM(stream)>>>(o, z, w, out, rows, DV, eps);
    return after_launch("gated_norm");
}

// ---------------------------------------------------------------------------------------------
// Helpers for the layer stack (batched rows, bf16 outputs feeding the projection GEMMs).
namespace {

// ZNorm of `rows` rows of D into bf16 (the GEMM input of the mixer projections).
__global__ void __launch_bounds__(256) znorm_bf16_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                         uint16_t* __restrict__ out, int D, float eps) {
    __shared__ float red[4];
    const float* xr = x + (size_t)blockIdx.x * D;
    float ss = 0.f;
    for (int i = threadIdx.x; i < D; i += 256) ss += xr[i] * xr[i];
    ss = block_sum(ss, red);
    const float inv = rsqrtf(ss / (float)D + eps);
    for (int i = threadIdx.x; i < D; i += 256) out[(size_t)blockIdx.x * D + i] = f2bf((xr[i] * inv) * (1.f + bf2f(w[i])));
}

// Row-resident ZNorm into bf16 for D % 1024 == 0, D <= 8192: each thread holds its D / 1024
// 16-byte pieces of the row in registers (one read of x), block sum, 8-byte bf16 stores.
template <int NV>
__global__ void __launch_bounds__(256) znorm_bf16_vec_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                             uint16_t* __restrict__ out, int D, float eps) {
    __shared__ float red[4];
    const float4* xr = (const float4*)(x + (size_t)blockIdx.x * D);
    const uint2* wr = (const uint2*)w;
    float4 v[NV];
    uint2 wp[NV];  // the norm weights are loaded with x, ahead of the block sum
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        v[i] = xr[threadIdx.x + 256 * i];
        wp[i] = wr[threadIdx.x + 256 * i];
    }
#pragma unroll
    for (int i = 0; i < NV; i++) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    ss = block_sum(ss, red);
    const float inv = rsqrtf(ss / (float)D + eps);
    uint2* orow = (uint2*)(out + (size_t)blockIdx.x * D);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int e = threadIdx.x + 256 * i;
        orow[e] = uint2{f2bf2((v[i].x * inv) * (1.f + bf_lo(wp[i].x)), (v[i].y * inv) * (1.f + bf_hi(wp[i].x))),
                        f2bf2((v[i].z * inv) * (1.f + bf_lo(wp[i].y)), (v[i].w * inv) * (1.f + bf_hi(wp[i].y)))};
    }
}

// ZNorm of x + sum_s part[s] (the split-K slices of the previous out projection, added in
// order s = 0, 1, ...): the sum is written back to x (the residual) and normed into bf16.
template <int NV>
__global__ void __launch_bounds__(256) znorm_bf16_acc_vec_kernel(float* __restrict__ x, const float* __restrict__ part,
                                                                 int nks, size_t slice, const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ out, int D, float eps) {
    __shared__ float red[4];
    float4* xr = (float4*)(x + (size_t)blockIdx.x * D);
    const uint2* wr = (const uint2*)w;
    // every load is issued before the first use: the norm weights (needed only after the block
    // sum), x and the first four slices (clamped indices past nks, masked out of the sum)
    uint2 wp[NV];
    float4 a[NV], ps[4][NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int e = threadIdx.x + 256 * i;
        if (out) wp[i] = wr[e];
        a[i] = xr[e];
#pragma unroll
        for (int s = 0; s < 4; s++)
            ps[s][i] = ((const float4*)(part + (size_t)(s < nks ? s : 0) * slice + (size_t)blockIdx.x * D))[e];
    }
    float4 v[NV];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int e = threadIdx.x + 256 * i;
        // slices added in order s = 0, 1, ...
        float4 p = ps[0][i];
#pragma unroll
        for (int s = 1; s < 4; s++)
            if (s < nks) {
                p.x += ps[s][i].x; p.y += ps[s][i].y; p.z += ps[s][i].z; p.w += ps[s][i].w;
            }
        for (int s = 4; s < nks; s++) {
            const float4 q = ((const float4*)(part + s * slice + (size_t)blockIdx.x * D))[e];
            p.x += q.x; p.y += q.y; p.z += q.z; p.w += q.w;
        }
        float4 y = a[i];
        y.x += p.x; y.y += p.y; y.z += p.z; y.w += p.w;
        xr[e] = y;
        v[i] = y;
        ss += y.x * y.x + y.y * y.y + y.z * y.z + y.w * y.w;
    }
    ss = block_sum(ss, red);
    const float inv = rsqrtf(ss / (float)D + eps);
    if (!out) return;
    uint2* orow = (uint2*)(out + (size_t)blockIdx.x * D);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int e = threadIdx.x + 256 * i;
        orow[e] = uint2{f2bf2((v[i].x * inv) * (1.f + bf_lo(wp[i].x)), (v[i].y * inv) * (1.f + bf_hi(wp[i].x))),
                        f2bf2((v[i].z * inv) * (1.f + bf_lo(wp[i].y)), (v[i].w * inv) * (1.f + bf_hi(wp[i].y)))};
    }
}

// Gated norm into bf16 for DV % 128 == 0: half a wave (32 lanes, 16-byte loads) per (row, head).
__global__ void __launch_bounds__(256) gated_norm_bf16_vec_kernel(const float* __restrict__ o,
                                                                  const float* __restrict__ z,
                                                                  const uint16_t* __restrict__ w,
                                                                  uint16_t* __restrict__ out, int rows, int DV,
                                                                  float eps) {
    const int item = blockIdx.x * 8 + threadIdx.x / 32, l32 = threadIdx.x % 32;
    const bool ok = item < rows;
    const size_t base = (size_t)(ok ? item : 0) * DV;
    float ss = 0.f;
    for (int i = 4 * l32; i < DV; i += 128) {
        const float4 a = *(const float4*)(o + base + i);
        ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
#pragma unroll
    for (int m = 16; m > 0; m >>= 1) ss += __shfl_xor(ss, m, WAVE);
    if (!ok) return;
    const float r = rsqrtf(ss / (float)DV + eps);
    for (int i = 4 * l32; i < DV; i += 128) {
        const float4 a = *(const float4*)(o + base + i);
        const float4 zz = *(const float4*)(z + base + i);
        const uint2 wp = *(const uint2*)(w + i);
        auto gate = [](float v) { return v / (1.f + expf(-v)); };
        *(uint2*)(out + base + i) =
            uint2{f2bf2(bf_lo(wp.x) * (a.x * r) * gate(zz.x), bf_hi(wp.x) * (a.y * r) * gate(zz.y)),
                  f2bf2(bf_lo(wp.y) * (a.z * r) * gate(zz.z), bf_hi(wp.y) * (a.w * r) * gate(zz.w))};
    }
}

__global__ void cast_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        y[i] = f2bf(x[i]);
}

// beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias) from projected rows ba [rows, 2HV]
// (b in columns [0, HV), a in [HV, 2HV)). g, beta [rows, HV].
__global__ void gates_from_proj_kernel(const float* __restrict__ ba, const uint16_t* __restrict__ a_log,
                                       const uint16_t* __restrict__ dt_bias, float* __restrict__ g,
                                       float* __restrict__ beta, int rows, int HV) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * HV) return;
    const int r = i / HV, j = i % HV;
    const float bb = ba[(size_t)r * 2 * HV + j], aa = ba[(size_t)r * 2 * HV + HV + j];
    beta[i] = 1.f / (1.f + expf(-bb));
    const float xx = aa + bf2f(dt_bias[j]);
    const float sp = xx > 20.f ? xx : log1pf(expf(xx));
    g[i] = -expf(bf2f(a_log[j])) * sp;
}

// Gated norm into bf16: out = w * rmsnorm(o) * silu(z), one wave per (row, head).
__global__ void __launch_bounds__(256) gated_norm_bf16_kernel(const float* __restrict__ o, const float* __restrict__ z,
                                                              const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                                              int rows, int DV, float eps) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int item = blockIdx.x * 4 + wave;
    if (item >= rows) return;
    const size_t base = (size_t)item * DV;
    float ss = 0.f;
    for (int i = lane; i < DV; i += WAVE) ss += o[base + i] * o[base + i];
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / (float)DV + eps);
    for (int i = lane; i < DV; i += WAVE) {
        const float zz = z[base + i];
        out[base + i] = f2bf(bf2f(w[i]) * (o[base + i] * r) * (zz / (1.f + expf(-zz))));
    }
}

// Batched conv + SiLU: x, y [B, T, C]; state [B, C, 3]; grid (ceil(C/64), B).
__global__ void __launch_bounds__(256) conv_silu_batched_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                const uint16_t* __restrict__ w,
                                                                float* __restrict__ state, int T, int C) {
    const int b = blockIdx.y;
    x += (size_t)b * T * C;
    y += (size_t)b * T * C;
    state += (size_t)b * C * 3;
    const int c = blockIdx.x * 64 + (threadIdx.x % 64), tl = threadIdx.x / 64;
    const bool ok = c < C;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f;
    if (ok) {
        s0 = state[(size_t)c * 3];
        s1 = state[(size_t)c * 3 + 1];
        s2 = state[(size_t)c * 3 + 2];
        const float w0 = bf2f(w[(size_t)c * 4]), w1 = bf2f(w[(size_t)c * 4 + 1]), w2 = bf2f(w[(size_t)c * 4 + 2]),
                    w3 = bf2f(w[(size_t)c * 4 + 3]);
        for (int t = tl; t < T; t += 4) {
            const float xm3 = t >= 3 ? x[(size_t)(t - 3) * C + c] : (t == 0 ? s0 : (t == 1 ? s1 : s2));
            const float xm2 = t >= 2 ? x[(size_t)(t - 2) * C + c] : (t == 0 ? s1 : s2);
            const float xm1 = t >= 1 ? x[(size_t)(t - 1) * C + c] : s2;
            y[(size_t)t * C + c] = conv4_silu(w0, w1, w2, w3, xm3, xm2, xm1, x[(size_t)t * C + c]);
        }
    }
    __syncthreads();
    if (ok && tl == 0) {
        const float h0 = T >= 3 ? x[(size_t)(T - 3) * C + c] : (T == 2 ? s2 : (T == 1 ? s1 : s0));
        const float h1 = T >= 2 ? x[(size_t)(T - 2) * C + c] : (T == 1 ? s2 : s1);
        const float h2 = T >= 1 ? x[(size_t)(T - 1) * C + c] : s2;
        state[(size_t)c * 3] = h0;
        state[(size_t)c * 3 + 1] = h1;
        state[(size_t)c * 3 + 2] = h2;
    }
}

// Batched conv + SiLU over token chunks, for C % 4 == 0 and 16-byte rows: x, y [B, T, C];
// state [B, C, 3] (oldest first). Each thread owns 4 channels x kConvTT consecutive tokens and
// keeps the last 3 inputs in registers, so every input is loaded once (plus a 3-token halo per
// thread) and a wave moves 1 KB per load and store instruction; the earlier layout (one channel
// per thread over every 4th token) loaded each input 4 times. The state is only read here (the
// inputs before token 0); conv_state_tail_kernel replaces it afterwards, in a second launch, since
// the chunk that reads the old state and the one that sees the last inputs are different
// workgroups.
constexpr int kConvTT = 16;
__global__ void __launch_bounds__(256) conv_silu_chunk_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                              const uint16_t* __restrict__ w,
                                                              const float* __restrict__ state, int T, int C) {
    const int b = blockIdx.z, c = (blockIdx.x * 64 + threadIdx.x % 64) * 4;
    const int t0 = (blockIdx.y * 4 + threadIdx.x / 64) * kConvTT;
    if (c >= C || t0 >= T) return;
    x += (size_t)b * T * C;
    y += (size_t)b * T * C;
    state += (size_t)b * C * 3;
    float wt[4][4];  // [channel][tap], tap 3 multiplies the newest input
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint2 wp = *(const uint2*)(w + (size_t)(c + e) * 4);
        wt[e][0] = bf_lo(wp.x);
        wt[e][1] = bf_hi(wp.x);
        wt[e][2] = bf_lo(wp.y);
        wt[e][3] = bf_hi(wp.y);
    }
    auto input = [&](int t) -> f32x4 {  // x[t] for t >= 0, the state's inputs for t in [-3, 0)
        if (t >= 0) return *(const f32x4*)(x + (size_t)t * C + c);
        f32x4 r;
#pragma unroll
        for (int e = 0; e < 4; e++) r[e] = state[(size_t)(c + e) * 3 + 3 + t];
        return r;
    };
    f32x4 h0 = input(t0 - 3), h1 = input(t0 - 2), h2 = input(t0 - 1);
    f32x4 xin[kConvTT];
#pragma unroll
    for (int i = 0; i < kConvTT; i++)
        xin[i] = t0 + i < T ? *(const f32x4*)(x + (size_t)(t0 + i) * C + c) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kConvTT; i++) {
        if (t0 + i < T) {
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; e++)
                o[e] = conv4_silu(wt[e][0], wt[e][1], wt[e][2], wt[e][3], h0[e], h1[e], h2[e], xin[i][e]);
            *(f32x4*)(y + (size_t)(t0 + i) * C + c) = o;
        }
        h0 = h1;
        h1 = h2;
        h2 = xin[i];
    }
}

// The conv state after a T-token feed: the last 3 inputs, taking the old state where T < 3.
__global__ void conv_state_tail_kernel(const float* __restrict__ x, float* __restrict__ state, int T, int C) {
    const int b = blockIdx.y, c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    x += (size_t)b * T * C;
    float* st = state + ((size_t)b * C + c) * 3;
    const float s1 = st[1], s2 = st[2];
    const float n0 = T >= 3 ? x[(size_t)(T - 3) * C + c] : (T == 2 ? s2 : s1);
    const float n1 = T >= 2 ? x[(size_t)(T - 2) * C + c] : s2;
    const float n2 = x[(size_t)(T - 1) * C + c];
    st[0] = n0;
    st[1] = n1;
    st[2] = n2;
}

// Embedding rows: out[i] = fp32(table[ids[i]]), D per row.
__global__ void embed_bf16_kernel(const uint16_t* __restrict__ table, const int* __restrict__ ids,
                                  float* __restrict__ out, int n, int D) {
    const int r = blockIdx.x;
    if (r >= n) return;
    const uint16_t* src = table + (size_t)ids[r] * D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) out[(size_t)r * D + i] = bf2f(src[i]);
}

}  // namespace

namespace aegist {
int launch_znorm_bf16(const float* x, const uint16_t* w, uint16_t* out, int rows, int D, float eps, hipStream_t st) {
    if (rows <= 0) return 0;
    const bool vec = D % 1024 == 0 && D <= 8192 && (uintptr_t)x % 16 == 0 && (uintptr_t)out % 8 == 0 &&
                     (uintptr_t)w % 8 == 0;
    switch (vec ? D / 1024 : 0) {
        case 1: znorm_bf16_vec_kernel<1><<<rows, 256, 0, st>>>(x, w, out, D, eps); break;
        case 2: znorm_bf16_vec_kernel<2><<<rows, 256, 0, st>>>(x, w, out, D, eps); break;
        case 4: znorm_bf16_vec_kernel<4><<<rows, 256, 0, st>>>(x, w, out, D, eps); break;
        case 8: znorm_bf16_vec_kernel<8><<<rows, 256, 0, st>>>(x, w, out, D, eps); break;
        default: znorm_bf16_kernel<<<rows, 256, 0, st>>>(x, w, out, D, eps);
    }
    return after_launch("znorm_bf16");
}
// x += sum of the split-K slices (in order), then ZNorm into out (out == nullptr: the sum only).
// Needs D % 1024 == 0, D <= 8192 and 16-byte aligned rows.
int launch_znorm_bf16_acc(float* x, const float* part, int nks, const uint16_t* w, uint16_t* out, int rows, int D,
                          float eps, hipStream_t st) {
    if (rows <= 0) return 0;
    if (D % 1024 || D > 8192 || (uintptr_t)x % 16 || (uintptr_t)part % 16)
        return fail(AEGIST_ERR_SHAPE, "znorm_acc: need D % 1024 == 0, D <= 8192, aligned rows");
    const size_t slice = (size_t)rows * D;
    switch (D / 1024) {
        case 1: znorm_bf16_acc_vec_kernel<1><<<rows, 256, 0, st>>>(x, part, nks, slice, w, out, D, eps); break;
        case 2: znorm_bf16_acc_vec_kernel<2><<<rows, 256, 0, st>>>(x, part, nks, slice, w, out, D, eps); break;
        case 4: znorm_bf16_acc_vec_kernel<4><<<rows, 256, 0, st>>>(x, part, nks, slice, w, out, D, eps); break;
        case 8: znorm_bf16_acc_vec_kernel<8><<<rows, 256, 0, st>>>(x, part, nks, slice, w, out, D, eps); break;
        default: return fail(AEGIST_ERR_SHAPE, "znorm_acc: D / 1024 must be 1, 2, 4 or 8");
    }
    return after_launch("znorm_bf16_acc");
}
int launch_cast_bf16(const float* x, uint16_t* y, size_t n, hipStream_t st) {
    if (n == 0) return 0;
    unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 16384);
    cast_bf16_kernel<<<blocks, 256, 0, st>>>(x, y, n);
    return after_launch("cast_bf16");
}
int launch_gates_from_proj(const float* ba, const uint16_t* a_log, const uint16_t* dt_bias, float* g, float* beta,
                           int rows, int HV, hipStream_t st) {
    if (rows <= 0) return 0;
    gates_from_proj_kernel<<<(rows * HV + 255) / 256, 256, 0, st>>>(ba, a_log, dt_bias, g, beta, rows, HV);
    return after_launch("gates_from_proj");
}
int launch_gated_norm_bf16(const float* o, const float* z, const uint16_t* w, uint16_t* out, int rows, int DV,
                           float eps, hipStream_t st) {
    if (rows <= 0) return 0;
    if (DV % 128 == 0 && (uintptr_t)o % 16 == 0 && (uintptr_t)z % 16 == 0 && (uintptr_t)out % 8 == 0 &&
        (uintptr_t)w % 8 == 0)
        gated_norm_bf16_vec_kernel<<<(rows + 7) / 8, 256, 0, st>>>(o, z, w, out, rows, DV, eps);
    else
        gated_norm_bf16_kernel<<<(rows + 3) / 4, 256, 0, st>>>(o, z, w, out, rows, DV, eps);
    return after_launch("gated_norm_bf16");
}
int launch_conv_silu_batched(const float* x, float* y, const uint16_t* w, float* state, int B, int T, int C,
                             hipStream_t st) {
    if (B <= 0 || T <= 0) return 0;
    if (C % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 && (uintptr_t)w % 8 == 0) {
        conv_silu_chunk_kernel<<<dim3((C / 4 + 63) / 64, (T + 4 * kConvTT - 1) / (4 * kConvTT), B), 256, 0, st>>>(
            x, y, w, state, T, C);
        int rc = after_launch("conv_silu_chunk");
        if (rc) return rc;
        conv_state_tail_kernel<<<dim3((C + 255) / 256, B), 256, 0, st>>>(x, state, T, C);
        return after_launch("conv_state_tail");
    }
    conv_silu_batched_kernel<<<dim3((C + 63) / 64, B), 256, 0, st>>>(x, y, w, state, T, C);
    return after_launch("conv_silu_batched");
}
int launch_embed_bf16(const uint16_t* table, const int* ids, float* out, int n, int D, hipStream_t st) {
    if (n <= 0) return 0;
    embed_bf16_kernel<<<n, 256, 0, st>>>(table, ids, out, n, D);
    return after_launch("embed_bf16");
}
}  // namespace aegist
