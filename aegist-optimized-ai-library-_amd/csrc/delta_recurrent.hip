// Gated delta rule, token by token (the recurrent form), for short sequences and the
// correctness configuration: S *= e^g; kv = S^T k; delta = (v - kv) beta; S += k delta^T;
// o = S^T q (hybrid.py:318-324 looped; the engine's delta_scan, hybrid.cu:240-300).
//
// The columns of S evolve independently (column j only needs k, q, v_j), so the work is split
// by column block: one wave64 per (sequence, value head, 16-column block) holds 128 x 16 of
// the state in VGPRs (32 rows x 1 column per lane) for the whole sequence. B = 1 with 32
// value heads gives 256 waves instead of the 32 workgroups of a head-per-block scan. Per
// token the wave reduces over rows with two xor shuffles; the next token's q/k/v/g/beta are
// prefetched into registers while the current one is processed.
#include "common.h"

using namespace aegist;

namespace {

constexpr int D = 128;
constexpr int CB = 16;  // columns per wave

struct SeqArgs {
    long long sb_qk, st_qk, sh_qk, sb_v, st_v, sh_v, sb_o, st_o, sh_o;
    long long sb_g, st_g;  // g / beta strides by sequence and token (value head contiguous)
};

template <typename Tin, typename Tout>
__global__ void __launch_bounds__(64) delta_recurrent_kernel(const Tin* __restrict__ q, const Tin* __restrict__ k,
                                                             const Tin* __restrict__ v, const float* __restrict__ g,
                                                             const float* __restrict__ beta, float* __restrict__ state,
                                                             Tout* __restrict__ out, SeqArgs a, int T, int HK, int HV,
                                                             int normalize, float qscale, float eps) {
    __shared__ float sk[D], sq[D];
    const int cb = blockIdx.x, hv = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
    const int c = lane % CB, rg = lane / CB;  // column within block, row group (32 rows)
    const int col = cb * CB + c;
    const int kh = hv / (HV / HK);
    float* S = state ? state + ((size_t)b * HV + hv) * D * D : nullptr;

    float s[32];
#pragma unroll
    for (int r = 0; r < 32; r++) s[r] = S ? S[(size_t)(rg * 32 + r) * D + col] : 0.f;

    const Tin* qb = q + b * a.sb_qk + kh * a.sh_qk;
    const Tin* kb = k + b * a.sb_qk + kh * a.sh_qk;
    const Tin* vb = v + b * a.sb_v + hv * a.sh_v;
    const float* gb = g + b * a.sb_g + hv;
    const float* bb = beta + b * a.sb_g + hv;

    // registers for the token being prefetched
    float nq0 = 0.f, nq1 = 0.f, nk0 = 0.f, nk1 = 0.f, nv = 0.f, ng = 0.f, nb = 0.f;
    auto fetch = [&](int t) {
        nq0 = Act<Tin>::ld(qb, t * a.st_qk + lane);
        nq1 = Act<Tin>::ld(qb, t * a.st_qk + lane + 64);
        nk0 = Act<Tin>::ld(kb, t * a.st_qk + lane);
        nk1 = Act<Tin>::ld(kb, t * a.st_qk + lane + 64);
        nv = Act<Tin>::ld(vb, t * a.st_v + col);
        ng = gb[t * a.st_g];
        nb = bb[t * a.st_g];
    };
    if (T > 0) fetch(0);
    for (int t = 0; t < T; t++) {
        float q0 = nq0, q1 = nq1, k0 = nk0, k1 = nk1, vv = nv, gg = ng, bt = nb;
        if (t + 1 < T) fetch(t + 1);
        if (normalize) {
            const float rq = rsqrtf(wave_sum(q0 * q0 + q1 * q1) + eps);
            const float rk = rsqrtf(wave_sum(k0 * k0 + k1 * k1) + eps);
            q0 = (q0 * rq) * qscale;
            q1 = (q1 * rq) * qscale;
            k0 *= rk;
            k1 *= rk;
        }
        __syncthreads();  // previous token's LDS reads are done
        sq[lane] = q0;
        sq[lane + 64] = q1;
        sk[lane] = k0;
        sk[lane + 64] = k1;
        __syncthreads();
        const float decay = expf(gg);
        float kv = 0.f;
#pragma unroll
        for (int r = 0; r < 32; r++) {
            s[r] *= decay;
            kv += s[r] * sk[rg * 32 + r];
        }
        kv = pair_sum32(pair_sum16(kv));
        const float delta = (vv - kv) * bt;
        float o = 0.f;
#pragma unroll
        for (int r = 0; r < 32; r++) {
            s[r] += sk[rg * 32 + r] * delta;
            o += s[r] * sq[rg * 32 + r];
        }
        o = pair_sum32(pair_sum16(o));
        if (rg == 0) Act<Tout>::st(out, b * a.sb_o + t * a.st_o + hv * a.sh_o + col, o);
    }
    if (S) {
#pragma unroll
        for (int r = 0; r < 32; r++) S[(size_t)(rg * 32 + r) * D + col] = s[r];
    }
}

template <typename Tin, typename Tout>
int launch2(const void* q, const void* k, const void* v, const float* g, const float* beta, float* state, void* out,
            const SeqArgs& a, int B, int T, int HK, int HV, int normalize, float qscale, float eps, hipStream_t st) {
    dim3 grid(D / CB, HV, B);
    delta_recurrent_kernel<Tin, Tout><<<grid, 64, 0, st>>>((const Tin*)q, (const Tin*)k, (const Tin*)v, g, beta, state,
                                                           (Tout*)out, a, T, HK, HV, normalize, qscale, eps);
    return after_launch("delta_recurrent");
}

}  // namespace

namespace aegist {
int launch_delta_recurrent(const void* q, const void* k, const void* v, int in_dtype, long long sb_qk, long long st_qk,
                           long long sh_qk, long long sb_v, long long st_v, long long sh_v, const float* g,
                           const float* beta, float* state, void* out, int out_dtype, long long sb_o, long long st_o,
                           long long sh_o, int B, int T, int HK, int HV, int normalize, float qscale, float eps,
                           hipStream_t st) {
    if (B < 0 || T < 0 || HK <= 0 || HV <= 0 || HV % HK) return fail(AEGIST_ERR_SHAPE, "delta_recurrent: need HV % HK == 0");
    if (B == 0) return 0;
    if (T == 0) return 0;
    SeqArgs a{sb_qk, st_qk, sh_qk, sb_v, st_v, sh_v, sb_o, st_o, sh_o, (long long)T * HV, HV};
    if (in_dtype == AEGIST_F32 && out_dtype == AEGIST_F32)
        return launch2<float, float>(q, k, v, g, beta, state, out, a, B, T, HK, HV, normalize, qscale, eps, st);
    if (in_dtype == AEGIST_F32 && out_dtype == AEGIST_BF16)
        return launch2<float, uint16_t>(q, k, v, g, beta, state, out, a, B, T, HK, HV, normalize, qscale, eps, st);
    if (in_dtype == AEGIST_BF16 && out_dtype == AEGIST_F32)
        return launch2<uint16_t, float>(q, k, v, g, beta, state, out, a, B, T, HK, HV, normalize, qscale, eps, st);
    if (in_dtype == AEGIST_BF16 && out_dtype == AEGIST_BF16)
        return launch2<uint16_t, uint16_t>(q, k, v, g, beta, state, out, a, B, T, HK, HV, normalize, qscale, eps, st);
    return fail(AEGIST_ERR_DTYPE, "delta_recurrent: dtypes must be AEGIST_F32 or AEGIST_BF16");
}
}  // namespace aegist

extern "C" int aegist_delta_recurrent(const void* q, const void* k, const void* v, int in_dtype, long long sb_qk,
                                      long long st_qk, long long sh_qk, long long sb_v, long long st_v, long long sh_v,
                                      const float* g, const float* beta, float* state, void* out, int out_dtype,
                                      long long sb_o, long long st_o, long long sh_o, int B, int T, int HK, int HV,
                                      int normalize, float qscale, float eps, void* stream) {
    return launch_delta_recurrent(q, k, v, in_dtype, sb_qk, st_qk, sh_qk, sb_v, st_v, sh_v, g, beta, state, out,
                                  out_dtype, sb_o, st_o, sh_o, B, T, HK, HV, normalize, qscale, eps,
                                  AEG_STREAM(stream));
}

// Engine mirror: y [T, C] fp32 rows q | k | v (already L2-normalised), gb [T, 2HV] (g, then
// beta), state [HV, 128, 128], o [T, HV, 128]. Sequences of 64+ tokens take the chunked path.
namespace aegist {
size_t delta_scan_chunked_ws_bytes(int T, int HK, int HV);
int delta_scan_chunked(const float* y, const float* gb, float* state, float* o, int T, int C, int HK, int HV,
                       void* ws, size_t ws_bytes,
                       hipStream_t st);
}

extern "C" size_t aegist_delta_scan_workspace_bytes(int T, int HK, int HV) {
    if (T < 64 || HK <= 0 || HV <= 0) return 0;
    return delta_scan_chunked_ws_bytes(T, HK, HV);
}

extern "C" int aegist_delta_scan_ws(const float* y, const float* gb, float* state, float* o, int T, int C, int HK,
                                    int HV, void* ws, size_t ws_bytes, void* stream) {
    if (T < 0 || HK <= 0 || HV <= 0 || HV % HK || C != 2 * HK * D + HV * D)
        return fail(AEGIST_ERR_SHAPE, "delta_scan: need C == 2*HK*128 + HV*128 and HV % HK == 0");
    if (T == 0) return 0;
    hipStream_t st = AEG_STREAM(stream);
    if (T >= 64) {
        int rc = check_workspace(ws, ws_bytes, delta_scan_chunked_ws_bytes(T, HK, HV), "delta_scan");
        if (rc) return rc;
        return delta_scan_chunked(y, gb, state, o, T, C, HK, HV, ws, ws_bytes, st);
    }
    // g and beta are interleaved per token in gb: present them through the strided kernel
    // by pointing g at gb and beta at gb + HV with a token stride of 2*HV.
    SeqArgs a{0, C, D, 0, C, D, 0, (long long)HV * D, D, 0, 2 * HV};
    dim3 grid(D / CB, HV, 1);
    delta_recurrent_kernel<float, float><<<grid, 64, 0, st>>>(y, y + (size_t)HK * D, y + (size_t)2 * HK * D, gb,
                                                              gb + HV, state, o, a, T, HK, HV, 0, 1.f, 0.f);
    return after_launch("delta_scan");
}

// The reference signature (no workspace argument): T >= 64 takes the workspace bound to this
// thread (aegist_bind_workspace).
extern "C" int aegist_delta_scan(const float* y, const float* gb, float* state, float* o, int T, int C, int HK, int HV,
                                 void* stream) {
    size_t bound = 0;
    void* ws = bound_workspace(&bound);
    return aegist_delta_scan_ws(y, gb, state, o, T, C, HK, HV, ws, bound, stream);
}
