// Chunked (C = 64) WY-form prefill of the gated delta rule on gfx950 MFMA.
//
// Per chunk with cum = cumsum(g) and the L2-normalised rows q_n, k_n (hybrid.py:327-361):
//   A     = strict_lower( beta_i e^{cum_i - cum_j} k_n,i . k_n,j )
//   u     = (I + A)^-1 (beta v),   w = (I + A)^-1 (beta e^{cum} k_n)
//   intra = lower_incl( e^{cum_i - cum_j} q_n,i . k_n,j )
//   v_new = u - w S;  o = e^{cum} (q_n S) + intra v_new;  S = e^{cum_last} S + k_n^T (e^{cum_last - cum} v_new)
//
// Two kernels per segment of up to SEG tokens (a segment's workspace stays resident in the
// MALL between the two launches). With more than one segment the workspace holds two segment
// buffers, and K2 of segment s and K1 of segment s+1 run as one grid (delta_chunk_fused) on the
// caller's stream: K2's few long-lived workgroups keep part of each CU busy, K1's fill the rest.
//  K1 delta_chunk_intra: one workgroup per (sequence, value head, chunk), fully parallel.
//     Normalises q, k in fp32 and keeps them as fp16 in LDS; k_n k_n^T and q_n k_n^T on
//     v_mfma_f32_16x16x32_f16 (lower-triangular blocks only); decay and beta applied in fp32 on
//     the accumulators; the inverses of the four 16 x 16 diagonal blocks of I + A by forward
//     substitution, then u and w by blocked forward substitution over the 256 right-hand-side
//     columns (beta v | beta e^cum k_n), each wave owning 64 columns of every row (no barrier).
//     Writes u (fp32), w (fp16), intra (fp16 hi + lo), cum, and - once per QK head - q_n and
//     k_n^T (fp16).
//  K2 delta_chunk_state: one workgroup per (sequence, value head, 32-column slice of S); the
//     columns of S are independent, so 4 slices per head run in parallel, the slices of one
//     head on one XCD (they share its L2 for the chunk operands). S lives in MFMA
//     accumulator registers (fp32) for the whole segment; each chunk it is copied to LDS as
//     fp16 (transposed, so the B operand is a 16-byte read), then w S and q_n S, intra v_new,
//     and the rank-64 state update k_n^T v' run on MFMA.
// Operands are fp16 (11-bit mantissa) rather than bf16, and the products that set the output's
// accuracy carry a low fp16 part (hi hi + hi lo + lo hi, ~22 bits): the Gram products run on the
// raw q / k rows (exact in fp16 for bf16 inputs) with the norms, beta and every decay applied in
// fp32 afterwards, and intra v_new is split on both sides. At config-4 data (T = 2048, 32 heads)
// o is within ~2e-4 of fp64; fp16-only intra v_new gives 6e-4, bf16 operands 4e-3.
#include "common.h"


#include <algorithm>

using namespace aegist;

namespace {

constexpr int D = 128;
constexpr int CH = 64;       // chunk length
constexpr int SEG = 2048;    // tokens per segment (workspace granularity)
#ifndef K2_NCT
#define K2_NCT 2              // 16-column tiles per K2 workgroup (4 workgroups per value head)
#endif
constexpr int QK_LD = D + 8; // fp16 row stride (elements) of the q/k tiles in LDS
constexpr int A_LD = 68;     // fp32 row stride of the A matrix in LDS (16-byte aligned rows)

typedef _Float16 half_t;
typedef short short4v_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
// raw buffer resource for the output stores: range (bytes) and the gfx9 word 3 (32-bit data,
// no swizzle); kOutDrop lies past the range, so a store at that offset is discarded
constexpr int kOutRange = 0x40000000;
constexpr int kOutDrop = 0x7ffffff0;
constexpr int kBufWord3 = 0x00020000;
constexpr int kFusedLdsPad = 2048;  // dynamic LDS bytes added to the fused launch (occupancy cap)

struct SeqLayout {
    long long sb_qk, st_qk, sh_qk, sb_v, st_v, sh_v, sb_o, st_o, sh_o;
    long long sb_g, st_g;  // g / beta strides by sequence and token; value head contiguous
};

// Workspace of one segment. Per (b, hv, chunk): u fp32 [64][128] stored in K2's accumulator
// fragment order (see u_frag), w fp16 [64][128], intra fp16 hi and lo [64][64] each, and the decay factors
// dec fp32 [3][64] = (e^{cum_i}, e^{cum_last - cum_i}, e^{cum_last}). Per (b, kh, chunk):
// qn fp16 [64][128], knT fp16 [128][64]. w, intra, qn and knT are stored in MFMA A-operand
// fragment order (afrag_coords).
// Plus the carried state [B, HV, 128, 128] fp32 when the caller passes none.
struct WsLayout {
    size_t u, w, intra, intra_lo, cum, qn, knt, state, total;
};

__host__ __device__ inline size_t al256(size_t x) { return (x + 255) / 256 * 256; }

__host__ __device__ inline WsLayout ws_layout(int B, int HK, int HV, int nch) {
    WsLayout L;
    size_t units_v = (size_t)B * HV * nch, units_k = (size_t)B * HK * nch;
    size_t off = 0;
    L.u = off; off += al256(units_v * CH * D * 4);
    L.w = off; off += al256(units_v * CH * D * 2);
    L.intra = off; off += al256(units_v * CH * CH * 2);
    L.intra_lo = off; off += al256(units_v * CH * CH * 2);
    L.cum = off; off += al256(units_v * 3 * CH * 4);
    L.qn = off; off += al256(units_k * CH * D * 2);
    L.knt = off; off += al256(units_k * CH * D * 2);
    L.state = off; off += al256((size_t)B * HV * D * D * 4);
    L.total = off;
    return L;
}

__device__ __forceinline__ half8 ld_h8(const half_t* p) { return *(const half8*)p; }

// MFMA A-operand fragment order. For A [M][K] (M % 16 == 0, K % 32 == 0), fragment (mb, ks)
// holds for lane l the 8 halves A[16 mb + l % 16][32 ks + 8 (l / 16) + i], i < 8 - exactly what
// lane l passes to v_mfma_f32_16x16x32_f16 for row block mb and k block ks. Fragments are
// stored contiguously, offset ((mb * K / 32 + ks) * 64 + l) * 8 halves, so a wave loads one
// operand with a single 1 KB contiguous access. Returns the (row, first column) of fragment
// slot f.
__device__ __forceinline__ void afrag_coords(int f, int KS, int& r, int& c0) {
    const int l = f % 64, ks = (f / 64) % KS, mb = f / (64 * KS);
    r = 16 * mb + l % 16;
    c0 = 32 * ks + 8 * (l / 16);
}

// 8 consecutive activations as fp32 (two 16-byte loads for fp32, one for bf16)
template <typename T> __device__ __forceinline__ void ld8(const T* p, float* o);
template <> __device__ __forceinline__ void ld8<float>(const float* p, float* o) {
    const float4 a = ((const float4*)p)[0], b = ((const float4*)p)[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
template <> __device__ __forceinline__ void ld8<uint16_t>(const uint16_t* p, float* o) {
    const uint4 a = *(const uint4*)p;
    o[0] = bf_lo(a.x); o[1] = bf_hi(a.x); o[2] = bf_lo(a.y); o[3] = bf_hi(a.y);
    o[4] = bf_lo(a.z); o[5] = bf_hi(a.z); o[6] = bf_lo(a.w); o[7] = bf_hi(a.w);
}

// Offset (in floats) of u[i][col] inside one chunk's u block, laid out as K2 reads it: slice
// sl = col / 32, wave wv = i / 16, column tile ct, then the 64 lanes (gq = (i % 16) / 4,
// n = col % 16) of a 16x16 accumulator, each holding rows 4gq .. 4gq+3 contiguously.
__device__ __forceinline__ int u_frag(int i, int col) {
    const int sl = col / 32, ct = (col % 32) / 16, n = col % 16, wv = i / 16, gq = (i % 16) / 4, j = i % 4;
    return ((((sl * 4 + wv) * 2 + ct) * 64) + gq * 16 + n) * 4 + j;
}

__device__ __forceinline__ f32x4 mfma16(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------------
// K1: intra-chunk work, one workgroup of 256 threads (4 waves) per (chunk c, value head hv,
// sequence b). The body is shared by the standalone kernel (grid (nch, HV, B)) and the fused
// launch below; its LDS is one struct so the fused kernel can overlay it with K2's.
template <bool kSplitV>
struct K1Smem {
    __attribute__((aligned(16))) half_t QV[CH][QK_LD];  // q_n tile, then v (fp16 hi)
    __attribute__((aligned(16))) half_t Vl[kSplitV ? CH : 1][QK_LD];
    __attribute__((aligned(16))) half_t Ks[CH][QK_LD];
    // A (strict lower), with the inverses of the diagonal blocks of I + A written over its
    // diagonal blocks; the w staging tile afterwards
    __attribute__((aligned(16))) float As[CH][A_LD];
    float cum_s[CH], beta_s[CH], g_s[CH], rq_s[CH], rk_s[CH];
    // intra is staged for fragment order in QV's space: q_n has been read into registers by then,
    // and v is written there only after the intra fragments have gone out. 53 KB in all for bf16
    // inputs: three workgroups per CU for the standalone K1 launch.
};

// step 5 reuses As for the w staging tile; intra is staged in fp32 (row pitch CH + 4) in QV's space
static_assert(sizeof(half_t) * CH * QK_LD >= CH * (CH + 4) * sizeof(float), "intra staging exceeds the q tile");
static_assert(sizeof(float) * CH * A_LD >= sizeof(half_t) * CH * QK_LD, "w staging exceeds As");

template <typename Tin>
__device__ __forceinline__ void chunk_intra_body(const Tin* __restrict__ q, const Tin* __restrict__ k,
                                                 const Tin* __restrict__ v, const float* __restrict__ g,
                                                 const float* __restrict__ beta, const SeqLayout& a, int t0, int T,
                                                 int HK, int HV, int normalize, float qscale, float eps,
                                                 unsigned char* __restrict__ ws, const WsLayout& L, int vec_in,
                                                 K1Smem<sizeof(Tin) == 4>& sm, int c, int hv, int b, int nch) {
    constexpr bool kSplitV = sizeof(Tin) == 4;  // fp32 v needs a low fp16 part; bf16 v is exact in fp16
    auto& QV = sm.QV;
    auto& Vl = sm.Vl;
    auto& Ks = sm.Ks;
    auto& As = sm.As;
    auto& cum_s = sm.cum_s;
    auto& beta_s = sm.beta_s;
    auto& g_s = sm.g_s;
    auto& rq_s = sm.rq_s;
    auto& rk_s = sm.rk_s;
    float (*It)[CH + 4] = (float (*)[CH + 4])&QV[0][0];

    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, n = lane % 16, gq = lane / 16;
    const int R = HV / HK, kh = hv / R;
    const bool writes_qk = (hv % R) == 0;
    const int tok0 = t0 + c * CH;
    const size_t vu = (size_t)(b * HV + hv) * nch + c;

    // ---- 1. q, k, v rows (thread = row, 32-element quarter); fp32 row norms; fp16 q_n, k_n
    const int row = tid / 4, qq = tid % 4, tok = tok0 + row;
    const bool valid = tok < T;
    float xv[32];
    {
        // beta / g first: their latency overlaps the row loads
        float beta_r = 0.f, g_r = 0.f;
        if (qq == 0 && valid) {
            beta_r = beta[b * a.sb_g + (long long)tok * a.st_g + hv];
            g_r = g[b * a.sb_g + (long long)tok * a.st_g + hv];
        }
        const Tin* qp = q + b * a.sb_qk + (long long)tok * a.st_qk + kh * a.sh_qk + qq * 32;
        const Tin* kp = k + b * a.sb_qk + (long long)tok * a.st_qk + kh * a.sh_qk + qq * 32;
        const Tin* vp = v + b * a.sb_v + (long long)tok * a.st_v + hv * a.sh_v + qq * 32;
        float xq[32], xk[32];
        if (valid && vec_in) {
#pragma unroll
            for (int e = 0; e < 32; e += 8) {
                ld8<Tin>(qp + e, xq + e);
                ld8<Tin>(kp + e, xk + e);
                ld8<Tin>(vp + e, xv + e);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 32; e++) {
                xq[e] = valid ? Act<Tin>::ld(qp, e) : 0.f;
                xk[e] = valid ? Act<Tin>::ld(kp, e) : 0.f;
                xv[e] = valid ? Act<Tin>::ld(vp, e) : 0.f;
            }
        }
        float ssq = 0.f, ssk = 0.f;
#pragma unroll
        for (int e = 0; e < 32; e++) {
            ssq += xq[e] * xq[e];
            ssk += xk[e] * xk[e];
        }
        ssq += lane_xor<1>(ssq);
        ssq += lane_xor<2>(ssq);
        ssk += lane_xor<1>(ssk);
        ssk += lane_xor<2>(ssk);
        const float rq = normalize ? rsqrtf(ssq + eps) * qscale : 1.f;
        const float rk = normalize ? rsqrtf(ssk + eps) : 1.f;
        // the tiles keep the raw rows (exact in fp16 for bf16 inputs; fp32 inputs add a low fp16
        // part, in Vl for k and in As's space for q, both free until step 3's products are done)
        half_t (*Ql)[QK_LD] = (half_t (*)[QK_LD])&As[0][0];
#pragma unroll
        for (int e = 0; e < 32; e += 8) {
            half8 hq, hk, lq, lk;
#pragma unroll
            for (int f = 0; f < 8; f++) {
                hq[f] = (half_t)xq[e + f];
                hk[f] = (half_t)xk[e + f];
                lq[f] = (half_t)(xq[e + f] - (float)hq[f]);
                lk[f] = (half_t)(xk[e + f] - (float)hk[f]);
            }
            *(half8*)&QV[row][qq * 32 + e] = hq;
            *(half8*)&Ks[row][qq * 32 + e] = hk;
            if constexpr (kSplitV) {
                *(half8*)&Ql[row][qq * 32 + e] = lq;
                *(half8*)&Vl[row][qq * 32 + e] = lk;
            }
        }
        if (qq == 0) {
            beta_s[row] = beta_r;
            g_s[row] = g_r;
            // padding rows (past T) carry zero factors
            rq_s[row] = valid ? rq : 0.f;
            rk_s[row] = valid ? rk : 0.f;
        }
    }
    lds_barrier();

    // ---- 2. cum = inclusive prefix sum of g (wave 0) and the decay factors K2 needs;
    // q_n rows and k_n^T for K2 (once per QK head)
    if (wave == 0) {
        float x = g_s[lane];
#pragma unroll
        for (int d = 1; d < WAVE; d <<= 1) {
            float y = __shfl_up(x, d, WAVE);
            if (lane >= d) x += y;
        }
        cum_s[lane] = x;
        const float last = __shfl(x, CH - 1, WAVE);
        float* dec = (float*)(ws + L.cum) + vu * 3 * CH;
        dec[lane] = rq_s[lane] * __expf(x);
        dec[CH + lane] = rk_s[lane] * __expf(last - x);
        dec[2 * CH + lane] = __expf(last);
    }
    if (writes_qk) {
        // q_n (A of q_n S: 64 x 128) and k_n^T (A of the state update: 128 dk x 64 rows) in
        // fragment order
        const size_t ku = ((size_t)(b * HK + kh) * nch + c);
        half8* qn = (half8*)((half_t*)(ws + L.qn) + ku * CH * D);
        half8* knt = (half8*)((half_t*)(ws + L.knt) + ku * CH * D);
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const int f = tid + 256 * it;
            int r, c0;
            afrag_coords(f, 4, r, c0);
            qn[f] = ld_h8(&QV[r][c0]);
            afrag_coords(f, 2, r, c0);  // r = dk, c0 = first chunk row
            half8 v;
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = Ks[c0 + i][r];
            knt[f] = v;
        }
    }
    lds_barrier();

    // ---- 3. k~ k~^T and q~ k~^T on MFMA over the raw rows (fp32 inputs: hi hi + hi lo + lo hi),
    // lower 16 x 16 blocks only: 10 blocks of each, 5 per wave: wave w forms the A blocks of row
    // block w (w + 1 of them) and the intra blocks of row block 3 - w (4 - w of them). All
    // products first (the low parts of q live in As's space), then A and intra with every row
    // factor (beta, the norms, the decays) applied in fp32, and the upper blocks cleared.
    {
        const int wv = __builtin_amdgcn_readfirstlane(wave);
        const int ra = wv, rb = 3 - wv;
        half_t (*Ql)[QK_LD] = (half_t (*)[QK_LD])&As[0][0];
        half8 ak[4], aq[4], akl[4], aql[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            ak[ks] = ld_h8(&Ks[16 * ra + n][32 * ks + 8 * gq]);
            aq[ks] = ld_h8(&QV[16 * rb + n][32 * ks + 8 * gq]);
            if constexpr (kSplitV) {
                akl[ks] = ld_h8(&Vl[16 * ra + n][32 * ks + 8 * gq]);
                aql[ks] = ld_h8(&Ql[16 * rb + n][32 * ks + 8 * gq]);
            }
        }
        f32x4 accA[4], accI[4];
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
            accA[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
            accI[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (cb > ra && cb > rb) continue;
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const half8 bh = ld_h8(&Ks[16 * cb + n][32 * ks + 8 * gq]);
                half8 bl;
                if constexpr (kSplitV) bl = ld_h8(&Vl[16 * cb + n][32 * ks + 8 * gq]);
                if (cb <= ra) {
                    accA[cb] = mfma16(ak[ks], bh, accA[cb]);
                    if constexpr (kSplitV) {
                        accA[cb] = mfma16(ak[ks], bl, accA[cb]);
                        accA[cb] = mfma16(akl[ks], bh, accA[cb]);
                    }
                }
                if (cb <= rb) {
                    accI[cb] = mfma16(aq[ks], bh, accI[cb]);
                    if constexpr (kSplitV) {
                        accI[cb] = mfma16(aq[ks], bl, accI[cb]);
                        accI[cb] = mfma16(aql[ks], bh, accI[cb]);
                    }
                }
            }
        }
        float ca[4], ba[4], cq[4], rqv[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            ca[j] = cum_s[16 * ra + 4 * gq + j];
            ba[j] = beta_s[16 * ra + 4 * gq + j] * rk_s[16 * ra + 4 * gq + j];
            cq[j] = cum_s[16 * rb + 4 * gq + j];
            rqv[j] = rq_s[16 * rb + 4 * gq + j];
        }
        lds_barrier();  // every product is done: As and It (QV's space) are written next
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
            const int jj = 16 * cb + n;
            const float cj = cum_s[jj], rkj = rk_s[jj];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = 16 * ra + 4 * gq + j;
                As[i][jj] = cb <= ra && jj < i ? ba[j] * rkj * (__expf(ca[j] - cj) * accA[cb][j]) : 0.f;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = 16 * rb + 4 * gq + j;
                It[i][jj] = cb <= rb && jj <= i ? rqv[j] * rkj * (__expf(cq[j] - cj) * accI[cb][j]) : 0.f;
            }
        }
    }
    lds_barrier();
    {   // intra (A of intra v_new: 64 x 64) in fragment order, as fp16 hi + lo (~22 bits: the
        // intra v_new product carries most of the output's rounding error otherwise)
        half8* intra = (half8*)((half_t*)(ws + L.intra) + vu * CH * CH);
        half8* intra_lo = (half8*)((half_t*)(ws + L.intra_lo) + vu * CH * CH);
#pragma unroll
        for (int it = 0; it < 2; it++) {
            const int f = tid + 256 * it;
            int r, c0;
            afrag_coords(f, 2, r, c0);
            const f32x4 x0 = *(const f32x4*)&It[r][c0], x1 = *(const f32x4*)&It[r][c0 + 4];
            half8 hi, lo;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float x = i < 4 ? x0[i] : x1[i - 4];
                hi[i] = (half_t)x;
                lo[i] = (half_t)(x - (float)hi[i]);
            }
            intra[f] = hi;
            intra_lo[f] = lo;
        }
    }
    lds_barrier();  // It (QV's space) has gone out; v is written there next

    // ---- 4. v (fp16 hi / lo) into the q tile's space; inverses of the diagonal blocks of I + A
#pragma unroll
    for (int e = 0; e < 32; e += 8) {
        half8 hv8, lv8;
#pragma unroll
        for (int f = 0; f < 8; f++) {
            const half_t h = (half_t)xv[e + f];
            hv8[f] = h;
            lv8[f] = (half_t)(xv[e + f] - (float)h);
        }
        *(half8*)&QV[row][qq * 32 + e] = hv8;
        if constexpr (kSplitV) *(half8*)&Vl[row][qq * 32 + e] = lv8;
    }
    {   // 4a. diagonal block wave: lane j < 16 solves column j of (I + A_ww)^-1; A[i][k] of the
        // block is broadcast from lane k with readlane
        const int j = lane & 15, o = 16 * wave;
        float acol[16], x[16];
#pragma unroll
        for (int i = 0; i < 16; i++) acol[i] = As[o + i][o + j];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float s = i == j ? 1.f : 0.f;
#pragma unroll
            for (int kk = 0; kk < i; kk++)
                s -= __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acol[i]), kk)) * x[kk];
            x[i] = s;
        }
        lds_barrier();  // every wave has read its A block column before X overwrites it
        if (lane < 16) {
#pragma unroll
            for (int i = 0; i < 16; i++) As[o + i][o + j] = x[i];
        }
    }
    lds_barrier();
    // ---- 5. u = (I + A)^-1 diag(beta) v and w = (I + A)^-1 diag(beta e^cum rk) k~ by blocked
    // forward substitution over the four 16-row blocks: block row r of U is
    //   U_r = D_r^-1 (R_r - sum_{k < r} A_rk U_k),   D_r^-1 = (I + A_rr)^-1 (step 4a),
    // with the 256 right-hand-side columns split over the waves (waves 0, 1: u columns
    // 64 (w % 2) ..; waves 2, 3: w columns), so a wave owns its columns of U for every row and
    // needs no barrier. Products on v_mfma_f32_16x16x32_f16 with both sides as fp16 hi + lo.
    // The k index of each product runs over two 16-row blocks in the order the accumulators hold
    // them (lane group g: rows 4 g .. 4 g + 3 of the first block, then of the second), so an
    // accumulator pair is a B operand as it stands; the A side reads A and D^-1 in that order.
    {
        const bool isw = wave >= 2;
        const int cbase = 64 * (wave & 1);
        half_t (*src)[QK_LD] = isw ? Ks : QV;  // raw k rows / v rows (fp16)
        typedef __attribute__((address_space(3))) short4v_t lds_s4;
        // row factors of this lane's rows 16 r + 4 gq + j
        f32x4 U[4][4];
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int ct = 0; ct < 4; ct++) U[r][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
        // A-side operand (rows 16 r + n, k slots of block pair (kb0, kb0 + 1)), hi / lo, negated
        // on request; columns of blocks >= nb_valid read as zero
        auto aop = [&](int r, int kb0, bool second, bool neg, half8& hi, half8& lo) {
            const f32x4 x0 = *(const f32x4*)&As[16 * r + n][16 * kb0 + 4 * gq];
            f32x4 x1 = f32x4{0.f, 0.f, 0.f, 0.f};
            if (second) x1 = *(const f32x4*)&As[16 * r + n][16 * (kb0 + 1) + 4 * gq];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float x = (i < 4 ? x0[i] : x1[i - 4]) * (neg ? -1.f : 1.f);
                const half_t h = (half_t)x;
                hi[i] = h;
                lo[i] = (half_t)(x - (float)h);
            }
        };
        auto split = [&](const f32x4& a, const f32x4& b, half8& hi, half8& lo) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float x = i < 4 ? a[i] : b[i - 4];
                const half_t h = (half_t)x;
                hi[i] = h;
                lo[i] = (half_t)(x - (float)h);
            }
        };
        const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float fr[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int t = 16 * r + 4 * gq + j;
                fr[j] = isw ? beta_s[t] * __expf(cum_s[t]) * rk_s[t] : beta_s[t];
            }
            f32x4 acc[4];
#pragma unroll
            for (int ct = 0; ct < 4; ct++) {
                // right-hand side rows 16 r + 4 gq .. +3 of column cbase + 16 ct + n: one
                // transpose read (lane k of a 16-lane group addresses row R + k / 4, columns
                // C + 4 (k % 4) .. +3; lane j receives rows R .. R + 3 of column C + j)
                const int R0 = 16 * r + 4 * gq, C0 = cbase + 16 * ct;
                const short4v_t h4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s4*)&src[R0 + (n >> 2)][C0 + 4 * (n & 3)]);
                // (bit-cast the whole vector: clang's __builtin_bit_cast of a vector element
                // reads element 0 whatever the index)
                const half4 hh = __builtin_bit_cast(half4, h4);
#pragma unroll
                for (int j = 0; j < 4; j++) acc[ct][j] = fr[j] * (float)hh[j];
                if constexpr (kSplitV) {
                    if (!isw) {
                        const short4v_t l4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (lds_s4*)&Vl[R0 + (n >> 2)][C0 + 4 * (n & 3)]);
                        const half4 ll = __builtin_bit_cast(half4, l4);
#pragma unroll
                        for (int j = 0; j < 4; j++) acc[ct][j] += fr[j] * (float)ll[j];
                    }
                }
            }
            // acc -= A_{r, (2m, 2m+1)} U_{(2m, 2m+1)} over the block pairs below r
#pragma unroll
            for (int m = 0; 2 * m < r; m++) {
                half8 ah, al;
                aop(r, 2 * m, 2 * m + 1 < r, true, ah, al);
#pragma unroll
                for (int ct = 0; ct < 4; ct++) {
                    half8 bh, bl;
                    split(U[2 * m][ct], 2 * m + 1 < r ? U[2 * m + 1][ct] : zero4, bh, bl);
                    acc[ct] = mfma16(ah, bh, acc[ct]);
                    acc[ct] = mfma16(ah, bl, acc[ct]);
                    acc[ct] = mfma16(al, bh, acc[ct]);
                }
            }
            // U_r = D_r^-1 acc (k slots of the second block are zero on both sides)
            half8 dh, dl;
            aop(r, r, false, false, dh, dl);
#pragma unroll
            for (int ct = 0; ct < 4; ct++) {
                half8 bh, bl;
                split(acc[ct], zero4, bh, bl);
                f32x4 y = mfma16(dh, bh, zero4);
                y = mfma16(dh, bl, y);
                U[r][ct] = mfma16(dl, bh, y);
            }
        }
        if (!isw) {
            float* u = (float*)(ws + L.u) + vu * CH * D;
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int ct = 0; ct < 4; ct++)
                    *(f32x4*)(u + u_frag(16 * r + 4 * gq, cbase + 16 * ct + n)) = U[r][ct];
        }
        lds_barrier();  // every wave is done with As and the v / k tiles: w is staged in As's space
        half_t (*Wst)[QK_LD] = (half_t (*)[QK_LD])&As[0][0];
        if (isw) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int ct = 0; ct < 4; ct++)
#pragma unroll
                    for (int j = 0; j < 4; j++) Wst[16 * r + 4 * gq + j][cbase + 16 * ct + n] = (half_t)U[r][ct][j];
        }
        lds_barrier();
        half8* wf = (half8*)((half_t*)(ws + L.w) + vu * CH * D);
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const int f = tid + 256 * it;
            int r, c0;
            afrag_coords(f, 4, r, c0);
            wf[f] = ld_h8(&Wst[r][c0]);
        }
    }
}

template <typename Tin>
__global__ void __launch_bounds__(256, 3) delta_chunk_intra(const Tin* __restrict__ q, const Tin* __restrict__ k,
                                                         const Tin* __restrict__ v, const float* __restrict__ g,
                                                         const float* __restrict__ beta, SeqLayout a, int t0, int T,
                                                         int HK, int HV, int normalize, float qscale, float eps,
                                                         unsigned char* __restrict__ ws, WsLayout L, int vec_in) {
    __shared__ K1Smem<sizeof(Tin) == 4> sm;
    chunk_intra_body<Tin>(q, k, v, g, beta, a, t0, T, HK, HV, normalize, qscale, eps, ws, L, vec_in, sm, blockIdx.x,
                          blockIdx.y, blockIdx.z, gridDim.x);
}

// ---------------------------------------------------------------------------------------------
// K2: sequential recurrence over the chunks of a segment. 1-D grid of (B HV rounded up to 8) x
// 128 / (16 NCT) blocks, 256 threads; Lb is the block's index in that grid.
// Wave w holds S rows [32w, 32w+32) x the slice's 16 NCT columns as 2 x NCT MFMA tiles.
template <int NCT>
struct K2Smem {
    // double-buffered by chunk parity: a wave cannot pass the next chunk's first barrier before
    // every wave has finished reading this chunk's tiles, so no end-of-chunk barrier is needed
    __attribute__((aligned(16))) half_t SsT[2][16 * NCT][D + 8];   // S^T (fp16): [column][dk]
    __attribute__((aligned(16))) half_t VnT[2][16 * NCT][CH + 8];  // v_new^T (fp16 hi)
    __attribute__((aligned(16))) half_t VlT[2][16 * NCT][CH + 8];  // v_new^T (fp16 lo)
    __attribute__((aligned(16))) half_t VdT[2][16 * NCT][CH + 8];  // (e^{cum_last-cum} v_new)^T
    __attribute__((aligned(16))) float Ot[4][16][16 * NCT + 4];  // output staging per wave
};

template <typename Tout, int NCT, bool VEC>
__device__ __forceinline__ void chunk_state_body(const unsigned char* __restrict__ ws, const WsLayout& L,
                                                 float* __restrict__ state, int load_state, Tout* __restrict__ out,
                                                 const SeqLayout& a, int t0, int T, int nch, int B, int HK, int HV,
                                                 K2Smem<NCT>& sm, int Lb) {
    auto& SsT = sm.SsT;
    auto& VnT = sm.VnT;
    auto& VlT = sm.VlT;
    auto& VdT = sm.VdT;
    auto& Ot = sm.Ot;

    // XCD-aware block mapping (1-D grid): blocks are dealt to the 8 XCDs round-robin, so unit
    // u = (m / NS) * 8 + xcd keeps all NS column slices of one (sequence, head) on one XCD,
    // where they share the chunk operands in that XCD's L2.
    constexpr int NS = D / (16 * NCT);
    const int xcd = Lb % 8, m = Lb / 8;
    const int unit = (m / NS) * 8 + xcd, sl = m % NS;
    if (unit >= B * HV) return;  // grid padded to a multiple of 8 units
    const int hv = unit % HV, b = unit / HV;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, n = lane % 16, gq = lane / 16;
    const int R = HV / HK, kh = hv / R;
    const int col0 = sl * 16 * NCT;
    float* Sg = state + (size_t)(b * HV + hv) * D * D;

    f32x4 S[2][NCT];
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int ct = 0; ct < NCT; ct++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                S[rt][ct][j] = load_state ? Sg[(size_t)(32 * wave + 16 * rt + 4 * gq + j) * D + col0 + 16 * ct + n] : 0.f;

    const size_t vbase = (size_t)(b * HV + hv) * nch, kbase = (size_t)(b * HK + kh) * nch;
    // operands of one chunk that do not depend on S; each part is refilled with the next chunk's
    // values while the current chunk computes (see step), hiding the L2 / HBM latency
    struct Ops {
        half8 wa[4], qa[4], ia[2], il[2], ka[2][2];
        f32x4 uu[NCT], ecum, edec;  // u fragment; e^{cum_i}, e^{cum_last - cum_i} for this lane's rows
        float gamma;              // e^{cum_last}
    };
    // part < 0: every operand; part 0..4: the slice of the fetch issued at that phase of step()
    auto fetch = [&](int c, Ops& o, int part = -1) {
        const size_t vu = vbase + c, ku = kbase + c;
        const half_t* Wc = (const half_t*)(ws + L.w) + vu * CH * D;
        const half_t* Qc = (const half_t*)(ws + L.qn) + ku * CH * D;
        const float* Uc = (const float*)(ws + L.u) + vu * CH * D;
        const half_t* Ic = (const half_t*)(ws + L.intra) + vu * CH * CH;
        const half_t* Ilc = (const half_t*)(ws + L.intra_lo) + vu * CH * CH;
        const half_t* KTc = (const half_t*)(ws + L.knt) + ku * CH * D;
        const float* dec = (const float*)(ws + L.cum) + vu * 3 * CH;
        // fragment-order operands (written so by K1): one contiguous 1 KB load per fragment.
        // Parts in the order step() consumes them: 0 = w, q_n (w S, q_n S); 1 = u, e^{cum_last -
        // cum} (v_new); 2 = intra, e^{cum} (output); 3 = k_n^T, e^{cum_last} (state update)
        if (part < 0 || part == 0)
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                o.wa[ks] = ld_h8(Wc + ((4 * wave + ks) * 64 + lane) * 8);
                o.qa[ks] = ld_h8(Qc + ((4 * wave + ks) * 64 + lane) * 8);
            }
        if (part < 0 || part == 1) {
#pragma unroll
            for (int ct = 0; ct < NCT; ct++)
                o.uu[ct] = *(const f32x4*)(Uc + u_frag(16 * wave + 4 * gq, col0 + 16 * ct + n));
            o.edec = *(const f32x4*)(dec + CH + 16 * wave + 4 * gq);
        }
        if (part < 0 || part == 2) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                o.ia[ks] = ld_h8(Ic + ((2 * wave + ks) * 64 + lane) * 8);
                o.il[ks] = ld_h8(Ilc + ((2 * wave + ks) * 64 + lane) * 8);
            }
            o.ecum = *(const f32x4*)(dec + 16 * wave + 4 * gq);
        }
        if (part < 0 || part == 3) {
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
#pragma unroll
                for (int ks = 0; ks < 2; ks++)
                    o.ka[rt][ks] = ld_h8(KTc + ((2 * (2 * wave + rt) + ks) * 64 + lane) * 8);
            o.gamma = dec[2 * CH];
        }
    };
    // per-chunk compute on operands `op`. Each part of `op` is refilled with chunk cn's values
    // right after its last use, so one register set suffices and the vector-memory path streams
    // the next chunk's operands while this chunk computes (a load burst would stall the wave at
    // issue; the operand volume per chunk is the bound of this loop)
    auto step = [&](int c, Ops& op, int cn) {
        const Ops& cur = op;
        auto issue = [&](int part) {
            __builtin_amdgcn_sched_barrier(0);
            fetch(cn, op, part);
            __builtin_amdgcn_sched_barrier(0);
        };
        const half8* wa = cur.wa;
        const half8* qa = cur.qa;
        const half8* ia = cur.ia;
        const half8* il = cur.il;
        const f32x4* uu = cur.uu;

        const int pb = c & 1;
        // (1) S -> LDS as fp16, transposed (a lane's 4 rows are adjacent in S^T: one 8-byte write)
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int ct = 0; ct < NCT; ct++) {
                const half4 h = {(half_t)S[rt][ct][0], (half_t)S[rt][ct][1], (half_t)S[rt][ct][2], (half_t)S[rt][ct][3]};
                *(half4*)&SsT[pb][16 * ct + n][32 * wave + 16 * rt + 4 * gq] = h;
            }
        __syncthreads();

        // (2) w S, then q_n S, for chunk rows [16 wave, 16 wave + 16): v_new needs only w S, so
        // its VALU work overlaps the q_n S products in the MFMA pipe
        half8 sb[NCT][4];
#pragma unroll
        for (int ct = 0; ct < NCT; ct++)
#pragma unroll
            for (int ks = 0; ks < 4; ks++) sb[ct][ks] = ld_h8(&SsT[pb][16 * ct + n][32 * ks + 8 * gq]);
        f32x4 WS[NCT], QS[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ct++) {
            WS[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) WS[ct] = mfma16(wa[ks], sb[ct][ks], WS[ct]);
        }
#pragma unroll
        for (int ct = 0; ct < NCT; ct++) {
            QS[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) QS[ct] = mfma16(qa[ks], sb[ct][ks], QS[ct]);
        }
        issue(0);
        // (3) v_new = u - w S; decayed copy for the state update
#pragma unroll
        for (int ct = 0; ct < NCT; ct++) {
            half4 hn, ln, hd;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float vn = uu[ct][j] - WS[ct][j];
                hn[j] = (half_t)vn;
                ln[j] = (half_t)(vn - (float)hn[j]);
                hd[j] = (half_t)(cur.edec[j] * vn);
            }
            *(half4*)&VnT[pb][16 * ct + n][16 * wave + 4 * gq] = hn;
            *(half4*)&VlT[pb][16 * ct + n][16 * wave + 4 * gq] = ln;
            *(half4*)&VdT[pb][16 * ct + n][16 * wave + 4 * gq] = hd;
        }
        issue(1);
        __syncthreads();

        // (4) intra v_new, then (5) S = e^{cum_last} S + k_n^T v' in the MFMA pipe; the output
        // staging and stores below overlap the state update
        f32x4 ov[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ct++) {
            ov[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                // intra v_new as hi hi + hi lo + lo hi
                const half8 vh = ld_h8(&VnT[pb][16 * ct + n][32 * ks + 8 * gq]);
                ov[ct] = mfma16(ia[ks], vh, ov[ct]);
                ov[ct] = mfma16(ia[ks], ld_h8(&VlT[pb][16 * ct + n][32 * ks + 8 * gq]), ov[ct]);
                ov[ct] = mfma16(il[ks], vh, ov[ct]);
            }
        }
        {
            const float gamma = cur.gamma;
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
#pragma unroll
                for (int ct = 0; ct < NCT; ct++) {
                    f32x4 acc = S[rt][ct] * gamma;
#pragma unroll
                    for (int ks = 0; ks < 2; ks++)
                        acc = mfma16(cur.ka[rt][ks], ld_h8(&VdT[pb][16 * ct + n][32 * ks + 8 * gq]), acc);
                    S[rt][ct] = acc;
                }
        }
        // o = e^{cum} q_n S + intra v_new
#pragma unroll
        for (int ct = 0; ct < NCT; ct++)
#pragma unroll
            for (int j = 0; j < 4; j++) Ot[wave][4 * gq + j][16 * ct + n] = cur.ecum[j] * QS[ct][j] + ov[ct][j];
        wave_sync();
        {   // this wave's 16 rows x 16 NCT columns: lane = (row, 8-column part), 64 / LPR rows
            // per pass
            constexpr int LPR = 2 * NCT;  // lanes per row
            constexpr int RPP = WAVE / LPR;
            const int tc = t0 + c * CH;  // first token of the chunk
            if constexpr (VEC) {
                // Raw buffer stores, issued on every lane: rows past T (or past the wave's 16)
                // get an offset beyond num_records and the hardware drops them. A store count
                // that does not depend on a branch lets the compiler's wait for the next chunk's
                // operands (issued before these stores) leave the stores in flight.
                const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                    out + b * a.sb_o + (long long)tc * a.st_o + hv * a.sh_o + col0, (short)0, kOutRange, kBufWord3);
#pragma unroll
                for (int r0 = 0; r0 < 16; r0 += RPP) {
                    const int r = r0 + lane / LPR, p8 = (lane % LPR) * 8, row = 16 * wave + r;
                    const bool ok = r < 16 && tc + row < T;
                    const int off = ok ? (int)(((long long)row * a.st_o + p8) * (long long)sizeof(Tout)) : kOutDrop;
                    // two 16-byte LDS reads per lane (row pitch and p8 keep them aligned)
                    const f32x4 s0 = *(const f32x4*)&Ot[wave][r & 15][p8];
                    const f32x4 s1 = *(const f32x4*)&Ot[wave][r & 15][p8 + 4];
                    if constexpr (sizeof(Tout) == 2) {
                        const u32x4 pk = {f2bf2(s0[0], s0[1]), f2bf2(s0[2], s0[3]), f2bf2(s1[0], s1[1]),
                                          f2bf2(s1[2], s1[3])};
                        __builtin_amdgcn_raw_buffer_store_b128(pk, rs, off, 0, 0);
                    } else {
                        const u32x4 lo = __builtin_bit_cast(u32x4, s0);
                        const u32x4 hi = __builtin_bit_cast(u32x4, s1);
                        __builtin_amdgcn_raw_buffer_store_b128(lo, rs, off, 0, 0);
                        __builtin_amdgcn_raw_buffer_store_b128(hi, rs, ok ? off + 16 : kOutDrop, 0, 0);
                    }
                }
            } else {
#pragma unroll
                for (int r0 = 0; r0 < 16; r0 += RPP) {
                    const int r = r0 + lane / LPR, p8 = (lane % LPR) * 8, tok = tc + 16 * wave + r;
                    if (r < 16 && tok < T) {
                        Tout* dst = out + b * a.sb_o + (long long)tok * a.st_o + hv * a.sh_o + col0 + p8;
                        const float* src = &Ot[wave][r][p8];
#pragma unroll
                        for (int e = 0; e < 8; e++) Act<Tout>::st(dst, e, src[e]);
                    }
                }
            }
        }
        issue(2);
        issue(3);
    };
    // the first chunk's operands in the order the loop refills them, with a discarded store where
    // the loop body has its output store, so the loop entry and the back edge carry the same
    // sequence of memory operations (static wait counts)
    Ops op;
    fetch(0, op, 0);
    fetch(0, op, 1);
    if constexpr (VEC) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(out, (short)0, kOutRange, kBufWord3);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, rs, kOutDrop, 0, 0);
        if constexpr (sizeof(Tout) == 4)
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, rs, kOutDrop - 64, 0, 0);
    }
    fetch(0, op, 2);
    fetch(0, op, 3);
    // the next-chunk index is clamped, not skipped, so every step issues the same loads
    for (int c = 0; c < nch; c++) step(c, op, min(c + 1, nch - 1));
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int ct = 0; ct < NCT; ct++)
#pragma unroll
            for (int j = 0; j < 4; j++) Sg[(size_t)(32 * wave + 16 * rt + 4 * gq + j) * D + col0 + 16 * ct + n] = S[rt][ct][j];
}

template <typename Tout, int NCT, bool VEC>
__global__ void __launch_bounds__(256, 2) delta_chunk_state(const unsigned char* __restrict__ ws, WsLayout L,
                                                         float* __restrict__ state, int load_state, Tout* __restrict__ out,
                                                         SeqLayout a, int t0, int T, int nch, int B, int HK,
                                                         int HV) {
    __shared__ K2Smem<NCT> sm;
    chunk_state_body<Tout, NCT, VEC>(ws, L, state, load_state, out, a, t0, T, nch, B, HK, HV, sm, blockIdx.x);
}

// One launch holding K2 of one segment (blocks [0, nk2)) and K1 of the next segment (the
// remaining blocks, chunk fastest): the two are independent (different workspace buffers), so
// the K1 workgroups fill the CUs around K2's without a second stream or events. LDS is the
// union of the two bodies' needs.
template <typename Tin, typename Tout, int NCT, bool VEC>
__global__ void __launch_bounds__(256, 3) delta_chunk_fused(
    // K2 of segment s
    const unsigned char* __restrict__ ws2, WsLayout L2, float* __restrict__ state, int load_state,
    Tout* __restrict__ out, int t0s, int nch2, int nk2,
    // K1 of segment s + 1
    const Tin* __restrict__ q, const Tin* __restrict__ k, const Tin* __restrict__ v, const float* __restrict__ g,
    const float* __restrict__ beta, int t0i, int nch1, unsigned char* __restrict__ ws1, WsLayout L1, int vec_in,
    int normalize, float qscale, float eps,
    // shared
    SeqLayout a, int T, int B, int HK, int HV) {
    __shared__ union {
        K1Smem<sizeof(Tin) == 4> k1;
        K2Smem<NCT> k2;
    } sm;
    if ((int)blockIdx.x < nk2) {
        chunk_state_body<Tout, NCT, VEC>(ws2, L2, state, load_state, out, a, t0s, T, nch2, B, HK, HV, sm.k2,
                                         blockIdx.x);
    } else {
        const int r = blockIdx.x - nk2, c = r % nch1, hv = (r / nch1) % HV, b = r / (nch1 * HV);
        chunk_intra_body<Tin>(q, k, v, g, beta, a, t0i, T, HK, HV, normalize, qscale, eps, ws1, L1, vec_in, sm.k1, c,
                              hv, b, nch1);
    }
}

// Chunks per segment: SEG tokens (the workspace of one segment, ~72 MB at B = 1 with 32 value
// heads, stays resident in the MALL between the two kernels that touch it).
int seg_chunks(int B, int T, int HV) {
    (void)B;
    (void)HV;
    return (std::min(T, SEG) + CH - 1) / CH;
}

}  // namespace

namespace aegist {

// Workspace: [carried state (when the caller passes none)][segment buffer 0][segment buffer 1]
// (the second buffer only when there is more than one segment: the intra-chunk work of the
// next segment then writes one buffer while the state work of this segment reads the other).
struct WsPlan {
    size_t state_off, seg_bytes, total;
    int nch_seg, nbuf;
};
static WsPlan ws_plan(int B, int T, int HK, int HV) {
    WsPlan p;
    p.nch_seg = seg_chunks(B, T, HV);
    p.seg_bytes = ws_layout(B, HK, HV, p.nch_seg).state;  // the per-segment part, 256-aligned
    p.nbuf = (T + CH - 1) / CH > p.nch_seg ? 2 : 1;
    p.state_off = 0;
    p.total = al256((size_t)B * HV * D * D * 4) + p.nbuf * p.seg_bytes;
    return p;
}

size_t delta_chunked_ws_bytes(int B, int T, int HK, int HV) {
    if (B <= 0 || T <= 0 || HK <= 0 || HV <= 0) return 256;
    return ws_plan(B, T, HK, HV).total;
}

template <typename Tin, typename Tout, bool VEC>
int run_segments(const Tin* q, const Tin* k, const Tin* v, const float* g, const float* beta, float* S,
                 bool has_state, Tout* out, const SeqLayout& a, int B, int T, int HK, int HV, int normalize,
                 float qscale, float eps, unsigned char* const segbuf[2], const WsPlan& plan, int vec_in,
                 hipStream_t st);

template <typename Tin, typename Tout>
int run_chunked(const Tin* q, const Tin* k, const Tin* v, const float* g, const float* beta, float* state, Tout* out,
                const SeqLayout& a, int B, int T, int HK, int HV, int normalize, float qscale, float eps, void* ws,
                size_t ws_bytes, hipStream_t st) {
    const WsPlan plan = ws_plan(B, T, HK, HV);
    if (!ws || ws_bytes < plan.total) return fail(AEGIST_ERR_WORKSPACE, "delta_chunked: workspace too small");
    unsigned char* w = (unsigned char*)ws;
    // the carried state: the caller's, or the workspace copy (starts at zero: K2 does not load it)
    float* S = state ? state : (float*)(w + plan.state_off);
    unsigned char* segbuf[2] = {w + al256((size_t)B * HV * D * D * 4), nullptr};
    segbuf[1] = segbuf[0] + plan.seg_bytes;
    // 16-byte input loads need 16-byte aligned rows (and 8-element runs)
    const long long ei = 16 / (long long)sizeof(Tin);
    const int vec_in = ((uintptr_t)q % 16 == 0) && ((uintptr_t)k % 16 == 0) && ((uintptr_t)v % 16 == 0) &&
                       a.sb_qk % ei == 0 && a.st_qk % ei == 0 && a.sh_qk % ei == 0 && a.sb_v % ei == 0 &&
                       a.st_v % ei == 0 && a.sh_v % ei == 0;
    // 16-byte buffer stores need 16-byte aligned rows, and the byte offsets of one chunk's rows
    // from its first must stay below the buffer range
    const long long ev = 16 / (long long)sizeof(Tout);
    const bool vec_out = ((uintptr_t)out % 16 == 0) && a.sb_o % ev == 0 && a.st_o % ev == 0 && a.sh_o % ev == 0 &&
                         a.st_o >= 0 && (long long)CH * a.st_o * (long long)sizeof(Tout) < kOutRange;
    return vec_out ? run_segments<Tin, Tout, true>(q, k, v, g, beta, S, state != nullptr, out, a, B, T, HK, HV,
                                                  normalize, qscale, eps, segbuf, plan, vec_in, st)
                   : run_segments<Tin, Tout, false>(q, k, v, g, beta, S, state != nullptr, out, a, B, T, HK, HV,
                                                   normalize, qscale, eps, segbuf, plan, vec_in, st);
}

template <typename Tin, typename Tout, bool VEC>
int run_segments(const Tin* q, const Tin* k, const Tin* v, const float* g, const float* beta, float* S,
                 bool has_state, Tout* out, const SeqLayout& a, int B, int T, int HK, int HV, int normalize,
                 float qscale, float eps, unsigned char* const segbuf[2], const WsPlan& plan, int vec_in,
                 hipStream_t st) {
    const int seg = plan.nch_seg * CH;
    const int nseg = (T + seg - 1) / seg;
    const int units8 = (B * HV + 7) / 8 * 8;

    auto seg_layout = [&](int s) {
        const int t0 = s * seg, nch = (std::min(seg, T - t0) + CH - 1) / CH;
        return std::make_pair(nch, ws_layout(B, HK, HV, nch));
    };
    const int nk2 = units8 * (D / (16 * K2_NCT));
    // segment 0's K1 alone; then K2 of segment s with K1 of segment s + 1 in one launch; the last
    // K2 alone. Stream order carries every dependency: K1(s + 1) rewrites the buffer K2(s - 1)
    // read one launch earlier.
    {
        const auto [nch, Ls] = seg_layout(0);
        delta_chunk_intra<Tin><<<dim3(nch, HV, B), 256, 0, st>>>(q, k, v, g, beta, a, 0, T, HK, HV, normalize, qscale,
                                                                eps, segbuf[0], Ls, vec_in);
        int rc = after_launch("delta_chunk_intra");
        if (rc) return rc;
    }
    for (int s = 0; s < nseg; s++) {
        const auto [nch2, L2] = seg_layout(s);
        const int load = (has_state || s > 0) ? 1 : 0;
        if (s + 1 < nseg) {
            const auto [nch1, L1] = seg_layout(s + 1);
            // 2 KB of (unused) dynamic LDS on top of the 53 KB union: at most two workgroups per
            // CU, so a K2 workgroup shares its CU with one K1 workgroup instead of two (measured
            // 0.233 -> 0.228 ms per 8k call). Padding the static union instead lets the compiler
            // see the lower occupancy and spend ~20 more VGPRs, which loses the gain.
            delta_chunk_fused<Tin, Tout, K2_NCT, VEC><<<nk2 + nch1 * HV * B, 256, kFusedLdsPad, st>>>(
                segbuf[s & 1], L2, S, load, out, s * seg, nch2, nk2, q, k, v, g, beta, (s + 1) * seg, nch1,
                segbuf[(s + 1) & 1], L1, vec_in, normalize, qscale, eps, a, T, B, HK, HV);
            int rc = after_launch("delta_chunk_fused");
            if (rc) return rc;
        } else {
            delta_chunk_state<Tout, K2_NCT, VEC><<<nk2, 256, 0, st>>>(segbuf[s & 1], L2, S, load, out, a, s * seg, T,
                                                                       nch2, B, HK, HV);
            int rc = after_launch("delta_chunk_state");
            if (rc) return rc;
        }
    }
    return 0;
}

int launch_delta_chunked(const void* q, const void* k, const void* v, int in_dtype, const SeqLayout& a,
                         const float* g, const float* beta, float* state, void* out, int out_dtype, int B, int T,
                         int HK, int HV, int normalize, float qscale, float eps, void* ws, size_t ws_bytes,
                         hipStream_t st) {
    if (B < 0 || T < 0 || HK <= 0 || HV <= 0 || HV % HK) return fail(AEGIST_ERR_SHAPE, "delta_chunked: need HV % HK == 0");
    if (B == 0 || T == 0) return 0;
#define AEG_CHUNKED(TI, TO)                                                                                          \
    return run_chunked<TI, TO>((const TI*)q, (const TI*)k, (const TI*)v, g, beta, state, (TO*)out, a, B, T, HK, HV, \
                               normalize, qscale, eps, ws, ws_bytes, st)
    if (in_dtype == AEGIST_F32 && out_dtype == AEGIST_F32) AEG_CHUNKED(float, float);
    if (in_dtype == AEGIST_F32 && out_dtype == AEGIST_BF16) AEG_CHUNKED(float, uint16_t);
    if (in_dtype == AEGIST_BF16 && out_dtype == AEGIST_F32) AEG_CHUNKED(uint16_t, float);
    if (in_dtype == AEGIST_BF16 && out_dtype == AEGIST_BF16) AEG_CHUNKED(uint16_t, uint16_t);
#undef AEG_CHUNKED
    return fail(AEGIST_ERR_DTYPE, "delta_chunked: dtypes must be AEGIST_F32 or AEGIST_BF16");
}

// Engine mirror for T >= 64: y [T, C] rows q | k | v (already normalised), gb [T, 2HV].
size_t delta_scan_chunked_ws_bytes(int T, int HK, int HV) { return delta_chunked_ws_bytes(1, T, HK, HV); }

int delta_scan_chunked(const float* y, const float* gb, float* state, float* o, int T, int C, int HK, int HV,
                       void* ws, size_t ws_bytes, hipStream_t st) {
    SeqLayout a{0, C, D, 0, C, D, 0, (long long)HV * D, D, 0, 2 * HV};
    return launch_delta_chunked(y, y + (size_t)HK * D, y + (size_t)2 * HK * D, AEGIST_F32, a, gb, gb + HV, state, o,
                                AEGIST_F32, 1, T, HK, HV, 0, 1.f, 0.f, ws, ws_bytes, st);
}

}  // namespace aegist

extern "C" size_t aegist_delta_chunked_workspace_bytes(int B, int T, int HV) {
    // HK only changes the q_n / k_n^T share; size for HK = HV (the largest). The segment length
    // depends on B, so take the largest need over batches 1..B: a workspace sized for (B, T)
    // then serves every call with B' <= B sequences of T' <= T tokens.
    size_t need = 256;
    for (int b = 1; b <= B; b++) need = std::max(need, delta_chunked_ws_bytes(b, T, HV, HV));
    return need;
}

extern "C" int aegist_delta_chunked(const void* q, const void* k, const void* v, int in_dtype, long long sb_qk,
                                    long long st_qk, long long sh_qk, long long sb_v, long long st_v, long long sh_v,
                                    const float* g, const float* beta, float* state, void* out, int out_dtype,
                                    long long sb_o, long long st_o, long long sh_o, int B, int T, int HK, int HV,
                                    int normalize, float qscale, float eps, void* workspace, size_t workspace_bytes,
                                    void* stream) {
    SeqLayout a{sb_qk, st_qk, sh_qk, sb_v, st_v, sh_v, sb_o, st_o, sh_o, (long long)T * HV, HV};
    return launch_delta_chunked(q, k, v, in_dtype, a, g, beta, state, out, out_dtype, B, T, HK, HV, normalize, qscale,
                                eps, workspace, workspace_bytes, AEG_STREAM(stream));
}
