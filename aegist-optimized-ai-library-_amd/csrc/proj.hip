// Projections around the mixer: the weight-streaming matmuls of QLinear
// (aegist/model.py:78-93: int8 weight, per-output-row absmax scale in bf16) and of plain bf16
// weights, as the engine runs them (aegist_rs/kernels/aegist.cu:84-172: gemv_i8, gemv_bf16,
// gemm_i8; called through HybridEngine::mm, aegist_rs/src/hybrid.rs:717-735):
//     Y[m, n] (+)= scale[n] * sum_k X[m, k] W[n, k]
// with fp32 accumulation. accumulate = 1 adds into Y (the residual add of the out-projections).
//
// At decode sizes (M = batch <= 64) the op streams the weight matrix once from HBM, so the
// kernel is built around that stream: each wave owns RT 16-row tiles of W and a contiguous run
// of 64-wide k steps, loads 16 bytes of int8 weights (or 32 of bf16) per lane per step, and
// feeds v_mfma_f32_16x16x32_bf16 with W as the A operand and X^T as the B operand, so every
// weight byte is used by MT 16-row tiles of X at once. Four waves of a workgroup interleave
// their k steps (neighbouring waves read neighbouring 64-byte runs of the same rows) and add
// their partial tiles through LDS at the end, where the row scale and the accumulate are fused
// into the store.
//
// int8 and bf16 weights are exact in bf16. An fp32 X is split into bf16 hi + lo
// (x = hi + lo + O(2^-17 |x|)) and both halves go through the MFMA, so the result matches an
// fp32 dot product to ~1e-5 relative; a bf16 X needs only the hi half.
#include "common.h"

#include <cstdlib>
#include <type_traits>

using namespace aegist;

namespace aegist {
bool gemm_bf16_fits(const void* X, long long ldx, const void* W, long long ldw, int M, int N, int K);
bool gemm_i8f32_fits(const void* X, long long ldx, const void* W, long long ldw, int M, int N, int K);
int launch_gemm_i8f32(const float* X, long long ldx, const int8_t* W, long long ldw, const uint16_t* scale, float* Y,
                      long long ldy, int M, int N, int K, int accumulate, hipStream_t st);
int launch_gemm_bf16(const uint16_t* X, long long ldx, const uint16_t* W, long long ldw, float* Y, long long ldy, int M,
                     int N, int K, int accumulate, hipStream_t st);
int launch_gemm_bf16_multi(const uint16_t* X, long long ldx, int nseg, const uint16_t* const* W, const long long* ldw,
                           float* const* Y, const long long* ldy, const int* N, int M, int K, int accumulate,
                           hipStream_t st);
}  // namespace aegist

namespace {

bool stream_enabled() {
    static const bool on = [] {
        const char* e = getenv("AEGIST_PROJ_STREAM");
        return !(e && e[0] == '0');
    }();
    return on;
}

constexpr int KSTEP = 64;  // k per wave step: 16 bytes of int8 (two MFMA k-blocks of 32) per lane
#ifndef PROJ_TARGET_WAVES
#define PROJ_TARGET_WAVES 2048  // waves per launch the shape heuristic aims for
#endif

typedef int int4v __attribute__((ext_vector_type(4)));

// 16 consecutive weights of one row starting at k (zero outside the row), as two bf16x8
// operands: lo = k .. k+7, hi = k+8 .. k+15.
template <typename TW> struct WLoad;
template <> struct WLoad<int8_t> {
    int4v raw;
    __device__ __forceinline__ void load(const int8_t* row, int k, int K, bool ok) {
        raw = (ok && k < K) ? *(const int4v*)(row + k) : int4v{0, 0, 0, 0};
    }
    __device__ __forceinline__ void cvt(bf16x8& a, bf16x8& b) const {
        // int8 -> fp32 is exact (one sign-extending byte conversion each) and |q| <= 128 keeps
        // 8 significant bits, so the top half of the fp32 pattern is the exact bf16; one byte
        // permute packs two of them
        uint32_t pa[4], pb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t d = (uint32_t)raw[i];
            const float f0 = (float)(int8_t)d, f1 = (float)(int8_t)(d >> 8);
            const float f2 = (float)(int8_t)(d >> 16), f3 = (float)(int8_t)(d >> 24);
            const uint32_t p01 = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
            const uint32_t p23 = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
            if (i < 2) {
                pa[2 * i] = p01;
                pa[2 * i + 1] = p23;
            } else {
                pb[2 * (i - 2)] = p01;
                pb[2 * (i - 2) + 1] = p23;
            }
        }
        a = __builtin_bit_cast(bf16x8, pa);
        b = __builtin_bit_cast(bf16x8, pb);
    }
};
template <> struct WLoad<uint16_t> {
    bf16x8 r0, r1;
    __device__ __forceinline__ void load(const uint16_t* row, int k, int K, bool ok) {
        if (ok && k < K) {
            r0 = *(const bf16x8*)(row + k);
            r1 = *(const bf16x8*)(row + k + 8);
        } else {
            r0 = bf16x8{0, 0, 0, 0, 0, 0, 0, 0};
            r1 = r0;
        }
    }
    __device__ __forceinline__ void cvt(bf16x8& a, bf16x8& b) const {
        a = r0;
        b = r1;
    }
};

// 16 consecutive activations of one row of X starting at k, as bf16 hi (and lo for fp32 X).
template <typename TX> struct XLoad;
template <> struct XLoad<float> {
    static constexpr bool kLo = true;
    f32x4 r[4];
    __device__ __forceinline__ void load(const float* row, int k, int K, bool ok) {
#pragma unroll
        for (int i = 0; i < 4; i++) r[i] = (ok && k < K) ? *(const f32x4*)(row + k + 4 * i) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // x = hi + lo with hi = x truncated to bf16 (exact difference) and lo rounded to bf16:
    // |x - hi - lo| <= 2^-16 |x|
    __device__ __forceinline__ void cvt(bf16x8& ha, bf16x8& hb, bf16x8& la, bf16x8& lb) const {
        uint32_t h[8], l[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float x0 = r[i / 2][2 * (i % 2)], x1 = r[i / 2][2 * (i % 2) + 1];
            h[i] = __builtin_amdgcn_perm(__float_as_uint(x1), __float_as_uint(x0), 0x07060302u);
            typedef float f2 __attribute__((ext_vector_type(2)));
            typedef __bf16 b2 __attribute__((ext_vector_type(2)));
            const f2 lo = {x0 - __uint_as_float(__float_as_uint(x0) & 0xffff0000u),
                           x1 - __uint_as_float(__float_as_uint(x1) & 0xffff0000u)};
            l[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, b2));
        }
        ha = __builtin_bit_cast(bf16x8, *(uint32_t(*)[4])h);
        hb = __builtin_bit_cast(bf16x8, *(uint32_t(*)[4])(h + 4));
        la = __builtin_bit_cast(bf16x8, *(uint32_t(*)[4])l);
        lb = __builtin_bit_cast(bf16x8, *(uint32_t(*)[4])(l + 4));
    }
};
template <> struct XLoad<uint16_t> {
    static constexpr bool kLo = false;
    bf16x8 r0, r1;
    __device__ __forceinline__ void load(const uint16_t* row, int k, int K, bool ok) {
        if (ok && k < K) {
            r0 = *(const bf16x8*)(row + k);
            r1 = *(const bf16x8*)(row + k + 8);
        } else {
            r0 = bf16x8{0, 0, 0, 0, 0, 0, 0, 0};
            r1 = r0;
        }
    }
    __device__ __forceinline__ void cvt(bf16x8& ha, bf16x8& hb, bf16x8&, bf16x8&) const {
        ha = r0;
        hb = r1;
    }
};

// Up to four weight matrices that share X (a layer's input projections) go in one launch;
// segment i owns workgroups [tile0[i], tile0[i+1]) along grid x.
constexpr int MAX_SEG = 4;
struct ProjSeg {
    const void* W;
    const uint16_t* scale;  // per-row scale or null
    float* Y;
    long long ldy;
    int N;
};
struct ProjSegs {
    ProjSeg s[MAX_SEG];
    int tile0[MAX_SEG + 1];
    int n;
};

// One workgroup: rows [n0, n0 + 16 RT) of one segment's W against rows [m0, m0 + 16 MT) of X,
// all of K. grid = (total row tiles of all segments, ceil(M / 16MT)); NWAVE waves split the k
// steps.
template <typename TW, typename TX, int MT, int RT, int NWAVE>
__global__ __launch_bounds__(64 * NWAVE) void proj_skinny_kernel(const TX* __restrict__ X, long long ldx,
                                                                 const ProjSegs segs, int M, int K, int accumulate) {
    __shared__ f32x4 red[NWAVE][RT * MT][WAVE];
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    const int r16 = lane % 16, g = lane / 16;
    int si = 0;
#pragma unroll
    for (int i = 1; i < MAX_SEG; i++)
        if (i < segs.n && (int)blockIdx.x >= segs.tile0[i]) si = i;
    const TW* __restrict__ W = (const TW*)segs.s[si].W;
    const uint16_t* __restrict__ scale = segs.s[si].scale;
    float* __restrict__ Y = segs.s[si].Y;
    const long long ldy = segs.s[si].ldy;
    const int N = segs.s[si].N;
    const int n0 = ((int)blockIdx.x - segs.tile0[si]) * 16 * RT, m0 = blockIdx.y * 16 * MT;

    const TW* wrow[RT];
    bool wok[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int n = n0 + 16 * rt + r16;
        wok[rt] = n < N;
        wrow[rt] = W + (size_t)(wok[rt] ? n : 0) * K;
    }
    const TX* xrow[MT];
    bool xok[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = m0 + 16 * mt + r16;
        xok[mt] = m < M;
        xrow[mt] = X + (size_t)(xok[mt] ? m : 0) * ldx;
    }

    f32x4 acc[RT][MT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[rt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // The epilogue's row scales (and, when accumulating, the old Y values) of the tiles this
    // wave finishes (tile t by wave t % NWAVE) are requested now, so they arrive with the
    // weights instead of costing a round trip at the end.
    // int8 weights (always with row scales): the loads are unconditional and their values are
    // only used in the epilogue (a guarded load whose value is used inside its branch waits for
    // it there, before the weight stream starts; measured 6% at M = 1). Without row scales or
    // accumulation every lane reads one word that the epilogue ignores (one cache line). bf16
    // weights (normally without scales) keep guarded loads, which then issue nothing.
    constexpr bool kEarly = std::is_same<TW, int8_t>::value;
    constexpr int NFIN = (RT * MT + NWAVE - 1) / NWAVE;  // tiles finished per wave, at most
    uint16_t sraw[NFIN][4];
    float fsc[NFIN][4], fy[NFIN][4];
#pragma unroll
    for (int u = 0; u < NFIN; u++) {
        const int t = wave + NWAVE * u, rt = t / MT, mt = t % MT;
        const int m = m0 + 16 * mt + r16;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + 16 * rt + 4 * g + j;
            const bool ok = t < RT * MT && n < N && m < M;
            if constexpr (kEarly) {
                const int nn = ok ? n : 0, mm = ok ? m : 0;
                sraw[u][j] = *(scale ? scale + nn : (const uint16_t*)W);
                fy[u][j] = *(accumulate ? Y + (size_t)mm * ldy + nn : Y);
            } else {
                fsc[u][j] = (ok && scale) ? bf2f(scale[n]) : 1.f;
                fy[u][j] = (ok && accumulate) ? Y[(size_t)m * ldy + n] : 0.f;
            }
        }
    }

    // loads of DEPTH steps are issued together, then consumed: with ~4 steps per wave that is
    // every load of the wave in flight at once
    constexpr int DEPTH = (XLoad<TX>::kLo ? MT * 16 : MT * 8) + RT * 8 <= 32 ? 4 : 2;
    WLoad<TW> wl[DEPTH][RT];
    XLoad<TX> xl[DEPTH][MT];
    auto fetch = [&](int buf, int step) {
        const int k = step * KSTEP + 16 * g;
#pragma unroll
        for (int rt = 0; rt < RT; rt++) wl[buf][rt].load(wrow[rt], k, K, wok[rt]);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) xl[buf][mt].load(xrow[mt], k, K, xok[mt]);
    };
    auto compute = [&](int buf) {
        bf16x8 xa[MT], xb[MT], la[MT], lb[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) xl[buf][mt].cvt(xa[mt], xb[mt], la[mt], lb[mt]);
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            bf16x8 wa, wb;
            wl[buf][rt].cvt(wa, wb);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xa[mt], acc[rt][mt], 0, 0, 0);
                acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb, xb[mt], acc[rt][mt], 0, 0, 0);
                if (XLoad<TX>::kLo) {
                    acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, la[mt], acc[rt][mt], 0, 0, 0);
                    acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb, lb[mt], acc[rt][mt], 0, 0, 0);
                }
            }
        }
    };

    // wave w takes steps w, w + NWAVE, ... (neighbouring waves read neighbouring runs of a row);
    // steps past the end load zeros and are skipped
    // rolling prefetch: a buffer is refilled with the step DEPTH rounds ahead as soon as it has
    // been consumed, so the next round's loads are in flight during this round's MFMAs
    const int nsteps = (K + KSTEP - 1) / KSTEP;
#pragma unroll
    for (int d = 0; d < DEPTH; d++) fetch(d, wave + d * NWAVE);
    for (int s0 = wave; s0 < nsteps; s0 += DEPTH * NWAVE) {
#pragma unroll
        for (int d = 0; d < DEPTH; d++) {
            const int st = s0 + d * NWAVE;
            if (st < nsteps) compute(d);
            const int nx = st + DEPTH * NWAVE;
            if (s0 + DEPTH * NWAVE < nsteps) fetch(d, nx);  // uniform: the next round exists
        }
    }

#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) red[wave][rt * MT + mt][lane] = acc[rt][mt];
    __syncthreads();
    // tile t is finished by wave t % NWAVE: lane holds column m = m0 + 16 mt + r16, rows
    // n 4g .. 4g+3
#pragma unroll
    for (int u = 0; u < NFIN; u++) {
        const int t = wave + NWAVE * u;
        if (t >= RT * MT) break;
        f32x4 v = red[0][t][lane];
#pragma unroll
        for (int w = 1; w < NWAVE; w++) v += red[w][t][lane];
        const int rt = t / MT, mt = t % MT;
        const int m = m0 + 16 * mt + r16;
        if (m >= M) continue;
        float* yrow = Y + (size_t)m * ldy;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + 16 * rt + 4 * g + j;
            if (n >= N) continue;
            if constexpr (kEarly)
                yrow[n] = (accumulate ? fy[u][j] : 0.f) + v[j] * (scale ? bf2f(sraw[u][j]) : 1.f);
            else
                yrow[n] = fy[u][j] + v[j] * fsc[u][j];
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Decode-size bf16 projections (M <= 16) with W staged through LDS. The row-tile pattern above
// (lane = (row, 32-byte run)) reads 16 rows x 128 bytes per pair of load instructions, and the
// DRAM side serves that at ~half the rate of contiguous reads (same box: a read-only kernel
// with that pattern 51% of HBM on 50 MB, 1 KB-contiguous reads 67%). Here every load
// instruction is a direct global -> LDS copy of 1 KB of one pair of W rows (512 bytes each) and
// the MFMA A operands are read back from LDS. Per workgroup: 16 NW rows of W (16 per wave, so
// a wave owns whole output rows and no cross-wave reduction is needed) over all of K, in chunks
// of KC = 256 k through an NS-stage ring (NS = 2 measured best: 3 to 5 stages were 2-50%
// slower); the X rows of each chunk ride in the same stage.
// Slots of 16 bytes in a staged row are XOR-swizzled by the row index (the global address of
// each lane is permuted, the 1 KB it covers is not), so the 16 rows a fragment read touches
// hit 16 different bank groups.
constexpr int SKC = 256;  // k per chunk
template <typename TX, int NW, int NS, int MT = 1>
struct StreamSmem {
    static constexpr int XB = 16 * MT * SKC * sizeof(TX);  // X bytes per stage (16 MT rows)
    __attribute__((aligned(16))) unsigned char w[NS][16 * NW][SKC * 2];
    __attribute__((aligned(16))) unsigned char x[NS][XB];
};

// 16 bytes per lane straight from global memory into LDS at lds + 16 lane (lds uniform). Kept
// in a device function: the builtin in a kernel body keeps the host pass from emitting the
// kernel's launch stub.
__device__ __forceinline__ void g2lds16(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
// The same copy with the nontemporal hint (cache-policy bit 1): the weight stream is read once
// per launch, and kept out of L2 / MALL it runs faster (config 4 decode step 1.637 -> 1.583 ms).
// The row-tile kernel's register loads measured slower with the hint, so they keep plain loads.
__device__ __forceinline__ void g2lds16_nt(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 2);
}

__device__ __forceinline__ void wait_vm(int n) {
    // s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt in bits 3:0
    // and 15:14, expcnt 6:4, lgkmcnt 11:8)
    switch (n) {
#define AEG_W(N) case N: __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8)); break;
        AEG_W(0) AEG_W(1) AEG_W(2) AEG_W(3) AEG_W(4) AEG_W(5) AEG_W(6) AEG_W(7) AEG_W(8) AEG_W(9) AEG_W(10)
        AEG_W(11) AEG_W(12) AEG_W(13) AEG_W(14) AEG_W(15) AEG_W(16) AEG_W(20) AEG_W(24) AEG_W(28) AEG_W(32)
        AEG_W(40) AEG_W(48)
#undef AEG_W
        default: __builtin_amdgcn_s_waitcnt(0);
    }
}

template <typename TX, int NW, int NS, int MT = 1>
__global__ __launch_bounds__(64 * NW) void proj_stream_kernel(const TX* __restrict__ X, long long ldx,
                                                               const ProjSegs segs, int M, int K, int accumulate,
                                                               float* __restrict__ part) {
    static_assert(MT == 1 || sizeof(TX) == 2, "several m tiles take bf16 X only");
    __shared__ StreamSmem<TX, NW, NS, MT> sm;
    constexpr int RW = 16 * NW;                       // W rows per workgroup
    constexpr int WI = RW / 2 / NW;                   // W load instructions per wave per stage (= 8)
    constexpr int XI = StreamSmem<TX, NW, NS, MT>::XB / 1024 / NW;  // X load instructions per wave per stage
    static_assert(XI * NW * 1024 == StreamSmem<TX, NW, NS, MT>::XB, "X stage must split evenly over the waves");
    constexpr int PER = WI + XI;                      // loads per wave per stage
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    const int r16 = lane % 16, g = lane / 16;
    int si = 0;
#pragma unroll
    for (int i = 1; i < MAX_SEG; i++)
        if (i < segs.n && (int)blockIdx.x >= segs.tile0[i]) si = i;
    const uint16_t* __restrict__ W = (const uint16_t*)segs.s[si].W;
    float* __restrict__ Y = segs.s[si].Y;
    const long long ldy = segs.s[si].ldy;
    const int N = segs.s[si].N;
    const int n0 = ((int)blockIdx.x - segs.tile0[si]) * RW;
    // split K (gridDim.y > 1, one weight matrix): chunks [c0, c1) of this workgroup, partial sums
    // to part[blockIdx.y][m][n] (the caller adds the splits in order)
    const int nall = K / SKC, ks = blockIdx.y, nks = gridDim.y;
    const int c0 = ks * nall / nks, c1 = (ks + 1) * nall / nks, nch = c1 - c0;

    // stage loads of chunk c: this wave's WI pairs of W rows and XI kilobytes of X rows
    auto issue = [&](int cc) {
        const int st = cc % NS, c = c0 + cc;
#pragma unroll
        for (int i = 0; i < WI; i++) {
            const int pr = wave * WI + i;             // row pair
            const int row = 2 * pr + lane / 32, slot = (lane % 32) ^ (row & 15);
            const int n = min(n0 + row, N - 1);
            const uint16_t* src = W + (size_t)n * K + (size_t)c * SKC + slot * 8;
            g2lds16_nt(src, &sm.w[st][2 * pr][0]);
        }
        constexpr int XROWB = SKC * (int)sizeof(TX);   // bytes of one X row per chunk
#pragma unroll
        for (int i = 0; i < XI; i++) {
            const int off = (wave * XI + i) * 1024 + lane * 16;  // byte offset in the stage's X block
            const int m = off / XROWB, kb = off % XROWB;
            const int mm = min(m, M - 1);
            const unsigned char* src = (const unsigned char*)(X + (size_t)mm * ldx + (size_t)c * SKC) + kb;
            g2lds16(src, &sm.x[st][(wave * XI + i) * 1024]);
        }
    };

    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NS - 1; c++)
        if (c < nch) issue(c);
    const int row = 16 * wave + r16;  // this lane's W row (A operand)
    for (int c = 0; c < nch; c++) {
        // chunk c's loads are done once only the later chunks' (at most NS - 2) are in flight
        const int later = min(NS - 2, nch - 1 - c);
        wait_vm(later * PER);
        lds_barrier();
        if (c + NS - 1 < nch) issue(c + NS - 1);  // into the stage chunk c - 1 used (all waves are past it)
        const int st = c % NS;
#pragma unroll
        for (int i = 0; i < SKC / 32; i++) {
            // k block i of the chunk: lane (row, g) takes slot 4 i + g of its row (swizzled)
            const bf16x8 a = *(const bf16x8*)&sm.w[st][row][((4 * i + g) ^ (row & 15)) * 16];
            if constexpr (sizeof(TX) == 2) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const bf16x8 b = *(const bf16x8*)&sm.x[st][((16 * mt + r16) * SKC + 32 * i + 8 * g) * 2];
                    acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[mt], 0, 0, 0);
                }
            } else {
                const float* xp = (const float*)&sm.x[st][(r16 * SKC + 32 * i + 8 * g) * 4];
                const f32x4 x0 = *(const f32x4*)xp, x1 = *(const f32x4*)(xp + 4);
                uint32_t h[4], l[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float v0 = e < 2 ? x0[2 * e] : x1[2 * e - 4], v1 = e < 2 ? x0[2 * e + 1] : x1[2 * e - 3];
                    h[e] = __builtin_amdgcn_perm(__float_as_uint(v1), __float_as_uint(v0), 0x07060302u);
                    typedef float f2 __attribute__((ext_vector_type(2)));
                    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
                    const f2 lo = {v0 - __uint_as_float(__float_as_uint(v0) & 0xffff0000u),
                                   v1 - __uint_as_float(__float_as_uint(v1) & 0xffff0000u)};
                    l[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, b2));
                }
                acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, h), acc[0], 0, 0, 0);
                acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, l), acc[0], 0, 0, 0);
            }
        }
    }
    // lane (m = 16 mt + r16, g) of tile mt holds Y[m][n0 + 16 wave + 4 g .. +3]
    const int nb = n0 + 16 * wave + 4 * g;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = 16 * mt + r16;
        if (m >= M || nb >= N) continue;
        if (part) {
            float* pp = part + ((size_t)ks * M + m) * N + nb;
            if (nb + 3 < N && (N % 4) == 0) {
                *(f32x4*)pp = acc[mt];
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (nb + j < N) pp[j] = acc[mt][j];
            }
            continue;
        }
        float* yp = Y + (size_t)m * ldy + nb;
        if (nb + 3 < N && ((uintptr_t)yp % 16) == 0) {
            f32x4 v = acc[mt];
            if (accumulate) v += *(const f32x4*)yp;
            *(f32x4*)yp = v;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (nb + j < N) yp[j] = (accumulate ? yp[j] : 0.f) + acc[mt][j];
        }
    }
}

// Y[m][n] (+)= sum over ks = 0 .. nks - 1, in that order, of part[ks][m][n] (the split-K slices
// of proj_stream_kernel); 4 columns per thread, N % 4 == 0.
__global__ void proj_splitk_reduce_kernel(const float* __restrict__ part, int nks, int M, int N, float* __restrict__ Y,
                                          long long ldy, int accumulate) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, n4 = N / 4;
    if (i >= M * n4) return;
    const int m = i / n4, n = 4 * (i % n4);
    const size_t slice = (size_t)M * N;
    const float* p = part + (size_t)m * N + n;
    f32x4 v = *(const f32x4*)p;
    for (int k = 1; k < nks; k++) v += *(const f32x4*)(p + k * slice);
    float* y = Y + (size_t)m * ldy + n;
    if (((uintptr_t)y % 16) == 0) {
        if (accumulate) v = *(const f32x4*)y + v;
        *(f32x4*)y = v;
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) y[j] = (accumulate ? y[j] : 0.f) + v[j];
    }
}

template <typename TX, int NW, int NS, int MT = 1>
int launch_stream(const TX* X, long long ldx, ProjSegs segs, int M, int K, int accumulate, hipStream_t st,
                  float* part = nullptr, int nks = 1) {
    int t = 0;
    for (int i = 0; i < segs.n; i++) {
        segs.tile0[i] = t;
        t += (segs.s[i].N + 16 * NW - 1) / (16 * NW);
    }
    segs.tile0[segs.n] = t;
    proj_stream_kernel<TX, NW, NS, MT><<<dim3(t, nks), 64 * NW, 0, st>>>(X, ldx, segs, M, K, accumulate, part);
    return 0;
}

template <typename TW, typename TX, int MT, int RT, int NW>
void launch_k(const TX* X, long long ldx, ProjSegs segs, int M, int K, int accumulate, hipStream_t st) {
    int t = 0;
    for (int i = 0; i < segs.n; i++) {
        segs.tile0[i] = t;
        t += (segs.s[i].N + 16 * RT - 1) / (16 * RT);
    }
    segs.tile0[segs.n] = t;
    const dim3 grid(t, (M + 16 * MT - 1) / (16 * MT));
    proj_skinny_kernel<TW, TX, MT, RT, NW><<<grid, 64 * NW, 0, st>>>(X, ldx, segs, M, K, accumulate);
}

// Shape of the launch: about 2048 waves in all (8 per CU, enough loads in flight to cover HBM
// latency) with at least two k steps per wave; two row tiles per wave where that is reachable
// (each activation load then feeds twice the weights), else one.
template <typename TW, typename TX, int MT>
void launch_mt(const TX* X, long long ldx, const ProjSegs& segs, int M, int K, int accumulate, hipStream_t st) {
    const long long gy = (M + 16 * MT - 1) / (16 * MT);
    const int nsteps = (K + KSTEP - 1) / KSTEP;
    long long t2 = 0, t1 = 0;
    for (int i = 0; i < segs.n; i++) {
        t2 += (segs.s[i].N + 31) / 32 * gy;
        t1 += (segs.s[i].N + 15) / 16 * gy;
    }
    constexpr int kTarget = PROJ_TARGET_WAVES;
#define AEG_PROJ(RT, NW) return launch_k<TW, TX, MT, RT, NW>(X, ldx, segs, M, K, accumulate, st)
    if (t2 * 4 >= kTarget) AEG_PROJ(2, 4);
    if (t2 * 8 >= kTarget && nsteps >= 16) AEG_PROJ(2, 8);
    if (t1 * 4 >= kTarget) AEG_PROJ(1, 4);
    if (t1 * 8 >= kTarget || nsteps < 32) {
        if (nsteps >= 16) AEG_PROJ(1, 8);
        AEG_PROJ(1, 4);
    }
    // sixteen waves per workgroup leave 128 registers per lane: one m tile only
    if constexpr (MT == 1) AEG_PROJ(1, 16);
    else AEG_PROJ(1, 8);
#undef AEG_PROJ
}

template <typename TW, typename TX>
int run_proj(const TX* X, long long ldx, const ProjSegs& segs, int M, int K, int accumulate, hipStream_t st) {
    // int8 weights with fp32 activations past 64 rows (the engine's gemm_i8): the tiled GEMM
    if constexpr (std::is_same<TW, int8_t>::value && std::is_same<TX, float>::value) {
        bool ok = M > 64;
        for (int i = 0; i < segs.n && ok; i++) ok = gemm_i8f32_fits(X, ldx, segs.s[i].W, K, M, segs.s[i].N, K);
        if (ok) {
            for (int i = 0; i < segs.n; i++) {
                int rc = launch_gemm_i8f32(X, ldx, (const int8_t*)segs.s[i].W, K, segs.s[i].scale, segs.s[i].Y,
                                           segs.s[i].ldy, M, segs.s[i].N, K, accumulate, st);
                if (rc) return rc;
            }
            return 0;
        }
    }
    // bf16 weights and activations past 64 rows: the tiled MFMA GEMM, all weights in one launch
    // (stacked along N) when each but the last has a multiple of 8 rows, else one launch each
    if constexpr (std::is_same<TW, uint16_t>::value && std::is_same<TX, uint16_t>::value) {
        bool ok = M > 64, stack8 = segs.n <= 3;
        for (int i = 0; i < segs.n && ok; i++) {
            ok = segs.s[i].scale == nullptr && gemm_bf16_fits(X, ldx, segs.s[i].W, K, M, segs.s[i].N, K);
            if (i + 1 < segs.n && segs.s[i].N % 8) stack8 = false;
        }
        if (ok && stack8) {
            const uint16_t* W[MAX_SEG];
            float* Y[MAX_SEG];
            long long ldw[MAX_SEG], ldy[MAX_SEG];
            int N[MAX_SEG];
            for (int i = 0; i < segs.n; i++) {
                W[i] = (const uint16_t*)segs.s[i].W;
                Y[i] = segs.s[i].Y;
                ldw[i] = K;
                ldy[i] = segs.s[i].ldy;
                N[i] = segs.s[i].N;
            }
            return launch_gemm_bf16_multi(X, ldx, segs.n, W, ldw, Y, ldy, N, M, K, accumulate, st);
        }
        if (ok) {
            for (int i = 0; i < segs.n; i++) {
                int rc = launch_gemm_bf16(X, ldx, (const uint16_t*)segs.s[i].W, K, segs.s[i].Y, segs.s[i].ldy, M,
                                          segs.s[i].N, K, accumulate, st);
                if (rc) return rc;
            }
            return 0;
        }
    }
    // bf16 weights at M <= 16 with K a multiple of the chunk, no row scales: the LDS-staged stream
    if constexpr (std::is_same<TW, uint16_t>::value) {
        bool scaled = false;
        for (int i = 0; i < segs.n; i++) scaled |= segs.s[i].scale != nullptr;
        // ... when it takes more than one workgroup per CU: at <= 256 workgroups (N <= 8192) the
        // row-tile kernel below, with its K split over the waves of a workgroup, keeps more loads
        // in flight (8192 x 2048: 10.9 against 11.7 us; 2048 x 4096: 10.5 against 14.9 us), and
        // above it the row-tile kernel's 8-wave workgroups need a second round on part of the
        // CUs (9216 x 2048: 16.3 against 12.8 us; 12352 x 2048: 16.9 against 13.3 us)
        long long tiles = 0;
        for (int i = 0; i < segs.n; i++) tiles += (segs.s[i].N + 31) / 32;
        if (M <= 16 && K % SKC == 0 && !scaled && tiles > 256 && stream_enabled()) {
            launch_stream<TX, 2, 2>(X, ldx, segs, M, K, accumulate, st);
            return after_launch("proj_stream");
        }
        // 17..64 rows of bf16 X and one weight whose rows give too few workgroups (2048 x 4096:
        // 64 workgroups of 32 rows): the same stream with all the rows' X staged once per chunk,
        // split over K into ~256 workgroups when the calling thread has bound a workspace for
        // the fp32 partials, which a second launch adds in slice order (deterministic). Measured
        // at M = 64: 2048 x 4096 21.2 -> 13.7 us; with enough rows (8192 x 2048 and the stack's
        // grouped input projections) the row-tile kernel below is as fast, so it keeps them.
        if constexpr (std::is_same<TX, uint16_t>::value) {
            const long long t = (segs.s[0].N + 31) / 32;
            if (M > 16 && M <= 64 && K % SKC == 0 && !scaled && segs.n == 1 && t < 192 && segs.s[0].N % 4 == 0 &&
                stream_enabled()) {
                const int nks = (int)std::min<long long>(K / SKC, (256 + t - 1) / t);
                size_t bound = 0;
                void* ws = bound_workspace(&bound);
                if (nks > 1 && ws && bound >= (size_t)nks * M * segs.s[0].N * 4) {
                    float* part = (float*)ws;
                    if (M <= 32) launch_stream<TX, 2, 2, 2>(X, ldx, segs, M, K, accumulate, st, part, nks);
                    else launch_stream<TX, 2, 2, 4>(X, ldx, segs, M, K, accumulate, st, part, nks);
                    int rc = after_launch("proj_stream64");
                    if (rc) return rc;
                    const ProjSeg& sg = segs.s[0];
                    const int nthr = M * (sg.N / 4);
                    proj_splitk_reduce_kernel<<<(nthr + 255) / 256, 256, 0, st>>>(part, nks, M, sg.N, sg.Y, sg.ldy,
                                                                                 accumulate);
                    return after_launch("proj_splitk_reduce");
                }
            }
        }
    }
    // m tiles per workgroup: the whole batch up to 64 rows of bf16 X (32 of fp32 X, whose hi/lo
    // operands take twice the registers), so the weights are read once; larger M is covered by
    // a grid of row groups
    if (M <= 16) {
        launch_mt<TW, TX, 1>(X, ldx, segs, M, K, accumulate, st);
    } else if constexpr (XLoad<TX>::kLo) {
        launch_mt<TW, TX, 2>(X, ldx, segs, M, K, accumulate, st);
    } else {
        if (M <= 32) launch_mt<TW, TX, 2>(X, ldx, segs, M, K, accumulate, st);
        else if (M <= 48) launch_mt<TW, TX, 3>(X, ldx, segs, M, K, accumulate, st);
        else launch_mt<TW, TX, 4>(X, ldx, segs, M, K, accumulate, st);
    }
    return after_launch("proj_skinny");
}

}  // namespace

namespace aegist {

// Y_i[m, n] (+)= scale_i[n] * sum_k X[m, k] W_i[n, k] for nseg (<= 4) weight matrices sharing X.
int launch_proj_multi(const void* X, int x_dtype, long long ldx, int w_dtype, int nseg, const void* const* W,
                      const uint16_t* const* scale, float* const* Y, const long long* ldy, const int* N, int M, int K,
                      int accumulate, hipStream_t st) {
    if (nseg < 1 || nseg > MAX_SEG) return fail(AEGIST_ERR_SHAPE, "proj: 1 to 4 weight matrices per launch");
    if (M < 0 || K < 0) return fail(AEGIST_ERR_SHAPE, "proj: negative size");
    if (K % 16) return fail(AEGIST_ERR_SHAPE, "proj: K must be a multiple of 16");
    const int xs = x_dtype == AEGIST_F32 ? 4 : 2;
    if (ldx < K || (ldx * xs) % 16 || (uintptr_t)X % 16)
        return fail(AEGIST_ERR_SHAPE, "proj: X needs 16-byte aligned rows (ldx >= K)");
    ProjSegs segs{};
    for (int i = 0; i < nseg; i++) {
        if (N[i] < 0) return fail(AEGIST_ERR_SHAPE, "proj: negative size");
        if (N[i] == 0) continue;
        if (ldy[i] < N[i]) return fail(AEGIST_ERR_SHAPE, "proj: ldy < N");
        if ((uintptr_t)W[i] % 16) return fail(AEGIST_ERR_SHAPE, "proj: W needs 16-byte aligned rows");
        segs.s[segs.n++] = ProjSeg{W[i], scale ? scale[i] : nullptr, Y[i], ldy[i], N[i]};
    }
    if (M == 0 || segs.n == 0) return 0;
    if (w_dtype == AEGIST_I8 && x_dtype == AEGIST_F32) return run_proj<int8_t, float>((const float*)X, ldx, segs, M, K, accumulate, st);
    if (w_dtype == AEGIST_I8 && x_dtype == AEGIST_BF16)
        return run_proj<int8_t, uint16_t>((const uint16_t*)X, ldx, segs, M, K, accumulate, st);
    if (w_dtype == AEGIST_BF16 && x_dtype == AEGIST_F32)
        return run_proj<uint16_t, float>((const float*)X, ldx, segs, M, K, accumulate, st);
    if (w_dtype == AEGIST_BF16 && x_dtype == AEGIST_BF16)
        return run_proj<uint16_t, uint16_t>((const uint16_t*)X, ldx, segs, M, K, accumulate, st);
    return fail(AEGIST_ERR_DTYPE, "proj: W must be AEGIST_I8 or AEGIST_BF16, X AEGIST_F32 or AEGIST_BF16");
}

// Split-K form for decode sizes: part[ks][m][n] = sum over the ks-th of nks slices of K of
// X[m, k] W[n, k] (bf16 X and W, M <= 16, K a multiple of 256 with at least nks chunks). The
// caller adds the nks slices in order (the layer stack does it inside the next ZNorm).
int launch_proj_splitk(const uint16_t* X, long long ldx, const uint16_t* W, float* part, int nks, int M, int N, int K,
                       hipStream_t st) {
    if (M < 1 || M > 16 || N < 1 || K % SKC || K / SKC < nks || nks < 1 || ldx < K || ldx % 8 || (uintptr_t)X % 16 ||
        (uintptr_t)W % 16)
        return fail(AEGIST_ERR_SHAPE, "proj_splitk: need M <= 16, K % 256 == 0, K / 256 >= splits, aligned rows");
    ProjSegs segs{};
    segs.s[0] = ProjSeg{W, nullptr, part, N, N};
    segs.n = 1;
    launch_stream<uint16_t, 2, 2>(X, ldx, segs, M, K, 0, st, part, nks);
    return after_launch("proj_stream_splitk");
}

int launch_proj(const void* X, int x_dtype, long long ldx, const void* W, int w_dtype, const uint16_t* scale, float* Y,
                long long ldy, int M, int N, int K, int accumulate, hipStream_t st) {
    return launch_proj_multi(X, x_dtype, ldx, w_dtype, 1, &W, &scale, &Y, &ldy, &N, M, K, accumulate, st);
}

}  // namespace aegist

extern "C" int aegist_gemv_i8(const float* x, const int8_t* W, const uint16_t* scale, float* y, int N, int K,
                              int accumulate, void* stream) {
    return launch_proj(x, AEGIST_F32, K, W, AEGIST_I8, scale, y, N, 1, N, K, accumulate, AEG_STREAM(stream));
}

extern "C" int aegist_gemv_bf16(const float* x, const uint16_t* W, float* y, int N, int K, void* stream) {
    return launch_proj(x, AEGIST_F32, K, W, AEGIST_BF16, nullptr, y, N, 1, N, K, 0, AEG_STREAM(stream));
}

extern "C" int aegist_gemm_i8(const float* X, const int8_t* W, const uint16_t* scale, float* Y, int M, int N, int K,
                              int accumulate, void* stream) {
    return launch_proj(X, AEGIST_F32, K, W, AEGIST_I8, scale, Y, N, M, N, K, accumulate, AEG_STREAM(stream));
}

extern "C" int aegist_linear(const void* X, int x_dtype, long long ldx, const void* W, int w_dtype,
                             const uint16_t* scale, float* Y, long long ldy, int M, int N, int K, int accumulate,
                             void* stream) {
    return launch_proj(X, x_dtype, ldx, W, w_dtype, scale, Y, ldy, M, N, K, accumulate, AEG_STREAM(stream));
}

extern "C" int aegist_linear_multi(const void* X, int x_dtype, long long ldx, int w_dtype, int n, const void* const* W,
                                   const uint16_t* const* scale, float* const* Y, const long long* ldy, const int* N,
                                   int M, int K, int accumulate, void* stream) {
    if (!W || !Y || !ldy || !N) return fail(AEGIST_ERR_SHAPE, "linear_multi: null argument array");
    return launch_proj_multi(X, x_dtype, ldx, w_dtype, n, W, scale, Y, ldy, N, M, K, accumulate, AEG_STREAM(stream));
}
