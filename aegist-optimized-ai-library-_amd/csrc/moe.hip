// Mixture-of-experts block for gfx950: router top-k, device-side grouping of the picks by
// expert, and the 4-bit SwiGLU experts on MFMA.
//
// Semantics (aegist/hybrid.py):
//   route        MoE.route :637-641          logits = h W_r^T; p = softmax(logits) in fp32; the K
//                                             largest (ties to the lower expert, hybrid.cu:35);
//                                             weights p / sum(top p)
//   experts      ExpertBank.forward :608-628 per pick: y = W_dn (silu(W_g h) * (W_u h)) * weight
//   dequantise   q4_dequantize :463-469       w = code * scale + min per 64-value group, codes
//                                             packed two per byte, even index in the low nibble
//   layout       expert_layout :472-482       [gu_q 2I x D/2 | gu_s 2I x D/64 f16 | gu_m | dn_q
//                                             D x I/2 | dn_s D x I/64 f16 | dn_m]
//   combine      MoE.forward :647-652         x += sum_k y_k + sigmoid(h . w_sg) * shared(h)
// Engine counterparts: router_topk hybrid.cu:317-362, moe_gu_* / moe_dn_* :386-558,
// moe_reduce :560-567, shared_gate_add :569-577; the host grouping of hybrid.rs:875-913 runs on
// the device here (no host sync per layer).
//
// Expert products on MFMA, exactly in the reference's fp32 sense: a 4-bit code c becomes the
// bf16 bit pattern 0x4300 | c = 128 + c (exact), the activations enter as bf16 hi + lo (~16
// significant bits), and per 64-value group the fp32 result is
//   y += s * (sum (128 + c)(x_hi + x_lo)) + (m - 128 s) * sum (x_hi + x_lo),
// i.e. s * sum c x + m * sum x with the scale and min applied per group in fp32.
// A dword of 8 codes (code j in bits 4j) yields the bf16 pairs (c0,c4) (c1,c5) (c2,c6)
// (c3,c7) with one and-or each, so the activations are stored in the same order within every
// 8-value chunk: x'[8q + 2j] = x[8q + j], x'[8q + 2j + 1] = x[8q + j + 4].
#include "common.h"

#include <algorithm>

namespace aegist {
int launch_proj(const void* X, int x_dtype, long long ldx, const void* W, int w_dtype, const uint16_t* scale, float* Y,
                long long ldy, int M, int N, int K, int accumulate, hipStream_t st);
}  // namespace aegist

using namespace aegist;

namespace {

constexpr int PB = 32;            // picks per expert tile (two 16-column MFMA tiles)
constexpr int PBB = 64;           // picks per big (prefill) tile: four 16-column MFMA tiles
constexpr int RB = 64;            // output rows per workgroup (4 waves x 16)
constexpr int MAX_E = 1024;       // experts per layer the grouping kernel handles

struct MoeTile {                  // one block of <= PB grouped picks of one expert
    unsigned long long base;      // the expert's row address (resolved from the pointer table)
    int p0, p1;                   // grouped positions [p0, p1)
};

struct ExpertOffsets {            // byte offsets inside one expert row (expert_layout)
    long long gu_s, gu_m, dn_q, dn_s, dn_m;
};
static ExpertOffsets expert_offsets(int D, int I) {
    ExpertOffsets o;
    o.gu_s = (long long)2 * I * (D / 2);
    o.gu_m = o.gu_s + (long long)2 * I * (D / 64) * 2;
    o.dn_q = o.gu_m + (long long)2 * I * (D / 64) * 2;
    o.dn_s = o.dn_q + (long long)D * (I / 2);
    o.dn_m = o.dn_s + (long long)D * (I / 64) * 2;
    return o;
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Loads through expert-row addresses taken from the pointer table: the compiler cannot tell
// those are global memory and would emit flat loads, which also count against the LDS wait
// counter (every LDS wait would then drain the prefetched code stream). Global address space.
template <typename T>
__device__ __forceinline__ T ld_global(const void* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}

// ---------------------------------------------------------------------------------------------
// Router top-K over precomputed logits [T, E] (the projection kernel computes h W^T): one wave
// per token, lane holds the probabilities of experts lane + 64 i in registers; softmax in fp32;
// K rounds of a wave argmax that prefers the lower expert on equal probabilities.
template <int NPER>  // experts per lane held in registers (E <= 64 NPER)
__global__ void __launch_bounds__(256) router_topk_kernel(const float* __restrict__ logits, int* __restrict__ idx,
                                                          float* __restrict__ wts, int T, int E, int K) {
    const int lane = threadIdx.x % WAVE, t = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    if (t >= T) return;
    const float* l = logits + (size_t)t * E;
    float p[NPER];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPER; i++) {
        const int e = lane + WAVE * i;
        p[i] = e < E ? l[e] : -INFINITY;
        m = fmaxf(m, p[i]);
    }
    m = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NPER; i++) {
        p[i] = lane + WAVE * i < E ? expf(p[i] - m) : 0.f;
        s += p[i];
    }
    s = wave_sum(s);
#pragma unroll
    for (int i = 0; i < NPER; i++) p[i] = lane + WAVE * i < E ? p[i] / s : -1.f;  // -1: not an expert
    float sel = 0.f;  // sum of the picked probabilities
    float myv = 0.f;  // lane k keeps pick k
    int mye = 0;
    for (int k = 0; k < K; k++) {
        float bv = -1.f;
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < NPER; i++)  // experts in increasing order: the first of equals wins
            if (p[i] > bv) {
                bv = p[i];
                bi = lane + WAVE * i;
            }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float v2 = __shfl_xor(bv, o, WAVE);
            const int i2 = __shfl_xor(bi, o, WAVE);
            if (v2 > bv || (v2 == bv && i2 < bi)) {
                bv = v2;
                bi = i2;
            }
        }
#pragma unroll
        for (int i = 0; i < NPER; i++)
            if (bi == lane + WAVE * i) p[i] = -2.f;  // taken
        if (lane == k) {
            myv = bv;
            mye = bi;
        }
        sel += bv;
    }
    if (lane < K) {
        idx[(size_t)t * K + lane] = mye;
        wts[(size_t)t * K + lane] = myv / sel;
    }
}

// ---------------------------------------------------------------------------------------------
// Grouping (one workgroup of 1024 threads): picks i = t K + k with expert idx[i]; out of range
// experts are dropped and counted. eoff[E + 1]: exclusive prefix of the counts; ptok / psrc:
// token and pick index of each grouped position. An expert's positions are cut into blocks
// (moe_group_kernel): blocks of <= 16 positions go to tiles1 (meta[0] of them), of 17..32 to
// tiles2 (meta[2]), of up to 64 to tiles3 (meta[3]), as (expert, p0, p1). meta[1] = dropped
// picks. The order of positions inside an expert is unspecified (atomics); no result depends on
// it (every pick's sums run in the same order whatever tile it lands in with whom).
__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int* total) {
    const int lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE, nw = blockDim.x / WAVE;
    int x = v;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const int y = __shfl_up(x, d, WAVE);
        if (lane >= d) x += y;
    }
    if (lane == WAVE - 1) wsum[w] = x;
    __syncthreads();
    int off = 0, tot = 0;
    for (int i = 0; i < nw; i++) {
        if (i < w) off += wsum[i];
        tot += wsum[i];
    }
    __syncthreads();
    *total = tot;
    return off + x - v;
}

// Tiles: with `big3` set, an expert with more than 32 picks has them all in ceil(c / 64) blocks
// of balanced size (tiles3, 33..64 picks each but for c = 65..95: 32..48); otherwise blocks of
// PB = 32 (tiles2) and a last one of <= 16 (tiles1).
__global__ void __launch_bounds__(1024) moe_group_kernel(const int* __restrict__ idx, int N, int K, int E,
                                                         const unsigned long long* __restrict__ eptr,
                                                         int* __restrict__ eoff, int* __restrict__ ptok,
                                                         int* __restrict__ psrc, MoeTile* __restrict__ tiles1,
                                                         MoeTile* __restrict__ tiles2, MoeTile* __restrict__ tiles3,
                                                         int big3, int* __restrict__ meta) {
    __shared__ int cnt[MAX_E], cur[MAX_E], wsum[16], bad;
    const int tid = threadIdx.x;
    for (int e = tid; e < MAX_E; e += blockDim.x) cnt[e] = 0;
    if (tid == 0) bad = 0;
    __syncthreads();
    for (int i = tid; i < N; i += blockDim.x) {
        const int e = idx[i];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
        else atomicAdd(&bad, 1);
    }
    __syncthreads();
    const int c = tid < E ? cnt[tid] : 0;
    const int n3 = big3 && c > 32 ? (c + PBB - 1) / PBB : 0;
    const int c3 = n3 > 0 ? c : 0, cr = c - c3, rem = cr % PB;
    const int small = rem > 0 && rem <= 16 ? 1 : 0;      // the last block, if it is small
    const int big = cr / PB + (rem > 16 ? 1 : 0);        // full blocks and a large last block
    int tot_c, tot_1, tot_2, tot_3;
    const int off = block_excl_scan(c, wsum, &tot_c);
    const int off1 = block_excl_scan(small, wsum, &tot_1);
    const int off2 = block_excl_scan(big, wsum, &tot_2);
    const int off3 = block_excl_scan(n3, wsum, &tot_3);
    if (tid < E) {
        eoff[tid] = off;
        cur[tid] = off;
        const unsigned long long base = c > 0 ? eptr[tid] : 0ull;
        for (int j = 0; j < n3; j++) tiles3[off3 + j] = MoeTile{base, off + c3 * j / n3, off + c3 * (j + 1) / n3};
        for (int j = 0; j < big; j++)
            tiles2[off2 + j] = MoeTile{base, off + c3 + j * PB, off + c3 + min(cr, (j + 1) * PB)};
        if (small) tiles1[off1] = MoeTile{base, off + c - rem, off + c};
    }
    if (tid == 0) {
        eoff[E] = tot_c;
        meta[0] = tot_1;
        meta[1] = bad;
        meta[2] = tot_2;
        meta[3] = tot_3;
    }
    __syncthreads();
    for (int i = tid; i < N; i += blockDim.x) {
        const int e = idx[i];
        if (e < 0 || e >= E) continue;
        const int pos = atomicAdd(&cur[e], 1);
        ptok[pos] = i / K;
        psrc[pos] = i;
    }
}

// ---------------------------------------------------------------------------------------------
// Activations for the expert products: xh / xl [rows][D] bf16 (hi truncated, lo = rounded
// remainder) in the chunk order above, xs [rows][D / 64] = sum over the group of (hi + lo).
// One thread per 8-value chunk; 8 threads of a 64-group reduce their sums by shuffles.
__device__ __forceinline__ void split8(const float* v, uint4& hi, uint4& lo, float& sum) {
    // element order within the chunk: v0 v4 v1 v5 v2 v6 v3 v7
    uint32_t H[4], L[4];
    sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float a = v[j], b = v[j + 4];
        const uint32_t ua = __float_as_uint(a) & 0xffff0000u, ub = __float_as_uint(b) & 0xffff0000u;
        const float ra = a - __uint_as_float(ua), rb = b - __uint_as_float(ub);
        typedef float f2 __attribute__((ext_vector_type(2)));
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        const uint32_t lp = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{ra, rb}), b2));
        H[j] = (ua >> 16) | ub;
        L[j] = lp;
        sum += (__uint_as_float(ua) + bf_lo(lp)) + (__uint_as_float(ub) + bf_hi(lp));
    }
    hi = uint4{H[0], H[1], H[2], H[3]};
    lo = uint4{L[0], L[1], L[2], L[3]};
}

__global__ void __launch_bounds__(256) moe_xprep_kernel(const float* __restrict__ h, int T, int D,
                                                        uint16_t* __restrict__ xh, uint16_t* __restrict__ xl,
                                                        float* __restrict__ xs) {
    const long long q = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // chunk index
    const long long nq = (long long)T * (D / 8);
    const bool ok = q < nq;
    const long long qq = ok ? q : nq - 1;
    const float* src = h + qq * 8;
    const float4 a = ((const float4*)src)[0], b = ((const float4*)src)[1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint4 hi, lo;
    float s;
    split8(v, hi, lo, s);
    s += __shfl_xor(s, 1, WAVE);
    s += __shfl_xor(s, 2, WAVE);
    s += __shfl_xor(s, 4, WAVE);
    if (!ok) return;
    ((uint4*)xh)[qq] = hi;
    ((uint4*)xl)[qq] = lo;
    if ((qq & 7) == 0) xs[qq / 8] = s;
}

// bf16 pairs (c_j, c_{j+4}) + 128 from a dword of 8 4-bit codes
__device__ __forceinline__ bf16x8 codes_bf16(uint32_t p) {
    const uint32_t d0 = (p & 0x000F000Fu) | 0x43004300u;
    const uint32_t d1 = ((p >> 4) & 0x000F000Fu) | 0x43004300u;
    const uint32_t d2 = ((p >> 8) & 0x000F000Fu) | 0x43004300u;
    const uint32_t d3 = ((p >> 12) & 0x000F000Fu) | 0x43004300u;
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(bf16x8, (u4v{d0, d1, d2, d3}));
}
__device__ __forceinline__ bf16x8 ld_bf8(const uint16_t* p) { return *(const bf16x8*)p; }
__device__ __forceinline__ f32x4 mfma_bf(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------------
// One expert matrix block (NM = 1 or 2 matrices sharing the activations; RB = 64 rows each)
// times a tile of <= 16 NT picks. The 64-groups are split over the 4 waves (wave w takes
// groups w, w + 4, ...), so each activation fragment is read once per workgroup; every wave
// covers all 64 rows as 4 row tiles and the waves' partial sums are added in LDS afterwards.
// Lane (n, g) accumulates rows 16 rt + 4g + j (j < 4) for picks 16 t + n. Per 64-group a lane
// holds the 16 codes [64 grp + 16 g, +16) of its row (one 8-byte load): dword ks feeds the
// MFMA of step ks, so each MFMA's 32 codes (8 per lane group) lie in one group; the
// activations are read at the same k. Codes stream through a register ring (the HBM stream),
// activations through a 2-slot ring.
constexpr int RTL = RB / 16;  // row tiles per wave

template <int NM, int NT>
struct BlockAcc {
    f32x4 acc[NM][RTL][NT];
};

// `stage` fills sc and gs (LDS); it runs after this wave's first code and activation loads are
// issued, so its global round trip overlaps theirs, and is followed by the workgroup barrier.
template <int NM, int NT, typename Stage>
__device__ __forceinline__ void expert_block(const unsigned char* __restrict__ qbase, const long long* qrow0, int Kdim,
                                             const float2* sc, const uint16_t* __restrict__ xh,
                                             const uint16_t* __restrict__ xl, const long long* xrow, const float* gs,
                                             BlockAcc<NM, NT>& out, int ngroups, Stage stage) {
    // groups of codes in flight per lane (per row tile and matrix): two for decode-sized tiles,
    // where the weight stream is the whole cost; one for two pick tiles (register budget)
    constexpr int PD = NT == 1 ? 2 : 1;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, n = lane % 16, g = lane / 16;
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int rt = 0; rt < RTL; rt++)
#pragma unroll
            for (int t = 0; t < NT; t++) out.acc[m][rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int nmine = ngroups > wave ? (ngroups - wave + 3) / 4 : 0;  // this wave's groups
    if (nmine == 0) {
        stage();
        __syncthreads();
        return;
    }
    const size_t rowbytes = Kdim / 2;
    const unsigned char* arow[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) arow[m] = qbase + (size_t)(qrow0[m] + n) * rowbytes + 8 * g;
    auto gaddr = [&](int i) { return 32 * (wave + 4 * min(i, nmine - 1)); };  // byte offset of my i-th group
    typedef uint32_t u2v __attribute__((ext_vector_type(2)));
    u2v ar[NM][RTL][PD];
#pragma unroll
    for (int u = 0; u < PD; u++)
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int rt = 0; rt < RTL; rt++) ar[m][rt][u] = ld_global<u2v>(arow[m] + 16 * rt * rowbytes + gaddr(u));
    constexpr int NB = NT == 1 ? 2 : 1;  // activation slots (prefetched a group ahead for one tile)
    bf16x8 bh[NB][NT][2], bl[NB][NT][2];  // [slot][tile][ks]
#define AEG_LOAD_B(slot, grp)                                                  \
    _Pragma("unroll") for (int t = 0; t < NT; t++)                             \
        _Pragma("unroll") for (int ks = 0; ks < 2; ks++) {                     \
            const long long k0 = xrow[t] + 64 * (grp) + 16 * g + 8 * ks;       \
            bh[slot][t][ks] = ld_bf8(xh + k0);                                 \
            bl[slot][t][ks] = ld_bf8(xl + k0);                                 \
        }
    AEG_LOAD_B(0, wave)
    stage();
    __syncthreads();
    for (int i0 = 0; i0 < nmine; i0 += PD) {
#pragma unroll
        for (int u = 0; u < PD; u++) {
            const int i = i0 + u;
            if (i >= nmine) break;
            const int grp = wave + 4 * i, slot = NB == 2 ? (u & 1) : 0;
            if constexpr (NB == 2) {
                if (i + 1 < nmine) {
                    AEG_LOAD_B((slot ^ 1), grp + 4)
                }
            } else if (i > 0) {
                AEG_LOAD_B(0, grp)
            }
            float X[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) X[t] = gs[(16 * t + n) * ngroups + grp];
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int rt = 0; rt < RTL; rt++) {
                    const u2v a2 = ar[m][rt][u];
                    // refill this ring slot with my group PD ahead (clamped: static wait counts)
                    ar[m][rt][u] = ld_global<u2v>(arow[m] + 16 * rt * rowbytes + gaddr(i + PD));
                    f32x4 P[NT];
#pragma unroll
                    for (int t = 0; t < NT; t++) P[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int ks = 0; ks < 2; ks++) {
                        const bf16x8 a = codes_bf16(ks ? a2.y : a2.x);
#pragma unroll
                        for (int t = 0; t < NT; t++) {
                            P[t] = mfma_bf(a, bh[slot][t][ks], P[t]);
                            P[t] = mfma_bf(a, bl[slot][t][ks], P[t]);
                        }
                    }
                    // y += s P + (m - 128 s) X for this row tile's rows and every pick tile
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float2 sm = sc[(m * RB + 16 * rt + 4 * g + j) * ngroups + grp];
#pragma unroll
                        for (int t = 0; t < NT; t++)
                            out.acc[m][rt][t][j] = fmaf(sm.x, P[t][j], fmaf(sm.y, X[t], out.acc[m][rt][t][j]));
                    }
                }
        }
    }
#undef AEG_LOAD_B
}

// Sum the 4 waves' partials of matrix m into red[pick][row] (row < RB), in wave order (the
// result does not depend on scheduling). red has PB rows of RB + 1 floats.
template <int NM, int NT>
__device__ __forceinline__ void reduce_waves(const BlockAcc<NM, NT>& a, int m, float (*red)[RB + 1]) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, n = lane % 16, g = lane / 16;
    for (int w = 0; w < 4; w++) {
        if (wave == w) {
#pragma unroll
            for (int rt = 0; rt < RTL; rt++)
#pragma unroll
                for (int t = 0; t < NT; t++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        float& r = red[16 * t + n][16 * rt + 4 * g + j];
                        r = (w == 0 ? 0.f : r) + a.acc[m][rt][t][j];
                    }
        }
        __syncthreads();
    }
}

// Stage (s, m - 128 s) of rows [row0, row0 + RB) x groups [0, G) of one matrix into sc[RB][G]:
// the block's scale and min entries are one contiguous run of RB G halves each, read as 16-byte
// pieces (8 per load), all loads of a thread issued before any is used.
__device__ __forceinline__ void stage_scales(float2* sc, const uint16_t* __restrict__ s,
                                             const uint16_t* __restrict__ mn, long long row0, int G) {
    const uint16_t* s0 = s + (size_t)row0 * G;
    const uint16_t* m0 = mn + (size_t)row0 * G;
    const int n8 = RB * G / 8;  // 16-byte pieces (RB G is a multiple of 8: G = K / 64, RB = 64)
    constexpr int MAXP = RB * 64 / 8 / 256;  // pieces per thread at the largest G (64)
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    u4v sv[MAXP], mv[MAXP];
#pragma unroll
    for (int u = 0; u < MAXP; u++) {
        const int i = threadIdx.x + 256 * u;
        if (i < n8) {
            sv[u] = ld_global<u4v>(s0 + 8 * i);
            mv[u] = ld_global<u4v>(m0 + 8 * i);
        }
    }
#pragma unroll
    for (int u = 0; u < MAXP; u++) {
        const int i = threadIdx.x + 256 * u;
        if (i < n8) {
            const uint32_t sw[4] = {sv[u].x, sv[u].y, sv[u].z, sv[u].w}, mw[4] = {mv[u].x, mv[u].y, mv[u].z, mv[u].w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float a = h2f((uint16_t)(sw[e / 2] >> (16 * (e & 1)))), b = h2f((uint16_t)(mw[e / 2] >> (16 * (e & 1))));
                sc[8 * i + e] = float2{a, b - 128.f * a};
            }
        }
    }
}

// Stage the activation group sums of the tile's picks: gs[pr][c] = src[row(pr) G + c] for
// pr < PB (rows past the tile repeat its last pick), all loads issued first.
__device__ __forceinline__ void stage_gsums(float* gs, const float* __restrict__ src, const int* __restrict__ rowmap,
                                            int p0, int np, int G) {
    constexpr int MAXP = PB * 64 / 256;
    float v[MAXP];
#pragma unroll
    for (int u = 0; u < MAXP; u++) {
        const int i = threadIdx.x + 256 * u;
        if (i < PB * G) {
            const int pr = i / G, c = i % G, p = p0 + min(pr, np - 1);
            v[u] = src[(size_t)(rowmap ? rowmap[p] : p) * G + c];
        }
    }
#pragma unroll
    for (int u = 0; u < MAXP; u++) {
        const int i = threadIdx.x + 256 * u;
        if (i < PB * G) gs[i] = v[u];
    }
}

// Gate / up: block (unit block ub of RB units) x tile. act[p][r] = silu(gate_r . x) * (up_r . x)
// for the tile's picks, stored as bf16 hi / lo in chunk order (ah, al [P][I]) with group sums
// as [P][I / 64] (the unit block is one 64-group of the down projection's input).
// Grid (I / RB unit blocks, tile-list capacity); the tile count and the tile record are read
// together, and the record carries the expert's row address (no pointer-table round trip).
template <int NT>  // pick tiles of 16: 1 for tiles of <= 16 picks, 2 for larger ones
__global__ void __launch_bounds__(256, 2) moe_gate_up_kernel(const MoeTile* __restrict__ tiles,
                                                          const int* __restrict__ ntiles,
                                                          const int* __restrict__ ptok, const uint16_t* __restrict__ xh,
                                                          const uint16_t* __restrict__ xl, const float* __restrict__ xs,
                                                          int D, int I, ExpertOffsets off, uint16_t* __restrict__ ah,
                                                          uint16_t* __restrict__ al, float* __restrict__ as) {
    // dynamic LDS: sc [2][RB][G] (s, m - 128 s) | gs [PB][G] activation group sums
    extern __shared__ float2 dyn[];
    __shared__ float ob[PB][RB + 1];     // gate sums, then act
    __shared__ float ub2[PB][RB + 1];    // up sums
    const int ub = blockIdx.x, tile = blockIdx.y;
    const MoeTile tl = tiles[tile];  // read before the count is known (capacity-sized list)
    if (tile >= *ntiles) return;
    const int G = D / 64, r0 = ub * RB;
    float2* sc = dyn;
    float* gs = (float*)(dyn + 2 * RB * G);
    const int p0 = tl.p0, np = tl.p1 - tl.p0;
    const unsigned char* base = (const unsigned char*)tl.base;
    auto stage = [&]() {
        stage_scales(sc, (const uint16_t*)(base + off.gu_s), (const uint16_t*)(base + off.gu_m), r0, G);
        stage_scales(sc + RB * G, (const uint16_t*)(base + off.gu_s), (const uint16_t*)(base + off.gu_m), I + r0, G);
        stage_gsums(gs, xs, ptok, p0, np, G);
    };
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE, n = lane % 16, g = lane / 16;
    long long xrow[2];
#pragma unroll
    for (int t = 0; t < 2; t++) xrow[t] = (long long)ptok[p0 + min(16 * t + n, np - 1)] * D;
    const long long qrow0[2] = {r0, I + r0};  // gate rows, up rows of this unit block
    BlockAcc<2, NT> acc;
    expert_block<2, NT>(base, qrow0, D, sc, xh, xl, xrow, gs, acc, G, stage);
    reduce_waves<2, NT>(acc, 0, ob);   // gate sums
    reduce_waves<2, NT>(acc, 1, ub2);  // up sums
    // 256 threads = 32 picks x 8 chunks of the 64 units
    const int pr = threadIdx.x / 8, q = threadIdx.x % 8;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = silu_f(ob[pr][8 * q + i]) * ub2[pr][8 * q + i];
    uint4 hi, lo;
    float s;
    split8(v, hi, lo, s);
    s += __shfl_xor(s, 1, WAVE);
    s += __shfl_xor(s, 2, WAVE);
    s += __shfl_xor(s, 4, WAVE);
    if (pr < np) {
        const size_t p = p0 + pr;
        *(uint4*)(ah + p * I + r0 + 8 * q) = hi;
        *(uint4*)(al + p * I + r0 + 8 * q) = lo;
        if (q == 0) as[p * (I / 64) + ub] = s;
    }
}

// Down: block (output rows [RB ob, RB ob + RB)) x tile. ypick[src][o] = wts[src] * (dn_o . act).
// Grid (D / RB output blocks, tile-list capacity), tile records as for gate / up.
template <int NT>
__global__ void __launch_bounds__(256, 2) moe_down_kernel(const MoeTile* __restrict__ tiles,
                                                       const int* __restrict__ ntiles,
                                                       const int* __restrict__ psrc, const float* __restrict__ wts,
                                                       const uint16_t* __restrict__ ah, const uint16_t* __restrict__ al,
                                                       const float* __restrict__ as, int D, int I, ExpertOffsets off,
                                                       float* __restrict__ ypick) {
    // dynamic LDS: sc [RB][G] | gs [PB][G]
    extern __shared__ float2 dyn[];
    __shared__ float red[PB][RB + 1];  // the waves' summed outputs
    const int ob = blockIdx.x, tile = blockIdx.y;
    const MoeTile tl = tiles[tile];
    if (tile >= *ntiles) return;
    const int G = I / 64, o0 = ob * RB;
    float2* sc = dyn;
    float* gs = (float*)(dyn + RB * G);
    const int p0 = tl.p0, np = tl.p1 - tl.p0;
    const unsigned char* base = (const unsigned char*)tl.base;
    auto stage = [&]() {
        stage_scales(sc, (const uint16_t*)(base + off.dn_s), (const uint16_t*)(base + off.dn_m), o0, G);
        stage_gsums(gs, as, nullptr, p0, np, G);
    };
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE, n = lane % 16, g = lane / 16;
    long long xrow[2];
#pragma unroll
    for (int t = 0; t < 2; t++) xrow[t] = (long long)(p0 + min(16 * t + n, np - 1)) * I;
    const long long qrow0[1] = {o0};
    BlockAcc<1, NT> acc;
    expert_block<1, NT>(base + off.dn_q, qrow0, I, sc, ah, al, xrow, gs, acc, G, stage);
    reduce_waves<1, NT>(acc, 0, red);
    // 256 threads = 32 picks x 8 runs of 8 rows: ypick[src][o0 + 8 q ..] = w * y
    const int pr = threadIdx.x / 8, q = threadIdx.x % 8;
    if (pr < np) {
        const int src = psrc[p0 + pr];
        const float w = wts[src];
        float* dst = ypick + (size_t)src * D + o0 + 8 * q;
        const float* r = &red[pr][8 * q];
        ((float4*)dst)[0] = float4{w * r[0], w * r[1], w * r[2], w * r[3]};
        ((float4*)dst)[1] = float4{w * r[4], w * r[5], w * r[6], w * r[7]};
    }
}

// ---------------------------------------------------------------------------------------------
// Prefill-sized tiles (up to 64 picks of an expert with more than 32): a workgroup of 4 waves covers UB = 128 rows
// of the output (gate / up: 128 units, i.e. 128 gate and 128 up rows; down: 128 output rows) for
// all the tile's picks. Each wave owns 32 rows of every matrix (RT 16-row tiles in all) and walks
// the 64-groups in order; the picks' activations of one group (hi and lo, 64 picks x 64 values)
// are staged once per workgroup in LDS by direct global -> LDS loads (double-buffered, 16-byte
// slots XOR-swizzled by the pick row), so each activation byte is fetched once per workgroup and
// each code byte once per tile, against once per 32 picks and once per 16 rows in the kernels
// above. Per group and row tile the 4 x 2 x 2 products on the group's codes give P, and the lane
// adds s P + (m - 128 s) X into its accumulators, the same fp32 formula as expert_block.
constexpr int NWB = 4;         // waves per big workgroup (two workgroups per CU)
constexpr int UB = 32 * NWB;   // rows per matrix per big workgroup

// Rows of sc and gs are padded by one word so that the rows one read touches (4 apart in sc, 1
// apart in gs) fall in different banks.
struct BigSmem {
    uint32_t sc[2 * UB * 33];                // (s | m << 16) fp16 pairs, [matrix row][group], G <= 32
    float gs[PBB * 33];                      // activation group sums [pick][group], G <= 32
};
constexpr int kActBytes = 2 * PBB * 128;     // one group's activations: hi, lo x 64 picks x 128 B

// Stage (s, m) pairs of nrow rows (row0 .. row0 + nrow) x G groups as packed fp16 pairs, rows
// G + 1 words apart.
__device__ __forceinline__ void stage_sc_packed(uint32_t* sc, const uint16_t* __restrict__ s,
                                                const uint16_t* __restrict__ mn, long long row0, int nrow, int G) {
    const uint16_t* s0 = s + (size_t)row0 * G;
    const uint16_t* m0 = mn + (size_t)row0 * G;
    const int n8 = nrow * G / 8;
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    for (int i = threadIdx.x; i < n8; i += blockDim.x) {
        const u4v sv = ld_global<u4v>(s0 + 8 * i), mv = ld_global<u4v>(m0 + 8 * i);
        const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w}, mw[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int k = 8 * i + e;  // row k / G, group k % G
            sc[k + k / G] = ((sw[e / 2] >> (16 * (e & 1))) & 0xffffu) | (((mw[e / 2] >> (16 * (e & 1))) & 0xffffu) << 16);
        }
    }
}

// The big-tile block: RT row tiles per wave (codes of row tile rt at code row qrow[rt] + lane n,
// scales at LDS row srow[rt] + .. of sc), activations of pick rows xrow(p) (element offset of the
// pick's row in xh / xl), groups [0, G). acc[rt][t]: lane (n, g) holds rows 4 g + j, pick 16 t + n.
template <int RT>
__device__ __forceinline__ void big_block(const unsigned char* __restrict__ qbase, const long long (&qrow)[RT],
                                          const int (&srow)[RT], int Kdim, const uint16_t* __restrict__ xh,
                                          const uint16_t* __restrict__ xl, const long long* __restrict__ xrow8,
                                          const uint32_t* sc, const float* gs, int G, unsigned char* act0,
                                          unsigned char* act1, f32x4 (&acc)[RT][4]) {
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
    const int n = lane % 16, g = lane / 16;
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const size_t rowbytes = Kdim / 2;
    const unsigned char* arow[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) arow[rt] = qbase + (size_t)(qrow[rt] + n) * rowbytes + 8 * g;
    typedef uint32_t u2v __attribute__((ext_vector_type(2)));
    // activation pieces: 16 per group (8 per array, 8 picks x 128 B each), 16 / NWB per wave;
    // lane L of piece q (pick 8 (q % 8) + L / 8) fetches the global 16-byte slot (L % 8) ^ sw(pick)
    // so that LDS slot L % 8 of the pick's row holds it
    constexpr int PPW = 16 / NWB;
    const uint16_t* src[PPW];
#pragma unroll
    for (int u = 0; u < PPW; u++) {
        const int q = PPW * wave + u, pk = 8 * (q % 8) + lane / 8;
        src[u] = (q < 8 ? xh : xl) + xrow8[pk] + ((lane % 8) ^ ((pk >> 1) & 7)) * 8;
    }
    typedef __attribute__((address_space(3))) void lds_void;
    auto stage = [&](unsigned char* buf, int grp) {
#pragma unroll
        for (int u = 0; u < PPW; u++)
            __builtin_amdgcn_global_load_lds(src[u] + 64 * grp, (lds_void*)(buf + (PPW * wave + u) * 1024), 16, 0, 0);
    };
    // codes of group grp for every row tile (ring of 2 groups)
    u2v ar[2][RT];
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) ar[u][rt] = ld_global<u2v>(arow[rt] + 32 * min(u, G - 1));
    stage(act0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    auto group = [&](const unsigned char* cur, unsigned char* nxt, int grp, int slot) {
        if (grp + 1 < G) stage(nxt, grp + 1);
        // this group's activation fragments: pick tile t, k step ks: LDS slot (2 g + ks) ^ sw(row)
        bf16x8 bh[4][2], bl[4][2];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int row = 16 * t + n;
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const int off = row * 128 + (((2 * g + ks) ^ ((row >> 1) & 7)) * 16);
                bh[t][ks] = *(const bf16x8*)(cur + off);
                bl[t][ks] = *(const bf16x8*)(cur + PBB * 128 + off);
            }
        }
        float X[4];
#pragma unroll
        for (int t = 0; t < 4; t++) X[t] = gs[(16 * t + n) * (G + 1) + grp];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const u2v a2 = ar[slot][rt];
            f32x4 P[4];
#pragma unroll
            for (int t = 0; t < 4; t++) P[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const bf16x8 a = codes_bf16(ks ? a2.y : a2.x);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    P[t] = mfma_bf(a, bh[t][ks], P[t]);
                    P[t] = mfma_bf(a, bl[t][ks], P[t]);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t pr = sc[(srow[rt] + 4 * g + j) * (G + 1) + grp];
                const float sv = h2f((uint16_t)(pr & 0xffffu)), mv = h2f((uint16_t)(pr >> 16));
                const float mp = mv - 128.f * sv;
#pragma unroll
                for (int t = 0; t < 4; t++) acc[rt][t][j] = fmaf(sv, P[t][j], fmaf(mp, X[t], acc[rt][t][j]));
            }
        }
        // refill this ring slot with the codes two groups ahead (clamped: static wait counts)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) ar[slot][rt] = ld_global<u2v>(arow[rt] + 32 * min(grp + 2, G - 1));
        // the next group's direct loads are older than the RT code loads just issued
        __builtin_amdgcn_s_waitcnt((RT & 15) | (7 << 4) | (15 << 8));
        __syncthreads();
    };
    int grp = 0;
    for (; grp + 2 <= G; grp += 2) {
        group(act0, act1, grp, 0);
        group(act1, act0, grp + 1, 1);
    }
    if (grp < G) group(act0, act1, grp, 0);
}

// Gate / up for big tiles: units [256 ub, 256 ub + 256) x one tile of <= 64 picks. act as in
// moe_gate_up_kernel (bf16 hi / lo in chunk order, group sums over 64 units).
__global__ void __launch_bounds__(64 * NWB, 2) moe_gate_up_big_kernel(const MoeTile* __restrict__ tiles,
                                                              const int* __restrict__ ntiles,
                                                              const int* __restrict__ ptok,
                                                              const uint16_t* __restrict__ xh,
                                                              const uint16_t* __restrict__ xl,
                                                              const float* __restrict__ xs, int D, int I,
                                                              ExpertOffsets off, uint16_t* __restrict__ ah,
                                                              uint16_t* __restrict__ al, float* __restrict__ as) {
    __shared__ BigSmem sm;
    __shared__ __attribute__((aligned(1024))) unsigned char act0[kActBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char act1[kActBytes];
    __shared__ float red[NWB][PBB];
    __shared__ long long xrow8[PBB];
    const int ub = blockIdx.x, tile = blockIdx.y;
    const MoeTile tl = tiles[tile];
    if (tile >= *ntiles) return;
    const int G = D / 64, u0 = ub * UB;
    const int p0 = tl.p0, np = tl.p1 - tl.p0;
    const unsigned char* base = (const unsigned char*)tl.base;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, n = lane % 16, g = lane / 16;
    // picks past the tile repeat its last one (their results are not stored)
    if (tid < PBB) xrow8[tid] = (long long)ptok[p0 + min(tid, np - 1)] * D;
    stage_sc_packed(sm.sc, (const uint16_t*)(base + off.gu_s), (const uint16_t*)(base + off.gu_m), u0, UB, G);
    stage_sc_packed(sm.sc + UB * (G + 1), (const uint16_t*)(base + off.gu_s), (const uint16_t*)(base + off.gu_m),
                    I + u0, UB, G);
    for (int i = tid; i < PBB * G; i += blockDim.x) {
        const int pr = i / G, c = i % G;
        sm.gs[pr * (G + 1) + c] = xs[(size_t)ptok[p0 + min(pr, np - 1)] * G + c];
    }
    __syncthreads();
    // wave w: units u0 + 32 w .. + 32: gate row tiles 0, 1 and up row tiles 2, 3
    const int wu = u0 + 32 * wave;
    const long long qrow[4] = {wu, wu + 16, I + wu, I + wu + 16};
    const int srow[4] = {32 * wave, 32 * wave + 16, UB + 32 * wave, UB + 32 * wave + 16};
    f32x4 acc[4][4];
    big_block<4>(base, qrow, srow, D, xh, xl, xrow8, sm.sc, sm.gs, G, act0, act1, acc);
    // act = silu(gate) * up; lane (n, g) of tile (rt, t) holds units wu + 16 rt + 4 g + j of pick
    // 16 t + n. A chunk of 8 units lies in lanes g = 2c and 2c + 1: the even lane takes the odd
    // lane's 4 values and writes the chunk (hi, lo in chunk order) and its sum.
    float wsum[4] = {0.f, 0.f, 0.f, 0.f};  // per pick tile: this lane's chunk sums
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            float a[4], o[4];
#pragma unroll
            for (int j = 0; j < 4; j++) a[j] = silu_f(acc[rt][t][j]) * acc[rt + 2][t][j];
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = __shfl_xor(a[j], 16, WAVE);
            if ((g & 1) == 0) {
                const float v[8] = {a[0], a[1], a[2], a[3], o[0], o[1], o[2], o[3]};
                uint4 hi, lo;
                float sum;
                split8(v, hi, lo, sum);
                wsum[t] += sum;
                const int pr = 16 * t + n;
                if (pr < np) {
                    const size_t p = p0 + pr;
                    const int u = wu + 16 * rt + 4 * g;  // the chunk's first unit
                    *(uint4*)(ah + p * I + u) = hi;
                    *(uint4*)(al + p * I + u) = lo;
                }
            }
        }
    // group sums: a 64-unit group is waves 2 k and 2 k + 1; per wave, the even lanes g = 0, 2 of
    // pick n hold its chunk sums
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const float s2 = wsum[t] + __shfl_xor(wsum[t], 32, WAVE);
        if (g == 0) red[wave][16 * t + n] = s2;
    }
    __syncthreads();
    if (tid < (UB / 64) * PBB) {
        const int k = tid / PBB, pr = tid % PBB;
        if (pr < np) as[(size_t)(p0 + pr) * (I / 64) + (u0 / 64) + k] = red[2 * k][pr] + red[2 * k + 1][pr];
    }
}

// Down for big tiles: output rows [256 ob, 256 ob + 256) x one tile of <= 64 picks; ypick[src][o] =
// wts[src] * (dn_o . act), as moe_down_kernel.
__global__ void __launch_bounds__(64 * NWB, 2) moe_down_big_kernel(const MoeTile* __restrict__ tiles,
                                                           const int* __restrict__ ntiles, const int* __restrict__ psrc,
                                                           const float* __restrict__ wts,
                                                           const uint16_t* __restrict__ ah,
                                                           const uint16_t* __restrict__ al,
                                                           const float* __restrict__ as, int D, int I,
                                                           ExpertOffsets off, float* __restrict__ ypick) {
    __shared__ BigSmem sm;
    __shared__ __attribute__((aligned(1024))) unsigned char act0[kActBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char act1[kActBytes];
    __shared__ long long xrow8[PBB];
    const int ob = blockIdx.x, tile = blockIdx.y;
    const MoeTile tl = tiles[tile];
    if (tile >= *ntiles) return;
    const int G = I / 64, o0 = ob * UB;
    const int p0 = tl.p0, np = tl.p1 - tl.p0;
    const unsigned char* base = (const unsigned char*)tl.base;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, n = lane % 16, g = lane / 16;
    if (tid < PBB) xrow8[tid] = (long long)(p0 + min(tid, np - 1)) * I;
    stage_sc_packed(sm.sc, (const uint16_t*)(base + off.dn_s), (const uint16_t*)(base + off.dn_m), o0, UB, G);
    for (int i = tid; i < PBB * G; i += blockDim.x) {
        const int pr = i / G, c = i % G;
        sm.gs[pr * (G + 1) + c] = as[(size_t)(p0 + min(pr, np - 1)) * G + c];
    }
    __syncthreads();
    const int wo = o0 + 32 * wave;
    const long long qrow[2] = {wo, wo + 16};
    const int srow[2] = {32 * wave, 32 * wave + 16};
    f32x4 acc[2][4];
    big_block<2>(base + off.dn_q, qrow, srow, I, ah, al, xrow8, sm.sc, sm.gs, G, act0, act1, acc);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int pr = 16 * t + n;
        if (pr >= np) continue;
        const int src = psrc[p0 + pr];
        const float w = wts[src];
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
            const f32x4 v = acc[rt][t];
            *(float4*)(ypick + (size_t)src * D + wo + 16 * rt + 4 * g) = float4{w * v[0], w * v[1], w * v[2], w * v[3]};
        }
    }
}

// x[t] += sum_k ypick[t K + k] (k in order) and, with a shared expert, + sigmoid(h_t . wg) ysh[t].
// Grid (T, D / 256): one thread per column; the K pick rows are loaded together.
__global__ void __launch_bounds__(256) moe_combine_kernel(float* __restrict__ x, const float* __restrict__ ypick,
                                                          const int* __restrict__ idx, int E,
                                                          const float* __restrict__ ysh, const float* __restrict__ h,
                                                          const uint16_t* __restrict__ wg, int D, int K) {
    __shared__ float red[8];
    const int t = blockIdx.x, i = blockIdx.y * blockDim.x + threadIdx.x;
    float gate = 0.f;
    if (ysh) {
        float a = 0.f;
        for (int c = threadIdx.x; c < D; c += blockDim.x) a += h[(size_t)t * D + c] * bf2f(wg[c]);
        gate = sigmoid_f(block_sum(a, red));
    }
    if (i >= D) return;
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; k++) {
        if (k < K) {
            const int e = idx[(size_t)t * K + k];
            v[k] = (e >= 0 && e < E) ? ypick[((size_t)t * K + k) * D + i] : 0.f;
        }
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++)
        if (k < K) s += v[k];
    float r = x[(size_t)t * D + i] + s;
    if (ysh) r += gate * ysh[(size_t)t * D + i];
    x[(size_t)t * D + i] = r;
}

// x[t] += sigmoid(h_t . wg) y[t] (the engine's shared_gate_add)
__global__ void __launch_bounds__(256) shared_gate_add_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                              const float* __restrict__ h,
                                                              const uint16_t* __restrict__ wg, int D) {
    __shared__ float red[8];
    const int t = blockIdx.x;
    float a = 0.f;
    for (int i = threadIdx.x; i < D; i += blockDim.x) a += h[(size_t)t * D + i] * bf2f(wg[i]);
    const float gate = sigmoid_f(block_sum(a, red));
    for (int i = threadIdx.x; i < D; i += blockDim.x) x[(size_t)t * D + i] += gate * y[(size_t)t * D + i];
}

__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ out,
                                long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = silu_f(g[i]) * u[i];
}

// AEGIST_MOE_BIG=0 keeps every tile at <= 32 picks (A/B runs).
static bool big_tiles_enabled() {
    const char* e = getenv("AEGIST_MOE_BIG");
    return !(e && e[0] == '0');
}

// Workspace plan of aegist_moe_experts.
struct MoePlan {
    size_t xh, xl, xs, ah, al, as, yp, eoff, ptok, psrc, tiles1, tiles2, tiles3, meta, total;
    int max1, max2, max3;  // tile-list capacities: <= 16 picks (one per expert), 17..32, 33..64
};
static size_t al256(size_t x) { return (x + 255) / 256 * 256; }
static MoePlan moe_plan(int T, int K, int D, int I, int E) {
    MoePlan p;
    const size_t N = (size_t)T * K;
    p.max1 = (int)std::min<size_t>(N, (size_t)E);
    // an expert with c picks has floor(c / PB) + [c % PB > 16] <= c / 17 large blocks
    p.max2 = (int)(N / 17);
    p.max3 = (int)(N / 16);  // ceil(c / 64) <= c / 16 for every c > 32
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o += al256(bytes);
        return at;
    };
    p.xh = take((size_t)T * D * 2);
    p.xl = take((size_t)T * D * 2);
    p.xs = take((size_t)T * (D / 64) * 4);
    p.ah = take(N * I * 2);
    p.al = take(N * I * 2);
    p.as = take(N * (I / 64) * 4);
    p.yp = take(N * D * 4);
    p.eoff = take((size_t)(E + 1) * 4);
    p.ptok = take(N * 4);
    p.psrc = take(N * 4);
    p.tiles1 = take((size_t)p.max1 * sizeof(MoeTile));
    p.tiles2 = take((size_t)std::max(p.max2, 1) * sizeof(MoeTile));
    p.tiles3 = take((size_t)std::max(p.max3, 1) * sizeof(MoeTile));
    p.meta = take(16);
    p.total = o;
    return p;
}

}  // namespace

extern "C" {

size_t aegist_router_topk_workspace_bytes(int T, int E) {
    return T > 0 && E > 0 ? (size_t)T * E * 4 : 0;
}

int aegist_router_topk_ws(const float* h, const uint16_t* W, int* idx, float* wts, int T, int D, int E, int K,
                          void* ws, size_t ws_bytes, void* stream) {
    AEG_REQUIRE(T >= 0 && D > 0 && D % 16 == 0, "router_topk: need D % 16 == 0");
    AEG_REQUIRE(E > 0 && E <= 64 * 64, "router_topk: need 0 < E <= 4096");
    AEG_REQUIRE(K > 0 && K <= 16 && K <= E, "router_topk: need 0 < K <= min(16, E)");
    if (T == 0) return 0;
    // logits [T, E] = h W^T on the projection kernel (fp32 h as bf16 hi + lo against the exact
    // bf16 W), in the workspace
    int rc = check_workspace(ws, ws_bytes, aegist_router_topk_workspace_bytes(T, E), "router_topk");
    if (rc) return rc;
    float* logits = (float*)ws;
    hipStream_t st = AEG_STREAM(stream);
    rc = launch_proj(h, AEGIST_F32, D, W, AEGIST_BF16, nullptr, logits, E, T, E, D, 0, st);
    if (rc) return rc;
    const unsigned grid = (T + 3) / 4;
    if (E <= 64) router_topk_kernel<1><<<grid, 256, 0, st>>>(logits, idx, wts, T, E, K);
    else if (E <= 256) router_topk_kernel<4><<<grid, 256, 0, st>>>(logits, idx, wts, T, E, K);
    else if (E <= 1024) router_topk_kernel<16><<<grid, 256, 0, st>>>(logits, idx, wts, T, E, K);
    else router_topk_kernel<64><<<grid, 256, 0, st>>>(logits, idx, wts, T, E, K);
    return after_launch("router_topk");
}

int aegist_router_topk(const float* h, const uint16_t* W, int* idx, float* wts, int T, int D, int E, int K,
                       void* stream) {
    size_t bound = 0;
    void* ws = bound_workspace(&bound);
    return aegist_router_topk_ws(h, W, idx, wts, T, D, E, K, ws, bound, stream);
}

size_t aegist_moe_workspace_bytes(int T, int K, int D, int I, int E) {
    if (T <= 0 || K <= 0 || D <= 0 || I <= 0 || E <= 0) return 256;
    return moe_plan(T, K, D, I, E).total;
}

int aegist_moe_experts(const float* h, const unsigned long long* eptr, const int* idx, const float* wts, float* x,
                       int T, int D, int I, int E, int K, const float* ysh, const uint16_t* wg, void* ws,
                       size_t ws_bytes, void* stream) {
    AEG_REQUIRE(T >= 0 && K > 0 && K <= 16, "moe_experts: need T >= 0, 0 < K <= 16");
    AEG_REQUIRE(D % 64 == 0 && D >= 64 && D <= 64 * 64, "moe_experts: need D % 64 == 0 and D <= 4096");
    AEG_REQUIRE(I % 64 == 0 && I >= 64 && I <= 64 * 64, "moe_experts: need I % 64 == 0 and I <= 4096");
    AEG_REQUIRE(E > 0 && E <= MAX_E, "moe_experts: need 0 < E <= 1024");
    AEG_REQUIRE((ysh == nullptr) == (wg == nullptr), "moe_experts: the shared output and its gate come together");
    AEG_REQUIRE((long long)T * K < (1LL << 31) / 2, "moe_experts: too many picks");
    if (T == 0) return 0;
    const MoePlan p = moe_plan(T, K, D, I, E);
    if (!ws || ws_bytes < p.total) return fail(AEGIST_ERR_WORKSPACE, "moe_experts: workspace too small");
    AEG_REQUIRE((uintptr_t)h % 16 == 0 && (uintptr_t)x % 16 == 0, "moe_experts: h and x must be 16-byte aligned");
    unsigned char* w = (unsigned char*)ws;
    hipStream_t st = AEG_STREAM(stream);
    const ExpertOffsets off = expert_offsets(D, I);
    const int N = T * K;
    int* eoff = (int*)(w + p.eoff);
    int* ptok = (int*)(w + p.ptok);
    int* psrc = (int*)(w + p.psrc);
    MoeTile* tiles1 = (MoeTile*)(w + p.tiles1);
    MoeTile* tiles2 = (MoeTile*)(w + p.tiles2);
    MoeTile* tiles3 = (MoeTile*)(w + p.tiles3);
    int* meta = (int*)(w + p.meta);
    uint16_t* xh = (uint16_t*)(w + p.xh);
    uint16_t* xl = (uint16_t*)(w + p.xl);
    float* xs = (float*)(w + p.xs);
    uint16_t* ah = (uint16_t*)(w + p.ah);
    uint16_t* al = (uint16_t*)(w + p.al);
    float* as = (float*)(w + p.as);
    float* yp = (float*)(w + p.yp);

    // experts with more than 32 picks take the big-tile kernels where the shapes allow, once the
    // batch is large enough for such experts to be common (16 picks per expert on average)
    const bool big = (long long)N >= 16LL * E && D % UB == 0 && I % UB == 0 && D / 64 <= 32 && I / 64 <= 32 &&
                     big_tiles_enabled();
    moe_group_kernel<<<1, 1024, 0, st>>>(idx, N, K, E, eptr, eoff, ptok, psrc, tiles1, tiles2, tiles3, big ? 1 : 0,
                                         meta);
    int rc = after_launch("moe_group");
    if (rc) return rc;
    const long long nq = (long long)T * (D / 8);
    moe_xprep_kernel<<<(unsigned)((nq + 255) / 256), 256, 0, st>>>(h, T, D, xh, xl, xs);
    if ((rc = after_launch("moe_xprep"))) return rc;
    // Picks with an out-of-range expert id are dropped: no tile covers them and the combine
    // skips their rows, so nothing has to be cleared.
    const size_t lds_gu = (size_t)(2 * RB + PB) * (D / 64) * 8, lds_dn = (size_t)(RB + PB) * (I / 64) * 8;
    // two launches per projection: tiles of <= 16 picks (one MFMA column tile, the decode case)
    // and larger tiles (two); a workgroup past its list's count exits at once
    moe_gate_up_kernel<1><<<dim3(I / RB, p.max1), 256, lds_gu, st>>>(tiles1, meta, ptok, xh, xl, xs, D, I, off, ah, al,
                                                                     as);
    if ((rc = after_launch("moe_gate_up"))) return rc;
    if (p.max2 > 0) {
        moe_gate_up_kernel<2><<<dim3(I / RB, p.max2), 256, lds_gu, st>>>(tiles2, meta + 2, ptok, xh, xl, xs, D, I, off,
                                                                         ah, al, as);
        if ((rc = after_launch("moe_gate_up"))) return rc;
    }
    if (big) {
        moe_gate_up_big_kernel<<<dim3(I / UB, p.max3), 64 * NWB, 0, st>>>(tiles3, meta + 3, ptok, xh, xl, xs, D, I, off, ah,
                                                                   al, as);
        if ((rc = after_launch("moe_gate_up_big"))) return rc;
    }
    moe_down_kernel<1><<<dim3(D / RB, p.max1), 256, lds_dn, st>>>(tiles1, meta, psrc, wts, ah, al, as, D, I, off, yp);
    if ((rc = after_launch("moe_down"))) return rc;
    if (p.max2 > 0) {
        moe_down_kernel<2><<<dim3(D / RB, p.max2), 256, lds_dn, st>>>(tiles2, meta + 2, psrc, wts, ah, al, as, D, I,
                                                                      off, yp);
        if ((rc = after_launch("moe_down"))) return rc;
    }
    if (big) {
        moe_down_big_kernel<<<dim3(D / UB, p.max3), 64 * NWB, 0, st>>>(tiles3, meta + 3, psrc, wts, ah, al, as, D, I, off,
                                                                yp);
        if ((rc = after_launch("moe_down_big"))) return rc;
    }
    moe_combine_kernel<<<dim3(T, (D + 255) / 256), 256, 0, st>>>(x, yp, idx, E, ysh, h, wg, D, K);
    return after_launch("moe_combine");
}

int aegist_shared_gate_add(float* x, const float* y, const float* h, const uint16_t* wg, int T, int D, void* stream) {
    AEG_REQUIRE(T >= 0 && D > 0, "shared_gate_add: bad shape");
    if (T == 0) return 0;
    shared_gate_add_kernel<<<T, 256, 0, AEG_STREAM(stream)>>>(x, y, h, wg, D);
    return after_launch("shared_gate_add");
}

int aegist_silu_mul(const float* g, const float* u, float* out, long long n, void* stream) {
    AEG_REQUIRE(n >= 0, "silu_mul: bad size");
    if (n == 0) return 0;
    silu_mul_kernel<<<(unsigned)((n + 255) / 256), 256, 0, AEG_STREAM(stream)>>>(g, u, out, n);
    return after_launch("silu_mul");
}

}  // extern "C"
