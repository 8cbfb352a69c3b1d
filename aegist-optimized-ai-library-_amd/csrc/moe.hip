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

using namespace aegist;

namespace {

constexpr int PB = 32;            // picks per expert tile (two 16-column MFMA tiles)
constexpr int RB = 64;            // output rows per workgroup (4 waves x 16)
constexpr int MAX_E = 1024;       // experts per layer the grouping kernel handles
constexpr int RT = 4;             // tokens per router workgroup

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

// ---------------------------------------------------------------------------------------------
// Router: RT tokens per workgroup of E threads (lane = expert, E <= 256 by launch: 256 threads
// cover up to 256 experts; more experts loop). x rows in LDS (broadcast reads); W rows bf16.
__global__ void __launch_bounds__(256) router_topk_kernel(const float* __restrict__ h, const uint16_t* __restrict__ W,
                                                          int* __restrict__ idx, float* __restrict__ wts, int T, int D,
                                                          int E, int K) {
    extern __shared__ float sm[];
    float* xs = sm;                     // [RT][D]
    float* lg = sm + RT * D;            // [RT][E]
    const int t0 = blockIdx.x * RT, tid = threadIdx.x;
    const int nt = min(RT, T - t0);
    for (int i = tid; i < RT * D; i += blockDim.x) {
        const int r = i / D;
        xs[i] = r < nt ? h[(size_t)(t0 + r) * D + (i % D)] : 0.f;
    }
    __syncthreads();
    for (int e = tid; e < E; e += blockDim.x) {
        const uint4* row = (const uint4*)(W + (size_t)e * D);
        float acc[RT];
#pragma unroll
        for (int r = 0; r < RT; r++) acc[r] = 0.f;
        for (int c = 0; c < D / 8; c++) {
            const uint4 p = row[c];
            const float w[8] = {bf_lo(p.x), bf_hi(p.x), bf_lo(p.y), bf_hi(p.y),
                                bf_lo(p.z), bf_hi(p.z), bf_lo(p.w), bf_hi(p.w)};
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const float4 a = *(const float4*)&xs[r * D + 8 * c], b = *(const float4*)&xs[r * D + 8 * c + 4];
                acc[r] += a.x * w[0] + a.y * w[1] + a.z * w[2] + a.w * w[3] + b.x * w[4] + b.y * w[5] + b.z * w[6] +
                          b.w * w[7];
            }
        }
#pragma unroll
        for (int r = 0; r < RT; r++) lg[r * E + e] = acc[r];
    }
    __syncthreads();
    // softmax + top-K: wave w takes tokens w, w + 4, ...; lane holds experts lane + 64 i
    const int wave = tid / WAVE, lane = tid % WAVE, nw = blockDim.x / WAVE;
    for (int r = wave; r < nt; r += nw) {
        const float* l = lg + r * E;
        float m = -INFINITY;
        for (int e = lane; e < E; e += WAVE) m = fmaxf(m, l[e]);
        m = wave_max(m);
        float s = 0.f;
        for (int e = lane; e < E; e += WAVE) s += expf(l[e] - m);
        s = wave_sum(s);
        float sel = 0.f;                 // sum of the picked probabilities
        int taken_lo = 0, taken_hi = 0;  // picked slots among this lane's experts e = lane + 64 i
        float myv = 0.f;                 // lane k keeps pick k
        int mye = 0;
        for (int k = 0; k < K; k++) {
            // this lane's best remaining expert (lowest index on ties: experts visited in order)
            float bv = -1.f;
            int bi = 0x7fffffff;
            for (int i = 0, e = lane; e < E; i++, e += WAVE) {
                const bool taken = i < 32 ? (taken_lo >> i) & 1 : (taken_hi >> (i - 32)) & 1;
                const float p = expf(l[e] - m) / s;
                if (!taken && p > bv) {
                    bv = p;
                    bi = e;
                }
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
            if ((bi % WAVE) == lane) {
                const int i = bi / WAVE;
                if (i < 32) taken_lo |= 1 << i;
                else taken_hi |= 1 << (i - 32);
            }
            if (lane == k) {
                myv = bv;
                mye = bi;
            }
            sel += bv;
        }
        if (lane < K) {
            idx[(size_t)(t0 + r) * K + lane] = mye;
            wts[(size_t)(t0 + r) * K + lane] = myv / sel;
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Grouping (one workgroup of 1024 threads): picks i = t K + k with expert idx[i]; out of range
// experts are dropped and counted. eoff[E + 1]: exclusive prefix of the counts; ptok / psrc:
// token and pick index of each grouped position; tiles: (expert, p0, p1) blocks of <= PB
// positions; meta[0] = tile count, meta[1] = dropped picks. The order of positions inside an
// expert is unspecified (atomics); no result depends on it.
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

__global__ void __launch_bounds__(1024) moe_group_kernel(const int* __restrict__ idx, int N, int K, int E,
                                                         int* __restrict__ eoff, int* __restrict__ ptok,
                                                         int* __restrict__ psrc, int4* __restrict__ tiles,
                                                         int* __restrict__ meta) {
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
    const int c = tid < E ? cnt[tid] : 0, ntl = (c + PB - 1) / PB;
    int tot_c, tot_t;
    const int off = block_excl_scan(c, wsum, &tot_c);
    const int toff = block_excl_scan(ntl, wsum, &tot_t);
    if (tid < E) {
        eoff[tid] = off;
        cur[tid] = off;
        for (int j = 0; j < ntl; j++) tiles[toff + j] = int4{tid, off + j * PB, off + min(c, (j + 1) * PB), 0};
    }
    if (tid == 0) {
        eoff[E] = tot_c;
        meta[0] = tot_t;
        meta[1] = bad;
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
// One expert matrix block (NM = 1 or 2 matrices sharing the activations) times a tile of <= PB
// picks: wave w owns rows rowA[m] + 16 w + (0..15) of matrix m; lane (n, g) accumulates rows
// 4g + j (j < 4) for picks 16 t + n (t < 2). Scale / min (as s and m - 128 s) for the block's
// rows are staged in LDS; the activation group sums per pick too.
template <int NM>
struct BlockAcc {
    f32x4 acc[NM][2];
};

// sc: NM tables of [RB][ngroups] (s, m - 128 s); gs: [PB][ngroups] activation group sums.
template <int NM>
__device__ __forceinline__ void expert_block(const unsigned char* __restrict__ qbase, const long long* qrow0, int Kdim,
                                             const float2* sc, const uint16_t* __restrict__ xh,
                                             const uint16_t* __restrict__ xl, const long long* xrow, const float* gs,
                                             BlockAcc<NM>& out, int ngroups) {
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, n = lane % 16, g = lane / 16;
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int t = 0; t < 2; t++) out.acc[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const size_t rowbytes = Kdim / 2;
    // A operand rows: matrix m, row qrow0[m] + 16 wave + n
    const unsigned char* arow[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) arow[m] = qbase + (size_t)(qrow0[m] + 16 * wave + n) * rowbytes;
    for (int grp = 0; grp < ngroups; grp++) {
        f32x4 P[NM][2];
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int t = 0; t < 2; t++) P[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const int k0 = 64 * grp + 32 * ks + 8 * g;
            bf16x8 bh[2], bl[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                bh[t] = ld_bf8(xh + xrow[t] + k0);
                bl[t] = ld_bf8(xl + xrow[t] + k0);
            }
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const bf16x8 a = codes_bf16(*(const uint32_t*)(arow[m] + k0 / 2));
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    P[m][t] = mfma_bf(a, bh[t], P[m][t]);
                    P[m][t] = mfma_bf(a, bl[t], P[m][t]);
                }
            }
        }
        // y += s P + (m - 128 s) X per row (lane rows 4g + j) and pick (lane column n of tile t)
        const float X0 = gs[n * ngroups + grp], X1 = gs[(16 + n) * ngroups + grp];
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float2 sm = sc[(m * RB + 16 * wave + 4 * g + j) * ngroups + grp];
                out.acc[m][0][j] = fmaf(sm.x, P[m][0][j], fmaf(sm.y, X0, out.acc[m][0][j]));
                out.acc[m][1][j] = fmaf(sm.x, P[m][1][j], fmaf(sm.y, X1, out.acc[m][1][j]));
            }
    }
}

// Stage (s, m - 128 s) of rows [row0, row0 + RB) x groups [0, G) of one matrix into sc[RB][G]
// (the rows' scale and min entries are contiguous: one pass over RB G values).
__device__ __forceinline__ void stage_scales(float2* sc, const uint16_t* __restrict__ s,
                                             const uint16_t* __restrict__ mn, long long row0, int G) {
    const size_t k0 = (size_t)row0 * G;
    for (int i = threadIdx.x; i < RB * G; i += blockDim.x) {
        const float sv = h2f(s[k0 + i]), mv = h2f(mn[k0 + i]);
        sc[i] = float2{sv, mv - 128.f * sv};
    }
}

// Gate / up: block (unit block ub of RB units) x tile. act[p][r] = silu(gate_r . x) * (up_r . x)
// for the tile's picks, stored as bf16 hi / lo in chunk order (ah, al [P][I]) with group sums
// as [P][I / 64] (the unit block is one 64-group of the down projection's input).
__global__ void __launch_bounds__(256) moe_gate_up_kernel(const unsigned long long* __restrict__ eptr,
                                                          const int4* __restrict__ tiles, const int* __restrict__ meta,
                                                          const int* __restrict__ ptok, const uint16_t* __restrict__ xh,
                                                          const uint16_t* __restrict__ xl, const float* __restrict__ xs,
                                                          int D, int I, ExpertOffsets off, uint16_t* __restrict__ ah,
                                                          uint16_t* __restrict__ al, float* __restrict__ as) {
    // dynamic LDS: sc [2][RB][G] (s, m - 128 s) | gs [PB][G] activation group sums
    extern __shared__ float2 dyn[];
    __shared__ float ob[PB][RB + 1];     // act staging
    const int tile = blockIdx.y, ub = blockIdx.x;
    if (tile >= meta[0]) return;
    const int4 tl = tiles[tile];
    const int e = tl.x, p0 = tl.y, np = tl.z - tl.y;
    const unsigned char* base = (const unsigned char*)eptr[e];
    const int G = D / 64, r0 = ub * RB;
    float2* sc = dyn;
    float* gs = (float*)(dyn + 2 * RB * G);
    stage_scales(sc, (const uint16_t*)(base + off.gu_s), (const uint16_t*)(base + off.gu_m), r0, G);
    stage_scales(sc + RB * G, (const uint16_t*)(base + off.gu_s), (const uint16_t*)(base + off.gu_m), I + r0, G);
    for (int i = threadIdx.x; i < PB * G; i += blockDim.x) {
        const int pr = i / G, c = i % G;
        gs[i] = xs[(size_t)ptok[p0 + min(pr, np - 1)] * G + c];
    }
    __syncthreads();
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE, n = lane % 16, g = lane / 16;
    long long xrow[2];
#pragma unroll
    for (int t = 0; t < 2; t++) xrow[t] = (long long)ptok[p0 + min(16 * t + n, np - 1)] * D;
    const long long qrow0[2] = {r0, I + r0};
    BlockAcc<2> acc;
    expert_block<2>(base, qrow0, D, sc, xh, xl, xrow, gs, acc, G);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int j = 0; j < 4; j++) ob[16 * t + n][16 * wave + 4 * g + j] = silu_f(acc.acc[0][t][j]) * acc.acc[1][t][j];
    __syncthreads();
    // 256 threads = 32 picks x 8 chunks of the 64 units
    const int pr = threadIdx.x / 8, q = threadIdx.x % 8;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = ob[pr][8 * q + i];
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
__global__ void __launch_bounds__(256) moe_down_kernel(const unsigned long long* __restrict__ eptr,
                                                       const int4* __restrict__ tiles, const int* __restrict__ meta,
                                                       const int* __restrict__ psrc, const float* __restrict__ wts,
                                                       const uint16_t* __restrict__ ah, const uint16_t* __restrict__ al,
                                                       const float* __restrict__ as, int D, int I, ExpertOffsets off,
                                                       float* __restrict__ ypick) {
    // dynamic LDS: sc [RB][G] | gs [PB][G]
    extern __shared__ float2 dyn[];
    const int tile = blockIdx.y, ob = blockIdx.x;
    if (tile >= meta[0]) return;
    const int4 tl = tiles[tile];
    const int e = tl.x, p0 = tl.y, np = tl.z - tl.y;
    const unsigned char* base = (const unsigned char*)eptr[e];
    const int G = I / 64, o0 = ob * RB;
    float2* sc = dyn;
    float* gs = (float*)(dyn + RB * G);
    stage_scales(sc, (const uint16_t*)(base + off.dn_s), (const uint16_t*)(base + off.dn_m), o0, G);
    for (int i = threadIdx.x; i < PB * G; i += blockDim.x) {
        const int pr = i / G, c = i % G;
        gs[i] = as[(size_t)(p0 + min(pr, np - 1)) * G + c];
    }
    __syncthreads();
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE, n = lane % 16, g = lane / 16;
    long long xrow[2];
#pragma unroll
    for (int t = 0; t < 2; t++) xrow[t] = (long long)(p0 + min(16 * t + n, np - 1)) * I;
    const long long qrow0[1] = {o0};
    BlockAcc<1> acc;
    expert_block<1>(base + off.dn_q, qrow0, I, sc, ah, al, xrow, gs, acc, G);
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int pr = 16 * t + n;
        if (pr >= np) continue;
        const int src = psrc[p0 + pr];
        const float w = wts[src];
        const f32x4 y = acc.acc[0][t];
        *(float4*)(ypick + (size_t)src * D + o0 + 16 * wave + 4 * g) = float4{w * y[0], w * y[1], w * y[2], w * y[3]};
    }
}

// x[t] += sum_k ypick[t K + k] (k in order) and, with a shared expert, + sigmoid(h_t . wg) ysh[t].
__global__ void __launch_bounds__(256) moe_combine_kernel(float* __restrict__ x, const float* __restrict__ ypick,
                                                          const int* __restrict__ idx, int E,
                                                          const float* __restrict__ ysh, const float* __restrict__ h,
                                                          const uint16_t* __restrict__ wg, int D, int K) {
    __shared__ float red[8];
    const int t = blockIdx.x;
    float gate = 0.f;
    if (ysh) {
        float a = 0.f;
        for (int i = threadIdx.x; i < D; i += blockDim.x) a += h[(size_t)t * D + i] * bf2f(wg[i]);
        gate = sigmoid_f(block_sum(a, red));
    }
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        float s = 0.f;
        for (int k = 0; k < K; k++) {
            const int e = idx[(size_t)t * K + k];
            if (e >= 0 && e < E) s += ypick[((size_t)t * K + k) * D + i];
        }
        float v = x[(size_t)t * D + i] + s;
        if (ysh) v += gate * ysh[(size_t)t * D + i];
        x[(size_t)t * D + i] = v;
    }
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

// Workspace plan of aegist_moe_experts.
struct MoePlan {
    size_t xh, xl, xs, ah, al, as, yp, eoff, ptok, psrc, tiles, meta, total;
    int max_tiles;
};
static size_t al256(size_t x) { return (x + 255) / 256 * 256; }
static MoePlan moe_plan(int T, int K, int D, int I, int E) {
    MoePlan p;
    const size_t N = (size_t)T * K;
    p.max_tiles = (int)((N + PB - 1) / PB + std::min<size_t>(N, (size_t)E));
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
    p.tiles = take((size_t)p.max_tiles * 16);
    p.meta = take(16);
    p.total = o;
    return p;
}

}  // namespace

extern "C" {

int aegist_router_topk(const float* h, const uint16_t* W, int* idx, float* wts, int T, int D, int E, int K,
                       void* stream) {
    AEG_REQUIRE(T >= 0 && D > 0 && D % 8 == 0, "router_topk: need D % 8 == 0");
    AEG_REQUIRE(E > 0 && E <= 64 * 64, "router_topk: need 0 < E <= 4096");
    AEG_REQUIRE(K > 0 && K <= 16 && K <= E, "router_topk: need 0 < K <= min(16, E)");
    if (T == 0) return 0;
    const size_t lds = (size_t)RT * (D + E) * 4;
    AEG_REQUIRE(lds <= 64 * 1024, "router_topk: RT * (D + E) floats must fit in 64 KiB of LDS");
    router_topk_kernel<<<(T + RT - 1) / RT, 256, lds, AEG_STREAM(stream)>>>(h, W, idx, wts, T, D, E, K);
    return after_launch("router_topk");
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
    int4* tiles = (int4*)(w + p.tiles);
    int* meta = (int*)(w + p.meta);
    uint16_t* xh = (uint16_t*)(w + p.xh);
    uint16_t* xl = (uint16_t*)(w + p.xl);
    float* xs = (float*)(w + p.xs);
    uint16_t* ah = (uint16_t*)(w + p.ah);
    uint16_t* al = (uint16_t*)(w + p.al);
    float* as = (float*)(w + p.as);
    float* yp = (float*)(w + p.yp);

    moe_group_kernel<<<1, 1024, 0, st>>>(idx, N, K, E, eoff, ptok, psrc, tiles, meta);
    int rc = after_launch("moe_group");
    if (rc) return rc;
    const long long nq = (long long)T * (D / 8);
    moe_xprep_kernel<<<(unsigned)((nq + 255) / 256), 256, 0, st>>>(h, T, D, xh, xl, xs);
    if ((rc = after_launch("moe_xprep"))) return rc;
    // Picks with an out-of-range expert id are dropped: no tile covers them and the combine
    // skips their rows, so nothing has to be cleared.
    const size_t lds_gu = (size_t)(2 * RB + PB) * (D / 64) * 8, lds_dn = (size_t)(RB + PB) * (I / 64) * 8;
    moe_gate_up_kernel<<<dim3(I / RB, p.max_tiles), 256, lds_gu, st>>>(eptr, tiles, meta, ptok, xh, xl, xs, D, I, off,
                                                                       ah, al, as);
    if ((rc = after_launch("moe_gate_up"))) return rc;
    moe_down_kernel<<<dim3(D / RB, p.max_tiles), 256, lds_dn, st>>>(eptr, tiles, meta, psrc, wts, ah, al, as, D, I,
                                                                    off, yp);
    if ((rc = after_launch("moe_down"))) return rc;
    moe_combine_kernel<<<T, 256, 0, st>>>(x, yp, idx, E, ysh, h, wg, D, K);
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
