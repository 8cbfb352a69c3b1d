// Chunked (C = 64) WY-form prefill of the gated delta rule on gfx950 MFMA, fused and
// sequence-parallel.
//
// Per chunk, with cum = cumsum(g), row norms rq, rk (L2 normalisation, q scale folded into rq)
// and the raw q, k, v rows (hybrid.py:327-361):
//   A      = strict_lower( beta_i rk_i rk_j e^{cum_i - cum_j} k_i . k_j )
//   v_new  = (I + A)^-1 ( beta v - beta rk e^{cum} (k S) )            [= u - w S]
//   o      = rq e^{cum} (q S) + intra v_new,   intra = lower_incl( rq_i rk_j e^{cum_i - cum_j} q_i . k_j )
//   S      = e^{cum_last} S + k^T ( rk e^{cum_last - cum} v_new )
//
// One workgroup (4 waves, one per SIMD) owns one (sequence, value head, segment of chunks) and
// walks its chunks with the state S [128 x 128] fp32 in MFMA accumulators, wave w owning value
// columns [32 w, 32 w + 32). Nothing per chunk goes through HBM: each period computes the chain
// of chunk c (the S-dependent products) and, interleaved with it, the intra-chunk operands of
// chunk c + 1 (Gram products, A, its diagonal-block inverses, intra), which land in
// double-buffered LDS. The triangular solve is a blocked forward substitution over the four
// 16-row blocks inside the chain (v_new_r = D_r (R_r - sum_{k<r} A_rk v_new_k), D_r the inverse
// of the r-th diagonal block of I + A, computed in fp32 per chunk), so it costs no separate
// inverse. Every product runs on v_mfma_f32_16x16x32_f16 (the substitution on 16x16x16);
// operands whose rounding reaches the output or the state carry an fp16 low part:
// R = (I + A) v_new's right-hand side and the state update's v_new (hi + lo), intra and v_new in
// the output (hi hi + hi lo + lo hi). The k, q, v tiles are the raw rows (exact in fp16 for bf16
// inputs) with every row factor applied in fp32 on the accumulators, so the fp16 operands stay
// well-scaled. Products keep their contraction index in a fixed permutation (within each 32
// block: 4g..4g+3 then 16+4g..16+4g+3 for lane group g) so that accumulator tiles are the next
// product's operands without any data movement.
//
// Sequence parallelism (batch x heads too few to fill the GPU, e.g. B = 1, 32 heads, 8192
// tokens): the chunks are split into P segments. Launch 1 runs segments 0..P-2 from a zero state
// (segment 0 from the initial state) while also carrying the segment's transition matrix M
// (S_end = M S_start + N, M propagated from I through the same chunk maps with no v term);
// a short combine launch chains S_{s+1} = M_s S_s + N_s over the segment boundaries; launch 2
// runs every segment again from its true start state and writes the outputs. With enough
// sequences x heads (P = 1) only launch 2 runs.
#include "common.h"

#include <algorithm>
#include <atomic>

using namespace aegist;

namespace {

constexpr int D = 128;
constexpr int CH = 64;
constexpr int NW = 4;              // chain waves per workgroup (and as many prep waves)
constexpr int NT2 = 2 * NW * WAVE; // threads per workgroup
// fp16 row strides in LDS: rows padded by 16 bytes, the measured best of 8 / 16 / 32 bytes for
// the chain's mix of 8-byte row reads, transpose reads and 16-byte row writes.
constexpr int RS = D + 8;          // 64 x 128 tiles (272 B rows)
constexpr int RSL = D + 8;         // low-part tiles of fp32 inputs (272 B)
constexpr int RA = CH + 8;         // 64 x 64 tiles (144 B rows)
constexpr int MIN_SEG_CHUNKS = 4;  // shortest segment the sequence split makes

typedef _Float16 half_t;
typedef short short4v_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) short4v_t lds_s4;

struct SeqLayout {
    long long sb_qk, st_qk, sh_qk, sb_v, st_v, sh_v, sb_o, st_o, sh_o;
    long long sb_g, st_g;  // g / beta strides by sequence and token; value head contiguous
};

// Per-token factor arrays of one chunk (fp32, 64 entries each) and the chunk decay. The Gram
// factors are kept as base-2 logarithms, so A_ij = 2^(la_i - mk_j) G_ij and
// intra_ij = 2^(lq_i - mk_j) (q k^T)_ij take one exponential per element:
// la = cum log2(e) + log2(beta rk), lq = cum log2(e) + log2(rq), mk = cum log2(e) - log2(rk).
struct Fact {
    float la[CH], mk[CH], beta[CH], fx[CH], fp[CH];
    float gam;
    float pad[3];
};

// LDS of one workgroup. kLo (fp32 inputs): the rows also keep their fp16 low parts, which the
// Gram products (k k^T, k q^T), the right-hand side's v and the state update use.
template <bool kLo>
struct Smem {
    static constexpr int NL = kLo ? 2 : 0;
    __attribute__((aligned(16))) half_t K[2][CH][RS];    // k rows (fp16), by chunk parity
    __attribute__((aligned(16))) half_t Q[CH][RS];       // rq e^cum q rows (fp16)
    __attribute__((aligned(16))) half_t V[CH][RS];       // v rows (fp16)
    __attribute__((aligned(16))) half_t AD[CH][RA];      // -A (strict lower blocks), D_r on the diagonal
    __attribute__((aligned(16))) half_t IH[CH][RA];      // intra (fp16 hi)
    __attribute__((aligned(16))) half_t IL[CH][RA];      // intra (fp16 lo)
    __attribute__((aligned(16))) Fact F[2];
    __attribute__((aligned(16))) half_t KL[NL][CH][RSL];      // k low parts, by chunk parity
    __attribute__((aligned(16))) half_t VL[NL / 2][CH][RSL];  // v low parts
};

static_assert(sizeof(Smem<false>) <= 160 * 1024 && sizeof(Smem<true>) <= 160 * 1024, "LDS of one workgroup exceeds a CU");

// Kernel parameters (one struct so both launches and the combine share them).
struct Params {
    const void* q;
    const void* k;
    const void* v;
    const float* g;
    const float* beta;
    void* out;
    SeqLayout a;
    int T, B, HK, HV, nch, P, L;  // P segments of L chunks
    int normalize;
    float qscale, eps;
    const float* init;  // initial state [B, HV, 128, 128] or null (zero)
    float* final_state; // where the last segment's end state goes (launch 2)
    float* starts;      // [B, HV, P, 128, 128] start state of every segment (P > 1)
    float* nbuf;        // [B, HV, P - 1, 128, 128] segment end state from the segment's start
    half_t* mbuf;       // [B, HV, P - 1, 128, 128] segment transition (row-major, fp16)
};

__device__ __forceinline__ f32x4 mfma32(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(half4 a, half4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ half8 cat8(half4 a, half4 b) {
    return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
// fp32 x4 -> fp16 x4, round to nearest even
__device__ __forceinline__ half4 h4(f32x4 x) {
    const half2v a = __builtin_convertvector((f32x2{x[0], x[1]}), half2v);
    const half2v b = __builtin_convertvector((f32x2{x[2], x[3]}), half2v);
    return half4{a[0], a[1], b[0], b[1]};
}
// x - (float)h for the fp16 in the low (res_l) or high (res_h) half of a packed pair: one
// v_fma_mix_f32 (h * -1 + x, the fp16 operand widened exactly), where the compiler would convert
// and subtract
__device__ __forceinline__ float res_l(uint32_t h, float x) {
    float r;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
    return r;
}
__device__ __forceinline__ float res_h(uint32_t h, float x) {
    float r;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
    return r;
}
// fp16 of x - hi (the low part of a hi + lo split whose high part is hi)
__device__ __forceinline__ half4 lo4(f32x4 x, half4 hi) {
    const uint2 hp = __builtin_bit_cast(uint2, hi);
    return h4(f32x4{res_l(hp.x, x[0]), res_h(hp.x, x[1]), res_l(hp.y, x[2]), res_h(hp.y, x[3])});
}
// hi + lo split: hi = fp16(x), lo = fp16(x - hi); hi + lo carries ~22 significant bits
__device__ __forceinline__ void split4(f32x4 x, half4& hi, half4& lo) {
    hi = h4(x);
    lo = lo4(x, hi);
}
__device__ __forceinline__ half4 ld4(const half_t* p) { return *(const half4*)p; }
// two 4-element runs of one row: the permuted 8-slot operand of one 32-wide k step
__device__ __forceinline__ half8 ld_perm(const half_t* row, int m, int g) {
    return cat8(ld4(row + 32 * m + 4 * g), ld4(row + 32 * m + 16 + 4 * g));
}
// transpose read: lane n of group g gets rows R..R+3 (R per group) of column C + n of a
// row-major fp16 tile with row stride `stride` (halfs)
__device__ __forceinline__ half4 ld_tr(const half_t* tile, int stride, int R, int C, int n) {
    const short4v_t s = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(tile + (R + (n >> 2)) * stride + C + 4 * (n & 3)));
    return __builtin_bit_cast(half4, s);
}

// Raw inputs of one chunk held by one wave: k and v rows of token tile `wave`, q rows of token
// tile 3 - wave; lane (n, g) holds features 32 ks + 8 g .. +7 of its row for ks = 0..3.
template <typename Tin> struct Raw;
template <> struct Raw<uint16_t> {
    uint4 k[4], q[4], v[4];
};
template <> struct Raw<float> {
    float4 k[8], q[8], v[8];
};
struct RawGB {
    float g, beta;
};

__device__ __forceinline__ void unpack8(const uint4* src, int ks, float* o) {
    const uint4 a = src[ks];
    o[0] = bf_lo(a.x); o[1] = bf_hi(a.x); o[2] = bf_lo(a.y); o[3] = bf_hi(a.y);
    o[4] = bf_lo(a.z); o[5] = bf_hi(a.z); o[6] = bf_lo(a.w); o[7] = bf_hi(a.w);
}
__device__ __forceinline__ void unpack8(const float4* src, int ks, float* o) {
    const float4 a = src[2 * ks], b = src[2 * ks + 1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

// Buffer resource over [base, base + bytes): loads past the end return zeros, stores are dropped
// (gfx9 word 3: 32-bit data, no swizzle).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, long long bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)min(bytes, 0x7fffffffLL), 0x00020000);
}

// 32 features (4 runs of 8 at 32 ks + 8 g) of the row at byte offset `off`; rows past the
// resource's range read as zeros
__device__ __forceinline__ void load_rows(__amdgpu_buffer_rsrc_t rs, int off, int g, uint4* dst) {
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
        dst[ks] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 2 * (32 * ks + 8 * g), 0, 0));
}
__device__ __forceinline__ void load_rows(__amdgpu_buffer_rsrc_t rs, int off, int g, float4* dst) {
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        dst[2 * ks] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 4 * (32 * ks + 8 * g), 0, 0));
        dst[2 * ks + 1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 4 * (32 * ks + 8 * g + 4), 0, 0));
    }
}

// Resources of one (sequence, value head): q / k rows of its QK head, v rows, g / beta, output.
struct Rsrc {
    __amdgpu_buffer_rsrc_t q, k, v, g, beta, out;
};

template <typename Tin, typename Tout>
__device__ __forceinline__ Rsrc make_rsrc(const Params& p, int b, int hv) {
    const int R = p.HV / p.HK, kh = hv / R;
    const long long last = (long long)(p.T - 1);
    Rsrc r;
    const long long off_qk = b * p.a.sb_qk + kh * p.a.sh_qk, len_qk = (last * p.a.st_qk + D) * (long long)sizeof(Tin);
    r.q = rsrc((const Tin*)p.q + off_qk, len_qk);
    r.k = rsrc((const Tin*)p.k + off_qk, len_qk);
    r.v = rsrc((const Tin*)p.v + b * p.a.sb_v + hv * p.a.sh_v, (last * p.a.st_v + D) * (long long)sizeof(Tin));
    const long long off_g = b * p.a.sb_g + hv, len_g = (last * p.a.st_g + 1) * 4;
    r.g = rsrc(p.g + off_g, len_g);
    r.beta = rsrc(p.beta + off_g, len_g);
    r.out = rsrc((Tout*)p.out + b * p.a.sb_o + hv * p.a.sh_o, (last * p.a.st_o + D) * (long long)sizeof(Tout));
    return r;
}

// Issue the global loads of chunk c (tokens past T read as zeros): kParts 1 = the k rows, g and
// beta (prep A's inputs), 2 = the q and v rows (prep B's), 3 = both.
template <typename Tin, bool kQ, int kParts = 3>
__device__ __forceinline__ void load_chunk(const Params& p, const Rsrc& rs, int c, int wave, int n, int g, int lane,
                                           Raw<Tin>& r, RawGB& gb) {
    const int tk = c * CH + 16 * wave + n, tq = c * CH + 16 * (3 - wave) + n;
    const int sz = (int)sizeof(Tin);
    if constexpr (kParts & 1) {
        load_rows(rs.k, tk * (int)p.a.st_qk * sz, g, r.k);
        const int go = (c * CH + lane) * (int)p.a.st_g * 4;
        gb.g = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs.g, go, 0, 0));
        gb.beta = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs.beta, go, 0, 0));
    }
    if constexpr (kParts & 2) {
        if constexpr (kQ) load_rows(rs.q, tq * (int)p.a.st_qk * sz, g, r.q);
        load_rows(rs.v, tk * (int)p.a.st_v * sz, g, r.v);
    }
}

// What prep A hands to prep B of the same chunk besides LDS: the cumulative decay at this
// lane's q row (tile 3 - wave).
struct Conv {
    float cum_q;
};

// Operands of chunk c that prep B computes in registers and the next period writes to LDS
// (AD, IH, IL are single-buffered: the chain of chunk c - 1 reads them until the period ends).
struct Deferred {
    half4 am[3];        // -A blocks (wave, jt) for jt < wave
    half4 d;            // D_wave[n][4 g .. 4 g + 3]
    half4 ih[4], il[4]; // intra blocks (3 - wave, jt) for jt <= 3 - wave
};

// acc + the sum of squares of 8 bf16 values (packed dot products), and a no-op form for fp32
__device__ __forceinline__ float dot2sq(const uint4* src, int ks, float acc) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    const uint4 a = src[ks];
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.x), __builtin_bit_cast(bf2, a.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.y), __builtin_bit_cast(bf2, a.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.z), __builtin_bit_cast(bf2, a.z), acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.w), __builtin_bit_cast(bf2, a.w), acc, false);
}
__device__ __forceinline__ float dot2sq(const float4*, int, float acc) { return acc; }

__device__ __forceinline__ half8 cvt8(const float* x) {
    const half4 a = h4(f32x4{x[0], x[1], x[2], x[3]}), b = h4(f32x4{x[4], x[5], x[6], x[7]});
    return cat8(a, b);
}
__device__ __forceinline__ half8 lo8(const float* x, half8 h) {
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; e++) y[e] = x[e] - (float)h[e];
    return cvt8(y);
}

// Prep phase A for chunk c into parity buffer `buf`: fp16 rows, norms, cumulative decays and the
// per-token factors; writes K[buf] rows of token tile `wave` and this wave's entries of F[buf].
template <typename Tin, bool kLo, bool kQ>
__device__ __forceinline__ void prep_a(const Params& p, Smem<kLo>& sm, int buf, const Raw<Tin>& r, const RawGB& gb,
                                       int wave, int n, int g, int lane, Conv& cv) {
    float ssk = 0.f;
    half8 k8[4], kl8[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        float x[8];
        unpack8(r.k, ks, x);
        if constexpr (kLo) {
#pragma unroll
            for (int e = 0; e < 8; e++) ssk += x[e] * x[e];
        } else {
            ssk = dot2sq(r.k, ks, ssk);
        }
        k8[ks] = cvt8(x);
        if constexpr (kLo) kl8[ks] = lo8(x, k8[ks]);
    }
    ssk = pair_sum32(pair_sum16(ssk));
    const float rk = p.normalize ? rsqrtf(ssk + p.eps) : 1.f;
    // k rows of tile `wave` (natural order)
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        *(half8*)&sm.K[buf][16 * wave + n][32 * ks + 8 * g] = k8[ks];
        if constexpr (kLo) *(half8*)&sm.KL[buf][16 * wave + n][32 * ks + 8 * g] = kl8[ks];
    }
    // inclusive prefix sum of g over the chunk (lane = token)
    float x = gb.g;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const float y = __shfl_up(x, d, WAVE);
        if (lane >= d) x += y;
    }
    const float cl = __shfl(x, CH - 1, WAVE);
    // this wave's tokens: factors of k rows (tile wave) and q rows (tile 3 - wave)
    constexpr float kLog2e = 1.4426950408889634f;
    const int tw = 16 * wave + n, tq = 16 * (3 - wave) + n;
    const float cum_t = __shfl(x, tw, WAVE), beta_t = __shfl(gb.beta, tw, WAVE);
    if constexpr (kQ) cv.cum_q = __shfl(x, tq, WAVE);
    Fact& F = sm.F[buf];
    if (g == 0) {
        const float c2 = cum_t * kLog2e, brk = beta_t * rk, lrk = __builtin_amdgcn_logf(rk);
        F.la[tw] = c2 + __builtin_amdgcn_logf(brk);
        F.mk[tw] = c2 - lrk;
        F.beta[tw] = beta_t;
        F.fx[tw] = brk * __expf(cum_t);
        F.fp[tw] = rk * __expf(cl - cum_t);
    }
    if (wave == 0 && lane == 0) F.gam = __expf(cl);
}

// Prep phase B for chunk c (after a barrier: K[buf] and F[buf] complete): the Gram products, -A
// blocks, the diagonal-block inverse D_wave and intra into `df` (written to LDS by the next
// period), and the q and v rows into Q and V.
template <typename Tin, bool kLo, bool kQ>
__device__ __forceinline__ void prep_b(const Params& p, Smem<kLo>& sm, int buf, const Raw<Tin>& r, const Conv& cv,
                                       int wave, int n, int g, Deferred& df) {
    const Fact& F = sm.F[buf];
    const int wv = wave;
    // this wave's q rows (tile 3 - wave: their norm and log factor) and v rows (tile wave), fp16
    // (+ lo parts for fp32 inputs)
    constexpr int NL = kLo ? 4 : 1;
    half8 cq[4], cql[NL];
    float lq_i = 0.f;
    if constexpr (kQ) {
        float ssq = 0.f;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            float x[8];
            unpack8(r.q, ks, x);
            if constexpr (kLo) {
#pragma unroll
                for (int e = 0; e < 8; e++) ssq += x[e] * x[e];
            } else {
                ssq = dot2sq(r.q, ks, ssq);
            }
            cq[ks] = cvt8(x);
            if constexpr (kLo) cql[ks] = lo8(x, cq[ks]);
        }
        ssq = pair_sum32(pair_sum16(ssq));
        const float rq = p.normalize ? rsqrtf(ssq + p.eps) * p.qscale : 1.f;
        lq_i = cv.cum_q * 1.4426950408889634f + __builtin_amdgcn_logf(rq);
    }
    // Gram tiles: C(jt, it) = MFMA(A = k rows of tile jt, B = rows of tile it), which holds
    // X[i = 16 it + n][j = 16 jt + 4 g + r] in lane (n, g) (the Gram matrix is symmetric).
    // G: it = wv, jt <= wv.  k q^T: it = 3 - wv, jt <= 3 - wv.
    const int iq = 3 - wv;
    // factors of this lane's rows
    const float la_i = F.la[16 * wv + n], mk_i = F.mk[16 * wv + n];
    // this wave's own k rows (the B operand of its Gram row block), read back from LDS
    half8 kb[4], kbl[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        kb[ks] = *(const half8*)&sm.K[buf][16 * wv + n][32 * ks + 8 * g];
        if constexpr (kLo) kbl[ks] = *(const half8*)&sm.KL[buf][16 * wv + n][32 * ks + 8 * g];
    }
#pragma unroll
    for (int jt = 0; jt < 4; jt++) {
        if (jt > wv && (!kQ || jt > iq)) continue;
        // fp32 inputs: the k rows of tile jt are re-read per product (registers for the lo parts)
        half8 ka[4], kal[4];
        if constexpr (!kLo) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++) ka[ks] = *(const half8*)&sm.K[buf][16 * jt + n][32 * ks + 8 * g];
        }
        auto kat = [&](int ks) -> half8 {
            if constexpr (kLo) return *(const half8*)&sm.K[buf][16 * jt + n][32 * ks + 8 * g];
            else return ka[ks];
        };
        auto kalt = [&](int ks) -> half8 { return *(const half8*)&sm.KL[buf][16 * jt + n][32 * ks + 8 * g]; };
        (void)kal;
        const f32x4 mkj = *(const f32x4*)&F.mk[16 * jt + 4 * g];
        if (jt <= wv) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const half8 a = kat(ks);
                acc = mfma32(a, kb[ks], acc);
                if constexpr (kLo) {
                    acc = mfma32(a, kbl[ks], acc);
                    acc = mfma32(kalt(ks), kb[ks], acc);
                }
            }
            f32x4 av;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int j = 16 * jt + 4 * g + r, i = 16 * wv + n;
                av[r] = j < i ? __builtin_amdgcn_exp2f(la_i - mkj[r]) * acc[r] : 0.f;
            }
            if (jt < wv) {
                df.am[jt < 3 ? jt : 2] = h4(-av);
            } else {
                // D = (I + N)^-1 = (I - N)(I + N^2)(I + N^4)(I + N^8) for the strictly lower
                // 16 x 16 block N = A_ww, on 16x16x16 MFMAs. Registers R(X) (lane (n, g) holding
                // X[n][4 g + r]) used as A are X, as B are X^T, and an MFMA's accumulator comes
                // back as R(C^T): so mfma(R(X^T), R(Y), C = R(Y)) = R(Y + Y X). N^T's entries are
                // the same Gram values (G is symmetric) with the factors of the swapped indices.
                const f32x4 laj = *(const f32x4*)&F.la[16 * wv + 4 * g];
                f32x4 avt, p0;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    avt[r] = n < 4 * g + r ? __builtin_amdgcn_exp2f(laj[r] - mk_i) * acc[r] : 0.f;
                    p0[r] = (n == 4 * g + r ? 1.f : 0.f) - av[r];
                }
                const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
                const half4 hn = h4(av), hnt = h4(avt);
                const half4 n2t = h4(mfma16(hn, hnt, z4)), n2 = h4(mfma16(hnt, hn, z4));
                const half4 n4t = h4(mfma16(n2, n2t, z4)), n4 = h4(mfma16(n2t, n2, z4));
                const half4 n8t = h4(mfma16(n4, n4t, z4));
                f32x4 pp = mfma16(n2t, h4(p0), p0);
                pp = mfma16(n4t, h4(pp), pp);
                pp = mfma16(n8t, h4(pp), pp);
                df.d = h4(pp);
            }
        }
        if (kQ && jt <= iq) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const half8 a = kat(ks);
                acc = mfma32(a, cq[ks], acc);
                if constexpr (kLo) {
                    acc = mfma32(a, cql[ks], acc);
                    acc = mfma32(kalt(ks), cq[ks], acc);
                }
            }
            f32x4 iv;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int j = 16 * jt + 4 * g + r, i = 16 * iq + n;
                iv[r] = j <= i ? __builtin_amdgcn_exp2f(lq_i - mkj[r]) * acc[r] : 0.f;
            }
            split4(iv, df.ih[jt], df.il[jt]);
        }
    }
    // q rows (scaled by rq e^cum) of tile iq and v rows of tile wv
    {
        const float f = __builtin_amdgcn_exp2f(lq_i);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            if constexpr (kQ) {
                half8 y;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float x = (float)cq[ks][e];
                    if constexpr (kLo) x += (float)cql[ks][e];
                    y[e] = (half_t)(f * x);
                }
                *(half8*)&sm.Q[16 * iq + n][32 * ks + 8 * g] = y;
            }
            float x[8];
            unpack8(r.v, ks, x);
            const half8 vh = cvt8(x);
            *(half8*)&sm.V[16 * wv + n][32 * ks + 8 * g] = vh;
            if constexpr (kLo) *(half8*)&sm.VL[0][16 * wv + n][32 * ks + 8 * g] = lo8(x, vh);
        }
    }
}

// The deferred operands of one chunk into AD / IH / IL.
template <bool kLo, bool kQ>
__device__ __forceinline__ void write_deferred(Smem<kLo>& sm, const Deferred& df, int wave, int n, int g) {
    const int wv = wave, iq = 3 - wave;
#pragma unroll
    for (int jt = 0; jt < 3; jt++)
        if (jt < wv) *(half4*)&sm.AD[16 * wv + n][16 * jt + 4 * g] = df.am[jt];
    *(half4*)&sm.AD[16 * wv + n][16 * wv + 4 * g] = df.d;
    if constexpr (!kQ) return;
#pragma unroll
    for (int jt = 0; jt < 4; jt++)
        if (jt <= iq) {
            *(half4*)&sm.IH[16 * iq + n][16 * jt + 4 * g] = df.ih[jt];
            *(half4*)&sm.IL[16 * iq + n][16 * jt + 4 * g] = df.il[jt];
        }
    if ((iq & 1) == 0) {  // the zero partner block of the 32-wide k step holding the diagonal
        *(half4*)&sm.IH[16 * iq + n][16 * (iq + 1) + 4 * g] = half4{0, 0, 0, 0};
        *(half4*)&sm.IL[16 * iq + n][16 * (iq + 1) + 4 * g] = half4{0, 0, 0, 0};
    }
}

// ---------------------------------------------------------------------------------------------
// The chain of one chunk for the 32 columns of one wave.

// The chain helpers work on NC 16-column tiles of S (wave columns col0 .. col0 + 16 NC) and take
// the LDS tiles by pointer: K / V rows with stride RS, their low parts (fp32 inputs) with stride
// RSL, the -A / D blocks with stride RA.

// X = k S (tokens x columns), C layout [token tile][column tile]
// Scheduling fence: keeps a prefetch stage's loads ahead of the products of the stage before.
#define SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

// X = k S and, with Q, o^T = S^T q~^T (the output's first term, transposed so a lane ends with 4
// consecutive columns of one token: A = S as it stands, B = the scaled q rows). The fragments of
// token tile t + 1 are requested before the products of tile t.
template <bool kQ, int NC>
__device__ __forceinline__ void chain_xo(const half_t* K, const half_t* Q, const half8 (&shi)[4][NC], int n, int g,
                                         f32x4 (&X)[4][NC], f32x4 (&O)[NC][4]) {
    // stages (t, k-product) then (t, q-product) (kQ), four fragments each, the next stage's
    // requested before this stage's products
    constexpr int ns = kQ ? 8 : 4;
    half8 fa[2][4];
    auto load = [&](int st, int sl) {
        const int t = kQ ? st / 2 : st;
        const half_t* base = (kQ && (st & 1)) ? Q : K;
#pragma unroll
        for (int m = 0; m < 4; m++) fa[sl][m] = ld_perm(base + (16 * t + n) * RS, m, g);
    };
    load(0, 0);
#pragma unroll
    for (int st = 0; st < ns; st++) {
        const int sl = st & 1, t = kQ ? st / 2 : st;
        const bool isq = kQ && (st & 1);
        if (st + 1 < ns) load(st + 1, sl ^ 1);
        SCHED_FENCE();
        f32x4 acc[NC];
#pragma unroll
        for (int ct = 0; ct < NC; ct++) acc[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 4; m++)
#pragma unroll
            for (int ct = 0; ct < NC; ct++)
                acc[ct] = isq ? mfma32(shi[m][ct], fa[sl][m], acc[ct]) : mfma32(fa[sl][m], shi[m][ct], acc[ct]);
#pragma unroll
        for (int ct = 0; ct < NC; ct++) {
            if (isq) O[ct][t] = acc[ct];
            else X[t][ct] = acc[ct];
        }
        SCHED_FENCE();
    }
}

// Right-hand side R = beta v - fx X (kWithV) or -fx X; VL: the v low parts or null
template <bool kWithV, int NC>
__device__ __forceinline__ void chain_r(const Fact& F, const half_t* V, const half_t* VL, int col0, int n, int g,
                                        f32x4 (&X)[4][NC]) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const f32x4 fx = *(const f32x4*)&F.fx[16 * t + 4 * g];
        f32x4 bt;
        if constexpr (kWithV) bt = *(const f32x4*)&F.beta[16 * t + 4 * g];
#pragma unroll
        for (int ct = 0; ct < NC; ct++) {
            f32x4 r = -(fx * X[t][ct]);
            if constexpr (kWithV) {
                const half4 vv = ld_tr(V, RS, 16 * t + 4 * g, col0 + 16 * ct, n);
                half4 vl = {0, 0, 0, 0};
                if (VL) vl = ld_tr(VL, RSL, 16 * t + 4 * g, col0 + 16 * ct, n);
#pragma unroll
                for (int e = 0; e < 4; e++) r[e] += bt[e] * ((float)vv[e] + (float)vl[e]);
            }
            X[t][ct] = r;
        }
    }
}

// v_new = (I + A)^-1 R by blocked forward substitution; R in, V out (both C layout), Vh = fp16(V).
// kZlo: the right-hand side of each D_r product as fp16 hi + lo.
template <bool kZlo, int NC>
__device__ __forceinline__ void chain_solve(const half_t* AD, int n, int g, const f32x4 (&R)[4][NC],
                                            f32x4 (&V)[4][NC], half4 (&Vh)[4][NC]) {
    half4 blk[4][4];  // -A_rk (k < r) and D_r, all requested up front
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int kk = 0; kk <= r; kk++) blk[r][kk] = ld4(AD + (16 * r + n) * RA + 16 * kk + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        f32x4 z[NC];
#pragma unroll
        for (int ct = 0; ct < NC; ct++) z[ct] = R[r][ct];
#pragma unroll
        for (int kk = 0; kk < r; kk++) {
#pragma unroll
            for (int ct = 0; ct < NC; ct++) z[ct] = mfma16(blk[r][kk], Vh[kk][ct], z[ct]);
        }
        const half4 dr = blk[r][r];
#pragma unroll
        for (int ct = 0; ct < NC; ct++) {
            half4 zh, zl;
            if constexpr (kZlo) {
                split4(z[ct], zh, zl);
                V[r][ct] = mfma16(dr, zl, mfma16(dr, zh, f32x4{0.f, 0.f, 0.f, 0.f}));
            } else {
                V[r][ct] = mfma16(dr, h4(z[ct]), f32x4{0.f, 0.f, 0.f, 0.f});
            }
            Vh[r][ct] = h4(V[r][ct]);
        }
    }
}

// S = gam S + k^T (fp V). kPlo: the B operand fp V as fp16 hi + lo (else hi); KL (the k low
// parts, or null) adds a third product.
template <bool kPlo, int NC>
__device__ __forceinline__ void chain_update(const Fact& F, const half_t* K, const half_t* KL, int n, int g,
                                             const f32x4 (&V)[4][NC], f32x4 (&S)[8][NC]) {
    half4 ph[4][NC], pl[4][NC];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const f32x4 fp = *(const f32x4*)&F.fp[16 * t + 4 * g];
#pragma unroll
        for (int ct = 0; ct < NC; ct++) {
            if constexpr (kPlo) split4(fp * V[t][ct], ph[t][ct], pl[t][ct]);
            else ph[t][ct] = h4(fp * V[t][ct]);
        }
    }
    const float gam = F.gam;
    half8 ka[2][2], kl[2][2];  // k^T fragments of feature tile ft, double-buffered
    auto load = [&](int ft, int sl) {
#pragma unroll
        for (int m = 0; m < 2; m++) {
            ka[sl][m] = cat8(ld_tr(K, RS, 32 * m + 4 * g, 16 * ft, n), ld_tr(K, RS, 32 * m + 16 + 4 * g, 16 * ft, n));
            if (kPlo && KL)
                kl[sl][m] = cat8(ld_tr(KL, RSL, 32 * m + 4 * g, 16 * ft, n),
                                 ld_tr(KL, RSL, 32 * m + 16 + 4 * g, 16 * ft, n));
        }
    };
    load(0, 0);
#pragma unroll
    for (int ft = 0; ft < 8; ft++) {
        const int sl = ft & 1;
        if (ft < 7) load(ft + 1, sl ^ 1);
        SCHED_FENCE();
        const half8* a = ka[sl];
        const half8* al = kl[sl];
#pragma unroll
        for (int ct = 0; ct < NC; ct++) {
            f32x4 acc = S[ft][ct] * gam;
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const half8 bh = cat8(ph[2 * m][ct], ph[2 * m + 1][ct]);
                acc = mfma32(a[m], bh, acc);
                if constexpr (kPlo) acc = mfma32(a[m], cat8(pl[2 * m][ct], pl[2 * m + 1][ct]), acc);
                if (kPlo && KL) acc = mfma32(al[m], bh, acc);
            }
            S[ft][ct] = acc;
        }
        SCHED_FENCE();
    }
}

template <int NC>
__device__ __forceinline__ void make_shi(const f32x4 (&S)[8][NC], half8 (&shi)[4][NC]) {
#pragma unroll
    for (int m = 0; m < 4; m++)
#pragma unroll
        for (int ct = 0; ct < NC; ct++) shi[m][ct] = cat8(h4(S[2 * m][ct]), h4(S[2 * m + 1][ct]));
}

// C-layout tiles of a [128][128] fp32 row-major matrix for the columns col0 .. col0 + 16 NC
template <int NC>
__device__ __forceinline__ void load_state(const float* src, int col0, int n, int g, f32x4 (&S)[8][NC]) {
#pragma unroll
    for (int ft = 0; ft < 8; ft++)
#pragma unroll
        for (int ct = 0; ct < NC; ct++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                S[ft][ct][r] = src ? src[(size_t)(16 * ft + 4 * g + r) * D + col0 + 16 * ct + n] : 0.f;
}
template <int NC>
__device__ __forceinline__ void store_state(float* dst, int col0, int n, int g, const f32x4 (&S)[8][NC]) {
#pragma unroll
    for (int ft = 0; ft < 8; ft++)
#pragma unroll
        for (int ct = 0; ct < NC; ct++)
#pragma unroll
            for (int r = 0; r < 4; r++) dst[(size_t)(16 * ft + 4 * g + r) * D + col0 + 16 * ct + n] = S[ft][ct][r];
}
template <int NC>
__device__ __forceinline__ void init_identity(int col0, int n, int g, f32x4 (&M)[8][NC]) {
#pragma unroll
    for (int ft = 0; ft < 8; ft++)
#pragma unroll
        for (int ct = 0; ct < NC; ct++)
#pragma unroll
            for (int r = 0; r < 4; r++) M[ft][ct][r] = (16 * ft + 4 * g + r == col0 + 16 * ct + n) ? 1.f : 0.f;
}
template <int NC>
__device__ __forceinline__ void store_transition(half_t* dst, int col0, int n, int g, const f32x4 (&M)[8][NC]) {
#pragma unroll
    for (int ft = 0; ft < 8; ft++)
#pragma unroll
        for (int ct = 0; ct < NC; ct++)
#pragma unroll
            for (int r = 0; r < 4; r++) dst[(size_t)(16 * ft + 4 * g + r) * D + col0 + 16 * ct + n] = (half_t)M[ft][ct][r];
}

// Workgroup -> (sequence, value head, segment). The value heads sharing a QK head go to the same
// XCD (block ids congruent mod 8), so their q / k rows are read through one L2.
__device__ __forceinline__ bool unit_of(int x, const Params& p, int nseg, int& b, int& hv, int& s) {
    const int R = p.HV / p.HK, xcd = x % 8, m = x / 8;
    const int r = m % R, grp = (m / R) * 8 + xcd;
    const int ngrp = p.B * nseg * p.HK;
    if (grp >= ngrp) return false;
    const int kh = grp % p.HK;
    s = (grp / p.HK) % nseg;
    b = grp / (p.HK * nseg);
    hv = kh * R + r;
    return true;
}

// ---------------------------------------------------------------------------------------------
// kOut: launch 2 (outputs from the segment's start state). !kOut: launch 1 (segment end state
// N and transition M from a zero start, segment 0 from the initial state).
// ---------------------------------------------------------------------------------------------
// Output products of one chunk, transposed (o^T) so a lane ends with 4 consecutive columns of one
// token: o^T = S^T (rq e^cum q)^T with A = S as it stands (the B-operand registers of S) and B =
// the scaled q rows, then o^T += v_new^T intra^T (hi hi + hi lo + lo hi) over the k steps on or
// below the diagonal.
template <int NC, typename Tout>
__device__ __forceinline__ void out_intra_store(const half_t* IH, const half_t* IL, const f32x4 (&V)[4][NC],
                                                const half4 (&Vh)[4][NC], f32x4 (&O)[NC][4],
                                                __amdgpu_buffer_rsrc_t out, int tok0, int st_o, int col0, int n, int g) {
    half4 Vl[4][NC];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int ct = 0; ct < NC; ct++) Vl[t][ct] = lo4(V[t][ct], Vh[t][ct]);
    // the six (token tile, k step) fragment pairs on or below the diagonal, each requested one
    // step ahead of its products
    constexpr int kIt[6] = {0, 1, 2, 2, 3, 3}, kM[6] = {0, 0, 0, 1, 0, 1};
    half8 fh[2], fl[2];
    fh[0] = ld_perm(IH + n * RA, 0, g);
    fl[0] = ld_perm(IL + n * RA, 0, g);
#pragma unroll
    for (int q = 0; q < 6; q++) {
        const int it = kIt[q], m = kM[q], sl = q & 1;
        if (q < 5) {
            fh[sl ^ 1] = ld_perm(IH + (16 * kIt[q + 1] + n) * RA, kM[q + 1], g);
            fl[sl ^ 1] = ld_perm(IL + (16 * kIt[q + 1] + n) * RA, kM[q + 1], g);
        }
        SCHED_FENCE();
        {
            const half8 ih = fh[sl], il = fl[sl];
#pragma unroll
            for (int ct = 0; ct < NC; ct++) {
                const half8 vh = cat8(Vh[2 * m][ct], Vh[2 * m + 1][ct]);
                const half8 vl = cat8(Vl[2 * m][ct], Vl[2 * m + 1][ct]);
                O[ct][it] = mfma32(vh, ih, O[ct][it]);
                O[ct][it] = mfma32(vh, il, O[ct][it]);
                O[ct][it] = mfma32(vl, ih, O[ct][it]);
            }
        }
        SCHED_FENCE();
    }
    // lane (n, g) of tile (ct, t) holds o[token tok0 + 16 t + n][col0 + 16 ct + 4 g .. + 3]; rows
    // past T fall outside the resource and are dropped
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int off = ((tok0 + 16 * t + n) * st_o + col0 + 4 * g) * (int)sizeof(Tout);
#pragma unroll
        for (int ct = 0; ct < NC; ct++) {
            const f32x4 o = O[ct][t];
            if constexpr (sizeof(Tout) == 2) {
                typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
                __builtin_amdgcn_raw_buffer_store_b64(u32x2{f2bf2(o[0], o[1]), f2bf2(o[2], o[3])}, out,
                                                      off + 32 * ct, 0, 0);
            } else {
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), out, off + 64 * ct, 0, 0);
            }
        }
    }
}

// The transition matrix's chain for one chunk (launch 1): M = gam M + k^T (fp solve(-fx k M)),
// fp16 hi operands throughout (its rounding reaches the result only through the segment
// combine).
template <int NC>
__device__ __forceinline__ void chain_transition(const Fact& F, const half_t* K, const half_t* AD, int n, int g,
                                                 f32x4 (&M)[8][NC]) {
    half8 mhi[4][NC];
    make_shi(M, mhi);
    f32x4 XM[4][NC], unused[NC][4];
    chain_xo<false>(K, nullptr, mhi, n, g, XM, unused);
    chain_r<false>(F, nullptr, nullptr, 0, n, g, XM);
    f32x4 VM[4][NC];
    half4 VMh[4][NC];
    chain_solve<true>(AD, n, g, XM, VM, VMh);
    chain_update<false>(F, K, nullptr, n, g, VM, M);
}

// Start / end of a segment's state (and transition) for the columns col0 .. col0 + 16 NC.
template <bool kOut, int NC>
__device__ __forceinline__ void seg_start(const Params& p, size_t unit, int s, int col0, int n, int g,
                                          f32x4 (&S)[8][NC]) {
    constexpr size_t DD = (size_t)D * D;
    if constexpr (kOut) {
        const float* src = p.P > 1 ? p.starts + (unit * p.P + s) * DD : (p.init ? p.init + unit * DD : nullptr);
        load_state(src, col0, n, g, S);
    } else {
        load_state(s == 0 && p.init ? p.init + unit * DD : nullptr, col0, n, g, S);
        if (s == 0) store_state(p.starts + unit * p.P * DD, col0, n, g, S);
    }
}
template <bool kOut, int NC>
__device__ __forceinline__ void seg_end(const Params& p, size_t unit, int s, int col0, int n, int g,
                                        const f32x4 (&S)[8][NC]) {
    constexpr size_t DD = (size_t)D * D;
    if constexpr (kOut) {
        if (s == p.P - 1) store_state(p.final_state + unit * DD, col0, n, g, S);
    } else {
        store_state(p.nbuf + (unit * (p.P - 1) + s) * DD, col0, n, g, S);
    }
}

// The workgroup is 8 waves, two per SIMD: waves 0..3 run the chain (wave w owning the value
// columns [32 w, 32 w + 32)), waves 4..7 the prep work of the next chunk (wave 4 + w: token tile w
// of the conversions, its five Gram tiles), so each SIMD interleaves one chain wave and one prep
// wave and neither carries the other's registers. Both roles meet at the two barriers of every
// period. WV (the wave index) is a template parameter so every wave-dependent choice is resolved
// at compile time and each period is one basic block.
template <typename Tin, typename Tout, bool kOut, int WV>
__device__ __forceinline__ void chain_body(const Params& p, Smem<sizeof(Tin) == 4>& sm, int b, int hv, int s,
                                           int lane) {
    constexpr bool kLo = sizeof(Tin) == 4;
    constexpr int col0 = 32 * WV;
    const int n = lane % 16, g = lane / 16;
    const int c0 = s * p.L, c1 = min(p.nch, c0 + p.L);
    const size_t unit = (size_t)(b * p.HV + hv);

    f32x4 S[8][2];
    seg_start<kOut>(p, unit, s, col0, n, g, S);
    const Rsrc rs = make_rsrc<Tin, Tout>(p, b, hv);
    lds_barrier();  // the prep waves' prologue: chunk c0's operands
    lds_barrier();

    const half_t* VL = kLo ? &sm.VL[0][0][0] : nullptr;
    for (int c = c0; c < c1; c++) {
        const int buf = c & 1;
        const half_t* KL = kLo ? &sm.KL[buf][0][0] : nullptr;
        // ---- phase 1: the products on S (the prep waves write chunk c's A / D / intra meanwhile)
        half8 shi[4][2];
        make_shi(S, shi);
        f32x4 X[4][2], O[2][4];
        chain_xo<kOut>(&sm.K[buf][0][0], &sm.Q[0][0], shi, n, g, X, O);
        chain_r<true>(sm.F[buf], &sm.V[0][0], VL, col0, n, g, X);
        lds_barrier();  // Q / V of chunk c are consumed; AD / IH / IL of chunk c are complete

        // ---- phase 2: substitution, output, state update
        f32x4 V[4][2];
        half4 Vh[4][2];
        chain_solve<true>(&sm.AD[0][0], n, g, X, V, Vh);
        if constexpr (kOut)
            out_intra_store<2, Tout>(&sm.IH[0][0], &sm.IL[0][0], V, Vh, O, rs.out, c * CH, (int)p.a.st_o, col0, n, g);
        chain_update<true>(sm.F[buf], &sm.K[buf][0][0], KL, n, g, V, S);
        lds_barrier();
    }
    seg_end<kOut>(p, unit, s, col0, n, g, S);
}

template <typename Tin, typename Tout, bool kQ, int WV>
__device__ __forceinline__ void prep_body(const Params& p, Smem<sizeof(Tin) == 4>& sm, int b, int hv, int s,
                                          int lane) {
    constexpr bool kLo = sizeof(Tin) == 4;
    constexpr int wave = WV - 4;  // token tile of this prep wave
    const int n = lane % 16, g = lane / 16;
    const int c0 = s * p.L, c1 = min(p.nch, c0 + p.L);
    const Rsrc rs = make_rsrc<Tin, Tout>(p, b, hv);
    Raw<Tin> raw;
    RawGB gb;
    Conv cv;
    Deferred df;
    // the transition launch: the segment's transition M (the chain on the identity with v = 0) runs
    // here, on these waves' spare phase-2 time; wave 4 + w owns the columns [32 w, 32 w + 32)
    constexpr bool kM = !kQ;
    f32x4 M[kM ? 8 : 1][2];
    if constexpr (kM) init_identity(32 * wave, n, g, M);
    // prep A (phase 1) reads the k rows, g and beta, prep B (phase 2) the q and v rows: each set
    // is requested right after its last use, a period ahead of its next
    load_chunk<Tin, kQ>(p, rs, c0, wave, n, g, lane, raw, gb);
    prep_a<Tin, kLo, kQ>(p, sm, c0 & 1, raw, gb, wave, n, g, lane, cv);
    load_chunk<Tin, kQ, 1>(p, rs, c0 + 1, wave, n, g, lane, raw, gb);
    lds_barrier();
    prep_b<Tin, kLo, kQ>(p, sm, c0 & 1, raw, cv, wave, n, g, df);
    load_chunk<Tin, kQ, 2>(p, rs, c0 + 1, wave, n, g, lane, raw, gb);
    lds_barrier();
    for (int c = c0; c < c1; c++) {
        const int nb = (c & 1) ^ 1;
        // ---- phase 1: chunk c's A / D / intra into LDS; prep A of chunk c + 1
        write_deferred<kLo, kQ>(sm, df, wave, n, g);
        prep_a<Tin, kLo, kQ>(p, sm, nb, raw, gb, wave, n, g, lane, cv);
        load_chunk<Tin, kQ, 1>(p, rs, c + 2, wave, n, g, lane, raw, gb);
        lds_barrier();
        // ---- phase 2: prep B of chunk c + 1 (Q and V are rewritten: the chain read them in phase 1)
        prep_b<Tin, kLo, kQ>(p, sm, nb, raw, cv, wave, n, g, df);
        __builtin_amdgcn_sched_barrier(0);  // the loads stay below prep B
        load_chunk<Tin, kQ, 2>(p, rs, c + 2, wave, n, g, lane, raw, gb);
        if constexpr (kM) {
            // chunk c's transition step (AD holds chunk c's blocks until the next period)
            __builtin_amdgcn_sched_barrier(0);
            chain_transition(sm.F[c & 1], &sm.K[c & 1][0][0], &sm.AD[0][0], n, g, M);
        }
        lds_barrier();
    }
    if constexpr (kM) {
        constexpr size_t DD = (size_t)D * D;
        store_transition(p.mbuf + ((size_t)(b * p.HV + hv) * (p.P - 1) + s) * DD, 32 * wave, n, g, M);
    }
}

template <typename Tin, typename Tout, bool kOut>
__global__ void __launch_bounds__(NT2, 2) delta_seg_kernel(Params p) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
    Smem<sizeof(Tin) == 4>& sm = *(Smem<sizeof(Tin) == 4>*)smem_raw;
    int b, hv, s;
    if (!unit_of(blockIdx.x, p, kOut ? p.P : p.P - 1, b, hv, s)) return;
    const int lane = threadIdx.x % WAVE;
    switch (__builtin_amdgcn_readfirstlane(threadIdx.x / WAVE)) {
        case 0: chain_body<Tin, Tout, kOut, 0>(p, sm, b, hv, s, lane); break;
        case 1: chain_body<Tin, Tout, kOut, 1>(p, sm, b, hv, s, lane); break;
        case 2: chain_body<Tin, Tout, kOut, 2>(p, sm, b, hv, s, lane); break;
        case 3: chain_body<Tin, Tout, kOut, 3>(p, sm, b, hv, s, lane); break;
        case 4: prep_body<Tin, Tout, kOut, 4>(p, sm, b, hv, s, lane); break;
        case 5: prep_body<Tin, Tout, kOut, 5>(p, sm, b, hv, s, lane); break;
        case 6: prep_body<Tin, Tout, kOut, 6>(p, sm, b, hv, s, lane); break;
        default: prep_body<Tin, Tout, kOut, 7>(p, sm, b, hv, s, lane); break;
    }
}

// Segment boundaries: S_1 = N_0, S_{s+1} = M_s S_s + N_s. One workgroup of 4 waves per
// (sequence, head, 16-column slice); wave w owns the rows [32 w, 32 w + 32). Computed transposed,
// S^T_{s+1} = S^T_s M_s^T + N^T_s, so a lane's accumulator holds 4 consecutive columns of one row
// (16-byte loads of N and stores of the start states) and M's rows enter as B operands with
// 16-byte loads; S^T_s, the A operand, goes through LDS as fp16 hi + lo (double-buffered, one
// barrier per step). Each wave's M / N operands are requested DEPTH steps ahead.
constexpr int CB_DEPTH = 3;
__global__ void __launch_bounds__(4 * WAVE) delta_seg_combine(Params p) {
    // the 8 column slices of one (sequence, head) on one XCD (block ids congruent mod 8), where
    // they share each M_s through that XCD's L2
    const int x = blockIdx.x, unit = (x / 64) * 8 + x % 8, slice = (x / 8) % 8;
    if (unit >= p.B * p.HV) return;
    __shared__ __attribute__((aligned(16))) half_t sth[2][16][D + 8], stl[2][16][D + 8];
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE, n = lane % 16, g = lane / 16;
    const int c0 = 16 * slice;
    constexpr size_t DD = (size_t)D * D;
    const float* N = p.nbuf + (size_t)unit * (p.P - 1) * DD;
    const half_t* Mb = p.mbuf + (size_t)unit * (p.P - 1) * DD;
    float* st = p.starts + (size_t)unit * p.P * DD;
    // step s's operands of this lane: M_s row (32 wave + 16 ft + n) as B fragments (k = 32 kb +
    // 8 g ..), N_s[row][c0 + 4 g ..] as the accumulator
    struct Ops {
        half8 b[2][4];
        f32x4 n[2];
    };
    auto load = [&](int s, Ops& o) {
        const float* Ns = N + (size_t)s * DD;
        const half_t* Ms = Mb + (size_t)s * DD;
#pragma unroll
        for (int ft = 0; ft < 2; ft++) {
            const int row = 32 * wave + 16 * ft + n;
            o.n[ft] = *(const f32x4*)(Ns + (size_t)row * D + c0 + 4 * g);
#pragma unroll
            for (int kb = 0; kb < 4; kb++) o.b[ft][kb] = *(const half8*)(Ms + (size_t)row * D + 32 * kb + 8 * g);
        }
    };
    // S^T rows of this lane's two tiles into LDS (hi + lo) and the fp32 start state to HBM
    auto publish = [&](int buf, int s1, const f32x4 (&v)[2]) {
#pragma unroll
        for (int ft = 0; ft < 2; ft++) {
            const int row = 32 * wave + 16 * ft + n;
            half4 h, l;
            split4(v[ft], h, l);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                sth[buf][4 * g + r][row] = h[r];
                stl[buf][4 * g + r][row] = l[r];
            }
            *(f32x4*)(st + (size_t)s1 * DD + (size_t)row * D + c0 + 4 * g) = v[ft];
        }
    };
    Ops ops[CB_DEPTH];
    f32x4 cur[2];
    {
        Ops o0;
        load(0, o0);  // (only its N part is used: S_1 = N_0)
#pragma unroll
        for (int d = 0; d < CB_DEPTH; d++)
            if (1 + d < p.P - 1) load(1 + d, ops[d]);
        cur[0] = o0.n[0];
        cur[1] = o0.n[1];
    }
    publish(0, 1, cur);  // S_1 = N_0
    lds_barrier();
    // steps s = 1 .. P - 2 (unrolled by the ring depth so every operand set is named statically)
    for (int s0 = 1; s0 < p.P - 1; s0 += CB_DEPTH) {
#pragma unroll
        for (int d = 0; d < CB_DEPTH; d++) {
            const int s = s0 + d;
            if (s >= p.P - 1) break;
            const int rb = (s - 1) & 1;  // S_s lives in buffer (s - 1) & 1
            half8 ah[4], al[4];
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                ah[kb] = *(const half8*)&sth[rb][n][32 * kb + 8 * g];
                al[kb] = *(const half8*)&stl[rb][n][32 * kb + 8 * g];
            }
            f32x4 acc[2] = {ops[d].n[0], ops[d].n[1]};
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int ft = 0; ft < 2; ft++) {
                    acc[ft] = mfma32(ah[kb], ops[d].b[ft][kb], acc[ft]);
                    acc[ft] = mfma32(al[kb], ops[d].b[ft][kb], acc[ft]);
                }
            if (s + CB_DEPTH < p.P - 1) load(s + CB_DEPTH, ops[d]);
            publish(rb ^ 1, s + 1, acc);
            lds_barrier();
        }
    }
}

__host__ __device__ inline size_t al256(size_t x) { return (x + 255) / 256 * 256; }

// Segment split: enough (sequence, head, segment) units to cover the GPU's CUs, segments of at
// least MIN_SEG_CHUNKS chunks.
struct Split {
    int nch, P, L;
};
Split split_for(int B, int T, int HV, int cus) {
    Split sp;
    sp.nch = (T + CH - 1) / CH;
    const int units = B * HV;
    int P = units >= cus ? 1 : std::max(1, cus / std::max(1, units));
    P = std::min(P, std::max(1, sp.nch / MIN_SEG_CHUNKS));
    sp.L = (sp.nch + P - 1) / P;
    sp.P = (sp.nch + sp.L - 1) / sp.L;
    return sp;
}

// CU count of the current device (256 when there is none), cached per device
int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
    if (dev < 64) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (dev < 64) cache[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

struct WsPlan {
    size_t state, starts, nbuf, mbuf, total;
};
WsPlan ws_plan(int B, int HV, const Split& sp, bool need_state) {
    WsPlan w;
    const size_t DD = (size_t)D * D, units = (size_t)B * HV;
    size_t off = 0;
    w.state = off;
    if (need_state) off += al256(units * DD * 4);
    w.starts = off;
    if (sp.P > 1) {
        off += al256(units * sp.P * DD * 4);
        w.nbuf = off;
        off += al256(units * (sp.P - 1) * DD * 4);
        w.mbuf = off;
        off += al256(units * (sp.P - 1) * DD * 2);
    } else {
        w.nbuf = w.mbuf = off;
    }
    w.total = std::max<size_t>(off, 256);
    return w;
}

}  // namespace

namespace aegist {

size_t delta_chunked_ws_bytes(int B, int T, int HK, int HV) {
    (void)HK;
    if (B <= 0 || T <= 0 || HV <= 0) return 256;
    return ws_plan(B, HV, split_for(B, T, HV, device_cus()), true).total;
}

template <typename Tin, typename Tout>
int run_chunked(const Tin* q, const Tin* k, const Tin* v, const float* g, const float* beta, float* state, Tout* out,
                const SeqLayout& a, int B, int T, int HK, int HV, int normalize, float qscale, float eps, void* ws,
                size_t ws_bytes, hipStream_t st) {
    const Split sp = split_for(B, T, HV, device_cus());
    const WsPlan wp = ws_plan(B, HV, sp, state == nullptr);
    if (wp.total > 256 || state == nullptr) {
        if (!ws || ws_bytes < wp.total) return fail(AEGIST_ERR_WORKSPACE, "delta_chunked: workspace too small");
    }
    // 16-byte row loads need 16-byte aligned rows; the output stores 8 (bf16) / 16 (fp32) bytes
    const long long ei = 16 / (long long)sizeof(Tin), eo = 4;
    const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)k % 16 == 0) && ((uintptr_t)v % 16 == 0) &&
                         a.sb_qk % ei == 0 && a.st_qk % ei == 0 && a.sh_qk % ei == 0 && a.sb_v % ei == 0 &&
                         a.st_v % ei == 0 && a.sh_v % ei == 0 && ((uintptr_t)out % (4 * sizeof(Tout)) == 0) &&
                         a.sb_o % eo == 0 && a.st_o % eo == 0 && a.sh_o % eo == 0;
    if (!aligned)
        return fail(AEGIST_ERR_SHAPE, "delta_chunked: q, k, v rows must be 16-byte aligned and output rows 4-element aligned");
    unsigned char* w = (unsigned char*)ws;
    Params p;
    p.q = q;
    p.k = k;
    p.v = v;
    p.g = g;
    p.beta = beta;
    p.out = out;
    p.a = a;
    p.T = T;
    p.B = B;
    p.HK = HK;
    p.HV = HV;
    p.nch = sp.nch;
    p.P = sp.P;
    p.L = sp.L;
    p.normalize = normalize;
    p.qscale = qscale;
    p.eps = eps;
    p.init = state;  // null: zero initial state
    p.final_state = state ? state : (float*)(w + wp.state);
    p.starts = sp.P > 1 ? (float*)(w + wp.starts) : nullptr;
    p.nbuf = sp.P > 1 ? (float*)(w + wp.nbuf) : nullptr;
    p.mbuf = sp.P > 1 ? (half_t*)(w + wp.mbuf) : nullptr;
    const size_t lds = sizeof(Smem<sizeof(Tin) == 4>);
    auto grid_for = [&](int nseg) {
        const int R = HV / HK, ngrp = B * nseg * HK;
        return (ngrp + 7) / 8 * 8 * R;
    };
    if (sp.P > 1) {
        delta_seg_kernel<Tin, Tout, false><<<grid_for(sp.P - 1), NT2, lds, st>>>(p);
        int rc = after_launch("delta_seg_kernel(transition)");
        if (rc) return rc;
        delta_seg_combine<<<(B * HV + 7) / 8 * 64, 4 * WAVE, 0, st>>>(p);
        rc = after_launch("delta_seg_combine");
        if (rc) return rc;
    }
    delta_seg_kernel<Tin, Tout, true><<<grid_for(sp.P), NT2, lds, st>>>(p);
    return after_launch("delta_seg_kernel(output)");
}

template <typename Tin, typename Tout>
static int set_lds_limits() {
    static int done = [] {
        const int bytes = (int)sizeof(Smem<sizeof(Tin) == 4>);
        const hipError_t e1 = hipFuncSetAttribute((const void*)delta_seg_kernel<Tin, Tout, false>,
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        const hipError_t e2 = hipFuncSetAttribute((const void*)delta_seg_kernel<Tin, Tout, true>,
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        return e1 == hipSuccess && e2 == hipSuccess ? 1 : -1;
    }();
    return done;
}

int launch_delta_chunked(const void* q, const void* k, const void* v, int in_dtype, const SeqLayout& a,
                         const float* g, const float* beta, float* state, void* out, int out_dtype, int B, int T,
                         int HK, int HV, int normalize, float qscale, float eps, void* ws, size_t ws_bytes,
                         hipStream_t st) {
    if (B < 0 || T < 0 || HK <= 0 || HV <= 0 || HV % HK) return fail(AEGIST_ERR_SHAPE, "delta_chunked: need HV % HK == 0");
    if (B == 0 || T == 0) return 0;
#define AEG_CHUNKED(TI, TO)                                                                                          \
    set_lds_limits<TI, TO>();                                                                                        \
    return run_chunked<TI, TO>((const TI*)q, (const TI*)k, (const TI*)v, g, beta, state, (TO*)out, a, B, T, HK, HV, \
                               normalize, qscale, eps, ws, ws_bytes, st)
    if (in_dtype == AEGIST_F32 && out_dtype == AEGIST_F32) { AEG_CHUNKED(float, float); }
    if (in_dtype == AEGIST_F32 && out_dtype == AEGIST_BF16) { AEG_CHUNKED(float, uint16_t); }
    if (in_dtype == AEGIST_BF16 && out_dtype == AEGIST_F32) { AEG_CHUNKED(uint16_t, float); }
    if (in_dtype == AEGIST_BF16 && out_dtype == AEGIST_BF16) { AEG_CHUNKED(uint16_t, uint16_t); }
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
    // the sequence split depends on B and T: take the largest need over batches 1..B and lengths
    // up to T (in chunk steps), so a workspace sized for (B, T) serves every smaller call
    size_t need = 256;
    const int nch = (std::max(T, 1) + CH - 1) / CH;
    for (int b = 1; b <= B; b++)
        for (int c = 1; c <= nch; c++) need = std::max(need, delta_chunked_ws_bytes(b, c * CH, HV, HV));
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
