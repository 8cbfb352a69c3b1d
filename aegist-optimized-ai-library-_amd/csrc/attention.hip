// Gated GQA attention for gfx950: split-K MFMA decode and a causal prefill kernel.
//
// Decode (one query per sequence). One workgroup of 4 waves per (sequence, KV head, split of
// the context). The G <= 8 query heads of a KV head share every K/V byte the workgroup
// reads, so the cache is streamed from HBM once (the reference kernel reads it once per
// query head). Scores and P.V run on v_mfma_f32_16x16x32_bf16: the 16 MFMA rows hold the G
// query heads twice, as a bf16 hi part (rows 0-7) and the bf16 residual (rows 8-15), so
// q (fp32) and P (fp32) enter the products with ~16 significant bits while K and V are the
// exact bf16 cache values; row h + row h+8 recovers the fp32-accurate result.
//   - K and V: each wave's next 32-key tile is requested a tile ahead into registers and staged
//     row-major in the wave's LDS (16-byte row pad); the K operand of lane (key n, group g) is
//     K[key n][32 ks + 8 g .. +8]; the V operand is read as 4 dims x 8 keys per lane with 64-bit
//     LDS reads, repacking pairs of keys into the bf16x8 operand; output column block 4p+j,
//     lane column n is dim 64p + 4n + j.
//   - P is transposed from the score layout to the A-operand layout through 1 KiB of LDS.
// Each wave runs its own online softmax over its tiles; the 4 waves merge in LDS and the
// workgroup writes (m, l, O) for its split. A merge kernel combines the splits with
// log-sum-exp weights and applies the sigmoid output gate. The decode entry point's prep (ZNorm,
// RoPE, cache append) runs inside the split launch when the rotary dim is 64.
//
// Semantics: hybrid.py:280-310 (grouped SDPA at T == 1, causal SDPA otherwise, sigmoid gate);
// engine kernels attn_prep / attention_gated (hybrid.cu:86-173).
#include "common.h"

#include <cstdlib>
#include <type_traits>
#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>

using namespace aegist;

namespace aegist {
struct RopeTable;
int launch_attn_prep(const void* qg, const void* k, const void* v, int in_dtype, const uint16_t* qw,
                     const uint16_t* kw, float* qn, uint16_t* kc, uint16_t* vc, int B, int T, int H, int KV, int HD,
                     int RD, int pos0, int cap, float eps, float theta, hipStream_t stream);
}  // namespace aegist

namespace {


constexpr int HD = 256;
constexpr int TILE = 32;             // keys per wave iteration
constexpr int VROW = HD * 2 + 16;    // bytes per staged V row (16 B pad against bank conflicts)

struct DecodeSplit {
    int nsplit, per_split;
};

// Splits sized so a launch has about 256 workgroups (one round of one workgroup per CU: the
// kernel runs one wave per SIMD), each split a multiple of 128 keys (one 32-key tile per wave
// per step), at most 256 splits per (sequence, KV head).
#ifndef ATTN_SPLIT_TARGET
#define ATTN_SPLIT_TARGET 192  // workgroups per decode launch the split count aims for (measured: 160-192 beat 128 and 224-1024)
#endif
int split_target() {
    static const int t = [] {
        const char* e = getenv("AEGIST_ATTN_SPLIT_TARGET");
        return e && atoi(e) > 0 ? atoi(e) : ATTN_SPLIT_TARGET;
    }();
    return t;
}
DecodeSplit choose_split(int B, int KV, int L) {
    int units = std::max(1, B * KV);
    int max_split = std::min(256, std::max(1, (L + 127) / 128));
    int ns = std::min(max_split, std::max(1, (split_target() + units - 1) / units));
    int per = (L + ns - 1) / ns;
    per = (per + 127) / 128 * 128;
    ns = (L + per - 1) / per;
    return {ns, per};
}

__device__ __forceinline__ uint16_t bf_bits(float f) { return f2bf(f); }

// Split fp32 x into bf16 hi + bf16 lo with hi + lo ~= x to ~16 significant bits.
__device__ __forceinline__ void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
    hi = f2bf(x);
    lo = f2bf(x - bf2f(hi));
}

template <typename TG>
struct GateLd {
    static __device__ __forceinline__ float ld(const TG* p, size_t i) { return Act<TG>::ld(p, i); }
};

// q:   [B, H, HD] fp32 (normed, roped), head h of KV head kvh is kvh*G + r
// kc, vc: [B, KV, cap, HD] bf16
// part: [B, KV, nsplit, G, HD] fp32 partial outputs (unnormalised), ml: [B, KV, nsplit, G, 2]
// attn_decode_merge_wide_kernel then combines the splits (a second launch: a device-scope
// release and counter atomic at the end of every split workgroup, with the last one merging,
// cost far more than the launch).
// Keys of a sparse (listed-block) query, attention_gated_list (next.cu:648-705): the query at
// position p = pos0 + b sees the R keys of each of its nsel[b] listed blocks, in list order, then
// the keys of its own incomplete block, positions complete R .. p (complete = (p + 1) / R).
// blist == nullptr: the plain range [0, L) of sequence b's cache.
struct KeyList {
    const int* blist;
    const int* nsel;
    int top, R, pos0;
};

// Reductions inside a wave without LDS permutes (a shuffle's wait would also drain the K / V
// reads in flight): over the 16 lanes of a row by DPP (quad xor 1, quad xor 2, half-row mirror,
// row mirror - the same lane pairs as an xor butterfly, so every lane ends with the same value,
// for sums too), and across the two wave halves by v_permlane32_swap.
__device__ __forceinline__ float dpp_f(float x, int ctrl_sel) {
    switch (ctrl_sel) {
        case 0: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
        case 1: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
        case 2: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
        default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
    }
}
__device__ __forceinline__ float row16_max(float x) {
#pragma unroll
    for (int i = 0; i < 4; i++) x = fmaxf(x, dpp_f(x, i));
    return x;
}
__device__ __forceinline__ float row16_sum(float x) {
#pragma unroll
    for (int i = 0; i < 4; i++) x = x + dpp_f(x, i);
    return x;
}
// x[l] + x[l ^ 32]
__device__ __forceinline__ float half_swap_sum(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

// The decode step's own prep folded into the split launch (rotary dim 64): every workgroup
// normalises and rotates its G query rows straight from qg while its first K / V tile is in
// flight, and the workgroup of the last split normalises and rotates the new key, appends the
// key and value rows to the cache at row pos and substitutes them into its staged tile (the tile
// it fetched holds whatever row pos held before). Same arithmetic as attn_prep_vec_kernel, so
// the appended rows and the queries are bit-identical to the separate prep launch's.
struct FusedPrep {
    const void* qg;            // [B, H, 2 HD]: query | gate (Tin)
    const void* kn;            // [B, KV, HD] new key rows (Tin)
    const void* vn;            // [B, KV, HD] new value rows (Tin)
    const uint16_t* qw;        // q / k ZNorm weights (bf16, applied as 1 + w)
    const uint16_t* kw;
    uint16_t* kc;              // the caches, written at row pos
    uint16_t* vc;
    int pos;
    float eps;
    float inv[32];             // RoPE inverse frequencies, rotary dim 64
};
constexpr int kFusedRD = 64;

// 4 consecutive elements as raw words (bf16: 8 bytes in .x, .y; fp32: 16 bytes) and unpacked
template <typename T> __device__ __forceinline__ uint4 ld_raw4(const T* p);
template <> __device__ __forceinline__ uint4 ld_raw4<uint16_t>(const uint16_t* p) {
    const uint2 a = *(const uint2*)p;
    return uint4{a.x, a.y, 0u, 0u};
}
template <> __device__ __forceinline__ uint4 ld_raw4<float>(const float* p) { return *(const uint4*)p; }
template <typename T> __device__ __forceinline__ void unpack4(uint4 a, float* o);
template <> __device__ __forceinline__ void unpack4<uint16_t>(uint4 a, float* o) {
    o[0] = bf_lo(a.x); o[1] = bf_hi(a.x); o[2] = bf_lo(a.y); o[3] = bf_hi(a.y);
}
template <> __device__ __forceinline__ void unpack4<float>(uint4 a, float* o) {
    o[0] = __uint_as_float(a.x); o[1] = __uint_as_float(a.y); o[2] = __uint_as_float(a.z); o[3] = __uint_as_float(a.w);
}

// piece ks (8 consecutive elements) of a raw row held as 16-byte words
template <typename T> __device__ __forceinline__ void unpack8(const uint4* raw, int ks, float* o);
template <> __device__ __forceinline__ void unpack8<uint16_t>(const uint4* raw, int ks, float* o) {
    const uint4 a = raw[ks];
    o[0] = bf_lo(a.x); o[1] = bf_hi(a.x); o[2] = bf_lo(a.y); o[3] = bf_hi(a.y);
    o[4] = bf_lo(a.z); o[5] = bf_hi(a.z); o[6] = bf_lo(a.w); o[7] = bf_hi(a.w);
}
template <> __device__ __forceinline__ void unpack8<float>(const uint4* raw, int ks, float* o) {
    const uint4 a = raw[2 * ks], c = raw[2 * ks + 1];
    o[0] = __uint_as_float(a.x); o[1] = __uint_as_float(a.y); o[2] = __uint_as_float(a.z); o[3] = __uint_as_float(a.w);
    o[4] = __uint_as_float(c.x); o[5] = __uint_as_float(c.y); o[6] = __uint_as_float(c.z); o[7] = __uint_as_float(c.w);
}

// TQ: float = the queries come normed and rotated in q; uint16_t / float with kFused = the prep
// is done here from fp.qg (bf16 / fp32 inputs).
template <bool kList, bool kFused = false, typename Tin = float, bool kNT = false>
__global__ void __launch_bounds__(256) attn_decode_split_kernel(const float* __restrict__ q,
                                                                const uint16_t* __restrict__ kc,
                                                                const uint16_t* __restrict__ vc,
                                                                float* __restrict__ part, float* __restrict__ ml,
                                                                int H, int KV, int L, int cap, int per_split,
                                                                float scale, KeyList kl, FusedPrep fp) {
    // V staging per wave during the loop; the 4-wave merge buffer reuses the same bytes after it
    __shared__ __attribute__((aligned(16))) unsigned char vbuf_raw[4 * TILE * VROW];
    __shared__ __attribute__((aligned(16))) unsigned char kbuf[4][TILE * VROW];
    __shared__ __attribute__((aligned(16))) uint16_t pbuf[4][16][TILE];
    __shared__ float wm[4][8], wl[4][8];
    unsigned char (*vbuf)[TILE * VROW] = (unsigned char (*)[TILE * VROW])vbuf_raw;
    float (*wo)[8][HD] = (float (*)[8][HD])vbuf_raw;
    static_assert(4 * 8 * HD * 4 <= 4 * TILE * VROW, "merge buffer fits in the V staging area");

    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, nsplit = gridDim.x;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int n = lane % 16, g = lane / 16;
    const int G = H / KV;
    // listed keys: this query's key count and the list -> cache position map (batch-1 cache)
    constexpr bool listed = kList;
    int Lb = L, nsR = 0, tail0 = 0, pq = 0;
    const int* bl = nullptr;
    if (listed) {
        const int p = kl.pos0 + b, complete = (p + 1) / kl.R;
        pq = p;
        nsR = kl.nsel[b] * kl.R;
        tail0 = complete * kl.R;
        Lb = nsR + (p + 1 - tail0);
        bl = kl.blist + (size_t)b * kl.top;
    }
    const int k0 = split * per_split, k1 = min(Lb, k0 + per_split);

    // ---- Q operand: rows 0..7 = hi(q*scale), rows 8..15 = lo; lane row n, k elems 8g..8g+7.
    // Rows past G read row 0 and scale it by 0: unconditional loads issue back to back.
    bf16x8 qa[8];
    if constexpr (!kFused) {
        const int r = n & 7;
        const bool lo = n >= 8;
        const bool valid = r < G;
        const float* qrow = q + ((size_t)b * H + kvh * G + (valid ? r : 0)) * HD;
        const float qscale = valid ? scale : 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float x = qrow[ks * 32 + 8 * g + i] * qscale;
                uint16_t h, l;
                split_bf16(x, h, l);
                qa[ks][i] = (short)(lo ? l : h);
            }
        }
    }

    const size_t cache_row = listed ? (size_t)kvh : (size_t)b * KV + kvh;
    // the new key / value rows (bf16, as appended) for the last split's staged tile
    __shared__ __attribute__((aligned(16))) uint16_t knew[HD], vnew[HD];
    // the wave of the last split whose tile holds row pos (tiles are dealt to the 4 waves in turn)
    const bool owns_new = kFused && split == nsplit - 1 && wave == ((fp.pos - k0) / TILE) % 4;
    const uint16_t* kbase = kc + cache_row * (size_t)cap * HD;
    const uint16_t* vbase = vc + cache_row * (size_t)cap * HD;
    // listed keys: lane l holds the cache position of row l % 32 of a tile, looked up one tile
    // before the tile's fetch so the list load's wait never holds back the K / V loads in flight.
    // The list entry is read at a clamped index whatever nsel says (no wait on nsel first); rows
    // past the split map to cached positions <= p (finite data, probability 0).
    auto tile_keys = [&](int t0) {
        const int j = t0 + (lane & 31);
        const int blk = bl[min(j / kl.R, kl.top - 1)];
        return j < nsR ? blk * kl.R + j % kl.R : min(tail0 + (j - nsR), pq);
    };

    // running softmax state for heads 4*(g%2)+j, j < 4 (duplicated in lanes g and g+2)
    float m_run[4], l_run[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        m_run[j] = -INFINITY;
        l_run[j] = 0.f;
    }
    f32x4 oacc[16];
#pragma unroll
    for (int i = 0; i < 16; i++) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    unsigned char* vb = vbuf[wave];
    unsigned char* kb_l = kbuf[wave];
    // The next tile's K and V rows (16 bytes per lane per step, 32 steps) are held in registers,
    // requested a full tile ahead, and written to the wave's LDS staging at the top of the next
    // iteration. Rows past the split are clamped to its last row (finite data, probability 0).
    constexpr int NST = (TILE * HD * 2) / (16 * WAVE);  // 16 steps per tensor
    uint4 kreg[NST], vreg[NST];
    auto fetch = [&](int t0, int kp) {
#pragma unroll
        for (int it = 0; it < NST; it++) {
            const int idx = it * WAVE + lane, row = idx / (HD * 2 / 16), cc = idx % (HD * 2 / 16);
            const int key = listed ? __shfl(kp, row, WAVE) : min(t0 + row, k1 - 1);
            if constexpr (kNT) {
                typedef unsigned u32x4nt __attribute__((ext_vector_type(4)));
                const u32x4nt kq = __builtin_nontemporal_load((const u32x4nt*)(kbase + (size_t)key * HD + cc * 8));
                const u32x4nt vq = __builtin_nontemporal_load((const u32x4nt*)(vbase + (size_t)key * HD + cc * 8));
                kreg[it] = uint4{kq.x, kq.y, kq.z, kq.w};
                vreg[it] = uint4{vq.x, vq.y, vq.z, vq.w};
            } else {
                kreg[it] = *(const uint4*)(kbase + (size_t)key * HD + cc * 8);
                vreg[it] = *(const uint4*)(vbase + (size_t)key * HD + cc * 8);
            }
        }
    };
    // fused prep: the raw query rows and norm weights are requested before the first tile, and
    // lane j holds cos / sin of pos * inv_freq[j % 32] (the 32 frequencies selected from scalar
    // registers: no vector-memory access behind the tile's loads)
    uint4 qraw[kFused ? 8 * sizeof(Tin) / 2 : 1], wraw[kFused ? 8 : 1];
    float rc = 0.f, rs = 0.f;
    uint4 knraw{}, vnraw{}, kwraw{};
    if constexpr (kFused) {
        const int r = n & 7;
        const Tin* qrow = (const Tin*)fp.qg + ((size_t)b * H + kvh * G + (r < G ? r : 0)) * 2 * HD;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            if constexpr (sizeof(Tin) == 2) {
                qraw[ks] = *(const uint4*)(qrow + ks * 32 + 8 * g);
            } else {
                qraw[2 * ks] = *(const uint4*)(qrow + ks * 32 + 8 * g);
                qraw[2 * ks + 1] = *(const uint4*)(qrow + ks * 32 + 8 * g + 4);
            }
            wraw[ks] = *(const uint4*)(fp.qw + ks * 32 + 8 * g);
        }
        if (owns_new) {
            const size_t o = ((size_t)b * KV + kvh) * HD + 4 * lane;
            knraw = ld_raw4<Tin>((const Tin*)fp.kn + o);
            vnraw = ld_raw4<Tin>((const Tin*)fp.vn + o);
            kwraw = ld_raw4<uint16_t>(fp.kw + 4 * lane);
        }
        float f = 0.f;
#pragma unroll
        for (int j = 0; j < 32; j++) f = (lane & 31) == j ? fp.inv[j] : f;
        sincosf((float)fp.pos * f, &rs, &rc);
    }
    const int first = k0 + wave * TILE, stride = 4 * TILE;
    int kp_next = 0;
    if (first < k1) {
        if constexpr (listed) {
            fetch(first, tile_keys(first));
            kp_next = tile_keys(min(first + stride, k1 - 1));
        } else {
            fetch(first, 0);
        }
    }
    if constexpr (kFused) {
        // query rows: ZNorm (sum of squares over the 4 lanes g of a row) and RoPE on dims < 64,
        // whose partners d, d + 32 sit in pieces ks = 0 and 1 of the same lane. The raw rows
        // were requested before the first tile (loads return in order).
        const bool lo = n >= 8, valid = (n & 7) < G;
        float ss = 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            float x[8];
            unpack8<Tin>(qraw, ks, x);
#pragma unroll
            for (int i = 0; i < 8; i++) ss += x[i] * x[i];
        }
        ss += __shfl_xor(ss, 16, WAVE);
        ss += __shfl_xor(ss, 32, WAVE);
        const float inv = rsqrtf(ss / (float)HD + fp.eps), qscale = valid ? scale : 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ks += 2) {
            float x0[8], x1[8], w0[8], w1[8];
            unpack8<Tin>(qraw, ks, x0);
            unpack8<Tin>(qraw, ks + 1, x1);
            unpack8<uint16_t>(wraw, ks, w0);
            unpack8<uint16_t>(wraw, ks + 1, w1);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float y0 = (x0[i] * inv) * (1.f + w0[i]), y1 = (x1[i] * inv) * (1.f + w1[i]);
                if (ks == 0) {
                    const float c = __shfl(rc, 8 * g + i, WAVE), sn = __shfl(rs, 8 * g + i, WAVE);
                    const float r0 = y0 * c + (-y1) * sn, r1 = y1 * c + y0 * sn;
                    y0 = r0;
                    y1 = r1;
                }
                uint16_t h, l;
                split_bf16(y0 * qscale, h, l);
                qa[ks][i] = (short)(lo ? l : h);
                split_bf16(y1 * qscale, h, l);
                qa[ks + 1][i] = (short)(lo ? l : h);
            }
        }
        if (owns_new) {
            // the new key row: lane l holds dims 4l .. 4l + 3 (the prep kernel's layout and order)
            const size_t rkv = (size_t)b * KV + kvh;
            const int e0 = 4 * lane;
            float x[4], vv[4], wn[4];
            unpack4<Tin>(knraw, x);
            unpack4<Tin>(vnraw, vv);
            unpack4<uint16_t>(kwraw, wn);
            float sk = (x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3]);
            sk = wave_sum(sk);
            const float ik = rsqrtf(sk / (float)HD + fp.eps);
            float y[4], o4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) y[e] = (x[e] * ik) * (1.f + wn[e]);
            constexpr int half = kFusedRD / 2;
            const int plane = e0 < half ? lane + half / 4 : lane - half / 4;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float yp = __shfl(y[e], plane < 0 ? 0 : (plane > 63 ? 63 : plane), WAVE);
                const int i = e0 + e;
                o4[e] = y[e];
                const float ce = __shfl(rc, i & (half - 1), WAVE), se = __shfl(rs, i & (half - 1), WAVE);
                if (i < kFusedRD) o4[e] = y[e] * ce + (i < half ? -yp : yp) * se;
            }
            const uint2 kb2 = uint2{f2bf2(o4[0], o4[1]), f2bf2(o4[2], o4[3])};
            const uint2 vb2 = uint2{f2bf2(vv[0], vv[1]), f2bf2(vv[2], vv[3])};
            const size_t o = (rkv * cap + fp.pos) * HD + e0;
            *(uint2*)(fp.kc + o) = kb2;
            *(uint2*)(fp.vc + o) = vb2;
            *(uint2*)&knew[e0] = kb2;
            *(uint2*)&vnew[e0] = vb2;  // read back only by this wave (LDS ops of a wave run in order)
        }
    }
    for (int t0 = first; t0 < k1; t0 += stride) {
#pragma unroll
        for (int it = 0; it < NST; it++) {
            const int idx = it * WAVE + lane, row = idx / (HD * 2 / 16), cc = idx % (HD * 2 / 16);
            uint2* dv = (uint2*)(vb + row * VROW + cc * 16);
            dv[0] = uint2{vreg[it].x, vreg[it].y};
            dv[1] = uint2{vreg[it].z, vreg[it].w};
            uint2* dk = (uint2*)(kb_l + row * VROW + cc * 16);
            dk[0] = uint2{kreg[it].x, kreg[it].y};
            dk[1] = uint2{kreg[it].z, kreg[it].w};
        }
        if constexpr (kFused) {
            // the last split's tile holding row pos: that row and the rows clamped to it (keys
            // past the split) take the new key / value, so no stale cache bytes enter P V
            if (owns_new && t0 + TILE > fp.pos) {
                for (int rr = max(fp.pos - t0, 0) + (lane >> 5); rr < TILE; rr += 2) {
                    const int cc = lane & 31;
                    *(uint4*)(kb_l + rr * VROW + cc * 16) = *(const uint4*)&knew[8 * cc];
                    *(uint4*)(vb + rr * VROW + cc * 16) = *(const uint4*)&vnew[8 * cc];
                }
            }
        }
        fetch(min(t0 + stride, k1 - 1), kp_next);  // next tile (unconditional: static wait counts)
        if constexpr (listed) kp_next = tile_keys(min(t0 + 2 * stride, k1 - 1));
        wave_sync();
        // ---- scores: two 16-key blocks
        f32x4 sc[2];
#pragma unroll
        for (int nb = 0; nb < 2; nb++) {
            int key = t0 + nb * 16 + n;
            const unsigned char* krow = kb_l + (nb * 16 + n) * VROW + 16 * g;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                bf16x8 kb = *(const bf16x8*)(krow + ks * 64);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], kb, acc, 0, 0, 0);
            }
            // rows 4g+j; combine hi (g<2) and lo (g>=2) parts: lane g and g^2 hold h and h+8
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float s = half_swap_sum(acc[j]);
                sc[nb][j] = key < k1 ? s : -INFINITY;
            }
        }
        // ---- online softmax per head (over 16 lanes n and 2 blocks)
        float p0[4], p1[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float mt = row16_max(fmaxf(sc[0][j], sc[1][j]));
            float mn = fmaxf(m_run[j], mt);  // finite: every tile has at least one valid key
            float corr = __expf(m_run[j] - mn);
            p0[j] = __expf(sc[0][j] - mn);
            p1[j] = __expf(sc[1][j] - mn);
            l_run[j] = l_run[j] * corr + p0[j] + p1[j];
            m_run[j] = mn;
            // rescale O rows held by this lane: rows 4g+j are heads 4(g%2)+j
#pragma unroll
            for (int i = 0; i < 16; i++) oacc[i][j] *= corr;
        }
        // ---- P -> LDS as A operand [16 rows][32 keys]: rows 0-7 hi, 8-15 lo
        {
            const int hb = 4 * (g & 1);
            const bool lo = g >= 2;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint16_t h0, l0, h1, l1;
                split_bf16(p0[j], h0, l0);
                split_bf16(p1[j], h1, l1);
                int row = (lo ? 8 : 0) + hb + j;
                pbuf[wave][row][n] = lo ? l0 : h0;
                pbuf[wave][row][16 + n] = lo ? l1 : h1;
            }
        }
        wave_sync();
        bf16x8 pa = *(const bf16x8*)&pbuf[wave][n][8 * g];
        // ---- O += P V
#pragma unroll
        for (int p = 0; p < 4; p++) {
            uint2 vq[8];
#pragma unroll
            for (int i = 0; i < 8; i++) vq[i] = *(const uint2*)(vb + (8 * g + i) * VROW + (64 * p + 4 * n) * 2);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                bf16x8 vop;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    uint32_t w = (j < 2) ? vq[i].x : vq[i].y;
                    vop[i] = (short)((j & 1) ? (w >> 16) : (w & 0xffffu));
                }
                oacc[4 * p + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vop, oacc[4 * p + j], 0, 0, 0);
            }
        }
        wave_sync();  // this tile's LDS reads complete before the next tile overwrites
    }
    __syncthreads();  // all waves done with their V staging before the merge reuses it

    // ---- combine hi/lo rows and reduce l over the 16 key lanes
#pragma unroll
    for (int j = 0; j < 4; j++) {
        l_run[j] = row16_sum(l_run[j]);
    }
#pragma unroll
    for (int i = 0; i < 16; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) oacc[i][j] = half_swap_sum(oacc[i][j]);
    if (g < 2) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int h = 4 * g + j;
            if (n == 0) {
                wm[wave][h] = m_run[j];
                wl[wave][h] = l_run[j];
            }
#pragma unroll
            for (int p = 0; p < 4; p++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) wo[wave][h][64 * p + 4 * n + jj] = oacc[4 * p + jj][j];
        }
    }
    __syncthreads();
    // ---- merge the 4 waves; thread = (head r, 32-dim slice)
    const int tid = threadIdx.x;
    const int r = tid / 32, d0 = (tid % 32) * 8;
    if (r < G) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, wm[w][r]);
        float Lsum = 0.f, f[4];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            f[w] = wm[w][r] == -INFINITY ? 0.f : __expf(wm[w][r] - M);
            Lsum += wl[w][r] * f[w];
        }
        size_t pidx = (((size_t)b * KV + kvh) * nsplit + split) * G + r;
        float* po = part + pidx * HD + d0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float a = 0.f;
#pragma unroll
            for (int w = 0; w < 4; w++) a += wo[w][r][d0 + i] * f[w];
            po[i] = a;
        }
        if (d0 == 0) {
            ml[pidx * 2] = M;
            ml[pidx * 2 + 1] = Lsum;
        }
    }
}

// Split merge spread over the GPU: one workgroup per (sequence, KV head, query head), so a
// long context's many splits are combined by B KV G workgroups instead of B KV. Thread t holds
// output dims 4 (t % 64) .. +3 for the splits s = t / 64 (mod 4); the four split groups are added
// in a fixed order through LDS, so the result does not depend on timing.
template <typename TG, typename Tout>
__global__ void __launch_bounds__(256) attn_decode_merge_wide_kernel(const float* __restrict__ part,
                                                                     const float* __restrict__ ml,
                                                                     const TG* __restrict__ gate,
                                                                     long long gate_row_stride, Tout* __restrict__ out,
                                                                     long long out_row_stride, int H, int KV, int nsplit) {
    __shared__ float fw[256];
    __shared__ float red[2][4];
    __shared__ f32x4 acc_s[3][64];
    const int G = H / KV;
    const int r = blockIdx.x % G, u = blockIdx.x / G, b = u / KV, kvh = u % KV;
    const int tid = threadIdx.x, q4 = tid % 64, sg = tid / 64, lane = tid % WAVE, wave = tid / WAVE;
    const size_t base = (size_t)u * nsplit;
    // statistics: thread t holds split t (nsplit <= 256)
    const float2 st = tid < nsplit ? *(const float2*)(ml + ((base + tid) * G + r) * 2) : float2{-INFINITY, 0.f};
    const size_t row = (size_t)b * H + kvh * G + r;
    float gv[4];
#pragma unroll
    for (int e = 0; e < 4; e++) gv[e] = gate ? Act<TG>::ld(gate, row * gate_row_stride + 4 * q4 + e) : 0.f;
    // this thread's splits s = sg, sg + 4, ..., in batches of SB loads in flight; the first batch
    // is issued here, ahead of the statistics' reductions
    constexpr int SB = 8;
    f32x4 v[SB];
    auto load_batch = [&](int s0) {
#pragma unroll
        for (int e = 0; e < SB; e++) {
            const int sp = min(s0 + 4 * e, nsplit - 1);
            v[e] = *(const f32x4*)(part + ((base + sp) * G + r) * HD + 4 * q4);
        }
    };
    load_batch(sg);
    float mx = wave_max(st.x);
    if (lane == 0) red[0][wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    const float f = st.x == -INFINITY ? 0.f : __expf(st.x - mx);
    fw[tid] = f;
    float ls = wave_sum(st.y * f);
    if (lane == 0) red[1][wave] = ls;
    __syncthreads();
    ls = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = sg; s0 < nsplit; s0 += 4 * SB) {
        if (s0 != sg) load_batch(s0);
#pragma unroll
        for (int e = 0; e < SB; e++) {
            const int sp = s0 + 4 * e;
            a += v[e] * (sp < nsplit ? fw[sp] : 0.f);
        }
    }
    if (sg > 0) acc_s[sg - 1][q4] = a;
    __syncthreads();
    if (sg == 0) {
        a = ((a + acc_s[0][q4]) + acc_s[1][q4]) + acc_s[2][q4];
        const float inv = 1.f / ls;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float y = a[e] * inv;
            if (gate) y *= sigmoid_f(gv[e]);
            Act<Tout>::st(out, row * out_row_stride + 4 * q4 + e, y);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Causal prefill, one workgroup of 4 waves per (sequence, query head, 4 queries): each wave
// owns one query, lanes own 4 dims, keys are walked with an online softmax. Correct for any
// T; used for short prefills.
struct Strides3 {
    long long b, t, h;  // element strides of a [.., HD] row by sequence, token, head
};

__global__ void __launch_bounds__(256) attn_prefill_simple_kernel(const float* __restrict__ q, Strides3 qs,
                                                                  const uint16_t* __restrict__ kc,
                                                                  const uint16_t* __restrict__ vc,
                                                                  const float* __restrict__ gate, Strides3 gs,
                                                                  float* __restrict__ out, Strides3 os, int H, int KV,
                                                                  int T, int pos, int cap, float scale) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int t = blockIdx.x * 4 + wave, h = blockIdx.y, b = blockIdx.z;
    if (t >= T) return;
    const int G = H / KV, kvh = h / G;
    const float* qr = q + b * qs.b + t * qs.t + h * qs.h;
    float qv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) qv[i] = qr[lane * 4 + i];
    const uint16_t* kb = kc + ((size_t)b * KV + kvh) * (size_t)cap * HD;
    const uint16_t* vb = vc + ((size_t)b * KV + kvh) * (size_t)cap * HD;
    float m = -INFINITY, l = 0.f, a[4] = {0.f, 0.f, 0.f, 0.f};
    const int L = pos + t + 1;
    for (int key = 0; key < L; key++) {
        uint2 kp = *(const uint2*)(kb + (size_t)key * HD + lane * 4);
        float s = qv[0] * bf_lo(kp.x) + qv[1] * bf_hi(kp.x) + qv[2] * bf_lo(kp.y) + qv[3] * bf_hi(kp.y);
        s = wave_sum(s) * scale;
        float mn = fmaxf(m, s);
        float corr = __expf(m - mn), p = __expf(s - mn);
        uint2 vp = *(const uint2*)(vb + (size_t)key * HD + lane * 4);
        l = l * corr + p;
        a[0] = a[0] * corr + p * bf_lo(vp.x);
        a[1] = a[1] * corr + p * bf_hi(vp.x);
        a[2] = a[2] * corr + p * bf_lo(vp.y);
        a[3] = a[3] * corr + p * bf_hi(vp.y);
        m = mn;
    }
    float* orow = out + b * os.b + t * os.t + h * os.h;
    const float* grow = gate ? gate + b * gs.b + t * gs.t + h * gs.h : nullptr;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float y = a[i] / l;
        if (grow) y *= sigmoid_f(grow[lane * 4 + i]);
        orow[lane * 4 + i] = y;
    }
}

// ---------------------------------------------------------------------------------------------
// Causal flash prefill on v_mfma_f32_16x16x32_f16, 16 queries per wave. One workgroup of 8 waves
// per (sequence, query head, 128 queries); wave w owns queries [16w, 16w + 16). Key tiles of 64
// rows. The 32-query kernels further down replace it; it serves the caches whose rows of one
// (sequence, KV head) pass 2 GiB (their buffer ranges are 32-bit) and A/B builds.
//
// Everything is computed transposed, so that a lane owns one query throughout:
//   S^T = K q^T     (A = K rows from LDS, B = q): lane (n, g) holds query n's scores for keys
//                   16 nb + 4 g + j (nb < 4, j < 4);
//   O^T += V^T P^T  (A = V^T through LDS transpose reads, B = P^T straight from the score
//                   registers): lane (n, g) accumulates query n's output dims 16 db + 4 g + j.
// The k index of a P V step runs over the 32 keys of two score blocks in the order the score
// registers hold them (lane group g: keys 4 g .. 4 g + 3 of block 2 ks, then of block 2 ks + 1);
// the V operand reads the same keys (ds_read_b64_tr_b16 hands lane j four consecutive keys of
// one dim), so P never goes through LDS and the online-softmax statistics of a query live in
// the four lanes n, n + 16, n + 32, n + 48 (max: two lane swaps; sum: kept per lane, reduced
// once at the end).
//
// K and V tiles are converted to fp16 as they are staged into LDS (exact for bf16 values in
// fp16's range), so q * scale and the probabilities enter as single fp16 operands (11
// significant bits; errors ~2e-4 of max|out|). Base-2 softmax (log2 e folded into the q scale);
// the accumulators are rescaled only when some query's running maximum moved; the causal mask
// is applied only on tiles that reach past a wave's first query; output * sigmoid(gate). A
// wave whose queries cannot see any key of a tile skips it.
// compile-time switches for A/B builds: PREFILL_W32 = 0 keeps every prefill on the 16-query
// kernel below, PREFILL_F16 = 0 ignores the workspace for the fp16 cache copy
#ifndef PREFILL_F16
#define PREFILL_F16 1
#endif
#ifndef PREFILL_W32
#define PREFILL_W32 1
#endif
constexpr int PQ = 128, PK = 64;  // queries per workgroup, keys per tile
constexpr int PW = PQ / 16;              // waves per workgroup
// LDS row strides (bf16 elements). K: 132 words = 4 mod 64 banks, so the 16 rows a 16-lane
// group reads with 16-byte loads cover all 64 banks. V: 136 words = 8 mod 64 banks: a transpose
// read touches 4 consecutive rows x 32 bytes per 16 lanes, and the two lane groups served in
// one cycle sit 4 rows (32 banks) apart.
constexpr int KLD = HD + 8, VLD = HD + 16;

typedef short short4v __attribute__((ext_vector_type(4)));

// A operand of O^T += V^T P^T for P V step ks and dim block db: lane (d, g) gets
// V[32 ks + 4 g + e][16 db + d] (e < 4), then V[32 ks + 16 + 4 g + e][16 db + d]. In a transpose
// read lane k addresses row R + k / 4, dims C + 4 (k % 4) .. +3; lane j receives rows R .. R + 3
// of dim C + j.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));  // (HIP's uint4 blocks register promotion)

// 8 bf16 (one 16-byte chunk of a cache row) -> 8 fp16, exact for |x| in fp16's normal range
// (bf16's 8-bit significand fits fp16's 11); the prefill kernel stages K and V tiles as fp16.
// Values beyond fp16's largest finite 65504 saturate to +-65504 (the output stays finite; bf16
// cache values that large differ from the reference by the clamp); below its normal range they
// round to fp16 subnormals.
__device__ __forceinline__ u32x4 bf8_to_f16(u32x4 x) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    constexpr float kMax = 65504.f;
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = __builtin_amdgcn_fmed3f(bf_lo(x[i]), -kMax, kMax);
        const float b = __builtin_amdgcn_fmed3f(bf_hi(x[i]), -kMax, kMax);
        r[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{a, b}), h2));
    }
    return r;
}

// max / sum over the four lanes n, n + 16, n + 32, n + 48 of a wave (its lane groups) by VALU
// lane swaps; a shuffle would be an LDS permute, whose wait also drains every LDS read in flight.
// Both halves of a swap pair combine in the same order, so every lane gets the same sum.
__device__ __forceinline__ float group4_max(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}
__device__ __forceinline__ float group4_sum(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

__device__ __forceinline__ bf16x8 vt_operand(const uint16_t* vt, int ks, int db, int lane) {
    const int g = lane / 16, k = lane % 16;
    const uint16_t* p = vt + (size_t)(32 * ks + 4 * g + (k >> 2)) * VLD + 16 * db + 4 * (k & 3);
    typedef __attribute__((address_space(3))) short4v lds_short4;
    const short4v a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(p));
    const short4v b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(p + 16 * VLD));
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__global__ void __launch_bounds__(64 * PW, 8 / PW) attn_prefill_mfma_kernel(const float* __restrict__ q, Strides3 qs,
                                                                     const uint16_t* __restrict__ kc,
                                                                     const uint16_t* __restrict__ vc,
                                                                     const float* __restrict__ gate, Strides3 gs,
                                                                     float* __restrict__ out, Strides3 os, int H,
                                                                     int KV, int T, int pos, int cap, float scale,
                                                                     int B, int per_xcd) {
    // double-buffered tiles (2 x 68.6 KB): tile t + 1 is written while tile t is read, one
    // barrier per tile
    __shared__ __attribute__((aligned(16))) uint16_t Kt2[2][PK * KLD];
    __shared__ __attribute__((aligned(16))) uint16_t Vt2[2][PK * VLD];

    // XCD-aware order (1-D grid of 8 per_xcd blocks, dealt round-robin to the 8 XCDs): XCD x
    // runs logical blocks [x per_xcd, (x + 1) per_xcd) in order, so the workgroups resident on
    // one XCD at a time belong to one (sequence, KV head) and share its K / V rows in that
    // XCD's L2. Within a (sequence, KV head): query head, then query blocks longest first.
    const int nqb = (T + PQ - 1) / PQ, G = H / KV;
    const int li = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (li >= nqb * H * B) return;
    const int qb = nqb - 1 - li % nqb, hh = (li / nqb) % G, kvh = (li / (nqb * G)) % KV, b = li / (nqb * H);
    const int h = kvh * G + hh;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, n = lane % 16, g = lane / 16;
    const int q0 = qb * PQ;  // first query (sequence-relative)
    const uint16_t* kbase = kc + ((size_t)b * KV + kvh) * (size_t)cap * HD;
    const uint16_t* vbase = vc + ((size_t)b * KV + kvh) * (size_t)cap * HD;

    // q operand (B of S^T): query n of this wave, dims 32 ks + 8 g .. +8, as fp16
    half8 qf[8];
    {
        const int t = min(q0 + 16 * wave + n, T - 1);
        const float* qr = q + b * qs.b + (long long)t * qs.t + h * qs.h;
        // scores in the log2 domain: exp(s) = exp2(s log2 e)
        const float sl = scale * 1.4426950408889634f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            const float4 a0 = *(const float4*)(qr + 32 * ks + 8 * g);
            const float4 a1 = *(const float4*)(qr + 32 * ks + 8 * g + 4);
            qf[ks] = half8{(_Float16)(a0.x * sl), (_Float16)(a0.y * sl), (_Float16)(a0.z * sl), (_Float16)(a0.w * sl),
                           (_Float16)(a1.x * sl), (_Float16)(a1.y * sl), (_Float16)(a1.z * sl), (_Float16)(a1.w * sl)};
        }
    }
    const int qpos = pos + q0 + 16 * wave + n;  // this lane's query position in the cache
    float m_run = -INFINITY, l_part = 0.f;     // l_part: this lane's share of the row sum
    f32x4 oacc[16];
#pragma unroll
    for (int i = 0; i < 16; i++) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int last_key = pos + min(q0 + PQ, T) - 1;  // keys [0, last_key] are visible to this block
    const int ntiles = last_key / PK + 1;
    const int wave_last = pos + min(q0 + 16 * wave + 15, T - 1);  // the last key this wave's rows see
    const int wave_first = pos + q0 + 16 * wave;                  // keys up to here need no mask
    // Tile staging: 16-byte chunk c8 of key row r; the next tile is held in registers, requested
    // a full tile ahead.
    constexpr int NSTEP = (PK * HD) / (8 * 64 * PW);
    constexpr int RSTEP = 64 * PW / (HD / 8);  // key rows between a thread's chunks
    const int r_own = tid / (HD / 8), c_own = (tid % (HD / 8)) * 8;
    u32x4 kreg[NSTEP], vreg[NSTEP];
#pragma unroll
    for (int it = 0; it < NSTEP; it++) {
        const size_t off = (size_t)min(r_own + it * RSTEP, last_key) * HD + c_own;
        kreg[it] = *(const u32x4*)(kbase + off);
        vreg[it] = *(const u32x4*)(vbase + off);
    }
    auto stage = [&](int buf) {
#pragma unroll
        for (int it = 0; it < NSTEP; it++) {
            const int r = r_own + it * RSTEP;
            *(u32x4*)&Kt2[buf][r * KLD + c_own] = bf8_to_f16(kreg[it]);
            *(u32x4*)&Vt2[buf][r * VLD + c_own] = bf8_to_f16(vreg[it]);
        }
    };
    auto request = [&](int t) {  // tile t (clamped: static wait counts) into the registers
        const int kn = min(t, ntiles - 1) * PK;
#pragma unroll
        for (int it = 0; it < NSTEP; it++) {
            const size_t off = (size_t)min(kn + r_own + it * RSTEP, last_key) * HD + c_own;
            kreg[it] = *(const u32x4*)(kbase + off);
            vreg[it] = *(const u32x4*)(vbase + off);
        }
    };
    stage(0);
    request(1);
    __syncthreads();
    for (int kt = 0; kt < ntiles; kt++) {
        const int key0 = kt * PK, cur = kt & 1;
        const uint16_t* Kt = Kt2[cur];
        const uint16_t* Vt = Vt2[cur];
        // tile kt + 1 into the other buffer: its last reader (tile kt - 1) passed the barrier
        // that ends the previous iteration
        if (kt + 1 < ntiles) stage(cur ^ 1);
        request(kt + 2);
        if (key0 <= wave_last) {  // else no query of this wave sees any key of this tile
        // ---- S^T for 4 blocks of 16 keys: sc[nb][j] = score of key key0 + 16 nb + 4 g + j
        f32x4 sc[4];
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                const half8 kb = *(const half8*)&Kt[(16 * nb + n) * KLD + 32 * ks + 8 * g];
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb, qf[ks], acc, 0, 0, 0);
            }
            sc[nb] = acc;
        }
        // causal mask, only on a tile that reaches past this wave's first query
        if (key0 + PK - 1 > wave_first) {
#pragma unroll
            for (int nb = 0; nb < 4; nb++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (key0 + 16 * nb + 4 * g + j > qpos) sc[nb][j] = -INFINITY;
        }
        float mt = sc[0][0];
#pragma unroll
        for (int nb = 0; nb < 4; nb++)
#pragma unroll
            for (int j = 0; j < 4; j++) mt = fmaxf(mt, sc[nb][j]);
        mt = group4_max(mt);
        const float mn = fmaxf(m_run, mt);
        const float ref = mn == -INFINITY ? 0.f : mn;
        const float corr = exp2f(m_run - ref);
        const bool moved = mn != m_run;
        m_run = mn;
        half8 pf[2];
        float ps = 0.f;
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int nb = 2 * ks + (e >> 2), j = e & 3;
                const float p = __builtin_amdgcn_exp2f(sc[nb][j] - ref);
                ps += p;
                pf[ks][e] = (_Float16)p;
            }
        l_part = l_part * corr + ps;
        if (__ballot(moved)) {
#pragma unroll
            for (int i = 0; i < 16; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) oacc[i][j] *= corr;
        }
#pragma unroll
        for (int db = 0; db < 16; db++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const half8 va = __builtin_bit_cast(half8, vt_operand(Vt, ks, db, lane));
                oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pf[ks], oacc[db], 0, 0, 0);
            }
        }
        __syncthreads();  // tile kt + 1 staged by every wave; tile kt's reads done
    }
    // ---- normalise, gate, store: lane holds query n, dims 16 db + 4 g .. +4
    const float l = group4_sum(l_part);
    // all sixteen gate loads are issued together (from a clamped row for queries past T, whose
    // stores are skipped): written per dim block behind the gate test, they had been issued and
    // waited for one at a time, ~13 us per workgroup at B = 16
    const int t = q0 + 16 * wave + n;
    const int tc = min(t, T - 1);
    f32x4 gf[16];
    if (gate) {
        const float* grow = gate + b * gs.b + (long long)tc * gs.t + h * gs.h;
#pragma unroll
        for (int db = 0; db < 16; db++) gf[db] = *(const f32x4*)(grow + 16 * db + 4 * g);
#pragma unroll
        for (int db = 0; db < 16; db++)
#pragma unroll
            for (int j = 0; j < 4; j++) gf[db][j] = sigmoid_rcp(gf[db][j]);
    } else {
#pragma unroll
        for (int db = 0; db < 16; db++) gf[db] = f32x4{1.f, 1.f, 1.f, 1.f};
    }
    float* orow = out + b * os.b + (long long)tc * os.t + h * os.h;
    const float inv = 1.f / l;
    if (t < T) {
#pragma unroll
        for (int db = 0; db < 16; db++) {
            const f32x4 y = oacc[db] * inv * gf[db];
            *(float4*)(orow + 16 * db + 4 * g) = float4{y[0], y[1], y[2], y[3]};
        }
    }
}


// ---------------------------------------------------------------------------------------------
// Causal prefill with 32 queries per wave: 4 waves x 32 queries = 128 queries per workgroup,
// one wave per SIMD (up to 512 registers: the 2 x 16 output tiles live in accumulators). Each K
// fragment and each V^T fragment read from LDS feeds two products (one per 16-query tile), half
// the LDS bytes per FLOP of the 16-query layout. One wave per SIMD leaves no other wave to fill
// the matrix pipe while a wave runs its softmax or stages tiles, so the loop is software-
// pipelined across tiles and the order of each iteration is fixed by scheduling fences:
//   phase 1: S^T of tile t + 1 (64 products), between them the fp16 staging of V tile t + 1 into
//            the other V buffer and the requests of K tile t + 2;
//   phase 2: O^T += V^T P^T of tile t (64 products), between them the softmax of tile t + 1, the
//            staging of K tile t + 2 into the K buffer tile t used and the requests of V t + 2;
//   barrier.
// K runs a tile ahead of V: iteration t reads K(t + 1) and V(t), writes K(t + 2) and V(t + 1).
// Both buffers written in an iteration were last read before the barrier that ended the
// previous one. The softmax reference is lazy: it moves only when a query's tile maximum exceeds
// it by more than 2^8, so probabilities stay <= 2^8 (exact range for fp16) and the accumulators
// are rescaled rarely - at the start of the next iteration, after P V of the tile that used the
// old reference. All four waves run every tile of their block; a tile none of a wave's queries
// sees gets fully masked (probabilities 0), which keeps the control flow uniform.
constexpr int WQ = 32, PQ2 = 128, PW2 = PQ2 / WQ;
// 4 consecutive outputs as fp32 (16 bytes) or bf16 (8 bytes, rounded to nearest even)
__device__ __forceinline__ void store4(float* p, f32x4 y) { *(float4*)p = float4{y[0], y[1], y[2], y[3]}; }
__device__ __forceinline__ void store4(uint16_t* p, f32x4 y) { *(uint2*)p = uint2{f2bf2(y[0], y[1]), f2bf2(y[2], y[3])}; }
constexpr int NST2 = (PK * HD) / (8 * 64 * PW2);  // 16-byte chunks per thread per tile (K; V alike)
constexpr int RST2 = 64 * PW2 / (HD / 8);         // key rows between a thread's chunks
constexpr float kLazyRef = 8.f;                    // log2 units
constexpr int kBufWord3 = 0x00020000;              // buffer resource word 3 on gfx9: 32-bit data, no swizzle

template <typename Tout>
__global__ void __launch_bounds__(64 * PW2, 1) attn_prefill_w32_kernel(const float* __restrict__ q, Strides3 qs,
                                                                       const uint16_t* __restrict__ kc,
                                                                       const uint16_t* __restrict__ vc,
                                                                       const float* __restrict__ gate, Strides3 gs,
                                                                       Tout* __restrict__ out, Strides3 os, int H,
                                                                       int KV, int T, int pos, int cap, float scale,
                                                                       int B, int per_xcd) {
    __shared__ __attribute__((aligned(16))) uint16_t Kt2[2][PK * KLD];
    __shared__ __attribute__((aligned(16))) uint16_t Vt2[2][PK * VLD];

    // same XCD-aware block order as attn_prefill_mfma_kernel
    const int nqb = (T + PQ2 - 1) / PQ2, G = H / KV;
    const int li = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (li >= nqb * H * B) return;
    const int qb = nqb - 1 - li % nqb, hh = (li / nqb) % G, kvh = (li / (nqb * G)) % KV, b = li / (nqb * H);
    const int h = kvh * G + hh;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, n = lane % 16, g = lane / 16;
    const int q0 = qb * PQ2;
    const uint16_t* kbase = kc + ((size_t)b * KV + kvh) * (size_t)cap * HD;
    const uint16_t* vbase = vc + ((size_t)b * KV + kvh) * (size_t)cap * HD;
    const int last_key = pos + min(q0 + PQ2, T) - 1;
    const int ntiles = last_key / PK + 1;
    const int wave_first = pos + q0 + WQ * wave;  // keys up to here need no mask

    // staging: chunk it of a thread is key row r_own + it RST2, dims c_own .. +7, read by raw
    // buffer loads whose range ends at the block's last key (rows past it, and tiles past the
    // last, read as zeros: those keys are masked for every query of the block)
    const int r_own = tid / (HD / 8), c_own = (tid % (HD / 8)) * 8;
    const int voff = (r_own * HD + c_own) * 2;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, (last_key + 1) * HD * 2,
                                                                       kBufWord3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, (last_key + 1) * HD * 2,
                                                                       kBufWord3);
    auto kload = [&](int t, int it) {
        return __builtin_amdgcn_raw_buffer_load_b128(krs, voff, (t * PK + it * RST2) * HD * 2, 0);
    };
    auto vload = [&](int t, int it) {
        return __builtin_amdgcn_raw_buffer_load_b128(vrs, voff, (t * PK + it * RST2) * HD * 2, 0);
    };
    u32x4 kreg[NST2], vreg[NST2];
#pragma unroll
    for (int it = 0; it < NST2; it++) {
        kreg[it] = kload(0, it);
        vreg[it] = vload(0, it);
    }

    // q operands: tile qt = query q0 + 32 wave + 16 qt + n, dims 32 ks + 8 g .. +8, scaled into
    // the log2 domain, fp16
    half8 qf[2][8];
    int qpos[2];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const int tq = q0 + WQ * wave + 16 * qt + n;
        qpos[qt] = pos + tq;
        const float* qr = q + b * qs.b + (long long)min(tq, T - 1) * qs.t + h * qs.h;
        const float sl = scale * 1.4426950408889634f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            const float4 a0 = *(const float4*)(qr + 32 * ks + 8 * g);
            const float4 a1 = *(const float4*)(qr + 32 * ks + 8 * g + 4);
            qf[qt][ks] = half8{(_Float16)(a0.x * sl), (_Float16)(a0.y * sl), (_Float16)(a0.z * sl),
                               (_Float16)(a0.w * sl), (_Float16)(a1.x * sl), (_Float16)(a1.y * sl),
                               (_Float16)(a1.z * sl), (_Float16)(a1.w * sl)};
        }
    }

    auto kdst = [&](int buf, int it) { return (u32x4*)&Kt2[buf][(r_own + it * RST2) * KLD + c_own]; };
    auto vdst = [&](int buf, int it) { return (u32x4*)&Vt2[buf][(r_own + it * RST2) * VLD + c_own]; };
    // tile 0 into buffers 0 and K(1) into K buffer 1; V(1) requested into the staging registers
    // (one set serves both tensors in the loop: V(t + 1) arrives there during the previous
    // iteration's P V phase and is converted in the S phase, which then requests K(t + 2) into
    // the same registers for the P V phase to convert)
#pragma unroll
    for (int it = 0; it < NST2; it++) {
        *kdst(0, it) = bf8_to_f16(kreg[it]);
        *vdst(0, it) = bf8_to_f16(vreg[it]);
    }
#pragma unroll
    for (int it = 0; it < NST2; it++) kreg[it] = kload(1, it);
#pragma unroll
    for (int it = 0; it < NST2; it++) *kdst(1, it) = bf8_to_f16(kreg[it]);
    u32x4 sreg[NST2];
#pragma unroll
    for (int it = 0; it < NST2; it++) sreg[it] = vload(1, it);
    __syncthreads();

    // S^T of the tile in K buffer kb_: sc[qt][nb][j] = score of key 16 nb + 4 g + j for query
    // tile qt. Dim step outer; K fragments two steps ahead through a 3-deep ring; `side(ks)` runs
    // after the products of step ks (its work is fenced into that step).
    f32x4 sc[2][4];
    auto scores = [&](const uint16_t* Kt, auto side) {
        half8 kb[3][4];
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
            kb[0][nb] = *(const half8*)&Kt[(16 * nb + n) * KLD + 8 * g];
            kb[1][nb] = *(const half8*)&Kt[(16 * nb + n) * KLD + 32 + 8 * g];
#pragma unroll
            for (int qt = 0; qt < 2; qt++) sc[qt][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
#pragma unroll
            for (int nb = 0; nb < 4; nb++)
#pragma unroll
                for (int qt = 0; qt < 2; qt++)
                    sc[qt][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[ks % 3][nb], qf[qt][ks], sc[qt][nb], 0, 0, 0);
            if (ks + 2 < 8) {
#pragma unroll
                for (int nb = 0; nb < 4; nb++)
                    kb[(ks + 2) % 3][nb] = *(const half8*)&Kt[(16 * nb + n) * KLD + 32 * (ks + 2) + 8 * g];
            }
            side(ks);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto mask = [&](int key0) {
        if (key0 + PK - 1 > wave_first) {
#pragma unroll
            for (int qt = 0; qt < 2; qt++)
#pragma unroll
                for (int nb = 0; nb < 4; nb++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if (key0 + 16 * nb + 4 * g + j > qpos[qt]) sc[qt][nb][j] = -INFINITY;
        }
    };

    // softmax state per query tile: lazy reference, this lane's share of the row sum
    float ref[2] = {-INFINITY, -INFINITY}, lsum[2] = {0.f, 0.f}, corr[2] = {1.f, 1.f}, mt[2];
    half8 pcur[2][2], pnext[2][2];
    bool pend = false;
    // softmax of the scores in sc, in pieces (so they can be spread between products):
    // piece 0 / 1: tile maximum of query tile 0 / 1; 2: cross-lane max; 3: reference update;
    // 4 .. 11: probabilities of 4 scores each (p = 2^(s - ref)); 12: pending-rescale flag
    auto softmax_piece = [&](int piece) {
        if (piece < 2) {
            const int qt = piece;
            float m = sc[qt][0][0];
#pragma unroll
            for (int nb = 0; nb < 4; nb++)
#pragma unroll
                for (int j = 0; j < 4; j++) m = fmaxf(m, sc[qt][nb][j]);
            mt[qt] = m;
        } else if (piece == 2) {
#pragma unroll
            for (int qt = 0; qt < 2; qt++) mt[qt] = group4_max(mt[qt]);
        } else if (piece == 3) {
            bool need_any = false;
#pragma unroll
            for (int qt = 0; qt < 2; qt++) {
                const bool need = mt[qt] > ref[qt] + kLazyRef;  // -inf tile maxima never move it
                corr[qt] = need ? exp2f(ref[qt] - mt[qt]) : 1.f;
                lsum[qt] *= corr[qt];
                ref[qt] = need ? mt[qt] : ref[qt];
                need_any |= need;
            }
            pend = __ballot(need_any) != 0;
        } else if (piece < 12) {
            const int e4 = piece - 4;  // scores 4 e4 .. 4 e4 + 3 of the 32: qt = e4 / 4, nb = e4 % 4
            const int qt = e4 >> 2, nb = e4 & 3;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float p = __builtin_amdgcn_exp2f(sc[qt][nb][j] - ref[qt]);
                lsum[qt] += p;
                // P^T operand of step ks = nb / 2: element 4 (nb % 2) + j
                pnext[qt][nb >> 1][4 * (nb & 1) + j] = (_Float16)p;
            }
        }
    };
    f32x4 oacc[2][16];
#pragma unroll
    for (int qt = 0; qt < 2; qt++)
#pragma unroll
        for (int db = 0; db < 16; db++) oacc[qt][db] = f32x4{0.f, 0.f, 0.f, 0.f};

    // tile 0: S, mask, softmax (the accumulators are zero: nothing to rescale)
    scores(Kt2[0], [&](int) {});
    mask(0);
#pragma unroll
    for (int piece = 0; piece < 12; piece++) softmax_piece(piece);
    pend = false;
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        pcur[qt][0] = pnext[qt][0];
        pcur[qt][1] = pnext[qt][1];
    }
    __syncthreads();

    // O^T += V^T P^T from V buffer Vt with pcur: 16 dim blocks of 4 products; V^T fragments three
    // blocks ahead through a 4-deep ring; `side(db)` runs after the products of block db
    auto pv = [&](const uint16_t* Vt, auto side) {
        bf16x8 vb[4][2];
#pragma unroll
        for (int d = 0; d < 3; d++) {
            vb[d][0] = vt_operand(Vt, 0, d, lane);
            vb[d][1] = vt_operand(Vt, 1, d, lane);
        }
#pragma unroll
        for (int db = 0; db < 16; db++) {
            if (db + 3 < 16) {
                vb[(db + 3) & 3][0] = vt_operand(Vt, 0, db + 3, lane);
                vb[(db + 3) & 3][1] = vt_operand(Vt, 1, db + 3, lane);
            }
#pragma unroll
            for (int ks = 0; ks < 2; ks++)  // the two products into one accumulator are not adjacent
#pragma unroll
                for (int qt = 0; qt < 2; qt++)
                    oacc[qt][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, vb[db & 3][ks]),
                                                                          pcur[qt][ks], oacc[qt][db], 0, 0, 0);
            side(db);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto rescale = [&]() {
        if (pend) {
#pragma unroll
            for (int qt = 0; qt < 2; qt++)
#pragma unroll
                for (int db = 0; db < 16; db++) oacc[qt][db] *= corr[qt];
        }
        pend = false;
    };

    for (int t = 0; t + 1 < ntiles; t++) {
        const int b1 = (t + 1) & 1, b0 = t & 1;
        // ---- phase 1: accumulators rescaled for tile t's reference; S^T of tile t + 1, with
        // V(t + 1) staged (chunk ks) and K(t + 2) requested (chunk ks) between the products
        rescale();
        scores(Kt2[b1], [&](int ks) {
            *vdst(b1, ks) = bf8_to_f16(sreg[ks]);
            sreg[ks] = kload(t + 2, ks);
        });
        mask((t + 1) * PK);
        // ---- phase 2: P V of tile t; the softmax of tile t + 1 over blocks 0 .. 11, K(t + 2)
        // staged and V(t + 2) requested over blocks 8 .. 15
        pv(Vt2[b0], [&](int db) {
            if (db < 12) softmax_piece(db);
            if (db >= 8) {
                const int it = db - 8;
                *kdst(b0, it) = bf8_to_f16(sreg[it]);
                sreg[it] = vload(t + 2, it);
            }
        });
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            pcur[qt][0] = pnext[qt][0];
            pcur[qt][1] = pnext[qt][1];
        }
        __syncthreads();
    }
    rescale();
    pv(Vt2[(ntiles - 1) & 1], [&](int) {});

    // ---- normalise, gate, store: lane holds query tile qt's query n, dims 16 db + 4 g .. +3;
    // all gate loads of a query tile issued together (clamped rows past T, stores skipped)
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const float l = group4_sum(lsum[qt]);
        const int tq = q0 + WQ * wave + 16 * qt + n;
        const int tc = min(tq, T - 1);
        f32x4 gf[16];
        if (gate) {
            const float* grow = gate + b * gs.b + (long long)tc * gs.t + h * gs.h;
#pragma unroll
            for (int db = 0; db < 16; db++) gf[db] = *(const f32x4*)(grow + 16 * db + 4 * g);
#pragma unroll
            for (int db = 0; db < 16; db++)
#pragma unroll
                for (int j = 0; j < 4; j++) gf[db][j] = sigmoid_rcp(gf[db][j]);
        } else {
#pragma unroll
            for (int db = 0; db < 16; db++) gf[db] = f32x4{1.f, 1.f, 1.f, 1.f};
        }
        Tout* orow = out + b * os.b + (long long)tc * os.t + h * os.h;
        const float inv = 1.f / l;
        if (tq < T) {
#pragma unroll
            for (int db = 0; db < 16; db++) store4(orow + 16 * db + 4 * g, oacc[qt][db] * inv * gf[db]);
        }
    }
}


// ---------------------------------------------------------------------------------------------
// fp16 copies of the K / V cache rows [0, rows) of every (sequence, KV head), rows padded to a
// whole tile with zeros: dst [B][KV][rows_pad][HD]. bf16 -> fp16 is exact for the values the
// normed keys and projected values hold (8-bit significand into 11). Converting once here
// replaces the per-tile conversion that every query block of every query head would repeat.
__global__ void attn_kv_f16_kernel(const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                                   uint16_t* __restrict__ kf, uint16_t* __restrict__ vf, int KV, int cap, int rows,
                                   int rows_pad, long long nchunks) {
    for (long long c = blockIdx.x * (long long)blockDim.x + threadIdx.x; c < nchunks;
         c += (long long)gridDim.x * blockDim.x) {
        const long long e = c * 8;                       // element offset in dst (one tensor)
        const long long bkv = e / ((long long)rows_pad * HD);
        const int r = (int)((e / HD) % rows_pad), d = (int)(e % HD);
        u32x4 ko = {0u, 0u, 0u, 0u}, vo = {0u, 0u, 0u, 0u};
        if (r < rows) {
            const size_t src = ((size_t)bkv * cap + r) * HD + d;
            ko = bf8_to_f16(*(const u32x4*)(kc + src));
            vo = bf8_to_f16(*(const u32x4*)(vc + src));
        }
        *(u32x4*)(kf + e) = ko;
        *(u32x4*)(vf + e) = vo;
    }
}

// The 32-query kernel fed from the fp16 copies: every tile arrives in LDS by direct buffer ->
// LDS loads (1 KB = two key rows per instruction, no registers, no conversion), issued at the
// start of the S phase and waited for before the iteration's barrier. LDS rows are unpadded
// (512 bytes); 16-byte slots are XOR-swizzled by the row (K: slot ^ (row & 15), V: slot ^
// 2 (row & 15)) through the global address each lane fetches, so the K fragment reads (16 rows,
// one slot each) and the V^T transpose reads (4 rows x 2 slots per 16 lanes) hit distinct banks.
// The loop is unrolled by two so that each buffer is its own array and the compiler can tell the
// direct loads into one buffer from the reads of the other.
constexpr int KSW = 1, VSW = 2;  // swizzle multipliers of (row & 15)

__device__ __forceinline__ int sw_slot(int slot, int row, int mul) { return slot ^ ((row & 15) * mul); }

__device__ __forceinline__ bf16x8 vt_operand_sw(const uint16_t* vt, int ks, int db, int lane) {
    const int g = lane / 16, k = lane % 16;
    const int r0 = 32 * ks + 4 * g + (k >> 2), r1 = r0 + 16;
    const int gs = 2 * db + ((k & 3) >> 1), within = (k & 1) * 4;
    typedef __attribute__((address_space(3))) short4v lds_short4;
    const short4v a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4*)(vt + r0 * HD + sw_slot(gs, r0, VSW) * 8 + within));
    const short4v b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4*)(vt + r1 * HD + sw_slot(gs, r1, VSW) * 8 + within));
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

template <typename Tout>
__global__ void __launch_bounds__(64 * PW2, 1) attn_prefill_w32f_kernel(const float* __restrict__ q, Strides3 qs,
                                                                        const uint16_t* __restrict__ kf,
                                                                        const uint16_t* __restrict__ vf, int rows_pad,
                                                                        const float* __restrict__ gate, Strides3 gs,
                                                                        Tout* __restrict__ out, Strides3 os, int H,
                                                                        int KV, int T, int pos, float scale, int B) {
    __shared__ __attribute__((aligned(1024))) uint16_t K0[PK * HD];
    __shared__ __attribute__((aligned(1024))) uint16_t K1[PK * HD];
    __shared__ __attribute__((aligned(1024))) uint16_t V0[PK * HD];
    __shared__ __attribute__((aligned(1024))) uint16_t V1[PK * HD];

    // persistent workgroups (one per CU) walk a static schedule of (query block, head, sequence)
    // items, longest query blocks first, so no CU waits on the dispatcher between items. The items
    // of a (sequence, KV head) pair stay on few XCDs, whose workgroups share the pair's K / V rows
    // in their L2: with pairs a multiple of 8, XCD x owns pairs x, x + 8, ...; with pairs dividing
    // 8, the rep = 8 / pairs XCDs x = p (mod pairs) split pair p's query heads (head x / pairs,
    // then every rep-th). Items of one query block index form a round, and rounds alternate
    // direction over the workgroups.
    const int nqb = (T + PQ2 - 1) / PQ2, G = H / KV, npairs = B * KV, xcd = blockIdx.x % 8;
    const bool g8 = gridDim.x % 8 == 0;
    const int rep = g8 && npairs % 8 == 0 ? 1 : (g8 && 8 % npairs == 0 && G % (8 / npairs) == 0 ? 8 / npairs : 0);
    const bool aff = rep != 0;
    const int np_x = !aff ? npairs : (rep == 1 ? npairs / 8 : 1), hpx = aff ? G / rep : G;
    const int P = aff ? gridDim.x / 8 : gridDim.x, jw = aff ? blockIdx.x / 8 : blockIdx.x;
    const int items = np_x * hpx * nqb;
    for (int round = 0;; round++) {
        const int m = round * P + ((round & 1) ? P - 1 - jw : jw);
        if (m >= items) break;
        const int qb = nqb - 1 - m / (np_x * hpx), pi = (m % (np_x * hpx)) / hpx, hl = m % hpx;
        const int pair = !aff ? pi : (rep == 1 ? xcd + 8 * pi : xcd % npairs);
        const int hh = rep > 1 ? hl * rep + xcd / npairs : hl;
        const int kvh = pair % KV, b = pair / KV;
        const int h = kvh * G + hh;
        const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, n = lane % 16, g = lane / 16;
        const int q0 = qb * PQ2;
        const size_t base = ((size_t)b * KV + kvh) * (size_t)rows_pad * HD;
        const int last_key = pos + min(q0 + PQ2, T) - 1;
        const int ntiles = last_key / PK + 1;
        const int wave_first = pos + q0 + WQ * wave;

        // direct loads: instruction i of this wave fills key rows 2 j, 2 j + 1 (j = 8 wave + i) of a
        // tile; lane L writes LDS slot L % 32 of row 2 j + L / 32 with global slot (L % 32) ^ swizzle
        const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)(kf + base), (short)0,
                                                                           rows_pad * HD * 2, kBufWord3);
        const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)(vf + base), (short)0,
                                                                           rows_pad * HD * 2, kBufWord3);
        int koff[8], voff[8];
    #pragma unroll
        for (int i = 0; i < 8; i++) {
            const int row = 2 * (8 * wave + i) + lane / 32, s = lane % 32;
            koff[i] = (row * HD + sw_slot(s, row, KSW) * 8) * 2;
            voff[i] = (row * HD + sw_slot(s, row, VSW) * 8) * 2;
        }
        typedef __attribute__((address_space(3))) void lds_void;
        auto load_k = [&](uint16_t* dst, int t) {
    #pragma unroll
            for (int i = 0; i < 8; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)(dst + (8 * wave + i) * 2 * HD), 16, koff[i],
                                                         t * PK * HD * 2, 0, 0);
        };
        auto load_v = [&](uint16_t* dst, int t) {
    #pragma unroll
            for (int i = 0; i < 8; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(dst + (8 * wave + i) * 2 * HD), 16, voff[i],
                                                         t * PK * HD * 2, 0, 0);
        };
        load_k(K0, 0);
        load_v(V0, 0);
        if (ntiles > 1) load_k(K1, 1);

        half8 qf[2][8];
        int qpos[2];
    #pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            const int tq = q0 + WQ * wave + 16 * qt + n;
            qpos[qt] = pos + tq;
            const float* qr = q + b * qs.b + (long long)min(tq, T - 1) * qs.t + h * qs.h;
            const float sl = scale * 1.4426950408889634f;
    #pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                const float4 a0 = *(const float4*)(qr + 32 * ks + 8 * g);
                const float4 a1 = *(const float4*)(qr + 32 * ks + 8 * g + 4);
                qf[qt][ks] = half8{(_Float16)(a0.x * sl), (_Float16)(a0.y * sl), (_Float16)(a0.z * sl),
                                   (_Float16)(a0.w * sl), (_Float16)(a1.x * sl), (_Float16)(a1.y * sl),
                                   (_Float16)(a1.z * sl), (_Float16)(a1.w * sl)};
            }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();

        f32x4 sc[2][4];
        float ref[2] = {-INFINITY, -INFINITY}, lsum[2] = {0.f, 0.f}, corr[2] = {1.f, 1.f};
        float lsave[2], mx[2];
        half8 pcur[2][2], pnext[2][2];
        bool pend = false;
        // masked: the tile may hold keys past some query of the block; tiles wholly before the
        // block's first query take the unmasked form (no compares or selects). nb0: first of the
        // two key blocks of 16 it covers.
        auto mask = [&](int key0, int nb0, auto masked) __attribute__((always_inline)) {
            if (decltype(masked)::value && key0 + PK - 1 > wave_first) {
    #pragma unroll
                for (int qt = 0; qt < 2; qt++)
    #pragma unroll
                    for (int nb = nb0; nb < nb0 + 2; nb++)
    #pragma unroll
                        for (int j = 0; j < 4; j++)
                            if (key0 + 16 * nb + 4 * g + j > qpos[qt]) sc[qt][nb][j] = -INFINITY;
            }
        };
        // Softmax of a tile, in pieces placed among the products. The exponentials are taken
        // against the current (lazy) reference straight away, so the first two key blocks' pieces
        // run among the last score products of the tile; each piece also keeps this lane's
        // maximum. finish() then checks whether some row's maximum passed the reference by more
        // than 2^8: only then (the first tile, and rarely after) are the row maxima reduced and,
        // where needed, the reference moved, the row sum rescaled and the exponentials taken again
        // - the same values and order of operations as reducing the maxima first.
        auto begin_tile = [&]() __attribute__((always_inline)) {
    #pragma unroll
            for (int qt = 0; qt < 2; qt++) {
                lsave[qt] = lsum[qt];
                mx[qt] = -INFINITY;
            }
        };
        auto exp_piece = [&](int qt, int nb) __attribute__((always_inline)) {
    #pragma unroll
            for (int j = 0; j < 4; j++) {
                mx[qt] = fmaxf(mx[qt], sc[qt][nb][j]);
                const float p = __builtin_amdgcn_exp2f(sc[qt][nb][j] - ref[qt]);
                lsum[qt] += p;
                pnext[qt][nb >> 1][4 * (nb & 1) + j] = (_Float16)p;
            }
            // pin the exponentials here, among this tile's products: otherwise they are sunk to
            // their first use after the loop's barrier, where nothing overlaps them
            if (nb & 1) asm volatile("" : "+v"(pnext[qt][nb >> 1]));
            asm volatile("" : "+v"(lsum[qt]));
        };
        auto finish = [&]() __attribute__((always_inline)) {
            bool over = false;
    #pragma unroll
            for (int qt = 0; qt < 2; qt++) over |= mx[qt] > ref[qt] + kLazyRef;
            pend = false;
            if (__ballot(over) != 0) {
                bool need_any = false;
    #pragma unroll
                for (int qt = 0; qt < 2; qt++) {
                    const float mt = group4_max(mx[qt]);
                    const bool need = mt > ref[qt] + kLazyRef;
                    corr[qt] = need ? exp2f(ref[qt] - mt) : 1.f;
                    lsum[qt] = lsave[qt] * corr[qt];
                    ref[qt] = need ? mt : ref[qt];
                    need_any |= need;
    #pragma unroll
                    for (int nb = 0; nb < 4; nb++)
    #pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const float p = __builtin_amdgcn_exp2f(sc[qt][nb][j] - ref[qt]);
                            lsum[qt] += p;
                            pnext[qt][nb >> 1][4 * (nb & 1) + j] = (_Float16)p;
                        }
                }
                pend = __ballot(need_any) != 0;
            }
        };
        // scores of a tile in two halves (key blocks 0-1, then 2-3), each over the 8 k steps;
        // the first half's masked softmax pieces run among the second half's products
        auto scores = [&](const uint16_t* Kt, int key0, auto masked) __attribute__((always_inline)) {
            auto kaddr = [&](int nb, int ks) {
                const int row = 16 * nb + n;
                return (const half8*)&Kt[row * HD + sw_slot(4 * ks + g, row, KSW) * 8];
            };
    #pragma unroll
            for (int h = 0; h < 2; h++) {
                half8 kb[3][2];
    #pragma unroll
                for (int i = 0; i < 2; i++) {
                    kb[0][i] = *kaddr(2 * h + i, 0);
                    kb[1][i] = *kaddr(2 * h + i, 1);
    #pragma unroll
                    for (int qt = 0; qt < 2; qt++) sc[qt][2 * h + i] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
    #pragma unroll
                for (int ks = 0; ks < 8; ks++) {
    #pragma unroll
                    for (int i = 0; i < 2; i++)
    #pragma unroll
                        for (int qt = 0; qt < 2; qt++)
                            sc[qt][2 * h + i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[ks % 3][i], qf[qt][ks],
                                                                                     sc[qt][2 * h + i], 0, 0, 0);
                    if (ks + 2 < 8) {
    #pragma unroll
                        for (int i = 0; i < 2; i++) kb[(ks + 2) % 3][i] = *kaddr(2 * h + i, ks + 2);
                    }
                    if (h == 1 && ks < 4) exp_piece(ks >> 1, ks & 1);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (h == 0) {
                    mask(key0, 0, masked);
                    begin_tile();
                }
            }
            mask(key0, 2, masked);
        };
        f32x4 oacc[2][16];
    #pragma unroll
        for (int qt = 0; qt < 2; qt++)
    #pragma unroll
            for (int db = 0; db < 16; db++) oacc[qt][db] = f32x4{0.f, 0.f, 0.f, 0.f};

        scores(K0, 0, std::true_type{});
    #pragma unroll
        for (int e = 0; e < 4; e++) exp_piece(e >> 1, 2 + (e & 1));
        finish();
        pend = false;
    #pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            pcur[qt][0] = pnext[qt][0];
            pcur[qt][1] = pnext[qt][1];
        }
        __syncthreads();  // K0 free for K(2)

        auto pv = [&](const uint16_t* Vt, auto side) {
            bf16x8 vb[4][2];
    #pragma unroll
            for (int d = 0; d < 3; d++) {
                vb[d][0] = vt_operand_sw(Vt, 0, d, lane);
                vb[d][1] = vt_operand_sw(Vt, 1, d, lane);
            }
    #pragma unroll
            for (int db = 0; db < 16; db++) {
                if (db + 3 < 16) {
                    vb[(db + 3) & 3][0] = vt_operand_sw(Vt, 0, db + 3, lane);
                    vb[(db + 3) & 3][1] = vt_operand_sw(Vt, 1, db + 3, lane);
                }
    #pragma unroll
                for (int ks = 0; ks < 2; ks++)
    #pragma unroll
                    for (int qt = 0; qt < 2; qt++)
                        oacc[qt][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, vb[db & 3][ks]),
                                                                              pcur[qt][ks], oacc[qt][db], 0, 0, 0);
                side(db);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        auto rescale = [&]() {
            if (pend) {
    #pragma unroll
                for (int qt = 0; qt < 2; qt++)
    #pragma unroll
                    for (int db = 0; db < 16; db++) oacc[qt][db] *= corr[qt];
            }
            pend = false;
        };
        // iteration t: S of K(t + 1) (buffer Kn), P V of V(t) (buffer Vc); loads of K(t + 2) into
        // the K buffer tile t used (Kc) and of V(t + 1) into the other V buffer (Vn)
        auto iteration = [&](int t, uint16_t* Kc, uint16_t* Kn, uint16_t* Vc, uint16_t* Vn, auto masked) {
            load_v(Vn, t + 1);
            if (t + 2 < ntiles) load_k(Kc, t + 2);
            rescale();
            scores(Kn, (t + 1) * PK, masked);
            pv(Vc, [&](int db) {
                if (db < 4) exp_piece(db >> 1, 2 + (db & 1));
            });
            finish();
    #pragma unroll
            for (int qt = 0; qt < 2; qt++) {
                pcur[qt][0] = pnext[qt][0];
                pcur[qt][1] = pnext[qt][1];
            }
            __builtin_amdgcn_s_waitcnt(0);  // this wave's direct loads have landed
            __syncthreads();
        };
        // tiles below nfree end at or before the block's first query: no key of theirs is masked
        const int nfree = (pos + q0 + 1) / PK;
        int t = 0;
        for (; t + 2 < ntiles && t + 2 < nfree; t += 2) {
            iteration(t, K0, K1, V0, V1, std::false_type{});
            iteration(t + 1, K1, K0, V1, V0, std::false_type{});
        }
        for (; t + 2 < ntiles; t += 2) {
            iteration(t, K0, K1, V0, V1, std::true_type{});
            iteration(t + 1, K1, K0, V1, V0, std::true_type{});
        }
        if (t + 1 < ntiles) {
            iteration(t, K0, K1, V0, V1, std::true_type{});
            t++;
        }
        rescale();
        pv((t & 1) ? V1 : V0, [&](int) {});

    #pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            const float l = group4_sum(lsum[qt]);
            const int tq = q0 + WQ * wave + 16 * qt + n;
            const int tc = min(tq, T - 1);
            f32x4 gf[16];
            if (gate) {
                const float* grow = gate + b * gs.b + (long long)tc * gs.t + h * gs.h;
    #pragma unroll
                for (int db = 0; db < 16; db++) gf[db] = *(const f32x4*)(grow + 16 * db + 4 * g);
    #pragma unroll
                for (int db = 0; db < 16; db++)
    #pragma unroll
                    for (int j = 0; j < 4; j++) gf[db][j] = sigmoid_rcp(gf[db][j]);
            } else {
    #pragma unroll
                for (int db = 0; db < 16; db++) gf[db] = f32x4{1.f, 1.f, 1.f, 1.f};
            }
            Tout* orow = out + b * os.b + (long long)tc * os.t + h * os.h;
            const float inv = 1.f / l;
            if (tq < T) {
    #pragma unroll
                for (int db = 0; db < 16; db++) store4(orow + 16 * db + 4 * g, oacc[qt][db] * inv * gf[db]);
            }
        }
        __syncthreads();  // every wave is done with the tile buffers before the next item's loads
    }
}

}  // namespace

namespace aegist {

size_t decode_workspace_bytes(int B, int H, int KV, int L, bool with_q) {
    DecodeSplit sp = choose_split(B, KV, L);
    int G = H / std::max(1, KV);
    size_t part = (size_t)B * KV * sp.nsplit * G * HD * 4;
    size_t ml = (size_t)B * KV * sp.nsplit * G * 2 * 4;
    size_t qb = with_q ? (size_t)B * H * HD * 4 : 0;
    auto al = [](size_t x) { return (x + 255) / 256 * 256; };
    return al(part) + al(ml) + al(qb);
}

// q [B, H, HD] fp32 -> out rows (b*H + h) * out_row_stride, gate rows (b*H + h) * gate_row_stride
template <typename TG, typename Tout>
int launch_decode_core(const float* q, const uint16_t* kc, const uint16_t* vc, const TG* gate, long long gate_stride,
                       Tout* out, long long out_stride, int B, int H, int KV, int L, int cap, float scale,
                       void* ws, size_t ws_bytes, hipStream_t st, KeyList kl = KeyList{nullptr, nullptr, 0, 0, 0},
                       const FusedPrep* fused = nullptr, int fused_dtype = 0) {
    if (KV <= 0 || H % KV || H / KV > 8) return fail(AEGIST_ERR_SHAPE, "attention decode: need H % KV == 0 and H/KV <= 8");
    if (L <= 0 || L > cap) return fail(AEGIST_ERR_SHAPE, "attention decode: need 0 < L <= cap");
    DecodeSplit sp = choose_split(B, KV, L);
    size_t need = decode_workspace_bytes(B, H, KV, L, false);
    if (!ws || ws_bytes < need) return fail(AEGIST_ERR_WORKSPACE, "attention decode: workspace too small");
    int G = H / KV;
    float* part = (float*)ws;
    size_t part_bytes = ((size_t)B * KV * sp.nsplit * G * HD * 4 + 255) / 256 * 256;
    float* ml = (float*)((char*)ws + part_bytes);
    const dim3 grid(sp.nsplit, KV, B);
    // Batched calls read the caches with nontemporal loads: each K / V byte is used once, and
    // kept out of L2 / MALL the stream runs faster (B = 64, L = 4096: 108 -> 94 us; B = 8,
    // L = 32768: 103 -> 93 us). A batch-1 call (two (sequence, KV head) units) measured 3-5%
    // slower that way at L = 131072, so it keeps ordinary loads.
    const bool nt = (long long)B * KV >= 8;
#define AEG_SPLIT(LIST, FUSED, TIN, F)                                                                          \
    do {                                                                                                         \
        if (nt)                                                                                                  \
            attn_decode_split_kernel<LIST, FUSED, TIN, true><<<grid, 256, 0, st>>>(q, kc, vc, part, ml, H, KV, L, \
                                                                                  cap, sp.per_split, scale, kl, F); \
        else                                                                                                     \
            attn_decode_split_kernel<LIST, FUSED, TIN, false><<<grid, 256, 0, st>>>(q, kc, vc, part, ml, H, KV, L, \
                                                                                   cap, sp.per_split, scale, kl, F); \
    } while (0)
    if (fused && fused_dtype == AEGIST_BF16)
        AEG_SPLIT(false, true, uint16_t, *fused);
    else if (fused)
        AEG_SPLIT(false, true, float, *fused);
    else if (kl.blist)
        AEG_SPLIT(true, false, float, FusedPrep{});
    else
        AEG_SPLIT(false, false, float, FusedPrep{});
#undef AEG_SPLIT
    int rc = after_launch("attention_decode_split");
    if (rc) return rc;
    attn_decode_merge_wide_kernel<TG, Tout><<<B * KV * G, 256, 0, st>>>(part, ml, gate, gate_stride, out, out_stride,
                                                                       H, KV, sp.nsplit);
    return after_launch("attention_decode_merge");
}

// compute units of the current device (cached per device; the persistent prefill grid)
static int device_cus() {
    static std::atomic<int> cus[64];  // per device; racing first calls store the same value
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int c = cus[dev].load(std::memory_order_relaxed);
    if (c <= 0) {
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

// bytes of the fp16 K / V copies the prefill kernel reads when given that much workspace
size_t prefill_f16_bytes(int B, int KV, int rows) {
    const size_t rows_pad = (size_t)(rows + PK - 1) / PK * PK;
    return 2 * (size_t)B * KV * rows_pad * HD * 2;
}

int launch_prefill_core(const float* q, Strides3 qs, const uint16_t* kc, const uint16_t* vc, const float* gate,
                        Strides3 gs, float* out, Strides3 os, int B, int H, int KV, int T, int pos, int cap,
                        float scale, hipStream_t st, void* ws = nullptr, size_t ws_bytes = 0,
                        uint16_t* out_bf16 = nullptr, bool* wrote_bf16 = nullptr) {
    // out_bf16: the 32-query kernels may write the output as bf16 there instead (same strides);
    // *wrote_bf16 says whether they did (the other kernels write fp32 to out)
    if (wrote_bf16) *wrote_bf16 = false;
    if (KV <= 0 || H % KV) return fail(AEGIST_ERR_SHAPE, "attention prefill: need H % KV == 0");
    if (pos < 0 || pos + T > cap) return fail(AEGIST_ERR_SHAPE, "attention prefill: rows exceed the cache capacity");
    // the MFMA kernel reads q and gate and writes out as 16-byte rows
    auto rows16 = [](const void* p, const Strides3& s) {
        return (uintptr_t)p % 16 == 0 && s.b % 4 == 0 && s.t % 4 == 0 && s.h % 4 == 0;
    };
    const bool vec = rows16(q, qs) && rows16(out, os) && (!gate || rows16(gate, gs));
    // the 32-query kernel addresses the cache rows of a (sequence, KV head) through a buffer
    // range in bytes (32-bit)
    const bool w32 = PREFILL_W32 && (long long)(pos + T) * HD * 2 <= 0x7fffffffLL;
    const int rows = pos + T, rows_pad = (rows + PK - 1) / PK * PK;
    if (T >= 16 && vec && w32 && ws && ws_bytes >= prefill_f16_bytes(B, KV, rows) && PREFILL_F16 &&
        (long long)rows_pad * HD * 2 <= 0x7fffffffLL && (uintptr_t)ws % 256 == 0) {
        uint16_t* kf = (uint16_t*)ws;
        uint16_t* vf = kf + (size_t)B * KV * rows_pad * HD;
        const long long nchunks = (long long)B * KV * rows_pad * HD / 8;
        const int cblocks = (int)std::min<long long>((nchunks + 255) / 256, 4096);
        attn_kv_f16_kernel<<<cblocks, 256, 0, st>>>(kc, vc, kf, vf, KV, cap, rows, rows_pad, nchunks);
        int rc = after_launch("attention_prefill_f16_copy");
        if (rc) return rc;
        const int nblk = (T + PQ2 - 1) / PQ2 * H * B;
        const int grid = std::min(nblk, device_cus());  // one workgroup per CU (128 KB of LDS each)
        if (out_bf16) {
            attn_prefill_w32f_kernel<uint16_t><<<grid, 64 * PW2, 0, st>>>(q, qs, kf, vf, rows_pad, gate, gs, out_bf16,
                                                                         os, H, KV, T, pos, scale, B);
            if (wrote_bf16) *wrote_bf16 = true;
        } else {
            attn_prefill_w32f_kernel<float><<<grid, 64 * PW2, 0, st>>>(q, qs, kf, vf, rows_pad, gate, gs, out, os, H,
                                                                      KV, T, pos, scale, B);
        }
    } else if (T >= 16 && vec && w32) {
        const int nblk = (T + PQ2 - 1) / PQ2 * H * B, per_xcd = (nblk + 7) / 8;
        if (out_bf16) {
            attn_prefill_w32_kernel<uint16_t><<<8 * per_xcd, 64 * PW2, 0, st>>>(q, qs, kc, vc, gate, gs, out_bf16, os, H,
                                                                               KV, T, pos, cap, scale, B, per_xcd);
            if (wrote_bf16) *wrote_bf16 = true;
        } else {
            attn_prefill_w32_kernel<float><<<8 * per_xcd, 64 * PW2, 0, st>>>(q, qs, kc, vc, gate, gs, out, os, H, KV, T,
                                                                            pos, cap, scale, B, per_xcd);
        }
    } else if (T >= 16 && vec) {
        const int nblk = (T + PQ - 1) / PQ * H * B, per_xcd = (nblk + 7) / 8;
        attn_prefill_mfma_kernel<<<8 * per_xcd, 64 * PW, 0, st>>>(q, qs, kc, vc, gate, gs, out, os, H, KV, T, pos, cap,
                                                                  scale, B, per_xcd);
    } else {
        attn_prefill_simple_kernel<<<dim3((T + 3) / 4, H, B), 256, 0, st>>>(q, qs, kc, vc, gate, gs, out, os, H, KV, T,
                                                                            pos, cap, scale);
    }
    return after_launch("attention_prefill");
}

// Wrappers for the layer stack: qn [B, T, H, HD], gate inside qg [B, T, H, 2 HD] (+HD),
// out [B, T, H, HD] fp32.
int stack_attn_decode(const float* qn, const uint16_t* kc, const uint16_t* vc, const float* qg, uint16_t* out, int B,
                      int H, int KV, int L, int cap, float scale, void* ws, size_t ws_bytes, hipStream_t st) {
    return launch_decode_core<float, uint16_t>(qn, kc, vc, qg + HD, 2 * HD, out, HD, B, H, KV, L, cap, scale, ws,
                                               ws_bytes, st);
}
// The stack's decode with the prep folded into the split launch (fp32 projections: qg [B, H, 2 HD],
// k / v [B, KV, HD]; rotary dim 64): appends row pos and writes the gated output as bf16.
int stack_attn_decode_fused(const float* qg, const float* kn, const float* vn, const uint16_t* qw, const uint16_t* kw,
                            uint16_t* kc, uint16_t* vc, uint16_t* out, int B, int H, int KV, int pos, int cap, float eps,
                            float theta, void* ws, size_t ws_bytes, hipStream_t st) {
    FusedPrep fp{qg, kn, vn, qw, kw, kc, vc, pos, eps, {}};
    int rc = aegist_rope_inv_freq(fp.inv, kFusedRD, theta);
    if (rc) return rc;
    return launch_decode_core<float, uint16_t>(nullptr, kc, vc, qg + HD, 2 * HD, out, HD, B, H, KV, pos + 1, cap,
                                               1.0f / sqrtf((float)HD), ws, ws_bytes, st, {}, &fp, AEGIST_F32);
}
int stack_attn_prefill(const float* qn, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out, int B,
                       int H, int KV, int T, int pos, int cap, float scale, void* ws, size_t ws_bytes, hipStream_t st,
                       uint16_t* out_bf16, bool* wrote_bf16) {
    Strides3 qs{(long long)T * H * HD, (long long)H * HD, HD};
    Strides3 gs{(long long)T * H * 2 * HD, (long long)H * 2 * HD, 2 * HD};
    return launch_prefill_core(qn, qs, kc, vc, qg + HD, gs, out, qs, B, H, KV, T, pos, cap, scale, st, ws, ws_bytes,
                               out_bf16, wrote_bf16);
}

}  // namespace aegist

extern "C" {

size_t aegist_attention_decode_workspace_bytes(int B, int H, int KV, int L) {
    return decode_workspace_bytes(B, H, KV, L, true);
}

int aegist_attention_decode(const void* qg, const void* k_new, const void* v_new, int in_dtype,
                            const uint16_t* q_norm_w, const uint16_t* k_norm_w, uint16_t* kc, uint16_t* vc, void* out,
                            int out_dtype, int B, int H, int KV, int HDv, int RD, int pos, int cap, float eps,
                            float theta, void* workspace, size_t workspace_bytes, void* stream) {
    AEG_REQUIRE(HDv == HD, "attention_decode: head_dim must be 256");
    AEG_REQUIRE(B >= 0 && H > 0 && KV > 0 && H % KV == 0 && H / KV <= 8, "attention_decode: need H % KV == 0, H/KV <= 8");
    AEG_REQUIRE(pos >= 0 && pos < cap, "attention_decode: need 0 <= pos < cap");
    if (B == 0) return 0;
    size_t need = decode_workspace_bytes(B, H, KV, pos + 1, true);
    if (!workspace || workspace_bytes < need)
        return fail(AEGIST_ERR_WORKSPACE, "attention_decode: workspace smaller than aegist_attention_decode_workspace_bytes()");
    hipStream_t st = AEG_STREAM(stream);
    size_t core = decode_workspace_bytes(B, H, KV, pos + 1, false);
    float* qn = (float*)((char*)workspace + core);
    // rotary dim 64 (the model's): the prep runs inside the split launch; otherwise its own launch
    FusedPrep fpp{qg, k_new, v_new, q_norm_w, k_norm_w, kc, vc, pos, eps, {}};
    const bool fuse = RD == kFusedRD && (in_dtype == AEGIST_BF16 || in_dtype == AEGIST_F32) &&
                      (uintptr_t)qg % 16 == 0 && (uintptr_t)k_new % 16 == 0 && (uintptr_t)v_new % 16 == 0 &&
                      (uintptr_t)q_norm_w % 16 == 0 && (uintptr_t)k_norm_w % 8 == 0 && (uintptr_t)kc % 8 == 0 &&
                      (uintptr_t)vc % 8 == 0;
    const FusedPrep* fused = nullptr;
    if (fuse) {
        int rc = aegist_rope_inv_freq(fpp.inv, RD, theta);
        if (rc) return rc;
        fused = &fpp;
    } else {
        int rc = launch_attn_prep(qg, k_new, v_new, in_dtype, q_norm_w, k_norm_w, qn, kc, vc, B, 1, H, KV, HD, RD, pos,
                                  cap, eps, theta, st);
        if (rc) return rc;
    }
    const float scale = 1.0f / sqrtf((float)HD);
    // gate = second half of each head's 2*HD row of qg
    if (in_dtype == AEGIST_F32) {
        const float* gate = (const float*)qg + HD;
        if (out_dtype == AEGIST_F32)
            return launch_decode_core<float, float>(qn, kc, vc, gate, 2 * HD, (float*)out, HD, B, H, KV, pos + 1, cap,
                                                    scale, workspace, core, st, {}, fused, in_dtype);
        if (out_dtype == AEGIST_BF16)
            return launch_decode_core<float, uint16_t>(qn, kc, vc, gate, 2 * HD, (uint16_t*)out, HD, B, H, KV, pos + 1,
                                                       cap, scale, workspace, core, st, {}, fused, in_dtype);
    } else if (in_dtype == AEGIST_BF16) {
        const uint16_t* gate = (const uint16_t*)qg + HD;
        if (out_dtype == AEGIST_F32)
            return launch_decode_core<uint16_t, float>(qn, kc, vc, gate, 2 * HD, (float*)out, HD, B, H, KV, pos + 1,
                                                       cap, scale, workspace, core, st, {}, fused, in_dtype);
        if (out_dtype == AEGIST_BF16)
            return launch_decode_core<uint16_t, uint16_t>(qn, kc, vc, gate, 2 * HD, (uint16_t*)out, HD, B, H, KV,
                                                          pos + 1, cap, scale, workspace, core, st, {}, fused, in_dtype);
    }
    return fail(AEGIST_ERR_DTYPE, "attention_decode: dtypes must be AEGIST_F32 or AEGIST_BF16");
}

// ---------------------------------------------------------------------------------------------
// attention_decode without a workspace argument and without allocating: its split-K partials,
// statistics and normed queries live in a file-scope device array (one copy per
// GPU, held until the process ends). Host code never passes the array's name to a kernel: the
// array's device address is looked up once per device with hipGetSymbolAddress and kept.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64] = {};  // per device, filled on the first call on that device

static int scratch_address(void** out) {
    int dev = 0;
    AEG_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return fail(AEGIST_ERR_SHAPE, "attention_decode_noalloc: device index beyond 63");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        AEG_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

int aegist_attention_decode_noalloc(const void* qg, const void* k_new, const void* v_new, int in_dtype,
                                    const uint16_t* q_norm_w, const uint16_t* k_norm_w, uint16_t* kc, uint16_t* vc,
                                    void* out, int out_dtype, int B, int H, int KV, int HDv, int RD, int pos, int cap,
                                    float eps, float theta, void* stream) {
    AEG_REQUIRE(B >= 0 && H > 0 && KV > 0 && H % KV == 0 && H / KV <= 8 && pos >= 0,
                "attention_decode_noalloc: need H % KV == 0, H/KV <= 8, pos >= 0");
    if (B == 0) return 0;
    const size_t need = decode_workspace_bytes(B, H, KV, pos + 1, true);
    if (need > kNoAllocScratchBytes)
        return fail(AEGIST_ERR_WORKSPACE, "attention_decode_noalloc: needs " + std::to_string(need) +
                                              " bytes of scratch, more than its fixed " +
                                              std::to_string(kNoAllocScratchBytes) +
                                              "; use aegist_attention_decode with a workspace");
    void* ws = nullptr;
    int rc = scratch_address(&ws);
    if (rc) return rc;
    // every byte of the scratch a call reads was written earlier in the same call, so it needs
    // no clearing between calls
    return aegist_attention_decode(qg, k_new, v_new, in_dtype, q_norm_w, k_norm_w, kc, vc, out, out_dtype, B, H, KV,
                                   HDv, RD, pos, cap, eps, theta, ws, kNoAllocScratchBytes, stream);
}

int aegist_attention_core(const float* q, const uint16_t* kc, const uint16_t* vc, const float* gate, float* out, int B,
                          int H, int KV, int T, int pos, int cap, float scale, void* workspace, size_t workspace_bytes,
                          void* stream) {
    AEG_REQUIRE(B >= 0 && T >= 0 && H > 0 && KV > 0 && H % KV == 0, "attention_core: need H % KV == 0");
    if (B == 0 || T == 0) return 0;
    hipStream_t st = AEG_STREAM(stream);
    if (T == 1) {
        // q [B, H, 1, HD] == [B, H, HD]; gate [B, 1, H*HD]; out [B, 1, H, HD]
        return launch_decode_core<float, float>(q, kc, vc, gate, HD, out, HD, B, H, KV, pos + 1, cap, scale, workspace,
                                                workspace_bytes, st);
    }
    // q [B, H, T, HD]; gate [B, T, H*HD]; out [B, T, H, HD]
    Strides3 qs{(long long)H * T * HD, HD, (long long)T * HD};
    Strides3 gs{(long long)T * H * HD, (long long)H * HD, HD};
    Strides3 os = gs;
    return launch_prefill_core(q, qs, kc, vc, gate, gs, out, os, B, H, KV, T, pos, cap, scale, st, workspace,
                               workspace_bytes);
}

size_t aegist_attention_core_workspace_bytes(int B, int H, int KV, int T, int pos) {
    if (B <= 0 || T <= 0 || H <= 0 || KV <= 0) return 0;
    if (T == 1) return aegist::decode_workspace_bytes(B, H, KV, pos + 1, false);
    return aegist::prefill_f16_bytes(B, KV, pos + T);
}

size_t aegist_attention_gated_workspace_bytes(int T, int H, int KV, int pos0) {
    if (T != 1 || H <= 0 || KV <= 0 || pos0 < 0) return 0;  // only the T == 1 split-K path uses scratch
    return decode_workspace_bytes(1, H, KV, pos0 + 1, false);
}

// Engine mirror: q = qn [T, H, HD] fp32 (from attn_prep), gate inside qg [T, H, 2*HD],
// out [T, H, HD]; batch 1, caches [KV, cap, HD]. `ws` holds the split-K partials of T == 1.
int aegist_attention_gated_ws(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out,
                              int T, int H, int KV, int pos0, int cap, float scale, void* ws, size_t ws_bytes,
                              void* stream) {
    AEG_REQUIRE(T >= 0 && H > 0 && KV > 0 && H % KV == 0, "attention_gated: need H % KV == 0");
    if (T == 0) return 0;
    hipStream_t st = AEG_STREAM(stream);
    if (T == 1) {
        AEG_REQUIRE(H / KV <= 8, "attention_gated: H/KV must be <= 8");
        const size_t need = decode_workspace_bytes(1, H, KV, pos0 + 1, false);
        int rc = check_workspace(ws, ws_bytes, need, "attention_gated");
        if (rc) return rc;
        return launch_decode_core<float, float>(q, kc, vc, qg + HD, 2 * HD, out, HD, 1, H, KV, pos0 + 1, cap, scale, ws,
                                                ws_bytes, st);
    }
    // engine layouts: q, out [T, H, HD]; gate rows inside qg [T, H, 2*HD]
    Strides3 qs{0, (long long)H * HD, HD};
    Strides3 gs{0, (long long)H * 2 * HD, 2 * HD};
    return launch_prefill_core(q, qs, kc, vc, qg + HD, gs, out, qs, 1, H, KV, T, pos0, cap, scale, st);
}

// The reference signature (no workspace argument): T == 1 takes the workspace bound to this
// thread (aegist_bind_workspace).
int aegist_attention_gated(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out, int T,
                           int H, int KV, int pos0, int cap, float scale, void* stream) {
    size_t bound = 0;
    void* ws = bound_workspace(&bound);
    return aegist_attention_gated_ws(q, kc, vc, qg, out, T, H, KV, pos0, cap, scale, ws, bound, stream);
}

static int list_lmax(int T, int pos0, int top, int R) {
    // longest key list: top blocks plus the keys of an incomplete block, and never more than the
    // last query's position + 1
    return std::min(top * R + R - 1, pos0 + T);
}

size_t aegist_attention_gated_list_workspace_bytes(int T, int H, int KV, int pos0, int top, int R) {
    if (T <= 0 || H <= 0 || KV <= 0 || top <= 0 || R <= 0 || pos0 < 0) return 0;
    return decode_workspace_bytes(T, H, KV, list_lmax(T, pos0, top, R), false);
}

// attention_gated over listed blocks (next.cu:648-705): the split-K decode kernel with one query
// token per "sequence" and its keys taken from the block list. Engine layouts as attention_gated.
int aegist_attention_gated_list_ws(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg,
                                   float* out, int T, int H, int KV, int pos0, int cap, float scale, const int* blist,
                                   const int* nsel, int top, int R, void* ws, size_t ws_bytes, void* stream) {
    AEG_REQUIRE(T >= 0 && H > 0 && KV > 0 && H % KV == 0 && H / KV <= 8,
                "attention_gated_list: need H % KV == 0 and H/KV <= 8");
    AEG_REQUIRE(top > 0 && R > 0 && pos0 >= 0 && pos0 + T <= cap, "attention_gated_list: bad list or positions");
    if (T == 0) return 0;
    const int Lmax = list_lmax(T, pos0, top, R);
    int rc = check_workspace(ws, ws_bytes, decode_workspace_bytes(T, H, KV, Lmax, false), "attention_gated_list");
    if (rc) return rc;
    return launch_decode_core<float, float>(q, kc, vc, qg + HD, 2 * HD, out, HD, T, H, KV, Lmax, cap, scale, ws,
                                            ws_bytes, AEG_STREAM(stream), KeyList{blist, nsel, top, R, pos0});
}

int aegist_attention_gated_list(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out,
                                int T, int H, int KV, int pos0, int cap, float scale, const int* blist,
                                const int* nsel, int top, int R, void* stream) {
    size_t bound = 0;
    void* ws = bound_workspace(&bound);
    return aegist_attention_gated_list_ws(q, kc, vc, qg, out, T, H, KV, pos0, cap, scale, blist, nsel, top, R, ws,
                                          bound, stream);
}

}  // extern "C"

