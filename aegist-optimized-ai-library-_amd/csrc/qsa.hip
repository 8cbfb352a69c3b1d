// QSA sparse-attention indexer of the second language core (QSAIndexer, aegist/hc.py:237-283;
// engine kernels idx_prep / idx_blocks / idx_scores / idx_select, aegist_rs/kernels/next.cu:
// 488-645, launched by NextEngine::mixer, aegist_rs/src/next.rs:1866-1910), and the gated norm
// with a choice of gate (gated_norm2, next.cu:129-142).
//
// Beyond idx_budget tokens of context, each query attends to its top = budget / R highest-scoring
// complete blocks of R keys plus its own incomplete block:
//   qi[t, h] = rope(znorm_qw(q_idx[t, h]), pos0 + t)              (index queries)
//   bk[b]    = rope(znorm_kw(mean_{j < R} kraw[b R + j]), b R)     (block keys)
//   sc[t, b] = sum_h relu(qi[t, h] . bk[b]) / sqrt(HD)            for b < (pos0 + t + 1) / R
//   blist[t] = the top blocks by score (ties to the lower block), listed in block order
// The attention over the listed blocks is attention_gated_list (attention.hip).
//
// Scores use fp32 MFMA (v_mfma_f32_16x16x4f32) so the selection sees fp32 products like the
// engine's; the selection builds the top-th largest score bit by bit from register-resident
// scores (counting with ballots), then compacts in block order with wave ballots.
#include "common.h"

using namespace aegist;

namespace {

constexpr int IHD = 128;  // indexer head dim (the engine requires 128, next.rs:156)

struct IdxRope {
    float inv[IHD / 2];
};

// One wave holds a 128-vector as x[0] = element lane, x[1] = element lane + 64. Zero-centred
// RMSNorm with weight (1 + w), then rotate-half RoPE on the first RD elements at `pos`.
__device__ __forceinline__ void norm_rope(float x[2], const uint16_t* __restrict__ w, float eps, int RD, int pos,
                                          const IdxRope& rope, float* buf, int lane) {
    float ss = wave_sum(x[0] * x[0] + x[1] * x[1]);
    const float r = rsqrtf(ss / (float)IHD + eps);
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int i = lane + 64 * e;
        x[e] = (1.f + bf2f(w[i])) * (x[e] * r);
        buf[i] = x[e];
    }
    wave_sync();
    const int half = RD / 2;
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int i = lane + 64 * e;
        if (i < RD) {
            const int j = i < half ? i : i - half;
            float s, c;
            sincosf((float)pos * rope.inv[j], &s, &c);
            const float rot = i < half ? -buf[i + half] : buf[i - half];
            x[e] = x[e] * c + rot * s;
        }
    }
}

// grid: ceil(T (H + 1) / 4) workgroups of 4 waves; wave = (t, head), head H is the key.
__global__ void __launch_bounds__(256) idx_prep_kernel(const float* __restrict__ qk, const uint16_t* __restrict__ qw,
                                                       float* __restrict__ qi, float* __restrict__ kraw, int T, int H,
                                                       int RD, int pos0, float eps, IdxRope rope) {
    __shared__ float buf[4][IHD];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int item = blockIdx.x * 4 + wave;
    if (item >= T * (H + 1)) return;
    const int t = item / (H + 1), h = item % (H + 1);
    const float* src = qk + ((size_t)t * (H + 1) + h) * IHD;
    float x[2] = {src[lane], src[lane + 64]};
    if (h == H) {  // the raw index key, kept for the block means
        float* dst = kraw + (size_t)(pos0 + t) * IHD;
        dst[lane] = x[0];
        dst[lane + 64] = x[1];
        return;
    }
    norm_rope(x, qw, eps, RD, pos0 + t, rope, buf[wave], lane);
    float* dst = qi + ((size_t)t * H + h) * IHD;
    dst[lane] = x[0];
    dst[lane + 64] = x[1];
}

// grid: ceil(n / 4) workgroups; wave = block b0 + i.
__global__ void __launch_bounds__(256) idx_blocks_kernel(const float* __restrict__ kraw, const uint16_t* __restrict__ kw,
                                                         float* __restrict__ bk, int b0, int n, int R, int RD,
                                                         float eps, IdxRope rope) {
    __shared__ float buf[4][IHD];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int i = blockIdx.x * 4 + wave;
    if (i >= n) return;
    const int b = b0 + i;
    float x[2] = {0.f, 0.f};
    for (int j = 0; j < R; j++) {
        const float* row = kraw + ((size_t)b * R + j) * IHD;
        x[0] += row[lane];
        x[1] += row[lane + 64];
    }
    x[0] /= (float)R;
    x[1] /= (float)R;
    norm_rope(x, kw, eps, RD, b * R, rope, buf[wave], lane);
    float* dst = bk + (size_t)b * IHD;
    dst[lane] = x[0];
    dst[lane + 64] = x[1];
}

// grid: (ceil(nb / 16), ceil(T / 4)); wave w scores query t = 4 by + w against blocks
// [16 bx, 16 bx + 16). Per head tile of 16, C[head][block] = q_t . bk^T on fp32 MFMA with the
// contraction index permuted so each lane streams 32 contiguous floats of its row: step s uses
// k = 32 (lane / 16) + s for both operands. relu per head, then the column sum over heads.
__global__ void __launch_bounds__(256) idx_scores_kernel(const float* __restrict__ qi, const float* __restrict__ bk,
                                                         float* __restrict__ sc, int T, int H, int pos0, int R,
                                                         int nbmax) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, n = lane % 16, g = lane / 16;
    const int t = blockIdx.y * 4 + wave, bb0 = blockIdx.x * 16;
    if (t >= T) return;
    const int nvis = (pos0 + t + 1) / R;
    if (bb0 >= nvis) return;
    const int blk = bb0 + n;
    float brow[32];
    {
        const float4* p = (const float4*)(bk + (size_t)min(blk, nvis - 1) * IHD + 32 * g);
#pragma unroll
        for (int v = 0; v < 8; v++) {
            const float4 f = p[v];
            brow[4 * v] = f.x;
            brow[4 * v + 1] = f.y;
            brow[4 * v + 2] = f.z;
            brow[4 * v + 3] = f.w;
        }
    }
    float tot = 0.f;
    for (int h0 = 0; h0 < H; h0 += 16) {
        const int h = h0 + n;
        float qrow[32];
        const float4* p = (const float4*)(qi + ((size_t)t * H + min(h, H - 1)) * IHD + 32 * g);
#pragma unroll
        for (int v = 0; v < 8; v++) {
            const float4 f = p[v];
            const float m = h < H ? 1.f : 0.f;
            qrow[4 * v] = f.x * m;
            qrow[4 * v + 1] = f.y * m;
            qrow[4 * v + 2] = f.z * m;
            qrow[4 * v + 3] = f.w * m;
        }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 32; s++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qrow[s], brow[s], acc, 0, 0, 0);
        // lane holds heads h0 + 4g + j (rows) for block bb0 + n (column); padded heads are 0
#pragma unroll
        for (int j = 0; j < 4; j++) tot += acc[j] > 0.f ? acc[j] : 0.f;
    }
    tot += __shfl_xor(tot, 16, WAVE);
    tot += __shfl_xor(tot, 32, WAVE);
    if (g == 0 && blk < nvis) sc[(size_t)t * nbmax + blk] = tot / sqrtf((float)IHD);
}

// One workgroup of 16 waves per query; thread tid holds the PER consecutive scores of blocks
// [tid PER, tid PER + PER) in registers. The top-th largest score bit pattern T is built from
// the most significant bit down, two bits per step: of the three candidates T | k << b (k = 1..3)
// the largest with at least `top` scores >= it is kept (scores are non-negative, so bit patterns
// order like values). A count is a compare-and-add over the thread's registers, wave totals from
// ballots of the count's bits, and one barrier for the three sums over waves. The listing is an
// exclusive prefix over threads of (above T, equal to T) counts, so each thread writes its own
// blocks in order: every block above T and the lowest-numbered blocks equal to T.
// PER = 0 (more than 32768 blocks): the thread's scores are re-read from global memory
// (L2-resident), chunk by chunk, instead of registers.
constexpr int SEL_THREADS = 1024, SEL_WAVES = SEL_THREADS / WAVE;

template <int PER>
__global__ void __launch_bounds__(SEL_THREADS) idx_select_kernel(const float* __restrict__ sc, int* __restrict__ blist,
                                                                 int* __restrict__ nsel, int top, int R, int pos0,
                                                                 int nbmax, int vec) {
    __shared__ unsigned wc[2][4][SEL_WAVES];
    const int t = blockIdx.x, tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int n = (pos0 + t + 1) / R;
    const unsigned* sg = (const unsigned*)(sc + (size_t)t * nbmax);
    int* out = blist + (size_t)t * top;
    if (n <= top) {  // every complete block
        for (int b = tid; b < n; b += SEL_THREADS) out[b] = b;
        if (tid == 0) nsel[t] = n;
        return;
    }
    // this thread's blocks: [lo, lo + per), per = PER or ceil(n / 1024)
    const int per = PER > 0 ? PER : (n + SEL_THREADS - 1) / SEL_THREADS;
    const int lo = tid * per;
    constexpr int NREG = PER > 0 ? PER : 1;
    unsigned u[NREG];
    if constexpr (PER > 0) {
#pragma unroll
        for (int i = 0; i < PER; i += 4) {
            if (vec && lo + i + 3 < n) {
                const uint4 v = *(const uint4*)(sg + lo + i);  // 16-byte aligned rows
                u[i] = v.x;
                u[i + 1] = v.y;
                u[i + 2] = v.z;
                u[i + 3] = v.w;
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) u[i + k] = lo + i + k < n ? sg[lo + i + k] : 0u;  // 0 never counts
            }
        }
    }
    auto val = [&](int i) -> unsigned {
        if constexpr (PER > 0) return u[i];
        return lo + i < n ? sg[lo + i] : 0u;
    };
    const unsigned long long below = (1ull << lane) - 1;
    const int cbits = 32 - __builtin_clz((unsigned)per);  // per-thread counts are <= per
    // wave total (and exclusive prefix below this lane) of a per-thread count, from ballots
    auto wave_count = [&](unsigned c, unsigned& pre) {
        unsigned tot = 0;
        pre = 0;
        for (int bit = 0; bit < cbits; bit++) {
            const unsigned long long m = __ballot((c >> bit) & 1u);
            tot += (unsigned)__popcll(m) << bit;
            pre += (unsigned)__popcll(m & below) << bit;
        }
        return tot;
    };
    int par = 0;
    unsigned T = 0;
    for (int bit = 29; bit >= -1; bit -= 2) {  // bits (30, 29), ..., (0, -); the sign bit is 0
        const int sh = bit < 0 ? 0 : bit;
        const int nk = bit < 0 ? 1 : 3;  // the last step decides bit 0 alone
        unsigned c[3] = {0u, 0u, 0u};
        for (int i = 0; i < per; i++) {
            const unsigned v = val(i);
#pragma unroll
            for (int k = 0; k < 3; k++) c[k] += v >= (T | ((unsigned)(k + 1) << sh));
        }
#pragma unroll
        for (int k = 0; k < 3; k++) {
            unsigned pre;
            const unsigned wt = wave_count(c[k], pre);
            if (lane == 0) wc[par][k][wave] = wt;
        }
        __syncthreads();
        unsigned tot[3] = {0u, 0u, 0u};
        for (int w = 0; w < SEL_WAVES; w++)
#pragma unroll
            for (int k = 0; k < 3; k++) tot[k] += wc[par][k][w];
        par ^= 1;  // the next step writes the other buffer: no second barrier needed
        for (int k = nk - 1; k >= 0; k--)
            if (tot[k] >= (unsigned)top) {
                T |= (unsigned)(k + 1) << sh;
                break;
            }
    }
    // listing: per-thread counts above / equal to T, exclusive prefix over threads
    unsigned gtc = 0, eqc = 0;
    for (int i = 0; i < per; i++) {
        const unsigned v = val(i);
        gtc += lo + i < n && v > T;
        eqc += lo + i < n && v == T;
    }
    unsigned gpre, epre;
    const unsigned gw = wave_count(gtc, gpre), ew = wave_count(eqc, epre);
    if (lane == 0) {
        wc[par][0][wave] = gw;
        wc[par][1][wave] = ew;
    }
    __syncthreads();
    unsigned gt_before = gpre, eq_before = epre, gt_total = 0;
    for (int w = 0; w < SEL_WAVES; w++) {
        const unsigned g = wc[par][0][w], e = wc[par][1][w];
        gt_total += g;
        if (w < wave) {
            gt_before += g;
            eq_before += e;
        }
    }
    const unsigned take_eq = (unsigned)top - gt_total;  // equal-valued blocks that make the top
    // this thread's output position: blocks above T before it plus the equal ones taken before it
    unsigned pos = gt_before + min(eq_before, take_eq), eq_seen = eq_before;
    for (int i = 0; i < per; i++) {
        if (lo + i >= n) break;
        const unsigned v = val(i);
        if (v > T) {
            out[pos++] = lo + i;
        } else if (v == T) {
            if (eq_seen < take_eq) out[pos++] = lo + i;
            eq_seen++;
        }
    }
    if (tid == 0) nsel[t] = top;
}

// out = w * rmsnorm(o) * act(z) per value head, act = sigmoid (sig != 0) or SiLU; one wave per
// (row, head).
__global__ void __launch_bounds__(256) gated_norm2_kernel(const float* __restrict__ o, const float* __restrict__ z,
                                                          const uint16_t* __restrict__ w, float* __restrict__ out,
                                                          int rows, int DV, float eps, int sig) {
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
        const float act = sig ? 1.f / (1.f + expf(-zz)) : zz / (1.f + expf(-zz));
        out[base + i] = bf2f(w[i]) * (o[base + i] * r) * act;
    }
}

int idx_rope(IdxRope* r, int RD, float theta) {
    if (RD <= 0 || (RD & 1) || RD > IHD) return fail(AEGIST_ERR_SHAPE, "indexer: rotary dim must be even and <= 128");
    return aegist_rope_inv_freq(r->inv, RD, theta);
}

}  // namespace

extern "C" {

int aegist_idx_prep(const float* qk, const uint16_t* qw, float* qi, float* kraw, int T, int H, int HD, int RD,
                    int pos0, float eps, float theta, void* stream) {
    AEG_REQUIRE(HD == IHD, "idx_prep: indexer head dim must be 128");
    AEG_REQUIRE(T >= 0 && H > 0 && pos0 >= 0, "idx_prep: bad shape");
    IdxRope rope;
    int rc = idx_rope(&rope, RD, theta);
    if (rc) return rc;
    const int items = T * (H + 1);
    if (items == 0) return 0;
    idx_prep_kernel<<<(items + 3) / 4, 256, 0, AEG_STREAM(stream)>>>(qk, qw, qi, kraw, T, H, RD, pos0, eps, rope);
    return after_launch("idx_prep");
}

int aegist_idx_blocks(const float* kraw, const uint16_t* kw, float* bk, int b0, int n, int R, int HD, int RD,
                      float eps, float theta, void* stream) {
    AEG_REQUIRE(HD == IHD, "idx_blocks: indexer head dim must be 128");
    AEG_REQUIRE(b0 >= 0 && n >= 0 && R > 0, "idx_blocks: bad shape");
    IdxRope rope;
    int rc = idx_rope(&rope, RD, theta);
    if (rc) return rc;
    if (n == 0) return 0;
    idx_blocks_kernel<<<(n + 3) / 4, 256, 0, AEG_STREAM(stream)>>>(kraw, kw, bk, b0, n, R, RD, eps, rope);
    return after_launch("idx_blocks");
}

int aegist_idx_scores(const float* qi, const float* bk, float* sc, int T, int H, int HD, int pos0, int R, int nbmax,
                      void* stream) {
    AEG_REQUIRE(HD == IHD, "idx_scores: indexer head dim must be 128");
    AEG_REQUIRE(T >= 0 && H > 0 && pos0 >= 0 && R > 0, "idx_scores: bad shape");
    AEG_REQUIRE((pos0 + T) / R <= nbmax, "idx_scores: nbmax smaller than the number of complete blocks");
    AEG_REQUIRE((uintptr_t)qi % 16 == 0 && (uintptr_t)bk % 16 == 0, "idx_scores: qi and bk must be 16-byte aligned");
    const int nb = (pos0 + T) / R;
    if (T == 0 || nb == 0) return 0;
    idx_scores_kernel<<<dim3((nb + 15) / 16, (T + 3) / 4), 256, 0, AEG_STREAM(stream)>>>(qi, bk, sc, T, H, pos0, R,
                                                                                       nbmax);
    return after_launch("idx_scores");
}

int aegist_idx_select(const float* sc, int* blist, int* nsel, int T, int top, int R, int pos0, int nbmax,
                      void* stream) {
    AEG_REQUIRE(T >= 0 && top > 0 && R > 0 && pos0 >= 0, "idx_select: bad shape");
    AEG_REQUIRE((pos0 + T) / R <= nbmax, "idx_select: nbmax smaller than the number of complete blocks");
    if (T == 0) return 0;
    const int nmax = (pos0 + T) / R;  // the most complete blocks any of these queries sees
    const int vec = nbmax % 4 == 0 && (uintptr_t)sc % 16 == 0;
    hipStream_t st = AEG_STREAM(stream);
    if (nmax <= 8 * SEL_THREADS)
        idx_select_kernel<8><<<T, SEL_THREADS, 0, st>>>(sc, blist, nsel, top, R, pos0, nbmax, vec);
    else if (nmax <= 32 * SEL_THREADS)
        idx_select_kernel<32><<<T, SEL_THREADS, 0, st>>>(sc, blist, nsel, top, R, pos0, nbmax, vec);
    else
        idx_select_kernel<0><<<T, SEL_THREADS, 0, st>>>(sc, blist, nsel, top, R, pos0, nbmax, vec);
    return after_launch("idx_select");
}

int aegist_gated_norm2(const float* o, const float* z, const uint16_t* w, float* out, int T, int HV, int DV, float eps,
                       int sig, void* stream) {
    AEG_REQUIRE(T >= 0 && HV > 0 && DV > 0, "gated_norm2: bad shape");
    const int rows = T * HV;
    if (rows == 0) return 0;
    gated_norm2_kernel<<<(rows + 3) / 4, 256, 0, AEG_STREAM(stream)>>>(o, z, w, out, rows, DV, eps, sig);
    return after_launch("gated_norm2");
}

}  // extern "C"
