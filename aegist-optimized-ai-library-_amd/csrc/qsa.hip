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
// engine's; the selection finds the top-th largest score by a three-digit radix select over
// register-resident scores (LDS histograms), then compacts in block order with wave ballots.
// Few queries over many blocks split each row over several workgroups first (local tops),
// then select among the candidates.
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

// Top-`top` of n values by (value desc, index asc), listed in index order. Values are
// non-negative floats or encoded bit patterns below 2^31, so bit patterns order like values.
// Thread tid holds the PER consecutive values [tid PER, tid PER + PER) in registers. The top-th
// largest bit pattern T is found by a most-significant-digit radix select over digits of bits
// 30..20, 19..10 and 9..0: each pass counts the values whose higher digits equal the ones decided
// so far into an LDS histogram (LDS atomics), and a suffix sum over the bins (wave scans plus
// one sum over waves) names the bin holding the still-wanted rank. The listing is an exclusive
// prefix over threads of (above T, equal to T) counts, so each thread emits its own values in
// order: every value above T and the lowest-indexed values equal to T. Requires n > top.
// emit(pos, i, v) receives the output position, the value's index and its bit pattern.
// PER = 0 (more than NT * 32 values): the thread's values are re-read from global memory
// (L2-resident), chunk by chunk, instead of registers.
// digit widths (a wider first digit spreads the atomics of clustered scores over more bins but
// lengthens the bin scans: 11 measured best of 11 / 12 / 13 at 32768 blocks)
constexpr int SEL_D1 = 11, SEL_D2 = 10, SEL_D3 = 31 - SEL_D1 - SEL_D2;
struct SelectLds {
    unsigned hist[1 << SEL_D1];
    unsigned wsum[16];   // per-wave bin totals (at most 16 waves)
    unsigned pick[2];    // the chosen digit and the count of values in higher bins
    unsigned wl[2][16];  // per-wave listing counts
};

template <int NT, int PER, typename Emit>
__device__ __forceinline__ void select_top(const unsigned* __restrict__ sg, int n, int top, int vec, SelectLds& L,
                                           Emit emit) {
    constexpr int NW = NT / WAVE;
    static_assert(NW <= 16 && SEL_D3 > 0, "select_top: at most 16 waves; three digits");
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int per = PER > 0 ? PER : (n + NT - 1) / NT;
    const int lo = tid * per;
    constexpr int NREG = PER > 0 ? PER : 1;
    unsigned u[NREG];
    for (int b = tid; b < (1 << SEL_D1); b += NT) L.hist[b] = 0u;
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
                for (int k = 0; k < 4; k++) u[i + k] = lo + i + k < n ? sg[lo + i + k] : 0u;
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
    unsigned T = 0, want = (unsigned)top;       // decided high digits; rank still wanted below them
    __syncthreads();
#pragma unroll
    for (int pass = 0; pass < 3; pass++) {
        const int nb = pass == 0 ? SEL_D1 : pass == 1 ? SEL_D2 : SEL_D3;
        const int sh = pass == 0 ? 31 - SEL_D1 : pass == 1 ? SEL_D3 : 0;
        const int nbins = 1 << nb, bpt = nbins > NT ? nbins / NT : 1;  // bins per thread (powers of 2)
#pragma unroll
        for (int i = 0; i < per; i++) {
            const unsigned v = val(i);
            if (lo + i < n && (v >> (sh + nb)) == (T >> (sh + nb)))
                atomicAdd(&L.hist[(v >> sh) & (nbins - 1)], 1u);
        }
        __syncthreads();
        // this thread's bins [tid bpt, tid bpt + bpt), read into registers and cleared for the
        // next pass (its first atomics come after this pass's last barrier)
        unsigned h[(1 << SEL_D1) > NT ? (1 << SEL_D1) / NT : 1], own = 0;
#pragma unroll
        for (int j = 0; j < bpt; j++) {
            h[j] = tid < nbins ? L.hist[tid * bpt + j] : 0u;
            own += h[j];
            if (tid < nbins) L.hist[tid * bpt + j] = 0u;
        }
        unsigned suf = own;  // inclusive suffix sum over lanes >= this one
#pragma unroll
        for (int d = 1; d < WAVE; d <<= 1) {
            const unsigned y = __shfl_down(suf, d, WAVE);
            if (lane + d < WAVE) suf += y;
        }
        if (lane == 0) L.wsum[wave] = suf;
        __syncthreads();
        unsigned above = suf - own;
        for (int w = wave + 1; w < NW; w++) above += L.wsum[w];
        if (above < want && above + own >= want) {  // the wanted rank is in one of this thread's bins
            bool found = false;
#pragma unroll
            for (int j = bpt - 1; j >= 0; j--) {
                if (!found && above + h[j] >= want) {
                    L.pick[0] = (unsigned)(tid * bpt + j);
                    L.pick[1] = above;
                    found = true;
                }
                above += h[j];
            }
        }
        __syncthreads();
        T |= L.pick[0] << sh;
        want -= L.pick[1];
    }
    // listing: per-thread counts above / equal to T, exclusive prefix over threads
    unsigned gtc = 0, eqc = 0;
#pragma unroll
    for (int i = 0; i < per; i++) {
        const unsigned v = val(i);
        gtc += lo + i < n && v > T;
        eqc += lo + i < n && v == T;
    }
    unsigned gpre, epre;
    const unsigned gw = wave_count(gtc, gpre), ew = wave_count(eqc, epre);
    if (lane == 0) {
        L.wl[0][wave] = gw;
        L.wl[1][wave] = ew;
    }
    __syncthreads();
    unsigned gt_before = gpre, eq_before = epre, gt_total = 0;
    for (int w = 0; w < NW; w++) {
        const unsigned g = L.wl[0][w], e = L.wl[1][w];
        gt_total += g;
        if (w < wave) {
            gt_before += g;
            eq_before += e;
        }
    }
    const unsigned take_eq = (unsigned)top - gt_total;  // equal-valued entries that make the top
    // this thread's output position: values above T before it plus the equal ones taken before it
    unsigned pos = gt_before + min(eq_before, take_eq), eq_seen = eq_before;
#pragma unroll
    for (int i = 0; i < per; i++) {
        const unsigned v = val(i);
        const bool in = lo + i < n, eq = in && v == T;
        const bool take = in && (v > T || (eq && eq_seen < take_eq));
        eq_seen += eq;
        if (take) emit(pos, lo + i, v);
        pos += take;
    }
}

// One workgroup of 16 waves per query over all of its complete blocks.
constexpr int SEL_THREADS = 1024, SEL_WAVES = SEL_THREADS / WAVE;

template <int PER>
__global__ void __launch_bounds__(SEL_THREADS) idx_select_kernel(const float* __restrict__ sc, int* __restrict__ blist,
                                                                 int* __restrict__ nsel, int top, int R, int pos0,
                                                                 int nbmax, int vec) {
    __shared__ SelectLds L;
    const int t = blockIdx.x, tid = threadIdx.x;
    const int n = (pos0 + t + 1) / R;
    int* out = blist + (size_t)t * top;
    if (n <= top) {  // every complete block
        for (int b = tid; b < n; b += SEL_THREADS) out[b] = b;
        if (tid == 0) nsel[t] = n;
        return;
    }
    select_top<SEL_THREADS, PER>((const unsigned*)(sc + (size_t)t * nbmax), n, top, vec, L,
                                 [&](unsigned pos, int i, unsigned) { out[pos] = i; });
    if (tid == 0) nsel[t] = top;
}

// Two-phase selection for few queries over many blocks (one workgroup per query leaves the rest
// of the GPU idle). Phase 1: workgroup (p, t) takes query t's blocks [p S, p S + S) and lists its
// local top `top` into candidate slots [(t P + p) top, ...) as (score bits + 1, block), in block
// order; a range of at most `top` blocks is copied whole and unused slots hold 0. The query's top
// blocks of the whole row are among the union of the ranges' local tops (a block beaten by `top`
// others within its range is beaten by them in the row). Phase 2 selects `top` of the P top slots
// of each query: valid slots are in block order, so ties still go to the lower block, and the
// +1 encoding keeps empty slots (0) out of every count.
constexpr int SEL1_THREADS = 256, SEL1_PER = 16, SEL1_RANGE = SEL1_THREADS * SEL1_PER;

__global__ void __launch_bounds__(SEL1_THREADS) idx_select_part_kernel(const float* __restrict__ sc,
                                                                       unsigned* __restrict__ cval,
                                                                       int* __restrict__ cidx, int top, int R,
                                                                       int pos0, int nbmax, int vec) {
    __shared__ SelectLds L;
    const int p = blockIdx.x, t = blockIdx.y, P = gridDim.x, tid = threadIdx.x;
    const int n = (pos0 + t + 1) / R;
    if (n <= top) return;  // phase 2 lists every block without reading the slots
    const int lo = p * SEL1_RANGE, len = min(max(n - lo, 0), SEL1_RANGE);
    const size_t base = ((size_t)t * P + p) * top;
    const unsigned* sg = (const unsigned*)(sc + (size_t)t * nbmax) + lo;
    if (len <= top) {
        for (int i = tid; i < top; i += SEL1_THREADS) {
            cval[base + i] = i < len ? sg[i] + 1u : 0u;
            cidx[base + i] = lo + i;
        }
        return;
    }
    select_top<SEL1_THREADS, SEL1_PER>(sg, len, top, vec, L, [&](unsigned pos, int i, unsigned v) {
        cval[base + pos] = v + 1u;
        cidx[base + pos] = lo + i;
    });
}

template <int PER>
__global__ void __launch_bounds__(SEL_THREADS) idx_select_merge_kernel(const unsigned* __restrict__ cval,
                                                                       const int* __restrict__ cidx,
                                                                       int* __restrict__ blist, int* __restrict__ nsel,
                                                                       int top, int R, int pos0, int P, int vec) {
    __shared__ SelectLds L;
    const int t = blockIdx.x, tid = threadIdx.x;
    const int n = (pos0 + t + 1) / R;
    int* out = blist + (size_t)t * top;
    if (n <= top) {
        for (int b = tid; b < n; b += SEL_THREADS) out[b] = b;
        if (tid == 0) nsel[t] = n;
        return;
    }
    const size_t m = (size_t)P * top;
    const int* ci = cidx + t * m;
    select_top<SEL_THREADS, PER>(cval + t * m, (int)m, top, vec, L,
                                 [&](unsigned pos, int i, unsigned) { out[pos] = ci[i]; });
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

// The two-phase form (few queries, many blocks) keeps its candidates in the workspace.
static bool idx_select_two_phase(int T, int top, int R, int pos0, size_t* cand_bytes) {
    const int nmax = (pos0 + T) / R;
    const int P = (nmax + SEL1_RANGE - 1) / SEL1_RANGE;
    const size_t m = (size_t)P * top;
    *cand_bytes = (size_t)T * m * 8;
    return T <= 16 && nmax > 8 * SEL_THREADS && 4 * m <= (size_t)nmax && m <= (size_t)32 * SEL_THREADS;
}

size_t aegist_idx_select_workspace_bytes(int T, int top, int R, int pos0) {
    if (T <= 0 || top <= 0 || R <= 0 || pos0 < 0) return 0;
    size_t cand = 0;
    return idx_select_two_phase(T, top, R, pos0, &cand) ? cand : 0;
}

int aegist_idx_select_ws(const float* sc, int* blist, int* nsel, int T, int top, int R, int pos0, int nbmax, void* ws,
                         size_t ws_bytes, void* stream) {
    AEG_REQUIRE(T >= 0 && top > 0 && R > 0 && pos0 >= 0, "idx_select: bad shape");
    AEG_REQUIRE((pos0 + T) / R <= nbmax, "idx_select: nbmax smaller than the number of complete blocks");
    if (T == 0) return 0;
    const int nmax = (pos0 + T) / R;  // the most complete blocks any of these queries sees
    const int vec = nbmax % 4 == 0 && (uintptr_t)sc % 16 == 0;
    hipStream_t st = AEG_STREAM(stream);
    const int P = (nmax + SEL1_RANGE - 1) / SEL1_RANGE;
    const size_t m = (size_t)P * top;
    // two phases when few queries see many blocks and the candidates are far fewer than the blocks
    size_t cand_bytes = 0;
    if (idx_select_two_phase(T, top, R, pos0, &cand_bytes)) {
        int rc = check_workspace(ws, ws_bytes, cand_bytes, "idx_select");
        if (rc) return rc;
        unsigned* cval = (unsigned*)ws;
        int* cidx = (int*)(cval + (size_t)T * m);
        idx_select_part_kernel<<<dim3(P, T), SEL1_THREADS, 0, st>>>(sc, cval, cidx, top, R, pos0, nbmax, vec);
        const int vec2 = m % 4 == 0;
        if (m <= 4 * SEL_THREADS)
            idx_select_merge_kernel<4><<<T, SEL_THREADS, 0, st>>>(cval, cidx, blist, nsel, top, R, pos0, P, vec2);
        else if (m <= 8 * SEL_THREADS)
            idx_select_merge_kernel<8><<<T, SEL_THREADS, 0, st>>>(cval, cidx, blist, nsel, top, R, pos0, P, vec2);
        else
            idx_select_merge_kernel<32><<<T, SEL_THREADS, 0, st>>>(cval, cidx, blist, nsel, top, R, pos0, P, vec2);
    } else if (nmax <= 8 * SEL_THREADS)
        idx_select_kernel<8><<<T, SEL_THREADS, 0, st>>>(sc, blist, nsel, top, R, pos0, nbmax, vec);
    else if (nmax <= 32 * SEL_THREADS)
        idx_select_kernel<32><<<T, SEL_THREADS, 0, st>>>(sc, blist, nsel, top, R, pos0, nbmax, vec);
    else
        idx_select_kernel<0><<<T, SEL_THREADS, 0, st>>>(sc, blist, nsel, top, R, pos0, nbmax, vec);
    return after_launch("idx_select");
}

int aegist_idx_select(const float* sc, int* blist, int* nsel, int T, int top, int R, int pos0, int nbmax,
                      void* stream) {
    size_t bound = 0;
    void* ws = bound_workspace(&bound);
    return aegist_idx_select_ws(sc, blist, nsel, T, top, R, pos0, nbmax, ws, bound, stream);
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
