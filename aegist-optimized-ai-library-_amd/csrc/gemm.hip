// Prefill-sized projections Y[M, N] (+)= X[M, K] W[N, K]^T with bf16 X and W, fp32 Y, on
// v_mfma_f32_16x16x32_bf16 (the products are exact; the sums are fp32).
//
// One workgroup of 8 waves per 256 x 256 output tile (two per SIMD), each wave 64 rows x 128
// columns held in 32 accumulator tiles (128 registers). K runs in steps of 64: both
// operand tiles (256 rows x 64 k of W and of X, 32 KB each) arrive in LDS by direct buffer -> LDS
// loads (1 KB per instruction, no registers), double-buffered, the next step's loads issued
// before this step's products. Each load instruction moves 8 whole 128-byte rows; in LDS the
// 16-byte slots of a row are XOR-swizzled by the row (through the global address each lane
// fetches), so no fragment read has a bank conflict. W is the A operand and X the B
// operand, so a lane's accumulator holds 4 consecutive output columns of one row and the
// epilogue writes 16-byte pieces of Y rows. Rows past M or N are loaded from the last row (their
// results are not stored). XCD-aware order: XCD x runs the logical tiles [x n / 8, (x + 1) n / 8),
// grouped so that the workgroups resident on one XCD share X and W tiles in its L2.
#include "common.h"

using namespace aegist;

namespace {

constexpr int GBM = 256, GBN = 256, GBK = 64;
constexpr int kTileBytes = GBM * GBK * 2;           // one operand tile
constexpr int kGroupM = 4;  // measured: 2 and 4 alike, 1 and 8 slower
constexpr int kBufWord3 = 0x00020000;               // buffer resource word 3 on gfx9: 32-bit data, no swizzle
// LDS tiles are row-major with 128-byte rows (64 k); the 16-byte slot s of row r holds the row's
// global slot s ^ sw(r). Rows 2 apart then start 8 slots (32 banks) apart in different slot
// orders, so the 16 rows of a fragment read hit 16 distinct bank groups.
__device__ __forceinline__ int sw(int row) { return (row >> 1) & 7; }

// Up to three weight matrices stacked along N: rows [n0, n0 + N) of the combined W (and columns of
// the combined output) belong to segment s, whose W rows have stride ldw and whose outputs go to
// Y (row stride ldy). Every segment but the last has N a multiple of 8 (one load piece never
// spans two segments).
constexpr int kMaxGemmSeg = 3;
struct GemmSeg {
    const uint16_t* W;
    float* Y;
    long long ldy;
    int n0, N, ldw;
};
struct GemmArgs {
    const uint16_t* X;
    GemmSeg seg[kMaxGemmSeg];
    const uint16_t* conv_w;  // conv epilogue: [N][4] bf16 taps, tap 3 on the newest row
    float* edge;             // conv epilogue: [M / 256][6][N] raw rows 0..2 and 253..255 of every tile
    int nseg, ldx, M, N, K, accumulate, tiles_n, ntiles, per_xcd;
};

// kConv: the output is silu(causal depthwise conv4 over rows) of the product instead of the
// product itself (the DeltaNet input projection followed by its short convolution): every M tile
// is 256 consecutive tokens of one sequence, a row's three predecessors come from neighbouring
// lanes (DPP row rotations), the previous 16-row tile or, across waves, LDS; the first three rows
// of a tile have their predecessors in another tile, so their outputs are left to
// conv_edge_kernel, which gets the raw first and last three rows of every tile through `edge`.
template <bool kConv>
__global__ void __launch_bounds__(512, 1) gemm_bf16_kernel(const GemmArgs ga) {
    __shared__ __attribute__((aligned(1024))) unsigned char A0[kTileBytes];  // W tile, buffer 0
    __shared__ __attribute__((aligned(1024))) unsigned char B0[kTileBytes];  // X tile, buffer 0
    __shared__ __attribute__((aligned(1024))) unsigned char A1[kTileBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char B1[kTileBytes];

    const int M = ga.M, N = ga.N, K = ga.K, tiles_n = ga.tiles_n, ntiles = ga.ntiles;
    const int li = (blockIdx.x % 8) * ga.per_xcd + blockIdx.x / 8;
    if (li >= ntiles) return;
    // grouped order: kGroupM M tiles x all N tiles per group, M fastest, so the ~32 workgroups
    // an XCD runs at once form a kGroupM x 8 block sharing X and W tiles in its L2
    const int tiles_m = (ntiles + tiles_n - 1) / tiles_n;
    const int grp = li / (kGroupM * tiles_n), first_m = grp * kGroupM;
    const int gsize = min(tiles_m - first_m, kGroupM);
    const int inner = li - grp * kGroupM * tiles_n;
    const int m0 = (first_m + inner % gsize) * GBM, n0 = (inner / gsize) * GBN;
    // the wave index as a scalar, so the LDS destinations of the direct loads are known uniform
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
    const int r16 = lane % 16, g = lane / 16;
    const int wm = wave >> 1, wn = wave & 1;  // rows 64 wm .., columns 128 wn ..

    // loads: the 64 1-KB pieces of a step (32 per operand, 8 rows x 128 bytes each: whole cache
    // lines) are dealt 8 per wave; piece j covers rows 8 (j % 32) .. +7, lane L row 8 (j % 32) +
    // L / 8, LDS slot L % 8, which holds global slot (L % 8) ^ sw(row). A W piece reads the
    // segment its first row falls in (rows past the last segment repeat its last row).
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void*)ga.X, (short)0, 0x7fffffff, kBufWord3);
    __amdgpu_buffer_rsrc_t prs[8];
    int voff[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
        const int j = wave * 8 + jj, tensor = j / 32, row = 8 * (j % 32) + lane / 8;
        const int gslot = (lane % 8) ^ sw(row);
        if (tensor == 0) {
            const int prow = n0 + 8 * (j % 32);  // uniform
            int si = 0;
#pragma unroll
            for (int q = 1; q < kMaxGemmSeg; q++)
                if (q < ga.nseg && prow >= ga.seg[q].n0) si = q;
            const GemmSeg& sg = ga.seg[si];
            prs[jj] = __builtin_amdgcn_make_buffer_rsrc((void*)sg.W, (short)0, 0x7fffffff, kBufWord3);
            voff[jj] = (min(n0 + row - sg.n0, sg.N - 1) * sg.ldw + 8 * gslot) * 2;
        } else {
            prs[jj] = xrs;
            voff[jj] = (min(m0 + row, M - 1) * ga.ldx + 8 * gslot) * 2;
        }
    }
    typedef __attribute__((address_space(3))) void lds_void;
    auto load_step = [&](unsigned char* At, unsigned char* Bt, int k0) {
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const int j = wave * 8 + jj, tensor = j / 32;
            unsigned char* dst = (tensor == 0 ? At : Bt) + (j % 32) * 1024;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(prs[jj], (lds_void*)dst, 16, voff[jj], k0 * 2, 0, 0);
        }
    };

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // products of one step: per 32-k half, 8 W fragments (rows 128 wn + 16 i) and 4 X fragments
    // (rows 64 wm + 16 j), 32 products. Fragment row 16 q + r16, global slot 4 ks + g sits at
    // byte (16 q + r16) 128 + ((4 ks + g) ^ sw(r16)) 16 of its tile (16 q leaves sw unchanged)
    const int aswz[2] = {((0 + g) ^ sw(r16)) * 16, ((4 + g) ^ sw(r16)) * 16};
    const int abase = (128 * wn + r16) * 128, bbase = (64 * wm + r16) * 128;
    auto compute = [&](const unsigned char* At, const unsigned char* Bt) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            bf16x8 a[8], b[2];
#pragma unroll
            for (int i = 0; i < 8; i++) a[i] = *(const bf16x8*)(At + abase + aswz[ks] + 16 * i * 128);
            b[0] = *(const bf16x8*)(Bt + bbase + aswz[ks]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (j + 1 < 4) b[(j + 1) & 1] = *(const bf16x8*)(Bt + bbase + aswz[ks] + 16 * (j + 1) * 128);
#pragma unroll
                for (int i = 0; i < 8; i++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j & 1], acc[i][j], 0, 0, 0);
            }
        }
    };

    const int nk = K / GBK;
    load_step(A0, B0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // unrolled by two so each buffer is a separate array (the compiler can then tell the direct
    // loads into one buffer from the reads of the other)
    int s = 0;
    for (; s + 2 <= nk; s += 2) {
        if (s + 1 < nk) load_step(A1, B1, (s + 1) * GBK);
        compute(A0, B0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (s + 2 < nk) load_step(A0, B0, (s + 2) * GBK);
        compute(A1, B1);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }
    if (s < nk) compute(A0, B0);

    // lane (c = r16, g) of tile (i, j) holds Y[m][n .. n + 3], m = m0 + 64 wm + 16 j + c,
    // n = n0 + 128 wn + 16 i + 4 g
    if constexpr (!kConv) {
        // each lane's segment is picked by selects over the (uniform) segment fields: indexing
        // the argument array by a lane value would read it from memory, one wait per access
        const GemmSeg s0 = ga.seg[0], s1 = ga.seg[1], s2 = ga.seg[2];
        const int b1 = ga.nseg > 1 ? s1.n0 : 0x7fffffff, b2 = ga.nseg > 2 ? s2.n0 : 0x7fffffff;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int n = n0 + 128 * wn + 16 * i + 4 * g;
            if (n >= N) continue;
            const bool in2 = n >= b2, in1 = !in2 && n >= b1;
            float* const Yb = in2 ? s2.Y : in1 ? s1.Y : s0.Y;
            const long long ldy = in2 ? s2.ldy : in1 ? s1.ldy : s0.ldy;
            const int nl = n - (in2 ? b2 : in1 ? b1 : 0);  // 4-aligned; boundaries are multiples of 8
            const int sN = in2 ? s2.N : in1 ? s1.N : s0.N;
            const bool vec = (ldy % 4) == 0 && ((uintptr_t)Yb % 16) == 0 && nl + 3 < sN;
            if (vec) {
                // stores take their data straight from the accumulators, which nothing writes
                // afterwards (a temporary would be reused by the next group and have to wait for
                // the store to finish); the old values of the 4 rows are all requested first
                if (ga.accumulate) {
                    f32x4 old[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int m = m0 + 64 * wm + 16 * j + r16;
                        old[j] = m < M ? *(const f32x4*)(Yb + (size_t)m * ldy + nl) : f32x4{0.f, 0.f, 0.f, 0.f};
                    }
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[i][j] += old[j];
                }
                // nontemporal: Y is written once and read by the next launch, and the stores kept
                // out of L2 leave it to the operand tiles (qkv 8192 x 2048 at M = 32768: 1190 -> 1100 us)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int m = m0 + 64 * wm + 16 * j + r16;
                    if (m < M) __builtin_nontemporal_store(acc[i][j], (f32x4*)(Yb + (size_t)m * ldy + nl));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int m = m0 + 64 * wm + 16 * j + r16;
                    if (m >= M) continue;
                    float* y = Yb + (size_t)m * ldy + nl;
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (nl + e < sN) y[e] = (ga.accumulate ? y[e] : 0.f) + acc[i][j][e];
                }
            }
        }
    } else {
        // one segment, M a multiple of 256, no accumulation (the launcher checks). The previous
        // wave along M (wave - 2) publishes its last 16-row tile through LDS.
        // the taps of the lane's 4 columns per 16-column group, requested before the exchange so
        // their latency hides behind it (columns past N read column 0)
        uint4 wq[8][2];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int n = n0 + 128 * wn + 16 * i + 4 * g;
            const uint16_t* wp = ga.conv_w + (size_t)(n < N ? n : 0) * 4;
            wq[i][0] = *(const uint4*)wp;        // columns n, n + 1
            wq[i][1] = *(const uint4*)(wp + 8);  // columns n + 2, n + 3
        }
        __syncthreads();  // every wave is past its last LDS operand read
        // [8 i][64 lanes] per wave, waves 0..3 in A0 and 4..7 in B0 (32 KB each)
        auto xch = [&](int w, int i) { return (f32x4*)(w < 4 ? A0 : B0) + ((w % 4) * 8 + i) * WAVE; };
#pragma unroll
        for (int i = 0; i < 8; i++) xch(wave, i)[lane] = acc[i][3];
        __syncthreads();
        const GemmSeg& sg = ga.seg[0];
        const int tile_m = m0 / GBM;
        // DPP row rotate right by k: lane r16 of each 16-lane row takes lane (r16 - k) mod 16
        auto ror = [](f32x4 v, auto kc) {
            f32x4 r;
#pragma unroll
            for (int e = 0; e < 4; e++)
                r[e] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v[e]), 0x120 + decltype(kc)::value, 0xf,
                                                               0xf, false));
            return r;
        };
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int n = n0 + 128 * wn + 16 * i + 4 * g;
            const bool nok = n < N;  // N is a multiple of 4
            const uint4 w01 = wq[i][0], w23 = wq[i][1];
            float wt[4][4];
            {
                const uint32_t wv[8] = {w01.x, w01.y, w01.z, w01.w, w23.x, w23.y, w23.z, w23.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    wt[e][0] = bf_lo(wv[2 * e]);
                    wt[e][1] = bf_hi(wv[2 * e]);
                    wt[e][2] = bf_lo(wv[2 * e + 1]);
                    wt[e][3] = bf_hi(wv[2 * e + 1]);
                }
            }
            // rows 13..15 of the previous wave's last tile, rotated as ror would
            f32x4 pw[3];
#pragma unroll
            for (int k = 1; k <= 3; k++)
                pw[k - 1] = wm > 0 ? xch(wave - 2, i)[16 * g + ((r16 - k) & 15)] : f32x4{0.f, 0.f, 0.f, 0.f};
            f32x4 prev_r1 = pw[0], prev_r2 = pw[1], prev_r3 = pw[2];  // rotations of the tile above
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const f32x4 x = acc[i][j];
                const f32x4 r1 = ror(x, std::integral_constant<int, 1>{});
                const f32x4 r2 = ror(x, std::integral_constant<int, 2>{});
                const f32x4 r3 = ror(x, std::integral_constant<int, 3>{});
                const f32x4 h2 = r16 >= 1 ? r1 : prev_r1;  // row m - 1
                const f32x4 h1 = r16 >= 2 ? r2 : prev_r2;  // row m - 2
                const f32x4 h0 = r16 >= 3 ? r3 : prev_r3;  // row m - 3
                prev_r1 = r1;
                prev_r2 = r2;
                prev_r3 = r3;
                const int lr = 64 * wm + 16 * j + r16, m = m0 + lr;
                if (!nok) continue;
                if (lr >= 3) {
                    f32x4 o;
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        o[e] = conv4_silu(wt[e][0], wt[e][1], wt[e][2], wt[e][3], h0[e], h1[e], h2[e], x[e]);
                    __builtin_nontemporal_store(o, (f32x4*)(sg.Y + (size_t)m * sg.ldy + n));
                }
                if (lr < 3 || lr >= GBM - 3)
                    *(f32x4*)(ga.edge + ((size_t)tile_m * 6 + (lr < 3 ? lr : lr - (GBM - 6))) * N + n) = x;
            }
        }
    }
}

// The conv outputs of the first three rows of every 256-row tile and the new conv state, from
// the raw edge rows the conv GEMM saved. One thread per (sequence, channel) walks the sequence's
// tiles in order: the rows before tile 0 are the old state (its inputs before token 0), before
// tile t > 0 the last three raw rows of tile t - 1; the state afterwards holds the last three raw
// rows of the sequence. y and edge as in gemm_bf16_kernel<true>, state [B, C, 3] oldest first.
__global__ void conv_edge_kernel(const float* __restrict__ edge, const uint16_t* __restrict__ w,
                                 float* __restrict__ y, long long ldy, float* __restrict__ state, int T, int C) {
    const int b = blockIdx.y, c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    const uint2 wp = *(const uint2*)(w + (size_t)c * 4);
    const float w0 = bf_lo(wp.x), w1 = bf_hi(wp.x), w2 = bf_lo(wp.y), w3 = bf_hi(wp.y);
    float* st = state + ((size_t)b * C + c) * 3;
    float h0 = st[0], h1 = st[1], h2 = st[2];
    const int nt = T / GBM;
    for (int t = 0; t < nt; t++) {
        const float* e = edge + (size_t)(b * nt + t) * 6 * C + c;
        const float x0 = e[0], x1 = e[C], x2 = e[2 * (size_t)C];
        const float xs[3] = {x0, x1, x2};
        float* yr = y + ((size_t)b * T + (size_t)t * GBM) * ldy + c;
#pragma unroll
        for (int r = 0; r < 3; r++) {
            yr[(size_t)r * ldy] = conv4_silu(w0, w1, w2, w3, h0, h1, h2, xs[r]);
            h0 = h1;
            h1 = h2;
            h2 = xs[r];
        }
        h0 = e[3 * (size_t)C];
        h1 = e[4 * (size_t)C];
        h2 = e[5 * (size_t)C];
    }
    st[0] = h0;
    st[1] = h1;
    st[2] = h2;
}


// ---------------------------------------------------------------------------------------------
// The engine's QLinear GEMM past 64 rows: Y[M, N] (+)= scale[n] X[M, K] W[N, K]^T with fp32 X,
// int8 W and bf16 row scales (aegist.cu:126-172). Same tiling, waves and order as above, K in
// steps of 32 through a 3-stage ring: per stage the W tile is 256 rows x 32 bytes (8 KB) and the X
// tile 256 rows x 128 bytes (32 KB), both by direct loads issued two steps ahead (120 KB of LDS:
// the destinations of direct loads stay below 128 KB). W fragments convert to bf16 exactly
// (|q| <= 127 keeps 8 significant bits); X fragments split into bf16 hi (truncated) + lo
// (rounded), two products per pair, so the result is within 2^-16 of an fp32 dot product, as in
// the weight-streaming kernel. Swizzles: W rows (2 slots of 16 bytes) by (row >> 3) & 1, X rows
// (8 slots) by (row >> 1) & 7, both conflict-free for 16-row fragment reads.
constexpr int GBK8 = 32;
constexpr int kWTile8 = GBM * GBK8;       // int8 W tile (8 KB)
constexpr int kXTile32 = GBM * GBK8 * 4;  // fp32 X tile (32 KB)
__device__ __forceinline__ int sww(int row) { return (row >> 3) & 1; }
__device__ __forceinline__ int swx(int row) { return (row >> 1) & 7; }

#define GEMM_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8))

__global__ void __launch_bounds__(512, 1) gemm_i8f32_kernel(const float* __restrict__ X, int ldx,
                                                            const int8_t* __restrict__ W, int ldw,
                                                            const uint16_t* __restrict__ scale,
                                                            float* __restrict__ Y, int ldy, int M, int N, int K,
                                                            int accumulate, int tiles_n, int ntiles, int per_xcd) {
    __shared__ __attribute__((aligned(1024))) unsigned char S0[kWTile8 + kXTile32];  // W tile, then X tile
    __shared__ __attribute__((aligned(1024))) unsigned char S1[kWTile8 + kXTile32];
    __shared__ __attribute__((aligned(1024))) unsigned char S2[kWTile8 + kXTile32];

    const int li = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (li >= ntiles) return;
    const int tiles_m = (ntiles + tiles_n - 1) / tiles_n;
    const int grp = li / (kGroupM * tiles_n), first_m = grp * kGroupM;
    const int gsize = min(tiles_m - first_m, kGroupM);
    const int inner = li - grp * kGroupM * tiles_n;
    const int m0 = (first_m + inner % gsize) * GBM, n0 = (inner / gsize) * GBN;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
    const int r16 = lane % 16, g = lane / 16;
    const int wm = wave >> 1, wn = wave & 1;

    // loads per stage: 8 W pieces (32 rows x 32 bytes) and 32 X pieces (8 rows x 128 bytes), 5 per
    // wave: W piece `wave`, X pieces 4 wave .. 4 wave + 3
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, 0x7fffffff, kBufWord3);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void*)X, (short)0, 0x7fffffff, kBufWord3);
    int voff[5];
    {
        const int row = 32 * wave + lane / 2, gslot = (lane % 2) ^ sww(row);
        voff[0] = min(n0 + row, N - 1) * ldw + 16 * gslot;
    }
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        const int row = 8 * (4 * wave + jj) + lane / 8, gslot = (lane % 8) ^ swx(row);
        voff[1 + jj] = min(m0 + row, M - 1) * ldx * 4 + 16 * gslot;
    }
    const int nk = K / GBK8;
    typedef __attribute__((address_space(3))) void lds_void;
    auto load = [&](unsigned char* St, int step) {
        if (step >= nk) return;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void*)(St + wave * 1024), 16, voff[0], step * GBK8, 0, 0);
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (lds_void*)(St + kWTile8 + (4 * wave + jj) * 1024), 16,
                                                     voff[1 + jj], step * GBK8 * 4, 0, 0);
    };
    // wait until this wave's loads of step t have landed, given the last step issued so far
    auto wait_step = [&](int t, int issued) {
        const int later = min(issued, nk - 1) - t;
        if (later >= 1) GEMM_WAIT_VM(5);
        else GEMM_WAIT_VM(0);
    };

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // W fragment (row 128 wn + 16 i + r16, k 8 g .. +7): 8 bytes at slot g / 2, half g % 2; X
    // fragment (row 64 wm + 16 j + r16, same k): 32 bytes = slots 2 g, 2 g + 1
    auto compute = [&](const unsigned char* St) {
        bf16x8 a[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int row = 128 * wn + 16 * i + r16;
            const uint2 q = *(const uint2*)(St + row * 32 + ((g / 2) ^ sww(row)) * 16 + (g % 2) * 8);
            uint32_t p[4];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t d = h ? q.y : q.x;
                const float f0 = (float)(int8_t)d, f1 = (float)(int8_t)(d >> 8);
                const float f2 = (float)(int8_t)(d >> 16), f3 = (float)(int8_t)(d >> 24);
                p[2 * h] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
                p[2 * h + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
            }
            a[i] = __builtin_bit_cast(bf16x8, p);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = 64 * wm + 16 * j + r16;
            const unsigned char* xr = St + kWTile8 + row * 128;
            const f32x4 x0 = *(const f32x4*)(xr + ((2 * g) ^ swx(row)) * 16);
            const f32x4 x1 = *(const f32x4*)(xr + ((2 * g + 1) ^ swx(row)) * 16);
            uint32_t hh[4], ll[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float v0 = e < 2 ? x0[2 * e] : x1[2 * e - 4], v1 = e < 2 ? x0[2 * e + 1] : x1[2 * e - 3];
                hh[e] = __builtin_amdgcn_perm(__float_as_uint(v1), __float_as_uint(v0), 0x07060302u);
                typedef float f2 __attribute__((ext_vector_type(2)));
                typedef __bf16 b2 __attribute__((ext_vector_type(2)));
                const f2 lo = {v0 - __uint_as_float(__float_as_uint(v0) & 0xffff0000u),
                               v1 - __uint_as_float(__float_as_uint(v1) & 0xffff0000u)};
                ll[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, b2));
            }
            const bf16x8 bh = __builtin_bit_cast(bf16x8, hh), bl = __builtin_bit_cast(bf16x8, ll);
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bh, acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bl, acc[i][j], 0, 0, 0);
        }
    };
    // step t: loads of step t + 2 into the stage step t - 1 used, products of step t, then this
    // wave's loads of step t + 1 waited for and published by the barrier
    auto step = [&](int t, unsigned char* Sc, unsigned char* Sn2) {
        load(Sn2, t + 2);
        compute(Sc);
        wait_step(t + 1, t + 2);
        __syncthreads();
    };
    load(S0, 0);
    load(S1, 1);
    wait_step(0, 1);
    __syncthreads();
    // unrolled by three so each stage is a separate array
    int s = 0;
    for (; s + 3 <= nk; s += 3) {
        step(s, S0, S2);
        step(s + 1, S1, S0);
        step(s + 2, S2, S1);
    }
    if (s < nk) step(s, S0, S2);
    if (s + 1 < nk) step(s + 1, S1, S0);

    const bool vec = (ldy % 4) == 0 && ((uintptr_t)Y % 16) == 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int n = n0 + 128 * wn + 16 * i + 4 * g;
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; e++) sc[e] = scale ? bf2f(scale[min(n + e, N - 1)]) : 1.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int m = m0 + 64 * wm + 16 * j + r16;
            if (m >= M) continue;
            float* yrow = Y + (size_t)m * ldy;
            if (vec && n + 3 < N) {
                f32x4 v = acc[i][j];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] *= sc[e];
                if (accumulate) v += *(const f32x4*)(yrow + n);
                __builtin_nontemporal_store(v, (f32x4*)(yrow + n));
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (n + e < N) yrow[n + e] = (accumulate ? yrow[n + e] : 0.f) + acc[i][j][e] * sc[e];
            }
        }
    }
}

}  // namespace

namespace aegist {

// whether launch_gemm_bf16 takes these operands
bool gemm_bf16_fits(const void* X, long long ldx, const void* W, long long ldw, int M, int N, int K) {
    return K > 0 && K % GBK == 0 && ldx >= K && ldw >= K && ldx % 8 == 0 && ldw % 8 == 0 && (uintptr_t)X % 16 == 0 &&
           (uintptr_t)W % 16 == 0 && (long long)M * ldx * 2 < 0x7fffffffLL && (long long)N * ldw * 2 < 0x7fffffffLL;
}

// whether launch_gemm_i8f32 takes these operands
bool gemm_i8f32_fits(const void* X, long long ldx, const void* W, long long ldw, int M, int N, int K) {
    return K > 0 && K % GBK8 == 0 && ldx >= K && ldw >= K && ldx % 4 == 0 && ldw % 16 == 0 && (uintptr_t)X % 16 == 0 &&
           (uintptr_t)W % 16 == 0 && (long long)M * ldx * 4 < 0x7fffffffLL && (long long)N * ldw < 0x7fffffffLL;
}

// Y[M, N] (+)= scale[n] X[M, K] W[N, K]^T, fp32 X, int8 W, bf16 scale (NULL = 1), fp32 Y.
int launch_gemm_i8f32(const float* X, long long ldx, const int8_t* W, long long ldw, const uint16_t* scale, float* Y,
                      long long ldy, int M, int N, int K, int accumulate, hipStream_t st) {
    if (M <= 0 || N <= 0) return 0;
    if (!gemm_i8f32_fits(X, ldx, W, ldw, M, N, K) || ldy < N)
        return fail(AEGIST_ERR_SHAPE, "gemm_i8: need K % 32 == 0, ld >= K, 16-byte aligned rows, operands < 2 GiB");
    const int tiles_m = (M + GBM - 1) / GBM, tiles_n = (N + GBN - 1) / GBN, ntiles = tiles_m * tiles_n;
    const int per_xcd = (ntiles + 7) / 8;
    gemm_i8f32_kernel<<<8 * per_xcd, 512, 0, st>>>(X, (int)ldx, W, (int)ldw, scale, Y, (int)ldy, M, N, K, accumulate,
                                                   tiles_n, ntiles, per_xcd);
    return after_launch("gemm_i8");
}

// Y_s[M, N_s] (+)= X[M, K] W_s[N_s, K]^T for nseg (<= 3) weights sharing X, in one launch: the
// weights are stacked along N (each segment but the last with N_s % 8 == 0), bf16 X (row stride
// ldx) and W_s (row stride ldw_s), fp32 Y_s (row stride ldy_s). Needs K % 64 == 0, 16-byte
// aligned rows of X and W_s, and buffer offsets below 2^31 (rows x stride x 2 bytes).
int launch_gemm_bf16_multi(const uint16_t* X, long long ldx, int nseg, const uint16_t* const* W, const long long* ldw,
                           float* const* Y, const long long* ldy, const int* N, int M, int K, int accumulate,
                           hipStream_t st) {
    if (nseg < 1 || nseg > kMaxGemmSeg) return fail(AEGIST_ERR_SHAPE, "gemm_bf16: 1 to 3 weights per launch");
    if (K % GBK || K <= 0) return fail(AEGIST_ERR_SHAPE, "gemm_bf16: K must be a positive multiple of 64");
    if (ldx < K || ldx % 8 || (uintptr_t)X % 16 || (long long)M * ldx * 2 >= 0x7fffffffLL)
        return fail(AEGIST_ERR_SHAPE, "gemm_bf16: X needs ldx >= K, 16-byte aligned rows, < 2 GiB");
    GemmArgs ga{};
    ga.X = X;
    int nt = 0;
    for (int i = 0; i < nseg; i++) {
        if (N[i] <= 0) continue;
        if (ldw[i] < K || ldy[i] < N[i] || ldw[i] % 8 || (uintptr_t)W[i] % 16 ||
            (long long)N[i] * ldw[i] * 2 >= 0x7fffffffLL)
            return fail(AEGIST_ERR_SHAPE, "gemm_bf16: need ldw >= K, ldy >= N, 16-byte aligned W rows, W < 2 GiB");
        if (ga.nseg > 0 && ga.seg[ga.nseg - 1].N % 8)
            return fail(AEGIST_ERR_SHAPE, "gemm_bf16: every weight but the last needs N % 8 == 0");
        ga.seg[ga.nseg++] = GemmSeg{W[i], Y[i], ldy[i], nt, N[i], (int)ldw[i]};
        nt += N[i];
    }
    if (M <= 0 || ga.nseg == 0) return 0;
    ga.ldx = (int)ldx;
    ga.M = M;
    ga.N = nt;
    ga.K = K;
    ga.accumulate = accumulate;
    const int tiles_m = (M + GBM - 1) / GBM;
    ga.tiles_n = (nt + GBN - 1) / GBN;
    ga.ntiles = tiles_m * ga.tiles_n;
    ga.per_xcd = (ga.ntiles + 7) / 8;
    gemm_bf16_kernel<false><<<8 * ga.per_xcd, 512, 0, st>>>(ga);
    return after_launch("gemm_bf16");
}

// Y[M, N] (+)= X[M, K] W[N, K]^T, one weight (as above).
int launch_gemm_bf16(const uint16_t* X, long long ldx, const uint16_t* W, long long ldw, float* Y, long long ldy, int M,
                     int N, int K, int accumulate, hipStream_t st) {
    if (M <= 0 || N <= 0) return 0;
    return launch_gemm_bf16_multi(X, ldx, 1, &W, &ldw, &Y, &ldy, &N, M, K, accumulate, st);
}

// Bytes of the edge buffer launch_gemm_bf16_conv needs for M rows of N channels.
size_t gemm_conv_edge_bytes(int M, int N) { return (size_t)(M / GBM) * 6 * N * 4; }

// Whether launch_gemm_bf16_conv takes these operands: B sequences of T tokens (M = B T), T a
// multiple of the 256-row tile, N a multiple of 4, aligned rows, operands below 2 GiB.
bool gemm_conv_fits(const void* X, long long ldx, const void* W, long long ldw, const void* conv_w, int B, int T, int N,
                    int K) {
    return B > 0 && T > 0 && T % GBM == 0 && N % 4 == 0 && (uintptr_t)conv_w % 16 == 0 &&
           gemm_bf16_fits(X, ldx, W, ldw, B * T, N, K);
}

// y[B T, N] = silu(conv4_t(X W^T)) per sequence with the causal depthwise conv over tokens (taps
// conv_w [N][4], the inputs before token 0 from state [B, N, 3], which then holds the last three
// raw rows): the projection and the DeltaNet short convolution in one GEMM launch plus a small
// edge launch, so the raw projection never reaches HBM. edge: gemm_conv_edge_bytes(B T, N).
int launch_gemm_bf16_conv(const uint16_t* X, long long ldx, const uint16_t* W, long long ldw, const uint16_t* conv_w,
                          float* state, float* y, long long ldy, float* edge, int B, int T, int N, int K,
                          hipStream_t st) {
    if (!gemm_conv_fits(X, ldx, W, ldw, conv_w, B, T, N, K) || ldy < N || ldy % 4 || (uintptr_t)y % 16 ||
        (uintptr_t)edge % 16)
        return fail(AEGIST_ERR_SHAPE, "gemm_bf16_conv: need T % 256 == 0, N % 4 == 0, aligned rows");
    const int M = B * T;
    GemmArgs ga{};
    ga.X = X;
    ga.seg[0] = GemmSeg{W, y, ldy, 0, N, (int)ldw};
    ga.nseg = 1;
    ga.conv_w = conv_w;
    ga.edge = edge;
    ga.ldx = (int)ldx;
    ga.M = M;
    ga.N = N;
    ga.K = K;
    ga.accumulate = 0;
    ga.tiles_n = (N + GBN - 1) / GBN;
    ga.ntiles = (M / GBM) * ga.tiles_n;
    ga.per_xcd = (ga.ntiles + 7) / 8;
    gemm_bf16_kernel<true><<<8 * ga.per_xcd, 512, 0, st>>>(ga);
    int rc = after_launch("gemm_bf16_conv");
    if (rc) return rc;
    conv_edge_kernel<<<dim3((N + 255) / 256, B), 256, 0, st>>>(edge, conv_w, y, ldy, state, T, N);
    return after_launch("conv_edge");
}

}  // namespace aegist
