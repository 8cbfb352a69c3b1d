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

__global__ void __launch_bounds__(512, 1) gemm_bf16_kernel(const uint16_t* __restrict__ X, int ldx,
                                                           const uint16_t* __restrict__ W, int ldw,
                                                           float* __restrict__ Y, int ldy, int M, int N, int K,
                                                           int accumulate, int tiles_n, int ntiles, int per_xcd) {
    __shared__ __attribute__((aligned(1024))) unsigned char A0[kTileBytes];  // W tile, buffer 0
    __shared__ __attribute__((aligned(1024))) unsigned char B0[kTileBytes];  // X tile, buffer 0
    __shared__ __attribute__((aligned(1024))) unsigned char A1[kTileBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char B1[kTileBytes];

    const int li = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
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
    // L / 8, LDS slot L % 8, which holds global slot (L % 8) ^ sw(row)
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, 0x7fffffff, kBufWord3);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void*)X, (short)0, 0x7fffffff, kBufWord3);
    int voff[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
        const int j = wave * 8 + jj, tensor = j / 32, row = 8 * (j % 32) + lane / 8;
        const int gslot = (lane % 8) ^ sw(row);
        voff[jj] = tensor == 0 ? (min(n0 + row, N - 1) * ldw + 8 * gslot) * 2
                               : (min(m0 + row, M - 1) * ldx + 8 * gslot) * 2;
    }
    typedef __attribute__((address_space(3))) void lds_void;
    auto load_step = [&](unsigned char* At, unsigned char* Bt, int k0) {
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const int j = wave * 8 + jj, tensor = j / 32;
            unsigned char* dst = (tensor == 0 ? At : Bt) + (j % 32) * 1024;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(tensor == 0 ? wrs : xrs, (lds_void*)dst, 16, voff[jj], k0 * 2, 0,
                                                     0);
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
    const bool vec = (ldy % 4) == 0 && ((uintptr_t)Y % 16) == 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int m = m0 + 64 * wm + 16 * j + r16;
        if (m >= M) continue;
        float* yrow = Y + (size_t)m * ldy;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int n = n0 + 128 * wn + 16 * i + 4 * g;
            if (vec && n + 3 < N) {
                f32x4 v = acc[i][j];
                if (accumulate) v += *(const f32x4*)(yrow + n);
                *(f32x4*)(yrow + n) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (n + e < N) yrow[n + e] = (accumulate ? yrow[n + e] : 0.f) + acc[i][j][e];
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

// Y[M, N] (+)= X[M, K] W[N, K]^T, bf16 X (row stride ldx) and W (row stride ldw), fp32 Y (row
// stride ldy). Needs K % 64 == 0, 16-byte aligned rows of X and W, and buffer offsets below 2^31
// (rows x stride x 2 bytes of each operand).
int launch_gemm_bf16(const uint16_t* X, long long ldx, const uint16_t* W, long long ldw, float* Y, long long ldy, int M,
                     int N, int K, int accumulate, hipStream_t st) {
    if (M <= 0 || N <= 0) return 0;
    if (K % GBK || K <= 0) return fail(AEGIST_ERR_SHAPE, "gemm_bf16: K must be a positive multiple of 64");
    if (ldx < K || ldw < K || ldy < N || ldx % 8 || ldw % 8 || (uintptr_t)X % 16 || (uintptr_t)W % 16)
        return fail(AEGIST_ERR_SHAPE, "gemm_bf16: need ld >= K, 16-byte aligned rows");
    if ((long long)M * ldx * 2 >= 0x7fffffffLL || (long long)N * ldw * 2 >= 0x7fffffffLL)
        return fail(AEGIST_ERR_SHAPE, "gemm_bf16: an operand passes 2 GiB");
    const int tiles_m = (M + GBM - 1) / GBM, tiles_n = (N + GBN - 1) / GBN, ntiles = tiles_m * tiles_n;
    const int per_xcd = (ntiles + 7) / 8;
    gemm_bf16_kernel<<<8 * per_xcd, 512, 0, st>>>(X, (int)ldx, W, (int)ldw, Y, (int)ldy, M, N, K, accumulate, tiles_n,
                                                  ntiles, per_xcd);
    return after_launch("gemm_bf16");
}

}  // namespace aegist
