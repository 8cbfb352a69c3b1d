// Shared device helpers for the gfx950 token-mixer kernels: bf16/fp16 conversion, wave64
// reductions, MFMA vector types, and the host-side error/launch plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

#include "../../include/aegist_mixer.h"

// ---------------------------------------------------------------------------------------------
// Vector types used as MFMA operands / accumulators.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define WAVE 64

// ---------------------------------------------------------------------------------------------
// bf16 <-> fp32. bf16 is the top half of an fp32; narrowing rounds to nearest even and maps
// NaN to a quiet NaN (one v_cvt_pk_bf16_f32 on gfx950, no branch).
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ float bf_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// two floats -> packed bf16 pair (a in the low half)
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
    typedef float f2v __attribute__((ext_vector_type(2)));
    typedef __bf16 b2v __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v{a, b}), b2v));
}

// Element load/store for the activation dtypes the ABI accepts (fp32 or bf16).
template <typename T> struct Act;
template <> struct Act<float> {
    static __device__ __forceinline__ float ld(const float* p, size_t i) { return p[i]; }
    static __device__ __forceinline__ void st(float* p, size_t i, float v) { p[i] = v; }
};
template <> struct Act<uint16_t> {
    static __device__ __forceinline__ float ld(const uint16_t* p, size_t i) { return bf2f(p[i]); }
    static __device__ __forceinline__ void st(uint16_t* p, size_t i, float v) { p[i] = f2bf(v); }
};

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + __expf(-x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + __expf(-x)); }
// sigmoid with the hardware reciprocal (1 ulp) in place of the IEEE division sequence; for
// epilogues that apply it to whole output tiles
__device__ __forceinline__ float sigmoid_rcp(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
// silu of the 4-tap causal conv at one channel: taps w0..w3 on inputs t-3, t-2, t-1, t, summed
// oldest first with explicit FMAs, so every prefill conv path rounds alike; the sigmoid takes the
// hardware reciprocal (1 ulp) instead of an IEEE division, which the GEMM epilogue that runs it
// over whole tiles cannot hide
__device__ __forceinline__ float conv4_silu(float w0, float w1, float w2, float w3, float h0, float h1, float h2,
                                            float x) {
    const float a = __builtin_fmaf(w3, x, __builtin_fmaf(w2, h2, __builtin_fmaf(w1, h1, w0 * h0)));
    return a * sigmoid_rcp(a);
}

// ---------------------------------------------------------------------------------------------
// wave64 reductions (butterfly; every lane ends with the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// Lane exchanges without LDS permutes (a permute's wait also drains every LDS read in flight):
// lane_xor<M> returns x from lane l ^ M for M = 1, 2 (DPP quad permutes) and 8 (DPP rotate of a
// 16-lane row by 8); pair_sum16 / pair_sum32 return x[l] + x[l ^ 16] / x[l] + x[l ^ 32]
// (v_permlane16_swap / v_permlane32_swap), the same bits on both lanes of a pair.
template <int M>
__device__ __forceinline__ float lane_xor(float x) {
    static_assert(M == 1 || M == 2 || M == 8, "lane_xor: M = 1, 2 or 8");
    constexpr int ctrl = M == 1 ? 0xB1 : M == 2 ? 0x4E : 0x128;
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float pair_sum16(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
__device__ __forceinline__ float pair_sum32(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

// Orders LDS traffic between the lanes of one wave (no workgroup barrier needed for
// wave-private buffers): stops compiler code motion and waits for outstanding LDS ops.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier that orders LDS traffic only: unlike __syncthreads it does not wait for the
// wave's outstanding global stores (and loads), so a barrier after a burst of stores costs no
// memory round trip. Global data passed between waves needs __syncthreads.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum over the block; `red` holds one float per wave. Every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* red) {
    int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE, nw = (blockDim.x + WAVE - 1) / WAVE;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// ---------------------------------------------------------------------------------------------
// Host side: thread-local error text and return-code helpers.
namespace aegist {
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_hip(hipError_t e, const char* what);
int after_launch(const char* what);  // launch error check; honours AEGIST_SYNC_LAUNCH
// The workspace the calling thread bound on its current device (aegist_bind_workspace) and its
// size; nullptr / 0 if none. Never allocates.
void* bound_workspace(size_t* bytes);
// AEGIST_ERR_WORKSPACE unless ws is non-null, 256-byte aligned and holds `need` bytes.
int check_workspace(const void* ws, size_t ws_bytes, size_t need, const char* who);
}  // namespace aegist

#define AEG_REQUIRE(cond, msg)                                              \
    do {                                                                    \
        if (!(cond)) return aegist::fail(AEGIST_ERR_SHAPE, std::string(msg)); \
    } while (0)

#define AEG_HIP(call)                                                  \
    do {                                                               \
        int _rc = aegist::check_hip((call), #call);                    \
        if (_rc) return _rc;                                           \
    } while (0)

#define AEG_STREAM(s) ((hipStream_t)(s))
