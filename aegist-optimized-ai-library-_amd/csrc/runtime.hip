// Host runtime of the C ABI: error text, device selection, memory helpers, the synthetic
// input generator and the RoPE table. Replaces the CUDA driver binding of the reference
// engine (aegist_rs/src/cuda.rs): thread-local current device instead of a context cache,
// hipError_t codes instead of CUresult strings.
#include "common.h"

#include <cmath>
#include <cstdlib>
#include <mutex>
#include <vector>

namespace aegist {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return 0;
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return (int)e;
}

static bool sync_launch() {
    static int v = [] {
        const char* s = std::getenv("AEGIST_SYNC_LAUNCH");
        return (s && s[0] && s[0] != '0') ? 1 : 0;
    }();
    return v != 0;
}

int after_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return check_hip(e, what);
    if (sync_launch()) {
        e = hipDeviceSynchronize();
        if (e != hipSuccess) return check_hip(e, what);
    }
    return 0;
}

// Workspace the engine-ABI mirrors use when their reference signature has no workspace
// argument: bound by the caller (aegist_bind_workspace), per thread and per device, so the
// library never allocates and two threads on two streams never share bytes. The engine
// preallocates its scratch the same way (hybrid.rs:630-650).
struct BoundWorkspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
static thread_local std::vector<BoundWorkspace> t_bound;

void* bound_workspace(size_t* bytes) {
    *bytes = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev >= (int)t_bound.size()) return nullptr;
    *bytes = t_bound[dev].bytes;
    return t_bound[dev].ptr;
}

int check_workspace(const void* ws, size_t ws_bytes, size_t need, const char* who) {
    if (need == 0) return 0;
    if (!ws || ws_bytes < need)
        return fail(AEGIST_ERR_WORKSPACE, std::string(who) + ": workspace of " + std::to_string(need) +
                                              " bytes required, got " + std::to_string(ws ? ws_bytes : 0) +
                                              " (pass one to the *_ws form, or bind one with aegist_bind_workspace)");
    if ((uintptr_t)ws % 256)
        return fail(AEGIST_ERR_WORKSPACE, std::string(who) + ": workspace must be 256-byte aligned");
    return 0;
}

}  // namespace aegist

using namespace aegist;

extern "C" {

const char* aegist_last_error(void) { return g_last_error.c_str(); }

const char* aegist_version(void) { return "aegist_mixer 0.1 (gfx950)"; }

int aegist_set_device(int device) { return check_hip(hipSetDevice(device), "hipSetDevice"); }

int aegist_bind_workspace(void* ws, size_t bytes) {
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    if (ws && (uintptr_t)ws % 256) return fail(AEGIST_ERR_WORKSPACE, "bind_workspace: must be 256-byte aligned");
    if ((int)t_bound.size() <= dev) t_bound.resize(dev + 1);
    t_bound[dev] = ws ? BoundWorkspace{ws, bytes} : BoundWorkspace{};
    return 0;
}

int aegist_malloc(void** ptr, size_t bytes) { return check_hip(hipMalloc(ptr, bytes), "hipMalloc"); }

int aegist_free(void* ptr) { return check_hip(hipFree(ptr), "hipFree"); }

int aegist_memcpy_htod(void* dst, const void* src, size_t bytes, void* stream) {
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, AEG_STREAM(stream)), "hipMemcpyAsync(HtoD)");
}

int aegist_memcpy_dtoh(void* dst, const void* src, size_t bytes, void* stream) {
    int rc = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, AEG_STREAM(stream)), "hipMemcpyAsync(DtoH)");
    if (rc) return rc;
    // a download is synchronous for the caller, as the reference's Buf::download (cuda.rs:239-270)
    return check_hip(hipStreamSynchronize(AEG_STREAM(stream)), "hipStreamSynchronize");
}

int aegist_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream) {
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, AEG_STREAM(stream)), "hipMemcpyAsync(DtoD)");
}

int aegist_memset(void* dst, int value, size_t bytes, void* stream) {
    return check_hip(hipMemsetAsync(dst, value, bytes, AEG_STREAM(stream)), "hipMemsetAsync");
}

int aegist_mem_info(size_t* free_bytes, size_t* total_bytes) {
    return check_hip(hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo");
}

int aegist_stream_sync(void* stream) { return check_hip(hipStreamSynchronize(AEG_STREAM(stream)), "hipStreamSynchronize"); }

int aegist_rope_inv_freq(float* inv_out, int RD, float theta) {
    if (RD <= 0 || (RD & 1)) return fail(AEGIST_ERR_SHAPE, "rope: rotary dim must be positive and even");
    for (int j = 0; j < RD / 2; j++) inv_out[j] = (float)(1.0 / std::pow((double)theta, (double)(2 * j) / (double)RD));
    return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// Counter-based normal generator: u64 = splitmix64(seed ^ golden * (i/2 + 1)); two uniforms
// from its halves; Box-Muller gives the pair (z0 for even i, z1 for odd i).
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

template <typename T>
__global__ void fill_normal_kernel(T* dst, size_t n, uint64_t seed, float mean, float std) {
    size_t pair = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; 2 * pair < n; pair += stride) {
        uint64_t r = splitmix64(seed ^ (0x9E3779B97F4A7C15ull * (pair + 1)));
        // 24-bit uniforms in (0, 1]
        float u1 = ((float)(uint32_t)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);
        float u2 = (float)(uint32_t)((r >> 8) & 0xffffffu) * (1.0f / 16777216.0f);
        float rad = sqrtf(-2.0f * logf(u1));
        float s, c;
        sincosf(6.2831853071795864f * u2, &s, &c);
        size_t i = 2 * pair;
        Act<T>::st(dst, i, mean + std * rad * c);
        if (i + 1 < n) Act<T>::st(dst, i + 1, mean + std * rad * s);
    }
}

extern "C" int aegist_fill_normal(void* dst, size_t n, int dtype, uint64_t seed, float mean, float std, void* stream) {
    if (n == 0) return 0;
    size_t pairs = (n + 1) / 2;
    unsigned blocks = (unsigned)std::min<size_t>((pairs + 255) / 256, 65536);
    if (dtype == AEGIST_F32)
        fill_normal_kernel<float><<<blocks, 256, 0, AEG_STREAM(stream)>>>((float*)dst, n, seed, mean, std);
    else if (dtype == AEGIST_BF16)
        fill_normal_kernel<uint16_t><<<blocks, 256, 0, AEG_STREAM(stream)>>>((uint16_t*)dst, n, seed, mean, std);
    else
        return fail(AEGIST_ERR_DTYPE, "fill_normal: dtype must be AEGIST_F32 or AEGIST_BF16");
    return after_launch("fill_normal");
}
