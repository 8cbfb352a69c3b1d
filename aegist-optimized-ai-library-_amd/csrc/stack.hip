// The hybrid mixer stack: a batched, native counterpart of HybridEngine::forward_chunk /
// HybridEngine::mixer (aegist_rs/src/hybrid.rs:760-861) and HybridBlock.forward with the MoE
// FFN replaced by the identity (aegist/hybrid.py:812-843): for every layer
//     x = x + mixer(znorm(x))
// where the mixer is the gated DeltaNet (hybrid.py:388-421) or the gated GQA attention
// (hybrid.py:280-311). The stack owns the recurrent state, conv state and bf16 KV cache of every
// layer (HybridCache, hybrid.py:171-260; the engine buffers of hybrid.rs:607-629).
//
// Projections are plain GEMMs (bf16 operands, fp32 accumulation and output; the out-projections
// accumulate straight into the fp32 residual): decode-sized ones on this library's
// weight-streaming MFMA kernel, prefill-sized ones on its tiled MFMA GEMM; every op is one of
// this library's kernels (no vendor BLAS).
#include "common.h"

#include <algorithm>
#include <vector>

namespace aegist {
int launch_znorm_bf16(const float* x, const uint16_t* w, uint16_t* out, int rows, int D, float eps, hipStream_t st);
int launch_znorm_bf16_acc(float* x, const float* part, int nks, const uint16_t* w, uint16_t* out, int rows, int D,
                          float eps, hipStream_t st);
int launch_proj_splitk(const uint16_t* X, long long ldx, const uint16_t* W, float* part, int nks, int M, int N, int K,
                       hipStream_t st);
int launch_cast_bf16(const float* x, uint16_t* y, size_t n, hipStream_t st);
int launch_gates_from_proj(const float* ba, const uint16_t* a_log, const uint16_t* dt_bias, float* g, float* beta,
                           int rows, int HV, hipStream_t st);
int launch_gated_norm_bf16(const float* o, const float* z, const uint16_t* w, uint16_t* out, int rows, int DV,
                           float eps, hipStream_t st);
int launch_conv_silu_batched(const float* x, float* y, const uint16_t* w, float* state, int B, int T, int C,
                             hipStream_t st);
int launch_embed_bf16(const uint16_t* table, const int* ids, float* out, int n, int D, hipStream_t st);
int launch_delta_decode_stack(const float* qkv, const uint16_t* conv_w, float* conv_state, const float* ba,
                              const uint16_t* a_log, const uint16_t* dt_bias, const float* z, const uint16_t* gnorm_w,
                              float gnorm_eps, float* state, uint16_t* ob, int B, int HK, int HV, float qscale,
                              float eps, hipStream_t st);
int launch_attn_prep(const void* qg, const void* k, const void* v, int in_dtype, const uint16_t* qw,
                     const uint16_t* kw, float* qn, uint16_t* kc, uint16_t* vc, int B, int T, int H, int KV, int HD,
                     int RD, int pos0, int cap, float eps, float theta, hipStream_t stream);
int stack_attn_decode(const float* qn, const uint16_t* kc, const uint16_t* vc, const float* qg, uint16_t* out, int B,
                      int H, int KV, int L, int cap, float scale, void* ws, size_t ws_bytes, hipStream_t st);
int stack_attn_decode_fused(const float* qg, const float* kn, const float* vn, const uint16_t* qw, const uint16_t* kw,
                            uint16_t* kc, uint16_t* vc, uint16_t* out, int B, int H, int KV, int pos, int cap, float eps,
                            float theta, void* ws, size_t ws_bytes, hipStream_t st);
int stack_attn_prefill(const float* qn, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out, int B,
                       int H, int KV, int T, int pos, int cap, float scale, void* ws, size_t ws_bytes, hipStream_t st,
                       uint16_t* out_bf16, bool* wrote_bf16);
size_t prefill_f16_bytes(int B, int KV, int rows);
bool gemm_bf16_fits(const void* X, long long ldx, const void* W, long long ldw, int M, int N, int K);
int launch_gemm_bf16(const uint16_t* X, long long ldx, const uint16_t* W, long long ldw, float* Y, long long ldy, int M,
                     int N, int K, int accumulate, hipStream_t st);
int launch_gemm_bf16_multi(const uint16_t* X, long long ldx, int nseg, const uint16_t* const* W, const long long* ldw,
                           float* const* Y, const long long* ldy, const int* N, int M, int K, int accumulate,
                           hipStream_t st);
bool gemm_conv_fits(const void* X, long long ldx, const void* W, long long ldw, const void* conv_w, int B, int T, int N,
                    int K);
int launch_gemm_bf16_conv(const uint16_t* X, long long ldx, const uint16_t* W, long long ldw, const uint16_t* conv_w,
                          float* state, float* y, long long ldy, float* edge, int B, int T, int N, int K,
                          hipStream_t st);
size_t decode_workspace_bytes(int B, int H, int KV, int L, bool with_q);
int launch_proj(const void* X, int x_dtype, long long ldx, const void* W, int w_dtype, const uint16_t* scale, float* Y,
                long long ldy, int M, int N, int K, int accumulate, hipStream_t st);
int launch_proj_multi(const void* X, int x_dtype, long long ldx, int w_dtype, int nseg, const void* const* W,
                      const uint16_t* const* scale, float* const* Y, const long long* ldy, const int* N, int M, int K,
                      int accumulate, hipStream_t st);
}  // namespace aegist

using namespace aegist;

namespace {

constexpr int D = 128;  // dk = dv

struct Buf {
    void* p = nullptr;
    size_t n = 0;
};

struct Stack {
    AegistStackConfig cfg;
    std::vector<AegistLayerWeights> w;
    std::vector<int> slot;  // per layer: index among its kind
    int n_delta = 0, n_attn = 0, length = 0, device = 0;
    // states
    float* conv = nullptr;     // [n_delta, maxB, C, 3]
    float* rec = nullptr;      // [n_delta, maxB, HV, 128, 128]
    uint16_t* kc = nullptr;    // [n_attn, maxB, KV, cap, HD]
    uint16_t* vc = nullptr;
    // per-call scratch (max_tokens rows)
    uint16_t* hb = nullptr;    // znorm out, bf16 [rows, d]
    float* proj = nullptr;     // qkv or q|gate [rows, max(C, 2 H HD)]
    float* z = nullptr;        // [rows, HV 128]
    float* kv2 = nullptr;      // k then v projections [2, rows, KV HD]
    float* ba = nullptr;       // [rows, 2 HV]
    float* g = nullptr;        // [rows, HV]
    float* beta = nullptr;     // [rows, HV]
    float* y = nullptr;        // conv out [rows, C], or attention q_n [rows, H, HD]
    float* o = nullptr;        // mixer core out [rows, max(HV 128, H HD)]
    uint16_t* ob = nullptr;    // bf16 copy of o (GEMM input)
    float* part = nullptr;     // split-K slices of the last out projection [kOutSplits, 16, d]
    int pend = 0;              // slices in `part` not yet added into the residual
    void* ws = nullptr;        // chunked prefill / attention decode workspace
    size_t ws_bytes = 0;
    // snapshots of the recurrent layers' conv and recurrent states (the KV cache is append-only,
    // so rewinding the length is enough for it); position -1 = empty slot
    float* snap_conv[AEGIST_STACK_SNAPSHOTS] = {};
    float* snap_rec[AEGIST_STACK_SNAPSHOTS] = {};
    int snap_pos[AEGIST_STACK_SNAPSHOTS] = {};
    std::vector<void*> allocs;

    int C() const { return 2 * cfg.hk * D + cfg.hv * D; }
    size_t conv_bytes() const { return (size_t)std::max(1, n_delta) * cfg.max_batch * C() * 3 * 4; }
    size_t rec_bytes() const { return (size_t)std::max(1, n_delta) * cfg.max_batch * cfg.hv * D * D * 4; }
};

int alloc(Stack* s, void** p, size_t bytes) {
    int rc = check_hip(hipMalloc(p, std::max<size_t>(bytes, 256)), "hipMalloc(stack)");
    if (!rc) s->allocs.push_back(*p);
    return rc;
}

// Y[M, N] (row-major, leading dim ldy) = A[M, K] (bf16 row-major) . W[N, K]^T (bf16 row-major)
//                                          + beta * Y,   beta in {0, 1}
// Decode-sized M (<= 64 rows) goes to the weight-streaming kernels (one pass over W), larger M
// to the tiled MFMA GEMM; shapes the GEMM does not take (K not a multiple of its k step) to the
// streaming kernels' row-group form.
int gemm(Stack*, const uint16_t* A, const uint16_t* W, float* Y, int M, int N, int K, int ldy, float beta,
         hipStream_t stream) {
    if (M > 64 && gemm_bf16_fits(A, K, W, K, M, N, K))
        return launch_gemm_bf16(A, K, W, K, Y, ldy, M, N, K, beta != 0.f, stream);
    if (K % 16 == 0)
        return launch_proj(A, AEGIST_BF16, K, W, AEGIST_BF16, nullptr, Y, ldy, M, N, K, beta != 0.f, stream);
    return fail(AEGIST_ERR_SHAPE, "stack: projection K must be a multiple of 16");
}

// Out projection x += A W^T. At decode sizes (M <= 16) it runs as kOutSplits slices of K whose
// partial sums the next layer's ZNorm (or the end of the forward) adds into x in a fixed order:
// the d_model = 2048 rows of W alone give only 64 workgroups, a quarter of the GPU.
constexpr int kOutSplits = 4;
int out_proj(Stack* s, const uint16_t* A, const uint16_t* W, float* x, int M, int N, int K, hipStream_t stream) {
    if (M <= 16 && K % 256 == 0 && K / 256 >= kOutSplits && N % 1024 == 0 && N <= 8192) {
        int rc = launch_proj_splitk(A, K, W, s->part, kOutSplits, M, N, K, stream);
        if (!rc) s->pend = kOutSplits;
        return rc;
    }
    return gemm(s, A, W, x, M, N, K, N, 1.f, stream);
}

// The input projections of one layer (up to four weights sharing A): one grouped launch at
// decode sizes, one GEMM each otherwise.
int gemm_group(Stack* s, const uint16_t* A, int n, const uint16_t* const* W, float* const* Y, const int* N,
               const long long* ldy, int M, int K, hipStream_t stream) {
    if (M <= 64 && K % 16 == 0)
        return launch_proj_multi(A, AEGIST_BF16, K, AEGIST_BF16, n, (const void* const*)W, nullptr, Y, ldy, N, M, K, 0,
                                 stream);
    // up to three weights in one tiled-GEMM launch (stacked along N): the narrow ones (the
    // DeltaNet b / a rows, 32 each) then ride in the last column tile of a wide one instead of
    // taking a whole launch of mostly idle 256-column tiles each
    bool one = n <= 3;
    for (int i = 0; i < n && one; i++) one = gemm_bf16_fits(A, K, W[i], K, M, N[i], K) && (i == n - 1 || N[i] % 8 == 0);
    if (one) {
        const long long ldw[3] = {K, K, K};
        return launch_gemm_bf16_multi(A, K, n, W, ldw, Y, ldy, N, M, K, 0, stream);
    }
    for (int i = 0; i < n; i++) {
        int rc = gemm(s, A, W[i], Y[i], M, N[i], K, (int)ldy[i], 0.f, stream);
        if (rc) return rc;
    }
    return 0;
}

#define RC(x)                  \
    do {                       \
        int _r = (x);          \
        if (_r) return _r;     \
    } while (0)

// AEGIST_GEMM_CONV=0 keeps the short convolution in its own launch (A/B runs, parity tests).
bool conv_gemm_enabled() {
    const char* e = getenv("AEGIST_GEMM_CONV");
    return !(e && e[0] == '0');
}

int delta_layer(Stack* s, const AegistLayerWeights& w, int sl, float* x, int B, int T, hipStream_t st) {
    const AegistStackConfig& c = s->cfg;
    const int rows = B * T, C = s->C(), HV = c.hv, HK = c.hk, dm = c.d_model;
    const size_t mb = (size_t)c.max_batch;
    float* conv = s->conv + (size_t)sl * mb * C * 3;
    float* rec = s->rec + (size_t)sl * mb * HV * D * D;
    // prefill in whole 256-token tiles: the qkv projection's GEMM applies the short convolution
    // and SiLU in its epilogue (the raw projection never reaches HBM; s->proj holds the tiles'
    // edge rows instead)
    const bool conv_fused = T > 1 && conv_gemm_enabled() && gemm_conv_fits(s->hb, dm, w.w_qkv, dm, w.conv_w, B, T, C, dm);
    if (conv_fused) {
        RC(launch_gemm_bf16_conv(s->hb, dm, w.w_qkv, dm, w.conv_w, conv, s->y, C, s->proj, B, T, C, dm, st));
        const uint16_t* W[3] = {w.w_z, w.w_b, w.w_a};
        float* Y[3] = {s->z, s->ba, s->ba + HV};
        const int N[3] = {HV * D, HV, HV};
        const long long ldy[3] = {HV * D, 2 * HV, 2 * HV};
        RC(gemm_group(s, s->hb, 3, W, Y, N, ldy, rows, dm, st));
    } else {
        const uint16_t* W[4] = {w.w_qkv, w.w_z, w.w_b, w.w_a};
        float* Y[4] = {s->proj, s->z, s->ba, s->ba + HV};
        const int N[4] = {C, HV * D, HV, HV};
        const long long ldy[4] = {C, HV * D, 2 * HV, 2 * HV};
        if (rows <= 64) {
            RC(gemm_group(s, s->hb, 4, W, Y, N, ldy, rows, dm, st));
        } else {
            RC(gemm_group(s, s->hb, 1, W, Y, N, ldy, rows, dm, st));
            RC(gemm_group(s, s->hb, 3, W + 1, Y + 1, N + 1, ldy + 1, rows, dm, st));
        }
    }
    const float qscale = 1.f / sqrtf((float)D);
    if (T == 1) {
        // decode: gates + conv-state update + conv + SiLU + L2-norm + delta step + gated norm,
        // one launch (hybrid.py:401-419)
        RC(launch_delta_decode_stack(s->proj, w.conv_w, conv, s->ba, w.a_log, w.dt_bias, s->z, w.gnorm_w, c.eps, rec,
                                     s->ob, B, HK, HV, qscale, 1e-6f, st));
        return out_proj(s, s->ob, w.w_out, x, rows, dm, HV * D, st);
    }
    RC(launch_gates_from_proj(s->ba, w.a_log, w.dt_bias, s->g, s->beta, rows, HV, st));
    {
        // prefill: conv over the chunk, then the fp32 token-by-token scan below 64 tokens (the
        // engine scans every length, hybrid.rs:845-852), the chunked WY form from 64 tokens up
        if (!conv_fused) RC(launch_conv_silu_batched(s->proj, s->y, w.conv_w, conv, B, T, C, st));
        const long long sb = (long long)T * C, so_b = (long long)T * HV * D;
        if (T < 64)
            RC(aegist_delta_recurrent(s->y, s->y + (size_t)HK * D, s->y + (size_t)2 * HK * D, AEGIST_F32, sb, C, D, sb,
                                      C, D, s->g, s->beta, rec, s->o, AEGIST_F32, so_b, (long long)HV * D, D, B, T, HK,
                                      HV, 1, qscale, 1e-6f, st));
        else
            RC(aegist_delta_chunked(s->y, s->y + (size_t)HK * D, s->y + (size_t)2 * HK * D, AEGIST_F32, sb, C, D, sb, C, D,
                                s->g, s->beta, rec, s->o, AEGIST_F32, so_b, (long long)HV * D, D, B, T, HK, HV, 1,
                                qscale, 1e-6f, s->ws, s->ws_bytes, st));
    }
    RC(launch_gated_norm_bf16(s->o, s->z, w.gnorm_w, s->ob, rows * HV, D, c.eps, st));
    return out_proj(s, s->ob, w.w_out, x, rows, dm, HV * D, st);
}

int attn_layer(Stack* s, const AegistLayerWeights& w, int sl, float* x, int B, int T, hipStream_t st) {
    const AegistStackConfig& c = s->cfg;
    const int rows = B * T, H = c.n_heads, KV = c.n_kv, HD = c.head_dim, dm = c.d_model;
    const size_t mb = (size_t)c.max_batch, cap = (size_t)c.max_context;
    uint16_t* kc = s->kc + (size_t)sl * mb * KV * cap * HD;
    uint16_t* vc = s->vc + (size_t)sl * mb * KV * cap * HD;
    float* kp = s->kv2;
    float* vp = s->kv2 + (size_t)c.max_tokens * KV * HD;
    {
        const uint16_t* W[3] = {w.w_q, w.w_k, w.w_v};
        float* Y[3] = {s->proj, kp, vp};
        const int N[3] = {2 * H * HD, KV * HD, KV * HD};
        const long long ldy[3] = {2 * H * HD, KV * HD, KV * HD};
        RC(gemm_group(s, s->hb, 3, W, Y, N, ldy, rows, dm, st));
    }
    if (T == 1 && c.rotary_dim == 64) {
        // decode: ZNorm, RoPE and the cache append inside the split launch
        RC(stack_attn_decode_fused(s->proj, kp, vp, w.q_norm, w.k_norm, kc, vc, s->ob, B, H, KV, s->length, (int)cap,
                                   c.eps, c.rope_theta, s->ws, s->ws_bytes, st));
        return out_proj(s, s->ob, w.w_o, x, rows, dm, H * HD, st);
    }
    RC(launch_attn_prep(s->proj, kp, vp, AEGIST_F32, w.q_norm, w.k_norm, s->y, kc, vc, B, T, H, KV, HD, c.rotary_dim,
                        s->length, (int)cap, c.eps, c.rope_theta, st));
    const float scale = 1.f / sqrtf((float)HD);
    if (T == 1) {
        // the split / merge kernels write the gated output as bf16 (the out projection's input)
        RC(stack_attn_decode(s->y, kc, vc, s->proj, s->ob, B, H, KV, s->length + 1, (int)cap, scale, s->ws,
                             s->ws_bytes, st));
    } else {
        // the attention output goes straight to the out projection's bf16 input when the prefill
        // kernel can write bf16, else through fp32 and a cast
        bool wrote_bf16 = false;
        RC(stack_attn_prefill(s->y, kc, vc, s->proj, s->o, B, H, KV, T, s->length, (int)cap, scale, s->ws,
                              s->ws_bytes, st, s->ob, &wrote_bf16));
        if (!wrote_bf16) RC(launch_cast_bf16(s->o, s->ob, (size_t)rows * H * HD, st));
    }
    return out_proj(s, s->ob, w.w_o, x, rows, dm, H * HD, st);
}

}  // namespace

extern "C" {

int aegist_stack_create(const AegistStackConfig* cfg, void** handle) {
    if (!cfg || !handle) return fail(AEGIST_ERR_SHAPE, "stack_create: null argument");
    const AegistStackConfig& c = *cfg;
    if (c.n_layers <= 0 || c.n_layers > AEGIST_MAX_LAYERS) return fail(AEGIST_ERR_SHAPE, "stack_create: bad n_layers");
    if (c.hk <= 0 || c.hv % c.hk || (c.hv / c.hk != 1 && c.hv / c.hk != 2 && c.hv / c.hk != 4))
        return fail(AEGIST_ERR_SHAPE, "stack_create: need HV / HK in {1, 2, 4}");
    if (c.head_dim != 256 || c.n_kv <= 0 || c.n_heads % c.n_kv || c.n_heads / c.n_kv > 8)
        return fail(AEGIST_ERR_SHAPE, "stack_create: need head_dim 256 and H / KV <= 8");
    if (c.max_batch <= 0 || c.max_tokens < c.max_batch || c.max_context <= 0 || c.d_model <= 0)
        return fail(AEGIST_ERR_SHAPE, "stack_create: bad capacities");
    Stack* s = new Stack();
    s->cfg = c;
    s->w.resize(c.n_layers);
    s->slot.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; l++) s->slot[l] = c.layer_is_attn[l] ? s->n_attn++ : s->n_delta++;
    int rc = check_hip(hipGetDevice(&s->device), "hipGetDevice");
    const size_t rows = c.max_tokens, C = s->C(), mb = c.max_batch;
    const int H = c.n_heads, KV = c.n_kv, HD = c.head_dim, HV = c.hv;
    const size_t wide = std::max<size_t>((size_t)HV * D, (size_t)H * HD);
    auto A = [&](void** p, size_t bytes) {
        if (!rc) rc = alloc(s, p, bytes);
    };
    A((void**)&s->conv, (size_t)std::max(1, s->n_delta) * mb * C * 3 * 4);
    A((void**)&s->rec, (size_t)std::max(1, s->n_delta) * mb * HV * D * D * 4);
    A((void**)&s->kc, (size_t)std::max(1, s->n_attn) * mb * KV * c.max_context * HD * 2);
    A((void**)&s->vc, (size_t)std::max(1, s->n_attn) * mb * KV * c.max_context * HD * 2);
    A((void**)&s->hb, rows * c.d_model * 2);
    A((void**)&s->part, (size_t)kOutSplits * std::min<size_t>(rows, 16) * c.d_model * 4);
    A((void**)&s->proj, rows * std::max<size_t>(C, (size_t)2 * H * HD) * 4);
    A((void**)&s->z, rows * HV * D * 4);
    A((void**)&s->kv2, 2 * rows * KV * HD * 4);
    A((void**)&s->ba, rows * 2 * HV * 4);
    A((void**)&s->g, rows * HV * 4);
    A((void**)&s->beta, rows * HV * 4);
    A((void**)&s->y, rows * std::max<size_t>(C, (size_t)H * HD) * 4);
    A((void**)&s->o, rows * wide * 4);
    A((void**)&s->ob, rows * wide * 2);
    s->ws_bytes = std::max(aegist_delta_chunked_workspace_bytes(c.max_batch, (int)std::min<size_t>(rows, 1 << 30), HV),
                           decode_workspace_bytes(c.max_batch, H, KV, c.max_context, false));
    // the attention prefill's fp16 copy of the cache rows, when it stays within 2 GiB (beyond
    // that the prefill converts its tiles itself)
    if (s->n_attn > 0 && prefill_f16_bytes(c.max_batch, KV, c.max_context) <= ((size_t)2 << 30))
        s->ws_bytes = std::max(s->ws_bytes, prefill_f16_bytes(c.max_batch, KV, c.max_context));
    A(&s->ws, s->ws_bytes);
    for (int i = 0; i < AEGIST_STACK_SNAPSHOTS; i++) {
        A((void**)&s->snap_conv[i], s->conv_bytes());
        A((void**)&s->snap_rec[i], s->rec_bytes());
    }
    if (rc) {
        aegist_stack_destroy(s);
        return rc;
    }
    *handle = s;
    return aegist_stack_reset(s, nullptr);
}

int aegist_stack_destroy(void* handle) {
    Stack* s = (Stack*)handle;
    if (!s) return 0;
    (void)hipDeviceSynchronize();
    for (void* p : s->allocs) (void)hipFree(p);
    delete s;
    return 0;
}

int aegist_stack_set_layer(void* handle, int layer, const AegistLayerWeights* w) {
    Stack* s = (Stack*)handle;
    if (!s || !w || layer < 0 || layer >= s->cfg.n_layers) return fail(AEGIST_ERR_SHAPE, "stack_set_layer: bad layer");
    s->w[layer] = *w;
    return 0;
}

int aegist_stack_reset(void* handle, void* stream) {
    Stack* s = (Stack*)handle;
    if (!s) return fail(AEGIST_ERR_SHAPE, "stack_reset: null handle");
    const AegistStackConfig& c = s->cfg;
    const size_t mb = c.max_batch;
    hipStream_t st = AEG_STREAM(stream);
    (void)c;
    (void)mb;
    AEG_HIP(hipMemsetAsync(s->conv, 0, s->conv_bytes(), st));
    AEG_HIP(hipMemsetAsync(s->rec, 0, s->rec_bytes(), st));
    s->length = 0;
    for (int i = 0; i < AEGIST_STACK_SNAPSHOTS; i++) s->snap_pos[i] = -1;
    return 0;
}

// Lm::snapshot of the engine (hybrid.rs:1060-1070): nothing to do if a snapshot at this length
// exists; else an empty slot, or the oldest snapshot's, takes the conv and recurrent states.
int aegist_stack_snapshot(void* handle, void* stream) {
    Stack* s = (Stack*)handle;
    if (!s) return fail(AEGIST_ERR_SHAPE, "stack_snapshot: null handle");
    int slot = 0;
    for (int i = 0; i < AEGIST_STACK_SNAPSHOTS; i++) {
        if (s->snap_pos[i] == s->length) return 0;
        if (s->snap_pos[i] < s->snap_pos[slot]) slot = i;  // empty (-1) sorts first, then oldest
    }
    hipStream_t st = AEG_STREAM(stream);
    AEG_HIP(hipMemcpyAsync(s->snap_conv[slot], s->conv, s->conv_bytes(), hipMemcpyDeviceToDevice, st));
    AEG_HIP(hipMemcpyAsync(s->snap_rec[slot], s->rec, s->rec_bytes(), hipMemcpyDeviceToDevice, st));
    s->snap_pos[slot] = s->length;
    return 0;
}

// Lm::crop (hybrid.rs:1029-1058): back to the latest snapshot at or before n; later snapshots are
// dropped. Without one the stack starts over from zero. Returns the length kept.
int aegist_stack_crop(void* handle, int n, void* stream) {
    Stack* s = (Stack*)handle;
    if (!s) return fail(AEGIST_ERR_SHAPE, "stack_crop: null handle");
    if (n < 0) return fail(AEGIST_ERR_SHAPE, "stack_crop: negative length");
    if (n >= s->length) return s->length;
    int best = -1;
    for (int i = 0; i < AEGIST_STACK_SNAPSHOTS; i++)
        if (s->snap_pos[i] >= 0 && s->snap_pos[i] <= n && (best < 0 || s->snap_pos[i] > s->snap_pos[best])) best = i;
    if (best < 0) {
        const int rc = aegist_stack_reset(s, stream);
        return rc ? rc : 0;
    }
    hipStream_t st = AEG_STREAM(stream);
    AEG_HIP(hipMemcpyAsync(s->conv, s->snap_conv[best], s->conv_bytes(), hipMemcpyDeviceToDevice, st));
    AEG_HIP(hipMemcpyAsync(s->rec, s->snap_rec[best], s->rec_bytes(), hipMemcpyDeviceToDevice, st));
    s->length = s->snap_pos[best];
    for (int i = 0; i < AEGIST_STACK_SNAPSHOTS; i++)
        if (s->snap_pos[i] > s->length) s->snap_pos[i] = -1;
    return s->length;
}

extern "C++" {
namespace {
// The pieces one sequence's state is made of, layer by layer, in the engine's saved-state order
// (NextEngine::state_pieces, next.rs:2471-2500): an attention layer's first n rows of K then of
// V for each KV head; a recurrent layer's conv state [C][3] then recurrent state [HV][dk][dv].
template <typename F>
void for_each_piece(const Stack* s, int b, int n, F&& f) {
    const AegistStackConfig& c = s->cfg;
    const size_t mb = c.max_batch, cap = c.max_context, HD = c.head_dim, KV = c.n_kv;
    for (int l = 0; l < c.n_layers; l++) {
        const size_t sl = s->slot[l];
        if (c.layer_is_attn[l]) {
            for (size_t h = 0; h < KV; h++) {
                const size_t at = ((sl * mb + b) * KV + h) * cap * HD;
                f((void*)(s->kc + at), (size_t)n * HD * 2);
                f((void*)(s->vc + at), (size_t)n * HD * 2);
            }
        } else {
            f((void*)(s->conv + (sl * mb + b) * s->C() * 3), (size_t)s->C() * 3 * 4);
            f((void*)(s->rec + (sl * mb + b) * c.hv * D * D), (size_t)c.hv * D * D * 4);
        }
    }
}
}  // namespace
}  // extern "C++"

size_t aegist_stack_state_bytes(void* handle, int n) {
    const Stack* s = (const Stack*)handle;
    if (!s || n < 0) return 0;
    size_t total = 0;
    for_each_piece(s, 0, n, [&](void*, size_t bytes) { total += bytes; });
    return total;
}

// Lm::save_state's payload (next.rs:2548-2563) for sequence b at the current length, into a host
// buffer; returns once the copy is complete.
int aegist_stack_save_state(void* handle, int b, void* host, size_t bytes, void* stream) {
    Stack* s = (Stack*)handle;
    if (!s) return fail(AEGIST_ERR_SHAPE, "stack_save_state: null handle");
    if (b < 0 || b >= s->cfg.max_batch) return fail(AEGIST_ERR_SHAPE, "stack_save_state: sequence index out of range");
    if (!host || bytes < aegist_stack_state_bytes(s, s->length))
        return fail(AEGIST_ERR_WORKSPACE, "stack_save_state: host buffer smaller than aegist_stack_state_bytes");
    hipStream_t st = AEG_STREAM(stream);
    unsigned char* dst = (unsigned char*)host;
    int rc = 0;
    for_each_piece(s, b, s->length, [&](void* src, size_t nb) {
        if (!rc && nb) rc = check_hip(hipMemcpyAsync(dst, src, nb, hipMemcpyDeviceToHost, st), "hipMemcpyAsync(save_state)");
        dst += nb;
    });
    if (rc) return rc;
    AEG_HIP(hipStreamSynchronize(st));
    return 0;
}

// Lm::load_state (next.rs:2565-2578, read_state :2502-2538) for sequence b: n tokens' state from a
// host buffer written by aegist_stack_save_state. The stack's length becomes n (all sequences
// share one length), the snapshots are cleared and one is taken at n. On an error the stack is
// left empty (reset). Returns once the copy is complete.
int aegist_stack_load_state(void* handle, int b, int n, const void* host, size_t bytes, void* stream) {
    Stack* s = (Stack*)handle;
    if (!s) return fail(AEGIST_ERR_SHAPE, "stack_load_state: null handle");
    hipStream_t st = AEG_STREAM(stream);
    auto bail = [&](int code, const std::string& msg) {
        (void)aegist_stack_reset(s, stream);
        return fail(code, msg);
    };
    if (b < 0 || b >= s->cfg.max_batch) return bail(AEGIST_ERR_SHAPE, "stack_load_state: sequence index out of range");
    if (n <= 0 || n >= s->cfg.max_context)
        return bail(AEGIST_ERR_SHAPE, "stack_load_state: " + std::to_string(n) + " tokens do not fit a context of " +
                                          std::to_string(s->cfg.max_context));
    if (!host || bytes < aegist_stack_state_bytes(s, n))
        return bail(AEGIST_ERR_WORKSPACE, "stack_load_state: host buffer smaller than aegist_stack_state_bytes");
    const unsigned char* src = (const unsigned char*)host;
    int rc = 0;
    for_each_piece(s, b, n, [&](void* dst, size_t nb) {
        if (!rc && nb) rc = check_hip(hipMemcpyAsync(dst, src, nb, hipMemcpyHostToDevice, st), "hipMemcpyAsync(load_state)");
        src += nb;
    });
    if (rc) return bail(rc, std::string("stack_load_state: ") + aegist_last_error());
    if ((rc = check_hip(hipStreamSynchronize(st), "hipStreamSynchronize"))) return bail(rc, aegist_last_error());
    s->length = n;
    for (int i = 0; i < AEGIST_STACK_SNAPSHOTS; i++) s->snap_pos[i] = -1;
    return aegist_stack_snapshot(s, stream);
}

int aegist_stack_length(void* handle) { return handle ? ((Stack*)handle)->length : -1; }

int aegist_stack_forward(void* handle, float* x, int B, int T, void* stream) {
    Stack* s = (Stack*)handle;
    if (!s) return fail(AEGIST_ERR_SHAPE, "stack_forward: null handle");
    const AegistStackConfig& c = s->cfg;
    if (B <= 0 || T <= 0 || B > c.max_batch || (size_t)B * T > (size_t)c.max_tokens)
        return fail(AEGIST_ERR_SHAPE, "stack_forward: B * T exceeds the stack's max_tokens / max_batch");
    if (s->length + T > c.max_context)
        return fail(AEGIST_ERR_SHAPE, "stack_forward: context of " + std::to_string(s->length + T) +
                                          " tokens exceeds the stack's max_context");
    for (int l = 0; l < c.n_layers; l++)
        if (!s->w[l].norm1) return fail(AEGIST_ERR_SHAPE, "stack_forward: layer " + std::to_string(l) + " has no weights");
    hipStream_t st = AEG_STREAM(stream);
    const int rows = B * T;
    s->pend = 0;
    for (int l = 0; l < c.n_layers; l++) {
        const AegistLayerWeights& w = s->w[l];
        if (s->pend) {
            const int p = s->pend;
            s->pend = 0;
            RC(launch_znorm_bf16_acc(x, s->part, p, w.norm1, s->hb, rows, c.d_model, c.eps, st));
        } else {
            RC(launch_znorm_bf16(x, w.norm1, s->hb, rows, c.d_model, c.eps, st));
        }
        if (c.layer_is_attn[l]) RC(attn_layer(s, w, s->slot[l], x, B, T, st));
        else RC(delta_layer(s, w, s->slot[l], x, B, T, st));
    }
    if (s->pend) {
        const int p = s->pend;
        s->pend = 0;
        RC(launch_znorm_bf16_acc(x, s->part, p, nullptr, nullptr, rows, c.d_model, c.eps, st));
    }
    s->length += T;
    return 0;
}

int aegist_embed_bf16(const uint16_t* table, const int* ids, float* out, int n, int D_, void* stream) {
    if (n < 0 || D_ <= 0) return fail(AEGIST_ERR_SHAPE, "embed: bad shape");
    return launch_embed_bf16(table, ids, out, n, D_, AEG_STREAM(stream));
}

}  // extern "C"
