/*
 * aegist_mixer.h — C ABI of the MI355X (gfx950) token-mixer library libaegist_mixer.so.
 *
 * Drop-in for the mixer kernels the Aegist Rust engine launches by name from its PTX module
 * (/root/reference/aegist-fast-35b/aegist_rs/src/hybrid.rs:515-537, launched in
 * HybridEngine::mixer hybrid.rs:787-861 and the identical arms of next.rs:1840-1972 and
 * max.rs:654-728), plus batched entry points for the gated DeltaNet decode step, chunked
 * DeltaNet prefill and split-K GQA decode.
 *
 * Conventions (replacing aegist_rs/src/cuda.rs):
 *  - Every function returns 0 on success, a positive hipError_t value on a runtime error, or
 *    a negative AEGIST_ERR_* code on a rejected argument. aegist_last_error() gives the text
 *    (thread-local). Nothing throws across the ABI.
 *  - All device pointers are caller-owned; no launch path allocates, frees or synchronises
 *    the device. Entry points that need scratch take a caller-provided workspace sized by the
 *    matching *_workspace_bytes query (256-byte aligned). The engine-ABI mirrors whose
 *    reference signature has no workspace argument (aegist_attention_gated, aegist_delta_scan,
 *    aegist_attention_gated_list, aegist_idx_select, aegist_router_topk) have an *_ws variant
 *    taking (ws, ws_bytes) explicitly; the reference-signature form uses the workspace the
 *    calling thread bound on its current device with aegist_bind_workspace (the engine's
 *    preallocated scratch, hybrid.rs:630-650) and fails with AEGIST_ERR_WORKSPACE if none or
 *    too little is bound. A bound workspace is reused by every such call of that thread:
 *    calls on one stream are ordered, calls of one thread on two streams must not overlap.
 *    aegist_stack_create allocates the stack's states and scratch once; aegist_malloc
 *    allocates. Nothing else allocates.
 *  - `stream` is a hipStream_t (NULL = the device's null stream). Every launch is
 *    asynchronous on that stream; no entry point synchronises unless named *_sync. Setting
 *    AEGIST_SYNC_LAUNCH=1 synchronises after each launch and reports errors at the launch.
 *  - Not re-entrant on one stream from several threads (same as the reference).
 *  - Activation dtypes: AEGIST_F32 or AEGIST_BF16 where an argument says so; state and conv
 *    state are always fp32; weights of the engine mirrors are bf16 (uint16_t bits).
 */
#ifndef AEGIST_MIXER_H
#define AEGIST_MIXER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { AEGIST_F32 = 0, AEGIST_BF16 = 1, AEGIST_I8 = 2 /* weights only */ };

enum {
    AEGIST_OK = 0,
    AEGIST_ERR_SHAPE = -1,     /* unsupported shape or argument (message names it) */
    AEGIST_ERR_WORKSPACE = -2, /* workspace missing or too small */
    AEGIST_ERR_DTYPE = -3,     /* dtype code not supported by this entry point */
};

/* ---------------------------------------------------------------------------------------
 * Runtime: device selection, errors, memory (replaces aegist_rs/src/cuda.rs:19-42, 62-86,
 * 194-316: cuInit/context-per-thread, cuMemAlloc/Free, HtoD/DtoH/DtoD copies, memset,
 * cuMemGetInfo).
 * ------------------------------------------------------------------------------------- */
const char* aegist_last_error(void);
const char* aegist_version(void);
int aegist_set_device(int device);
/* Binds caller-owned device memory (256-byte aligned, `bytes` long; NULL unbinds) as the
 * workspace of the reference-signature engine mirrors for the calling thread on its current
 * device. The library never frees it. Replaces the engine's preallocated scratch buffers
 * (hybrid.rs:630-650), which the reference kernels receive as plain pointers. */
int aegist_bind_workspace(void* ws, size_t bytes);
int aegist_malloc(void** ptr, size_t bytes);
int aegist_free(void* ptr);
int aegist_memcpy_htod(void* dst, const void* src, size_t bytes, void* stream);
int aegist_memcpy_dtoh(void* dst, const void* src, size_t bytes, void* stream);
int aegist_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream);
int aegist_memset(void* dst, int value, size_t bytes, void* stream);
int aegist_mem_info(size_t* free_bytes, size_t* total_bytes);
int aegist_stream_sync(void* stream);

/* Synthetic inputs: n values ~ N(mean, std) from a counter-based generator
 * (splitmix64 -> Box-Muller; element i depends only on (seed, i)), written as fp32 or bf16.
 * No reference counterpart: the bench and tests use it to build inputs on the device. */
int aegist_fill_normal(void* dst, size_t n, int dtype, uint64_t seed, float mean, float std, void* stream);

/* ---------------------------------------------------------------------------------------
 * Engine-ABI mirrors: same argument lists as the reference kernels (fp32 activations, bf16
 * weights, batch 1, layouts of hybrid.rs), plus `stream`.
 * ------------------------------------------------------------------------------------- */

/* Zero-centred RMSNorm out = (1 + w) * x / rms(x), `rows` rows of D.
 * Replaces znorm, aegist_rs/kernels/hybrid.cu:69-78 (launched hybrid.rs:737-740). */
int aegist_znorm(const float* x, const uint16_t* w, float* out, int rows, int D, float eps, void* stream);

/* Per (token, head): ZNorm of the query (first HD of each head's 2*HD in qg) and of k,
 * rotate-half RoPE on the first RD dims at position pos0 + t; q -> qn [T,H,HD] fp32;
 * k, v -> bf16 caches [KV,cap,HD] at pos0 + t.
 * Replaces attn_prep, hybrid.cu:86-116 (launched hybrid.rs:800-809). */
int aegist_attn_prep(const float* qg, const float* k, const float* v, const uint16_t* qw, const uint16_t* kw,
                     float* qn, uint16_t* kc, uint16_t* vc, int T, int H, int KV, int HD, int RD, int pos0, int cap,
                     float eps, float theta, void* stream);

/* Causal GQA attention of T queries at positions pos0.. over cache rows [0, pos0+t], then
 * out = attention * sigmoid(gate) with gate = the second HD of each head in qg.
 * HD must be 256. T == 1 runs the split-K decode kernel, T > 1 the MFMA flash kernel.
 * Replaces attention_gated, hybrid.cu:121-173 (launched hybrid.rs:810-818). */
int aegist_attention_gated(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out, int T,
                           int H, int KV, int pos0, int cap, float scale, void* stream);
/* Workspace of attention_gated (non-zero only for T == 1: the split-K partials). */
size_t aegist_attention_gated_workspace_bytes(int T, int H, int KV, int pos0);
/* attention_gated with an explicit workspace. */
int aegist_attention_gated_ws(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out,
                              int T, int H, int KV, int pos0, int cap, float scale, void* ws, size_t ws_bytes,
                              void* stream);

/* beta = sigmoid(h . Wb[j]); g = -exp(A_log[j]) * softplus(h . Wa[j] + dt_bias[j]).
 * gb [T, 2*HV]: g in [0, HV), beta in [HV, 2*HV).
 * Replaces delta_gates, hybrid.cu:179-200 (launched hybrid.rs:827-834). */
int aegist_delta_gates(const float* h, const uint16_t* wb, const uint16_t* wa, const uint16_t* a_log,
                       const uint16_t* dt_bias, float* gb, int T, int D, int HV, void* stream);

/* Depthwise causal conv (kernel 4) over T new rows continuing from state [C,3] (oldest
 * first, updated), then SiLU. x, y [T,C] fp32; w [C,4] bf16 (w[3] hits the newest input).
 * Replaces conv_silu, hybrid.cu:205-221 (launched hybrid.rs:835-839). */
int aegist_conv_silu(const float* x, float* y, const uint16_t* w, float* state, int T, int C, void* stream);

/* In place on y [T,C]: L2-normalise the first 2*nq heads of dk (queries then keys), eps
 * inside the rsqrt of the sum; queries also times qscale.
 * Replaces l2norm_heads, hybrid.cu:225-232 (launched hybrid.rs:840-844). */
int aegist_l2norm_heads(float* y, int T, int C, int nq, int dk, float qscale, float eps, void* stream);

/* Gated delta rule over T tokens: y [T,C] rows q (HK heads) | k (HK heads) | v (HV heads),
 * already L2-normalised; gb [T,2HV] from delta_gates; state [HV,128,128] fp32 (row = key
 * dim), updated; o [T,HV,128] fp32. dk = dv = 128.
 * T == 1: fused decode step; T < 64: recurrent scan; T >= 64: chunked WY prefill (MFMA).
 * Replaces delta_scan, hybrid.cu:240-300 (launched hybrid.rs:845-852). */
int aegist_delta_scan(const float* y, const float* gb, float* state, float* o, int T, int C, int HK, int HV,
                      void* stream);
/* Workspace of delta_scan (non-zero only for T >= 64: the chunked prefill's per-chunk operands). */
size_t aegist_delta_scan_workspace_bytes(int T, int HK, int HV);
/* delta_scan with an explicit workspace. */
int aegist_delta_scan_ws(const float* y, const float* gb, float* state, float* o, int T, int C, int HK, int HV,
                         void* ws, size_t ws_bytes, void* stream);

/* out = w * rmsnorm(o) * silu(z) per value head. o, z, out [T,HV,DV] fp32; w [DV] bf16.
 * Replaces gated_norm, hybrid.cu:303-311 (launched hybrid.rs:853-857). */
int aegist_gated_norm(const float* o, const float* z, const uint16_t* w, float* out, int T, int HV, int DV, float eps,
                      void* stream);

/* ---------------------------------------------------------------------------------------
 * Batched gated DeltaNet (the reference is batch 1 only; these add B and strides).
 * Semantics: aegist/hybrid.py:314-421 (l2norm :314, delta_rule_step :318-324,
 * delta_rule_chunked :327-361, GatedDeltaNet.forward :388-421). dk = dv = 128; HV % HK == 0
 * and HV / HK in {1, 2, 4}.
 * ------------------------------------------------------------------------------------- */

/* One decode token per sequence, fused: conv-state update + depthwise conv (kernel 4) +
 * SiLU + split + L2-norm + q * qscale + gated delta step.
 *   qkv        [B, C] pre-conv projection (qkv_dtype), C = 2*HK*128 + HV*128, rows q|k|v
 *   conv_w     [C, 4] bf16
 *   conv_state [B, C, 3] fp32, oldest first, updated
 *   g, beta    [B, HV] fp32 (log decay, write strength)
 *   state      [B, HV, 128, 128] fp32, updated in place
 *   out        [B, HV, 128] (out_dtype)
 * Replaces the T == 1 path conv_silu -> l2norm_heads -> delta_scan
 * (hybrid.rs:835-852; hybrid.py:393-413). */
int aegist_delta_decode_step(const void* qkv, int qkv_dtype, const uint16_t* conv_w, float* conv_state,
                             const float* g, const float* beta, float* state, void* out, int out_dtype, int B, int HK,
                             int HV, float qscale, float eps, void* stream);

/* Sequence layout shared by the recurrent and chunked entry points. Element strides (not
 * bytes) for batch, token and head; the head dim is contiguous. For the engine's y [T,C]
 * rows: q = y, k = y + HK*128, v = y + 2*HK*128, token stride C, head stride 128.
 * q, k are indexed by QK head (HK of them); v, out by value head; value head h reads QK head
 * h / (HV/HK). g, beta [B, T, HV] fp32 contiguous. If `normalize` is non-zero the kernels
 * L2-normalise q and k (eps) and scale q by qscale (hybrid.py:408-410); otherwise they use
 * q, k as given. */
int aegist_delta_recurrent(const void* q, const void* k, const void* v, int in_dtype, long long sb_qk,
                           long long st_qk, long long sh_qk, long long sb_v, long long st_v, long long sh_v,
                           const float* g, const float* beta, float* state, void* out, int out_dtype,
                           long long sb_o, long long st_o, long long sh_o, int B, int T, int HK, int HV,
                           int normalize, float qscale, float eps, void* stream);

/* Chunked (C = 64) WY-form prefill of the same recurrence, MFMA (fp16 operands after fp32
 * per-row normalisation, fp32 accumulation and state). state may be NULL (zero initial state,
 * final state not returned) or [B,HV,128,128] fp32 in/out. Needs workspace of
 * aegist_delta_chunked_workspace_bytes(B, T, HV) bytes (256-byte aligned). */
size_t aegist_delta_chunked_workspace_bytes(int B, int T, int HV);
int aegist_delta_chunked(const void* q, const void* k, const void* v, int in_dtype, long long sb_qk,
                         long long st_qk, long long sh_qk, long long sb_v, long long st_v, long long sh_v,
                         const float* g, const float* beta, float* state, void* out, int out_dtype, long long sb_o,
                         long long st_o, long long sh_o, int B, int T, int HK, int HV, int normalize, float qscale,
                         float eps, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * Batched gated GQA attention (hybrid.py:265-311). HD = 256, H / KV <= 8, RD even <= HD.
 * ------------------------------------------------------------------------------------- */

/* RoPE inverse-frequency table inv[j] = 1 / theta^(2j/RD), j < RD/2, evaluated in double
 * and rounded once to fp32 (hybrid.py:154 uses an fp32 pow). Every attention entry point
 * uses this table; exported so a CPU checker can use the identical values. */
int aegist_rope_inv_freq(float* inv_out, int RD, float theta);

/* Decode: one query token per sequence at position `pos` (all sequences share the length).
 *   qg     [B, H, 2*HD] (in_dtype): query | gate per head (hybrid.py:285-286)
 *   k_new, v_new [B, KV, HD] (in_dtype): projections of the new token
 *   q_norm_w, k_norm_w [HD] bf16: ZNorm weights (hybrid.py:276-277)
 *   kc, vc [B, KV, cap, HD] bf16 caches; row `pos` is written here
 *   out    [B, H, HD] (out_dtype) = softmax(q K^T / sqrt(HD)) V * sigmoid(gate) over rows
 *          [0, pos]
 * Split-K over the context with a log-sum-exp merge; needs
 * aegist_attention_decode_workspace_bytes(B, H, KV, pos + 1) bytes of workspace. */
size_t aegist_attention_decode_workspace_bytes(int B, int H, int KV, int L);
int aegist_attention_decode(const void* qg, const void* k_new, const void* v_new, int in_dtype,
                            const uint16_t* q_norm_w, const uint16_t* k_norm_w, uint16_t* kc, uint16_t* vc,
                            void* out, int out_dtype, int B, int H, int KV, int HD, int RD, int pos, int cap,
                            float eps, float theta, void* workspace, size_t workspace_bytes, void* stream);

/* aegist_attention_decode without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, serving loops that forbid hipMalloc). No counterpart in the
 * reference. Its scratch is a fixed 32 MiB device array inside the library, one per GPU, held
 * until the process ends; shapes needing more (aegist_attention_decode_workspace_bytes above
 * 32 MiB: a batch of thousands of sequences) fail with AEGIST_ERR_WORKSPACE. Allocates nothing;
 * every scratch byte a call reads it wrote earlier in the same call, so nothing is cleared. All calls on one GPU share the array: calls that overlap
 * on one GPU (two streams, two threads) race and must not be issued. */
int aegist_attention_decode_noalloc(const void* qg, const void* k_new, const void* v_new, int in_dtype,
                                    const uint16_t* q_norm_w, const uint16_t* k_norm_w, uint16_t* kc, uint16_t* vc,
                                    void* out, int out_dtype, int B, int H, int KV, int HDv, int RD, int pos, int cap,
                                    float eps, float theta, void* stream);

/* Attention core only (no prep): q [B, H, T, HD] fp32 already normed and roped, caches
 * [B, KV, cap, HD] bf16 holding rows [0, pos + T), gate [B, T, H*HD] fp32 or NULL (no gate).
 * out [B, T, H, HD] fp32. Causal with offset: query t sees rows [0, pos + t].
 * T == 1 uses split-K (workspace as above with L = pos + 1); T > 1 the flash kernel, whose
 * workspace is optional: with aegist_attention_core_workspace_bytes(B, H, KV, T, pos) bytes
 * (256-byte aligned) the cache rows are converted to fp16 once into it and the kernel loads
 * them straight into LDS; with less (or NULL) each workgroup converts the tiles it stages.
 * Both give the same results (the same fp16 conversion: exact for bf16 values within fp16's
 * range; values beyond +-65504 saturate there, where the reference would keep them). */
size_t aegist_attention_core_workspace_bytes(int B, int H, int KV, int T, int pos);
int aegist_attention_core(const float* q, const uint16_t* kc, const uint16_t* vc, const float* gate, float* out,
                          int B, int H, int KV, int T, int pos, int cap, float scale, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * Hybrid mixer stack: per layer x = x + mixer(znorm(x)) with the MoE FFN as identity
 * (HybridBlock.forward, aegist/hybrid.py:812-843; HybridEngine::forward_chunk / mixer,
 * aegist_rs/src/hybrid.rs:760-861). The stack owns every layer's recurrent state, conv state
 * and bf16 KV cache (HybridCache, hybrid.py:171-260; engine buffers hybrid.rs:607-629); all
 * sequences of a batch share one length. Projections: bf16 operands, fp32 accumulation; up to
 * 64 rows on this library's weight-streaming kernel (aegist_linear), more on its tiled MFMA
 * GEMM; every op runs on this library's kernels. Weights are caller-owned bf16,
 * row-major [out, in] as torch nn.Linear stores them.
 * ------------------------------------------------------------------------------------- */
#define AEGIST_MAX_LAYERS 64

typedef struct AegistStackConfig {
    int n_layers;
    int d_model;
    int hk, hv;                   /* DeltaNet QK / V heads (dk = dv = 128) */
    int n_heads, n_kv, head_dim;  /* attention (head_dim 256) */
    int rotary_dim;
    float rope_theta, eps;        /* eps: ZNorm and GatedNorm */
    int max_batch;                /* sequences per forward call */
    int max_tokens;               /* B * T per forward call */
    int max_context;              /* KV-cache capacity per sequence */
    unsigned char layer_is_attn[AEGIST_MAX_LAYERS];
} AegistStackConfig;

typedef struct AegistLayerWeights {
    const uint16_t* norm1;                        /* [d] ZNorm weight */
    /* gated DeltaNet (hybrid.py:372-384) */
    const uint16_t *w_qkv, *w_z, *w_b, *w_a;      /* [C, d], [HV*128, d], [HV, d], [HV, d] */
    const uint16_t *conv_w, *a_log, *dt_bias;     /* [C, 4], [HV], [HV] */
    const uint16_t *gnorm_w, *w_out;              /* [128], [d, HV*128] */
    /* gated attention (hybrid.py:270-278) */
    const uint16_t *w_q, *w_k, *w_v, *w_o;        /* [2*H*HD, d], [KV*HD, d] x2, [d, H*HD] */
    const uint16_t *q_norm, *k_norm;              /* [HD] ZNorm weights */
} AegistLayerWeights;

int aegist_stack_create(const AegistStackConfig* cfg, void** handle);
int aegist_stack_destroy(void* handle);
int aegist_stack_set_layer(void* handle, int layer, const AegistLayerWeights* weights);
/* length = 0, recurrent and conv states zeroed (HybridCache.reset, hybrid.py:258-263) */
int aegist_stack_reset(void* handle, void* stream);
int aegist_stack_length(void* handle);
/* x [B, T, d] fp32 residual stream, updated in place; T == 1 takes the decode kernels,
 * T > 1 the prefill kernels. Positions continue from aegist_stack_length(). */
int aegist_stack_forward(void* handle, float* x, int B, int T, void* stream);
/* Snapshots (Lm::snapshot / crop, aegist_rs/src/model.rs:368-372; engine hybrid.rs:1029-1070):
 * AEGIST_STACK_SNAPSHOTS slots hold the recurrent layers' conv and recurrent states at a length
 * (the KV cache is append-only, so the length alone rewinds it). snapshot is a no-op when one
 * exists at the current length, else it fills an empty slot or replaces the oldest. crop(n)
 * returns to the latest snapshot at or before n (dropping later ones) and returns the length
 * kept; with none it resets the stack and returns 0; n >= length keeps everything. */
#define AEGIST_STACK_SNAPSHOTS 2
int aegist_stack_snapshot(void* handle, void* stream);
int aegist_stack_crop(void* handle, int n, void* stream);
/* Saved state of one sequence (Lm::save_state / load_state payload, next.rs:2471-2578): per
 * layer in order, an attention layer's first n rows of K then V per KV head (bf16), a recurrent
 * layer's conv state [C][3] then state [HV][128][128] (fp32). state_bytes(n) sizes the buffer
 * for n tokens. save copies sequence b at the current length into host memory; load copies n
 * tokens' state of sequence b back, sets the length to n (shared by all sequences), clears the
 * snapshots and takes one at n; on an error the stack is reset. Both return when done. The file
 * framing (magic, JSON header with the token ids) is the host's (aegist_mixer.state_file). */
size_t aegist_stack_state_bytes(void* handle, int n);
int aegist_stack_save_state(void* handle, int b, void* host, size_t bytes, void* stream);
int aegist_stack_load_state(void* handle, int b, int n, const void* host, size_t bytes, void* stream);
/* out[i, :] = fp32(table[ids[i], :]) for n ids; the engine's embedding lookup
 * (hybrid.rs:743-758) done on the device. */
int aegist_embed_bf16(const uint16_t* table, const int* ids, float* out, int n, int D, void* stream);

/* -------------------------------------------------------------------------------------
 * Second language core: QSA sparse-attention indexer and the gated norm with a choice of gate
 * (QSAIndexer, aegist/hc.py:237-283; NextEngine::mixer, aegist_rs/src/next.rs:1866-1925).
 * Engine layouts, batch 1: qk [T, (H+1)*128] fp32 (H index query heads then one index key);
 * qi [T, H, 128]; kraw [cap, 128] fp32 raw index keys; bk [cap/R, 128] fp32 block keys;
 * sc [T, nbmax]; blist [T, top] int32; nsel [T] int32. The indexer head dim must be 128.
 * ------------------------------------------------------------------------------------- */
/* idx_prep, next.cu:488-503: qi = rope(znorm(q)) at pos0 + t; kraw[pos0 + t] = raw key */
int aegist_idx_prep(const float* qk, const uint16_t* qw, float* qi, float* kraw, int T, int H, int HD, int RD,
                    int pos0, float eps, float theta, void* stream);
/* idx_blocks, next.cu:505-520: bk[b] = rope(znorm(mean of kraw[b R .. b R + R - 1]), b R) for
 * b in [b0, b0 + n) */
int aegist_idx_blocks(const float* kraw, const uint16_t* kw, float* bk, int b0, int n, int R, int HD, int RD,
                      float eps, float theta, void* stream);
/* idx_scores, next.cu:522-541: sc[t, b] = sum_h relu(qi[t, h] . bk[b]) / sqrt(128) for the
 * blocks complete at the query's position (b < (pos0 + t + 1) / R) */
int aegist_idx_scores(const float* qi, const float* bk, float* sc, int T, int H, int HD, int pos0, int R, int nbmax,
                      void* stream);
/* idx_select, next.cu:543-625: per query, all n complete blocks when n <= top (nsel = n), else
 * the top highest scores (ties to the lower block), listed in block order (nsel = top). Scores
 * must be finite and non-negative (idx_scores' relu guarantees it): they are ordered by their
 * bit patterns. Up to 16 queries over more than 8192 blocks stage candidates in the workspace. */
int aegist_idx_select(const float* sc, int* blist, int* nsel, int T, int top, int R, int pos0, int nbmax,
                      void* stream);
size_t aegist_idx_select_workspace_bytes(int T, int top, int R, int pos0);
int aegist_idx_select_ws(const float* sc, int* blist, int* nsel, int T, int top, int R, int pos0, int nbmax, void* ws,
                         size_t ws_bytes, void* stream);
/* attention_gated_list, next.cu:627-705: attention_gated for query t over the R keys of each
 * listed block plus its own incomplete block (positions (pos0 + t + 1) / R * R .. pos0 + t) */
int aegist_attention_gated_list(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out,
                                int T, int H, int KV, int pos0, int cap, float scale, const int* blist,
                                const int* nsel, int top, int R, void* stream);
size_t aegist_attention_gated_list_workspace_bytes(int T, int H, int KV, int pos0, int top, int R);
int aegist_attention_gated_list_ws(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg,
                                   float* out, int T, int H, int KV, int pos0, int cap, float scale, const int* blist,
                                   const int* nsel, int top, int R, void* ws, size_t ws_bytes, void* stream);
/* gated_norm2, next.cu:129-142: out = w * rmsnorm(o) * (sig ? sigmoid(z) : silu(z)) */
int aegist_gated_norm2(const float* o, const float* z, const uint16_t* w, float* out, int T, int HV, int DV, float eps,
                       int sig, void* stream);

/* -------------------------------------------------------------------------------------
 * Projections (QLinear, aegist/model.py:78-93: int8 weight W [N, K] with a per-output-row bf16
 * absmax scale; and plain bf16 weights):  Y[m, n] (+)= scale[n] * sum_k X[m, k] W[n, k],
 * fp32 accumulation; accumulate != 0 adds into Y (the fused residual add). K % 16 == 0 and
 * 16-byte aligned X / W rows. Weight-streaming MFMA kernel: one pass over W for M <= 64.
 * ------------------------------------------------------------------------------------- */
/* gemv_i8, aegist_rs/kernels/aegist.cu:85-91 (launched by HybridEngine::mm, hybrid.rs:717-724) */
int aegist_gemv_i8(const float* x, const int8_t* W, const uint16_t* scale, float* y, int N, int K, int accumulate,
                   void* stream);
/* gemv_bf16, aegist_rs/kernels/aegist.cu:108-124 (the tied output head) */
int aegist_gemv_bf16(const float* x, const uint16_t* W, float* y, int N, int K, void* stream);
/* gemm_i8, aegist_rs/kernels/aegist.cu:126-172 (HybridEngine::mm for t > 1, hybrid.rs:725-734) */
int aegist_gemm_i8(const float* X, const int8_t* W, const uint16_t* scale, float* Y, int M, int N, int K,
                   int accumulate, void* stream);
/* Strided form of the three above: X dtype AEGIST_F32 | AEGIST_BF16 (row stride ldx elements),
 * W dtype AEGIST_I8 | AEGIST_BF16, scale NULL = 1, Y fp32 with row stride ldy. 17..64 rows of
 * bf16 X against one bf16 weight of under 6144 rows (K % 256 == 0, N % 4 == 0, no scale) split
 * K when the calling thread has bound a workspace (aegist_bind_workspace) of at least
 * splits * M * N * 4 bytes (splits <= 256 * 32 / N, at most K / 256): fp32 partials, added in
 * slice order by a second launch (deterministic; the same result to fp32 rounding as the
 * unsplit kernel, which runs otherwise). */
int aegist_linear(const void* X, int x_dtype, long long ldx, const void* W, int w_dtype, const uint16_t* scale,
                  float* Y, long long ldy, int M, int N, int K, int accumulate, void* stream);
/* Grouped form: n (1..4) weight matrices W[i] [N[i], K] of one dtype that share the input X
 * (a layer's input projections, e.g. in_qkv | in_z | in_b | in_a of GatedDeltaNet,
 * hybrid.py:372-384, or q | k | v of GatedAttention, hybrid.py:270-275) in one launch:
 * Y[i][m, n] (+)= scale[i][n] * sum_k X[m, k] W[i][n, k]. W, scale (may be NULL, or hold NULLs),
 * Y, ldy and N are host arrays of n entries. */
int aegist_linear_multi(const void* X, int x_dtype, long long ldx, int w_dtype, int n, const void* const* W,
                        const uint16_t* const* scale, float* const* Y, const long long* ldy, const int* N, int M,
                        int K, int accumulate, void* stream);

/* -------------------------------------------------------------------------------------
 * Mixture of experts: the block after the mixer in every layer (MoE, aegist/hybrid.py:631-652;
 * HybridEngine::moe, aegist_rs/src/hybrid.rs:863-955). h [T, D] fp32 (the norm2 output), x
 * [T, D] fp32 residual. Experts are 4-bit SwiGLU experts of hidden size I in 64-value groups,
 * each one packed row in the layout of expert_layout (aegist/hybrid.py:472-482):
 * [gu_q 2I x D/2 u8 | gu_s 2I x D/64 f16 | gu_m | dn_q D x I/2 | dn_s D x I/64 f16 | dn_m],
 * gate rows first in gu; w = code * scale + min, the even element in the low nibble
 * (q4_dequantize, :463-469). D % 64 == 0, I % 64 == 0, E <= 1024, K <= 16.
 * ------------------------------------------------------------------------------------- */
/* router_topk, hybrid.cu:317-362 (MoE.route, hybrid.py:637-641): logits = h W^T with W bf16
 * [E, D]; p = softmax(logits) in fp32; idx [T, K] = the K largest in descending order (ties to
 * the lower expert); wts [T, K] = p / sum of the picked p. */
int aegist_router_topk(const float* h, const uint16_t* W, int* idx, float* wts, int T, int D, int E, int K,
                       void* stream);
/* Workspace of router_topk (the [T, E] fp32 logits). */
size_t aegist_router_topk_workspace_bytes(int T, int E);
int aegist_router_topk_ws(const float* h, const uint16_t* W, int* idx, float* wts, int T, int D, int E, int K,
                          void* ws, size_t ws_bytes, void* stream);
/* Workspace (device bytes) of aegist_moe_experts for up to T tokens. */
size_t aegist_moe_workspace_bytes(int T, int K, int D, int I, int E);
/* The routed experts (ExpertBank.forward, hybrid.py:608-628) added into the residual:
 * x[t] += sum_k wts[t, k] * W_dn (silu(W_g h[t]) * (W_u h[t])) with the weights of expert
 * idx[t, k], and, when ysh is not NULL, + sigmoid(h[t] . wg) * ysh[t] (the gated shared expert,
 * ysh [T, D] its output, wg bf16 [D]). eptr: device array of E expert-row addresses (any
 * placement: one contiguous [E, row] array, or pooled slots). Replaces the engine's host
 * grouping (hybrid.rs:875-913, here on the device: no host sync) and moe_gu_gemv / gemm,
 * moe_dn_gemv / gemm, moe_reduce (hybrid.cu:386-567). Picks with an expert id outside [0, E)
 * add nothing. */
int aegist_moe_experts(const float* h, const unsigned long long* eptr, const int* idx, const float* wts, float* x,
                       int T, int D, int I, int E, int K, const float* ysh, const uint16_t* wg, void* ws,
                       size_t ws_bytes, void* stream);
/* shared_gate_add, hybrid.cu:569-577: x[t] += sigmoid(h[t] . wg) * y[t] */
int aegist_shared_gate_add(float* x, const float* y, const float* h, const uint16_t* wg, int T, int D, void* stream);
/* silu_mul, aegist.cu:174-178: out = silu(g) * u over n elements (the shared expert's SwiGLU) */
int aegist_silu_mul(const float* g, const float* u, float* out, long long n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AEGIST_MIXER_H */
