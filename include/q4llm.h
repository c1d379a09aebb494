/*
 * q4llm.h -- C ABI of the MI355X (gfx950) int4 LLM hot path.
 *
 * Every entry point:
 *   - takes plain device pointers and sizes (no framework types), owned by the caller;
 *   - validates all arguments on the host first and returns a negative Q4_ERR_* code without
 *     touching the device when they are wrong;
 *   - is stream ordered and asynchronous: it enqueues kernels on `stream` (a hipStream_t, NULL =
 *     the default stream) and never synchronises the host;
 *   - allocates no device memory; scratch space is passed in as `workspace`.
 *
 * Data formats follow the reference LlamaQ4 module (scripts/llm/llama_q4.py):
 *   qweight [N, K/8] int32: nibble b (bits 4b..4b+3) of word w holds k = 8w + b, stored as q + 8
 *                           in [0, 15] (llama_q4.py:25-38);
 *   scales  [N, K/group] fp16 (bit patterns passed as uint16_t);
 *   KV caches [max_ctx, n_kv, head_dim] fp16, position-first, written in place (llama_q4.py:222-223).
 *
 * dtype codes: Q4_F32 = 0, Q4_F16 = 1.
 */
#ifndef Q4LLM_H
#define Q4LLM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  Q4_OK = 0,
  Q4_ERR_NULL = -1,       /* a required pointer is NULL */
  Q4_ERR_SHAPE = -2,      /* sizes violate the documented divisibility / range rules */
  Q4_ERR_ALIGN = -3,      /* a pointer is not aligned as documented */
  Q4_ERR_DTYPE = -4,      /* unknown or unsupported dtype code */
  Q4_ERR_WORKSPACE = -5,  /* workspace missing or smaller than the *_workspace_bytes query */
  Q4_ERR_RANGE = -6,      /* a position / bucket / length is out of range */
  Q4_ERR_UNSUPPORTED = -7,/* valid request this build does not implement (documented limit) */
  Q4_ERR_HIP = -100       /* a HIP runtime call failed; q4llm_last_hip_error() has the code */
};

enum { Q4_F32 = 0, Q4_F16 = 1 };

/* prologue codes of q4_gemv_fused / q4_gemv_epilogue */
enum { Q4_PRO_NONE = 0, Q4_PRO_RMSNORM = 1, Q4_PRO_SWIGLU = 2 };

/* epilogue codes of q4_gemv_epilogue */
enum { Q4_EPI_SWIGLU = 1, Q4_EPI_ROPE_KV = 2 };

/* Human-readable text for a status code (static storage). */
const char* q4llm_status_string(int status);
/* The hipError_t of the last failed HIP call made by this library on this thread (0 if none). */
int q4llm_last_hip_error(void);
/* ABI version of this header: bumped when a signature changes. */
int q4llm_abi_version(void);

/* Kernel-choice overrides, for tests and tuning sweeps only; no counterpart in the reference
 * (whose kernels come from IREE's compiler). With no override set, every entry point picks its
 * kernels by its fixed shape rule, and nothing in the library reads the process environment.
 * An override takes effect for calls made after it returns (a HIP graph keeps the kernels it was
 * captured with). The store is process-wide: callers that change it while another thread launches
 * get either choice for that launch. */
enum {
  Q4_DBG_ATTN_S = 0,              /* decode attention keys per split: 32, 64 or 128 */
  Q4_DBG_ATTN_PS = 1,             /* prefill attention keys per split: a multiple of 32, <= 512 */
  Q4_DBG_ATTN_GENERIC = 2,        /* nonzero: every attention call on the generic split kernel */
  Q4_DBG_ATTN_COMBINE_WG = 3,     /* nonzero: prefill attention merges with the workgroup combine */
  Q4_DBG_GEMM_TILE = 4,           /* gemm_f16_nt tile entry (q4_config_info "gemm" index) */
  Q4_DBG_GEMM_SPLIT = 5,          /* gemm_f16_nt_ws K split count */
  Q4_DBG_GEMV_CFG = 6,            /* q4_gemv VALU entry */
  Q4_DBG_MX_CFG = 7,              /* matrix-core GEMV entry */
  Q4_DBG_GEMV_NO_MX = 8,          /* nonzero: fp32-x GEMVs on the reference layout stay on the VALU kernel */
  Q4_DBG_MX_GRID = 9,             /* workgroup cap of the grid-stride matrix-core GEMV entries */
  Q4_DBG_PREFILL_REF_LAYOUT = 10, /* nonzero: prefill projections read the reference layout, not T16 */
  Q4_DBG_LINEAR_TILE = 11,        /* q4_linear_ws tile entry (then no K split and no fused SwiGLU) */
  Q4_DBG_SWIGLU_UNFUSED = 12,     /* nonzero: prefill gate/up GEMM and SwiGLU as separate kernels */
  Q4_DBG_NO_T16 = 13,             /* nonzero: q4llm_step's decode GEMVs read the reference layout */
  Q4_DBG_REDUCE_SPLITS = 14,      /* nonzero: q4llm_step's K-split prefill projections add their partials
                                     with the reduce kernel instead of leaving them to the next kernel */
  Q4_DBG_COUNT = 15
};
#define Q4_DBG_UNSET (-2147483647 - 1)
/* Sets override `key` to `value` (Q4_DBG_UNSET clears it). Q4_ERR_RANGE for an unknown key. */
int q4_debug_override(int key, int value);
/* The current value of override `key` (Q4_DBG_UNSET when not set) in *value. */
int q4_debug_override_get(int key, int* value);
/* Clears every override. */
void q4_debug_clear(void);

/* ---------------------------------------------------------------------------------------------
 * int4 weight format (reference: scripts/llm/llama_q4.py)
 * ------------------------------------------------------------------------------------------- */

/* Replaces quantize_q4 (llama_q4.py:25-38). w [N, K] fp32 row-major -> qweight [N, K/8] int32 and
 * scales [N, K/group] fp16. scale = max(amax|w_g|, 1e-8) / 7 in fp32, q = round-half-even(w / scale)
 * clamped to [-8, 7], stored as q + 8; the scale is cast to fp16 after q is computed.
 * Requires K % 8 == 0, K % group == 0, group % 8 == 0. Bit-exact with the reference. */
int q4_quantize(const float* w, int32_t* qweight, uint16_t* scales, int64_t N, int64_t K,
                int group, void* stream);

/* Replaces unpack_q4 (llama_q4.py:41-45): nibbles [N, K] uint8 in [0, 15]. K % 8 == 0. */
int q4_unpack(const int32_t* qweight, uint8_t* nibbles, int64_t N, int64_t K, void* stream);

/* Replaces dequantize_q4 (llama_q4.py:48-51): w [N, K] = (nibble - 8) * fp32(scale) written as
 * w_dtype (Q4_F32 is exact; Q4_F16 rounds to nearest even). */
int q4_dequant(const int32_t* qweight, const uint16_t* scales, void* w, int w_dtype, int64_t N,
               int64_t K, int group, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Projections (reference: QLinear.forward / _gemv_fused, llama_q4.py:69-90)
 * ------------------------------------------------------------------------------------------- */

/* Decode GEMV, replaces QLinear._gemv_fused (llama_q4.py:74-90) and QLinear.forward at M == 1
 * (llama_q4.py:69-72): y[n] = residual[n] + sum_k x[k] * (nib[n,k] - 8) * scale[n, k/group].
 * x: K elements of x_dtype; y: N elements of y_dtype; residual: NULL or N fp32 (only with
 * y_dtype == Q4_F32; may alias y). Accumulation is fp32.
 * Requires K % 8 == 0, K % group == 0, group % 8 == 0, K < 2^28, 4-byte aligned qweight/x and
 * 2-byte aligned y. Shapes with K % 32 == 0, group = 32 * 2^j, K <= 16384 and 16-byte aligned
 * qweight/x take the staged kernels; the rest take a one-wave-per-row generic kernel. */
int q4_gemv(const int32_t* qweight, const uint16_t* scales, const void* x, int x_dtype, void* y,
            int y_dtype, const float* residual, int64_t N, int64_t K, int group, void* stream);

/* Decode GEMV with the preceding element-wise step fused into its x staging (fp32 x and y):
 *   Q4_PRO_RMSNORM: x' = rms_norm(x, aux, eps) over K, aux = norm weight [K] (the input /
 *                   post-attention norms before QLinear, llama_q4.py:141-142, 215-216, 234-235);
 *   Q4_PRO_SWIGLU:  x holds 2K values (gate | up) and x' = silu(gate) * up (llama_q4.py:236).
 * then y = residual + W x' exactly as q4_gemv. Needs the vectorised GEMV layout (K % 32 == 0,
 * group = 32 * 2^j, K <= 8192), otherwise Q4_ERR_UNSUPPORTED. x must not alias y.
 * The rms_norm form stages x * aux and scales each finished row by r = 1 / sqrt(mean(x^2) + eps):
 * W ((x * r) * aux) up to fp32 rounding. */
int q4_gemv_fused(const int32_t* qweight, const uint16_t* scales, const float* x, int prologue,
                  const float* aux, float eps, float* y, const float* residual, int64_t N, int64_t K,
                  int group, void* stream);

/* RoPE tables and KV caches of the Q4_EPI_ROPE_KV epilogue: cos_t / sin_t [max_ctx, head_dim]
 * fp32 (llama_q4.py:184-192), k_cache / v_cache fp16 [max_ctx, n_kv, head_dim], start: device
 * int32 [1] holding the position of the token. */
typedef struct q4_rope_kv {
  const float* cos_t;
  const float* sin_t;
  uint16_t* k_cache;
  uint16_t* v_cache;
  const int32_t* start;
  int n_q, n_kv, head_dim, max_ctx;
} q4_rope_kv;

/* Decode GEMV whose rows are finished in pairs by the step that follows the projection in
 * LlamaQ4.step (fp32 x and y, optional Q4_PRO_RMSNORM prologue as in q4_gemv_fused):
 *   Q4_EPI_SWIGLU:  W is the fused [gate | up] weight (N = 2 * inter); y[i] = silu(g_i) * u_i
 *                   with g = W[:inter] x', u = W[inter:] x' (llama_q4.py:236); y has inter values.
 *   Q4_EPI_ROPE_KV: W is the fused [q | k | v] weight (N = (n_q + 2 n_kv) * head_dim); y = qkv
 *                   with q and k rotated at pos = start[0] (llama_q4.py:205-207, 218-221), and the
 *                   k and v rows written as fp16 to k_cache / v_cache at row pos (llama_q4.py:
 *                   222-223). pos outside [0, max_ctx) leaves y unrotated and the caches untouched.
 * Replaces the q4_gemv + silu_mul_f32 and q4_gemv + rope_kv_write pairs of one decode token.
 * Same layout requirements as q4_gemv_fused; N even. x must not alias y. */
int q4_gemv_epilogue(const int32_t* qweight, const uint16_t* scales, const float* x, int prologue,
                     const float* aux, float eps, int epilogue, const q4_rope_kv* rope, float* y, int64_t N,
                     int64_t K, int group, void* stream);

/* ---------------------------------------------------------------------------------------------
 * T16: the decode GEMV's device copy of an int4 weight (no counterpart in the reference, whose
 * [N, K/8] layout stays the interface; built once from it at load time)
 * ------------------------------------------------------------------------------------------- */

/* Row pairing of a T16 copy: which rows share a 16-row tile, matching the GEMV epilogue it feeds. */
enum { Q4_PAIR_NONE = 0, Q4_PAIR_SWIGLU = 1, Q4_PAIR_ROPE = 2 };

/* Bytes of the T16 copy of an [N, K] weight with `group` (32 or 128) and `pairing` (Q4_PAIR_ROPE
 * takes head_dim; the others ignore it): tiles [ceil(rows/16)][K padded to 4 groups / 128][16][64 B]
 * and scales [ceil(rows/16)][tiles of 4 groups][4][16] fp16. Q4_ERR_UNSUPPORTED when the decode
 * GEMV does not take the shape (the caller keeps the reference layout for it). */
int q4_t16_bytes(int64_t N, int64_t K, int group, int pairing, int head_dim, size_t* tile_bytes,
                 size_t* scale_bytes);

/* Writes the T16 copy of (qweight [N, K/8] int32, scales [N, K/group] fp16): each 16-row tile holds
 * its rows' 128-k segments as contiguous 1 KB blocks, in the row order of the GEMV's 16-row blocks
 * (Q4_PAIR_SWIGLU: pairs p with rows p and p + N/2; Q4_PAIR_ROPE: rows (head, d) and
 * (head, d + head_dim/2) of the fused qkv weight); padding is zero. A permutation of the bytes. */
int q4_t16_pack(const int32_t* qweight, const uint16_t* scales, int64_t N, int64_t K, int group,
                int pairing, int head_dim, void* tiles, void* tile_scales, void* stream);

/* Decode GEMV on a T16 copy, fp32 x and y: the same results as q4_gemv / q4_gemv_fused /
 * q4_gemv_epilogue on the reference layout (QLinear._gemv_fused, llama_q4.py:74-90) with prologue
 * Q4_PRO_NONE or Q4_PRO_RMSNORM and epilogue 0 (plain, optional fp32 residual), Q4_EPI_SWIGLU or
 * Q4_EPI_ROPE_KV (rope required), the copy packed with the matching pairing. x must not alias y. */
int q4_gemv_t16(const void* tiles, const void* tile_scales, const float* x, int prologue,
                const float* aux, float eps, int epilogue, const q4_rope_kv* rope, float* y,
                const float* residual, int64_t N, int64_t K, int group, void* stream);

/* Prefill projection, replaces QLinear.forward at M > 1 (llama_q4.py:72,
 * F.linear(x, dequantize_q4(W))): y[M, N] = residual + x[M, K] @ dequant(W)^T, x and y fp32.
 * Runs on the fp16 matrix cores with x split into two fp16 terms and the int4 values exact in
 * fp16, the group scale applied in fp32 per K-group, so the result carries fp32-level accuracy.
 * Requires K % 64 == 0, group % 32 == 0, K % group == 0, |x| < 65504. residual: NULL or [M, N] fp32
 * (may alias y). */
int q4_linear(const float* x, int64_t M, const int32_t* qweight, const uint16_t* scales, float* y,
              const float* residual, int64_t N, int64_t K, int group, void* stream);

/* Workspace bytes q4_linear_ws needs for M rows of K: the fp16 hi and lo planes of x (4 * M * K). */
int q4_linear_workspace_bytes(int64_t M, int64_t K, size_t* bytes);

/* Workspace bytes with which q4_linear_ws also splits the reduction over K for this shape (a chunk of
 * M <= 256 rows whose output tiles alone would leave compute units idle): the planes, rounded up to
 * 256 bytes, plus n_split * M * N fp32 partials; equal to q4_linear_workspace_bytes(M, K) where no
 * split applies. */
int q4_linear_ws_split_bytes(int64_t M, int64_t N, int64_t K, int group, size_t* bytes);

/* q4_linear (QLinear.forward at M > 1, llama_q4.py:72) with a caller workspace: x is split once into
 * fp16 hi/lo planes in `workspace`, then a multi-stage matrix-core pipeline streams both planes and
 * the packed int4 weights (two launches on `stream`). Same contract and accuracy as q4_linear;
 * workspace >= q4_linear_workspace_bytes(M, K), 16-byte aligned. With workspace_bytes >=
 * q4_linear_ws_split_bytes(M, N, K, group) the GEMM may split K over several workgroups per output
 * tile and add their partials (in a fixed order) and the residual in a third launch. */
int q4_linear_ws(const float* x, int64_t M, const int32_t* qweight, const uint16_t* scales, float* y,
                 const float* residual, int64_t N, int64_t K, int group, void* workspace,
                 size_t workspace_bytes, void* stream);

/* fp16 GEMM C[M,N] = A[M,K] @ B[N,K]^T ("NT", gemm/shapes.py:4-6, S2 prefill_nt), fp32
 * accumulation, fp16 output, row-major with leading dimensions lda/ldb/ldc (in elements).
 * M == 1 runs a memory-bound fp16 GEMV. Requires K % 8 == 0, lda/ldb % 8 == 0, 16-byte aligned
 * A and B. */
int gemm_f16_nt(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t M, int64_t N, int64_t K,
                int64_t lda, int64_t ldb, int64_t ldc, void* stream);

/* Bytes of device workspace gemm_f16_nt_ws needs for an M x N x K problem (0: it does not split K
 * for this shape). */
int gemm_f16_nt_ws_bytes(int64_t M, int64_t N, int64_t K, size_t* bytes);
/* gemm_f16_nt with a caller-provided device workspace (16-byte aligned, at least
 * gemm_f16_nt_ws_bytes bytes; it may be NULL when that query gives 0): for shapes whose output tiles
 * alone leave CUs idle, K is split over several workgroups per tile, each writing an fp32 partial
 * into the workspace, and a second launch adds the partials in a fixed order and writes C, so the
 * result does not depend on timing. Same argument rules and result tolerance as gemm_f16_nt;
 * Q4_ERR_WORKSPACE when the workspace is missing or too small. Replaces the same call of the
 * reference's harness (gemm/harness/vk_gemm_bench.c dispatch of one NT problem) where the caller
 * can hold a workspace. */
int gemm_f16_nt_ws(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t M, int64_t N, int64_t K,
                   int64_t lda, int64_t ldb, int64_t ldc, void* workspace, size_t workspace_bytes,
                   void* stream);

/* ---------------------------------------------------------------------------------------------
 * Attention over a KV bucket (reference: LlamaQ4.step, llama_q4.py:204-232)
 * ------------------------------------------------------------------------------------------- */

/* Bytes of workspace attn_bucket needs for C query rows, n_q heads, head_dim hd, bucket L. */
int attn_workspace_bytes(int C, int n_q, int n_kv, int hd, int L, size_t* bytes);

/* GQA attention of C query rows at positions start[0] + c over k_cache/v_cache[:L]
 * (llama_q4.py:224-232): s = q . k * scale, keys with key_pos > pos masked (the reference's -1e30
 * fill), softmax in fp32, o = p . v. q: C rows of n_q * hd fp32 (RoPE applied) q_row_stride
 * floats apart (n_q * hd when packed; the row pitch of a fused qkv buffer otherwise), caches
 * [>= L, n_kv, hd] fp16, out [C, n_q * hd] fp32. `start` is a device int32 (read by the kernels, so
 * the launch can be replayed from a graph). Split-K over the bucket length with a log-sum-exp
 * combine. Requires n_q % n_kv == 0, hd in {64, 128}; keys at or beyond L are never read, so a
 * position >= L attends to the whole bucket. */
int attn_bucket(const float* q, int q_row_stride, const uint16_t* k_cache, const uint16_t* v_cache,
                float* out, int C, int n_q, int n_kv, int hd, int L, const int32_t* start, float scale,
                void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Element-wise / gather ops of LlamaQ4.step (llama_q4.py:141-142, 194-239)
 * ------------------------------------------------------------------------------------------- */

/* rms_norm (llama_q4.py:141-142): out[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * w, rows of D fp32.
 * `row` NULL: all M rows; else the single row row[0] (device int32, clamped to [0, M)) of x -> out[0]. */
int rmsnorm_f32(const float* x, const float* w, float* out, int64_t M, int64_t D, float eps,
                const int32_t* row, void* stream);

/* RoPE + in-place KV write (llama_q4.py:205-207, 218-223): for c < C, pos = start[0] + c:
 * q = q*cos[pos] + rotate_half(q)*sin[pos] (in place in qkv), k likewise, then
 * k_cache[pos] = fp16(k), v_cache[pos] = fp16(v). qkv [C, (n_q + 2 n_kv) * hd] fp32,
 * cos/sin [max_ctx, hd] fp32. Positions >= max_ctx are skipped (the host checks ranges). */
int rope_kv_write(float* qkv, const float* cos_t, const float* sin_t, uint16_t* k_cache,
                  uint16_t* v_cache, int C, int n_q, int n_kv, int hd, int max_ctx,
                  const int32_t* start, void* stream);

/* SwiGLU (llama_q4.py:236): out[m, i] = silu(gu[m, i]) * gu[m, inter + i], gu [M, 2*inter]. */
int silu_mul_f32(const float* gu, float* out, int64_t M, int64_t inter, void* stream);

/* QEmbedding.lookup (llama_q4.py:106-119): out[c] = dequant(row tokens[c]) fp32, tokens device
 * int32 [C]; tokens outside [0, vocab) give a zero row (the reference's `valid` mask). */
int q4_embed_lookup(const int32_t* qweight, const uint16_t* scales, const int32_t* tokens, float* out,
                    int C, int64_t vocab, int64_t D, int group, void* stream);

/* torch.argmax(logits, -1) (llama_q4.py:239): first index of the maximum of V fp32 values,
 * written as int32 to out[0]. workspace >= argmax_workspace_bytes(V). */
int argmax_workspace_bytes(int64_t V, size_t* bytes);
int argmax_f32(const float* logits, int64_t V, int32_t* out, void* workspace, size_t workspace_bytes,
               void* stream);

/* ---------------------------------------------------------------------------------------------
 * Whole-model step (the exported entry points prefill_c{C}_l{L} / decode_l{L} /
 * decode_logits_l{L}, scripts/llm/export_llama.py:1-10,35-49; LlamaQ4.step llama_q4.py:199-239)
 * ------------------------------------------------------------------------------------------- */

/* Optional T16 copies (q4_t16_pack) of a weight for the decode GEMVs, also read by the prefill
 * GEMM's 64x256 tile: tiles and tile scales, both NULL when absent (decode and prefill then read
 * the reference layout). wqkv takes Q4_PAIR_ROPE pairing, wgu Q4_PAIR_SWIGLU, wo, wdown and the
 * LM head Q4_PAIR_NONE. */
typedef struct q4llm_t16 {
  const void* tiles;
  const void* scales;
} q4llm_t16;

typedef struct q4llm_layer {
  const int32_t* wqkv_q;  const uint16_t* wqkv_s;   /* [(n_q + 2 n_kv) hd, dim] */
  const int32_t* wo_q;    const uint16_t* wo_s;     /* [dim, n_q hd] */
  const int32_t* wgu_q;   const uint16_t* wgu_s;    /* [2 inter, dim] (gate rows then up rows) */
  const int32_t* wdown_q; const uint16_t* wdown_s;  /* [dim, inter] */
  const float* ln_in;     const float* ln_post;     /* [dim] */
  q4llm_t16 wqkv_t, wo_t, wgu_t, wdown_t;           /* optional decode copies */
} q4llm_layer;

typedef struct q4llm_model {
  int dim, n_layers, n_heads, n_kv, head_dim, inter, vocab, group, max_ctx;
  float eps;
  const int32_t* embed_q; const uint16_t* embed_s;  /* tied embedding / LM head [vocab, dim] */
  const float* ln_f;                                 /* [dim] */
  const float* cos_t; const float* sin_t;            /* RoPE tables [max_ctx, head_dim] */
  const q4llm_layer* layers;                         /* host array of n_layers */
  q4llm_t16 embed_t;                                 /* optional decode copy of the LM head */
} q4llm_model;

/* Workspace bytes for one step with C tokens and bucket L. */
int q4llm_step_workspace_bytes(const q4llm_model* m, int C, int L, size_t* bytes);

/* One LlamaQ4.step: tokens [C] int32, start [1], last [1] (device), caches = 2 * n_layers device
 * pointers (k0, v0, k1, v1, ...) each [max_ctx, n_kv, head_dim] fp16 written in place at
 * start..start+C-1; attention reads cache[:L]. Writes the greedy next token (int32) to next[0]
 * and, if logits != NULL, the [vocab] fp32 logits of row `last`. The host checks C, L against
 * max_ctx; start + C <= L is the caller's schedule contract (llm_runner.c:143-149). The tokens are
 * read by the step's first kernel and next is written by its last, so for C == 1 `tokens` may be
 * `next` itself (a decode loop that feeds each token back on the device). */
int q4llm_step(const q4llm_model* m, const int32_t* tokens, int C, const int32_t* start,
               const int32_t* last, void* const* caches, int L, int32_t* next, float* logits,
               void* workspace, size_t workspace_bytes, void* stream);

/* Size of the per-GPU scratch array of q4llm_step_noalloc: 64 MiB. That covers every decode step
 * (C == 1; the Llama-3.2-3B shape needs 1.15 MiB) and prefill chunks up to that size (3B shape:
 * C = 256 at L <= 512 needs 61.6 MiB; q4llm_step_workspace_bytes gives the figure for a shape). */
#define Q4LLM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* q4llm_step without a workspace argument and without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The step's scratch is a file-scope device
 * array of Q4LLM_NOALLOC_SCRATCH_BYTES, one per GPU, held until the process ends; its device
 * address is looked up with hipGetSymbolAddress on the first call on each device (make that first
 * call outside graph capture). Same arguments, kernels and results as q4llm_step; returns
 * Q4_ERR_WORKSPACE when q4llm_step_workspace_bytes(m, C, L) exceeds Q4LLM_NOALLOC_SCRATCH_BYTES.
 * Every call on one GPU shares that GPU's array (the last call's contents stay in it; nothing in it
 * needs to start at zero): calls that overlap on one GPU, from two streams or two threads, race. */
int q4llm_step_noalloc(const q4llm_model* m, const int32_t* tokens, int C, const int32_t* start,
                       const int32_t* last, void* const* caches, int L, int32_t* next, float* logits,
                       void* stream);

/* q4llm_step, then start[0] += C on the device, done by the step's last kernel: the decode loop's
 * position step (pos += 1, runner/llm_runner.c:233-245) without a kernel of its own. With
 * tokens == next, a graph of one q4llm_step_feed call replays consecutive decode steps with no
 * host input between them. */
int q4llm_step_feed(const q4llm_model* m, const int32_t* tokens, int C, int32_t* start,
                    const int32_t* last, void* const* caches, int L, int32_t* next, float* logits,
                    void* workspace, size_t workspace_bytes, void* stream);

/* start[0] += delta on the device, stream ordered: the decode loop's position step (pos += 1,
 * runner/llm_runner.c:233-245) for a loop that feeds the next token and position back on the
 * device; one kernel, so it can be captured with q4llm_step into one graph. */
int q4llm_advance_position(int32_t* start, int delta, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Measurement and tuning hooks (counterparts of gemm/roofline.py:27-70 and of the tuner's
 * candidate timing, scripts/tune/kernel_tuner.py:144-227; not part of the model path)
 * ------------------------------------------------------------------------------------------- */

/* Streaming read of `bytes` (multiple of 16): workgroups of 256 threads, each thread issuing
 * loads_per_thread (1, 2, 4 or 8) 16-byte loads up front. sink: one float, never written in practice. */
int q4_probe_read(const void* buf, int64_t bytes, float* sink, int loads_per_thread, void* stream);
/* Empty kernel launch (launch-floor probe). */
int q4_probe_empty(int grid, int block, void* stream);
/* One wave that sleeps on the device for about `microseconds` (0 .. 1 s; bounded by the constant-rate
 * real-time counter and by a sleep count): lets a benchmark queue a timed region on `stream` before
 * the device reaches it, so host latency stays out of the region (the harness's warm-up spacing,
 * gemm/harness/vk_gemm_bench.c:426-448). */
int q4_probe_wait(int64_t microseconds, void* stream);
/* Number of entries in the explicit GEMV / GEMM tile lists, and the same entry points with a
 * forced entry (cfg < 0: automatic) and, for the GEMV, a grid (0: automatic; grid-stride entries
 * only). gemm_f16_nt_cfg's `split` is reserved and must be 0. */
int q4_gemv_num_configs(void);
int q4_gemv_cfg(const int32_t* qweight, const uint16_t* scales, const void* x, int x_dtype, void* y,
                int y_dtype, const float* residual, int64_t N, int64_t K, int group, int cfg, int grid,
                void* stream);
int gemm_f16_num_configs(void);
/* Number of q4_linear_ws tile entries (the Q4_DBG_LINEAR_TILE override selects one for sweeps and tests). */
int q4_linear_ws_num_configs(void);
int gemm_f16_nt_cfg(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t M, int64_t N, int64_t K,
                    int64_t lda, int64_t ldb, int64_t ldc, int cfg, int split, void* stream);
/* The entries of the explicit tile lists, for host-side checks of their index mapping (each call
 * fills `info` and returns Q4_ERR_RANGE past the last entry):
 *   q4_gemv_config_info:    lanes per row, chunks per lane, rows per lane, waves, x words, grid-stride
 *   q4_gemv_mx_config_info: row blocks per workgroup, waves per row block, tiles per wave, used rows
 *                           per 16-row block, grid-stride (q4_gemv_mx_num_configs entries)
 *   gemm_f16_config_info:   BM, BN, wave rows, wave columns, stages, BK, pipelined substeps
 *   q4_linear_ws_config_info: BM, BN, wave rows, wave columns, stages, k-split, pipelined (0/1) */
int q4_gemv_config_info(int cfg, int* info);
int q4_gemv_mx_num_configs(void);
int q4_gemv_mx_config_info(int cfg, int* info);
int gemm_f16_config_info(int cfg, int* info);
int q4_linear_ws_config_info(int cfg, int* info);

#ifdef __cplusplus
}
#endif
#endif /* Q4LLM_H */
