// One LlamaQ4 step (scripts/llm/llama_q4.py:199-239) as a sequence of gfx950 kernels on one stream.
//
// This is the body of the reference's exported entry points prefill_c{C}_l{L} / decode_l{L} /
// decode_logits_l{L} (scripts/llm/export_llama.py:35-49): tokens, start and last are device buffers
// and every kernel reads them on the device, so one (C, L) step can be captured once into a HIP
// graph and replayed for every call of that entry point. Nothing here allocates or synchronises;
// activations live in the caller's workspace, the KV caches are the caller's and are written in place.
//
// Per layer (x fp32 activations, as the reference):
//   x = rms_norm(h, ln_in); qkv = x W_qkv^T; RoPE(q, k) + fp16 K/V rows at start..start+C-1;
//   o = attention over cache[:L]; h = h + o W_o^T; x = rms_norm(h, ln_post); gu = x W_gu^T;
//   h = h + (silu(gate) * up) W_down^T
// then x = rms_norm(h[last], ln_f), logits = x E^T (tied int4 embedding), next = argmax(logits).
// Projections: C == 1 -> q4_gemv (fp32 in/out, residual fused; norms, RoPE + cache writes and SwiGLU
// fused into the GEMVs); C > 1 -> q4_linear (fused int4 MFMA GEMM with split-fp16 activations and
// per-group fp32 scales, residual fused; its fp16 x planes live in the step workspace and are written
// directly by the norm, attention-merge and SwiGLU kernels that produce them).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdlib>
#include <mutex>

#include "q4_common.h"
#include "q4_internal.h"
#include "q4llm.h"

namespace {

struct Layout {
  size_t h, x, qkv, o, gu, act, xf, logits, attn, amax, lin, part, total;
  size_t attn_bytes, amax_bytes, lin_bytes, part_bytes;
};

size_t up256(size_t b) { return (b + 255) / 256 * 256; }

// Shapes the matrix-core prefill GEMM takes: K % 64 == 0 and group % 32 == 0 (its stages hold 64 k
// and at most two scale groups).
bool linear_fits(int K, int group) { return K % 64 == 0 && group % 32 == 0 && K % group == 0; }

int layout_for(const q4llm_model* m, int C, int L, Layout* lo) {
  const size_t f = sizeof(float);
  const int nq = m->n_heads * m->head_dim, nkv = m->n_kv * m->head_dim;
  size_t attn = 0, amax = 0;
  if (int st = attn_workspace_bytes(C, m->n_heads, m->n_kv, m->head_dim, L, &attn)) return st;
  if (int st = argmax_workspace_bytes(m->vocab, &amax)) return st;
  // the LM head GEMV's per-workgroup argmax partials: at most one per 8 vocabulary rows (its launch
  // entries use 8 or 16 rows per workgroup)
  amax = std::max(amax, static_cast<size_t>((m->vocab + 7) / 8) * sizeof(q4::ArgBest));
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t o = off; off += up256(bytes); return o; };
  lo->h = take(f * C * m->dim);
  lo->x = take(f * C * m->dim);
  lo->qkv = take(f * C * (nq + 2 * nkv));
  lo->o = take(f * C * nq);
  lo->gu = take(f * C * 2 * m->inter);
  lo->act = take(f * C * m->inter);
  lo->xf = take(f * m->dim);
  lo->logits = take(f * m->vocab);
  // K-split partials of the prefill projections (the largest of the four). They share their region with
  // the attention workspace: the qkv partials are added (by RoPE + KV write) before the attention runs,
  // and the o and down partials are written after it and added (by the next rms_norm) before the next.
  size_t part = 0;
  if (C > 1) {
    const int64_t shapes[4][2] = {{nq + 2 * nkv, m->dim}, {m->dim, nq}, {2 * static_cast<int64_t>(m->inter), m->dim},
                                  {m->dim, m->inter}};
    for (const auto& nk : shapes)
      if (linear_fits(static_cast<int>(nk[1]), m->group) && (m->group & (m->group - 1)) == 0)
        part = std::max(part, q4::linear_split_part_bytes(C, nk[0], nk[1], m->group));
  }
  lo->attn = take(std::max(attn, part));
  lo->part = lo->attn;
  lo->part_bytes = part;
  lo->amax = take(amax);
  lo->attn_bytes = attn;
  lo->amax_bytes = amax;
  // prefill projections: the fp16 hi/lo planes of their input (largest K of the four)
  size_t lin = 0;
  if (C > 1) {
    int64_t kmax = 0;
    for (int k : {m->dim, nq, m->inter})
      if (linear_fits(k, m->group) && k > kmax) kmax = k;
    if (kmax > 0)
      if (int st = q4_linear_workspace_bytes(C, kmax, &lin)) return st;
  }
  lo->lin = take(lin);
  lo->lin_bytes = lin;
  lo->total = off;
  return Q4_OK;
}

int check_model(const q4llm_model* m) {
  if (!m || !m->layers || !m->embed_q || !m->embed_s || !m->ln_f || !m->cos_t || !m->sin_t) return Q4_ERR_NULL;
  if (m->dim <= 0 || m->n_layers <= 0 || m->n_heads <= 0 || m->n_kv <= 0 || m->head_dim <= 0 || m->inter <= 0 ||
      m->vocab <= 0 || m->group <= 0 || m->max_ctx <= 0)
    return Q4_ERR_SHAPE;
  if (m->n_heads % m->n_kv) return Q4_ERR_SHAPE;
  for (int i = 0; i < m->n_layers; ++i) {
    const q4llm_layer& l = m->layers[i];
    if (!l.wqkv_q || !l.wqkv_s || !l.wo_q || !l.wo_s || !l.wgu_q || !l.wgu_s || !l.wdown_q || !l.wdown_s ||
        !l.ln_in || !l.ln_post)
      return Q4_ERR_NULL;
  }
  return Q4_OK;
}

// y = residual + x W^T for C rows (C == 1: GEMV, else the fused int4 GEMM with its x planes in ws).
// A prefill projection whose K or group the GEMM does not take (group 8 or 16, K % 64 != 0: legal
// in the reference, llama_q4.py:31) runs one GEMV per row, each with the same fp32 arithmetic.
int proj(int C, const float* x, const int32_t* q, const uint16_t* s, float* y, const float* res, int N, int K, int group,
         void* ws, size_t ws_bytes, void* stream) {
  if (C == 1) return q4_gemv(q, s, x, Q4_F32, y, Q4_F32, res, N, K, group, stream);
  if (linear_fits(K, group)) return q4_linear_ws(x, C, q, s, y, res, N, K, group, ws, ws_bytes, stream);
  for (int r = 0; r < C; ++r) {
    const int64_t xo = static_cast<int64_t>(r) * K, yo = static_cast<int64_t>(r) * N;
    if (int st = q4_gemv(q, s, x + xo, Q4_F32, y + yo, Q4_F32, res ? res + yo : nullptr, N, K, group, stream))
      return st;
  }
  return Q4_OK;
}

// The fused decode GEMVs (qkv and gate/up, K = dim) need the vectorised layout: K % 32 == 0,
// group = 32 * 2^j, K <= 8192 (the largest paired-row entry covers 256 chunks of 32 per row).
bool gemv_fusable(int D, int group) {
  const int gc = group / 32;
  const bool pow2 = group % 32 == 0 && gc > 0 && (gc & (gc - 1)) == 0;
  return pow2 && D % 32 == 0 && D <= 8192;
}

}  // namespace

extern "C" int q4llm_step_workspace_bytes(const q4llm_model* m, int C, int L, size_t* bytes) {
  if (!bytes) return Q4_ERR_NULL;
  if (int st = check_model(m)) return st;
  if (C <= 0 || L <= 0 || L > m->max_ctx || C > m->max_ctx) return Q4_ERR_RANGE;
  Layout lo;
  if (int st = layout_for(m, C, L, &lo)) return st;
  *bytes = lo.total;
  return Q4_OK;
}

namespace {
// One step; with `advance` not null, start[0] += C on the device after the next token is written
// (q4llm_step_feed).
int step_impl(const q4llm_model* m, const int32_t* tokens, int C, const int32_t* start, const int32_t* last,
              void* const* caches, int L, int32_t* next, float* logits, void* workspace, size_t workspace_bytes,
              void* stream, int32_t* advance) {
  if (int st = check_model(m)) return st;
  if (!tokens || !start || !last || !caches || !next || !workspace) return Q4_ERR_NULL;
  if (C <= 0 || L <= 0 || L > m->max_ctx || C > m->max_ctx) return Q4_ERR_RANGE;
  for (int i = 0; i < 2 * m->n_layers; ++i)
    if (!caches[i]) return Q4_ERR_NULL;
  Layout lo;
  if (int st = layout_for(m, C, L, &lo)) return st;
  if (workspace_bytes < lo.total) return Q4_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  float* h = reinterpret_cast<float*>(ws + lo.h);
  float* x = reinterpret_cast<float*>(ws + lo.x);
  float* qkv = reinterpret_cast<float*>(ws + lo.qkv);
  float* o = reinterpret_cast<float*>(ws + lo.o);
  float* gu = reinterpret_cast<float*>(ws + lo.gu);
  float* act = reinterpret_cast<float*>(ws + lo.act);
  float* xf = reinterpret_cast<float*>(ws + lo.xf);
  float* lg = logits ? logits : reinterpret_cast<float*>(ws + lo.logits);
  void* attn_ws = ws + lo.attn;
  void* amax_ws = ws + lo.amax;
  void* lin_ws = ws + lo.lin;
  float* part = lo.part_bytes ? reinterpret_cast<float*>(ws + lo.part) : nullptr;

  const int D = m->dim, hd = m->head_dim, nh = m->n_heads, nkv = m->n_kv;
  const int nq_w = nh * hd, qkv_w = (nh + 2 * nkv) * hd;
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
#define Q4_TRY(expr)            \
  do {                          \
    const int st_ = (expr);     \
    if (st_ != Q4_OK) return st_; \
  } while (0)

  // Decode (C == 1), when the shapes take the vectorised GEMV (true for every BASELINE model), runs
  // five kernels per layer: qkv GEMV with the input norm in its x staging and RoPE + the K/V cache
  // writes in its epilogue; attention; o-projection + residual; gate/up GEMV with the post-attention
  // norm and SwiGLU in its epilogue; down-projection + residual; after the layers the LM head GEMV
  // takes the final norm in its x staging. Prefill uses the separate kernels.
  const bool fused = C == 1 && gemv_fusable(D, m->group);
  // Prefill with a power-of-two group: the norms, the attention merge and SwiGLU write their results
  // straight as the fp16 (hi, lo) planes the following projection reads (in the lin workspace).
  const int kmax = std::max(D, std::max(nq_w, m->inter));
  const bool planes = C > 1 && (m->group & (m->group - 1)) == 0 && linear_fits(D, m->group) &&
                      linear_fits(nq_w, m->group) && linear_fits(m->inter, m->group);
  uint16_t* xh = static_cast<uint16_t*>(lin_ws);
  uint16_t* xl = xh + static_cast<size_t>(C) * kmax;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  // decode GEMVs on the T16 copies where the model has them (Q4_DBG_NO_T16 set: the reference layout)
  const bool use_t16 = fused && !q4::debug_flag(Q4_DBG_NO_T16);
  auto has = [&](const q4llm_t16& t) { return use_t16 && t.tiles && t.scales; };
  // prefill projections on the 64x256 tile read the same T16 copies (fewer cache lines per load)
  auto src = [&](const q4llm_t16& t, int pairing) {
    return q4::T16Src{t.tiles, static_cast<const uint16_t*>(t.scales), pairing, hd};
  };
  Q4_TRY(q4_embed_lookup(m->embed_q, m->embed_s, tokens, h, C, m->vocab, D, m->group, stream));
  // K-split partials left by the last prefill projection for the kernel after it to add (0: none)
  int pending = 0;
  // (Q4_DBG_REDUCE_SPLITS set: every K split is reduced by its projection's own reduce kernel)
  const bool reduce_splits = q4::debug_flag(Q4_DBG_REDUCE_SPLITS);
  const bool defer_norm = planes && q4::rmsnorm_takes_partials(D) && !reduce_splits;
  for (int i = 0; i < m->n_layers; ++i) {
    const q4llm_layer& ly = m->layers[i];
    uint16_t* kc = static_cast<uint16_t*>(caches[2 * i]);
    uint16_t* vc = static_cast<uint16_t*>(caches[2 * i + 1]);
    if (fused) {
      const q4_rope_kv rope{m->cos_t, m->sin_t, kc, vc, start, nh, nkv, hd, m->max_ctx};
      if (has(ly.wqkv_t))
        Q4_TRY(q4_gemv_t16(ly.wqkv_t.tiles, ly.wqkv_t.scales, h, Q4_PRO_RMSNORM, ly.ln_in, m->eps, Q4_EPI_ROPE_KV,
                           &rope, qkv, nullptr, qkv_w, D, m->group, stream));
      else
        Q4_TRY(q4_gemv_epilogue(ly.wqkv_q, ly.wqkv_s, h, Q4_PRO_RMSNORM, ly.ln_in, m->eps, Q4_EPI_ROPE_KV, &rope, qkv,
                                qkv_w, D, m->group, stream));
    } else if (planes) {
      Q4_TRY(q4::rmsnorm_planes(h, ly.ln_in, xh, xl, C, D, m->eps, st, part, pending));
      pending = 0;
      // the qkv partials are added by the RoPE + KV-write kernel
      const bool defer_rope = q4::rope_kv_takes_partials(qkv, m->cos_t, m->sin_t, kc, vc, hd) && !reduce_splits;
      int qkv_split = 0;
      const q4::T16Src qkv_t = src(ly.wqkv_t, Q4_PAIR_ROPE);
      Q4_TRY(q4::q4_linear_planes(xh, xl, C, ly.wqkv_q, ly.wqkv_s, qkv, nullptr, qkv_w, D, m->group, st, part,
                                  lo.part_bytes, defer_rope ? &qkv_split : nullptr, &qkv_t));
      if (qkv_split > 0)
        Q4_TRY(q4::rope_kv_partials(qkv, part, qkv_split, m->cos_t, m->sin_t, kc, vc, C, nh, nkv, hd, m->max_ctx, start,
                                    st));
      else
        Q4_TRY(rope_kv_write(qkv, m->cos_t, m->sin_t, kc, vc, C, nh, nkv, hd, m->max_ctx, start, stream));
    } else {
      Q4_TRY(rmsnorm_f32(h, ly.ln_in, x, C, D, m->eps, nullptr, stream));
      Q4_TRY(proj(C, x, ly.wqkv_q, ly.wqkv_s, qkv, nullptr, qkv_w, D, m->group, lin_ws, lo.lin_bytes, stream));
      Q4_TRY(rope_kv_write(qkv, m->cos_t, m->sin_t, kc, vc, C, nh, nkv, hd, m->max_ctx, start, stream));
    }
    if (planes) {
      Q4_TRY(q4::attn_bucket_planes(qkv, qkv_w, kc, vc, xh, xl, C, nh, nkv, hd, L, start, scale, attn_ws,
                                    lo.attn_bytes, st));
      // the o-projection's partials are added to h by the post-attention norm
      const q4::T16Src wo_t = src(ly.wo_t, Q4_PAIR_NONE);
      Q4_TRY(q4::q4_linear_planes(xh, xl, C, ly.wo_q, ly.wo_s, h, h, D, nq_w, m->group, st, part, lo.part_bytes,
                                  defer_norm ? &pending : nullptr, &wo_t));
    } else {
      Q4_TRY(attn_bucket(qkv, qkv_w, kc, vc, o, C, nh, nkv, hd, L, start, scale, attn_ws, lo.attn_bytes, stream));
      if (has(ly.wo_t))
        Q4_TRY(q4_gemv_t16(ly.wo_t.tiles, ly.wo_t.scales, o, Q4_PRO_NONE, nullptr, 0.0f, 0, nullptr, h, h, D, nq_w,
                           m->group, stream));
      else
        Q4_TRY(proj(C, o, ly.wo_q, ly.wo_s, h, h, D, nq_w, m->group, lin_ws, lo.lin_bytes, stream));
    }
    if (fused) {
      if (has(ly.wgu_t))
        Q4_TRY(q4_gemv_t16(ly.wgu_t.tiles, ly.wgu_t.scales, h, Q4_PRO_RMSNORM, ly.ln_post, m->eps, Q4_EPI_SWIGLU,
                           nullptr, act, nullptr, 2 * m->inter, D, m->group, stream));
      else
        Q4_TRY(q4_gemv_epilogue(ly.wgu_q, ly.wgu_s, h, Q4_PRO_RMSNORM, ly.ln_post, m->eps, Q4_EPI_SWIGLU, nullptr, act,
                                2 * m->inter, D, m->group, stream));
      if (has(ly.wdown_t))
        Q4_TRY(q4_gemv_t16(ly.wdown_t.tiles, ly.wdown_t.scales, act, Q4_PRO_NONE, nullptr, 0.0f, 0, nullptr, h, h, D,
                           m->inter, m->group, stream));
      else
        Q4_TRY(q4_gemv(ly.wdown_q, ly.wdown_s, act, Q4_F32, h, Q4_F32, h, D, m->inter, m->group, stream));
    } else if (planes) {
      Q4_TRY(q4::rmsnorm_planes(h, ly.ln_post, xh, xl, C, D, m->eps, st, part, pending));
      pending = 0;
      // gate/up + SwiGLU in one kernel where the shape takes it (its planes go to the gu buffer, which
      // holds the [C, 2 inter] fp32 otherwise), else the GEMM and silu_mul as two kernels
      uint16_t* ah = reinterpret_cast<uint16_t*>(gu);
      uint16_t* al = ah + static_cast<int64_t>(C) * m->inter;
      const q4::T16Src wgu_t = src(ly.wgu_t, Q4_PAIR_SWIGLU), wdown_t = src(ly.wdown_t, Q4_PAIR_NONE);
      const int fused =
          q4::q4_linear_planes_swiglu(xh, xl, C, ly.wgu_q, ly.wgu_s, ah, al, 2 * m->inter, D, m->group, st, &wgu_t);
      // the down projection's partials are added to h by the next layer's input norm (or the final norm)
      if (fused == Q4_OK) {
        Q4_TRY(q4::q4_linear_planes(ah, al, C, ly.wdown_q, ly.wdown_s, h, h, D, m->inter, m->group, st, part,
                                    lo.part_bytes, defer_norm ? &pending : nullptr, &wdown_t));
      } else {
        if (fused != Q4_ERR_UNSUPPORTED) return fused;
        // a K split of gate/up is added by the silu_mul kernel (Q4_DBG_SWIGLU_UNFUSED set: by its own
        // reduce kernel first); same sums, same order
        int gu_split = 0;
        Q4_TRY(q4::q4_linear_planes(xh, xl, C, ly.wgu_q, ly.wgu_s, gu, nullptr, 2 * m->inter, D, m->group, st, part,
                                    lo.part_bytes, q4::debug_flag(Q4_DBG_SWIGLU_UNFUSED) || reduce_splits ? nullptr : &gu_split,
                                    &wgu_t));
        Q4_TRY(q4::silu_mul_planes(gu, xh, xl, C, m->inter, st, part, gu_split));
        Q4_TRY(q4::q4_linear_planes(xh, xl, C, ly.wdown_q, ly.wdown_s, h, h, D, m->inter, m->group, st, part,
                                    lo.part_bytes, defer_norm ? &pending : nullptr, &wdown_t));
      }
    } else {
      Q4_TRY(rmsnorm_f32(h, ly.ln_post, x, C, D, m->eps, nullptr, stream));
      Q4_TRY(proj(C, x, ly.wgu_q, ly.wgu_s, gu, nullptr, 2 * m->inter, D, m->group, lin_ws, lo.lin_bytes, stream));
      Q4_TRY(silu_mul_f32(gu, act, C, m->inter, stream));
      Q4_TRY(proj(C, act, ly.wdown_q, ly.wdown_s, h, h, D, m->inter, m->group, lin_ws, lo.lin_bytes, stream));
    }
  }
  if (fused && has(m->embed_t)) {
    // one row: the final norm is the LM head's prologue, and its workgroups leave argmax partials of
    // the logits they store, so one more kernel picks the token (and advances the position)
    auto* partials = static_cast<q4::ArgBest*>(amax_ws);
    int n_partials = 0;
    Q4_TRY(q4::gemv_t16_launch(m->embed_t.tiles, m->embed_t.scales, h, Q4_PRO_RMSNORM, m->ln_f, m->eps, 0, nullptr, lg,
                               nullptr, m->vocab, D, m->group, st, partials,
                               static_cast<int>(lo.amax_bytes / sizeof(q4::ArgBest)), &n_partials));
    Q4_TRY(q4::argmax_final_launch(partials, n_partials, next, advance, C, st));
    return Q4_OK;
  }
  if (fused) {  // one row: the final norm is the LM head's prologue
    Q4_TRY(q4_gemv_fused(m->embed_q, m->embed_s, h, Q4_PRO_RMSNORM, m->ln_f, m->eps, lg, nullptr, m->vocab, D,
                         m->group, stream));
  } else if (pending > 0) {
    Q4_TRY(q4::rmsnorm_row_partials(h, m->ln_f, xf, C, D, m->eps, last, part, pending, st));
    Q4_TRY(q4_gemv(m->embed_q, m->embed_s, xf, Q4_F32, lg, Q4_F32, nullptr, m->vocab, D, m->group, stream));
  } else {
    Q4_TRY(rmsnorm_f32(h, m->ln_f, xf, C, D, m->eps, last, stream));
    Q4_TRY(q4_gemv(m->embed_q, m->embed_s, xf, Q4_F32, lg, Q4_F32, nullptr, m->vocab, D, m->group, stream));
  }
  Q4_TRY(argmax_f32(lg, m->vocab, next, amax_ws, lo.amax_bytes, stream));
  if (advance) Q4_TRY(q4llm_advance_position(advance, C, stream));
#undef Q4_TRY
  return Q4_OK;
}
}  // namespace

extern "C" int q4llm_step(const q4llm_model* m, const int32_t* tokens, int C, const int32_t* start, const int32_t* last,
                          void* const* caches, int L, int32_t* next, float* logits, void* workspace,
                          size_t workspace_bytes, void* stream) {
  return step_impl(m, tokens, C, start, last, caches, L, next, logits, workspace, workspace_bytes, stream, nullptr);
}

extern "C" int q4llm_step_feed(const q4llm_model* m, const int32_t* tokens, int C, int32_t* start, const int32_t* last,
                               void* const* caches, int L, int32_t* next, float* logits, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (!start) return Q4_ERR_NULL;
  return step_impl(m, tokens, C, start, last, caches, L, next, logits, workspace, workspace_bytes, stream, start);
}

// ------------------------------------------------------------------------------------------------
// q4llm_step_noalloc: q4llm_step with its workspace in a file-scope device array
// ------------------------------------------------------------------------------------------------

// One array per GPU: each device that loads this library holds its own copy, at its own address,
// until the process ends. In host code `scratch` names a host-side stand-in, never a device address:
// the device address comes from hipGetSymbolAddress, once per device, and only that is used.
__device__ __align__(256) unsigned char scratch[Q4LLM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// The device address of `scratch` on the device that runs `stream`, looked up on first use with
// that device current.
int scratch_address(void* stream, void** out) {
  int dev = 0;
  Q4_CHECK_HIP(hipStreamGetDevice(q4::as_stream(stream), &dev));
  if (dev < 0 || dev >= kMaxDevices) return Q4_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    int cur = 0;
    Q4_CHECK_HIP(hipGetDevice(&cur));
    if (cur != dev) Q4_CHECK_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) Q4_CHECK_HIP(hipSetDevice(cur));
    if (e != hipSuccess) return q4::hip_fail(e);
    if (!p) return Q4_ERR_NULL;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return Q4_OK;
}

}  // namespace

extern "C" int q4llm_step_noalloc(const q4llm_model* m, const int32_t* tokens, int C, const int32_t* start,
                                  const int32_t* last, void* const* caches, int L, int32_t* next, float* logits,
                                  void* stream) {
  // every host-side check of q4llm_step first, and the size limit, before any HIP call
  size_t need = 0;
  if (int st = q4llm_step_workspace_bytes(m, C, L, &need)) return st;
  if (need > Q4LLM_NOALLOC_SCRATCH_BYTES) return Q4_ERR_WORKSPACE;
  if (!tokens || !start || !last || !caches || !next) return Q4_ERR_NULL;
  void* ws = nullptr;
  if (int st = scratch_address(stream, &ws)) return st;
  // No part of the workspace has to start at zero: every kernel of the step writes each scratch
  // value it later reads within the same call.
  return q4llm_step(m, tokens, C, start, last, caches, L, next, logits, ws, Q4LLM_NOALLOC_SCRATCH_BYTES, stream);
}
