// Entry points shared between the library's translation units and not part of the C ABI: the
// prefill step hands activations to its projections as fp16 (hi, lo) planes written by the
// producing kernel (store_x_planes layout), instead of fp32 rows split by a kernel of their own.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>

#include "q4llm.h"

namespace q4 {

// Kernel-choice overrides set through q4_debug_override (q4_status.cpp): Q4_DBG_UNSET when the key
// is not set. The launch paths consult these instead of the process environment.
extern std::atomic<int> g_debug[Q4_DBG_COUNT];
inline int debug_override(int key) { return g_debug[key].load(std::memory_order_relaxed) ^ Q4_DBG_UNSET; }
inline bool debug_set(int key) { return debug_override(key) != Q4_DBG_UNSET; }
// a flag override: set and nonzero
inline bool debug_flag(int key) {
  const int v = debug_override(key);
  return v != Q4_DBG_UNSET && v != 0;
}

// (value, index) of a running argmax: the first index of the maximum, a NaN counting as larger than
// every number (torch.argmax, llama_q4.py:239).
struct ArgBest {
  float v;
  int32_t i;
};

// Arguments of the decode GEMVs' fused epilogues: the RoPE tables, KV caches and position of the
// RoPE + KV-write epilogue, and, for plain rows, an optional buffer of per-workgroup argmax partials
// of the stored rows (one ArgBest per workgroup of the launch; null: none).
struct GemvEpi {
  const float* cos_t;
  const float* sin_t;
  uint16_t* kc;
  uint16_t* vc;
  const int32_t* start;
  int n_q, n_kv, hd, max_ctx;
  ArgBest* amax;
  int amax_cap;  // entries amax holds: a launch needing more workgroups is refused
};

// Matrix-core decode GEMV (q4_gemv_mx.hip); `tiled`: the weights are a T16 copy. Returns
// Q4_ERR_UNSUPPORTED (nothing launched) for shapes it does not take; *grid_out (if not null) receives
// the number of workgroups launched.
int gemv_mx_launch(const int32_t* qweight, const uint16_t* scales, const float* x, const float* aux, float eps, float* y,
                   const float* residual, int64_t N, int64_t K, int group, int prologue, int epilogue,
                   const GemvEpi* ep, hipStream_t stream, bool tiled, int* grid_out = nullptr);

// q4_gemv_t16 with argmax partials of the stored rows written to amax (amax_cap entries; plain rows
// only); *grid receives the number of partials written.
int gemv_t16_launch(const void* tiles, const void* tile_scales, const float* x, int prologue, const float* aux, float eps,
                    int epilogue, const q4_rope_kv* rope, float* y, const float* residual, int64_t N, int64_t K, int group,
                    hipStream_t stream, ArgBest* amax, int amax_cap, int* grid);

// The final pass of argmax_f32 over n partials: out[0] = the best index; with `advance` not null,
// advance[0] += delta afterwards in the same kernel.
int argmax_final_launch(const ArgBest* partials, int n, int32_t* out, int32_t* advance, int delta, hipStream_t st);

// K split of a prefill projection: n_split workgroups per output tile, nk_split 64-k stages each.
struct LinearSplit {
  int n_split, nk_split;
};
LinearSplit linear_split_plan(int64_t M, int64_t N, int64_t K, int group);
// bytes of K-split partials q4_linear_planes uses for this shape (0: it takes no K split)
size_t linear_split_part_bytes(int64_t M, int64_t N, int64_t K, int group);

// q4_linear_ws's GEMM on given planes (power-of-two group); with `part` (at least
// linear_split_part_bytes, 16-byte aligned) it may split K and reduce the partials in a second kernel.
// With `deferred` not null, a K split leaves its partials in `part` unreduced and sets *deferred to the
// number of splits (0 when the result went to y); the caller's next kernel then completes y.
// The decode T16 copy of the same weight (q4_t16_pack: tiles, scales, and the pairing and head size it
// was packed with), which the 64x256 tile reads instead of qw / sc when it takes the projection: its
// 1 KB loads then touch 16 cache lines instead of 32.
struct T16Src {
  const void* tiles;
  const uint16_t* scales;
  int pairing, head_dim;
};
int q4_linear_planes(const uint16_t* xh, const uint16_t* xl, int64_t M, const int32_t* qw, const uint16_t* sc,
                     float* y, const float* res, int64_t N, int64_t K, int group, hipStream_t st,
                     float* part = nullptr, size_t part_bytes = 0, int* deferred = nullptr,
                     const T16Src* t16 = nullptr);
// The gate/up projection with silu(gate) * up written as the [M, N / 2] planes oh / ol (ol = oh + M N / 2)
// of the down projection; Q4_ERR_UNSUPPORTED when the shape does not take the fused tile (the caller then
// runs q4_linear_planes + silu_mul_planes).
int q4_linear_planes_swiglu(const uint16_t* xh, const uint16_t* xl, int64_t M, const int32_t* qw, const uint16_t* sc,
                            uint16_t* oh, uint16_t* ol, int64_t N, int64_t K, int group, hipStream_t st,
                            const T16Src* t16 = nullptr);
// rmsnorm_f32 of M rows (no row selection), written as planes. With n_split > 0 each row of x is first
// completed with the K-split partials `part` of the projection that produced it (x += sum of n_split
// [M, D] planes, written back to x); requires rmsnorm_takes_partials(D).
bool rmsnorm_takes_partials(int64_t D);
int rmsnorm_planes(float* x, const float* w, uint16_t* xh, uint16_t* xl, int64_t M, int64_t D, float eps,
                   hipStream_t st, const float* part = nullptr, int n_split = 0);
// rmsnorm_f32 of the selected row row[0] after completing it with the K-split partials (as above).
int rmsnorm_row_partials(float* x, const float* w, float* out, int64_t M, int64_t D, float eps, const int32_t* row,
                         const float* part, int n_split, hipStream_t st);
// rope_kv_write with the qkv rows summed from the K-split partials of the qkv projection.
bool rope_kv_takes_partials(const float* qkv, const float* cos_t, const float* sin_t, const uint16_t* kc,
                            const uint16_t* vc, int hd);
int rope_kv_partials(float* qkv, const float* part, int n_split, const float* cos_t, const float* sin_t, uint16_t* kc,
                     uint16_t* vc, int C, int n_q, int n_kv, int hd, int max_ctx, const int32_t* start, hipStream_t st);
// silu_mul_f32, written as planes. With n_split > 0 gu is not read: gate and up are the sums of the
// n_split K-split partials `part` ([M, 2 inter] fp32 each) of the gate/up projection, added in the
// order of linear_reduce_kernel.
int silu_mul_planes(const float* gu, uint16_t* xh, uint16_t* xl, int64_t M, int64_t inter, hipStream_t st,
                    const float* part = nullptr, int n_split = 0);
// attn_bucket for C > 1, its output written as planes.
int attn_bucket_planes(const float* q, int q_row_stride, const uint16_t* k_cache, const uint16_t* v_cache,
                       uint16_t* xh, uint16_t* xl, int C, int n_q, int n_kv, int hd, int L, const int32_t* start,
                       float scale, void* workspace, size_t workspace_bytes, hipStream_t stream);

}  // namespace q4
