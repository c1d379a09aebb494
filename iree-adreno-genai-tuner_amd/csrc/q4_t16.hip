// T16: the device layout of an int4 weight for the matrix-core decode GEMV (q4_gemv_mx.hip).
//
// The reference layout ([N, K/8] int32 words, [N, K/group] fp16 scales; llama_q4.py:25-38) stays
// the interface. A decode GEMV reads a 16-row block 64 bytes (128 k) at a time, so in that layout
// one load instruction touches 16 rows K/2 bytes apart; measured on the MI355X with the kernel's
// own wave shape, the same bytes read ~1 us faster per 3B projection when each 16-row x 64-byte
// segment is one contiguous 1 KB (16384x3072: 6.04 -> 5.06 us, 5120x3072: 3.90 -> 2.98 us,
// 3072x8192: 4.56 -> 3.49 us). T16 stores exactly that:
//   tiles  [n_t16][nseg][16 rows][64 bytes]   nseg = K padded to 4 groups, in 128-k segments
//   scales [n_t16][n_tiles][4 groups][16 rows] fp16, n_tiles = K padded / (4 group)
// with the rows of each 16-row tile in the GEMV's virtual order: rows 16t .. 16t+15 of the weight
// for plain use, or, for the paired epilogues, pairs 8t .. 8t+7 first and their partners after
// (SwiGLU: rows p and p + N/2; RoPE: rows (head, d) and (head, d + hd/2)). Padding (rows past N,
// k past K) is zero. Packing is a pure permutation done once, at load time, on the device.
#include "q4_common.h"
#include "q4_internal.h"

namespace q4 {

bool gemv_mx_takes_t16(int64_t N, int64_t K, int group, bool pair);

namespace {

struct T16Shape {
  int64_t n_t16, nseg, n_tiles;
};

int t16_shape(int64_t N, int64_t K, int group, int pairing, int head_dim, T16Shape* s) {
  if (N <= 0 || K <= 0 || group <= 0 || group % 8 || K % 8 || K % group) return Q4_ERR_SHAPE;
  if (K % 32 || (group != 32 && group != 128)) return Q4_ERR_UNSUPPORTED;  // valid, not taken
  if (pairing != Q4_PAIR_NONE && pairing != Q4_PAIR_SWIGLU && pairing != Q4_PAIR_ROPE) return Q4_ERR_DTYPE;
  if (pairing != Q4_PAIR_NONE && N % 2) return Q4_ERR_SHAPE;
  if (pairing == Q4_PAIR_ROPE) {
    const int hh = head_dim / 2;
    if (head_dim <= 0 || head_dim % 2 || hh % 8 || (hh & (hh - 1)) || N % head_dim) return Q4_ERR_SHAPE;
  }
  if (!gemv_mx_takes_t16(N, K, group, pairing != Q4_PAIR_NONE)) return Q4_ERR_UNSUPPORTED;
  const int64_t tile_k = 4 * group;
  s->n_tiles = (K + tile_k - 1) / tile_k;
  s->nseg = s->n_tiles * tile_k / 128;
  s->n_t16 = pairing == Q4_PAIR_NONE ? (N + 15) / 16 : (N / 2 + 7) / 8;
  if (s->n_t16 * s->nseg * 1024 >= (int64_t{1} << 31)) return Q4_ERR_SHAPE;  // 32-bit buffer offsets
  return Q4_OK;
}

// Weight row held by virtual row vr (-1: padding).
__device__ __forceinline__ int64_t t16_row(int64_t vr, int64_t N, int pairing, int hd) {
  if (pairing == Q4_PAIR_NONE) return vr < N ? vr : -1;
  const int64_t v = vr & 15, p = (vr >> 4) * 8 + (v & 7);
  if (p >= N / 2) return -1;
  if (pairing == Q4_PAIR_SWIGLU) return p + (v >= 8 ? N / 2 : 0);
  const int64_t hh = hd / 2, head = p / hh, d = p - head * hh;
  return head * hd + d + (v >= 8 ? hh : 0);
}

// One thread per 16-byte piece (32 nibbles) of a tile.
__global__ __launch_bounds__(256) void t16_pack_weights(const uint4* __restrict__ qw, uint4* __restrict__ out, int64_t N,
                                                        int64_t K, int pairing, int hd, int64_t nseg, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t tile = i / (nseg * 64), rem = i - tile * (nseg * 64);
  const int64_t seg = rem / 64, piece = rem - seg * 64;
  const int64_t v = piece / 4, b = piece % 4;
  const int64_t row = t16_row(tile * 16 + v, N, pairing, hd);
  const int64_t k0 = seg * 128 + 32 * b;
  out[i] = row >= 0 && k0 < K ? qw[(row * K + k0) / 32] : make_uint4(0, 0, 0, 0);
}

// One thread per fp16 scale slot.
__global__ __launch_bounds__(256) void t16_pack_scales(const uint16_t* __restrict__ sc, uint16_t* __restrict__ out,
                                                       int64_t N, int64_t kg, int pairing, int hd, int64_t n_tiles,
                                                       int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t v = i % 16, q = (i / 16) % 4, T = (i / 64) % n_tiles, tile = i / (64 * n_tiles);
  const int64_t row = t16_row(tile * 16 + v, N, pairing, hd);
  const int64_t g = 4 * T + q;
  out[i] = row >= 0 && g < kg ? sc[row * kg + g] : uint16_t{0};
}

}  // namespace
}  // namespace q4

using namespace q4;

extern "C" int q4_t16_bytes(int64_t N, int64_t K, int group, int pairing, int head_dim, size_t* tile_bytes,
                            size_t* scale_bytes) {
  if (!tile_bytes || !scale_bytes) return Q4_ERR_NULL;
  T16Shape s;
  if (int st = t16_shape(N, K, group, pairing, head_dim, &s)) return st;
  *tile_bytes = static_cast<size_t>(s.n_t16 * s.nseg * 1024);
  *scale_bytes = static_cast<size_t>(s.n_t16 * s.n_tiles * 128);
  return Q4_OK;
}

extern "C" int q4_t16_pack(const int32_t* qweight, const uint16_t* scales, int64_t N, int64_t K, int group, int pairing,
                           int head_dim, void* tiles, void* tile_scales, void* stream) {
  if (!qweight || !scales || !tiles || !tile_scales) return Q4_ERR_NULL;
  T16Shape s;
  if (int st = t16_shape(N, K, group, pairing, head_dim, &s)) return st;
  if (!aligned(qweight, 16) || !aligned(tiles, 16) || !aligned(tile_scales, 8) || !aligned(scales, 2))
    return Q4_ERR_ALIGN;
  const hipStream_t st = as_stream(stream);
  const int64_t nw = s.n_t16 * s.nseg * 64, ns = s.n_t16 * s.n_tiles * 64;
  hipLaunchKernelGGL(t16_pack_weights, dim3(static_cast<unsigned>((nw + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<const uint4*>(qweight), static_cast<uint4*>(tiles), N, K, pairing, head_dim,
                     s.nseg, nw);
  if (int e = launch_status()) return e;
  hipLaunchKernelGGL(t16_pack_scales, dim3(static_cast<unsigned>((ns + 255) / 256)), dim3(256), 0, st, scales,
                     static_cast<uint16_t*>(tile_scales), N, K / group, pairing, head_dim, s.n_tiles, ns);
  return launch_status();
}

extern "C" int q4_gemv_t16(const void* tiles, const void* tile_scales, const float* x, int prologue, const float* aux,
                           float eps, int epilogue, const q4_rope_kv* rope, float* y, const float* residual, int64_t N,
                           int64_t K, int group, void* stream) {
  return q4::gemv_t16_launch(tiles, tile_scales, x, prologue, aux, eps, epilogue, rope, y, residual, N, K, group,
                             q4::as_stream(stream), nullptr, 0, nullptr);
}

int q4::gemv_t16_launch(const void* tiles, const void* tile_scales, const float* x, int prologue, const float* aux,
                        float eps, int epilogue, const q4_rope_kv* rope, float* y, const float* residual, int64_t N,
                        int64_t K, int group, hipStream_t stream, ArgBest* amax, int amax_cap, int* grid) {
  if (!tiles || !tile_scales || !x || !y) return Q4_ERR_NULL;
  if (prologue != Q4_PRO_NONE && prologue != Q4_PRO_RMSNORM) return Q4_ERR_DTYPE;
  if (epilogue != 0 && epilogue != Q4_EPI_SWIGLU && epilogue != Q4_EPI_ROPE_KV) return Q4_ERR_DTYPE;
  if (prologue == Q4_PRO_RMSNORM && !aux) return Q4_ERR_NULL;
  const int pairing = epilogue == Q4_EPI_SWIGLU ? Q4_PAIR_SWIGLU : epilogue == Q4_EPI_ROPE_KV ? Q4_PAIR_ROPE : Q4_PAIR_NONE;
  if (epilogue != 0 && residual) return Q4_ERR_SHAPE;
  const int hd = epilogue == Q4_EPI_ROPE_KV && rope ? rope->head_dim : 0;
  T16Shape s;
  if (epilogue == Q4_EPI_ROPE_KV && !rope) return Q4_ERR_NULL;
  if (int st = t16_shape(N, K, group, pairing, hd, &s)) return st;
  if (!aligned(tiles, 16) || !aligned(tile_scales, 8) || !aligned(x, 16) || (aux && !aligned(aux, 16)) ||
      !aligned(y, 4))
    return Q4_ERR_ALIGN;
  // other workgroups may still be staging x while y is written, so x must not alias y
  if (static_cast<const void*>(x) == static_cast<const void*>(y)) return Q4_ERR_SHAPE;
  GemvEpi ea{};
  if (amax && epilogue != 0) return Q4_ERR_SHAPE;  // argmax partials are for plain rows
  ea.amax = amax;
  ea.amax_cap = amax_cap;
  if (epilogue == Q4_EPI_ROPE_KV) {
    if (!rope->cos_t || !rope->sin_t || !rope->k_cache || !rope->v_cache || !rope->start) return Q4_ERR_NULL;
    if (rope->n_q <= 0 || rope->n_kv <= 0 || rope->max_ctx <= 0) return Q4_ERR_SHAPE;
    if (N != static_cast<int64_t>(rope->n_q + 2 * rope->n_kv) * rope->head_dim) return Q4_ERR_SHAPE;
    ea = GemvEpi{rope->cos_t, rope->sin_t, rope->k_cache, rope->v_cache, rope->start, rope->n_q, rope->n_kv,
                 rope->head_dim, rope->max_ctx, nullptr, 0};
  }
  return gemv_mx_launch(static_cast<const int32_t*>(tiles), static_cast<const uint16_t*>(tile_scales), x, aux, eps, y,
                        residual, N, K, group, prologue, epilogue, &ea, stream, true, grid);
}
