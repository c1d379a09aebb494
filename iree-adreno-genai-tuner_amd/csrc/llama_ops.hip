// Element-wise, normalisation and selection kernels of LlamaQ4.step
// (scripts/llm/llama_q4.py:141-142, 194-239).
//
// Floating-point contraction is disabled in this file so that each multiply and add rounds like
// the reference's separate tensor ops (x * cos + rotate_half(x) * sin, x * r * w, ...); with the
// same operation order the element-wise results are bit-identical to the CPU ops, and only the
// reductions (sum of squares, exp) differ in the last bits.
#include "q4_common.h"
#include "q4_internal.h"

#include <cmath>

#pragma clang fp contract(off)

namespace q4 {
namespace {

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
// 16 bytes at byte offset off of the buffer; out of range (e.g. 0x80000000): zeros, no memory access.
// The whole vector is bit-cast: bit-casting single elements of the loaded vector compiled to four
// copies of element 0 with this compiler.
__device__ __forceinline__ float4 load_f4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const f32x4 f = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  return make_float4(f.x, f.y, f.z, f.w);
}

// rms_norm: one workgroup (TH threads) per row. x*x is rounded before the sum (x.pow(2)), the
// mean is sum / D, r = 1 / sqrt(mean + eps) (both correctly rounded), out = (x * r) * w. Rows of at
// most 4096 values (D % 4 == 0) are held in registers, loaded with all 16-byte loads in flight; the
// norm weights are loaded with them, so no memory round trip follows the row reduction.
// With xh != nullptr the row goes to the fp16 (hi, lo) planes of a prefill projection instead of out.
// With n_split > 0 (rows held in registers only) x is first completed with the K-split partials of the
// projection that produced it, x += psum[0] + ... + psum[n_split - 1] (each [M, D]; the order of
// linear_reduce_kernel, so the same bits), and the completed row is written back to x. The first PB
// partials load with the row, the rest one round trip each (PB 12 for more than 6 partials: the 128-row
// prefill chunks have 8 and 10; 6 otherwise, where the 12-wide form measured 1.3% slower prefill).
// TH is 256, or 1024 for the prefill planes; each thread holds 1024 / TH float4s of the row.
template <int PB = 6, int TH = 256>
__global__ __launch_bounds__(TH) void rmsnorm_kernel(const float* x, const float* __restrict__ w,
                                                      float* __restrict__ out, int64_t M, int64_t D, float eps,
                                                      const int32_t* __restrict__ row_sel,
                                                      uint16_t* __restrict__ xh, uint16_t* __restrict__ xl,
                                                      const float* __restrict__ psum = nullptr, int n_split = 0) {
  // a selected row outside [0, M) is clamped (the reference's index_select would raise)
  const int64_t row = row_sel ? min(max(static_cast<int64_t>(row_sel[0]), int64_t{0}), M - 1) : blockIdx.x;
  const float* xr = x + row * D;
  float* orow = out + static_cast<int64_t>(blockIdx.x) * D;
  static_assert(TH == 256 || TH == 1024, "threads per row");
  constexpr int kV = 1024 / TH;
  constexpr int kW = TH / 64;  // waves
  const bool vec = D % 4 == 0 && D <= 4 * TH * kV;
  float4 v[kV], wv[kV];
  float s = 0.0f;
  if (vec) {
    // Buffer loads: float4s past the row come back as zeros without a branch, so every load of the
    // row, its norm weights and (n_split > 0) its K-split partials is in flight before the first use.
    const __amdgpu_buffer_rsrc_t xres = row_rsrc(xr, static_cast<uint32_t>(D) * 4u);
    const __amdgpu_buffer_rsrc_t wres = row_rsrc(w, static_cast<uint32_t>(D) * 4u);
#pragma unroll
    for (int i = 0; i < kV; ++i) v[i] = load_f4(xres, (threadIdx.x + i * TH) * 16u);
#pragma unroll
    for (int i = 0; i < kV; ++i) wv[i] = load_f4(wres, (threadIdx.x + i * TH) * 16u);
    if (n_split > 0) {
      // partial sp of this row: psum[sp][row][:]; the first kPb splits load with the row, the sums run
      // in ascending split order, as in linear_reduce_kernel
      constexpr int kPb = PB;
      const uint32_t row_bytes = static_cast<uint32_t>(D) * 4u;
      const uint32_t plane_bytes = static_cast<uint32_t>(M * D) * 4u;
      const __amdgpu_buffer_rsrc_t pres = row_rsrc(psum, plane_bytes * static_cast<uint32_t>(n_split));
      const uint32_t prow = static_cast<uint32_t>(row) * row_bytes;
      float4 pb[kV][kPb];
#pragma unroll
      for (int sp = 0; sp < kPb; ++sp)
#pragma unroll
        for (int i = 0; i < kV; ++i)
          pb[i][sp] = load_f4(pres, sp < n_split && (threadIdx.x + i * TH) * 16u < row_bytes
                                        ? sp * plane_bytes + prow + (threadIdx.x + i * TH) * 16u
                                        : 0x80000000u);
#pragma unroll
      for (int i = 0; i < kV; ++i) {
        const int64_t j = threadIdx.x + i * TH;
        float4 a = pb[i][0];
#pragma unroll
        for (int sp = 1; sp < kPb; ++sp)
          if (sp < n_split) {
            a.x += pb[i][sp].x;
            a.y += pb[i][sp].y;
            a.z += pb[i][sp].z;
            a.w += pb[i][sp].w;
          }
        for (int sp = kPb; sp < n_split; ++sp) {
          const float4 c = load_f4(pres, j * 16 < row_bytes ? sp * plane_bytes + prow + j * 16u : 0x80000000u);
          a.x += c.x;
          a.y += c.y;
          a.z += c.z;
          a.w += c.w;
        }
        v[i] = make_float4(v[i].x + a.x, v[i].y + a.y, v[i].z + a.z, v[i].w + a.w);
        if (j < D / 4) reinterpret_cast<float4*>(const_cast<float*>(xr))[j] = v[i];
      }
    }
#pragma unroll
    for (int i = 0; i < kV; ++i) {
      const float a = v[i].x * v[i].x, b = v[i].y * v[i].y, c = v[i].z * v[i].z, d = v[i].w * v[i].w;
      s += (a + b) + (c + d);
    }
  } else {
    for (int64_t i = threadIdx.x; i < D; i += TH) {
      const float t = xr[i];
      const float sq = t * t;
      s += sq;
    }
  }
  s = group_sum<64>(s);
  __shared__ float part[kW];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  // wave sums added as a pairwise tree in wave order
  float t4[kW];
#pragma unroll
  for (int q = 0; q < kW; ++q) t4[q] = part[q];
#pragma unroll
  for (int w2 = kW / 2; w2 >= 1; w2 /= 2)
#pragma unroll
    for (int q = 0; q < w2; ++q) t4[q] = t4[2 * q] + t4[2 * q + 1];
  const float total = t4[0];
  const float mean = total / static_cast<float>(D);
  const float r = 1.0f / sqrtf(mean + eps);
  if (vec) {
#pragma unroll
    for (int i = 0; i < kV; ++i) {
      const int64_t j = threadIdx.x + i * TH;
      if (j < D / 4) {
        const float4 ww = wv[i];
        const float4 y =
            make_float4((v[i].x * r) * ww.x, (v[i].y * r) * ww.y, (v[i].z * r) * ww.z, (v[i].w * r) * ww.w);
        if (xh) {
          // lanes 2l and 2l + 1 hold float4s j and j + 1 (j even for lane 2l): lane 2l stores the chunk
          const float nx = __shfl_xor(y.x, 1, 64), ny = __shfl_xor(y.y, 1, 64);
          const float nz = __shfl_xor(y.z, 1, 64), nw = __shfl_xor(y.w, 1, 64);
          if ((j & 1) == 0) {
            const float e8[8] = {y.x, y.y, y.z, y.w, nx, ny, nz, nw};
            store_x_planes8(xh, xl, (static_cast<int64_t>(blockIdx.x) * D + 4 * j) / 8, e8);
          }
        } else {
          reinterpret_cast<float4*>(orow)[j] = y;
        }
      }
    }
  } else {
    for (int64_t i = threadIdx.x; i < D; i += TH) {
      const float t = xr[i] * r;
      const float y = t * w[i];
      if (xh) store_x_planes(xh, xl, static_cast<int64_t>(blockIdx.x) * D + i, y);
      else orow[i] = y;
    }
  }
}

// RoPE on q and k of qkv rows (in place) and the fp16 KV row writes, one thread per (row, head,
// d < hd/2) pair; rotate_half(x) = cat(-x[hd/2:], x[:hd/2]) (llama_q4.py:194-197).
__global__ __launch_bounds__(256) void rope_kv_kernel(float* __restrict__ qkv, const float* __restrict__ cos_t,
                                                      const float* __restrict__ sin_t, uint16_t* __restrict__ kc,
                                                      uint16_t* __restrict__ vc, int C, int n_q, int n_kv, int hd,
                                                      int max_ctx, const int32_t* __restrict__ start_p) {
  const int half = hd / 2;
  const int heads = n_q + 2 * n_kv;
  const int64_t total = static_cast<int64_t>(C) * heads * half;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= total) return;
  const int d = static_cast<int>(t % half);
  const int head = static_cast<int>((t / half) % heads);
  const int c = static_cast<int>(t / (static_cast<int64_t>(half) * heads));
  const int pos = start_p[0] + c;
  if (pos < 0 || pos >= max_ctx) return;
  float* row = qkv + (static_cast<int64_t>(c) * heads + head) * hd;
  const float x1 = row[d], x2 = row[d + half];
  if (head < n_q + n_kv) {  // q or k: rotate
    const float* cp = cos_t + static_cast<int64_t>(pos) * hd;
    const float* sp = sin_t + static_cast<int64_t>(pos) * hd;
    const float a = x1 * cp[d];
    const float b = (-x2) * sp[d];
    const float lo = a + b;
    const float e = x2 * cp[d + half];
    const float f = x1 * sp[d + half];
    const float hi = e + f;
    if (head < n_q) {
      row[d] = lo;
      row[d + half] = hi;
    } else {
      row[d] = lo;
      row[d + half] = hi;
      uint16_t* dst = kc + (static_cast<int64_t>(pos) * n_kv + (head - n_q)) * hd;
      dst[d] = float_to_half_bits(lo);
      dst[d + half] = float_to_half_bits(hi);
    }
  } else {  // v: copy into the cache
    uint16_t* dst = vc + (static_cast<int64_t>(pos) * n_kv + (head - n_q - n_kv)) * hd;
    dst[d] = float_to_half_bits(x1);
    dst[d + half] = float_to_half_bits(x2);
  }
}

// The same for hd % 8 == 0 with four consecutive d per thread: 16-byte loads of the row halves and
// the cos / sin entries, 16-byte row stores, 8-byte cache stores; the row loads are issued before
// the position is known. Same expressions, so the same bits as rope_kv_kernel.
// With n_split > 0 the rows are not read from qkv but summed from the K-split partials of the qkv
// projection (part[s], each [C, (n_q + 2 n_kv) hd], in the order of linear_reduce_kernel); the rotated q
// and k are written to qkv as usual (v only to the cache).
__global__ __launch_bounds__(256) void rope_kv4_kernel(float* __restrict__ qkv, const float* __restrict__ cos_t,
                                                       const float* __restrict__ sin_t, uint16_t* __restrict__ kc,
                                                       uint16_t* __restrict__ vc, int C, int n_q, int n_kv, int hd,
                                                       int max_ctx, const int32_t* __restrict__ start_p,
                                                       const float* __restrict__ part = nullptr, int n_split = 0) {
  const int half = hd / 2, q4 = half / 4;
  const int heads = n_q + 2 * n_kv;
  const int64_t total = static_cast<int64_t>(C) * heads * q4;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= total) return;
  const int d = static_cast<int>(t % q4) * 4;
  const int head = static_cast<int>((t / q4) % heads);
  const int c = static_cast<int>(t / (static_cast<int64_t>(q4) * heads));
  float* row = qkv + (static_cast<int64_t>(c) * heads + head) * hd;
  float4 x1, x2;
  if (n_split > 0) {
    const int64_t plane4 = static_cast<int64_t>(C) * heads * hd / 4;  // hd % 4 == 0
    const float* pr = part + (row - qkv);
    x1 = sum_partials4(reinterpret_cast<const float4*>(pr + d), plane4, n_split);
    x2 = sum_partials4(reinterpret_cast<const float4*>(pr + d + half), plane4, n_split);
  } else {
    x1 = *reinterpret_cast<const float4*>(row + d);
    x2 = *reinterpret_cast<const float4*>(row + d + half);
  }
  const int pos = start_p[0] + c;
  if (pos < 0 || pos >= max_ctx) return;
  auto half4 = [](float a, float b, float c4, float e) {
    return make_uint2(static_cast<uint32_t>(float_to_half_bits(a)) | (static_cast<uint32_t>(float_to_half_bits(b)) << 16),
                      static_cast<uint32_t>(float_to_half_bits(c4)) | (static_cast<uint32_t>(float_to_half_bits(e)) << 16));
  };
  if (head < n_q + n_kv) {  // q or k: rotate
    const float* cp = cos_t + static_cast<int64_t>(pos) * hd;
    const float* sp = sin_t + static_cast<int64_t>(pos) * hd;
    const float4 c1 = *reinterpret_cast<const float4*>(cp + d), s1 = *reinterpret_cast<const float4*>(sp + d);
    const float4 c2 = *reinterpret_cast<const float4*>(cp + d + half);
    const float4 s2 = *reinterpret_cast<const float4*>(sp + d + half);
    auto rot_lo = [](float a1, float a2, float cc, float ss) {
      const float a = a1 * cc;
      const float b = (-a2) * ss;
      return a + b;
    };
    auto rot_hi = [](float a1, float a2, float cc, float ss) {
      const float e = a2 * cc;
      const float f = a1 * ss;
      return e + f;
    };
    const float4 lo = make_float4(rot_lo(x1.x, x2.x, c1.x, s1.x), rot_lo(x1.y, x2.y, c1.y, s1.y),
                                  rot_lo(x1.z, x2.z, c1.z, s1.z), rot_lo(x1.w, x2.w, c1.w, s1.w));
    const float4 hi = make_float4(rot_hi(x1.x, x2.x, c2.x, s2.x), rot_hi(x1.y, x2.y, c2.y, s2.y),
                                  rot_hi(x1.z, x2.z, c2.z, s2.z), rot_hi(x1.w, x2.w, c2.w, s2.w));
    *reinterpret_cast<float4*>(row + d) = lo;
    *reinterpret_cast<float4*>(row + d + half) = hi;
    if (head >= n_q) {
      uint16_t* dst = kc + (static_cast<int64_t>(pos) * n_kv + (head - n_q)) * hd;
      *reinterpret_cast<uint2*>(dst + d) = half4(lo.x, lo.y, lo.z, lo.w);
      *reinterpret_cast<uint2*>(dst + d + half) = half4(hi.x, hi.y, hi.z, hi.w);
    }
  } else {  // v: copy into the cache
    uint16_t* dst = vc + (static_cast<int64_t>(pos) * n_kv + (head - n_q - n_kv)) * hd;
    *reinterpret_cast<uint2*>(dst + d) = half4(x1.x, x1.y, x1.z, x1.w);
    *reinterpret_cast<uint2*>(dst + d + half) = half4(x2.x, x2.y, x2.z, x2.w);
  }
}

__device__ __forceinline__ float silu_mul1(float g, float u) {
  const float e = expf(-g);
  const float den = 1.0f + e;
  const float sg = g / den;
  return sg * u;
}

// silu(g) * u with silu(x) = x / (1 + exp(-x)) (F.silu), gu = [M, 2 * inter] (gate then up).
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gu, float* __restrict__ out,
                                                       int64_t M, int64_t inter) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= M * inter) return;
  const int64_t m = t / inter, i = t % inter;
  out[t] = silu_mul1(gu[m * 2 * inter + i], gu[m * 2 * inter + inter + i]);
}

// The same into the fp16 (hi, lo) planes of the down projection: one thread per 8-element chunk
// (inter % 8 == 0), two 16-byte loads of gate and of up, one 16-byte store per plane. With n_split > 0
// each of the four 16-byte values is the sum of the n_split partials part[s] ([M, 2 inter] each) in
// ascending order (sum_partials4, as linear_reduce_kernel adds them), and gu is not read.
__global__ __launch_bounds__(256) void silu_mul_planes_kernel(const float* __restrict__ gu, uint16_t* __restrict__ xh,
                                                              uint16_t* __restrict__ xl, int64_t M, int64_t inter,
                                                              const float* __restrict__ part, int n_split) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // chunk of the [M, inter] result
  if (c >= M * inter / 8) return;
  const int64_t m = (8 * c) / inter, i = (8 * c) % inter;
  const int64_t g_off = m * 2 * inter + i, u_off = g_off + inter;
  float4 g0, g1, u0, u1;
  if (n_split > 0) {
    const int64_t stride = M * 2 * inter / 4;  // one partial, in float4
    const float4* p4 = reinterpret_cast<const float4*>(part);
    g0 = sum_partials4(p4 + g_off / 4, stride, n_split);
    g1 = sum_partials4(p4 + g_off / 4 + 1, stride, n_split);
    u0 = sum_partials4(p4 + u_off / 4, stride, n_split);
    u1 = sum_partials4(p4 + u_off / 4 + 1, stride, n_split);
  } else {
    const float4* gp = reinterpret_cast<const float4*>(gu + g_off);
    const float4* up = reinterpret_cast<const float4*>(gu + u_off);
    g0 = gp[0];
    g1 = gp[1];
    u0 = up[0];
    u1 = up[1];
  }
  const float e8[8] = {silu_mul1(g0.x, u0.x), silu_mul1(g0.y, u0.y), silu_mul1(g0.z, u0.z), silu_mul1(g0.w, u0.w),
                       silu_mul1(g1.x, u1.x), silu_mul1(g1.y, u1.y), silu_mul1(g1.z, u1.z), silu_mul1(g1.w, u1.w)};
  store_x_planes8(xh, xl, c, e8);
}

// argmax with torch.argmax semantics: the first index of the maximum; a NaN counts as the maximum
// (the first NaN wins).
struct Best {
  float v;
  int32_t i;
};

__device__ __forceinline__ bool better(float a, int32_t ia, float b, int32_t ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}

__device__ __forceinline__ Best block_best(Best b) {
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(b.v, m, 64);
    const int32_t oi = __shfl_xor(b.i, m, 64);
    if (better(ov, oi, b.v, b.i)) { b.v = ov; b.i = oi; }
  }
  __shared__ float sv[4];
  __shared__ int32_t si[4];
  if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = b.v; si[threadIdx.x >> 6] = b.i; }
  __syncthreads();
  Best r{sv[0], si[0]};
  for (int w = 1; w < 4; ++w)
    if (better(sv[w], si[w], r.v, r.i)) { r.v = sv[w]; r.i = si[w]; }
  return r;
}

// Each thread issues its kArgE coalesced loads (stride 256 inside the block's span) before comparing
// them, so one pass costs one memory round trip; `better` breaks ties by index, so the visiting
// order does not matter.
constexpr int kArgE = 4;

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ x, int64_t V,
                                                             Best* __restrict__ ws) {
  Best b{-INFINITY, INT32_MAX};
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * kArgE; base < V;
       base += static_cast<int64_t>(gridDim.x) * 256 * kArgE) {
    float v[kArgE];
#pragma unroll
    for (int u = 0; u < kArgE; ++u) {
      const int64_t i = base + u * 256 + threadIdx.x;
      v[u] = x[i < V ? i : V - 1];
    }
#pragma unroll
    for (int u = 0; u < kArgE; ++u) {
      const int64_t i = base + u * 256 + threadIdx.x;
      if (i < V && better(v[u], static_cast<int32_t>(i), b.v, b.i)) { b.v = v[u]; b.i = static_cast<int32_t>(i); }
    }
  }
  const Best r = block_best(b);
  if (threadIdx.x == 0) ws[blockIdx.x] = r;
}

// advance: null, or the decode position, advanced by delta once the token is written (a decode
// graph that feeds itself needs no kernel of its own for it).
__global__ __launch_bounds__(256) void argmax_final_kernel(const Best* __restrict__ ws, int n, int32_t* __restrict__ out,
                                                           int32_t* __restrict__ advance, int delta) {
  // every partial a thread reads in one pass is loaded before any is compared (one memory round
  // trip per 2048 partials)
  constexpr int kPer = 8;
  Best b{-INFINITY, INT32_MAX};
  for (int base = 0; base < n; base += 256 * kPer) {
    Best v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = base + u * 256 + threadIdx.x;
      v[u] = i < n ? ws[i] : Best{-INFINITY, INT32_MAX};
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      if (better(v[u].v, v[u].i, b.v, b.i)) b = v[u];
  }
  const Best r = block_best(b);
  if (threadIdx.x == 0) {
    out[0] = r.i;
    if (advance) advance[0] += delta;
  }
}

int argmax_blocks(int64_t V) {
  const int64_t b = (V + 256 * kArgE - 1) / (256 * kArgE);
  return static_cast<int>(b < 1 ? 1 : (b > 512 ? 512 : b));
}

}  // namespace
}  // namespace q4

using namespace q4;

extern "C" int rmsnorm_f32(const float* x, const float* w, float* out, int64_t M, int64_t D, float eps,
                           const int32_t* row, void* stream) {
  if (!x || !w || !out) return Q4_ERR_NULL;
  if (M <= 0 || D <= 0) return Q4_ERR_SHAPE;
  if (D % 4 == 0 && (!aligned(x, 16) || !aligned(w, 16) || !aligned(out, 16))) return Q4_ERR_ALIGN;
  const unsigned grid = row ? 1u : static_cast<unsigned>(M);
  hipLaunchKernelGGL(rmsnorm_kernel<>, dim3(grid), dim3(256), 0, as_stream(stream), x, w, out, M, D, eps, row,
                     nullptr, nullptr);
  return launch_status();
}

extern "C" int rope_kv_write(float* qkv, const float* cos_t, const float* sin_t, uint16_t* k_cache, uint16_t* v_cache,
                             int C, int n_q, int n_kv, int hd, int max_ctx, const int32_t* start, void* stream) {
  if (!qkv || !cos_t || !sin_t || !k_cache || !v_cache || !start) return Q4_ERR_NULL;
  if (C <= 0 || n_q <= 0 || n_kv <= 0 || hd <= 0 || hd % 2 || max_ctx <= 0) return Q4_ERR_SHAPE;
  if (hd % 8 == 0 && aligned(qkv, 16) && aligned(cos_t, 16) && aligned(sin_t, 16) && aligned(k_cache, 8) &&
      aligned(v_cache, 8)) {
    const int64_t total = static_cast<int64_t>(C) * (n_q + 2 * n_kv) * (hd / 8);
    hipLaunchKernelGGL(rope_kv4_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                       as_stream(stream), qkv, cos_t, sin_t, k_cache, v_cache, C, n_q, n_kv, hd, max_ctx, start);
    return launch_status();
  }
  const int64_t total = static_cast<int64_t>(C) * (n_q + 2 * n_kv) * (hd / 2);
  hipLaunchKernelGGL(rope_kv_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, as_stream(stream),
                     qkv, cos_t, sin_t, k_cache, v_cache, C, n_q, n_kv, hd, max_ctx, start);
  return launch_status();
}

extern "C" int silu_mul_f32(const float* gu, float* out, int64_t M, int64_t inter, void* stream) {
  if (!gu || !out) return Q4_ERR_NULL;
  if (M <= 0 || inter <= 0) return Q4_ERR_SHAPE;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>((M * inter + 255) / 256)), dim3(256), 0,
                     as_stream(stream), gu, out, M, inter);
  return launch_status();
}

namespace q4 {

bool rmsnorm_takes_partials(int64_t D) { return D % 4 == 0 && D <= 4 * 256 * 4; }

int rmsnorm_planes(float* x, const float* w, uint16_t* xh, uint16_t* xl, int64_t M, int64_t D, float eps,
                   hipStream_t st, const float* part, int n_split) {
  if (!x || !w || !xh || !xl) return Q4_ERR_NULL;
  if (M <= 0 || D <= 0 || D % 8) return Q4_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(xh, 16) || !aligned(xl, 16)) return Q4_ERR_ALIGN;
  if (n_split > 0 && (!part || !aligned(part, 16) || !rmsnorm_takes_partials(D) ||
                      static_cast<int64_t>(n_split) * M * D * 4 >= (int64_t{1} << 31)))
    return Q4_ERR_UNSUPPORTED;
  // 1024 threads per row: each thread holds one float4 of the row and its partials, so a row's loads
  // are spread over 16 waves instead of 4
  if (n_split > 6)
    hipLaunchKernelGGL((rmsnorm_kernel<12, 1024>), dim3(static_cast<unsigned>(M)), dim3(1024), 0, st, x, w, nullptr, M,
                       D, eps, nullptr, xh, xl, part, n_split);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<6, 1024>), dim3(static_cast<unsigned>(M)), dim3(1024), 0, st, x, w, nullptr, M,
                       D, eps, nullptr, xh, xl, part, n_split);
  return launch_status();
}

int rmsnorm_row_partials(float* x, const float* w, float* out, int64_t M, int64_t D, float eps, const int32_t* row,
                         const float* part, int n_split, hipStream_t st) {
  if (!x || !w || !out || !row || !part) return Q4_ERR_NULL;
  if (M <= 0 || D <= 0 || n_split <= 0 || !rmsnorm_takes_partials(D)) return Q4_ERR_SHAPE;
  if (static_cast<int64_t>(n_split) * M * D * 4 >= (int64_t{1} << 31)) return Q4_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(out, 16) || !aligned(part, 16)) return Q4_ERR_ALIGN;
  if (n_split > 6)
    hipLaunchKernelGGL(rmsnorm_kernel<12>, dim3(1), dim3(256), 0, st, x, w, out, M, D, eps, row, nullptr, nullptr, part,
                       n_split);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<6>, dim3(1), dim3(256), 0, st, x, w, out, M, D, eps, row, nullptr, nullptr, part,
                       n_split);
  return launch_status();
}

bool rope_kv_takes_partials(const float* qkv, const float* cos_t, const float* sin_t, const uint16_t* kc,
                            const uint16_t* vc, int hd) {
  return hd % 8 == 0 && aligned(qkv, 16) && aligned(cos_t, 16) && aligned(sin_t, 16) && aligned(kc, 8) &&
         aligned(vc, 8);
}

int rope_kv_partials(float* qkv, const float* part, int n_split, const float* cos_t, const float* sin_t, uint16_t* kc,
                     uint16_t* vc, int C, int n_q, int n_kv, int hd, int max_ctx, const int32_t* start, hipStream_t st) {
  if (!qkv || !part || !cos_t || !sin_t || !kc || !vc || !start) return Q4_ERR_NULL;
  if (C <= 0 || n_q <= 0 || n_kv <= 0 || hd <= 0 || max_ctx <= 0 || n_split <= 0) return Q4_ERR_SHAPE;
  if (!rope_kv_takes_partials(qkv, cos_t, sin_t, kc, vc, hd) || !aligned(part, 16)) return Q4_ERR_UNSUPPORTED;
  const int64_t total = static_cast<int64_t>(C) * (n_q + 2 * n_kv) * (hd / 8);
  hipLaunchKernelGGL(rope_kv4_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, st, qkv, cos_t,
                     sin_t, kc, vc, C, n_q, n_kv, hd, max_ctx, start, part, n_split);
  return launch_status();
}

int silu_mul_planes(const float* gu, uint16_t* xh, uint16_t* xl, int64_t M, int64_t inter, hipStream_t st,
                    const float* part, int n_split) {
  if (n_split > 0 ? !part : !gu) return Q4_ERR_NULL;
  if (!xh || !xl) return Q4_ERR_NULL;
  if (M <= 0 || inter <= 0 || inter % 8 || n_split < 0) return Q4_ERR_SHAPE;
  if ((n_split > 0 ? !aligned(part, 16) : !aligned(gu, 16)) || !aligned(xh, 16) || !aligned(xl, 16)) return Q4_ERR_ALIGN;
  hipLaunchKernelGGL(silu_mul_planes_kernel, dim3(static_cast<unsigned>((M * inter / 8 + 255) / 256)), dim3(256), 0,
                     st, gu, xh, xl, M, inter, part, n_split);
  return launch_status();
}

}  // namespace q4

extern "C" int argmax_workspace_bytes(int64_t V, size_t* bytes) {
  if (!bytes) return Q4_ERR_NULL;
  if (V <= 0 || V > INT32_MAX) return Q4_ERR_SHAPE;
  *bytes = static_cast<size_t>(argmax_blocks(V)) * sizeof(Best);
  return Q4_OK;
}

extern "C" int argmax_f32(const float* logits, int64_t V, int32_t* out, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (!logits || !out || !workspace) return Q4_ERR_NULL;
  size_t need = 0;
  if (int st = argmax_workspace_bytes(V, &need)) return st;
  if (workspace_bytes < need) return Q4_ERR_WORKSPACE;
  if (!aligned(workspace, 8)) return Q4_ERR_ALIGN;
  const int nb = argmax_blocks(V);
  const hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(nb), dim3(256), 0, st, logits, V, static_cast<Best*>(workspace));
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, st, static_cast<const Best*>(workspace), nb, out,
                     nullptr, 0);
  return launch_status();
}

namespace q4 {
static_assert(sizeof(ArgBest) == sizeof(Best) && alignof(ArgBest) == alignof(Best), "one partial layout");

int argmax_final_launch(const ArgBest* partials, int n, int32_t* out, int32_t* advance, int delta, hipStream_t st) {
  if (!partials || !out) return Q4_ERR_NULL;
  if (n <= 0) return Q4_ERR_SHAPE;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, st, reinterpret_cast<const Best*>(partials), n, out,
                     advance, delta);
  return launch_status();
}
}  // namespace q4

namespace q4 {
namespace {
__global__ void advance_position_kernel(int32_t* __restrict__ start, int delta) {
  if (threadIdx.x == 0) start[0] += delta;
}
}  // namespace
}  // namespace q4

extern "C" int q4llm_advance_position(int32_t* start, int delta, void* stream) {
  if (!start) return Q4_ERR_NULL;
  if (!aligned(start, 4)) return Q4_ERR_ALIGN;
  hipLaunchKernelGGL(advance_position_kernel, dim3(1), dim3(64), 0, as_stream(stream), start, delta);
  return launch_status();
}
