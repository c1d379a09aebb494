// Decode int4 GEMV for gfx950: y[n] = residual[n] + sum_k x[k] * (nib[n,k] - 8) * scale[n, k/group].
//
// Replaces QLinear._gemv_fused (scripts/llm/llama_q4.py:74-90), the fused decode form the
// reference exports; numerically it is the same contraction as F.linear(x, dequantize_q4(W))
// (llama_q4.py:72).
//
// Memory-bound design (no MFMA):
//   * The packed weight is streamed exactly once with 16-byte loads. A "chunk" is 16 bytes of one
//     row = 4 words = 32 consecutive k. LPR lanes cover consecutive chunks of a row, so every load
//     instruction of a row segment reads LPR*16 contiguous bytes.
//   * Each lane owns R consecutive rows and CPL chunk slots per pass over K; rows of the same chunk
//     reuse the x values read once from LDS.
//   * All global reads are raw buffer loads: a lane whose chunk or row lies past the end gets an
//     out-of-range offset, which the hardware answers with zeros without touching memory. The
//     loads therefore need no branches, and the compiler issues them back to back.
//   * Order at kernel start: x loads (L2), then the first work item's weight and scale loads (HBM),
//     then x is staged into LDS (this waits for x only: loads complete in issue order), barrier.
//     Inside the loop the next item's weights are loaded before the current item is computed.
//   * x sits in LDS in a slot-major layout (slot j of chunk c at [j][c]): lanes reading
//     consecutive chunks hit consecutive 16-byte LDS words.
//   * The row reduction over the LPR lanes is a DPP prefix sum (row_shr / row_bcast).
//   * Nibble decode:
//       fp32 x: bytes of (w & 0x0F0F0F0F) and ((w >> 4) & 0x0F0F0F0F) are converted with
//               v_cvt_f32_ubyte{0..3} and FMA'd with x; the "-8" is applied once per chunk as
//               8 * sum(x_chunk), so the per-element work is one convert and one FMA.
//       fp16 x: masks place nibble pairs in the mantissa of fp16 pairs with a fixed exponent
//               (1024 + n or 64 + n), v_dot2_f32_f16 multiplies them with (x_b, x_b+4) pairs,
//               and the constant offsets (plus the -8) are removed per chunk with a precomputed
//               sum of x. Four dot2 and five bit operations per 8 nibbles.
//     Both paths accumulate in fp32.
#include "q4_common.h"
#include "q4_internal.h"

#include <array>
#include <cstdlib>
#include <utility>

namespace q4 {
namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxK = 16384;
constexpr uint32_t kOOB = 0x80000000u;    // buffer offset past every resource this kernel builds
constexpr int kBufferFlags = 0x00020000;  // gfx9 raw buffer resource word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), kBufferFlags);
}

// kAux: cache-policy bits of the load (2 = nt: streamed once, do not keep in the caches)
template <int kAux = 0>
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kAux);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// fp16 scales: streamed once per launch like the weights (nontemporal)
__device__ __forceinline__ uint16_t buf_load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 2);
}

template <bool kF16X>
struct XLayout {
  // uint4 slots per chunk in LDS: fp16 x -> one uint4 per word (4 half2 pairs); fp32 -> two.
  static constexpr int kSlots = kF16X ? 4 : 8;
};

// LDS: x slots [kSlots][cpr] uint4, per-word correction shares [K/8] float, one junk chunk
// (kSlots uint4 + 1 float, rounded up) that absorbs the stores of out-of-range words.
template <bool kF16X>
inline size_t lds_bytes(int64_t K) {
  const int64_t cpr = K / 32;
  return static_cast<size_t>(cpr) * (XLayout<kF16X>::kSlots * 16 + 16) + XLayout<kF16X>::kSlots * 16 + 16;
}

// x slots of one chunk for dot_chunk_f32: per word j two float4, {x0,x2,x4,x6} and {x1,x3,x5,x7}
struct XChunkF32 {
  float4 p[8];
};

__device__ __forceinline__ XChunkF32 x_chunk_f32(const float4* __restrict__ xs, int cpr, int c) {
  XChunkF32 x;
#pragma unroll
  for (int j = 0; j < 8; ++j) x.p[j] = xs[j * cpr + c];
  return x;
}

__device__ __forceinline__ float dot_chunk_f32(const uint4& w, const XChunkF32& x) {
  float t = 0.0f;
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = words[j] & 0x0F0F0F0Fu;
    const uint32_t hi = (words[j] >> 4) & 0x0F0F0F0Fu;
    const float4 xe = x.p[2 * j];
    const float4 xo = x.p[2 * j + 1];
    t = fmaf(xe.x, static_cast<float>(lo & 0xFFu), t);
    t = fmaf(xe.y, static_cast<float>((lo >> 8) & 0xFFu), t);
    t = fmaf(xe.z, static_cast<float>((lo >> 16) & 0xFFu), t);
    t = fmaf(xe.w, static_cast<float>(lo >> 24), t);
    t = fmaf(xo.x, static_cast<float>(hi & 0xFFu), t);
    t = fmaf(xo.y, static_cast<float>((hi >> 8) & 0xFFu), t);
    t = fmaf(xo.z, static_cast<float>((hi >> 16) & 0xFFu), t);
    t = fmaf(xo.w, static_cast<float>(hi >> 24), t);
  }
  return t;
}

__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

// x slots of one chunk for dot_chunk_f16: xs slot j (one uint4 per word) holds the half2 pairs
// (x0,x4), (x1,x5), (x2,x6), (x3,x7)
struct XChunkF16 {
  uint4 p[4];
};

__device__ __forceinline__ XChunkF16 x_chunk_f16(const uint4* __restrict__ xs, int cpr, int c) {
  XChunkF16 x;
#pragma unroll
  for (int j = 0; j < 4; ++j) x.p[j] = xs[j * cpr + c];
  return x;
}

// 9 VALU operations per 8 nibbles: one shift, four v_and_or_b32 (exponent patterns from F16Magic),
// four v_dot2_f32_f16.
__device__ __forceinline__ float dot_chunk_f16(const uint4& w, const XChunkF16& x, const F16Magic& mg) {
  float t = 0.0f;
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t v = words[j];
    const uint32_t v8 = v >> 8;
    const uint4 xp = x.p[j];
    // (1024 + n0, 1024 + n4), (64 + n1, 64 + n5), (1024 + n2, 1024 + n6), (64 + n3, 64 + n7)
    const uint32_t m0 = (v & 0x000F000Fu) | mg.e1024;
    const uint32_t m1 = (v & 0x00F000F0u) | mg.e64;
    const uint32_t m2 = (v8 & 0x000F000Fu) | mg.e1024;
    const uint32_t m3 = (v8 & 0x00F000F0u) | mg.e64;
    t = __builtin_amdgcn_fdot2(as_h2(m0), as_h2(xp.x), t, false);
    t = __builtin_amdgcn_fdot2(as_h2(m1), as_h2(xp.y), t, false);
    t = __builtin_amdgcn_fdot2(as_h2(m2), as_h2(xp.z), t, false);
    t = __builtin_amdgcn_fdot2(as_h2(m3), as_h2(xp.w), t, false);
  }
  return t;
}

// x words (8 elements each) held per thread during staging: K <= 8 * XW * threads.
template <bool kF16X, int XW>
struct XWords {
  uint4 v[kF16X ? XW : 2 * XW];
};

// Global -> registers for this thread's x words (word wd = threadIdx.x + i * blockDim.x).
template <bool kF16X, int XW>
__device__ __forceinline__ void stage_load(__amdgpu_buffer_rsrc_t xr, XWords<kF16X, XW>& r) {
#pragma unroll
  for (int i = 0; i < XW; ++i) {
    const uint32_t wd = threadIdx.x + i * blockDim.x;
    if constexpr (kF16X) {
      r.v[i] = buf_load16(xr, wd * 16u);
    } else {
      r.v[2 * i] = buf_load16(xr, wd * 32u);
      r.v[2 * i + 1] = buf_load16(xr, wd * 32u + 16u);
    }
  }
}

// Registers -> LDS in the slot layout, plus each word's share of its chunk correction
// (sum_k x_k * offset_k; offset 8 on the fp32 path, base + 8 on the fp16 path with base 1024 for
// even nibble index and 64 for odd). Out-of-range words write to the junk chunk (no branches).
template <bool kF16X, int XW>
__device__ __forceinline__ void stage_store(const XWords<kF16X, XW>& r, int nwords, int cpr, uint4* __restrict__ xs,
                                            float* __restrict__ corr_w, uint4* __restrict__ junk) {
#pragma unroll
  for (int i = 0; i < XW; ++i) {
    const int wd = threadIdx.x + i * blockDim.x;
    const bool ok = wd < nwords;
    const int c = wd >> 2, j = wd & 3;
    float* cdst = ok ? corr_w + wd : reinterpret_cast<float*>(junk + XLayout<kF16X>::kSlots);
    if constexpr (kF16X) {
      const uint4 a = r.v[i];  // x0..x7 as 4 x half2 (low half = even element)
      uint4* dst = ok ? xs + j * cpr + c : junk;
      *dst = make_uint4((a.x & 0xFFFFu) | (a.z << 16), (a.x >> 16) | (a.z & 0xFFFF0000u),
                        (a.y & 0xFFFFu) | (a.w << 16), (a.y >> 16) | (a.w & 0xFFFF0000u));
      const uint32_t h[4] = {a.x, a.y, a.z, a.w};
      float s = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float xv = half_bits_to_float(static_cast<uint16_t>(h[k >> 1] >> (16 * (k & 1))));
        s = fmaf(xv, (k & 1) ? 72.0f : 1032.0f, s);
      }
      *cdst = s;
    } else {
      const float4 a = __builtin_bit_cast(float4, r.v[2 * i]);
      const float4 b = __builtin_bit_cast(float4, r.v[2 * i + 1]);
      float4* d0 = reinterpret_cast<float4*>(ok ? xs + (2 * j) * cpr + c : junk);
      float4* d1 = reinterpret_cast<float4*>(ok ? xs + (2 * j + 1) * cpr + c : junk + 1);
      *d0 = make_float4(a.x, a.z, b.x, b.z);
      *d1 = make_float4(a.y, a.w, b.y, b.w);
      *cdst = 8.0f * (((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)));
    }
  }
}

// ------------------------------------------------------------------------------------------
// Fused prologues of the fp32 model path (x is transformed while it is staged):
//   kProNorm:   x' = rms_norm(x, w, eps) = (x * r) * w, r = 1 / sqrt(mean(x^2) + eps)
//               (llama_q4.py:141-142; the norm before the qkv and gate/up projections)
//   kProSwiglu: x holds [gate | up] (2K values), x' = silu(gate) * up (llama_q4.py:236)
// Every workgroup computes the same r with the same reduction order, so all row blocks see the
// same x'. Contraction is off in these helpers so each product and sum rounds like the
// reference's separate tensor ops.
// ------------------------------------------------------------------------------------------
constexpr int kProNone = 0, kProNorm = 1, kProSwiglu = 2;

__device__ __forceinline__ float sumsq8(const uint4& a, const uint4& b) {
#pragma clang fp contract(off)
  const float4 p = __builtin_bit_cast(float4, a), q = __builtin_bit_cast(float4, b);
  const float s0 = p.x * p.x, s1 = p.y * p.y, s2 = p.z * p.z, s3 = p.w * p.w;
  const float s4 = q.x * q.x, s5 = q.y * q.y, s6 = q.z * q.z, s7 = q.w * q.w;
  return ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7));
}

__device__ __forceinline__ uint4 mul4(const uint4& xv, const uint4& wv) {
  const float4 p = __builtin_bit_cast(float4, xv), w = __builtin_bit_cast(float4, wv);
  return __builtin_bit_cast(uint4, make_float4(p.x * w.x, p.y * w.y, p.z * w.z, p.w * w.w));
}

__device__ __forceinline__ float silu_mul1(float g, float u) {
#pragma clang fp contract(off)
  const float e = expf(-g);
  const float den = 1.0f + e;
  const float sg = g / den;
  return sg * u;
}

__device__ __forceinline__ uint4 swiglu4(const uint4& gv, const uint4& uv) {
  const float4 g = __builtin_bit_cast(float4, gv), u = __builtin_bit_cast(float4, uv);
  return __builtin_bit_cast(uint4, make_float4(silu_mul1(g.x, u.x), silu_mul1(g.y, u.y), silu_mul1(g.z, u.z),
                                               silu_mul1(g.w, u.w)));
}

// ------------------------------------------------------------------------------------------
// Paired-row epilogues of the decode step (R == 2: a lane's two rows form a pair p):
//   kEpiSwiglu: rows p and p + N/2 (gate and up of the fused [gate | up] weight);
//               y[p] = silu(gate) * up, y has N/2 values (llama_q4.py:236).
//   kEpiRope:   rows (head, d) and (head, d + hd/2) of the fused [q | k | v] weight; q and k are
//               rotated at pos = start[0] (x * cos + rotate_half(x) * sin, llama_q4.py:205-207,
//               218-221) and written to y; k and v are also written to the fp16 caches at row pos
//               (llama_q4.py:222-223). pos outside [0, max_ctx) leaves y unrotated and the caches
//               untouched.
// ------------------------------------------------------------------------------------------
constexpr int kEpiNone = 0, kEpiSwiglu = 1, kEpiRope = 2;

using EpiArgs = GemvEpi;

__device__ __forceinline__ void rope_pair(float x1, float x2, float c1, float s1, float c2, float s2, float& lo,
                                          float& hi) {
#pragma clang fp contract(off)
  const float a = x1 * c1;
  const float b = (-x2) * s1;
  lo = a + b;
  const float e = x2 * c2;
  const float f = x1 * s2;
  hi = e + f;
}

template <int LPR, int CPL, int R>
struct Item {
  uint4 w[R][CPL];
  uint16_t s[R][CPL];  // raw fp16 bits; converted at compute time so no wait sits between loads
};

// One workgroup = WAVES waves; a "work item" is one row block (R * 64/LPR rows per wave) times
// one pass of LPR * CPL chunks over K. kMulti == false: exactly one item per workgroup
// (grid = row blocks, LPR * CPL >= K/32), computed straight from the registers its loads land in,
// so the compute of each chunk starts as soon as that chunk arrives. kMulti == true: a grid-stride
// loop over items with two register sets (A/B) used alternately, so the next item streams in while
// the current one is computed and no register copies force early waits.
template <bool kF16X, bool kF16Y, int LPR, int CPL, int R, int WAVES, int XW, bool kMulti, int kPro = kProNone,
          int kEpi = kEpiNone>
__global__ __launch_bounds__(WAVES * 64) void q4_gemv_kernel(
    const int32_t* __restrict__ qw, const uint16_t* __restrict__ scales, const void* __restrict__ x,
    void* y, const float* residual, int N, int K, int gshift, const float* __restrict__ aux, float eps,
    EpiArgs ea) {
  static_assert(kPro == kProNone || !kF16X, "fused prologues take fp32 x");
  static_assert(kEpi == kEpiNone || (R == 2 && !kF16X && !kF16Y), "paired epilogues take fp32 x/y, R == 2");
  __shared__ float red[WAVES];  // per-wave sums of squares of the rms_norm prologue
  extern __shared__ uint4 smem[];
  constexpr int kRowsPerWave = R * (64 / LPR);
  constexpr int kRows = kRowsPerWave * WAVES;
  constexpr int kSlots = XLayout<kF16X>::kSlots;
  // chunk c covers k in [32c, 32c + 32); the group is 32 << gshift elements, so the scale of
  // chunk c is scale[c >> gshift]
  const int cpr = K / 32;
  const int spr = cpr >> gshift;  // scales per row
  const int nwords = K / 8;
  uint4* xs = smem;
  float* corr_w = reinterpret_cast<float*>(smem + kSlots * cpr);
  uint4* junk = smem + kSlots * cpr + cpr;  // corr_w takes cpr uint4

  const __amdgpu_buffer_rsrc_t wres = make_rsrc(qw, static_cast<uint32_t>(N) * static_cast<uint32_t>(K / 2));
  const __amdgpu_buffer_rsrc_t sres = make_rsrc(scales, static_cast<uint32_t>(N) * spr * 2u);
  const __amdgpu_buffer_rsrc_t xres =
      make_rsrc(x, static_cast<uint32_t>(K) * (kF16X ? 2u : 4u) * (kPro == kProSwiglu ? 2u : 1u));

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lr = lane % LPR;
  const int rg = lane / LPR;
  const int n_blocks = (N + kRows - 1) / kRows;
  const int n_kpass = kMulti ? (cpr + LPR * CPL - 1) / (LPR * CPL) : 1;

  auto item_row0 = [&](int it) {
    return (blockIdx.x + (it / n_kpass) * gridDim.x) * kRows + wave * kRowsPerWave + rg * R;
  };
  // Weight row of virtual row v: v itself, or for the paired epilogues row b = v & 1 of pair
  // p = v >> 1; pairs past N/2 map to row N (out of range: zeros, no traffic).
  auto phys_row = [&](int v) -> int {
    if constexpr (kEpi == kEpiNone) {
      return v;
    } else {
      const int pr = v >> 1, b = v & 1;
      if (pr >= (N >> 1)) return N;
      if constexpr (kEpi == kEpiSwiglu) {
        return pr + b * (N >> 1);
      } else {
        const int hh = ea.hd >> 1;
        const int head = pr / hh;
        return head * ea.hd + (pr - head * hh) + b * hh;
      }
    }
  };
  // Loads of one item. Rows past N fall outside the buffer resource by themselves; chunks past
  // the row get kOOB; both return zeros without memory traffic, so no branches are needed.
  auto load_item = [&](int it, Item<LPR, CPL, R>& d) {
    const int kp = it % n_kpass;
    const int row0 = item_row0(it);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t row = static_cast<uint32_t>(phys_row(row0 + r));
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = kp * (LPR * CPL) + i * LPR + lr;
        const uint32_t woff = c < cpr ? row * static_cast<uint32_t>(K / 2) + c * 16u : kOOB;
        const uint32_t soff = c < cpr ? (row * spr + (c >> gshift)) * 2u : kOOB;
        d.w[r][i] = buf_load16<2>(wres, woff);
        d.s[r][i] = buf_load2(sres, soff);
      }
    }
  };
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  float rnorm = 1.0f;  // rms_norm scale, applied to the finished rows
  auto epilogue_pair = [&](int pr, float ya, float yb) {
    float* yf = reinterpret_cast<float*>(y);
    if constexpr (kEpi == kEpiSwiglu) {
      yf[pr] = silu_mul1(ya, yb);
    } else {
      const int hd = ea.hd, hh = hd >> 1;
      const int head = pr / hh, d = pr - head * hh;
      const int ra = head * hd + d;
      const int pos = ea.start[0];
      if (pos < 0 || pos >= ea.max_ctx) {
        yf[ra] = ya;
        yf[ra + hh] = yb;
      } else if (head < ea.n_q + ea.n_kv) {
        const float* cp = ea.cos_t + static_cast<int64_t>(pos) * hd;
        const float* sp = ea.sin_t + static_cast<int64_t>(pos) * hd;
        float lo, hi;
        rope_pair(ya, yb, cp[d], sp[d], cp[d + hh], sp[d + hh], lo, hi);
        yf[ra] = lo;
        yf[ra + hh] = hi;
        if (head >= ea.n_q) {
          uint16_t* dst = ea.kc + (static_cast<int64_t>(pos) * ea.n_kv + (head - ea.n_q)) * hd;
          dst[d] = float_to_half_bits(lo);
          dst[d + hh] = float_to_half_bits(hi);
        }
      } else {
        yf[ra] = ya;
        yf[ra + hh] = yb;
        uint16_t* dst = ea.vc + (static_cast<int64_t>(pos) * ea.n_kv + (head - ea.n_q - ea.n_kv)) * hd;
        dst[d] = float_to_half_bits(ya);
        dst[d + hh] = float_to_half_bits(yb);
      }
    }
  };
  // Accumulate one item; on the last K pass reduce over the LPR lanes and store.
  auto compute_item = [&](int it, const Item<LPR, CPL, R>& d) {
    const int kp = it % n_kpass;
    const F16Magic mg = f16_magic();
    // out-of-range slots carry zero weights and a zero scale; clamp only the LDS address
    auto chunk = [&](int i) { return min(kp * (LPR * CPL) + i * LPR + lr, cpr - 1); };
    // fp16 x with up to 6 waves (measured: 5120x3072 3.86 -> 3.76 us, 3072x8192 4.94 -> 4.88 us; the
    // 8-wave 16384x3072 entry lost 0.5-1 us, so it keeps reading x per chunk): every x slot and
    // correction of the item is read from LDS before the first weight is used, so the chunks that land
    // last carry only their own arithmetic
    if constexpr (kF16X && WAVES <= 6) {
      XChunkF16 xc[CPL];
      float cc[CPL];
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        xc[i] = x_chunk_f16(xs, cpr, chunk(i));
        const float4 cw = reinterpret_cast<const float4*>(corr_w)[chunk(i)];
        cc[i] = (cw.x + cw.y) + (cw.z + cw.w);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < CPL; ++i)
#pragma unroll
        for (int r = 0; r < R; ++r)
          acc[r] = fmaf(half_bits_to_float(d.s[r][i]), dot_chunk_f16(d.w[r][i], xc[i], mg) - cc[i], acc[r]);
    } else if constexpr (!kF16X && CPL <= 3) {
      // fp32 x, the same order (3072x3072 o-projection: 3.62 -> 3.36 us, 5120x3072 4.73 -> 4.34 us)
      XChunkF32 xc[CPL];
      float cc[CPL];
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        xc[i] = x_chunk_f32(reinterpret_cast<const float4*>(xs), cpr, chunk(i));
        const float4 cw = reinterpret_cast<const float4*>(corr_w)[chunk(i)];
        cc[i] = (cw.x + cw.y) + (cw.z + cw.w);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < CPL; ++i)
#pragma unroll
        for (int r = 0; r < R; ++r)
          acc[r] = fmaf(half_bits_to_float(d.s[r][i]), dot_chunk_f32(d.w[r][i], xc[i]) - cc[i], acc[r]);
    } else {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = chunk(i);
        const float4 cw = reinterpret_cast<const float4*>(corr_w)[c];
        const float cc = (cw.x + cw.y) + (cw.z + cw.w);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float t;
          if constexpr (kF16X) t = dot_chunk_f16(d.w[r][i], x_chunk_f16(xs, cpr, c), mg);
          else t = dot_chunk_f32(d.w[r][i], x_chunk_f32(reinterpret_cast<const float4*>(xs), cpr, c));
          acc[r] = fmaf(half_bits_to_float(d.s[r][i]), t - cc, acc[r]);
        }
      }
    }
    if (kp == n_kpass - 1) {
      const int row0 = item_row0(it);
      float v[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        v[r] = segment_sum_to_last<LPR>(acc[r]);
        if constexpr (kPro == kProNorm) v[r] *= rnorm;
        acc[r] = 0.0f;
      }
      if constexpr (kEpi == kEpiNone) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int row = row0 + r;
          if (lr == LPR - 1 && row < N) {
            if constexpr (kF16Y) {
              reinterpret_cast<uint16_t*>(y)[row] = float_to_half_bits(v[r]);
            } else {
              reinterpret_cast<float*>(y)[row] = residual ? residual[row] + v[r] : v[r];
            }
          }
        }
      } else {
        const int pr = row0 >> 1;
        if (lr == LPR - 1 && pr < (N >> 1)) epilogue_pair(pr, v[0], v[1]);
      }
    }
  };

  XWords<kF16X, XW> xr;
  stage_load<kF16X, XW>(xres, xr);
  XWords<kF16X, XW> ar;  // second operand of the prologue: norm weights, or the `up` half
  if constexpr (kPro == kProNorm) stage_load<kF16X, XW>(make_rsrc(aux, static_cast<uint32_t>(K) * 4u), ar);
  if constexpr (kPro == kProSwiglu) {
#pragma unroll
    for (int i = 0; i < XW; ++i) {
      const uint32_t wd = threadIdx.x + i * blockDim.x;
      ar.v[2 * i] = buf_load16(xres, static_cast<uint32_t>(K) * 4u + wd * 32u);
      ar.v[2 * i + 1] = buf_load16(xres, static_cast<uint32_t>(K) * 4u + wd * 32u + 16u);
    }
  }
  Item<LPR, CPL, R> a;
  load_item(0, a);  // a workgroup without items gets rows past N: out of range, no traffic
  if constexpr (kPro == kProNorm) {
    // Sum of squares for r = 1 / sqrt(mean(x^2) + eps); x * w is staged and the finished rows
    // are scaled by r, so the reduction shares the staging barrier. Words past K load as zeros.
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < XW; ++i) ss += sumsq8(xr.v[2 * i], xr.v[2 * i + 1]);
    ss = group_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
#pragma unroll
    for (int i = 0; i < XW; ++i) {
      xr.v[2 * i] = mul4(xr.v[2 * i], ar.v[2 * i]);
      xr.v[2 * i + 1] = mul4(xr.v[2 * i + 1], ar.v[2 * i + 1]);
    }
  }
  auto norm_scale = [&]() {
    if constexpr (kPro == kProNorm) {
      float total = 0.0f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) total += red[w];
      const float mean = total / static_cast<float>(K);
      rnorm = 1.0f / sqrtf(mean + eps);
    }
  };
  if constexpr (kPro == kProSwiglu) {
#pragma unroll
    for (int i = 0; i < 2 * XW; ++i) xr.v[i] = swiglu4(xr.v[i], ar.v[i]);
  }
  if constexpr (!kMulti) {
    stage_store<kF16X, XW>(xr, nwords, cpr, xs, corr_w, junk);
    __syncthreads();
    norm_scale();
    compute_item(0, a);
  } else {
    Item<LPR, CPL, R> b;
    load_item(1, b);
    stage_store<kF16X, XW>(xr, nwords, cpr, xs, corr_w, junk);
    __syncthreads();
    norm_scale();
    const int my_blocks = static_cast<int>(blockIdx.x) < n_blocks ? (n_blocks - 1 - blockIdx.x) / gridDim.x + 1 : 0;
    const int n_items = my_blocks * n_kpass;
    // items past the end are out-of-range loads (zeros) whose rows lie past N, so computing them
    // adds nothing and stores nothing
    for (int it = 0; it < n_items; it += 2) {
      compute_item(it, a);
      load_item(it + 2, a);
      compute_item(it + 1, b);
      load_item(it + 3, b);
    }
  }
}

// Generic fallback for shapes the vectorised kernel does not take (K % 32 != 0, group not 32 times a
// power of two, K too large for the staged layout): one wave per row, one word per lane step, fp32 math.
template <bool kF16X, bool kF16Y>
__global__ __launch_bounds__(256) void q4_gemv_generic(
    const int32_t* __restrict__ qw, const uint16_t* __restrict__ scales, const void* __restrict__ x,
    void* y, const float* residual, int N, int K, int group, const float*, float, EpiArgs) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= N) return;
  const int words = K / 8;
  float acc = 0.0f;
  for (int wd = lane; wd < words; wd += 64) {
    const uint32_t v = static_cast<uint32_t>(qw[static_cast<int64_t>(row) * words + wd]);
    const float s = half_bits_to_float(scales[static_cast<int64_t>(row) * (K / group) + (wd * 8) / group]);
    float t = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      float xv;
      if constexpr (kF16X) xv = half_bits_to_float(reinterpret_cast<const uint16_t*>(x)[wd * 8 + b]);
      else xv = reinterpret_cast<const float*>(x)[wd * 8 + b];
      t = fmaf(xv, static_cast<float>(static_cast<int>((v >> (4 * b)) & 15u) - 8), t);
    }
    acc = fmaf(s, t, acc);
  }
  acc = group_sum<64>(acc);
  if (lane == 0) {
    if constexpr (kF16Y) reinterpret_cast<uint16_t*>(y)[row] = float_to_half_bits(acc);
    else reinterpret_cast<float*>(y)[row] = residual ? residual[row] + acc : acc;
  }
}

// ------------------------------------------------------------------------------------------
// Launch configurations: an explicit list, chosen per shape by a fixed rule.
// ------------------------------------------------------------------------------------------

struct Cfg {
  int lpr, cpl, r, waves, xw;
  bool multi;
};

// The instantiated tile list (index stable: the Q4_DBG_GEMV_CFG override and q4_gemv_cfg select entries by index).
// Single-item entries need lpr * cpl >= K/32; every entry needs K/8 <= xw * 64 * waves.
constexpr Cfg kCfgs[] = {
    {32, 3, 2, 5, 2, false},   // 0: K<=3072, 20 rows/WG (N=5120 -> 256 WGs)
    {32, 3, 1, 5, 2, false},   // 1: K<=3072, 10 rows/WG
    {32, 3, 1, 2, 4, false},   // 2: K<=3072, 4 rows/WG
    {64, 2, 1, 4, 2, false},   // 3: K<=4096, 4 rows/WG
    {16, 6, 1, 5, 2, false},   // 4: K<=3072, 20 rows/WG, 16 lanes per row
    {16, 6, 2, 8, 1, false},   // 5: K<=3072, 64 rows/WG (N=16384 -> 256 WGs)
    {32, 3, 2, 8, 1, false},   // 6: K<=3072, 32 rows/WG
    {32, 3, 1, 8, 1, false},   // 7: K<=3072, 16 rows/WG
    {32, 3, 1, 6, 1, false},   // 8: K<=3072, 12 rows/WG (N=3072 -> 256 WGs)
    {8, 12, 1, 4, 2, false},   // 9: K<=3072, 32 rows/WG, 8 lanes per row
    {64, 4, 1, 4, 4, false},   // 10: K<=8192, 4 rows/WG
    {32, 8, 1, 6, 4, false},   // 11: K<=8192, 12 rows/WG (N=3072 -> 256 WGs)
    {64, 4, 2, 6, 4, false},   // 12: K<=8192, 12 rows/WG, 2 rows per lane
    {64, 4, 1, 8, 2, false},   // 13: K<=8192, 8 rows/WG
    {8, 1, 1, 4, 1, false},    // 14: K<=256, 32 rows/WG (tiny)
    {8, 3, 1, 4, 1, false},    // 15: K<=768, 32 rows/WG (tiny down-projection, K=704)
    {16, 2, 1, 4, 1, false},   // 16: K<=1024, 16 rows/WG
    {32, 4, 1, 8, 1, false},   // 17: K<=4096, 16 rows/WG
    {64, 8, 1, 4, 8, false},   // 18: K<=16384, 4 rows/WG
    {16, 6, 1, 8, 1, true},    // 19: grid-stride, K=3072 in one pass, 32 rows per item (LM head)
    {32, 3, 1, 8, 1, true},    // 20: grid-stride, 16 rows per item
    {16, 6, 2, 8, 1, true},    // 21: grid-stride, 64 rows per item
    {64, 2, 1, 4, 8, true},    // 22: grid-stride, any K <= 16384 in passes of 128 chunks
};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

// group argument: the generic kernel takes the group size, the vectorised kernel log2(group / 32)
using KernelFn = void (*)(const int32_t*, const uint16_t*, const void*, void*, const float*, int, int, int,
                          const float*, float, EpiArgs);

// Paired epilogues exist only for the two-rows-per-lane entries (nullptr elsewhere).
template <bool F16X, bool F16Y, int I, int PRO, int EPI>
constexpr KernelFn kernel_of() {
  constexpr Cfg c = kCfgs[I];
  if constexpr (EPI != kEpiNone && c.r != 2) {
    return nullptr;
  } else {
    return q4_gemv_kernel<F16X, F16Y, c.lpr, c.cpl, c.r, c.waves, c.xw, c.multi, PRO, EPI>;
  }
}

template <bool F16X, bool F16Y, int PRO, int EPI, int... Is>
constexpr auto make_table(std::integer_sequence<int, Is...>) {
  return std::array<KernelFn, sizeof...(Is)>{kernel_of<F16X, F16Y, Is, PRO, EPI>()...};
}

using Seq = std::make_integer_sequence<int, kNumCfgs>;
const auto kTabF32F32 = make_table<false, false, kProNone, kEpiNone>(Seq{});
const auto kTabF32F16 = make_table<false, true, kProNone, kEpiNone>(Seq{});
const auto kTabF16F32 = make_table<true, false, kProNone, kEpiNone>(Seq{});
const auto kTabF16F16 = make_table<true, true, kProNone, kEpiNone>(Seq{});
const auto kTabNorm = make_table<false, false, kProNorm, kEpiNone>(Seq{});
const auto kTabSwiglu = make_table<false, false, kProSwiglu, kEpiNone>(Seq{});
const auto kTabEpiSwiglu = make_table<false, false, kProNone, kEpiSwiglu>(Seq{});
const auto kTabEpiRope = make_table<false, false, kProNone, kEpiRope>(Seq{});
const auto kTabNormEpiSwiglu = make_table<false, false, kProNorm, kEpiSwiglu>(Seq{});
const auto kTabNormEpiRope = make_table<false, false, kProNorm, kEpiRope>(Seq{});

int rows_per_block(const Cfg& c) { return c.r * (64 / c.lpr) * c.waves; }

bool cfg_fits(const Cfg& c, int64_t N, int64_t K) {
  const int64_t cpr = K / 32;
  if (K / 8 > static_cast<int64_t>(c.xw) * 64 * c.waves) return false;
  if (!c.multi && static_cast<int64_t>(c.lpr) * c.cpl < cpr) return false;
  if (!c.multi && (N + rows_per_block(c) - 1) / rows_per_block(c) > 65535) return false;
  return true;
}

// Fixed rule: measured entries for the shapes of the 3B model and the benchmark; otherwise the
// fitting single-item entry with the least padding in K and rows and the most even spread of
// workgroups over 256 CUs, or the grid-stride entry when no single-item entry fits. `paired`
// (the paired-row epilogues) restricts the choice to single-item entries with two rows per lane.
int choose_cfg(int64_t N, int64_t K, bool paired) {
  auto usable = [&](int i) { return cfg_fits(kCfgs[i], N, K) && (!paired || (kCfgs[i].r == 2 && !kCfgs[i].multi)); };
  const int ov = debug_override(Q4_DBG_GEMV_CFG);
  if (ov >= 0 && ov < kNumCfgs && usable(ov)) return ov;
  if (paired) {
    if (K == 3072 && N == 5120) return 0;
    if (K == 3072 && N == 16384) return 6;
  } else {
    if (K == 3072) {
      // 5120 rows: 20 rows per workgroup with 16 lanes per row, 256 workgroups, one per CU, equal
      // bytes everywhere. Against the 10-row entry (512 workgroups, two per CU), three alternating
      // rounds on one MI355X: plain stream launches 3.74-3.76 us against 3.83-3.89 (20 launches),
      // 3.65 against 3.78 (256); graph replays 3.43 against 3.42. Stream launches are how a caller of
      // the C ABI issues single GEMVs, and the model's fp32-x projections take the matrix-core kernel.
      if (N == 5120) return 4;
      if (N == 16384) return 7;
      if (N == 3072) return 8;
      if (N > 65536) return 19;
    }
    if (K == 8192 && N == 3072) return 10;
  }
  const int64_t cpr = K / 32;
  int best = paired ? -1 : 22;
  double best_score = 1e30;
  for (int i = 0; i < kNumCfgs; ++i) {
    const Cfg& c = kCfgs[i];
    if (c.multi || !usable(i)) continue;
    const int64_t span = static_cast<int64_t>(c.lpr) * c.cpl;
    const double k_waste = static_cast<double>(span) / cpr;
    const int64_t blocks = (N + rows_per_block(c) - 1) / rows_per_block(c);
    const double row_waste = static_cast<double>(blocks * rows_per_block(c)) / N;
    const int64_t rounds = (blocks + 255) / 256;
    const double balance = static_cast<double>(rounds * 256) / blocks;
    const double score = k_waste * row_waste * balance * (rounds > 8 ? 1.5 : 1.0);
    if (score < best_score) { best_score = score; best = i; }
  }
  return best;
}

int set_lds_limit(KernelFn fn, size_t bytes) {
  if (bytes <= 64 * 1024) return Q4_OK;
  Q4_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)));
  return Q4_OK;
}

}  // namespace

// Matrix-core GEMV for fp32 x / fp32 y (q4_gemv_mx.hip); Q4_ERR_UNSUPPORTED for shapes it does not
// take. `ep` points at an EpiArgs (same field order as the kernel's own struct).


// Runs config `cfg` (-1 = automatic choice) with `grid_override` workgroups (0 = automatic).
// Automatic fp32-x / fp32-y launches go to the matrix-core kernel when it takes the shape.
int q4_gemv_launch(const int32_t* qweight, const uint16_t* scales, const void* x, int x_dtype, void* y,
                   int y_dtype, const float* residual, int64_t N, int64_t K, int group, int cfg,
                   int grid_override, hipStream_t stream, int prologue = kProNone, const float* aux = nullptr,
                   float eps = 0.0f, int epilogue = kEpiNone, const EpiArgs& ea = EpiArgs{}) {
  const bool f16x = x_dtype == Q4_F16, f16y = y_dtype == Q4_F16;
  if (cfg < 0 && !f16x && !f16y && prologue != kProSwiglu) {
    const int st = gemv_mx_launch(qweight, scales, static_cast<const float*>(x), aux, eps, static_cast<float*>(y),
                                  residual, N, K, group, prologue, epilogue, &ea, stream, false);
    if (st != Q4_ERR_UNSUPPORTED) return st;
  }
  const bool paired = epilogue != kEpiNone;
  int ci = cfg >= 0 && cfg < kNumCfgs ? cfg : choose_cfg(N, K, paired);
  if (paired && (ci < 0 || kCfgs[ci].r != 2 || kCfgs[ci].multi || !cfg_fits(kCfgs[ci], N, K)))
    return Q4_ERR_UNSUPPORTED;
  if (!cfg_fits(kCfgs[ci], N, K)) ci = 22;
  const Cfg& c = kCfgs[ci];
  const int threads = c.waves * 64;
  const int gchunks = group / 32;
  const bool pow2_group = group % 32 == 0 && (gchunks & (gchunks - 1)) == 0;
  // 32-bit buffer offsets: rows past N (up to three grid strides of prefetch) must not wrap
  const int64_t max_row = N + 3LL * 1024 * rows_per_block(c);
  const bool vec = (K % 32 == 0) && pow2_group && K <= kMaxK && cfg_fits(c, N, K) &&
                   N * (K / 2) < (int64_t{1} << 31) && max_row * (K / 2) < (int64_t{1} << 32) &&
                   aligned(qweight, 16) && aligned(x, 16);
  if (!vec && (prologue != kProNone || paired)) return Q4_ERR_UNSUPPORTED;
  if (!vec) {
    const dim3 grid(static_cast<unsigned>((N + 3) / 4)), block(256);
    const EpiArgs none{};
    if (f16x && f16y) hipLaunchKernelGGL((q4_gemv_generic<true, true>), grid, block, 0, stream, qweight, scales, x, y, residual, (int)N, (int)K, group, nullptr, 0.0f, none);
    else if (f16x) hipLaunchKernelGGL((q4_gemv_generic<true, false>), grid, block, 0, stream, qweight, scales, x, y, residual, (int)N, (int)K, group, nullptr, 0.0f, none);
    else if (f16y) hipLaunchKernelGGL((q4_gemv_generic<false, true>), grid, block, 0, stream, qweight, scales, x, y, residual, (int)N, (int)K, group, nullptr, 0.0f, none);
    else hipLaunchKernelGGL((q4_gemv_generic<false, false>), grid, block, 0, stream, qweight, scales, x, y, residual, (int)N, (int)K, group, nullptr, 0.0f, none);
    return launch_status();
  }
  KernelFn fn = f16x ? (f16y ? kTabF16F16[ci] : kTabF16F32[ci]) : (f16y ? kTabF32F16[ci] : kTabF32F32[ci]);
  if (prologue == kProNorm) fn = kTabNorm[ci];
  if (prologue == kProSwiglu) fn = kTabSwiglu[ci];
  if (epilogue == kEpiSwiglu) fn = prologue == kProNorm ? kTabNormEpiSwiglu[ci] : kTabEpiSwiglu[ci];
  if (epilogue == kEpiRope) fn = prologue == kProNorm ? kTabNormEpiRope[ci] : kTabEpiRope[ci];
  if (!fn) return Q4_ERR_UNSUPPORTED;
  const size_t lds = f16x ? lds_bytes<true>(K) : lds_bytes<false>(K);
  if (int st = set_lds_limit(fn, lds)) return st;
  const int64_t blocks = (N + rows_per_block(c) - 1) / rows_per_block(c);
  // Single-item entries: one row block per workgroup. Grid-stride entries: 1024 workgroups (4 per
  // CU; x is staged once per workgroup) unless overridden.
  int64_t grid = blocks;
  if (c.multi) {
    grid = blocks < 1024 ? blocks : 1024;
    if (grid_override > 0) grid = grid_override < blocks ? grid_override : blocks;
  }
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(threads), lds, stream, qweight, scales, x, y,
                     residual, (int)N, (int)K, __builtin_ctz(gchunks), aux, eps, ea);
  return launch_status();
}

int q4_gemv_num_cfgs() { return kNumCfgs; }

}  // namespace q4

namespace {
int gemv_args(const int32_t* qweight, const uint16_t* scales, const void* x, int x_dtype, void* y, int y_dtype,
              const float* residual, int64_t N, int64_t K, int group) {
  if (!qweight || !scales || !x || !y) return Q4_ERR_NULL;
  if (N <= 0 || K <= 0 || group <= 0 || K % 8 || group % 8 || K % group) return Q4_ERR_SHAPE;
  if (N > INT32_MAX || K > INT32_MAX / 8) return Q4_ERR_SHAPE;
  if ((x_dtype != Q4_F32 && x_dtype != Q4_F16) || (y_dtype != Q4_F32 && y_dtype != Q4_F16)) return Q4_ERR_DTYPE;
  if (residual && y_dtype != Q4_F32) return Q4_ERR_DTYPE;
  if (!q4::aligned(qweight, 4) || !q4::aligned(x, 4) || !q4::aligned(y, 2)) return Q4_ERR_ALIGN;
  return Q4_OK;
}
}  // namespace

extern "C" int q4_gemv(const int32_t* qweight, const uint16_t* scales, const void* x, int x_dtype, void* y,
                       int y_dtype, const float* residual, int64_t N, int64_t K, int group, void* stream) {
  if (int st = gemv_args(qweight, scales, x, x_dtype, y, y_dtype, residual, N, K, group)) return st;
  return q4::q4_gemv_launch(qweight, scales, x, x_dtype, y, y_dtype, residual, N, K, group, -1, 0,
                            q4::as_stream(stream));
}

extern "C" int q4_gemv_cfg(const int32_t* qweight, const uint16_t* scales, const void* x, int x_dtype, void* y,
                           int y_dtype, const float* residual, int64_t N, int64_t K, int group, int cfg,
                           int grid, void* stream) {
  if (int st = gemv_args(qweight, scales, x, x_dtype, y, y_dtype, residual, N, K, group)) return st;
  if (cfg >= q4::q4_gemv_num_cfgs() || grid < 0) return Q4_ERR_RANGE;
  return q4::q4_gemv_launch(qweight, scales, x, x_dtype, y, y_dtype, residual, N, K, group, cfg, grid,
                            q4::as_stream(stream));
}

extern "C" int q4_gemv_num_configs(void) { return q4::q4_gemv_num_cfgs(); }

namespace q4 {
int q4_gemv_cfg_info(int i, int* out) {
  if (i < 0 || i >= kNumCfgs) return Q4_ERR_RANGE;
  const Cfg& c = kCfgs[i];
  const int v[6] = {c.lpr, c.cpl, c.r, c.waves, c.xw, c.multi ? 1 : 0};
  for (int j = 0; j < 6; ++j) out[j] = v[j];
  return Q4_OK;
}
}  // namespace q4

extern "C" int q4_gemv_config_info(int cfg, int* info) {
  if (!info) return Q4_ERR_NULL;
  return q4::q4_gemv_cfg_info(cfg, info);
}

extern "C" int q4_gemv_fused(const int32_t* qweight, const uint16_t* scales, const float* x, int prologue,
                             const float* aux, float eps, float* y, const float* residual, int64_t N, int64_t K,
                             int group, void* stream) {
  if (int st = gemv_args(qweight, scales, x, Q4_F32, y, Q4_F32, residual, N, K, group)) return st;
  if (prologue != Q4_PRO_RMSNORM && prologue != Q4_PRO_SWIGLU) return Q4_ERR_DTYPE;
  if (prologue == Q4_PRO_RMSNORM && !aux) return Q4_ERR_NULL;
  if (prologue == Q4_PRO_RMSNORM && !q4::aligned(aux, 16)) return Q4_ERR_ALIGN;
  // other workgroups may still be staging x while y is written, so x must not alias y
  if (static_cast<const void*>(x) == static_cast<const void*>(y)) return Q4_ERR_SHAPE;
  return q4::q4_gemv_launch(qweight, scales, x, Q4_F32, y, Q4_F32, residual, N, K, group, -1, 0,
                            q4::as_stream(stream), prologue, aux, eps);
}

extern "C" int q4_gemv_epilogue(const int32_t* qweight, const uint16_t* scales, const float* x, int prologue,
                                const float* aux, float eps, int epilogue, const q4_rope_kv* rope, float* y,
                                int64_t N, int64_t K, int group, void* stream) {
  if (int st = gemv_args(qweight, scales, x, Q4_F32, y, Q4_F32, nullptr, N, K, group)) return st;
  if (prologue != Q4_PRO_NONE && prologue != Q4_PRO_RMSNORM) return Q4_ERR_DTYPE;
  if (epilogue != Q4_EPI_SWIGLU && epilogue != Q4_EPI_ROPE_KV) return Q4_ERR_DTYPE;
  if (prologue == Q4_PRO_RMSNORM && !aux) return Q4_ERR_NULL;
  if (prologue == Q4_PRO_RMSNORM && !q4::aligned(aux, 16)) return Q4_ERR_ALIGN;
  if (static_cast<const void*>(x) == static_cast<const void*>(y)) return Q4_ERR_SHAPE;
  if (N % 2) return Q4_ERR_SHAPE;
  q4::EpiArgs ea{};
  if (epilogue == Q4_EPI_ROPE_KV) {
    if (!rope || !rope->cos_t || !rope->sin_t || !rope->k_cache || !rope->v_cache || !rope->start) return Q4_ERR_NULL;
    if (rope->n_q <= 0 || rope->n_kv <= 0 || rope->head_dim <= 0 || rope->head_dim % 2 || rope->max_ctx <= 0)
      return Q4_ERR_SHAPE;
    if (N != static_cast<int64_t>(rope->n_q + 2 * rope->n_kv) * rope->head_dim) return Q4_ERR_SHAPE;
    ea = q4::EpiArgs{rope->cos_t, rope->sin_t, rope->k_cache, rope->v_cache, rope->start,
                     rope->n_q, rope->n_kv, rope->head_dim, rope->max_ctx};
  }
  const int pro = prologue == Q4_PRO_RMSNORM ? q4::kProNorm : q4::kProNone;
  const int epi = epilogue == Q4_EPI_SWIGLU ? q4::kEpiSwiglu : q4::kEpiRope;
  return q4::q4_gemv_launch(qweight, scales, x, Q4_F32, y, Q4_F32, nullptr, N, K, group, -1, 0,
                            q4::as_stream(stream), pro, aux, eps, epi, ea);
}
