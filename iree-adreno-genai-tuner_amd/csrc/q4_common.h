// Shared definitions of the gfx950 int4 LLM library: status handling, launch helpers and the
// small device utilities every kernel file uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <type_traits>

#include "q4llm.h"

namespace q4 {

// Records the HIP error for q4llm_last_hip_error() and maps it to Q4_ERR_HIP.
int hip_fail(hipError_t e);

#define Q4_CHECK_HIP(expr)                      \
  do {                                          \
    hipError_t e_ = (expr);                     \
    if (e_ != hipSuccess) return q4::hip_fail(e_); \
  } while (0)

// Launch status of the last kernel on this thread.
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? Q4_OK : hip_fail(e);
}

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int kWave = 64;

// ------------------------------------------------------------------------------------------
// Device helpers
// ------------------------------------------------------------------------------------------

// The fp16 exponent patterns that int4 nibble masks are OR'ed with (nibble -> 1024 + n or 64 + n),
// held in VGPRs. gfx9's three-operand encoding takes no literal and reads at most one SGPR, so with
// the mask and the pattern both constants the compiler splits (w & mask) | pattern into an AND and
// an OR; with the pattern in a VGPR it is one v_and_or_b32 (mask in an SGPR).
struct F16Magic {
  uint32_t e1024, e64;  // 0x6400 = 1024.0 and 0x5400 = 64.0 in both halves
};

__device__ __forceinline__ F16Magic f16_magic() {
  F16Magic m;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(m.e1024));
  asm("v_mov_b32 %0, 0x54005400" : "=v"(m.e64));
  return m;
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  // Round to nearest even (v_cvt_f16_f32 under the default rounding mode).
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// p[0] + p[stride] + ... + p[(n - 1) stride] (n >= 1), added in ascending order, so the result has the
// same bits as a plain loop; the first kBatch loads are issued together before any is waited for (a
// loop over a runtime count would wait for each load before issuing the next).
__device__ __forceinline__ float4 sum_partials4(const float4* __restrict__ p, int64_t stride, int n) {
  constexpr int kBatch = 8;
  float4 b[kBatch];
#pragma unroll
  for (int s = 0; s < kBatch; ++s)
    if (s < n) b[s] = p[s * stride];
  float4 a = b[0];
#pragma unroll
  for (int s = 1; s < kBatch; ++s)
    if (s < n) {
      a.x += b[s].x;
      a.y += b[s].y;
      a.z += b[s].z;
      a.w += b[s].w;
    }
  for (int s = kBatch; s < n; ++s) {
    const float4 c = p[s * stride];
    a.x += c.x;
    a.y += c.y;
    a.z += c.z;
    a.w += c.w;
  }
  return a;
}

// Sum over groups of `width` consecutive lanes (width a power of two <= 64); every lane of the
// group receives the total. Uses cross-lane permutes; the summation tree is fixed, so results are
// deterministic.
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = width / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

template <int width>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int m = width / 2; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// DPP sum over aligned segments of `width` lanes (power of two <= 64). The total lands in the LAST
// lane of each segment (lane % width == width - 1); other lanes hold partial sums. Row shifts build
// prefix sums inside each 16-lane DPP row, row_bcast15/31 carry them across rows.
template <int width>
__device__ __forceinline__ float segment_sum_to_last(float v) {
  auto shr = [](float x, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                  decltype(ctrl)::value, 0xf, 0xf, true));
  };
  if constexpr (width >= 2) v += shr(v, std::integral_constant<int, 0x111>{});  // row_shr:1
  if constexpr (width >= 4) v += shr(v, std::integral_constant<int, 0x112>{});  // row_shr:2
  if constexpr (width >= 8) v += shr(v, std::integral_constant<int, 0x114>{});  // row_shr:4
  if constexpr (width >= 16) v += shr(v, std::integral_constant<int, 0x118>{}); // row_shr:8
  if constexpr (width >= 32)  // row_bcast:15 into rows 1 and 3
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xa, 0xf, false));
  if constexpr (width >= 64)  // row_bcast:31 into rows 2 and 3
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xc, 0xf, false));
  return v;
}

// The fp16 (hi, lo) planes a prefill projection takes as its x operand: hi = fp16(v) (round to
// nearest even), lo = fp16(v - hi); element k of a row sits at position (k & ~7) | 2 (k & 3) |
// ((k >> 2) & 1), i.e. each 8-element chunk in the order (0, 4, 1, 5, 2, 6, 3, 7), the k order in
// which the projection decodes a packed int4 word.
__device__ __forceinline__ void store_x_planes(uint16_t* __restrict__ xh, uint16_t* __restrict__ xl, int64_t k,
                                               float v) {
  const _Float16 hi = static_cast<_Float16>(v);
  const _Float16 lo = static_cast<_Float16>(v - static_cast<float>(hi));
  const int64_t p = (k & ~int64_t{7}) | ((k & 3) << 1) | ((k >> 2) & 1);
  xh[p] = __builtin_bit_cast(uint16_t, hi);
  xl[p] = __builtin_bit_cast(uint16_t, lo);
}

// Eight consecutive elements 8c .. 8c + 7 of a row (v[i] = element 8c + i) as one 16-byte store per
// plane (same values and layout as eight store_x_planes calls).
__device__ __forceinline__ void store_x_planes8(uint16_t* __restrict__ xh, uint16_t* __restrict__ xl, int64_t c,
                                                const float (&v)[8]) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float a = v[p], b = v[p + 4];  // positions 2p and 2p + 1 hold elements p and p + 4
    const _Float16 ha = static_cast<_Float16>(a), hb = static_cast<_Float16>(b);
    const _Float16 la = static_cast<_Float16>(a - static_cast<float>(ha));
    const _Float16 lb = static_cast<_Float16>(b - static_cast<float>(hb));
    h[p] = __builtin_bit_cast(uint16_t, ha) | (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hb)) << 16);
    l[p] = __builtin_bit_cast(uint16_t, la) | (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lb)) << 16);
  }
  reinterpret_cast<uint4*>(xh)[c] = make_uint4(h[0], h[1], h[2], h[3]);
  reinterpret_cast<uint4*>(xl)[c] = make_uint4(l[0], l[1], l[2], l[3]);
}

}  // namespace q4
