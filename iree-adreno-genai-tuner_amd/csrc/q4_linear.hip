// Prefill projection y[M, N] = residual + x[M, K] @ dequant(W)^T on the gfx950 matrix cores.
//
// Replaces QLinear.forward at M > 1 (scripts/llm/llama_q4.py:72, F.linear(x, dequantize_q4(W)) in
// fp32) with a fused int4 GEMM that keeps fp32-level accuracy on fp16 MFMA:
//   * x (fp32) is split into x_hi = fp16(x) and x_lo = fp16(x - x_hi); x_hi + x_lo carries about 22
//     significant bits, close to fp32's 24;
//   * the int4 weights are dequantized in the LDS staging path to (nibble - 8) in fp16, which is
//     exact, and the fp16 group scale is NOT folded in (the product of a 4-bit and an 11-bit
//     significand would not fit fp16);
//   * per 16-k step two MFMAs accumulate x_hi.w and x_lo.w in fp32; each product is exact in fp32;
//   * at every group boundary the group's partial sum is multiplied by the fp32 scale and added to
//     the output accumulator, i.e. y = sum_g s_g * sum_{k in g} x_k (nib_k - 8), the same
//     contraction as the reference up to summation order.
// Same tiling as the fp16 GEMM: block tile BM x BN, BK = 64, 2 x 2 waves of 32x32x16 MFMA tiles,
// double-buffered LDS staging with 16-byte row padding, raw buffer loads (out-of-range = zeros).
// Requires K % 64 == 0 and group % 32 == 0 (the host checks); |x| must stay below 65504 (fp16 range).
#include "q4_common.h"

#include <cstdlib>

namespace q4 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;
constexpr int PITCH = BK + 8;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ i32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

template <int BM, int BN>
struct LinCfg {
  static constexpr int kThreads = 256;  // 2 x 2 waves
  static constexpr int WTM = BM / 2, WTN = BN / 2;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int A_CH = BM * BK / 4;   // float4 chunks of the fp32 A tile
  static constexpr int B_CH = BN * BK / 32;  // 16-byte chunks (32 nibbles) of the int4 B tile
  static constexpr int A_LD = (A_CH + kThreads - 1) / kThreads;
  static constexpr int B_LD = (B_CH + kThreads - 1) / kThreads;
  // per stage: A_hi [BM][PITCH], A_lo [BM][PITCH], B [BN][PITCH] halfs, scales [BN][2] floats
  static constexpr size_t kStageHalfs = (2 * BM + BN) * PITCH;
  static constexpr size_t kLds = 2 * (kStageHalfs * 2 + BN * 2 * 4);
};

template <int BM, int BN>
__global__ __launch_bounds__(256) void q4_linear_kernel(const float* __restrict__ X, const int32_t* __restrict__ QW,
                                                        const uint16_t* __restrict__ SC, float* Y, const float* R,
                                                        int M, int N, int K, int group, int tiles_n) {
  using G = LinCfg<BM, BN>;
  extern __shared__ uint4 smem4[];
  auto stage_h = [&](int s) { return reinterpret_cast<uint16_t*>(smem4) + s * G::kStageHalfs; };
  float* sc_base = reinterpret_cast<float*>(reinterpret_cast<uint16_t*>(smem4) + 2 * G::kStageHalfs);
  auto stage_s = [&](int s) { return sc_base + s * BN * 2; };

  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int spr = K / group;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(X, static_cast<uint32_t>(M) * K * 4u);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(QW, static_cast<uint32_t>(N) * (K / 2));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  i32x4 ra[G::A_LD], rb[G::B_LD];
  float rs[2];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < G::A_LD; ++i) {
      const int ch = tid + i * G::kThreads;
      const int r = ch / (BK / 4), c4 = ch % (BK / 4);
      const int row = m0 + r;
      const bool ok = ch < G::A_CH && row < M;
      ra[i] = buf_load16(xr, ok ? (static_cast<uint32_t>(row) * K + k0 + c4 * 4) * 4u : 0x80000000u);
    }
#pragma unroll
    for (int i = 0; i < G::B_LD; ++i) {
      const int ch = tid + i * G::kThreads;
      const int r = ch / (BK / 32), c32 = ch % (BK / 32);
      const int row = n0 + r;
      const bool ok = ch < G::B_CH && row < N;
      rb[i] = buf_load16(wr, ok ? static_cast<uint32_t>(row) * (K / 2) + (k0 + c32 * 32) / 2 : 0x80000000u);
    }
    // scales of the (at most two) groups touching [k0, k0 + BK) for column tid (tid < BN)
    const int g0 = k0 / group, g1 = (k0 + BK - 1) / group;
    const int col = n0 + tid;
    rs[0] = rs[1] = 0.0f;
    if (tid < BN && col < N) {
      rs[0] = half_bits_to_float(SC[static_cast<int64_t>(col) * spr + g0]);
      rs[1] = half_bits_to_float(SC[static_cast<int64_t>(col) * spr + g1]);
    }
  };
  auto lstore = [&](int s) {
    uint16_t* ah = stage_h(s);
    uint16_t* al = ah + BM * PITCH;
    uint16_t* bs = ah + 2 * BM * PITCH;
#pragma unroll
    for (int i = 0; i < G::A_LD; ++i) {
      const int ch = tid + i * G::kThreads;
      if (ch >= G::A_CH) continue;
      const int r = ch / (BK / 4), c4 = ch % (BK / 4);
      uint16_t hi[4], lo[4];
      // whole-vector bit cast (a bit cast of a single vector element was mis-lowered: every lane of
      // the vector read element 0)
      const float4 xv = __builtin_bit_cast(float4, ra[i]);
      const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = xs[e];
        const _Float16 h = static_cast<_Float16>(v);
        hi[e] = __builtin_bit_cast(uint16_t, h);
        lo[e] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v - static_cast<float>(h)));
      }
      *reinterpret_cast<uint2*>(ah + r * PITCH + c4 * 4) =
          make_uint2(hi[0] | (static_cast<uint32_t>(hi[1]) << 16), hi[2] | (static_cast<uint32_t>(hi[3]) << 16));
      *reinterpret_cast<uint2*>(al + r * PITCH + c4 * 4) =
          make_uint2(lo[0] | (static_cast<uint32_t>(lo[1]) << 16), lo[2] | (static_cast<uint32_t>(lo[3]) << 16));
    }
#pragma unroll
    for (int i = 0; i < G::B_LD; ++i) {
      const int ch = tid + i * G::kThreads;
      if (ch >= G::B_CH) continue;
      const int r = ch / (BK / 32), c32 = ch % (BK / 32);
      uint32_t h[16];
      const uint4 wv = __builtin_bit_cast(uint4, rb[i]);
      const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        const uint32_t w = words[wd];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          // (nibble 2p, nibble 2p+1) -> two fp16 values (n - 8), exact
          const float a = static_cast<float>(static_cast<int>((w >> (8 * p)) & 15u) - 8);
          const float b = static_cast<float>(static_cast<int>((w >> (8 * p + 4)) & 15u) - 8);
          h[wd * 4 + p] = float_to_half_bits(a) | (static_cast<uint32_t>(float_to_half_bits(b)) << 16);
        }
      }
      uint4* dst = reinterpret_cast<uint4*>(bs + r * PITCH + c32 * 32);
      dst[0] = make_uint4(h[0], h[1], h[2], h[3]);
      dst[1] = make_uint4(h[4], h[5], h[6], h[7]);
      dst[2] = make_uint4(h[8], h[9], h[10], h[11]);
      dst[3] = make_uint4(h[12], h[13], h[14], h[15]);
    }
    if (tid < BN) {
      stage_s(s)[tid * 2] = rs[0];
      stage_s(s)[tid * 2 + 1] = rs[1];
    }
  };

  float16v acc[G::TM][G::TN], part[G::TM][G::TN];
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) { acc[i][j][e] = 0.0f; part[i][j][e] = 0.0f; }

  const int nk = K / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int s = kt & 1;
    const int k0 = kt * BK;
    if (kt + 1 < nk) gload(k0 + BK);
    const uint16_t* ah = stage_h(s);
    const uint16_t* al = ah + BM * PITCH;
    const uint16_t* bs = ah + 2 * BM * PITCH;
    const float* ss = stage_s(s);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      half8 fh[G::TM], fl[G::TM], fb[G::TN];
#pragma unroll
      for (int i = 0; i < G::TM; ++i) {
        const int r = wm * G::WTM + i * 32 + (lane & 31);
        fh[i] = *reinterpret_cast<const half8*>(ah + r * PITCH + kk + 8 * (lane >> 5));
        fl[i] = *reinterpret_cast<const half8*>(al + r * PITCH + kk + 8 * (lane >> 5));
      }
#pragma unroll
      for (int j = 0; j < G::TN; ++j) {
        const int r = wn * G::WTN + j * 32 + (lane & 31);
        fb[j] = *reinterpret_cast<const half8*>(bs + r * PITCH + kk + 8 * (lane >> 5));
      }
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j) {
          part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fh[i], fb[j], part[i][j], 0, 0, 0);
          part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fl[i], fb[j], part[i][j], 0, 0, 0);
        }
      const int k = k0 + kk;
      if ((k + 16) % group == 0) {  // group ends after this 16-k step: apply its scale
        const int gi = k / group - k0 / group;  // 0 or 1 within this tile
#pragma unroll
        for (int j = 0; j < G::TN; ++j) {
          const float sc = ss[(wn * G::WTN + j * 32 + (lane & 31)) * 2 + gi];
#pragma unroll
          for (int i = 0; i < G::TM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              acc[i][j][e] = fmaf(part[i][j][e], sc, acc[i][j][e]);
              part[i][j][e] = 0.0f;
            }
        }
      }
    }
    if (kt + 1 < nk) lstore(s ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * G::WTM + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
        const int col = n0 + wn * G::WTN + j * 32 + (lane & 31);
        if (row < M && col < N) {
          const int64_t o = static_cast<int64_t>(row) * N + col;
          Y[o] = R ? R[o] + acc[i][j][e] : acc[i][j][e];
        }
      }
}

struct LinTile {
  int bm, bn;
};
constexpr LinTile kLinTiles[] = {{128, 128}, {128, 64}, {64, 64}};
using LinFn = void (*)(const float*, const int32_t*, const uint16_t*, float*, const float*, int, int, int, int, int);
constexpr LinFn kLinFns[] = {q4_linear_kernel<128, 128>, q4_linear_kernel<128, 64>, q4_linear_kernel<64, 64>};
constexpr size_t kLinLds[] = {LinCfg<128, 128>::kLds, LinCfg<128, 64>::kLds, LinCfg<64, 64>::kLds};

}  // namespace

int q4_linear_launch(const float* x, int64_t M, const int32_t* qw, const uint16_t* sc, float* y, const float* res,
                     int64_t N, int64_t K, int group, int cfg, hipStream_t st) {
  int ti = cfg;
  if (ti < 0 || ti > 2) {
    ti = 2;
    for (int i = 0; i < 3; ++i) {
      const int64_t tiles = ((M + kLinTiles[i].bm - 1) / kLinTiles[i].bm) * ((N + kLinTiles[i].bn - 1) / kLinTiles[i].bn);
      if (tiles >= 256) { ti = i; break; }
    }
  }
  const LinTile& t = kLinTiles[ti];
  const int tiles_n = static_cast<int>((N + t.bn - 1) / t.bn);
  const int tiles = static_cast<int>((M + t.bm - 1) / t.bm) * tiles_n;
  if (kLinLds[ti] > 64 * 1024) {
    Q4_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kLinFns[ti]),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLinLds[ti])));
  }
  hipLaunchKernelGGL(kLinFns[ti], dim3(tiles), dim3(256), kLinLds[ti], st, x, qw, sc, y, res, (int)M, (int)N, (int)K,
                     group, tiles_n);
  return launch_status();
}

}  // namespace q4

extern "C" int q4_linear(const float* x, int64_t M, const int32_t* qweight, const uint16_t* scales, float* y,
                         const float* residual, int64_t N, int64_t K, int group, void* stream) {
  if (!x || !qweight || !scales || !y) return Q4_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0 || group <= 0) return Q4_ERR_SHAPE;
  if (K % 64 || group % 32 || K % group) return Q4_ERR_SHAPE;
  if (M * K * 4 >= (int64_t{1} << 31) || N * (K / 2) >= (int64_t{1} << 31) || M > INT32_MAX || N > INT32_MAX)
    return Q4_ERR_SHAPE;
  if (!q4::aligned(x, 16) || !q4::aligned(qweight, 16) || !q4::aligned(y, 4)) return Q4_ERR_ALIGN;
  return q4::q4_linear_launch(x, M, qweight, scales, y, residual, N, K, group, -1, q4::as_stream(stream));
}
