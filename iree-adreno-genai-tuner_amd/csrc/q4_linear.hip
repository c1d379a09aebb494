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
#include "q4_internal.h"

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

// ------------------------------------------------------------------------------------------------
// Workspace variant (q4_linear_ws): x is split once per call, then a multi-stage MFMA pipeline.
//
//   * split_x_kernel writes x_hi = fp16(x) and x_lo = fp16(x - x_hi) as two [M, K] fp16 planes, each
//     8-element chunk stored in the order (0, 4, 1, 5, 2, 6, 3, 7);
//   * the weight operand is decoded in registers straight from the packed word: the masks
//     (w >> 4i) & 0x000F000F | 0x64006400 make the fp16 pair (1024 + n_i, 1024 + n_{i+4}) and one
//     packed fp16 add of -1032 gives (n - 8) exactly, in the same (0, 4, 1, 5, ...) order, so the
//     MFMA's k products pair up with the x planes (the order of k inside one MFMA does not matter);
//   * x_hi, x_lo, the packed weights and the step's group scales stream into an NST-stage LDS ring
//     with direct global -> LDS loads (the fp16 GEMM's pipeline; x rows use its conflict-free
//     swizzle), so no VGPR is loaded in the loop and NST-1 K steps are in flight; the scales get the
//     same lookahead as the tiles (loaded into registers one step ahead, they held every step to a
//     memory round trip: loads complete in issue order);
//   * per 16-k step two MFMAs (x_hi, x_lo) accumulate a group partial in fp32; at each group end the
//     partial is scaled by the fp32 group scale into the output. A wave reads all of its operands of
//     a stage before its first MFMA, so the LDS latency is paid once per stage;
//   * with a k split (KS = 2), two waves share each 32x32 output tile and take half of the 16-k steps
//     of every stage: twice the waves per CU to hide latency at the small M of a prefill chunk; their
//     sums meet in LDS at the end.
// ------------------------------------------------------------------------------------------------

constexpr uint32_t kOOBw = 0x80000000u;

__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(dst), 16, off, 0, 0, 0);
}

// 4 bytes per lane from global memory straight into LDS: lane i's dword lands at dst + 4 i.
__device__ __forceinline__ void load_lds4(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(dst), 4, off, 0, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One thread per 8-element chunk of x: two 16-byte loads, two 16-byte stores.
__global__ __launch_bounds__(256) void split_x_kernel(const float* __restrict__ x, uint16_t* __restrict__ xh,
                                                      uint16_t* __restrict__ xl, int64_t chunks) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= chunks) return;
  const float4 a = reinterpret_cast<const float4*>(x)[2 * c];
  const float4 b = reinterpret_cast<const float4*>(x)[2 * c + 1];
  const float v[8] = {a.x, b.x, a.y, b.y, a.z, b.z, a.w, b.w};  // order 0, 4, 1, 5, 2, 6, 3, 7
  uint32_t h[4], l[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const _Float16 h0 = static_cast<_Float16>(v[2 * p]), h1 = static_cast<_Float16>(v[2 * p + 1]);
    const _Float16 l0 = static_cast<_Float16>(v[2 * p] - static_cast<float>(h0));
    const _Float16 l1 = static_cast<_Float16>(v[2 * p + 1] - static_cast<float>(h1));
    h[p] = __builtin_bit_cast(uint16_t, h0) | (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h1)) << 16);
    l[p] = __builtin_bit_cast(uint16_t, l0) | (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l1)) << 16);
  }
  reinterpret_cast<uint4*>(xh)[c] = make_uint4(h[0], h[1], h[2], h[3]);
  reinterpret_cast<uint4*>(xl)[c] = make_uint4(l[0], l[1], l[2], l[3]);
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Packed word of 8 nibbles (k = 8c + b at nibble b) -> the fp16 operand (n_b - 8) in k order
// (0, 4, 1, 5, 2, 6, 3, 7). Nibbles 0 and 4 (and 2 and 6 after a shift by 8) sit in the low
// mantissa bits and become 1024 + n under exponent 0x6400; nibbles 1 and 5 (3 and 7) sit 4 bits
// higher, where exponent 0x5400 makes them 64 + n. One packed add of -1032 or -72 then gives
// n - 8, exactly (all values are small fp16 integers). 9 VALU operations per word.
__device__ __forceinline__ half8 nibbles_to_half8(uint32_t w, const F16Magic& mg) {
  const half2v b1024 = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
  const half2v b64 = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
  const uint32_t w8 = w >> 8;
  const half2v p0 = __builtin_bit_cast(half2v, (w & 0x000F000Fu) | mg.e1024) + b1024;   // n0, n4
  const half2v p1 = __builtin_bit_cast(half2v, (w & 0x00F000F0u) | mg.e64) + b64;       // n1, n5
  const half2v p2 = __builtin_bit_cast(half2v, (w8 & 0x000F000Fu) | mg.e1024) + b1024;  // n2, n6
  const half2v p3 = __builtin_bit_cast(half2v, (w8 & 0x00F000F0u) | mg.e64) + b64;      // n3, n7
  return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

template <int BM, int BN, int WM, int WN, int NST, int KS>
struct LinWsCfg {
  static constexpr int kWaves = WM * WN * KS, kThreads = 64 * kWaves;
  static constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
  static constexpr int kXRow = 128;                        // bytes per x row per stage (64 fp16)
  static constexpr int kWRow = 32;                         // bytes per weight row per stage (64 nibbles)
  static constexpr int kSBlk = (BN + 63) / 64;             // 64-column blocks of the scale slots
  static constexpr int kStage = 2 * BM * kXRow + BN * kWRow + 2 * kSBlk * 256;  // + 2 scale slots
  static constexpr int kAI = (BM / 8 + kWaves - 1) / kWaves;  // x direct loads per wave, per plane
  static constexpr int kBI = (BN / 32 + kWaves - 1) / kWaves;  // weight direct loads per wave (32 rows each)
  static constexpr int kSI = (2 * kSBlk + kWaves - 1) / kWaves;  // scale direct loads per wave
  static constexpr int kLPW = 2 * kAI + kBI + kSI;
  static constexpr size_t kLds = static_cast<size_t>(NST) * kStage + 1024;  // + junk for spare loads
  static_assert(TM >= 1 && TN >= 1 && WTM * WM == BM && WTN * WN == BN && BM % 32 == 0 && BN % 32 == 0,
                "tile shape");
  static_assert(NST >= 2 && NST <= 8 && kLPW * (NST - 1) < 64, "stages: vmcnt holds at most 63");
  static_assert(KS == 1 || KS == 2 || KS == 4, "k split over 1, 2 or 4 wave groups");
  static constexpr size_t kRed = static_cast<size_t>(KS - 1) * WM * WN * TM * TN * 16 * 64 * 4;
  static_assert(kRed <= static_cast<size_t>(NST) * kStage, "k-split reduction fits in the stages");
};

// silu(g) * u rounded like the separate tensor ops (llama_q4.py:236), as in the element-wise kernels.
__device__ __forceinline__ float silu_mul_exact(float g, float u) {
#pragma clang fp contract(off)
  const float e = expf(-g);
  const float den = 1.0f + e;
  const float sg = g / den;
  return sg * u;
}

// EPI = 1 (SwiGLU): the N columns are the fused [gate | up] weight's 2 I rows, taken in 32-column blocks
// alternately from gate and up (block B <- rows (B & 1) I + 32 (B >> 1) + [0, 32)), so the two tiles of
// a wave hold the gate and up values of the same 32 outputs in the same lanes; the epilogue writes
// silu(gate) * up for [M, I] into the fp16 (hi, lo) planes at Y (hi) and Y + M I (lo), the input of the
// down projection. R must be null.
// Split over K (n_split > 1, EPI = 0): workgroup s * tiles + t takes output tile t over the 64-k stages
// [s * nk_split, (s + 1) * nk_split) (whole groups) and writes its sum, without the residual, to the
// partial buffer P[s] ([M, N] fp32 each); linear_reduce_kernel then adds the residual and the partials.
// T16 (the decode GEMV's layout, q4_t16.hip; pipelined tile only): QW and SC are the T16 tiles and
// scales of the weight, whose rows sit in the layout's virtual order (t16_pair / t16_hd: the pairing
// and head size it was packed with). Columns are virtual rows: a 64-k stage of 32 of them is half of
// each 64-byte row of two 16-row tiles (16 cache lines per 1 KB load instead of 32 in the reference
// layout), a group's scales of a tile are 32 contiguous bytes, and the epilogue writes each virtual
// column to its weight row (EPI 1 on the SwiGLU pairing: gate and up of a pair sit 8 columns apart,
// exchanged by DPP).
template <int BM, int BN, int WM, int WN, int NST, int KS, int EPI = 0, bool PIPE = false, bool T16 = false>
__global__ __launch_bounds__(64 * WM * WN * KS) void q4_linear_ws_kernel(
    const uint16_t* __restrict__ XH, const uint16_t* __restrict__ XL, const int32_t* __restrict__ QW,
    const uint16_t* __restrict__ SC, float* Y, const float* R, int M, int N, int K, int group, int tiles_n,
    int n_split = 1, int nk_split = 0, float* __restrict__ P = nullptr, int t16_pair = 0, int t16_hd = 0) {
  using G = LinWsCfg<BM, BN, WM, WN, NST, KS>;
  static_assert(EPI == 0 || T16 || (G::TN % 2 == 0 && G::WTN % 64 == 0 && BN % 64 == 0),
                "SwiGLU pairs tiles 2j, 2j + 1");
  static_assert(!T16 || (PIPE && BN % 128 == 0 && (2 * (BN / 128) + G::kWaves - 1) / G::kWaves == G::kSI),
                "T16: the pipelined loop, scale loads of 128 columns in the reference layout's count");
  // weight row of virtual column v
  auto phys = [&](int v) -> int {
    if constexpr (EPI == 0) {
      return v;
    } else {
      const int blk = v >> 5;
      return (blk & 1) * (N >> 1) + ((blk >> 1) << 5) + (v & 31);
    }
  };
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int n_tiles = static_cast<int>(gridDim.x) / n_split;
  const int ksp = static_cast<int>(blockIdx.x) / n_tiles, tile = static_cast<int>(blockIdx.x) - ksp * n_tiles;
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int gshift = __builtin_ctz(group);  // the host passes power-of-two groups only
  const int spr = K >> gshift;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // wave -> (k group ks, tile row wm, tile column wn): the KS wave groups share the tile and each
  // takes 4 / KS of the four 16-k steps of every 64-k stage; their sums meet in LDS at the end.
  const int ks = wave / (WM * WN), wt = wave - ks * (WM * WN);
  const int wm = wt / WN, wn = wt % WN;
  constexpr int KK = 4 / KS;
  const uint32_t xbytes = static_cast<uint32_t>(M) * K * 2u;
  const __amdgpu_buffer_rsrc_t hr = make_rsrc(XH, xbytes);
  const __amdgpu_buffer_rsrc_t lr = make_rsrc(XL, xbytes);
  // T16 geometry: 16-row tiles of nseg 128-k segments (K padded to 4 groups); scales per tile in
  // [n_tiles][4 groups][16 rows]
  const int t16_tiles_k = (K + 4 * group - 1) / (4 * group);
  const int t16_nseg = t16_tiles_k * group / 32;
  const int n_t16 = t16_pair == 0 ? (N + 15) / 16 : N / 16;
  const __amdgpu_buffer_rsrc_t wr =
      T16 ? make_rsrc(QW, static_cast<uint32_t>(n_t16) * t16_nseg * 1024u) : make_rsrc(QW, static_cast<uint32_t>(N) * (K / 2));
  const __amdgpu_buffer_rsrc_t sr = T16 ? make_rsrc(SC, static_cast<uint32_t>(n_t16) * t16_tiles_k * 128u)
                                        : make_rsrc(SC, (static_cast<uint32_t>(N) * spr * 2u + 3u) & ~3u);

  // x planes: instruction j fills rows 8b..8b+7 (b = wave + j * kWaves < BM / 8) of a 128-byte-row
  // plane; the lane for slot (lane % 8) of row r = 8b + lane / 8 fetches chunk (lane % 8) ^ ((r >> 1) & 7).
  // When the waves do not divide BM / 8, the spare instructions load nothing into the junk area, so
  // every wave issues the same number of loads per step.
  uint32_t xoff[G::kAI];
  int xchunk[G::kAI];
  bool xreal[G::kAI];
#pragma unroll
  for (int j = 0; j < G::kAI; ++j) {
    const int b = wave + j * G::kWaves;
    const int r = 8 * b + (lane >> 3);
    xreal[j] = b < BM / 8;
    xchunk[j] = (lane & 7) ^ ((r >> 1) & 7);
    xoff[j] = xreal[j] && m0 + r < M ? static_cast<uint32_t>(m0 + r) * K * 2u + xchunk[j] * 16u : kOOBw;
  }
  // weights: instruction j fills rows 32b..32b+31 (b = wave + j * kWaves < BN / 32) with 32-byte rows,
  // lane -> (row lane / 2, half lane % 2); spare instructions load nothing into a junk area.
  uint32_t woff[G::kBI];
  bool wreal[G::kBI];
#pragma unroll
  for (int j = 0; j < G::kBI; ++j) {
    const int b = wave + j * G::kWaves;
    const int r = 32 * b + (lane >> 1);
    wreal[j] = b < BN / 32;
    if constexpr (T16) {
      // lane -> (tile half lane / 32, row (lane % 32) / 2, 16-byte piece lane % 2) of 32 virtual rows
      const int t = (n0 + 32 * b) / 16 + (lane >> 5);
      woff[j] = wreal[j] && t < n_t16
                    ? static_cast<uint32_t>(t) * t16_nseg * 1024u + ((lane & 31) >> 1) * 64u + (lane & 1) * 16u
                    : kOOBw;
    } else {
      woff[j] = wreal[j] && n0 + r < N ? static_cast<uint32_t>(phys(n0 + r)) * (K / 2) + (lane & 1) * 16u : kOOBw;
    }
  }
  unsigned char* junk = lds + NST * G::kStage;
  // Every step issues the same loads (steps past K load zeros into a free stage), so the number of
  // vector-memory operations in flight is the same on every path: the exact waits below and the
  // compiler's own waits for the scale registers then agree.
  const int nk = K / 64;
  const int kt_begin = n_split > 1 ? ksp * nk_split : 0;
  const int kt_end = n_split > 1 ? min(nk, kt_begin + nk_split) : nk;
  // Load idx (0 <= idx < kLPW, a constant after unrolling) of K step kt into `stage`: the x_hi and x_lo
  // rows of instruction idx / 2 (idx < 2 kAI), then the weight rows, then the scale words.
  auto issue_one = [&](int idx, int kt, int stage) {
    const int k0 = kt * 64;
    const bool kin = kt < kt_end;
    unsigned char* sh = lds + stage * G::kStage;
    unsigned char* sl = sh + BM * G::kXRow;
    unsigned char* sw = sl + BM * G::kXRow;
    if (idx < 2 * G::kAI) {
      const int j = idx / 2;
      const uint32_t off = kin && xoff[j] != kOOBw ? xoff[j] + k0 * 2u : kOOBw;
      if (idx % 2 == 0) load_lds16(hr, xreal[j] ? sh + (wave + j * G::kWaves) * 1024 : junk, off);
      else load_lds16(lr, xreal[j] ? sl + (wave + j * G::kWaves) * 1024 : junk, off);
    } else if (idx < 2 * G::kAI + G::kBI) {
      const int j = idx - 2 * G::kAI;
      const uint32_t kofs = T16 ? static_cast<uint32_t>(kt >> 1) * 1024u + (kt & 1) * 32u : static_cast<uint32_t>(k0 / 2);
      load_lds16(wr, wreal[j] ? sw + (wave + j * G::kWaves) * 1024 : junk,
                 kin && woff[j] != kOOBw ? woff[j] + kofs : kOOBw);
    } else if constexpr (T16) {
      // Scales: instruction i = wave + j * kWaves (< 2 BN / 128) fills slot i / (BN / 128) (the step's
      // first or last group) for the 128 virtual columns of part i % (BN / 128): lane -> rows 2 (lane % 8)
      // and + 1 of tile lane / 8 of the part, stored as fp16 in column order.
      unsigned char* ss = sw + BN * G::kWRow;
      const int g0 = k0 >> gshift, g1 = (k0 + 63) >> gshift;
      const int j = idx - 2 * G::kAI - G::kBI;
      const int i = wave + j * G::kWaves;
      constexpr int kParts = BN / 128;
      const bool real = i < 2 * kParts;
      const int slot = i / kParts, part = i - slot * kParts;
      const int t = n0 / 16 + part * 8 + (lane >> 3);
      const int g = slot ? g1 : g0;
      const uint32_t e = ((static_cast<uint32_t>(t) * t16_tiles_k + (g >> 2)) * 4u + (g & 3)) * 16u + 2u * (lane & 7);
      load_lds4(sr, real ? ss + slot * (BN * 2) + part * 256 : junk, real && kin && t < n_t16 ? e * 2u : kOOBw);
    } else {
      // Scales: instruction i = wave + j * kWaves (< 2 kSBlk) fills slot i / kSBlk (the step's first or
      // last group; a 64-k step touches at most two groups of >= 32) for the 64 columns of block
      // i % kSBlk: lane -> column, the aligned dword holding its fp16 scale (the buffer range is rounded
      // up to 4 bytes; device allocations are 256-byte granular). Spare instructions fill the junk area.
      unsigned char* ss = sw + BN * G::kWRow;
      const int g0 = k0 >> gshift, g1 = (k0 + 63) >> gshift;
      const int j = idx - 2 * G::kAI - G::kBI;
      const int i = wave + j * G::kWaves;
      const bool real = i < 2 * G::kSBlk;
      const int slot = i / G::kSBlk, blk = i - slot * G::kSBlk;
      const int col = n0 + blk * 64 + lane;
      const uint32_t e = static_cast<uint32_t>(phys(col)) * spr + (slot ? g1 : g0);
      load_lds4(sr, real ? ss + (slot * G::kSBlk + blk) * 256 : junk,
                real && kin && col < N ? (e >> 1) * 4u : kOOBw);
    }
  };
  auto issue = [&](int kt, int stage) {
#pragma unroll
    for (int idx = 0; idx < G::kLPW; ++idx) issue_one(idx, kt, stage);
  };

  auto scale_elem = [&](int j, int g) -> uint32_t {
    const int col = n0 + wn * G::WTN + j * 32 + (lane & 31);
    return static_cast<uint32_t>(phys(col)) * spr + g;
  };
  // scale of group g for this lane's column in tile column j, from slot `slot` of the stage at ss
  auto scale_of = [&](const unsigned char* ss, int slot, int j, int g) {
    const int cl = wn * G::WTN + j * 32 + (lane & 31);
    const uint32_t v = *reinterpret_cast<const uint32_t*>(ss + slot * G::kSBlk * 256 + cl * 4);
    return half_bits_to_float(static_cast<uint16_t>(v >> (16 * (scale_elem(j, g) & 1))));
  };

  float16v acc[G::TM][G::TN], part[G::TM][G::TN];
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = part[i][j][e] = 0.0f;

  const int arow = wm * G::WTM + (lane & 31);
  const int brow = wn * G::WTN + (lane & 31);
  // Every load of a step (x planes, weights, scales) goes straight to LDS; when at most NST-2 steps'
  // loads of this wave are in flight, its part of step kt has landed, and the barrier publishes the
  // whole stage. No VGPR is loaded in the loop, so the compiler adds no waits of its own.
  auto step = [&](int kt) {
    wait_vmcnt<(NST - 2) * G::kLPW>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(kt + NST - 1, (kt + NST - 1) % NST);
    asm volatile("" ::: "memory");
    const unsigned char* sh = lds + (kt % NST) * G::kStage;
    const unsigned char* sl = sh + BM * G::kXRow;
    const unsigned char* sw = sl + BM * G::kXRow;
    const unsigned char* ss = sw + BN * G::kWRow;
    const int k0 = kt * 64;
    const F16Magic mg = f16_magic();
    // All operand reads of the step first (x_hi, x_lo and the nibble words of the 4 16-k steps), so the
    // LDS latency is paid once per step instead of once per 16-k step.
    half8 fh[KK][G::TM], fl[KK][G::TM];
    uint32_t fw[KK][G::TN];
#pragma unroll
    for (int q = 0; q < KK; ++q) {
      const int kk = ks * KK + q;
      const int c = 2 * kk + (lane >> 5);  // this lane's 8-k chunk of the 16-k step
      const int xs = (c ^ ((lane >> 1) & 7)) << 4;
#pragma unroll
      for (int i = 0; i < G::TM; ++i) {
        fh[q][i] = *reinterpret_cast<const half8*>(sh + (arow + 32 * i) * G::kXRow + xs);
        fl[q][i] = *reinterpret_cast<const half8*>(sl + (arow + 32 * i) * G::kXRow + xs);
      }
#pragma unroll
      for (int j = 0; j < G::TN; ++j) fw[q][j] = *reinterpret_cast<const uint32_t*>(sw + (brow + 32 * j) * G::kWRow + 4 * c);
    }
    __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the MFMAs that use them
#pragma unroll
    for (int q = 0; q < KK; ++q) {
      const int kk = ks * KK + q;
      half8 fb[G::TN];
#pragma unroll
      for (int j = 0; j < G::TN; ++j) fb[j] = nibbles_to_half8(fw[q][j], mg);
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j) {
          part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fh[q][i], fb[j], part[i][j], 0, 0, 0);
          part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fl[q][i], fb[j], part[i][j], 0, 0, 0);
        }
      const int k = k0 + 16 * kk;
      // Apply the group's scale when the group ends with this 16-k step, or (k split) when this is the
      // wave's last 16-k step of the stage and its group ends inside the stage (another wave group
      // holds the rest of it).
      const bool ends_here = ((k + 16) & (group - 1)) == 0;
      const bool ends_in_stage = KS > 1 && q == KK - 1 && ((((k >> gshift) + 1) << gshift) <= k0 + 64);
      if (ends_here || ends_in_stage) {
        const int g = k >> gshift;
        const int gi = g - (k0 >> gshift);
#pragma unroll
        for (int j = 0; j < G::TN; ++j) {
          const float sc = scale_of(ss, gi, j, g);
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
  };
  if constexpr (!PIPE) {
#pragma unroll
    for (int s = 0; s < NST - 1; ++s) issue(kt_begin + s, (kt_begin + s) % NST);
    for (int kt = kt_begin; kt < kt_end; ++kt) step(kt);
  } else {
    // Software pipeline (one wave group): the operands of each 16-k step are read into one of two
    // fragment sets while the MFMAs of the previous one run from the other, so the LDS reads overlap
    // the matrix core instead of preceding it. K step l of this workgroup (l = kt - kt_begin) sits in
    // buffer l % NST. The one barrier per step comes after this wave's reads of step l and before its
    // last MFMAs: past it every wave is done with buffer l % NST, and step l + 1 has landed, whose
    // first 16-k operands are then read while the last MFMAs of step l run. Step l issues the loads of
    // step l + NST - 1 into the buffer freed at the previous barrier (step l - 1's; buffer NST - 1 is
    // still unused at l = 0), spread over its first three 16-k steps, one between MFMAs. Every step
    // issues the same kLPW loads (past kt_end: zeros), so the vmcnt counts below are constants.
    static_assert(KS == 1, "the pipelined loop runs one wave group over all four 16-k steps");
    constexpr int KK = 4;
    const int nl = kt_end - kt_begin;
    half8 fh[2][G::TM], fl[2][G::TM];
    uint32_t fw[2][G::TN];
    uint32_t sw0[G::TN], sw1[G::TN];  // scale words of the step's slots 0 and 1
    const F16Magic mg = f16_magic();
    auto read_sub = [&](int l, int kk, int set) {
      const unsigned char* sh = lds + (l % NST) * G::kStage;
      const unsigned char* sl = sh + BM * G::kXRow;
      const unsigned char* sw = sl + BM * G::kXRow;
      const int c = 2 * kk + (lane >> 5);  // this lane's 8-k chunk of the 16-k step
      const int xs = (c ^ ((lane >> 1) & 7)) << 4;
#pragma unroll
      for (int i = 0; i < G::TM; ++i) {
        fh[set][i] = *reinterpret_cast<const half8*>(sh + (arow + 32 * i) * G::kXRow + xs);
        fl[set][i] = *reinterpret_cast<const half8*>(sl + (arow + 32 * i) * G::kXRow + xs);
      }
#pragma unroll
      for (int j = 0; j < G::TN; ++j) fw[set][j] = *reinterpret_cast<const uint32_t*>(sw + (brow + 32 * j) * G::kWRow + 4 * c);
    };
    auto read_scales = [&](int l) {
      const unsigned char* ss = lds + (l % NST) * G::kStage + 2 * BM * G::kXRow + BN * G::kWRow;
#pragma unroll
      for (int j = 0; j < G::TN; ++j) {
        const int cl = wn * G::WTN + j * 32 + (lane & 31);
        if constexpr (T16) {
          sw0[j] = *reinterpret_cast<const uint16_t*>(ss + cl * 2);
          sw1[j] = *reinterpret_cast<const uint16_t*>(ss + BN * 2 + cl * 2);
        } else {
          sw0[j] = *reinterpret_cast<const uint32_t*>(ss + cl * 4);
          sw1[j] = *reinterpret_cast<const uint32_t*>(ss + G::kSBlk * 256 + cl * 4);
        }
      }
    };
    // The MFMAs of 16-k step q from fragment set `set` (x_hi products of every tile, then x_lo, so
    // consecutive MFMAs write different tiles), with loads [q kLPW / 3, (q + 1) kLPW / 3) of K step
    // kt_begin + ld (q < 3) placed one after each of the first MFMAs.
    auto mfma_sub = [&](int set, int q, int ld, auto zero) {
      half8 fb[G::TN];
#pragma unroll
      for (int j = 0; j < G::TN; ++j) fb[j] = nibbles_to_half8(fw[set][j], mg);
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j)
          part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fh[set][i], fb[j], decltype(zero)::value ? float16v{} : part[i][j],
                                                             0, 0, 0);
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j)
          part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fl[set][i], fb[j], part[i][j], 0, 0, 0);
      if (q < KK - 1) {
#pragma unroll
        for (int idx = q * G::kLPW / (KK - 1); idx < (q + 1) * G::kLPW / (KK - 1); ++idx)
          issue_one(idx, kt_begin + ld, ld % NST);
        constexpr int kMaxLoads = (G::kLPW + KK - 2) / (KK - 1);
#pragma unroll
        for (int l = 0; l < kMaxLoads; ++l) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one vector-memory load
        }
      }
    };
    // Group end after 16-k step q of K step l: scale this lane's group sums into the outputs.
    auto scale_end = [&](int l, int q) {
      const int k0 = (kt_begin + l) * 64, k = k0 + 16 * q;
      if (((k + 16) & (group - 1)) == 0) {
        const int g = k >> gshift;
        const bool second = g != (k0 >> gshift);
#pragma unroll
        for (int j = 0; j < G::TN; ++j) {
          const uint32_t v = second ? sw1[j] : sw0[j];
          const float sc = half_bits_to_float(static_cast<uint16_t>(T16 ? v : v >> (16 * (scale_elem(j, g) & 1))));
#pragma unroll
          for (int i = 0; i < G::TM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              acc[i][j][e] = fmaf(part[i][j][e], sc, acc[i][j][e]);
              part[i][j][e] = 0.0f;
            }
        }
      }
    };
#pragma unroll
    for (int s = 0; s < NST - 1; ++s) issue(kt_begin + s, s);
    wait_vmcnt<(NST - 2) * G::kLPW>();  // step 0 landed
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_sub(0, 0, 0);
    // One K step; par = 0 / 1: its parity inside a group of 128 (two steps; K splits cut whole groups,
    // so kt_begin is even): the group's first MFMAs take a zero accumulator and its scale is applied
    // once after the last MFMAs of the odd step, with no zeroing and no branch. par = -1: any group,
    // checked after every 16-k step.
    using no = std::false_type;
    auto step_body = [&](int l, auto par) {
      constexpr int kPar = decltype(par)::value;
      const int ld = l + NST - 1;
#pragma unroll
      for (int kk = 0; kk < KK - 1; ++kk) {
        read_sub(l, kk + 1, (kk + 1) & 1);
        if (kk == 0 && kPar != 0) read_scales(l);
        __builtin_amdgcn_sched_barrier(0);
        if (kPar == 0 && kk == 0) mfma_sub(0, 0, ld, std::true_type{});
        else mfma_sub(kk & 1, kk, ld, no{});
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kPar < 0) scale_end(l, kk);
      }
      if (l + 1 < nl) {
        // this wave's loads of step l + 1 landed (steps up to l + NST - 1 issued); its reads of step l
        // done (lgkmcnt(0)) before the barrier frees the buffer
        wait_vmcnt<(NST - 2) * G::kLPW>();
        __builtin_amdgcn_s_waitcnt(0xC07F);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        read_sub(l + 1, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      mfma_sub(1, KK - 1, -1, no{});
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kPar < 0) {
        scale_end(l, KK - 1);
      } else if constexpr (kPar == 1) {
        const int g = ((kt_begin + l) * 64) >> gshift;
#pragma unroll
        for (int j = 0; j < G::TN; ++j) {
          const float sc = half_bits_to_float(static_cast<uint16_t>(T16 ? sw0[j] : sw0[j] >> (16 * (scale_elem(j, g) & 1))));
#pragma unroll
          for (int i = 0; i < G::TM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = fmaf(part[i][j][e], sc, acc[i][j][e]);
        }
      }
    };
    if (group == 128) {
      for (int l = 0; l < nl; l += 2) {
        step_body(l, std::integral_constant<int, 0>{});
        step_body(l + 1, std::integral_constant<int, 1>{});
      }
    } else {
      for (int l = 0; l < nl; ++l) step_body(l, std::integral_constant<int, -1>{});
    }
    wait_vmcnt<0>();  // the last steps' (zero) loads have landed before the waves exit
  }

  if constexpr (KS > 1) {
    // k-split: wave groups 1..KS-1 hand their sums to group 0 through LDS (the stage memory; the
    // out-of-range loads of the last steps must land before it is reused). Layout [group][wave][tile]
    // [e][lane]: every access is one 256-byte row.
    wait_vmcnt<0>();
    __syncthreads();
    float* red = reinterpret_cast<float*>(lds);
    auto slot = [&](int g2, int i, int j, int e) {
      return red + ((((g2 * (WM * WN) + wt) * G::TM + i) * G::TN + j) * 16 + e) * 64 + lane;
    };
    if (ks > 0) {
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) *slot(ks - 1, i, j, e) = acc[i][j][e];
    }
    __syncthreads();  // waits for this wave's LDS writes (lgkmcnt) before the barrier
    if (ks > 0) return;
#pragma unroll
    for (int g2 = 0; g2 < KS - 1; ++g2)
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] += *slot(g2, i, j, e);
  }

  if constexpr (EPI == 1 && T16) {
    // Virtual column c of a 16-column group: gate row 8 (c / 16) + c % 8 for c % 16 < 8, its up row 8
    // columns later. Tiles j and j + 1 are paired so that every lane finishes one pair: lanes with
    // c % 16 < 8 keep gate of tile j and receive its up from lane l ^ 8, lanes with c % 16 >= 8 keep up
    // of tile j + 1 and receive its gate (one DPP row rotate by 8 per two outputs).
    static_assert(G::TN % 2 == 0, "tiles are paired");
    const int I = N >> 1;
    uint16_t* oh = reinterpret_cast<uint16_t*>(Y);
    uint16_t* ol = oh + static_cast<int64_t>(M) * I;
    const bool hi8 = (lane & 8) != 0;
#pragma unroll
    for (int i = 0; i < G::TM; ++i)
#pragma unroll
      for (int j = 0; j < G::TN; j += 2)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float keep = hi8 ? acc[i][j + 1][e] : acc[i][j][e];
          const float send = hi8 ? acc[i][j][e] : acc[i][j + 1][e];
          const float got =
              __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0x128, 0xF, 0xF, false));
          const float g = hi8 ? got : keep, u = hi8 ? keep : got;
          const int row = m0 + wm * G::WTM + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
          const int vc = n0 + wn * G::WTN + (j + (hi8 ? 1 : 0)) * 32 + (lane & 31);
          const int pr = 8 * (vc >> 4) + (vc & 7);
          if (row < M && pr < I) store_x_planes(oh, ol, static_cast<int64_t>(row) * I + pr, silu_mul_exact(g, u));
        }
    return;
  } else if constexpr (EPI == 1) {
    const int I = N >> 1;
    uint16_t* oh = reinterpret_cast<uint16_t*>(Y);
    uint16_t* ol = oh + static_cast<int64_t>(M) * I;
#pragma unroll
    for (int i = 0; i < G::TM; ++i)
#pragma unroll
      for (int j = 0; j < G::TN; j += 2)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = m0 + wm * G::WTM + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
          const int col = n0 + wn * G::WTN + j * 32 + (lane & 31);  // the gate column; col + 32 is up
          if (row < M && col < N)
            store_x_planes(oh, ol, static_cast<int64_t>(row) * I + phys(col),
                           silu_mul_exact(acc[i][j][e], acc[i][j + 1][e]));
        }
    return;
  }
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * G::WTM + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
        int col = n0 + wn * G::WTN + j * 32 + (lane & 31);
        if constexpr (T16) {
          if (t16_pair == Q4_PAIR_ROPE) {
            // virtual column -> pair p = 8 (c / 16) + c % 8, rows (head, d) and (head, d + hd / 2)
            const int pr = 8 * (col >> 4) + (col & 7), hh = t16_hd >> 1, sh = __builtin_ctz(hh);
            const int head = pr >> sh;
            col = pr < (N >> 1) ? head * t16_hd + (pr - (head << sh)) + ((col & 8) ? hh : 0) : N;
          } else if (t16_pair == Q4_PAIR_SWIGLU) {
            // virtual column -> pair p = 8 (c / 16) + c % 8: gate row p, or up row N / 2 + p
            const int pr = 8 * (col >> 4) + (col & 7);
            col = pr < (N >> 1) ? pr + ((col & 8) ? (N >> 1) : 0) : N;
          }
        }
        if (row < M && col < N) {
          const int64_t o = static_cast<int64_t>(row) * N + col;
          if (n_split > 1) P[static_cast<int64_t>(ksp) * M * N + o] = acc[i][j][e];
          else Y[o] = R ? R[o] + acc[i][j][e] : acc[i][j][e];
        }
      }
}

// y = residual + sum_s P[s] over n = M N / 4 float4 elements, the splits added in ascending order
// (fixed, so results do not depend on scheduling); y may alias the residual.
__global__ __launch_bounds__(256) void linear_reduce_kernel(const float4* __restrict__ P, const float4* R, float4* Y,
                                                            int64_t n, int n_split) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  float4 a = sum_partials4(P + i, n, n_split);
  if (R) {
    const float4 r = R[i];
    a = make_float4(r.x + a.x, r.y + a.y, r.z + a.z, r.w + a.w);
  }
  Y[i] = a;
}

struct LinWsTile {
  int bm, bn, wm, wn, nst, ks;
  bool pipe;
};
// Explicit tile list (index stable for Q4_DBG_LINEAR_TILE sweeps): the entries the rules below pick. Swept
// and removed (slower on every 3B prefill shape at M = 128, 256 and 1024): 4-wave 64x64, 32x64 and
// 64x128 wave tiles on 128x128, 64x128, 128x64 and 64x256, 32x128 wave tiles (4 or 8 waves on 64x256,
// 128x128, 128x256, 64x512), 64x64 waves on 128x256, k-split 2-wave and 64x64 / 128x64 / 32x96 /
// 32x128 / 32x160 variants.
constexpr LinWsTile kLinWsTiles[] = {
    {64, 64, 2, 2, 4, 1},    // 0: 4 waves of 32x32, 4 stages (77 KB)
    {32, 64, 1, 2, 4, 2},    // 1: 4 waves: 2 tiles of 32x32, each k-split over 2 waves (52 KB)
    {64, 256, 2, 4, 4, 1, true},  // 2: 8 waves of 32x64, software-pipelined: one workgroup per CU for
                                  // 256-row chunks, and the K split
};
constexpr int kSplitTile = 2;  // the K-split tile (linear_split_plan) and the SwiGLU-epilogue tile
using LinWsFn = void (*)(const uint16_t*, const uint16_t*, const int32_t*, const uint16_t*, float*, const float*, int,
                         int, int, int, int, int, int, float*, int, int);
template <int I>
constexpr LinWsFn lin_ws_fn() {
  constexpr LinWsTile t = kLinWsTiles[I];
  return q4_linear_ws_kernel<t.bm, t.bn, t.wm, t.wn, t.nst, t.ks, 0, t.pipe>;
}
// the K-split / SwiGLU tile with the weight in the T16 layout (EPI 0 or 1)
template <int EPI>
constexpr LinWsFn lin_ws_t16_fn() {
  constexpr LinWsTile t = kLinWsTiles[kSplitTile];
  return q4_linear_ws_kernel<t.bm, t.bn, t.wm, t.wn, t.nst, t.ks, EPI, true, true>;
}
template <int I>
constexpr size_t lin_ws_lds() {
  constexpr LinWsTile t = kLinWsTiles[I];
  return LinWsCfg<t.bm, t.bn, t.wm, t.wn, t.nst, t.ks>::kLds;
}
constexpr LinWsFn kLinWsFns[] = {lin_ws_fn<0>(), lin_ws_fn<1>(), lin_ws_fn<2>()};
constexpr size_t kLinWsLds[] = {lin_ws_lds<0>(), lin_ws_lds<1>(), lin_ws_lds<2>()};
static_assert(kLinWsTiles[kSplitTile].pipe && kLinWsTiles[kSplitTile].ks == 1, "the T16 variants need the pipelined loop");

// A T16 source the K-split tile can read: both pointers, a group the layout takes, whole 16-row tiles
// for the paired orders, 16-byte aligned tiles (Q4_DBG_PREFILL_REF_LAYOUT set: the reference layout).
bool t16_usable(const T16Src* t, int64_t N, int group, int pairing_needed) {
  if (!t || !t->tiles || !t->scales || debug_flag(Q4_DBG_PREFILL_REF_LAYOUT)) return false;
  if ((group != 32 && group != 128) || !aligned(t->tiles, 16) || !aligned(t->scales, 4)) return false;
  if (pairing_needed >= 0 && t->pairing != pairing_needed) return false;
  if (t->pairing == Q4_PAIR_SWIGLU) return N % 16 == 0;
  if (t->pairing == Q4_PAIR_ROPE) {
    const int hh = t->head_dim / 2;
    return N % 16 == 0 && t->head_dim > 0 && hh % 8 == 0 && (hh & (hh - 1)) == 0 && N % t->head_dim == 0;
  }
  return t->pairing == Q4_PAIR_NONE;
}
static_assert(sizeof(kLinWsFns) / sizeof(kLinWsFns[0]) == sizeof(kLinWsTiles) / sizeof(kLinWsTiles[0]),
              "one kernel per tile entry");
constexpr int kNumLinWs = sizeof(kLinWsTiles) / sizeof(kLinWsTiles[0]);

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

int q4_linear_ws_num_tiles() { return kNumLinWs; }

int q4_linear_ws_tile_info(int i, int* out) {
  if (i < 0 || i >= kNumLinWs) return Q4_ERR_RANGE;
  const LinWsTile& t = kLinWsTiles[i];
  const int v[7] = {t.bm, t.bn, t.wm, t.wn, t.nst, t.ks, t.pipe ? 1 : 0};
  for (int j = 0; j < 7; ++j) out[j] = v[j];
  return Q4_OK;
}

namespace {
// What the pipelined GEMM's index arithmetic assumes: every 64-k stage lies in whole groups of a
// power of two >= 32 (at most two scale slots per stage, groups found by shifts), K a multiple of
// 64, and 32-bit element offsets.
int planes_args(const uint16_t* xh, const uint16_t* xl, int64_t M, const int32_t* qw, const uint16_t* sc, int64_t N,
                int64_t K, int group) {
  if (!xh || !xl || !qw || !sc) return Q4_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0 || group < 32 || (group & (group - 1)) || K % 64 || K % group) return Q4_ERR_SHAPE;
  if (M * K * 4 >= (int64_t{1} << 31) || N * (K / 2) >= (int64_t{1} << 31) || M > INT32_MAX || N > INT32_MAX)
    return Q4_ERR_SHAPE;
  if (!aligned(xh, 16) || !aligned(xl, 16) || !aligned(qw, 16)) return Q4_ERR_ALIGN;
  return Q4_OK;
}
}  // namespace

// K split of the 64x256 tile (kSplitTile) for a chunk of M <= 256 rows whose tiles alone would leave
// CUs idle: about 256 / tiles splits, each a whole number of groups (64-k stages, at least one group).
LinearSplit linear_split_plan(int64_t M, int64_t N, int64_t K, int group) {
  LinearSplit p{1, 0};
  if (M <= 0 || M > 256 || K % 64 || group <= 0) return p;
  const int64_t tiles = ((M + 63) / 64) * ((N + 255) / 256);
  const int64_t s0 = 256 / tiles;
  if (s0 < 2) return p;
  const int nk = static_cast<int>(K / 64), gst = group > 64 ? group / 64 : 1;
  int nk_s = static_cast<int>((nk + s0 - 1) / s0);
  nk_s = (nk_s + gst - 1) / gst * gst;
  const int S = (nk + nk_s - 1) / nk_s;
  if (S < 2) return p;
  p.n_split = S;
  p.nk_split = nk_s;
  return p;
}

size_t linear_split_part_bytes(int64_t M, int64_t N, int64_t K, int group) {
  const LinearSplit p = linear_split_plan(M, N, K, group);
  return p.n_split > 1 ? static_cast<size_t>(p.n_split) * M * N * sizeof(float) : 0;
}

// The pipelined GEMM on x given as fp16 (hi, lo) planes (store_x_planes layout, [M, K] each);
// power-of-two groups only. Tile rule from a sweep of every entry over the 3B prefill shapes at
// M = 128, 256 and 1024 (graph replays on one MI355X): with a partial buffer `part` of at least
// linear_split_part_bytes, the K-split 64x256 tile where linear_split_plan gives a split (every M <= 256
// chunk of the 3072-, 5120- and 8192-wide projections), then linear_reduce_kernel; otherwise the 32x64
// k-split tile while it gives at most 768 workgroups, else 64x64. Q4_DBG_LINEAR_TILE overrides (no K split).
int q4_linear_planes(const uint16_t* xh, const uint16_t* xl, int64_t M, const int32_t* qw, const uint16_t* sc,
                     float* y, const float* res, int64_t N, int64_t K, int group, hipStream_t st, float* part,
                     size_t part_bytes, int* deferred, const T16Src* t16) {
  if (int e = planes_args(xh, xl, M, qw, sc, N, K, group)) return e;
  if (!y) return Q4_ERR_NULL;
  if (deferred) *deferred = 0;
  int ti = -1;
  const int ov = debug_override(Q4_DBG_LINEAR_TILE);
  if (ov >= 0 && ov < kNumLinWs) ti = ov;
  const LinearSplit sp = linear_split_plan(M, N, K, group);
  if (ti < 0 && part && sp.n_split > 1 && part_bytes >= linear_split_part_bytes(M, N, K, group) &&
      (M * N) % 4 == 0 && aligned(part, 16) && aligned(y, 16) && (!res || aligned(res, 16)) &&
      static_cast<int64_t>(sp.n_split) * M * N < (int64_t{1} << 31)) {
    constexpr int T = kSplitTile;
    const LinWsTile& t = kLinWsTiles[T];
    const int tiles_n = static_cast<int>((N + t.bn - 1) / t.bn);
    const int tiles = static_cast<int>((M + t.bm - 1) / t.bm) * tiles_n;
    const bool use_t16 = t16_usable(t16, N, group, -1);
    const LinWsFn fn = use_t16 ? lin_ws_t16_fn<0>() : kLinWsFns[T];
    if (kLinWsLds[T] > 64 * 1024) {
      Q4_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(kLinWsLds[T])));
    }
    hipLaunchKernelGGL(fn, dim3(tiles * sp.n_split), dim3(64 * t.wm * t.wn * t.ks), kLinWsLds[T], st, xh, xl,
                       use_t16 ? static_cast<const int32_t*>(t16->tiles) : qw, use_t16 ? t16->scales : sc, y, res,
                       (int)M, (int)N, (int)K, group, tiles_n, sp.n_split, sp.nk_split, part,
                       use_t16 ? t16->pairing : 0, use_t16 ? t16->head_dim : 0);
    if (int e = launch_status()) return e;
    if (deferred) {
      *deferred = sp.n_split;
      return Q4_OK;
    }
    const int64_t n4 = M * N / 4;
    hipLaunchKernelGGL(linear_reduce_kernel, dim3(static_cast<unsigned>((n4 + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const float4*>(part), reinterpret_cast<const float4*>(res),
                       reinterpret_cast<float4*>(y), n4, sp.n_split);
    return launch_status();
  }
  // Rule from a sweep at M = 128, 256, 1024: the 32x64 k-split tile while it gives <= 768 workgroups,
  // else 64x64; and 64x256 when, at M <= 256, it alone gives one workgroup per CU (the gate/up
  // projection of a 256-row chunk: 256x16384x3072 82 -> 69 us, x re-read over 4x fewer column tiles).
  if (ti < 0) {
    const int64_t wide = ((M + 63) / 64) * ((N + 255) / 256);
    if (M <= 256 && wide >= 256) ti = kSplitTile;
    else ti = ((M + 31) / 32) * ((N + 63) / 64) <= 768 ? 1 : 0;
  }
  const LinWsTile& t = kLinWsTiles[ti];
  const int tiles_n = static_cast<int>((N + t.bn - 1) / t.bn);
  const int tiles = static_cast<int>((M + t.bm - 1) / t.bm) * tiles_n;
  const bool use_t16 = ti == kSplitTile && t16_usable(t16, N, group, -1);
  const LinWsFn fn = use_t16 ? lin_ws_t16_fn<0>() : kLinWsFns[ti];
  if (kLinWsLds[ti] > 64 * 1024) {
    Q4_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(kLinWsLds[ti])));
  }
  hipLaunchKernelGGL(fn, dim3(tiles), dim3(64 * t.wm * t.wn * t.ks), kLinWsLds[ti], st, xh, xl,
                     use_t16 ? static_cast<const int32_t*>(t16->tiles) : qw, use_t16 ? t16->scales : sc, y, res, (int)M,
                     (int)N, (int)K, group, tiles_n, 1, 0, nullptr, use_t16 ? t16->pairing : 0,
                     use_t16 ? t16->head_dim : 0);
  return launch_status();
}

// The gate/up projection with the SwiGLU epilogue (EPI = 1) on the tile the fixed rule picks for it at
// M <= 256 (64x256, one workgroup per CU); other shapes return Q4_ERR_UNSUPPORTED and the caller runs
// q4_linear_planes + silu_mul_planes. oh / ol: the [M, N / 2] output planes (must not alias xh / xl).
int q4_linear_planes_swiglu(const uint16_t* xh, const uint16_t* xl, int64_t M, const int32_t* qw, const uint16_t* sc,
                            uint16_t* oh, uint16_t* ol, int64_t N, int64_t K, int group, hipStream_t st,
                            const T16Src* t16) {
  if (int e = planes_args(xh, xl, M, qw, sc, N, K, group)) return e;
  if (!oh || !ol) return Q4_ERR_NULL;
  if (debug_set(Q4_DBG_LINEAR_TILE) || debug_flag(Q4_DBG_SWIGLU_UNFUSED)) return Q4_ERR_UNSUPPORTED;
  constexpr LinWsTile t = kLinWsTiles[kSplitTile];
  const int64_t wide = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
  if (!(M <= 256 && wide >= 256) || N % t.bn || (N / 2) % 32 || ol != oh + M * (N / 2)) return Q4_ERR_UNSUPPORTED;
  const bool use_t16 = t16_usable(t16, N, group, Q4_PAIR_SWIGLU);
  const LinWsFn fn = use_t16 ? lin_ws_t16_fn<1>() : q4_linear_ws_kernel<t.bm, t.bn, t.wm, t.wn, t.nst, t.ks, 1, t.pipe>;
  constexpr size_t lds = LinWsCfg<t.bm, t.bn, t.wm, t.wn, t.nst, t.ks>::kLds;
  if (lds > 64 * 1024) {
    Q4_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds)));
  }
  const int tiles_n = static_cast<int>(N / t.bn);
  const int tiles = static_cast<int>((M + t.bm - 1) / t.bm) * tiles_n;
  hipLaunchKernelGGL(fn, dim3(tiles), dim3(64 * t.wm * t.wn * t.ks), lds, st, xh, xl,
                     use_t16 ? static_cast<const int32_t*>(t16->tiles) : qw, use_t16 ? t16->scales : sc,
                     reinterpret_cast<float*>(oh), nullptr, (int)M, (int)N, (int)K, group, tiles_n, 1, 0, nullptr,
                     use_t16 ? t16->pairing : 0, use_t16 ? t16->head_dim : 0);
  return launch_status();
}

// ws holds the planes (M K fp16 each) and, past them (from a 256-byte boundary), ws_bytes permitting,
// the K-split partials.
int q4_linear_ws_launch(const float* x, int64_t M, const int32_t* qw, const uint16_t* sc, float* y, const float* res,
                        int64_t N, int64_t K, int group, void* ws, size_t ws_bytes, hipStream_t st) {
  // the pipelined kernel indexes groups by shifts: other group sizes take the workspace-free kernel
  if (group & (group - 1)) return q4_linear_launch(x, M, qw, sc, y, res, N, K, group, -1, st);
  uint16_t* xh = static_cast<uint16_t*>(ws);
  uint16_t* xl = xh + M * K;
  const int64_t chunks = M * K / 8;
  hipLaunchKernelGGL(split_x_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0, st, x, xh, xl,
                     chunks);
  if (int e = launch_status()) return e;
  const size_t planes = (static_cast<size_t>(M) * K * 4 + 255) / 256 * 256;
  float* part = ws_bytes > planes ? reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + planes) : nullptr;
  return q4_linear_planes(xh, xl, M, qw, sc, y, res, N, K, group, st, part, part ? ws_bytes - planes : 0);
}

}  // namespace q4

namespace {
int linear_args(const float* x, int64_t M, const int32_t* qweight, const uint16_t* scales, float* y, int64_t N,
                int64_t K, int group) {
  if (!x || !qweight || !scales || !y) return Q4_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0 || group <= 0) return Q4_ERR_SHAPE;
  if (K % 64 || group % 32 || K % group) return Q4_ERR_SHAPE;
  if (M * K * 4 >= (int64_t{1} << 31) || N * (K / 2) >= (int64_t{1} << 31) || M > INT32_MAX || N > INT32_MAX)
    return Q4_ERR_SHAPE;
  if (!q4::aligned(x, 16) || !q4::aligned(qweight, 16) || !q4::aligned(y, 4)) return Q4_ERR_ALIGN;
  return Q4_OK;
}
}  // namespace

extern "C" int q4_linear_ws_num_configs(void) { return q4::q4_linear_ws_num_tiles(); }

extern "C" int q4_linear_ws_config_info(int cfg, int* info) {
  if (!info) return Q4_ERR_NULL;
  return q4::q4_linear_ws_tile_info(cfg, info);
}

extern "C" int q4_linear_workspace_bytes(int64_t M, int64_t K, size_t* bytes) {
  if (!bytes) return Q4_ERR_NULL;
  if (M <= 0 || K <= 0 || K % 64) return Q4_ERR_SHAPE;
  *bytes = static_cast<size_t>(M) * static_cast<size_t>(K) * 4;  // x_hi and x_lo planes, fp16
  return Q4_OK;
}

extern "C" int q4_linear_ws_split_bytes(int64_t M, int64_t N, int64_t K, int group, size_t* bytes) {
  if (!bytes) return Q4_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 || group <= 0) return Q4_ERR_SHAPE;
  const size_t planes = (static_cast<size_t>(M) * K * 4 + 255) / 256 * 256;
  const size_t part = (group & (group - 1)) == 0 ? q4::linear_split_part_bytes(M, N, K, group) : 0;
  *bytes = part ? planes + part : static_cast<size_t>(M) * K * 4;
  return Q4_OK;
}

extern "C" int q4_linear_ws(const float* x, int64_t M, const int32_t* qweight, const uint16_t* scales, float* y,
                            const float* residual, int64_t N, int64_t K, int group, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (int st = linear_args(x, M, qweight, scales, y, N, K, group)) return st;
  if (!workspace) return Q4_ERR_NULL;
  if (workspace_bytes < static_cast<size_t>(M) * static_cast<size_t>(K) * 4) return Q4_ERR_WORKSPACE;
  if (!q4::aligned(workspace, 16)) return Q4_ERR_ALIGN;
  return q4::q4_linear_ws_launch(x, M, qweight, scales, y, residual, N, K, group, workspace, workspace_bytes,
                                 q4::as_stream(stream));
}

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
