// fp16 GEMM C[M,N] = A[M,K] @ B[N,K]^T on the gfx950 matrix cores (fp32 accumulation, fp16 out).
//
// Contract of the reference's GEMM study (gemm/shapes.py:1-66): row-major fp16 operands, B stored
// as a PyTorch Linear weight [N, K] ("NT", S2 prefill_nt), checked against an fp32 reference. The
// reference searched a schedule space per shape (gemm/schedule.py); here the tile space is an
// explicit list of CDNA4 tiles and a fixed rule picks one per shape.
//
// Kernel structure:
//   * block tile BM x BN, K step BK = 64; WGM x WGN waves, each owning a (BM/WGM) x (BN/WGN) tile
//     made of 32x32 v_mfma_f32_32x32x16_f16 tiles;
//   * A and B tiles are staged global -> registers -> LDS, double buffered: the loads of step k+1
//     are in flight while step k runs on the matrix cores;
//   * LDS rows are padded by 16 bytes so the 16-byte operand reads of a wave are conflict free;
//   * global reads are raw buffer loads: rows past M/N and k past K read out of range and return
//     zeros, so ragged edges need no branches;
//   * workgroups are ordered XCD-major: consecutive tiles along N land on the same XCD and share
//     its L2 for the A panel.
// MFMA operand layout used: lane l supplies row (l % 32) of A (column of B) and 8 consecutive k at
// 8 * (l / 32); A and B use the same k pattern, so the product is independent of the order in which
// the hardware consumes the k elements of a lane. Accumulator j of lane l holds
// (row 8 * (j / 4) + 4 * (l / 32) + j % 4, col l % 32).
#include "q4_common.h"

#include <cstdlib>

namespace q4 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;
constexpr int PITCH = BK + 8;  // LDS row pitch in halfs (16-byte pad)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <int BM, int BN, int WGM, int WGN>
struct GemmCfg {
  static constexpr int kWaves = WGM * WGN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int WTM = BM / WGM;  // wave tile
  static constexpr int WTN = BN / WGN;
  static constexpr int TM = WTM / 32;   // 32x32 MFMA tiles per wave
  static constexpr int TN = WTN / 32;
  static constexpr int A_CH = BM * BK / 8;  // 16-byte chunks per A tile
  static constexpr int B_CH = BN * BK / 8;
  static constexpr int A_LD = (A_CH + kThreads - 1) / kThreads;
  static constexpr int B_LD = (B_CH + kThreads - 1) / kThreads;
  static constexpr size_t kLds = 2ull * (BM + BN) * PITCH * 2;
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 32x32 MFMA tile");
};

template <int BM, int BN, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_f16_nt_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ Cm, int M, int N, int K,
    int lda, int ldb, int ldc, int tiles_m, int tiles_n, int k_per_split, int xcd_remap) {
  using G = GemmCfg<BM, BN, WGM, WGN>;
  extern __shared__ uint4 smem4[];
  uint16_t* lds = reinterpret_cast<uint16_t*>(smem4);
  uint16_t* As[2] = {lds, lds + BM * PITCH};
  uint16_t* Bs[2] = {lds + 2 * BM * PITCH, lds + 2 * BM * PITCH + BN * PITCH};

  // XCD-major tile order: workgroup b runs on XCD b % 8; give XCD x a contiguous tile range.
  int bid = blockIdx.x;
  const int ntiles = tiles_m * tiles_n;
  if (xcd_remap) bid = (bid % 8) * (ntiles / 8) + bid / 8;
  const int tm = bid / tiles_n, tn = bid % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kz = blockIdx.y;  // split-K slice
  const int kbeg = kz * k_per_split;
  const int kend = min(K, kbeg + k_per_split);

  const __amdgpu_buffer_rsrc_t ar = make_rsrc(A, static_cast<uint32_t>(M - 1) * lda * 2u + K * 2u);
  const __amdgpu_buffer_rsrc_t br = make_rsrc(B, static_cast<uint32_t>(N - 1) * ldb * 2u + K * 2u);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  uint4 ra[G::A_LD], rb[G::B_LD];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < G::A_LD; ++i) {
      const int ch = tid + i * G::kThreads;
      const int r = ch / (BK / 8), c8 = ch % (BK / 8);
      const int row = m0 + r, k = k0 + c8 * 8;
      const bool ok = ch < G::A_CH && row < M && k < kend;
      ra[i] = buf_load16(ar, ok ? (static_cast<uint32_t>(row) * lda + k) * 2u : 0x80000000u);
    }
#pragma unroll
    for (int i = 0; i < G::B_LD; ++i) {
      const int ch = tid + i * G::kThreads;
      const int r = ch / (BK / 8), c8 = ch % (BK / 8);
      const int row = n0 + r, k = k0 + c8 * 8;
      const bool ok = ch < G::B_CH && row < N && k < kend;
      rb[i] = buf_load16(br, ok ? (static_cast<uint32_t>(row) * ldb + k) * 2u : 0x80000000u);
    }
  };
  auto lstore = [&](int s) {
#pragma unroll
    for (int i = 0; i < G::A_LD; ++i) {
      const int ch = tid + i * G::kThreads;
      if (ch < G::A_CH) *reinterpret_cast<uint4*>(As[s] + (ch / (BK / 8)) * PITCH + (ch % (BK / 8)) * 8) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < G::B_LD; ++i) {
      const int ch = tid + i * G::kThreads;
      if (ch < G::B_CH) *reinterpret_cast<uint4*>(Bs[s] + (ch / (BK / 8)) * PITCH + (ch % (BK / 8)) * 8) = rb[i];
    }
  };

  float16v acc[G::TM][G::TN];
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int nk = (kend - kbeg + BK - 1) / BK;
  gload(kbeg);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < nk) gload(kbeg + (kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      half8 af[G::TM], bf[G::TN];
#pragma unroll
      for (int i = 0; i < G::TM; ++i) {
        const int r = wm * G::WTM + i * 32 + (lane & 31);
        af[i] = *reinterpret_cast<const half8*>(As[s] + r * PITCH + kk + 8 * (lane >> 5));
      }
#pragma unroll
      for (int j = 0; j < G::TN; ++j) {
        const int r = wn * G::WTN + j * 32 + (lane & 31);
        bf[j] = *reinterpret_cast<const half8*>(Bs[s] + r * PITCH + kk + 8 * (lane >> 5));
      }
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore(s ^ 1);
    __syncthreads();
  }

  // Epilogue: fp16 stores (split-K slices > 0 never occur on this path; see host).
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * G::WTM + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
        const int col = n0 + wn * G::WTN + j * 32 + (lane & 31);
        if (row < M && col < N) Cm[static_cast<int64_t>(row) * ldc + col] = float_to_half_bits(acc[i][j][e]);
      }
}

// fp16 GEMV for M == 1 (the gemv_nt shape): one wave per 4 rows of B, 16 lanes per row,
// v_dot2_f32_f16 with fp32 accumulation. Memory bound.
__global__ __launch_bounds__(256) void gemv_f16_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ B,
                                                       uint16_t* __restrict__ c, int N, int K, int ldb) {
  typedef _Float16 half2v __attribute__((ext_vector_type(2)));
  const int lane = threadIdx.x & 63;
  const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + lane / 16;
  const int lr = lane % 16;
  const __amdgpu_buffer_rsrc_t br = make_rsrc(B, static_cast<uint32_t>(N - 1) * ldb * 2u + K * 2u);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a, K * 2u);
  float acc = 0.0f;
  for (int k = lr * 8; k < K; k += 128) {
    const uint4 w = buf_load16(br, row < N ? (static_cast<uint32_t>(row) * ldb + k) * 2u : 0x80000000u);
    const uint4 x = buf_load16(xr, k * 2u);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, w.x), __builtin_bit_cast(half2v, x.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, w.y), __builtin_bit_cast(half2v, x.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, w.z), __builtin_bit_cast(half2v, x.z), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, w.w), __builtin_bit_cast(half2v, x.w), acc, false);
  }
  acc = segment_sum_to_last<16>(acc);
  if (lr == 15 && row < N) c[row] = float_to_half_bits(acc);
}

struct TileCfg {
  int bm, bn, wgm, wgn;
};
// Explicit CDNA4 tile list (index stable for q4_gemm_cfg / Q4_GEMM_CFG).
constexpr TileCfg kTiles[] = {
    {256, 256, 2, 2},  // 0: large square problems (1 workgroup per CU at 4096^2)
    {256, 128, 2, 2},  // 1
    {128, 128, 2, 2},  // 2
    {128, 64, 2, 2},   // 3: M = 256 prefill shapes: enough workgroups for 256 CUs
    {64, 64, 2, 2},    // 4: small / skinny problems
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

using GemmFn = void (*)(const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, int, int, int, int, int);

template <int I>
constexpr GemmFn gemm_fn() {
  return gemm_f16_nt_kernel<kTiles[I].bm, kTiles[I].bn, kTiles[I].wgm, kTiles[I].wgn>;
}
template <int I>
constexpr size_t gemm_lds() {
  return GemmCfg<kTiles[I].bm, kTiles[I].bn, kTiles[I].wgm, kTiles[I].wgn>::kLds;
}
constexpr GemmFn kGemmFns[] = {gemm_fn<0>(), gemm_fn<1>(), gemm_fn<2>(), gemm_fn<3>(), gemm_fn<4>()};
constexpr size_t kGemmLds[] = {gemm_lds<0>(), gemm_lds<1>(), gemm_lds<2>(), gemm_lds<3>(), gemm_lds<4>()};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Fixed rule: the largest tile that still gives at least one full wave of workgroups per CU
// (256); otherwise the tile with the most workgroups.
int choose_tile(int64_t M, int64_t N) {
  const char* ov = getenv("Q4_GEMM_CFG");
  if (ov && *ov) {
    const int i = atoi(ov);
    if (i >= 0 && i < kNumTiles) return i;
  }
  for (int i = 0; i < kNumTiles; ++i)
    if (cdiv(M, kTiles[i].bm) * cdiv(N, kTiles[i].bn) >= 256) return i;
  return kNumTiles - 1;
}

}  // namespace

int gemm_f16_launch(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                    int64_t ldb, int64_t ldc, int cfg, hipStream_t st) {
  if (M == 1 && cfg < 0) {
    const unsigned grid = static_cast<unsigned>(cdiv(N, 16));
    hipLaunchKernelGGL(gemv_f16_kernel, dim3(grid), dim3(256), 0, st, A, B, C, (int)N, (int)K, (int)ldb);
    return launch_status();
  }
  const int ti = cfg >= 0 && cfg < kNumTiles ? cfg : choose_tile(M, N);
  const TileCfg& t = kTiles[ti];
  const int tiles_m = static_cast<int>(cdiv(M, t.bm)), tiles_n = static_cast<int>(cdiv(N, t.bn));
  const int ntiles = tiles_m * tiles_n;
  const size_t lds = kGemmLds[ti];
  if (lds > 64 * 1024) {
    Q4_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kGemmFns[ti]),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  }
  const int remap = (ntiles % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL(kGemmFns[ti], dim3(ntiles, 1), dim3(64 * t.wgm * t.wgn), lds, st, A, B, C, (int)M, (int)N,
                     (int)K, (int)lda, (int)ldb, (int)ldc, tiles_m, tiles_n, (int)K, remap);
  return launch_status();
}

int gemm_f16_num_tiles() { return kNumTiles; }

}  // namespace q4

namespace {
int gemm_args(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t M, int64_t N, int64_t K, int64_t lda,
              int64_t ldb, int64_t ldc) {
  if (!A || !B || !C) return Q4_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0 || K % 8 || lda < K || ldb < K || ldc < N || lda % 8 || ldb % 8) return Q4_ERR_SHAPE;
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return Q4_ERR_SHAPE;
  if ((M - 1) * lda * 2 + K * 2 >= (int64_t{1} << 31) || (N - 1) * ldb * 2 + K * 2 >= (int64_t{1} << 31)) return Q4_ERR_SHAPE;
  if (!q4::aligned(A, 16) || !q4::aligned(B, 16) || !q4::aligned(C, 2)) return Q4_ERR_ALIGN;
  return Q4_OK;
}
}  // namespace

extern "C" int gemm_f16_nt(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t M, int64_t N, int64_t K,
                           int64_t lda, int64_t ldb, int64_t ldc, void* stream) {
  if (int st = gemm_args(A, B, C, M, N, K, lda, ldb, ldc)) return st;
  return q4::gemm_f16_launch(A, B, C, M, N, K, lda, ldb, ldc, -1, q4::as_stream(stream));
}

extern "C" int gemm_f16_nt_cfg(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t M, int64_t N, int64_t K,
                               int64_t lda, int64_t ldb, int64_t ldc, int cfg, int split, void* stream) {
  (void)split;
  if (int st = gemm_args(A, B, C, M, N, K, lda, ldb, ldc)) return st;
  if (cfg >= q4::gemm_f16_num_tiles()) return Q4_ERR_RANGE;
  return q4::gemm_f16_launch(A, B, C, M, N, K, lda, ldb, ldc, cfg, q4::as_stream(stream));
}

extern "C" int gemm_f16_num_configs(void) { return q4::gemm_f16_num_tiles(); }
