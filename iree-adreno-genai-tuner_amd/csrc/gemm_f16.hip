// fp16 GEMM C[M,N] = A[M,K] @ B[N,K]^T on the gfx950 matrix cores (fp32 accumulation, fp16 out).
//
// Contract of the reference's GEMM study (gemm/shapes.py:1-66): row-major fp16 operands, B stored
// as a PyTorch Linear weight [N, K] ("NT", S2 prefill_nt), checked against an fp32 reference. The
// reference searched a schedule space per shape (gemm/schedule.py); here the tile space is an
// explicit list of CDNA4 tiles and a fixed rule picks one per shape.
//
// Kernel structure:
//   * block tile BM x BN, K step BK = 64 or 32 (one 128- or 64-byte LDS row per operand row);
//     WM x WN waves, each owning a (BM/WM) x (BN/WN) tile of 32x32 v_mfma_f32_32x32x16_f16 tiles;
//   * NST-stage ring of LDS stages filled by direct global -> LDS 16-byte loads (buffer loads with
//     the LDS bit, gfx950): no VGPRs are spent on staging, and the loads of the next NST-1 K steps
//     are in flight while the current step runs on the matrix cores; each wave waits only for the
//     oldest stage's loads (an exact vmcnt), then one barrier per K step publishes the stage and
//     frees the one read in the previous step;
//   * a direct load writes 64 lanes x 16 bytes contiguously (1 KB of whole rows), so the layout is
//     chosen on the global side: the lane for LDS slot s of row r fetches chunk s ^ swz(r), which
//     makes the MFMA operand reads conflict free without padding (see swz below);
//   * global reads are raw buffer loads: rows past M/N and k past K read out of range and land as
//     zeros, so ragged edges need no branches;
//   * workgroups are ordered XCD-major and grouped: each XCD gets a compact block of tiles (4 tile
//     rows at a time), so its A and B panel slices are reused from its own L2.
// MFMA operand layout used: lane l supplies row (l % 32) of A (column of B) and 8 consecutive k at
// 8 * (l / 32); A and B use the same k pattern, so the product is independent of the order in which
// the hardware consumes the k elements of a lane. Accumulator j of lane l holds
// (row 8 * (j / 4) + 4 * (l / 32) + j % 4, col l % 32).
#include "q4_common.h"
#include "q4_internal.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace q4 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes per lane from global memory straight into LDS: lane i's bytes land at dst + 16 i (dst
// is wave-uniform). Out-of-range offsets land zeros; `soff` (a uniform addend) is used only where
// the whole access is in range.
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t off, uint32_t soff = 0) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(dst), 16, off,
                                           static_cast<int>(soff), 0, 0);
}

// s_waitcnt with only the vector-memory counter constrained (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int BM, int BN, int WM, int WN, int NST, int BK>
struct GemmCfg {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int WTM = BM / WM;  // wave tile
  static constexpr int WTN = BN / WN;
  static constexpr int TM = WTM / 32;  // 32x32 MFMA tiles per wave
  static constexpr int TN = WTN / 32;
  static constexpr int kRow = BK * 2;                  // bytes per LDS row: 128 (BK 64) or 64 (BK 32)
  static constexpr int kRowsPerInst = 1024 / kRow;     // rows one direct-load instruction fills
  static constexpr int kStage = (BM + BN) * kRow;
  // direct-load instructions per wave and stage; when the waves do not divide the row blocks, the spare
  // instructions load nothing into a 1 KB junk area after the stages, so every wave issues the same
  // number per stage
  static constexpr int kAI = (BM / kRowsPerInst + kWaves - 1) / kWaves;
  static constexpr int kBI = (BN / kRowsPerInst + kWaves - 1) / kWaves;
  static constexpr bool kJunk = (BM / kRowsPerInst) % kWaves != 0 || (BN / kRowsPerInst) % kWaves != 0;
  static constexpr size_t kLds = static_cast<size_t>(NST) * kStage + (kJunk ? 1024 : 0);
  static_assert(kLds <= 160 * 1024, "LDS per workgroup");
  static constexpr int kLPW = kAI + kBI;
  static_assert(BK == 32 || BK == 64, "K step");
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 32x32 MFMA tile");
  static_assert(BM % kRowsPerInst == 0 && BN % kRowsPerInst == 0 && WTM * WM == BM && WTN * WN == BN,
                "tile shape");
  static_assert(NST >= 2 && NST <= 4 && kLPW * (NST - 2) < 64, "stage count");
};

// LDS swizzle: chunk c (16 bytes) of tile row r sits at slot c ^ swz(r). The LDS serves 16 lanes x
// 16 bytes per clock from 16 bank groups (256 bytes); an MFMA operand read takes 16 consecutive
// rows at one chunk, which the swizzle spreads over all 16 groups:
//   BK 64 (128-byte rows, 2 per 256 bytes): swz(r) = (r >> 1) & 7;
//   BK 32 (64-byte rows, 4 per 256 bytes):  swz(r) = (r >> 2) & 3.
template <int BK>
__device__ __forceinline__ int swz(int r) {
  return BK == 64 ? (r >> 1) & 7 : (r >> 2) & 3;
}

// Wait until this wave has at most `after` stages of kLPW direct loads in flight (after <= MAXA;
// vector-memory loads complete in issue order).
template <int LPW, int MAXA>
__device__ __forceinline__ void wait_stages(int after) {
  static_assert(MAXA * LPW < 64, "vmcnt holds at most 63 loads");
  if constexpr (MAXA >= 3)
    if (after >= 3) return wait_vmcnt<3 * LPW>();
  if constexpr (MAXA >= 2)
    if (after >= 2) return wait_vmcnt<2 * LPW>();
  if constexpr (MAXA >= 1)
    if (after >= 1) return wait_vmcnt<LPW>();
  wait_vmcnt<0>();
}

template <int BM, int BN, int WM, int WN, int NST, int BK, bool PIPE>
__global__ __launch_bounds__(64 * WM * WN) void gemm_f16_nt_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ Cm, int M, int N, int K,
    int lda, int ldb, int ldc, int tiles_m, int tiles_n, int xcd_remap, int n_split, int nk_split,
    float* __restrict__ P) {
  using G = GemmCfg<BM, BN, WM, WN, NST, BK>;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];

  // XCD-major tile order: workgroup b runs on XCD b % 8; give XCD x a contiguous range of the
  // tile sequence. The sequence walks groups of kGroupM tile rows column by column, so the range an
  // XCD holds is a compact block (4 x 8 tiles for 32 tiles) whose A and B panels stay in its L2.
  // With a K split (n_split > 1) the sequence is the tile sequence once per K range: workgroup
  // g of the sequence computes K range g / ntiles of tile g % ntiles, so an XCD's block shares its
  // K range and reuses its panel slices the same way.
  int g = blockIdx.x;
  const int ntiles = tiles_m * tiles_n;
  if (xcd_remap) g = (g % 8) * (static_cast<int>(gridDim.x) / 8) + g / 8;
  const int ksp = g / ntiles;
  const int bid = g - ksp * ntiles;
  constexpr int kGroupM = 4;
  const int group = bid / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = bid - group * (kGroupM * tiles_n);
  const int tm = first_m + in_group % gsize, tn = in_group / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  const __amdgpu_buffer_rsrc_t ar = make_rsrc(A, static_cast<uint32_t>(M - 1) * lda * 2u + K * 2u);
  const __amdgpu_buffer_rsrc_t br = make_rsrc(B, static_cast<uint32_t>(N - 1) * ldb * 2u + K * 2u);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

  // Direct loads: instruction j of this wave fills row block b = wave + j * kWaves (kRowsPerInst
  // rows) of the stage; the lane for LDS slot s = lane % (BK / 8) of tile row
  // r = b * kRowsPerInst + lane / (BK / 8) fetches chunk s ^ swz(r). With an even number of waves
  // (or BK 32) swz(r) does not depend on j, so one per-lane offset per operand serves every
  // instruction: instruction j adds j row blocks of the wave stride, a uniform value that full
  // tiles pass as the load's scalar offset (no per-load vector arithmetic or registers).
  static_assert(BK == 32 || G::kWaves % 2 == 0, "the lane's chunk is the same for every row block");
  constexpr int kCpr = BK / 8;  // chunks per row
  constexpr int kRowsPerJ = G::kWaves * G::kRowsPerInst;
  const int r0 = wave * G::kRowsPerInst + lane / kCpr;
  const int chunk = (lane % kCpr) ^ swz<BK>(r0);
  const uint32_t a_lane = static_cast<uint32_t>(m0 + r0) * lda * 2u + chunk * 16u;
  const uint32_t b_lane = static_cast<uint32_t>(n0 + r0) * ldb * 2u + chunk * 16u;
  const uint32_t a_step = static_cast<uint32_t>(kRowsPerJ) * lda * 2u;
  const uint32_t b_step = static_cast<uint32_t>(kRowsPerJ) * ldb * 2u;
  const int a_left = M - m0 - r0, b_left = N - n0 - r0;  // in-range rows from this lane's first row
  const bool full_tile = m0 + BM <= M && n0 + BN <= N;
  unsigned char* junk = lds + NST * G::kStage;
  auto issue = [&](int kt, int stage) {
    const int k0 = kt * BK;
    unsigned char* sa = lds + stage * G::kStage;
    unsigned char* sb = sa + BM * G::kRow;
    auto dst = [&](unsigned char* base, int j, int blocks) {
      return wave + j * G::kWaves < blocks ? base + (wave + j * G::kWaves) * 1024 : junk;
    };
    if (full_tile && k0 + BK <= K) {
      const uint32_t ao = a_lane + k0 * 2u, bo = b_lane + k0 * 2u;
#pragma unroll
      for (int j = 0; j < G::kAI; ++j) load_lds16(ar, dst(sa, j, BM / G::kRowsPerInst), ao, j * a_step);
#pragma unroll
      for (int j = 0; j < G::kBI; ++j) load_lds16(br, dst(sb, j, BN / G::kRowsPerInst), bo, j * b_step);
    } else {
      // edge tile or ragged last K step: rows past M / N and k past K read out of range (zeros)
      const bool kin = k0 + 8 * chunk < K;
#pragma unroll
      for (int j = 0; j < G::kAI; ++j)
        load_lds16(ar, dst(sa, j, BM / G::kRowsPerInst),
                   kin && j * kRowsPerJ < a_left ? a_lane + j * a_step + k0 * 2u : kOOB);
#pragma unroll
      for (int j = 0; j < G::kBI; ++j)
        load_lds16(br, dst(sb, j, BN / G::kRowsPerInst),
                   kin && j * kRowsPerJ < b_left ? b_lane + j * b_step + k0 * 2u : kOOB);
    }
  };

  float16v acc[G::TM][G::TN];
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Operand reads: row r of the tile at chunk c lives at r * kRow + ((c ^ swz(r)) << 4); the rows
  // read start at multiples of 32, so swz(r) == swz(lane & 31).
  const int arow = wm * G::WTM + (lane & 31);
  const int brow = wn * G::WTN + (lane & 31);
  auto compute = [&](int stage) {
    const unsigned char* sa = lds + stage * G::kStage;
    const unsigned char* sb = sa + BM * G::kRow;
    // Every operand read of the stage first, then the MFMAs: the LDS latency is paid once per stage.
    half8 af[BK / 16][G::TM], bf[BK / 16][G::TN];
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int sw = ((2 * kk + (lane >> 5)) ^ swz<BK>(lane & 31)) << 4;
#pragma unroll
      for (int i = 0; i < G::TM; ++i) af[kk][i] = *reinterpret_cast<const half8*>(sa + (arow + 32 * i) * G::kRow + sw);
#pragma unroll
      for (int j = 0; j < G::TN; ++j) bf[kk][j] = *reinterpret_cast<const half8*>(sb + (brow + 32 * j) * G::kRow + sw);
    }
    // Keep the reads ahead of the MFMAs (measured: 2048x3072x8192 135.8 -> 117.6 us, the other
    // config-3 shapes equal or faster; without the barrier the scheduler interleaves them again).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk)
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kk][i], bf[kk][j], acc[i][j], 0, 0, 0);
  };

  // K steps [kt0, kt0 + nk) of this workgroup: all of them, or K range ksp of a K split.
  const int nk_all = (K + BK - 1) / BK;
  const int kt0 = n_split > 1 ? ksp * nk_split : 0;
  const int nk = n_split > 1 ? min(nk_split, nk_all - kt0) : nk_all;
  auto barrier = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  if constexpr (!PIPE) {
#pragma unroll
    for (int s = 0; s < NST - 1; ++s)
      if (s < nk) issue(kt0 + s, s);
    for (int kt = 0; kt < nk; ++kt) {
      // This wave's loads of stage kt are complete once at most `after` later stages are in flight.
      wait_stages<G::kLPW, NST - 2>(min(NST - 2, nk - 1 - kt));
      barrier();  // every wave's stage-kt loads landed; stage kt-1 is no longer read
      if (kt + NST - 1 < nk) issue(kt0 + kt + NST - 1, (kt + NST - 1) % NST);
      compute(kt % NST);
    }
  } else {
    // Software pipeline: the operands of each 16-k substep are read into one of two fragment sets
    // while the MFMAs of the previous substep run from the other, so the LDS reads overlap the matrix
    // core instead of preceding it. All NST stages are prefetched; the one barrier per K step sits
    // after this wave's reads of the step (and before its last MFMAs): past it every wave is done
    // reading stage kt, whose buffer then takes stage kt + NST, and stage kt + 1 has landed, whose
    // first substep is read while the last MFMAs of step kt run. The direct loads of stage kt + NST
    // are spread over the first KK - 1 substeps of step kt + 1, one between MFMAs, so the wait for the
    // load queue overlaps the matrix core; they are all issued before the next boundary, which keeps
    // its vmcnt count exact (and, with two stages, issues the stage it waits for).
    constexpr int KK = BK / 16;
    static_assert(KK % 2 == 0, "the last substep of a step uses fragment set 1");
    half8 fa[2][G::TM], fb[2][G::TN];
    auto read_sub = [&](int stage, int kk, int set) {
      const unsigned char* sa = lds + stage * G::kStage;
      const unsigned char* sb = sa + BM * G::kRow;
      const int sw = ((2 * kk + (lane >> 5)) ^ swz<BK>(lane & 31)) << 4;
#pragma unroll
      for (int i = 0; i < G::TM; ++i) fa[set][i] = *reinterpret_cast<const half8*>(sa + (arow + 32 * i) * G::kRow + sw);
#pragma unroll
      for (int j = 0; j < G::TN; ++j) fb[set][j] = *reinterpret_cast<const half8*>(sb + (brow + 32 * j) * G::kRow + sw);
    };
    // Loads of this workgroup's K step kl (K steps kt0 + kl, buffer kl % NST) given to substep
    // q < KK - 1: A loads [q kAI / (KK - 1), (q + 1) kAI / (KK - 1)), B loads likewise. kFast: a full
    // tile and a whole K step (offsets need no range checks).
    auto issue_part = [&](auto fast, int kl, int q) {
      constexpr bool kFast = decltype(fast)::value;
      const int k0 = (kt0 + kl) * BK;
      unsigned char* sa = lds + (kl % NST) * G::kStage;
      unsigned char* sb = sa + BM * G::kRow;
      auto dst = [&](unsigned char* base, int j, int blocks) {
        return wave + j * G::kWaves < blocks ? base + (wave + j * G::kWaves) * 1024 : junk;
      };
      const bool kin = kFast || k0 + 8 * chunk < K;
#pragma unroll
      for (int j = q * G::kAI / (KK - 1); j < (q + 1) * G::kAI / (KK - 1); ++j) {
        if constexpr (kFast) load_lds16(ar, dst(sa, j, BM / G::kRowsPerInst), a_lane + k0 * 2u, j * a_step);
        else load_lds16(ar, dst(sa, j, BM / G::kRowsPerInst), kin && j * kRowsPerJ < a_left ? a_lane + j * a_step + k0 * 2u : kOOB);
      }
#pragma unroll
      for (int j = q * G::kBI / (KK - 1); j < (q + 1) * G::kBI / (KK - 1); ++j) {
        if constexpr (kFast) load_lds16(br, dst(sb, j, BN / G::kRowsPerInst), b_lane + k0 * 2u, j * b_step);
        else load_lds16(br, dst(sb, j, BN / G::kRowsPerInst), kin && j * kRowsPerJ < b_left ? b_lane + j * b_step + k0 * 2u : kOOB);
      }
    };
    // MFMAs of one substep with that substep's share of the loads interleaved (one load after each
    // of the first MFMAs).
    auto mfma_sub = [&](int set, auto fast, int kl, int q) {
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
      if (kl >= 0) issue_part(fast, kl, q);
      constexpr int kLoads = (G::kAI + G::kBI + KK - 2) / (KK - 1);
#pragma unroll
      for (int l = 0; l < kLoads && l < G::TM * G::TN; ++l) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one vector-memory load
      }
      __builtin_amdgcn_sched_group_barrier(0x008, G::TM * G::TN, 0);
    };
    auto main_loop = [&](auto fast) {
#pragma unroll
      for (int s = 0; s < NST; ++s)
        if (s < nk) {
#pragma unroll
          for (int q = 0; q < KK - 1; ++q) issue_part(std::false_type{}, s, q);
        }
      wait_stages<G::kLPW, NST - 1>(min(NST - 1, nk - 1));
      barrier();
      read_sub(0, 0, 0);
      for (int kt = 0; kt < nk; ++kt) {
        const int st = kt % NST;
        // stage kt - 1 + NST goes into the buffer freed at the last boundary (none in step 0)
        const int kl = kt >= 1 && kt - 1 + NST < nk ? kt - 1 + NST : -1;
#pragma unroll
        for (int kk = 0; kk < KK - 1; ++kk) {
          read_sub(st, kk + 1, (kk + 1) & 1);
          __builtin_amdgcn_sched_barrier(0);
          mfma_sub(kk & 1, fast, kl, kk);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (kt + 1 < nk) {
          // this wave's stage kt + 1 loads landed (stages up to kt - 1 + NST issued)
          wait_stages<G::kLPW, NST - 2>(min(NST - 2, nk - kt - 2));
          __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of stage kt done
          barrier();
          read_sub((kt + 1) % NST, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        mfma_sub((KK - 1) & 1, fast, -1, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // the prologue's loads take the checked path (they are few); the loop's are checked only for
    // edge tiles and a ragged K
    if (full_tile && K % BK == 0) main_loop(std::true_type{});
    else main_loop(std::false_type{});
  }

  // Epilogue (lane l holds column l % 32 of each 32x32 tile): fp16 stores, or with a K split the
  // fp32 partial of K range ksp into P[ksp][M][N].
  float* __restrict__ Pk = P + static_cast<int64_t>(ksp) * M * N;
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * G::WTM + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
        const int col = n0 + wn * G::WTN + j * 32 + (lane & 31);
        if (row < M && col < N) {
          if (n_split > 1) Pk[static_cast<int64_t>(row) * N + col] = acc[i][j][e];
          else Cm[static_cast<int64_t>(row) * ldc + col] = float_to_half_bits(acc[i][j][e]);
        }
      }
}

// C = fp16(sum over s of P[s]) for a K split: four consecutive outputs per thread (N % 4 == 0), the
// partials added in the fixed order s = 0, 1, ..., n_split - 1, so results do not depend on which
// workgroup finished first. kPacked: one 8-byte store per thread (ldc % 4 == 0, C 8-byte aligned).
template <bool kPacked>
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(const float* __restrict__ P, uint16_t* __restrict__ Cm,
                                                                int M, int N, int ldc, int n_split) {
  const int64_t mn = static_cast<int64_t>(M) * N;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= mn) return;
  const float4 v = sum_partials4(reinterpret_cast<const float4*>(P + i), mn / 4, n_split);
  const int row = static_cast<int>(i / N), col = static_cast<int>(i - static_cast<int64_t>(row) * N);
  uint16_t* c = Cm + static_cast<int64_t>(row) * ldc + col;
  if (kPacked) {
    *reinterpret_cast<uint2*>(c) = make_uint2(float_to_half_bits(v.x) | (uint32_t{float_to_half_bits(v.y)} << 16),
                                              float_to_half_bits(v.z) | (uint32_t{float_to_half_bits(v.w)} << 16));
  } else {
    c[0] = float_to_half_bits(v.x);
    c[1] = float_to_half_bits(v.y);
    c[2] = float_to_half_bits(v.z);
    c[3] = float_to_half_bits(v.w);
  }
}

// fp16 GEMV for M == 1 (the gemv_nt shape): each wave owns kRows rows; its 64 lanes cover K in
// 16-byte chunks (8 k), kKc chunks per lane per pass, so one pass spans 512 * kKc k. Every load of a
// pass (x and the rows) is issued before any use; v_dot2_f32_f16 with fp32 accumulation, then a
// reduction over the wave. Rows past N and k past K read out of range (zeros). Memory bound.
// fp16 GEMV (M == 1): C[0, n] = sum_k A[0, k] B[n, k]. kSplit waves share each row, wave q taking the
// q-th contiguous part of every K pass; lane l of a wave reads 16 consecutive bytes of a row per load,
// so one load instruction covers 1 KB of it. All loads of a pass are issued before use; the wave sums
// are combined through LDS in wave order.
template <int kKc, int kWaves, int kSplit>
__global__ __launch_bounds__(64 * kWaves) void gemv_f16_kernel(const uint16_t* __restrict__ a,
                                                               const uint16_t* __restrict__ B,
                                                               uint16_t* __restrict__ c, int N, int K, int ldb) {
  typedef _Float16 half2v __attribute__((ext_vector_type(2)));
  static_assert(kWaves % kSplit == 0, "whole rows per workgroup");
  __shared__ float red[kWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int part = wave % kSplit;
  const int row = blockIdx.x * (kWaves / kSplit) + wave / kSplit;
  const __amdgpu_buffer_rsrc_t br = make_rsrc(B, static_cast<uint32_t>(N - 1) * ldb * 2u + K * 2u);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a, K * 2u);
  float acc = 0.0f;
  constexpr int kPass = 512 * kKc * kSplit;  // k per pass over all parts
  for (int kb = 0; kb < K; kb += kPass) {
    uint4 xv[kKc], wv[kKc];
#pragma unroll
    for (int i = 0; i < kKc; ++i) {
      const int k = kb + ((part * kKc + i) * 64 + lane) * 8;
      xv[i] = buf_load16(xr, k < K ? k * 2u : kOOB);
      wv[i] = buf_load16(br, k < K && row < N ? (static_cast<uint32_t>(row) * ldb + k) * 2u : kOOB);
    }
#pragma unroll
    for (int i = 0; i < kKc; ++i) {
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, wv[i].x), __builtin_bit_cast(half2v, xv[i].x), acc, false);
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, wv[i].y), __builtin_bit_cast(half2v, xv[i].y), acc, false);
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, wv[i].z), __builtin_bit_cast(half2v, xv[i].z), acc, false);
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, wv[i].w), __builtin_bit_cast(half2v, xv[i].w), acc, false);
    }
  }
  const float v = group_sum<64>(acc);
  if constexpr (kSplit == 1) {
    if (lane == 0 && row < N) c[row] = float_to_half_bits(v);
  } else {
    if (lane == 0) red[wave] = v;
    __syncthreads();
    if (part == 0 && lane == 0 && row < N) {
      float t = red[wave];
#pragma unroll
      for (int q = 1; q < kSplit; ++q) t += red[wave + q];
      c[row] = float_to_half_bits(t);
    }
  }
}

struct TileCfg {
  int bm, bn, wgm, wgn, nst, bk;
  bool sp = false;  // software-pipelined substeps (gemm_f16_nt_kernel<..., true>)
};
// Explicit CDNA4 tile list (index stable for gemm_f16_nt_cfg / the Q4_DBG_GEMM_TILE override).
constexpr TileCfg kTiles[] = {
    {256, 256, 2, 4, 2, 64},        // 0: 8 waves of 128x64, 2 stages of K 64 (128 KB LDS)
    {128, 128, 2, 2, 2, 64},        // 1: 4 waves of 64x64, 2 stages (64 KB, two workgroups per CU)
    {128, 128, 2, 2, 4, 64, true},  // 2: 4 waves of 64x64, 4 stages (128 KB), pipelined substeps
    {64, 96, 2, 3, 4, 64, true},    // 3: 6 waves of 32x32, 4 stages (81 KB), pipelined: M = 256, N = 5120 on 216 CUs
    {128, 64, 2, 2, 4, 64},         // 4: 4 waves of 64x32, 4 stages (96 KB)
    {64, 64, 2, 2, 4, 64},          // 5: 4 waves of 32x32, 4 stages (64 KB)
    {128, 160, 2, 5, 4, 64, true},  // 6: 10 waves of 64x32, 4 stages (145 KB), pipelined: M = 1024, N = 5120
                                    //    in exactly 256 tiles
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

using GemmFn = void (*)(const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, int, int, int, int, int,
                        int, float*);

template <int I>
constexpr GemmFn gemm_fn() {
  constexpr TileCfg t = kTiles[I];
  return gemm_f16_nt_kernel<t.bm, t.bn, t.wgm, t.wgn, t.nst, t.bk, t.sp>;
}
template <int I>
constexpr size_t gemm_lds() {
  constexpr TileCfg t = kTiles[I];
  return GemmCfg<t.bm, t.bn, t.wgm, t.wgn, t.nst, t.bk>::kLds;
}
constexpr GemmFn kGemmFns[] = {gemm_fn<0>(), gemm_fn<1>(), gemm_fn<2>(), gemm_fn<3>(),
                               gemm_fn<4>(), gemm_fn<5>(), gemm_fn<6>()};
constexpr size_t kGemmLds[] = {gemm_lds<0>(), gemm_lds<1>(), gemm_lds<2>(), gemm_lds<3>(),
                               gemm_lds<4>(), gemm_lds<5>(), gemm_lds<6>()};
static_assert(sizeof(kGemmFns) / sizeof(kGemmFns[0]) == kNumTiles, "one kernel per tile entry");

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Fixed rule, from sweeps of every entry (and K splits of 1-8) over the config-3 shapes on one
// MI355X (graph replays, weights rotated past the MALL):
//   * M >= 512: 256x256 when that alone fills the 256 CUs (4096^3: 1.05 PFLOP/s); else the pipelined
//     128x160 entry when its tiles make one round of 240-256 workgroups (1024x5120x3072: 256 tiles,
//     46.0 -> 41.7 us against 128x128); else 128x128 with two workgroups per CU (2048x3072x8192:
//     117 us; 128x160 there gives 320 tiles, 179 us, and 128x192 256 tiles, 129 us); K splits only
//     lost here;
//   * M < 512 with a workspace (gemm_f16_nt_ws): the pipelined 128x128 entry with K split so the
//     tiles times the split come closest to 256 workgroups (256x5120x3072: 80 tiles x 3, 23.1 us;
//     256x3072x8192: 48 x 5, 29 us; 256x16384x3072: 256 x 1, 40 us);
//   * M < 512 without one: the largest 4-stage tile that still gives >= 160 workgroups (pipelined
//     128x128, then 64x96 where it fills the CUs in one round, then 128x64, 64x64).
// Measured and not in the list: whole-256-row tiles (256x64, 64x256, 256x32), 4 waves of 128x128 on
// 256x256 tiles (2 stages of K 64, or 4-5 stages of K 32) and of 64x128 / 128x64, 8 waves on 256x128
// and 128x256, K steps of 128, the plain schedule on the 4-stage 128x128 and 64x96 tiles (the
// pipelined ones replace them), the pipelined schedule on the 8-wave 256x256 and the two-workgroup
// 128x128 entries, and a ping-pong schedule of two 4-wave groups on 256x256: each equal or slower on
// every config-3 shape.
// Problems under 4 GFLOP (under ~2 us of matrix-core time at the dense peak) are set by latency and
// by how many CUs stream at once, not by the tile's operand reuse.
bool small_problem(int64_t M, int64_t N, int64_t K) { return 2.0 * M * N * K < 4e9; }

int choose_tile(int64_t M, int64_t N, int64_t K, bool split_ok) {
  const int ov = debug_override(Q4_DBG_GEMM_TILE);
  if (ov >= 0 && ov < kNumTiles) return ov;
  (void)split_ok;
  // small problems (the reference's S1-S6 and S8): 64x64, the K split below (swept on every entry and
  // splits of 1-32: S1 1024^3 15.3 -> 9.0 us, S3 15.3 -> 8.3, S5 19.5 -> 12.0, S8 12.7 -> 7.2)
  if (small_problem(M, N, K)) return 5;
  auto tiles = [&](int i) { return cdiv(M, kTiles[i].bm) * cdiv(N, kTiles[i].bn); };
  if (M >= 512) return tiles(0) >= 256 ? 0 : (tiles(6) >= 240 && tiles(6) <= 256 ? 6 : 1);
  if (split_ok && N % 4 == 0) return 2;
  if (tiles(2) >= 160) return 2;
  // 64x96 when it covers the CUs in one round (256x5120x3072: 160 workgroups of 128x64 -> 216 of 64x96,
  // 17% fewer bytes per CU, 27.6 -> 23.6 us)
  if (tiles(3) >= 160 && tiles(3) <= 256) return 3;
  for (int i : {4, 5})
    if (tiles(i) >= 160) return i;
  return 5;
}

}  // namespace

// K split of tile entry ti: n_split K ranges of nk_split K steps each (the last may be shorter, none
// empty); {1, 0} for no split. Only when N % 4 == 0 (the reduce kernel's four-column rows): M < 512
// takes the split that brings the workgroups closest to 256 without exceeding it, each range at least
// four K steps. The Q4_DBG_GEMM_SPLIT override forces a split count for sweeps.
struct GemmSplit {
  int n_split, nk_split;
};
GemmSplit gemm_split_plan(int64_t M, int64_t N, int64_t K, int ti) {
  GemmSplit p{1, 0};
  const TileCfg& t = kTiles[ti];
  if (N % 4 || M <= 1) return p;
  const int nk = static_cast<int>(cdiv(K, t.bk));
  const int64_t tiles = cdiv(M, t.bm) * cdiv(N, t.bn);
  int want = M < 512 ? static_cast<int>(std::min<int64_t>(256 / tiles, nk / 4)) : 1;
  // small problems: about 256 workgroups (256 / tiles rounded), each K range at least 8 K steps
  if (small_problem(M, N, K)) want = static_cast<int>(std::min<int64_t>((512 / tiles + 1) / 2, nk / 8));
  if (debug_set(Q4_DBG_GEMM_SPLIT)) want = debug_override(Q4_DBG_GEMM_SPLIT);
  if (want <= 1 || nk < 2) return p;
  const int nk_s = static_cast<int>(cdiv(nk, std::min(want, nk)));
  const int S = static_cast<int>(cdiv(nk, nk_s));
  if (S < 2) return p;
  p.n_split = S;
  p.nk_split = nk_s;
  return p;
}

size_t gemm_split_bytes(int64_t M, int64_t N, int64_t K, int ti) {
  const GemmSplit sp = gemm_split_plan(M, N, K, ti);
  return sp.n_split > 1 ? static_cast<size_t>(sp.n_split) * M * N * sizeof(float) : 0;
}

int gemm_f16_launch(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                    int64_t ldb, int64_t ldc, int cfg, hipStream_t st, float* part = nullptr, size_t part_bytes = 0) {
  if (M == 1 && cfg < 0) {
    // One row per wave, 4 waves per workgroup; rows longer than 3072 are split over two waves (passes
    // of up to 4096 k per row). Measured on one MI355X, graph replays over rotating B copies, against
    // two rows per wave in 4-wave workgroups: 1x3072x3072 5.79 -> 5.22 us, 1x4096x4096 8.96 -> 7.79 us
    // (7.93 without the split), 1x5120x3072 8.03 -> 7.36 us. Two rows per wave in 6- or 8-wave
    // workgroups and one row per wave in 6- or 8-wave workgroups measured between the two.
    constexpr int kWaves = 4;
    const int split = K > 3072 ? 2 : 1;
    const unsigned grid = static_cast<unsigned>(cdiv(N, kWaves / split));
    auto go = [&](auto kc) {
      constexpr int KC = decltype(kc)::value;
      if (split == 2)
        hipLaunchKernelGGL((gemv_f16_kernel<KC / 2, kWaves, 2>), dim3(grid), dim3(64 * kWaves), 0, st, A, B, C, (int)N,
                           (int)K, (int)ldb);
      else
        hipLaunchKernelGGL((gemv_f16_kernel<KC, kWaves, 1>), dim3(grid), dim3(64 * kWaves), 0, st, A, B, C, (int)N,
                           (int)K, (int)ldb);
    };
    if (K <= 1024) go(std::integral_constant<int, 2>{});
    else if (K <= 2048) go(std::integral_constant<int, 4>{});
    else if (K <= 3072) go(std::integral_constant<int, 6>{});
    else go(std::integral_constant<int, 8>{});
    return launch_status();
  }
  const int ti = cfg >= 0 && cfg < kNumTiles ? cfg : choose_tile(M, N, K, part != nullptr);
  const TileCfg& t = kTiles[ti];
  const int tiles_m = static_cast<int>(cdiv(M, t.bm)), tiles_n = static_cast<int>(cdiv(N, t.bn));
  const int ntiles = tiles_m * tiles_n;
  const size_t lds = kGemmLds[ti];
  if (lds > 64 * 1024) {
    Q4_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kGemmFns[ti]),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  }
  GemmSplit sp{1, 0};
  if (part) {
    sp = gemm_split_plan(M, N, K, ti);
    if (sp.n_split > 1 && (part_bytes < static_cast<size_t>(sp.n_split) * M * N * sizeof(float) || !aligned(part, 16)))
      return Q4_ERR_WORKSPACE;
  }
  const int grid = ntiles * sp.n_split;
  const int remap = (grid % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL(kGemmFns[ti], dim3(grid, 1), dim3(64 * t.wgm * t.wgn), lds, st, A, B, C, (int)M, (int)N, (int)K,
                     (int)lda, (int)ldb, (int)ldc, tiles_m, tiles_n, remap, sp.n_split, sp.nk_split, part);
  if (int e = launch_status()) return e;
  if (sp.n_split > 1) {
    const unsigned blocks = static_cast<unsigned>(cdiv(M * N / 4, 256));
    if (ldc % 4 == 0 && aligned(C, 8))
      hipLaunchKernelGGL(gemm_split_reduce_kernel<true>, dim3(blocks), dim3(256), 0, st, part, C, (int)M, (int)N,
                         (int)ldc, sp.n_split);
    else
      hipLaunchKernelGGL(gemm_split_reduce_kernel<false>, dim3(blocks), dim3(256), 0, st, part, C, (int)M, (int)N,
                         (int)ldc, sp.n_split);
    return launch_status();
  }
  return Q4_OK;
}

// Workspace bytes gemm_f16_nt_ws uses for this shape (0: no K split).
size_t gemm_f16_ws_bytes(int64_t M, int64_t N, int64_t K) {
  if (M == 1) return 0;
  return gemm_split_bytes(M, N, K, choose_tile(M, N, K, true));
}

int gemm_f16_num_tiles() { return kNumTiles; }

int gemm_f16_tile_info(int i, int* out) {
  if (i < 0 || i >= kNumTiles) return Q4_ERR_RANGE;
  const TileCfg& t = kTiles[i];
  const int v[7] = {t.bm, t.bn, t.wgm, t.wgn, t.nst, t.bk, t.sp ? 1 : 0};
  for (int j = 0; j < 7; ++j) out[j] = v[j];
  return Q4_OK;
}

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

extern "C" int gemm_f16_nt_ws_bytes(int64_t M, int64_t N, int64_t K, size_t* bytes) {
  if (!bytes) return Q4_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return Q4_ERR_SHAPE;
  *bytes = q4::gemm_f16_ws_bytes(M, N, K);
  return Q4_OK;
}

extern "C" int gemm_f16_nt_ws(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t M, int64_t N, int64_t K,
                              int64_t lda, int64_t ldb, int64_t ldc, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (int st = gemm_args(A, B, C, M, N, K, lda, ldb, ldc)) return st;
  if (M > 1 && !workspace && q4::gemm_f16_ws_bytes(M, N, K) > 0) return Q4_ERR_WORKSPACE;
  return q4::gemm_f16_launch(A, B, C, M, N, K, lda, ldb, ldc, -1, q4::as_stream(stream),
                             static_cast<float*>(workspace), workspace_bytes);
}

extern "C" int gemm_f16_nt_cfg(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t M, int64_t N, int64_t K,
                               int64_t lda, int64_t ldb, int64_t ldc, int cfg, int split, void* stream) {
  (void)split;
  if (int st = gemm_args(A, B, C, M, N, K, lda, ldb, ldc)) return st;
  if (cfg >= q4::gemm_f16_num_tiles()) return Q4_ERR_RANGE;
  return q4::gemm_f16_launch(A, B, C, M, N, K, lda, ldb, ldc, cfg, q4::as_stream(stream));
}

extern "C" int gemm_f16_num_configs(void) { return q4::gemm_f16_num_tiles(); }

extern "C" int gemm_f16_config_info(int cfg, int* info) {
  if (!info) return Q4_ERR_NULL;
  return q4::gemm_f16_tile_info(cfg, info);
}
