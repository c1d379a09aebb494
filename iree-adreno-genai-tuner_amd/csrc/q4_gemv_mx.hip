// Decode int4 GEMV with fp32 activations on the gfx950 int8 matrix cores.
//
// Computes the fp32 model path of QLinear._gemv_fused / QLinear.forward at M == 1
// (scripts/llm/llama_q4.py:69-90):
//   y[n] = residual[n] + sum_g scale[n, g] * sum_{k in g} (nib[n, k] - 8) * x[k]
// with the same fused prologue (rms_norm) and paired-row epilogues (SwiGLU, RoPE + KV-cache write)
// as the VALU kernel in q4_gemv.hip, which it replaces for these shapes.
//
// Why matrix cores for a memory-bound GEMV: with fp32 x, decoding a nibble and multiplying it on
// the vector ALU costs about 2.3 instructions (byte convert + FMA + masks), which for a whole
// Llama-3.2-3B token is as much VALU time as the HBM time of its weights. Here:
//   * x is made exact integers per quantization group g: X = rint(x * 2^sh_g), |X| <= 2^30, with
//     sh_g from the group's largest |x| (the rounding error is below 2^-30 of that element, far
//     under fp32 accumulation error). X is split into four signed base-256 digits ("limbs") b_j,
//     X = sum_j b_j 2^(8j), each in [-128, 127].
//   * The nibbles enter v_mfma_i32_16x16x64_i8 unchanged as unsigned bytes (word & 0x0F0F0F0F and
//     (word >> 4) & 0x0F0F0F0F: three instructions per 8 nibbles), the limbs as the other operand.
//     The 16 output columns hold 4 quantization groups x 4 limbs: in each MFMA a lane group's 16 k
//     values belong to one group, and the B operand is non-zero only in the 4 columns of that
//     group's slot. One int32 accumulator therefore collects, exactly, per row and per
//     (group, limb): D = sum_{k in g} nib * b_j.
//   * Per group the exact correction D - 8 * S_j (S_j = sum_{k in g} b_j) gives
//     sum (nib - 8) b_j; it is converted to fp32 (exact, |D| < 2^24), multiplied by
//     2^(8j - sh_g) (exact) and by the fp16 group scale, and accumulated in fp32.
//   So the products are exact and only the fp32 sums round, as in F.linear.
//
// Layout of one MFMA (lane l: row l % 16, lane group b = l / 16, column c = l % 16):
//   A (weights) : lane l loads 16 bytes = words 4b..4b+3 of a 128-k "segment" of its row (one
//                 16-byte load per lane covers 16 rows x 64 contiguous bytes); MFMA half h uses
//                 words 4b+2h, 4b+2h+1 as {lo(w0), hi(w0), lo(w1), hi(w1)}.
//   B (x limbs) : 16-k block beta = 8*segment + 2b + h; prepared once per workgroup in LDS in the
//                 same in-lane byte order (byte i of dword d <-> k = 8(d/2) + 2i + d%2 of the block).
//   D           : lane l holds rows 4b + t (t = 0..3) of column c = 4 * slot + limb.
// A "tile" is 4 consecutive groups (4G k values); its MFMAs share one accumulator, after which the
// per-group epilogue above runs. A workgroup owns one 16-row block (or, for very tall matrices, a
// grid-stride list of them); its waves split the tiles of the block along K and combine their row
// sums through LDS in a fixed order, so results are deterministic.
//
// Global reads are raw buffer loads: rows past N, k past K and groups past K/G read out of range
// and return zeros without memory traffic, so the load stream has no branches.
#include "q4_common.h"
#include "q4_internal.h"

#include <array>
#include <cstdlib>
#include <utility>

namespace q4 {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kOOB = 0x80000000u;  // past every buffer resource built here
constexpr int kBufferFlags = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), kBufferFlags);
}

__device__ __forceinline__ i32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Weight stream: read once per launch, marked nontemporal (cache policy bit 1).
__device__ __forceinline__ i32x4 load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
}

__device__ __forceinline__ uint16_t load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 2);
}

__device__ __forceinline__ uint2 load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
  const i32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 2);
  return make_uint2(static_cast<uint32_t>(v.x), static_cast<uint32_t>(v.y));
}

constexpr int kProNone = 0, kProNorm = 1;
constexpr int kEpiNone = 0, kEpiSwiglu = 1, kEpiRope = 2;

using MxEpi = GemvEpi;

// argmax order of llama_ops.hip: the first index of the maximum, NaN above every number
__device__ __forceinline__ bool arg_better(float a, int32_t ia, float b, int32_t ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
#pragma clang fp contract(off)
  const float e = expf(-g);
  const float den = 1.0f + e;
  const float sg = g / den;
  return sg * u;
}

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

// Sum of squares of 16 fp32 values in a fixed order (the rms_norm prologue).
__device__ __forceinline__ float sumsq16(const float* v) {
#pragma clang fp contract(off)
  float s[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = v[2 * i] * v[2 * i];
    const float b = v[2 * i + 1] * v[2 * i + 1];
    s[i] = a + b;
  }
  return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

// Reductions over aligned groups of `width` lanes (2, 4, 8 or 16) with DPP moves: xor-1 and xor-2
// quad permutes, then the half-row and row mirrors. Every lane of a group ends with the group's
// result, and all lanes combine the same values, so the result is identical across the group.
template <int ctrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xf, 0xf, false));
}
template <int ctrl>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, ctrl, 0xf, 0xf, false);
}
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E, kRowHalfMirror = 0x141, kRowMirror = 0x140;

template <int width>
__device__ __forceinline__ float dpp_sum(float v) {
  if constexpr (width >= 2) v += dpp_f<kQuadXor1>(v);
  if constexpr (width >= 4) v += dpp_f<kQuadXor2>(v);
  if constexpr (width >= 8) v += dpp_f<kRowHalfMirror>(v);
  if constexpr (width >= 16) v += dpp_f<kRowMirror>(v);
  return v;
}
template <int width>
__device__ __forceinline__ int dpp_isum(int v) {
  if constexpr (width >= 2) v += dpp_i<kQuadXor1>(v);
  if constexpr (width >= 4) v += dpp_i<kQuadXor2>(v);
  if constexpr (width >= 8) v += dpp_i<kRowHalfMirror>(v);
  if constexpr (width >= 16) v += dpp_i<kRowMirror>(v);
  return v;
}
template <int width>
__device__ __forceinline__ float dpp_max(float v) {
  if constexpr (width >= 2) v = fmaxf(v, dpp_f<kQuadXor1>(v));
  if constexpr (width >= 4) v = fmaxf(v, dpp_f<kQuadXor2>(v));
  if constexpr (width >= 8) v = fmaxf(v, dpp_f<kRowHalfMirror>(v));
  if constexpr (width >= 16) v = fmaxf(v, dpp_f<kRowMirror>(v));
  return v;
}

// Physical weight row of virtual row v of row block rb (16 virtual rows per block; RPB of them
// used). Pair epilogues put row p of the pair set in virtual row i < 8 and its partner in i + 8.
// Returns -1 for rows that do not exist.
template <int EPI, int RPB>
__device__ __forceinline__ int phys_row(int rb, int v, int N, const MxEpi& ea) {
  if constexpr (EPI == kEpiNone) {
    const int r = rb * RPB + v;
    return (v < RPB && r < N) ? r : -1;
  } else {
    const int p = rb * 8 + (v & 7);
    if (p >= (N >> 1)) return -1;
    if constexpr (EPI == kEpiSwiglu) {
      return p + (v >= 8 ? (N >> 1) : 0);
    } else {
      const int hsh = __builtin_ctz(static_cast<unsigned>(ea.hd)) - 1;  // head_dim / 2 is a power of two
      const int hh = 1 << hsh;
      const int head = p >> hsh;
      return head * ea.hd + (p & (hh - 1)) + (v >= 8 ? hh : 0);
    }
  }
}

// LDS layout of the workgroup (bytes):
//   Bc   [nblk][4] x 16   x limbs per 16-k block and limb, MFMA byte order
//   zero 16               zeros for lanes whose column is not this block's slot
//   Sg   [ngrp][4] int32  per-group limb sums S_j
//   P2   [ngrp] float     2^-sh_g
//   part [2][W][16] float row partials of the waves (double buffered)
//   red  [W] float        sums of squares (rms_norm)
struct MxLds {
  uint32_t bc, zero, sg, p2, part, red, total;
};

__host__ __device__ inline MxLds mx_lds(int nblk, int ngrp, int W) {
  MxLds l;
  l.bc = 0;
  l.zero = l.bc + nblk * 64;
  l.sg = l.zero + 16;
  l.p2 = l.sg + ngrp * 16;
  l.part = l.p2 + ((ngrp * 4 + 15) & ~15);
  l.red = l.part + 2 * W * 16 * 4;
  l.total = l.red + ((W * 4 + 15) & ~15);
  return l;
}

// Signed base-256 digits of X (|X| <= 2^30) as the four bytes of one word: with
// Y = X + 0x808080, digit j < 3 is byte j of Y minus 128 and digit 3 is the top byte, so
// X = sum_j digit_j 2^(8j) exactly, every digit in [-128, 127]; xor-ing 0x80 into bytes 0..2 turns
// "byte - 128" into the digit's two's-complement byte.
__device__ __forceinline__ uint32_t limb_bytes(int X) {
  return (static_cast<uint32_t>(X) + 0x808080u) ^ 0x808080u;
}

// Transposes 4 words of 4 bytes: out[j] = (a_j, b_j, c_j, d_j) (byte 0 first).
__device__ __forceinline__ void transpose4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t out[4]) {
  // v_perm_b32 selects bytes of {src0, src1}: selector byte s < 4 -> src1 byte s, 4..7 -> src0 byte s-4.
  const uint32_t p = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
  const uint32_t q = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
  const uint32_t r = __builtin_amdgcn_perm(d, c, 0x05010400u);  // c0 d0 c1 d1
  const uint32_t t = __builtin_amdgcn_perm(d, c, 0x07030602u);  // c2 d2 c3 d3
  out[0] = __builtin_amdgcn_perm(r, p, 0x05040100u);            // a0 b0 c0 d0
  out[1] = __builtin_amdgcn_perm(r, p, 0x07060302u);            // a1 b1 c1 d1
  out[2] = __builtin_amdgcn_perm(t, q, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(t, q, 0x07060302u);
}

// G: group size (32 or 128). A workgroup owns RBW row blocks at once; WPB waves work on each row
// block, splitting its tiles along K (at most TPW tiles per wave), so the workgroup has
// W = RBW * WPB waves and converts x once for all of them. MULTI: grid-stride over groups of RBW
// row blocks with the next group's loads in flight. RPB: used rows per 16-row block (16, or 8 to
// spread a short matrix over more workgroups). DNP / DP: s_sleep before the first weight loads of the
// waves without / with x blocks (below).
template <int G, int RBW, int WPB, int TPW, bool MULTI, int PRO, int EPI, int RPB, bool TL = false, int DNP = 0,
          int DP = 0>
__global__ __launch_bounds__(RBW * WPB * 64) void q4_gemv_mx_kernel(
    const int32_t* __restrict__ qw, const uint16_t* __restrict__ scales, const float* __restrict__ x,
    const float* __restrict__ aux, float eps, float* y, const float* residual, int N, int K, int n_tiles,
    int n_rb, MxEpi ea) {
  constexpr int W = RBW * WPB;
  static_assert(EPI == kEpiNone || RPB == 16, "paired epilogues use full 16-row blocks");
  constexpr int kSegPerTile = (4 * G) / 128;  // 128-k segments per tile of 4 groups
  static_assert((4 * G) % 128 == 0, "group must be a multiple of 32");
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int ngrp = n_tiles * 4;
  const int nblk = n_tiles * (4 * G / 16);  // 16-k blocks covered by the tiles (K padded)
  const MxLds L = mx_lds(nblk, ngrp, W);
  uint4* Bc = reinterpret_cast<uint4*>(lds + L.bc);
  int* Sg = reinterpret_cast<int*>(lds + L.sg);
  float* P2 = reinterpret_cast<float*>(lds + L.p2);
  float* part = reinterpret_cast<float*>(lds + L.part);
  float* red = reinterpret_cast<float*>(lds + L.red);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rbl = wave / WPB, wp = wave - rbl * WPB;  // row block within the group, K part
  const int b = lane >> 4, c = lane & 15;
  const int q = c >> 2, j = c & 3;
  const int kg = K / G;  // real groups

  // TL: the weights are in the T16 layout (q4_t16_pack): 16-row tiles in this kernel's virtual row
  // order, 1 KB per (tile, 128-k segment), and scales [tile][4-group tile][group slot][16 rows].
  const int nseg = n_tiles * kSegPerTile;
  const int n_t16 = EPI == kEpiNone ? (N + 15) / 16 : ((N >> 1) + 7) / 8;
  const __amdgpu_buffer_rsrc_t wres =
      TL ? rsrc(qw, static_cast<uint32_t>(n_t16) * nseg * 1024u)
         : rsrc(qw, static_cast<uint32_t>(N) * static_cast<uint32_t>(K / 2));
  const __amdgpu_buffer_rsrc_t sres =
      TL ? rsrc(scales, static_cast<uint32_t>(n_t16) * n_tiles * 128u) : rsrc(scales, static_cast<uint32_t>(N) * kg * 2u);

  // ---- weight and scale loads of one row block (this wave's tiles) ----
  // Every wave owns exactly TPW tiles (the host only picks entries with n_tiles == WPB * TPW), so
  // the load stream has no conditions on the tile.
  const int t0 = wp * TPW;
  struct Regs {
    i32x4 a[TPW][kSegPerTile];
    uint16_t s[TPW][4];
  };
  const uint32_t row_bytes = static_cast<uint32_t>(K / 2);
  auto issue = [&](int rb, Regs& R) {
    if constexpr (TL) {
      // virtual row of this lane's weights (row c of the RPB used rows of block rb) and of its first
      // scale row (4b); rows past the tiles read out of range (zeros, no traffic)
      const bool live = rb < n_rb;
      const int vr = rb * RPB + c, vs = rb * RPB + 4 * b;
      const bool rok = live && c < RPB && (EPI != kEpiNone || vr < N);
      const bool sok = live && 4 * b < RPB;
      const uint32_t abase = rok ? (static_cast<uint32_t>(vr >> 4) * nseg) * 1024u + (vr & 15) * 64u + 16u * b : kOOB;
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const int T = t0 + i;
#pragma unroll
        for (int sg = 0; sg < kSegPerTile; ++sg) {
          const int seg = T * kSegPerTile + sg;
          const bool ok = seg * 128 + 32 * b < K;
          R.a[i][sg] = load16_nt(wres, ok && abase != kOOB ? abase + 1024u * seg : kOOB);
        }
        const uint2 sv = load8(
            sres, sok ? ((static_cast<uint32_t>(vs >> 4) * n_tiles + T) * 64u + q * 16u + (vs & 15)) * 2u : kOOB);
        R.s[i][0] = static_cast<uint16_t>(sv.x);
        R.s[i][1] = static_cast<uint16_t>(sv.x >> 16);
        R.s[i][2] = static_cast<uint16_t>(sv.y);
        R.s[i][3] = static_cast<uint16_t>(sv.y >> 16);
      }
      return;
    }
    // byte offset of this lane's first weight chunk and of its 4 scale rows (kOOB: no such row)
    const int arow = rb < n_rb ? phys_row<EPI, RPB>(rb, c, N, ea) : -1;
    const uint32_t abase = arow >= 0 ? static_cast<uint32_t>(arow) * row_bytes + 16u * b : kOOB;
    uint32_t sbase[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int sr = rb < n_rb ? phys_row<EPI, RPB>(rb, 4 * b + t, N, ea) : -1;
      sbase[t] = sr >= 0 ? (static_cast<uint32_t>(sr) * kg + q) * 2u : kOOB;
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int T = t0 + i;
#pragma unroll
      for (int sg = 0; sg < kSegPerTile; ++sg) {
        const int seg = T * kSegPerTile + sg;
        const bool ok = seg * 128 + 32 * b < K;
        R.a[i][sg] = load16_nt(wres, ok ? abase + 64u * seg : kOOB);
      }
      const bool gok = 4 * T + q < kg;
#pragma unroll
      for (int t = 0; t < 4; ++t) R.s[i][t] = load2(sres, gok ? sbase[t] + 8u * T : kOOB);
    }
  };

  Regs R0;
  const int wg0 = blockIdx.x;
  ArgBest best{-INFINITY, INT32_MAX};  // argmax of the rows this thread stores (plain epilogue)

  // ---- prologue: x (optionally x * norm weight) -> per-group integer limbs in LDS ----
  // Single pass: thread tid owns 16-k block tid (the host guarantees 64 W >= blocks); the G/16
  // blocks of one group sit in consecutive lanes of one wave. The waves holding blocks load x
  // before issuing their weight loads, in one straight-line sequence: vector-memory loads retire
  // in issue order, so x issued after the weights would make the prologue wait for the whole
  // weight stream (and a branch between the x loads and their use lets the compiler sink them
  // below the weight loads).
  // Every workgroup reads the same x, which the previous kernel left in memory, not in this XCD's L2;
  // issued together with the weight stream of the whole chip, its misses queue behind weight misses
  // and the prologue, with every MFMA after it, ends late. A short s_sleep (DNP, DP: units of 64
  // clocks) before the first weight loads lets the x misses reach the memory queues first: measured
  // on the MI355X with the 3B decode shapes (T16 weights, rotated past the MALL), 6 on the
  // weight-only waves takes 0.29 us off the qkv entry's 4.72 us, 6 there and 4 on the x waves 0.38 us
  // off the gate/up entry's 7.05 us, 2 on the x waves of the 8192-wide down projection (all of its
  // waves hold x blocks) 0.15 us off 4.87 us; the o-projection's entry gains nothing.
  const __amdgpu_buffer_rsrc_t xres = rsrc(x, static_cast<uint32_t>(K) * 4u);
  const __amdgpu_buffer_rsrc_t ares = rsrc(aux, PRO == kProNorm ? static_cast<uint32_t>(K) * 4u : 0u);
  const int beta = tid;
  const bool valid = beta < nblk;
  const bool pro_wave = wave * 64 < nblk;  // wave-uniform
  float ssq = 0.0f;
  constexpr int kLanesPerGroup = G / 16;
  if (!pro_wave) {
    if constexpr (DNP > 0) __builtin_amdgcn_s_sleep(DNP);
    issue(wg0 * RBW + rbl, R0);
  } else {
    i32x4 xr[4], ar[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t off = valid && 16 * beta < K ? static_cast<uint32_t>(16 * beta + 4 * i) * 4u : kOOB;
      xr[i] = load16(xres, off);
      if constexpr (PRO == kProNorm) ar[i] = load16(ares, off);
    }
    if constexpr (DP > 0) {
      __builtin_amdgcn_sched_barrier(0);  // the x loads stay above the sleep
      __builtin_amdgcn_s_sleep(DP);
    }
    issue(wg0 * RBW + rbl, R0);
    __builtin_amdgcn_sched_barrier(0);  // no x arithmetic above the weight loads
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[4 * i] = __int_as_float(xr[i].x);
      v[4 * i + 1] = __int_as_float(xr[i].y);
      v[4 * i + 2] = __int_as_float(xr[i].z);
      v[4 * i + 3] = __int_as_float(xr[i].w);
    }
    if constexpr (PRO == kProNorm) {
      ssq = sumsq16(v);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[4 * i] *= __int_as_float(ar[i].x);
        v[4 * i + 1] *= __int_as_float(ar[i].y);
        v[4 * i + 2] *= __int_as_float(ar[i].z);
        v[4 * i + 3] *= __int_as_float(ar[i].w);
      }
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
    m = dpp_max<kLanesPerGroup>(m);
    int E = m > 0.0f ? __builtin_amdgcn_frexp_expf(m) : 0;
    E = E < -96 ? -96 : (E > 100 ? 100 : E);
    const int sh = 30 - E;
    // |x * 2^sh| < 2^30; truncation toward zero errs by < 2^-30 of the group's largest |x|
    uint32_t z[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) z[e] = limb_bytes(static_cast<int>(ldexpf(v[e], sh)));
    // MFMA byte order of a block: dword d holds elements 8(d/2) + (d%2) + 2i, i = 0..3 (byte i);
    // dw[jj][d] is that dword for limb jj.
    uint32_t dw[4][4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int e0 = 8 * (d >> 1) + (d & 1);
      uint32_t tr[4];
      transpose4(z[e0], z[e0 + 2], z[e0 + 4], z[e0 + 6], tr);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dw[jj][d] = tr[jj];
    }
    int s[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      int a = __builtin_amdgcn_sdot4(static_cast<int>(dw[jj][0]), 0x01010101, 0, false);
      a = __builtin_amdgcn_sdot4(static_cast<int>(dw[jj][1]), 0x01010101, a, false);
      a = __builtin_amdgcn_sdot4(static_cast<int>(dw[jj][2]), 0x01010101, a, false);
      a = __builtin_amdgcn_sdot4(static_cast<int>(dw[jj][3]), 0x01010101, a, false);
      s[jj] = dpp_isum<kLanesPerGroup>(a);
    }
    if (valid) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) Bc[4 * beta + jj] = make_uint4(dw[jj][0], dw[jj][1], dw[jj][2], dw[jj][3]);
      if (beta % kLanesPerGroup == 0) {
        const int g = beta / kLanesPerGroup;
        reinterpret_cast<int4*>(Sg)[g] = make_int4(s[0], s[1], s[2], s[3]);
        P2[g] = ldexpf(1.0f, -sh);
      }
    }
  }
  if (tid == 0) reinterpret_cast<uint4*>(lds + L.zero)[0] = make_uint4(0, 0, 0, 0);
  float rnorm = 1.0f;
  if constexpr (PRO == kProNorm) {
    ssq = group_sum<64>(ssq);
    if (lane == 0) red[wave] = ssq;
  }
  __syncthreads();
  if constexpr (PRO == kProNorm) {
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) total += red[w];
    const float mean = total / static_cast<float>(K);
    rnorm = 1.0f / sqrtf(mean + eps);
  }

  // ---- one group of row blocks: MFMAs over this wave's tiles, cross-wave sum, epilogue ----
  // x-limb operand of MFMA (segment seg, half h) for this lane: Bc entry 32 seg + 8b + 4h + j when
  // the 16-k block's group slot is this lane's column slot q, else the zero entry.
  const uint4* zero16 = reinterpret_cast<const uint4*>(lds + L.zero);
  const uint4* lane_bc = Bc + 8 * b + j;
  auto compute = [&](int wg, const Regs& R, int buf) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int T = t0 + i;
      {
        i32x4 bv[kSegPerTile][2];
#pragma unroll
        for (int sg = 0; sg < kSegPerTile; ++sg) {
          const int seg = T * kSegPerTile + sg;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            // group slot of the 16-k block: the segment's place in the tile when a group spans
            // whole segments (G >= 128; tiles start at segment multiples of 4), else the lane group
            bool active;
            if constexpr (G == 128) active = q == sg;
            else if constexpr (G == 32) active = q == b;
            else active = q == (((16 * (8 * seg + 2 * b + h)) / G) & 3);
            const uint4 bu = *(active ? lane_bc + (32 * seg + 4 * h) : zero16);
            bv[sg][h] = i32x4{static_cast<int>(bu.x), static_cast<int>(bu.y), static_cast<int>(bu.z),
                              static_cast<int>(bu.w)};
          }
        }
        i32x4 D = {0, 0, 0, 0};
#pragma unroll
        for (int sg = 0; sg < kSegPerTile; ++sg) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t w0 = static_cast<uint32_t>(h ? R.a[i][sg].z : R.a[i][sg].x);
            const uint32_t w1 = static_cast<uint32_t>(h ? R.a[i][sg].w : R.a[i][sg].y);
            const i32x4 av = {static_cast<int>(w0 & 0x0F0F0F0Fu), static_cast<int>((w0 >> 4) & 0x0F0F0F0Fu),
                              static_cast<int>(w1 & 0x0F0F0F0Fu), static_cast<int>((w1 >> 4) & 0x0F0F0F0Fu)};
            D = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv[sg][h], D, 0, 0, 0);
          }
        }
        const int g = 4 * T + q;
        const int sj = Sg[4 * g + j];
        const float mj = P2[g] * static_cast<float>(1u << (8 * j));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float f = static_cast<float>(D[t] - 8 * sj) * mj;
          acc[t] = fmaf(half_bits_to_float(R.s[i][t]), f, acc[t]);
        }
      }
    }
    // sum over the 16 columns (4 groups x 4 limbs) of each row
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = dpp_sum<16>(acc[t]);
    float* pw = part + (buf * W + wave) * 16;
    if (c == 0) {
#pragma unroll
      for (int t = 0; t < 4; ++t) pw[4 * b + t] = acc[t];
    }
    __syncthreads();
    // thread tid < 16 RBW finishes virtual row v = tid % 16 of row block tid / 16
    if (tid >= 16 * RBW) return;
    const int orl = tid >> 4, v = tid & 15;
    const int rb = wg * RBW + orl;
    const float* pb = part + (buf * W + orl * WPB) * 16;
    auto row_total = [&](int vv) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < WPB; ++w) s += pb[w * 16 + vv];
      return s * rnorm;
    };
    if (rb >= n_rb) return;
    if constexpr (EPI == kEpiNone) {
      const int row = rb * RPB + v;
      if (v < RPB && row < N) {
        const float r = row_total(v);
        const float out = residual ? residual[row] + r : r;
        y[row] = out;
        if (arg_better(out, row, best.v, best.i)) best = ArgBest{out, row};
      }
    } else if constexpr (EPI == kEpiSwiglu) {
      const int p = rb * 8 + v;
      if (v < 8 && p < (N >> 1)) y[p] = silu_mul(row_total(v), row_total(v + 8));
    } else {
      const int pr = rb * 8 + v;
      if (v < 8 && pr < (N >> 1)) {
        const float ya = row_total(v), yb = row_total(v + 8);
        const int hd = ea.hd, hh = hd >> 1;
        const int head = pr / hh, d = pr - head * hh;
        const int ra = head * hd + d;
        const int pos = ea.start[0];
        if (pos < 0 || pos >= ea.max_ctx) {
          y[ra] = ya;
          y[ra + hh] = yb;
        } else if (head < ea.n_q + ea.n_kv) {
          const float* cp = ea.cos_t + static_cast<int64_t>(pos) * hd;
          const float* sp = ea.sin_t + static_cast<int64_t>(pos) * hd;
          float lo, hi;
          rope_pair(ya, yb, cp[d], sp[d], cp[d + hh], sp[d + hh], lo, hi);
          y[ra] = lo;
          y[ra + hh] = hi;
          if (head >= ea.n_q) {
            uint16_t* dst = ea.kc + (static_cast<int64_t>(pos) * ea.n_kv + (head - ea.n_q)) * hd;
            dst[d] = float_to_half_bits(lo);
            dst[d + hh] = float_to_half_bits(hi);
          }
        } else {
          y[ra] = ya;
          y[ra + hh] = yb;
          uint16_t* dst = ea.vc + (static_cast<int64_t>(pos) * ea.n_kv + (head - ea.n_q - ea.n_kv)) * hd;
          dst[d] = float_to_half_bits(ya);
          dst[d + hh] = float_to_half_bits(yb);
        }
      }
    }
  };

  if constexpr (!MULTI) {
    compute(wg0, R0, 0);
  } else {
    // Grid-stride over groups of RBW row blocks with two register sets: the next group streams
    // in while the current one is computed. Groups past the end load nothing (out of range) and
    // store nothing. compute() returns early only after its barrier, so every wave reaches every
    // barrier of the loop.
    Regs R1;
    const int n_wg = (n_rb + RBW - 1) / RBW;
    const int stride = gridDim.x;
    const int my = wg0 < n_wg ? (n_wg - 1 - wg0) / stride + 1 : 0;
    issue((wg0 + stride) * RBW + rbl, R1);
    for (int it = 0; it < my; it += 2) {
      compute(wg0 + it * stride, R0, 0);
      issue((wg0 + (it + 2) * stride) * RBW + rbl, R0);
      if (it + 1 < my) compute(wg0 + (it + 1) * stride, R1, 1);
      issue((wg0 + (it + 3) * stride) * RBW + rbl, R1);
    }
  }
  if constexpr (EPI == kEpiNone) {
    // per-workgroup argmax partial of the stored rows (they all sit in the first wave: 16 RBW <= 64)
    if (ea.amax && wave == 0) {
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(best.v, m, 64);
        const int32_t oi = __shfl_xor(best.i, m, 64);
        if (arg_better(ov, oi, best.v, best.i)) best = ArgBest{ov, oi};
      }
      if (lane == 0) ea.amax[blockIdx.x] = best;
    }
  }
}

using MxFn = void (*)(const int32_t*, const uint16_t*, const float*, const float*, float, float*, const float*, int, int,
                      int, int, MxEpi);

// Explicit launch-shape list (index stable: the Q4_DBG_MX_CFG override selects an entry): row blocks per workgroup,
// waves per row block, largest tiles per wave, used rows per 16-row block, grid-stride, and the
// s_sleep of the weight-only and of the x waves before their first weight loads.
struct MxCfg {
  int rbw, wpb, tpw, rpb;
  bool multi;
  int dnp = 0, dp = 0;
};
constexpr MxCfg kMxCfgs[] = {
    {1, 1, 2, 16, false},   // 0: 2 tiles (K = 8 G: the tiny model's 256-wide rows)
    {1, 1, 2, 8, false},    // 1
    {1, 2, 3, 16, false},   // 2: 6 tiles (K = 24 G), 2 waves per row block
    {1, 2, 3, 8, false},    // 3
    {1, 3, 2, 16, false},   // 4: 6 tiles, 3 waves per row block
    {1, 3, 2, 8, false},    // 5
    {2, 3, 2, 16, false},   // 6
    {2, 3, 2, 8, false},    // 7
    {4, 3, 2, 16, false, 6, 4},  // 8
    {1, 6, 1, 16, false},   // 9: 6 tiles, one per wave
    {1, 6, 1, 8, false},    // 10
    {2, 6, 1, 16, false, 6, 0},  // 11
    {2, 6, 1, 8, false},    // 12
    {1, 8, 2, 16, false, 0, 2},  // 13: 16 tiles (K = 64 G: the 8192-wide down projection)
    {1, 8, 2, 8, false},    // 14
    {2, 8, 2, 8, false},    // 15
    {1, 16, 1, 8, false},   // 16
    {1, 3, 2, 16, true},    // 17: grid-stride (tall matrices), 6 tiles
    {2, 3, 2, 16, true},    // 18
    {1, 6, 1, 16, true},    // 19
    {4, 3, 2, 16, true},    // 20
};
constexpr int kNumMxCfgs = sizeof(kMxCfgs) / sizeof(kMxCfgs[0]);

template <int G, int PRO, int EPI, bool TL, int I>
constexpr MxFn mx_fn() {
  constexpr MxCfg c = kMxCfgs[I];
  if constexpr (EPI != kEpiNone && c.rpb != 16) {
    return nullptr;
  } else if constexpr (G == 32 && !(I == 0 || I == 1 || I == 2 || I == 3 || I == 17)) {
    return nullptr;  // the group-32 (tiny model) shapes use a short list
  } else {
    return q4_gemv_mx_kernel<G, c.rbw, c.wpb, c.tpw, c.multi, PRO, EPI, c.rpb, TL, c.dnp, c.dp>;
  }
}

template <int G, int PRO, int EPI, bool TL, int... Is>
constexpr std::array<MxFn, sizeof...(Is)> mx_table(std::integer_sequence<int, Is...>) {
  return {mx_fn<G, PRO, EPI, TL, Is>()...};
}

template <int G, int PRO, int EPI, bool TL>
const std::array<MxFn, kNumMxCfgs>& mx_tab() {
  static constexpr auto t = mx_table<G, PRO, EPI, TL>(std::make_integer_sequence<int, kNumMxCfgs>{});
  return t;
}

template <int G, bool TL>
MxFn mx_lookup_tl(int pro, int epi, int ci) {
  if (pro == kProNone && epi == kEpiNone) return mx_tab<G, kProNone, kEpiNone, TL>()[ci];
  if (pro == kProNorm && epi == kEpiNone) return mx_tab<G, kProNorm, kEpiNone, TL>()[ci];
  if (pro == kProNorm && epi == kEpiSwiglu) return mx_tab<G, kProNorm, kEpiSwiglu, TL>()[ci];
  if (pro == kProNorm && epi == kEpiRope) return mx_tab<G, kProNorm, kEpiRope, TL>()[ci];
  if (pro == kProNone && epi == kEpiSwiglu) return mx_tab<G, kProNone, kEpiSwiglu, TL>()[ci];
  if (pro == kProNone && epi == kEpiRope) return mx_tab<G, kProNone, kEpiRope, TL>()[ci];
  return nullptr;
}

template <int G>
MxFn mx_lookup(int pro, int epi, int ci, bool tiled) {
  return tiled ? mx_lookup_tl<G, true>(pro, epi, ci) : mx_lookup_tl<G, false>(pro, epi, ci);
}

bool mx_fits(const MxCfg& c, int n_tiles, int nblk) {
  // every wave owns exactly tpw tiles (n_tiles == wpb * tpw), and the x prologue is a single pass
  // of one 16-k block per thread (64 waves >= nblk)
  return n_tiles == c.wpb * c.tpw && 64 * c.rbw * c.wpb >= nblk;
}

// Fixed rule. Measured entries for the Llama-3.2-3B decode shapes (graph replays over rotating
// weights on one MI355X; VALU kernel in brackets), reference layout: qkv 5120x3072 + RoPE pairs
// 5.31 us [5.62], gate/up 16384x3072 + SwiGLU pairs 7.74 us [8.81], down 3072x8192 6.03 us [6.54],
// LM head 128256x3072 36.6 us [55.6]; the 3072x3072 o-projection stays on the VALU kernel there.
// T16 layout (nontemporal weight loads): qkv 5.02, gate/up 7.48, down 5.26, LM head 36.2 and the
// o-projection 3.09 us on entry 4. Other shapes: the first fitting entry in list order (8 used rows
// per block when 16 give fewer than 256 row blocks), grid-stride entries for matrices taller than
// 4096 row blocks.
// Returns -1 when the VALU kernel should run.
int mx_choose(int n_tiles, int nblk, int64_t n_rb16, bool pair, bool tiled) {
  auto fits = [&](int i) { return mx_fits(kMxCfgs[i], n_tiles, nblk) && (!pair || kMxCfgs[i].rpb == 16); };
  const int ov = debug_override(Q4_DBG_MX_CFG);
  if (ov >= 0 && ov < kNumMxCfgs && fits(ov)) return ov;
  if (n_tiles == 6 && pair) return n_rb16 <= 512 ? 11 : 8;
  if (n_tiles == 6 && !pair && n_rb16 > 4096) return 19;
  // the 3072x3072 o-projection: the VALU kernel on the reference layout (3.25 us) beats the matrix
  // cores there, while on the T16 layout full 16-row blocks, 3 waves of 2 tiles, take 3.09 us
  if (n_tiles == 6 && !pair && n_rb16 == 192) return tiled ? 4 : -1;
  if (n_tiles == 16 && !pair && n_rb16 <= 512) return 13;
  if (!pair && n_rb16 > 4096) {
    for (int i = 0; i < kNumMxCfgs; ++i)
      if (kMxCfgs[i].multi && fits(i)) return i;
    return -1;
  }
  const bool half = !pair && n_rb16 < 256;
  for (int i = 0; i < kNumMxCfgs; ++i) {
    const MxCfg& c = kMxCfgs[i];
    if (c.multi || !fits(i)) continue;
    if ((c.rpb == 8) != half) continue;
    return i;
  }
  return -1;
}

}  // namespace

int gemv_mx_num_cfgs() { return kNumMxCfgs; }

int gemv_mx_cfg_info(int i, int* out) {
  if (i < 0 || i >= kNumMxCfgs) return Q4_ERR_RANGE;
  const MxCfg& c = kMxCfgs[i];
  const int v[5] = {c.rbw, c.wpb, c.tpw, c.rpb, c.multi ? 1 : 0};
  for (int j = 0; j < 5; ++j) out[j] = v[j];
  return Q4_OK;
}

// Whether the matrix-core GEMV takes an (N, K, group) weight in the T16 layout (q4_t16.hip).
bool gemv_mx_takes_t16(int64_t N, int64_t K, int group, bool pair) {
  if (K % 32 || K > 16384 || N <= 0 || (group != 32 && group != 128) || K % group) return false;
  if (pair && N % 2) return false;
  const int tile_k = 4 * group;
  const int n_tiles = static_cast<int>((K + tile_k - 1) / tile_k);
  const int64_t n_rb16 = pair ? (N / 2 + 7) / 8 : (N + 15) / 16;
  if (n_rb16 > (int64_t{1} << 30)) return false;
  return mx_choose(n_tiles, n_tiles * (tile_k / 16), n_rb16, pair, true) >= 0;
}

// Launches the matrix-core GEMV; returns Q4_ERR_UNSUPPORTED (nothing launched) for shapes it does
// not take, so the caller can use the VALU kernel. x and y fp32; prologue 0 = none, 1 = rms_norm;
// epilogue 0 = none, 1 = SwiGLU pairs, 2 = RoPE + KV pairs (ep describes the latter).
int gemv_mx_launch(const int32_t* qweight, const uint16_t* scales, const float* x, const float* aux, float eps, float* y,
                   const float* residual, int64_t N, int64_t K, int group, int prologue, int epilogue,
                   const GemvEpi* ep, hipStream_t stream, bool tiled, int* grid_out) {
  if (!tiled && debug_flag(Q4_DBG_GEMV_NO_MX)) return Q4_ERR_UNSUPPORTED;
  if (K % 32 || K > 16384 || N <= 0) return Q4_ERR_UNSUPPORTED;
  if (group != 32 && group != 128) return Q4_ERR_UNSUPPORTED;
  if (K % group) return Q4_ERR_UNSUPPORTED;
  if (!tiled && N * (K / 2) >= (int64_t{1} << 31)) return Q4_ERR_UNSUPPORTED;
  if (!aligned(qweight, 16) || !aligned(x, 16) || (aux && !aligned(aux, 16))) return Q4_ERR_UNSUPPORTED;
  if (epilogue != kEpiNone && (N % 2 || residual)) return Q4_ERR_UNSUPPORTED;
  MxEpi ea{};
  if (ep) ea.amax = epilogue == kEpiNone ? ep->amax : nullptr;
  if (epilogue == kEpiRope) {
    ea = *ep;
    ea.amax = nullptr;
    // 8 consecutive pairs stay inside one head; head_dim / 2 a power of two (shift-based row map)
    if (ea.hd <= 0 || (ea.hd / 2) % 8 || ((ea.hd / 2) & (ea.hd / 2 - 1))) return Q4_ERR_UNSUPPORTED;
  }
  const int tile_k = 4 * group;
  const int n_tiles = static_cast<int>((K + tile_k - 1) / tile_k);
  const bool pair = epilogue != kEpiNone;
  const int64_t n_rb16 = pair ? (N / 2 + 7) / 8 : (N + 15) / 16;
  const int nblk = n_tiles * (tile_k / 16);
  const int ci = mx_choose(n_tiles, nblk, n_rb16, pair, tiled);
  if (ci < 0) return Q4_ERR_UNSUPPORTED;
  const MxFn fn = group == 128 ? mx_lookup<128>(prologue, epilogue, ci, tiled)
                               : mx_lookup<32>(prologue, epilogue, ci, tiled);
  if (!fn) return Q4_ERR_UNSUPPORTED;
  const MxCfg& c = kMxCfgs[ci];
  const int64_t n_rb = pair ? n_rb16 : (N + c.rpb - 1) / c.rpb;
  if (n_rb > (int64_t{1} << 30)) return Q4_ERR_UNSUPPORTED;
  const int ngrp = n_tiles * 4;
  const int W = c.rbw * c.wpb;
  const size_t lds = mx_lds(nblk, ngrp, W).total;
  if (lds > 64 * 1024) {
    Q4_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds)));
  }
  const int64_t n_wg = (n_rb + c.rbw - 1) / c.rbw;
  int64_t grid = n_wg;
  if (c.multi) {
    const int gv = debug_override(Q4_DBG_MX_GRID);
    const int64_t cap = gv != Q4_DBG_UNSET && gv > 0 ? gv : 1024;
    grid = n_wg < cap ? n_wg : cap;
  }
  if (ea.amax && grid > ep->amax_cap) return Q4_ERR_WORKSPACE;
  if (grid_out) *grid_out = static_cast<int>(grid);
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(64 * W), lds, stream, qweight, scales, x, aux, eps, y,
                     residual, static_cast<int>(N), static_cast<int>(K), n_tiles, static_cast<int>(n_rb), ea);
  return launch_status();
}

}  // namespace q4

extern "C" int q4_gemv_mx_num_configs(void) { return q4::gemv_mx_num_cfgs(); }
extern "C" int q4_gemv_mx_config_info(int cfg, int* info) {
  if (!info) return Q4_ERR_NULL;
  return q4::gemv_mx_cfg_info(cfg, info);
}
