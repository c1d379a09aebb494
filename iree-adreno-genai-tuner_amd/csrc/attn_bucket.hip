// KV-bucketed GQA attention for gfx950 (decode and chunked prefill share this kernel).
//
// Replaces the attention block of LlamaQ4.step (scripts/llm/llama_q4.py:204-232): for query row c
// at position pos = start + c and query head h (KV head h / g), scores s = (q . k) * scale over
// keys 0..L-1 of the position-first fp16 cache, keys with key_pos > pos masked (the reference fills
// them with -1e30; exp of that minus any finite max is exactly 0 in fp32, so skipping them gives
// the same softmax), softmax in fp32, o = p . v.
//
// Split-K over the bucket: workgroup (split, kv head, query block) handles S consecutive keys for
// CB query rows x g query heads. It stages its queries and its V tile in LDS, computes the scores
// with LPK = hd/8 lanes per key (one 16-byte K load per lane, DPP reduction across the LPK lanes),
// takes the split-local max m and sum l of exp(s - m), and writes (m, l, o = sum exp(s - m) v) to
// the workspace. The combine kernel merges the splits of each (row, head) with the log-sum-exp
// rule. Splits whose first key lies past every query position of the block are skipped (decode
// reads only the valid prefix of the bucket). `start` is read on the device.
#include "q4_common.h"
#include "q4_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>

namespace q4 {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kMaxQ = 64;  // queries (rows x group heads) per workgroup

struct AttnPlan {
  int S;         // keys per split
  int CB;        // query rows per workgroup
  int n_splits;  // ceil(L / S)
  int n_cblk;    // ceil(C / CB)
  bool mfma;     // prefill chunk on the matrix cores (attn_prefill_mfma_kernel)
};

constexpr int kMfmaMaxG = 8;  // query heads per KV head (one wave each) of the matrix-core prefill

AttnPlan plan_for(int C, int n_q, int n_kv, int L) {
  const int g = n_q / n_kv;
  AttnPlan p;
  p.mfma = false;
  if (C == 1) {
    p.CB = 1;
    p.S = L <= 1024 ? 32 : (L <= 2048 ? 64 : 128);
    const int ov = debug_override(Q4_DBG_ATTN_S);  // sweep override: keys per split (32, 64 or 128)
    if (ov == 32 || ov == 64 || ov == 128) p.S = ov;
  } else if (g <= kMfmaMaxG && !debug_flag(Q4_DBG_ATTN_GENERIC)) {
    p.mfma = true;
    p.CB = 32;
    p.S = L <= 256 ? 64 : 128;
    const int ov = debug_override(Q4_DBG_ATTN_PS);  // sweep override: keys per split (a multiple of 32, <= 512)
    if (ov != Q4_DBG_UNSET && ov >= 32 && ov <= 512 && ov % 32 == 0) p.S = ov;
  } else {
    p.CB = kMaxQ / g < C ? kMaxQ / g : C;
    p.S = 64;
  }
  p.n_splits = (L + p.S - 1) / p.S;
  p.n_cblk = (C + p.CB - 1) / p.CB;
  return p;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void unpack8(const uint4& u, float* f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = half_bits_to_float(static_cast<uint16_t>(w[i] & 0xFFFFu));
    f[2 * i + 1] = half_bits_to_float(static_cast<uint16_t>(w[i] >> 16));
  }
}

// LDS layout (floats): Q [nq][HD] | P [nq][S] | V tile [S][HD] as fp16 (uint4 rows)
template <int HD, int S>
__global__ __launch_bounds__(kThreads) void attn_split_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    float* __restrict__ ws_ml, float* __restrict__ ws_o, int C, int n_q, int n_kv, int L, int CB,
    const int32_t* __restrict__ start_p, float scale, int q_stride) {
  constexpr int LPK = HD / 8;          // lanes per key (8 halfs = 16 bytes each)
  constexpr int KPI = 64 / LPK;        // keys per wave instruction
  constexpr int KPW = S / 4;           // keys per wave
  constexpr int NKI = KPW / KPI;       // key instructions per wave
  static_assert(NKI >= 1, "split too small for the wave layout");
  extern __shared__ float lds[];
  const int g = n_q / n_kv;
  const int split = blockIdx.x, hk = blockIdx.y, cb = blockIdx.z;
  const int n_splits = gridDim.x;
  const int k0 = split * S;
  const int c0 = cb * CB;
  const int rows = min(CB, C - c0);
  const int nq = rows * g;
  const int start = start_p[0];
  float* Qs = lds;                                  // [nq][HD]
  float* Ps = Qs + kMaxQ * HD;                      // [nq][S]
  uint4* Vs = reinterpret_cast<uint4*>(Ps + kMaxQ * S);  // [S][HD/8]

  // Split entirely past the last position of the block: empty partials.
  const int last_pos = start + c0 + rows - 1;
  const bool empty = k0 > last_pos;
  if (empty) {
    for (int i = threadIdx.x; i < nq; i += kThreads) {
      const int c = c0 + i / g, h = hk * g + i % g;
      const size_t idx = (static_cast<size_t>(c) * n_q + h) * n_splits + split;
      ws_ml[2 * idx] = -INFINITY;
      ws_ml[2 * idx + 1] = 0.0f;
    }
    return;  // the combine kernel never reads o of an empty split
  }

  const uint32_t cache_bytes = static_cast<uint32_t>(L) * n_kv * HD * 2u;
  const __amdgpu_buffer_rsrc_t kres = make_rsrc(kc, cache_bytes);
  const __amdgpu_buffer_rsrc_t vres = make_rsrc(vc, cache_bytes);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  // 1. Issue this wave's K loads (rows past L are out of range: zeros) and the V tile loads.
  uint4 kreg[NKI];
#pragma unroll
  for (int i = 0; i < NKI; ++i) {
    const int key = k0 + wave * KPW + i * KPI + lane / LPK;
    kreg[i] = buf_load16(kres, (static_cast<uint32_t>(key) * n_kv + hk) * (HD * 2u) + (lane % LPK) * 16u);
  }
  constexpr int VCH = S * HD / 8;  // 16-byte chunks in the V tile
  uint4 vreg[(VCH + kThreads - 1) / kThreads];
#pragma unroll
  for (int i = 0; i < (VCH + kThreads - 1) / kThreads; ++i) {
    const int ch = threadIdx.x + i * kThreads;
    const int key = k0 + ch / LPK;
    vreg[i] = buf_load16(vres, ch < VCH ? (static_cast<uint32_t>(key) * n_kv + hk) * (HD * 2u) + (ch % LPK) * 16u
                                        : 0x80000000u);
  }
  // 2. Stage the queries (fp32) of this block: query i = (row c0 + i / g, head hk * g + i % g).
  for (int e = threadIdx.x; e < nq * (HD / 4); e += kThreads) {
    const int i = e / (HD / 4), d4 = e % (HD / 4);
    const int c = c0 + i / g, h = hk * g + i % g;
    reinterpret_cast<float4*>(Qs)[i * (HD / 4) + d4] =
        reinterpret_cast<const float4*>(q + static_cast<size_t>(c) * q_stride + static_cast<size_t>(h) * HD)[d4];
  }
#pragma unroll
  for (int i = 0; i < (VCH + kThreads - 1) / kThreads; ++i) {
    const int ch = threadIdx.x + i * kThreads;
    if (ch < VCH) Vs[ch] = vreg[i];
  }
  __syncthreads();

  // 3. Scores: lane covers dims [8*(lane % LPK), +8) of key (lane / LPK); DPP sum over LPK lanes.
#pragma unroll
  for (int i = 0; i < NKI; ++i) {
    const int kl = wave * KPW + i * KPI + lane / LPK;  // key index within the split
    const int key = k0 + kl;
    float kf[8];
    unpack8(kreg[i], kf);
    const int d0 = (lane % LPK) * 8;
    for (int qi = 0; qi < nq; ++qi) {
      const float4 a = reinterpret_cast<const float4*>(Qs + qi * HD + d0)[0];
      const float4 b = reinterpret_cast<const float4*>(Qs + qi * HD + d0)[1];
      float s = a.x * kf[0];
      s = fmaf(a.y, kf[1], s);
      s = fmaf(a.z, kf[2], s);
      s = fmaf(a.w, kf[3], s);
      s = fmaf(b.x, kf[4], s);
      s = fmaf(b.y, kf[5], s);
      s = fmaf(b.z, kf[6], s);
      s = fmaf(b.w, kf[7], s);
      s = segment_sum_to_last<LPK>(s);
      if (lane % LPK == LPK - 1) {
        const int pos = start + c0 + qi / g;
        Ps[qi * S + kl] = (key <= pos && key < L) ? s * scale : -INFINITY;
      }
    }
  }
  __syncthreads();

  // 4. Split-local softmax statistics: one wave per query, S / 64 keys per lane.
  for (int qi = wave; qi < nq; qi += kThreads / 64) {
    float m = -INFINITY;
    for (int k = lane; k < S; k += 64) m = fmaxf(m, Ps[qi * S + k]);
    m = group_max<64>(m);
    float l = 0.0f;
    for (int k = lane; k < S; k += 64) {
      const float sv = Ps[qi * S + k];
      const float p = sv == -INFINITY ? 0.0f : expf(sv - m);
      Ps[qi * S + k] = p;
      l += p;
    }
    l = group_sum<64>(l);
    if (lane == 0) {
      const int c = c0 + qi / g, h = hk * g + qi % g;
      const size_t idx = (static_cast<size_t>(c) * n_q + h) * n_splits + split;
      ws_ml[2 * idx] = m;
      ws_ml[2 * idx + 1] = l;
    }
  }
  __syncthreads();

  // 5. o = sum_k p[q][k] v[k]. Work units are (query, 8-dim slice) pairs; when there are fewer
  //    pairs than threads the keys of the split are divided among KSPLIT thread groups and the
  //    group partials are summed through LDS (reusing the score area, no longer needed).
  const int pairs = nq * LPK;
  int ksplit = 1;
  while (ksplit * 2 * pairs <= kThreads && ksplit * 2 <= S / 4) ksplit *= 2;
  __syncthreads();  // every wave has finished reading P's row statistics above
  if (ksplit == 1) {
    for (int pr = threadIdx.x; pr < pairs; pr += kThreads) {
      const int qi = pr / LPK, d8 = pr % LPK;
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int k = 0; k < S; ++k) {
        const float p = Ps[qi * S + k];
        float vf[8];
        unpack8(Vs[k * LPK + d8], vf);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = fmaf(p, vf[j], acc[j]);
      }
      const int c = c0 + qi / g, h = hk * g + qi % g;
      float* dst = ws_o + ((static_cast<size_t>(c) * n_q + h) * n_splits + split) * HD + d8 * 8;
      reinterpret_cast<float4*>(dst)[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
      reinterpret_cast<float4*>(dst)[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
  } else {
    float* red = Qs;  // [ksplit][pairs][8] floats; the queries are no longer needed
    const int pr = threadIdx.x % pairs, ks = threadIdx.x / pairs;
    if (ks < ksplit) {
      const int qi = pr / LPK, d8 = pr % LPK;
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int k = ks; k < S; k += ksplit) {
        const float p = Ps[qi * S + k];
        float vf[8];
        unpack8(Vs[k * LPK + d8], vf);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = fmaf(p, vf[j], acc[j]);
      }
      float4* r4 = reinterpret_cast<float4*>(red + (ks * pairs + pr) * 8);
      r4[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
      r4[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
    __syncthreads();
    if (threadIdx.x < pairs) {
      const int qi = threadIdx.x / LPK, d8 = threadIdx.x % LPK;
      float4 a = make_float4(0, 0, 0, 0), b = make_float4(0, 0, 0, 0);
      for (int k2 = 0; k2 < ksplit; ++k2) {
        const float4* r4 = reinterpret_cast<const float4*>(red + (k2 * pairs + threadIdx.x) * 8);
        a.x += r4[0].x; a.y += r4[0].y; a.z += r4[0].z; a.w += r4[0].w;
        b.x += r4[1].x; b.y += r4[1].y; b.z += r4[1].z; b.w += r4[1].w;
      }
      const int c = c0 + qi / g, h = hk * g + qi % g;
      float* dst = ws_o + ((static_cast<size_t>(c) * n_q + h) * n_splits + split) * HD + d8 * 8;
      reinterpret_cast<float4*>(dst)[0] = a;
      reinterpret_cast<float4*>(dst)[1] = b;
    }
  }
}

// Merge the splits of each (row, head), one thread per 8 dims of one (row, head): no LDS and no
// barrier. Every (m, l) and this thread's 8 o values of the first kB splits are requested before
// the position is read (range-checked buffer loads: zeros past the workspace), so the merge costs one
// memory round trip; splits past the position are masked by selection (their workspace entries may
// hold anything). M, the denominator and the numerator run over the splits in ascending order.
template <int HD>
__global__ __launch_bounds__(256) void attn_combine8_kernel(const float* __restrict__ ws_ml, const float* __restrict__ ws_o,
                                                          float* __restrict__ out, int64_t rows, int n_q, int n_splits,
                                                          int S, const int32_t* __restrict__ start_p,
                                                          uint16_t* __restrict__ xh, uint16_t* __restrict__ xl) {
  constexpr int kB = 8, D8 = HD / 8;
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= rows * D8) return;
  const int64_t ch = t / D8;  // (row, head) = c * n_q + h
  const int d8 = static_cast<int>(t - ch * D8);
  const int c = static_cast<int>(ch / n_q);
  const uint32_t n_ent = static_cast<uint32_t>(rows) * n_splits;
  const __amdgpu_buffer_rsrc_t mr = make_rsrc(ws_ml, n_ent * 8u);
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(ws_o, n_ent * HD * 4u);
  const uint32_t e0 = static_cast<uint32_t>(ch) * n_splits;
  f32x2 ml[kB];
  f32x4 oa[kB], ob[kB];
#pragma unroll
  for (int j = 0; j < kB; ++j) {
    const bool in = j < n_splits;
    ml[j] = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(mr, in ? (e0 + j) * 8u : 0x80000000u, 0, 0));
    const uint32_t oo = in ? ((e0 + j) * HD + 8 * d8) * 4u : 0x80000000u;
    oa[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(orr, oo, 0, 0));
    ob[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(orr, oo + 16u, 0, 0));
  }
  const int pos = start_p[0] + c;
  const int ns = min(n_splits, pos / S + 1);
  float M = -INFINITY;
#pragma unroll
  for (int j = 0; j < kB; ++j)
    if (j < ns) M = fmaxf(M, ml[j].x);
  for (int j = kB; j < ns; ++j) M = fmaxf(M, ws_ml[2 * (static_cast<size_t>(e0) + j)]);
  float den = 0.0f, num[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) num[e] = 0.0f;
  auto add = [&](float m, float l, const f32x4& a, const f32x4& b) {
    const float w = m == -INFINITY ? 0.0f : expf(m - M);
    den = fmaf(w, l, den);
    num[0] = fmaf(w, a.x, num[0]);
    num[1] = fmaf(w, a.y, num[1]);
    num[2] = fmaf(w, a.z, num[2]);
    num[3] = fmaf(w, a.w, num[3]);
    num[4] = fmaf(w, b.x, num[4]);
    num[5] = fmaf(w, b.y, num[5]);
    num[6] = fmaf(w, b.z, num[6]);
    num[7] = fmaf(w, b.w, num[7]);
  };
#pragma unroll
  for (int j = 0; j < kB; ++j)
    if (j < ns) add(ml[j].x, ml[j].y, oa[j], ob[j]);
  for (int j = kB; j < ns; ++j) {
    const size_t e = static_cast<size_t>(e0) + j;
    const float4* op = reinterpret_cast<const float4*>(ws_o + e * HD + 8 * d8);
    const float4 a = op[0], b = op[1];
    add(ws_ml[2 * e], ws_ml[2 * e + 1], f32x4{a.x, a.y, a.z, a.w}, f32x4{b.x, b.y, b.z, b.w});
  }
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = num[e] / den;
  if (xh) {
    store_x_planes8(xh, xl, ch * D8 + d8, v);  // the o-projection's x planes
  } else {
    float4* dst = reinterpret_cast<float4*>(out + ch * HD + 8 * d8);
    dst[0] = make_float4(v[0], v[1], v[2], v[3]);
    dst[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// Merge the splits of each (row, head): o = sum_i e^(m_i - M) o_i / sum_i e^(m_i - M) l_i.
// One workgroup of HD threads per (row, head); only the splits holding keys <= pos are used. The loads
// that do not need the position are issued first: this thread's dim of the first kBatch splits' o
// partials and (thread i) split i's (m, l), so the merge costs one memory round trip, overlapped with
// the read of the position; splits past it are then masked by selection (their workspace entries may
// hold anything). The max and the denominator are block reductions through LDS, the numerator is
// summed in ascending split order.
template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(const float* __restrict__ ws_ml, const float* __restrict__ ws_o,
                                                         float* __restrict__ out, int n_q, int n_splits, int S,
                                                         const int32_t* __restrict__ start_p, uint16_t* __restrict__ xh,
                                                         uint16_t* __restrict__ xl) {
  constexpr int kBatch = 32;
  constexpr int NW = HD / 64 > 0 ? HD / 64 : 1;
  __shared__ float wts[512];
  __shared__ float red[NW];
  const int c = blockIdx.x / n_q, h = blockIdx.x % n_q;
  const int d = threadIdx.x;
  const size_t base = (static_cast<size_t>(c) * n_q + h) * n_splits;
  float ov[kBatch];
#pragma unroll
  for (int j = 0; j < kBatch; ++j) ov[j] = j < n_splits ? ws_o[(base + j) * HD + d] : 0.0f;
  float2 ml = make_float2(-INFINITY, 0.0f);
  if (d < n_splits) ml = reinterpret_cast<const float2*>(ws_ml)[base + d];
  const int pos = start_p[0] + c;
  const int ns = min(n_splits, pos / S + 1);  // splits holding keys <= pos (n_splits <= 512: host)
  float mloc = d < ns ? ml.x : -INFINITY;
  for (int i = d + HD; i < ns; i += HD) mloc = fmaxf(mloc, ws_ml[2 * (base + i)]);
  const float mw = group_max<64>(mloc);
  if ((d & 63) == 0) red[d >> 6] = mw;
  __syncthreads();
  float M = red[0];
  for (int w = 1; w < NW; ++w) M = fmaxf(M, red[w]);
  __syncthreads();
  float den = 0.0f;
  if (d < ns) {
    const float w = ml.x == -INFINITY ? 0.0f : expf(ml.x - M);
    wts[d] = w;
    den = fmaf(w, ml.y, den);
  }
  for (int i = d + HD; i < ns; i += HD) {
    const float m = ws_ml[2 * (base + i)];
    const float w = m == -INFINITY ? 0.0f : expf(m - M);
    wts[i] = w;
    den = fmaf(w, ws_ml[2 * (base + i) + 1], den);
  }
  den = group_sum<64>(den);
  if ((d & 63) == 0) red[d >> 6] = den;
  __syncthreads();
  float D = 0.0f;
  for (int w = 0; w < NW; ++w) D += red[w];
  float num = 0.0f;
#pragma unroll
  for (int j = 0; j < kBatch; ++j)
    if (j < ns) num = fmaf(wts[j], ov[j], num);
  for (int i = kBatch; i < ns; ++i) num = fmaf(wts[i], ws_o[(base + i) * HD + d], num);
  const size_t k = (static_cast<size_t>(c) * n_q + h) * HD + d;
  if (xh) store_x_planes(xh, xl, static_cast<int64_t>(k), num / D);  // the o-projection's x planes
  else out[k] = num / D;
}

// ---- Decode (one query row): a register-resident split kernel and a merge that needs no position ----
//
// Workgroup (split, kv head) of 4 waves covers S = 4 * NK * KPI keys for the G query heads of the
// group. In each wave, LPK = HD / 8 lanes hold one key (8 dims, one 16-byte load of K and one of V
// per lane and key), KPI = 64 / LPK keys side by side, NK such rows. Scores are summed over the
// LPK lanes of a key with DPP (a butterfly in which partners add the same two values, so those
// lanes hold bit-identical results); each key group (column of keys) then keeps its own partial
// (m, l, o) over its NK keys in registers and writes it to LDS, and the workgroup merges the 4 KPI
// partials at once, instead of merging the key groups in registers with two lane swaps per value
// (48 per query head at G = 3). Measured on the MI355X with the 3B shapes (G = 3, split + merge,
// KV caches of 28 layers rotated): L = 256 5.81 -> 5.35 us, L = 1024 6.27 -> 5.79 us, L = 4096
// 9.80 -> 9.38 us. With G = 8 pairs of key groups are merged in registers (XR) so the partials
// fit in 32 KB of LDS.
//
// Splits wholly past `pos` write m = -inf, l = 0 and o = 0, so the merge reads every split without
// knowing `pos`. Splits in the first half of the bucket (never empty when the bucket is the
// smallest one >= pos + 1) issue their K/V loads before `pos` arrives; the others wait for it and
// load nothing when empty.

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Sum over the LPK (8 or 16) aligned lanes of a key: row_mirror (i <-> 15 - i), row_half_mirror
// (i <-> 7 - i in each half row), then quad_perm xor 1 and xor 2 -- the xor masks 15, 7, 1, 2 span
// the lane index bits, so every lane ends with the full sum.
template <int LPK>
__device__ __forceinline__ float key_sum(float v) {
  if constexpr (LPK == 16) v += dpp<0x140>(v);
  v += dpp<0x141>(v);
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  return v;
}

template <bool kMax>
__device__ __forceinline__ float combine2(float a, float b) {
  return kMax ? fmaxf(a, b) : a + b;
}

// Lane swaps: xor 16 by v_permlane16_swap (odd rows of one copy trade places with even rows of
// the other), xor 32 by v_permlane32_swap (upper half of one copy with the lower half of the
// other). The swaps are inline asm: given one value for both operands, this compiler folds the
// builtins' two results into the first.
// The s_nop 1 on each side covers the VALU-write -> permlane-read and the DPP-read hazards.
template <bool kMax>
__device__ __forceinline__ float swap_combine16(float v) {
  unsigned a = __builtin_bit_cast(unsigned, v), b = a;
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return combine2<kMax>(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

template <bool kMax>
__device__ __forceinline__ float swap_combine32(float v) {
  unsigned a = __builtin_bit_cast(unsigned, v), b = a;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return combine2<kMax>(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

template <int HD, int NK, int G>
__global__ __launch_bounds__(kThreads) void attn_decode_split_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    float* __restrict__ ws_ml, float* __restrict__ ws_o, int n_kv, int L, const int32_t* __restrict__ start_p,
    float scale) {
  constexpr int LPK = HD / 8, KPI = 64 / LPK, KPW = NK * KPI, S = 4 * KPW;
  // partials per wave: one per key group, or one per pair of groups (XR == 1: lanes l and l ^ 32
  // combined in registers) where NP partials of o would not fit in 32 KB of LDS
  constexpr int XR = 4 * KPI * G * HD * 4 > 32768 ? 1 : 0;
  constexpr int P = KPI >> XR, NP = 4 * P;
  static_assert(G * NP <= kThreads, "one thread per (query, partial)");
  __shared__ float4 red_o[NP][G][HD / 4];
  __shared__ float2 red_ml[NP][G];
  __shared__ float fw[G][NP];
  __shared__ float Mj[G];
  const int split = blockIdx.x, hk = blockIdx.y, n_splits = gridDim.x;
  const int k0 = split * S;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kg = lane / LPK, d8 = lane % LPK;
  const int key0 = k0 + wave * KPW + kg;  // key of row i is key0 + i * KPI
  const uint32_t cache_bytes = static_cast<uint32_t>(L) * n_kv * HD * 2u;
  const __amdgpu_buffer_rsrc_t kres = make_rsrc(kc, cache_bytes);
  const __amdgpu_buffer_rsrc_t vres = make_rsrc(vc, cache_bytes);
  const uint32_t off0 = (static_cast<uint32_t>(key0) * n_kv + hk) * (HD * 2u) + d8 * 16u;
  const uint32_t row_step = static_cast<uint32_t>(KPI) * n_kv * (HD * 2u);

  // Queries first (independent of everything), then K/V: early splits before `pos` is known.
  float4 qa[G], qb[G];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const float4* qp = reinterpret_cast<const float4*>(q + static_cast<size_t>(hk * G + j) * HD + d8 * 8);
    qa[j] = qp[0];
    qb[j] = qp[1];
  }
  uint4 kreg[NK], vreg[NK];
  int pos;
  if (2 * (k0 + S) <= L) {
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      kreg[i] = buf_load16(kres, off0 + i * row_step);
      vreg[i] = buf_load16(vres, off0 + i * row_step);
    }
    pos = start_p[0];
  } else {
    pos = start_p[0];
    const uint32_t dead = k0 > pos ? 0x80000000u : 0u;  // out of range: zeros, no traffic
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      kreg[i] = buf_load16(kres, (off0 + i * row_step) | dead);
      vreg[i] = buf_load16(vres, (off0 + i * row_step) | dead);
    }
  }

  // Scores of the G queries against the wave's keys (identical in the LPK lanes of a key).
  float s[G][NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    float kf[8];
    unpack8(kreg[i], kf);
    const int key = key0 + i * KPI;
    const bool live = key <= pos && key < L;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float d = qa[j].x * kf[0];
      d = fmaf(qa[j].y, kf[1], d);
      d = fmaf(qa[j].z, kf[2], d);
      d = fmaf(qa[j].w, kf[3], d);
      d = fmaf(qb[j].x, kf[4], d);
      d = fmaf(qb[j].y, kf[5], d);
      d = fmaf(qb[j].z, kf[6], d);
      d = fmaf(qb[j].w, kf[7], d);
      d = key_sum<LPK>(d);
      s[j][i] = live ? d * scale : -INFINITY;
    }
  }
  // Softmax statistics and o = sum_k p_k v_k per key group (the LPK lanes of one key column hold
  // its NK keys), or per pair of key groups when XR == 1. No lane swaps for o: each group's partial
  // goes to LDS and the workgroup merges all NP of them at once.
  float m[G], l[G], o[G][8];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    float mj = s[j][0];
#pragma unroll
    for (int i = 1; i < NK; ++i) mj = fmaxf(mj, s[j][i]);
    if constexpr (XR == 1) mj = swap_combine32<true>(mj);
    m[j] = mj;
    float lj = 0.0f;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      s[j][i] = s[j][i] == -INFINITY ? 0.0f : expf(s[j][i] - mj);
      lj += s[j][i];
    }
    l[j] = lj;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[j][e] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    float vf[8];
    unpack8(vreg[i], vf);
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[j][e] = fmaf(s[j][i], vf[e], o[j][e]);
  }
  if constexpr (XR == 1) {
#pragma unroll
    for (int j = 0; j < G; ++j) {
      l[j] = swap_combine32<false>(l[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[j][e] = swap_combine32<false>(o[j][e]);
    }
  }
  if (kg < P) {
    const int pi = wave * P + kg;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      red_o[pi][j][2 * d8] = make_float4(o[j][0], o[j][1], o[j][2], o[j][3]);
      red_o[pi][j][2 * d8 + 1] = make_float4(o[j][4], o[j][5], o[j][6], o[j][7]);
    }
    if (d8 == 0) {
#pragma unroll
      for (int j = 0; j < G; ++j) red_ml[pi][j] = make_float2(m[j], l[j]);
    }
  }
  __syncthreads();

  // Merge the NP partials: weights f_p = e^(m_p - M) (thread -> (query j, partial p)), then
  // o = sum_p f_p o_p and l = sum_p f_p l_p in ascending p (thread -> (query j, 4 dims)).
  if (threadIdx.x < G * NP) {
    const int j = threadIdx.x / NP, pi = threadIdx.x % NP;
    float M = red_ml[0][j].x;
#pragma unroll
    for (int w = 1; w < NP; ++w) M = fmaxf(M, red_ml[w][j].x);
    const float mp = red_ml[pi][j].x;
    fw[j][pi] = mp == -INFINITY ? 0.0f : expf(mp - M);
    if (pi == 0) Mj[j] = M;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < G * (HD / 4); e += kThreads) {
    const int j = e / (HD / 4), d4 = e % (HD / 4);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int w = 0; w < NP; ++w) {
      const float f = fw[j][w];
      const float4 ow = red_o[w][j][d4];
      acc.x = fmaf(f, ow.x, acc.x);
      acc.y = fmaf(f, ow.y, acc.y);
      acc.z = fmaf(f, ow.z, acc.z);
      acc.w = fmaf(f, ow.w, acc.w);
    }
    const size_t idx = static_cast<size_t>(hk * G + j) * n_splits + split;
    reinterpret_cast<float4*>(ws_o + idx * HD)[d4] = acc;
    if (d4 == 0) {
      float den = 0.0f;
#pragma unroll
      for (int w = 0; w < NP; ++w) den = fmaf(fw[j][w], red_ml[w][j].y, den);
      ws_ml[2 * idx] = Mj[j];
      ws_ml[2 * idx + 1] = den;
    }
  }
}

// Decode merge over n_splits <= MS (32 or 64) partials of each head: every split's (m, l) and o are
// read unconditionally (empty splits hold -inf, 0, 0), so there is no dependence on `pos`. Lane j of
// each wave (and lane j + 32 when MS == 32) loads split j's (m, l); the max and the denominator are
// butterflies over those lanes, and the weights reach every thread through v_readlane for the
// numerator, which is summed in ascending split order.
constexpr int kDecodeMaxSplits = 64;

template <int MS, bool kMax>
__device__ __forceinline__ float butterfly(float v) {
  v = combine2<kMax>(v, dpp<0x140>(v));  // row_mirror
  v = combine2<kMax>(v, dpp<0x141>(v));  // row_half_mirror
  v = combine2<kMax>(v, dpp<0xB1>(v));   // xor 1
  v = combine2<kMax>(v, dpp<0x4E>(v));   // xor 2
  v = swap_combine16<kMax>(v);           // xor 16
  if constexpr (MS == 64) v = swap_combine32<kMax>(v);
  return v;
}

template <int HD, int MS>
__global__ __launch_bounds__(HD) void attn_decode_merge_kernel(const float* __restrict__ ws_ml,
                                                              const float* __restrict__ ws_o, float* __restrict__ out,
                                                              int n_splits) {
  const int h = blockIdx.x, d = threadIdx.x;
  const size_t base = static_cast<size_t>(h) * n_splits;
  // Buffer resources cover exactly this head's n_splits partials: loads past them return 0.
  const __amdgpu_buffer_rsrc_t ores = make_rsrc(ws_o + base * HD, static_cast<uint32_t>(n_splits) * HD * 4u);
  const __amdgpu_buffer_rsrc_t mres = make_rsrc(ws_ml + 2 * base, static_cast<uint32_t>(n_splits) * 8u);
  float ov[MS];
#pragma unroll
  for (int j = 0; j < MS; ++j)
    ov[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ores, (j * HD + d) * 4u, 0, 0));
  const int js = d & (MS - 1);
  const float mraw = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(mres, js * 8u, 0, 0));
  const float lraw = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(mres, js * 8u + 4u, 0, 0));
  const float mj = js < n_splits ? mraw : -INFINITY;
  const float M = butterfly<MS, true>(mj);
  const float w = mj == -INFINITY ? 0.0f : expf(mj - M);
  const float den = butterfly<MS, false>(w * lraw);
  float num = 0.0f;
#pragma unroll
  for (int j = 0; j < MS; ++j)
    num = fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), j)), ov[j], num);
  out[static_cast<size_t>(h) * HD + d] = num / den;
}

template <int HD, int NK, int G>
int launch_decode3(const float* q, const uint16_t* kc, const uint16_t* vc, float* ws_ml, float* ws_o, float* out,
                   int n_splits, int n_kv, int L, const int32_t* start, float scale, hipStream_t st) {
  hipLaunchKernelGGL((attn_decode_split_kernel<HD, NK, G>), dim3(n_splits, n_kv), dim3(kThreads), 0, st, q, kc, vc,
                     ws_ml, ws_o, n_kv, L, start, scale);
  if (n_splits <= 32)
    hipLaunchKernelGGL((attn_decode_merge_kernel<HD, 32>), dim3(n_kv * G), dim3(HD), 0, st, ws_ml, ws_o, out, n_splits);
  else
    hipLaunchKernelGGL((attn_decode_merge_kernel<HD, 64>), dim3(n_kv * G), dim3(HD), 0, st, ws_ml, ws_o, out, n_splits);
  return launch_status();
}

template <int HD, int NK>
int launch_decode2(int g, const float* q, const uint16_t* kc, const uint16_t* vc, float* ws_ml, float* ws_o,
                   float* out, int n_splits, int n_kv, int L, const int32_t* start, float scale, hipStream_t st) {
  switch (g) {
    case 1: return launch_decode3<HD, NK, 1>(q, kc, vc, ws_ml, ws_o, out, n_splits, n_kv, L, start, scale, st);
    case 2: return launch_decode3<HD, NK, 2>(q, kc, vc, ws_ml, ws_o, out, n_splits, n_kv, L, start, scale, st);
    case 3: return launch_decode3<HD, NK, 3>(q, kc, vc, ws_ml, ws_o, out, n_splits, n_kv, L, start, scale, st);
    case 4: return launch_decode3<HD, NK, 4>(q, kc, vc, ws_ml, ws_o, out, n_splits, n_kv, L, start, scale, st);
    case 8: return launch_decode3<HD, NK, 8>(q, kc, vc, ws_ml, ws_o, out, n_splits, n_kv, L, start, scale, st);
    default: return Q4_ERR_UNSUPPORTED;
  }
}

// The register-resident decode path covers group sizes 1, 2, 3, 4, 8 and at most 64 splits.
bool decode_fast(int C, int n_q, int n_kv, const AttnPlan& p) {
  const int g = n_q / n_kv;
  return C == 1 && p.n_splits <= kDecodeMaxSplits && (g <= 4 || g == 8) && !debug_flag(Q4_DBG_ATTN_GENERIC);
}

int launch_decode(const AttnPlan& p, int hd, int g, const float* q, const uint16_t* kc, const uint16_t* vc,
                  float* ws_ml, float* ws_o, float* out, int n_kv, int L, const int32_t* start, float scale,
                  hipStream_t st) {
  const int n = p.n_splits;
  if (hd == 128) {  // KPI = 4 keys per wave row: NK = S / 16
    if (p.S == 32) return launch_decode2<128, 2>(g, q, kc, vc, ws_ml, ws_o, out, n, n_kv, L, start, scale, st);
    if (p.S == 64) return launch_decode2<128, 4>(g, q, kc, vc, ws_ml, ws_o, out, n, n_kv, L, start, scale, st);
    return launch_decode2<128, 8>(g, q, kc, vc, ws_ml, ws_o, out, n, n_kv, L, start, scale, st);
  }
  // hd == 64: KPI = 8: NK = S / 32
  if (p.S == 32) return launch_decode2<64, 1>(g, q, kc, vc, ws_ml, ws_o, out, n, n_kv, L, start, scale, st);
  if (p.S == 64) return launch_decode2<64, 2>(g, q, kc, vc, ws_ml, ws_o, out, n, n_kv, L, start, scale, st);
  return launch_decode2<64, 4>(g, q, kc, vc, ws_ml, ws_o, out, n, n_kv, L, start, scale, st);
}

// ---- Prefill (C > 1): flash attention on the fp16 matrix cores ----------------------------------
//
// Workgroup (key split, KV head, block of 32 query rows) with one wave per query head of the group.
// Per 32-key block: S^T = K Q^T (v_mfma_f32_32x32x16_f16, K from LDS as the A operand, the fp32
// queries split into fp16 hi + lo as two B operands, so the products keep fp32-level accuracy), the
// mask (key <= pos, key < L) and an online softmax per query (a lane holds one query column; the
// other half of its keys sits in lane ^ 32), then O^T += V^T P^T with P split into fp16 hi + lo the
// same way. The S^T accumulator is used directly as the P^T operand: its keys are fed in a fixed
// permutation (lane half h supplies keys 16u + 8(i/4) + 4h + i%4) and V^T is read from LDS in the
// same order, so no transpose of P is needed. O^T's column is the lane's query, so the softmax
// rescale is per lane. The partial (m, l, o) of each (row, head, split) goes to the workspace and
// attn_combine8_kernel merges the splits. Each key block's K/V rows are loaded into registers two
// blocks ahead (two register sets) while the blocks before it are computed; the workgroup has at
// least 4 waves for that staging (waves past the group size only stage).
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

template <int HD>
__device__ __forceinline__ int kswz(int r) {  // 16-byte chunk swizzle of a key row in LDS
  return HD == 128 ? (r & 15) : ((r >> 1) & 7);
}

template <int HD>
__global__ __launch_bounds__(64 * kMfmaMaxG) void attn_prefill_mfma_kernel(
    const float* __restrict__ q, int q_stride, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    float* __restrict__ ws_ml, float* __restrict__ ws_o, int C, int n_q, int n_kv, int L, int S,
    const int32_t* __restrict__ start_p, float scale) {
  constexpr int KSTEPS = HD / 16;       // 16-dim k-steps of the score MFMAs
  constexpr int OT = HD / 32;           // 32-dim output tiles
  constexpr int KCH = HD / 8;           // 16-byte chunks per key row
  constexpr int VT_PITCH = 32 * 2 + 8;  // bytes per V^T row: 32 keys + 8 bytes (conflict-free 8-byte reads)
  constexpr int kMaxCh = 32 * KCH / 256; // staging chunks per thread (at least 4 waves)
  __shared__ __attribute__((aligned(16))) unsigned char Ks[32 * HD * 2];
  __shared__ __attribute__((aligned(16))) unsigned char Vt[HD * VT_PITCH];
  const int g = n_q / n_kv;
  const int split = blockIdx.x, hk = blockIdx.y, qb = blockIdx.z;
  const int n_splits = gridDim.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool computes = wave < g;       // waves past the group size only stage K and V
  const int h = hk * g + (computes ? wave : 0);
  const int half = lane >> 5, ql = lane & 31;
  const int nthr = blockDim.x;
  const int c0 = qb * 32;
  const int start = start_p[0];
  const int pos_max = start + min(c0 + 31, C - 1);
  const int k0 = split * S;
  const int k_end = min(min(k0 + S, L), pos_max + 1);
  if (k0 >= k_end) return;  // no row of the block sees a key of this split: the merge never reads it
  const int c = c0 + ql;
  const bool row_ok = computes && c < C;
  const int pos = start + c;

  // Q^T operand (column = this lane's query, k = dims 16 t + 8 half + i), split into fp16 hi + lo
  half8 qh[KSTEPS], qlo[KSTEPS];
#pragma unroll
  for (int t = 0; t < KSTEPS; ++t) {
    float f[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (row_ok) {
      const float4* qp = reinterpret_cast<const float4*>(q + static_cast<size_t>(c) * q_stride +
                                                         static_cast<size_t>(h) * HD + 16 * t + 8 * half);
      const float4 a = qp[0], b = qp[1];
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const _Float16 hi = static_cast<_Float16>(f[i]);
      qh[t][i] = hi;
      qlo[t][i] = static_cast<_Float16>(f[i] - static_cast<float>(hi));
    }
  }

  const uint32_t cache_bytes = static_cast<uint32_t>(L) * n_kv * HD * 2u;
  const __amdgpu_buffer_rsrc_t kres = make_rsrc(kc, cache_bytes);
  const __amdgpu_buffer_rsrc_t vres = make_rsrc(vc, cache_bytes);
  // K/V rows of a 32-key block: chunk ch = threadIdx.x + i * nthr (row ch / KCH, 16-byte chunk ch % KCH);
  // keys past L read out of range (zeros).
  // Two register sets: block kb's rows are requested two blocks ahead of their use.
  uint4 kpa[kMaxCh], vpa[kMaxCh], kpb[kMaxCh], vpb[kMaxCh];
  auto load_block = [&](int kb, uint4 (&kpre)[kMaxCh], uint4 (&vpre)[kMaxCh]) {
#pragma unroll
    for (int i = 0; i < kMaxCh; ++i) {
      const int ch = threadIdx.x + i * nthr;
      const int r = ch / KCH, cc = ch - (ch / KCH) * KCH;
      const uint32_t off = ch < 32 * KCH ? (static_cast<uint32_t>(kb + r) * n_kv + hk) * (HD * 2u) + cc * 16u
                                         : 0x80000000u;
      kpre[i] = buf_load16(kres, off);
      vpre[i] = buf_load16(vres, off);
    }
  };
  auto stage_block = [&](const uint4 (&kpre)[kMaxCh], const uint4 (&vpre)[kMaxCh]) {
#pragma unroll
    for (int i = 0; i < kMaxCh; ++i) {
      const int ch = threadIdx.x + i * nthr;
      if (ch < 32 * KCH) {
        const int r = ch / KCH, cc = ch - (ch / KCH) * KCH;
        *reinterpret_cast<uint4*>(Ks + r * (HD * 2) + ((cc ^ kswz<HD>(r)) << 4)) = kpre[i];
        const uint32_t w[4] = {vpre[i].x, vpre[i].y, vpre[i].z, vpre[i].w};
#pragma unroll
        for (int j = 0; j < 8; ++j)
          *reinterpret_cast<uint16_t*>(Vt + (cc * 8 + j) * VT_PITCH + r * 2) =
              static_cast<uint16_t>(w[j >> 1] >> (16 * (j & 1)));
      }
    }
  };

  float16v o[OT];
#pragma unroll
  for (int tt = 0; tt < OT; ++tt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[tt][e] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  auto block = [&](int kb, uint4 (&kpre)[kMaxCh], uint4 (&vpre)[kMaxCh]) {
    stage_block(kpre, vpre);
    __syncthreads();
    if (kb + 64 < k_end) load_block(kb + 64, kpre, vpre);  // in flight during the next two blocks

    // S^T = K Q^T: 32 keys (rows) x 32 queries (columns)
    float16v sacc;
#pragma unroll
    for (int e = 0; e < 16; ++e) sacc[e] = 0.0f;
#pragma unroll
    for (int t = 0; t < KSTEPS; ++t) {
      const half8 ka = *reinterpret_cast<const half8*>(Ks + ql * (HD * 2) + (((2 * t + half) ^ kswz<HD>(ql)) << 4));
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qh[t], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qlo[t], sacc, 0, 0, 0);
    }
    float sv[16];
    float mb = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int key = kb + 8 * (e >> 2) + 4 * half + (e & 3);
      const bool ok = row_ok && key <= pos && key < L;
      sv[e] = ok ? sacc[e] * scale : -INFINITY;
      mb = fmaxf(mb, sv[e]);
    }
    mb = swap_combine32<true>(mb);
    const float m_new = fmaxf(m, mb);
    const float alpha = m == -INFINITY ? 0.0f : expf(m - m_new);
    float ls = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      sv[e] = sv[e] == -INFINITY ? 0.0f : expf(sv[e] - m_new);
      ls += sv[e];
    }
    ls = swap_combine32<false>(ls);
    l = l * alpha + ls;
    m = m_new;
#pragma unroll
    for (int tt = 0; tt < OT; ++tt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[tt][e] *= alpha;

    // O^T += V^T P^T over two 16-key steps
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      half8 ph, pl;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const _Float16 hi = static_cast<_Float16>(sv[8 * u + i]);
        ph[i] = hi;
        pl[i] = static_cast<_Float16>(sv[8 * u + i] - static_cast<float>(hi));
      }
#pragma unroll
      for (int tt = 0; tt < OT; ++tt) {
        const unsigned char* vrow = Vt + (32 * tt + ql) * VT_PITCH;
        const uint2 v0 = *reinterpret_cast<const uint2*>(vrow + (16 * u + 4 * half) * 2);
        const uint2 v1 = *reinterpret_cast<const uint2*>(vrow + (16 * u + 8 + 4 * half) * 2);
        const uint4 vv = make_uint4(v0.x, v0.y, v1.x, v1.y);
        const half8 va = __builtin_bit_cast(half8, vv);
        o[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ph, o[tt], 0, 0, 0);
        o[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl, o[tt], 0, 0, 0);
      }
    }
    __syncthreads();  // every wave is done with this block's K and V^T
  };
  load_block(k0, kpa, vpa);
  if (k0 + 32 < k_end) load_block(k0 + 32, kpb, vpb);
  for (int kb = k0; kb < k_end; kb += 64) {
    block(kb, kpa, vpa);
    if (kb + 32 < k_end) block(kb + 32, kpb, vpb);
  }

  if (row_ok) {
    const size_t idx = (static_cast<size_t>(c) * n_q + h) * n_splits + split;
    if (half == 0) {
      ws_ml[2 * idx] = m;
      ws_ml[2 * idx + 1] = l;
    }
#pragma unroll
    for (int tt = 0; tt < OT; ++tt)
#pragma unroll
      for (int a = 0; a < 4; ++a)
        reinterpret_cast<float4*>(ws_o + idx * HD + 32 * tt + 8 * a + 4 * half)[0] =
            make_float4(o[tt][4 * a], o[tt][4 * a + 1], o[tt][4 * a + 2], o[tt][4 * a + 3]);
  }
}

size_t lds_bytes(int HD, int S) {
  return (static_cast<size_t>(kMaxQ) * HD + static_cast<size_t>(kMaxQ) * S) * 4 + static_cast<size_t>(S) * HD * 2;
}

template <int HD, int S>
int launch_split(const AttnPlan& p, const float* q, int q_stride, const uint16_t* kc, const uint16_t* vc, float* ws_ml,
                 float* ws_o, int C, int n_q, int n_kv, int L, const int32_t* start, float scale, hipStream_t st) {
  const size_t lds = lds_bytes(HD, S);
  if (lds > 64 * 1024) {
    Q4_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(attn_split_kernel<HD, S>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  }
  hipLaunchKernelGGL((attn_split_kernel<HD, S>), dim3(p.n_splits, n_kv, p.n_cblk), dim3(kThreads), lds, st, q, kc, vc,
                     ws_ml, ws_o, C, n_q, n_kv, L, p.CB, start, scale, q_stride);
  return launch_status();
}

}  // namespace
}  // namespace q4

using namespace q4;

namespace {
// (m, l) pairs of n partials, rounded up to 16 bytes so the o partials that follow stay aligned
size_t ml_floats(size_t n) { return (2 * n + 3) / 4 * 4; }

int attn_args(int C, int n_q, int n_kv, int hd, int L) {
  if (C <= 0 || n_q <= 0 || n_kv <= 0 || L <= 0) return Q4_ERR_SHAPE;
  if (n_q % n_kv) return Q4_ERR_SHAPE;
  if (n_q / n_kv > kMaxQ) return Q4_ERR_UNSUPPORTED;
  if (hd != 64 && hd != 128) return Q4_ERR_UNSUPPORTED;
  if (plan_for(C, n_q, n_kv, L).n_splits > 512) return Q4_ERR_UNSUPPORTED;  // combine holds <= 512 weights
  if (static_cast<int64_t>(L) * n_kv * hd * 2 >= (int64_t{1} << 31)) return Q4_ERR_SHAPE;
  return Q4_OK;
}
}  // namespace

extern "C" int attn_workspace_bytes(int C, int n_q, int n_kv, int hd, int L, size_t* bytes) {
  if (!bytes) return Q4_ERR_NULL;
  if (int st = attn_args(C, n_q, n_kv, hd, L)) return st;
  const AttnPlan p = plan_for(C, n_q, n_kv, L);
  const size_t n = static_cast<size_t>(C) * n_q * p.n_splits;
  *bytes = ml_floats(n) * sizeof(float) + n * hd * sizeof(float);
  return Q4_OK;
}

namespace {
// out: fp32 [C, n_q * hd]; or, with xh != nullptr (prefill only), the fp16 (hi, lo) planes of the
// o-projection's input in place of out.
int attn_bucket_impl(const float* q, int q_row_stride, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                     uint16_t* xh, uint16_t* xl, int C, int n_q, int n_kv, int hd, int L, const int32_t* start,
                     float scale, void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !(out || xh) || !start || !workspace) return Q4_ERR_NULL;
  if (xh && (!xl || C == 1)) return Q4_ERR_SHAPE;
  if (int st = attn_args(C, n_q, n_kv, hd, L)) return st;
  if (q_row_stride < n_q * hd || q_row_stride % 4) return Q4_ERR_SHAPE;
  size_t need = 0;
  attn_workspace_bytes(C, n_q, n_kv, hd, L, &need);
  if (workspace_bytes < need) return Q4_ERR_WORKSPACE;
  if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(workspace, 16)) return Q4_ERR_ALIGN;
  const AttnPlan p = plan_for(C, n_q, n_kv, L);
  float* ws_ml = static_cast<float*>(workspace);
  float* ws_o = ws_ml + ml_floats(static_cast<size_t>(C) * n_q * p.n_splits);
  const hipStream_t st = as_stream(stream);
  if (decode_fast(C, n_q, n_kv, p))
    return launch_decode(p, hd, n_q / n_kv, q, k_cache, v_cache, ws_ml, ws_o, out, n_kv, L, start, scale, st);
  int rc = Q4_OK;
  if (p.mfma) {
    const dim3 grid(p.n_splits, n_kv, p.n_cblk), block(64 * std::max(n_q / n_kv, 4));
    if (hd == 128)
      hipLaunchKernelGGL(attn_prefill_mfma_kernel<128>, grid, block, 0, st, q, q_row_stride, k_cache, v_cache, ws_ml,
                         ws_o, C, n_q, n_kv, L, p.S, start, scale);
    else
      hipLaunchKernelGGL(attn_prefill_mfma_kernel<64>, grid, block, 0, st, q, q_row_stride, k_cache, v_cache, ws_ml,
                         ws_o, C, n_q, n_kv, L, p.S, start, scale);
    rc = launch_status();
  } else if (hd == 128) {
    if (p.S == 32) rc = launch_split<128, 32>(p, q, q_row_stride, k_cache, v_cache, ws_ml, ws_o, C, n_q, n_kv, L, start, scale, st);
    else if (p.S == 64) rc = launch_split<128, 64>(p, q, q_row_stride, k_cache, v_cache, ws_ml, ws_o, C, n_q, n_kv, L, start, scale, st);
    else rc = launch_split<128, 128>(p, q, q_row_stride, k_cache, v_cache, ws_ml, ws_o, C, n_q, n_kv, L, start, scale, st);
  } else {
    if (p.S == 32) rc = launch_split<64, 32>(p, q, q_row_stride, k_cache, v_cache, ws_ml, ws_o, C, n_q, n_kv, L, start, scale, st);
    else if (p.S == 64) rc = launch_split<64, 64>(p, q, q_row_stride, k_cache, v_cache, ws_ml, ws_o, C, n_q, n_kv, L, start, scale, st);
    else rc = launch_split<64, 128>(p, q, q_row_stride, k_cache, v_cache, ws_ml, ws_o, C, n_q, n_kv, L, start, scale, st);
  }
  if (rc) return rc;
  const int64_t rows = static_cast<int64_t>(C) * n_q;
  if (rows * p.n_splits * hd * 4 < (int64_t{1} << 31) && (!xh || (aligned(xh, 16) && aligned(xl, 16))) &&
      (xh || aligned(out, 16)) && !debug_flag(Q4_DBG_ATTN_COMBINE_WG)) {
    const unsigned blocks = static_cast<unsigned>((rows * (hd / 8) + 255) / 256);
    if (hd == 128)
      hipLaunchKernelGGL(attn_combine8_kernel<128>, dim3(blocks), dim3(256), 0, st, ws_ml, ws_o, out, rows, n_q,
                         p.n_splits, p.S, start, xh, xl);
    else
      hipLaunchKernelGGL(attn_combine8_kernel<64>, dim3(blocks), dim3(256), 0, st, ws_ml, ws_o, out, rows, n_q,
                         p.n_splits, p.S, start, xh, xl);
    return launch_status();
  }
  if (hd == 128)
    hipLaunchKernelGGL(attn_combine_kernel<128>, dim3(C * n_q), dim3(128), 0, st, ws_ml, ws_o, out, n_q, p.n_splits,
                       p.S, start, xh, xl);
  else
    hipLaunchKernelGGL(attn_combine_kernel<64>, dim3(C * n_q), dim3(64), 0, st, ws_ml, ws_o, out, n_q, p.n_splits,
                       p.S, start, xh, xl);
  return launch_status();
}
}  // namespace

extern "C" int attn_bucket(const float* q, int q_row_stride, const uint16_t* k_cache, const uint16_t* v_cache,
                           float* out, int C, int n_q, int n_kv, int hd, int L, const int32_t* start, float scale,
                           void* workspace, size_t workspace_bytes, void* stream) {
  if (!out) return Q4_ERR_NULL;
  return attn_bucket_impl(q, q_row_stride, k_cache, v_cache, out, nullptr, nullptr, C, n_q, n_kv, hd, L, start, scale,
                          workspace, workspace_bytes, stream);
}

namespace q4 {
int attn_bucket_planes(const float* q, int q_row_stride, const uint16_t* k_cache, const uint16_t* v_cache,
                       uint16_t* xh, uint16_t* xl, int C, int n_q, int n_kv, int hd, int L, const int32_t* start,
                       float scale, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!xh || !xl) return Q4_ERR_NULL;
  return attn_bucket_impl(q, q_row_stride, k_cache, v_cache, nullptr, xh, xl, C, n_q, n_kv, hd, L, start, scale,
                          workspace, workspace_bytes, stream);
}
}  // namespace q4
