// int4 weight format kernels: quantize, unpack, dequantize and the int4 embedding row gather.
//
// Format (reference scripts/llm/llama_q4.py:25-51): qweight [N, K/8] int32, nibble b of word w
// holds k = 8w + b as q + 8 in [0, 15]; scales [N, K/group] fp16. All four kernels are
// load-time or support work (not the decode hot loop); they are written for exactness first and
// coalesced where it is free.
#include "q4_common.h"

namespace q4 {
namespace {

// One thread per K-group of one row. Follows quantize_q4 (llama_q4.py:30-38) operation by
// operation so the result is bit-identical: amax in fp32, max(amax, 1e-8f), a correctly rounded
// fp32 division by 7, q = rint(w / scale) (round half to even, as torch.round), clamp to
// [-8, 7], + 8; the scale is rounded to fp16 only after q is formed.
__global__ void quantize_kernel(const float* __restrict__ w, int32_t* __restrict__ qw,
                                uint16_t* __restrict__ scales, int64_t N, int64_t K, int group) {
  const int64_t groups_per_row = K / group;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= N * groups_per_row) return;
  const int64_t row = gid / groups_per_row;
  const int64_t g = gid % groups_per_row;
  const float* src = w + row * K + g * group;
  float amax = 0.0f;
  for (int i = 0; i < group; ++i) amax = fmaxf(amax, fabsf(src[i]));
  const float scale = fmaxf(amax, 1e-8f) / 7.0f;
  int32_t* dst = qw + row * (K / 8) + g * (group / 8);
  for (int wd = 0; wd < group / 8; ++wd) {
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      float q = __builtin_rintf(src[wd * 8 + b] / scale);
      q = fminf(fmaxf(q, -8.0f), 7.0f);
      word |= static_cast<uint32_t>(static_cast<int>(q) + 8) << (4 * b);
    }
    dst[wd] = static_cast<int32_t>(word);
  }
  scales[row * groups_per_row + g] = float_to_half_bits(scale);
}

// unpack_q4 (llama_q4.py:41-45): one thread per word, 8 nibbles out as bytes.
__global__ void unpack_kernel(const int32_t* __restrict__ qw, uint8_t* __restrict__ out,
                              int64_t n_words) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_words) return;
  const uint32_t word = static_cast<uint32_t>(qw[i]);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    lo |= ((word >> (4 * b)) & 15u) << (8 * b);
    hi |= ((word >> (4 * (b + 4))) & 15u) << (8 * b);
  }
  reinterpret_cast<uint2*>(out)[i] = make_uint2(lo, hi);
}

// dequantize_q4 (llama_q4.py:48-51): (nibble - 8) * fp32(scale); exact in fp32.
template <typename OutT>
__global__ void dequant_kernel(const int32_t* __restrict__ qw, const uint16_t* __restrict__ scales,
                               OutT* __restrict__ out, int64_t N, int64_t K, int group) {
  const int64_t words_per_row = K / 8;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N * words_per_row) return;
  const int64_t row = i / words_per_row;
  const int64_t wd = i % words_per_row;
  const float s = half_bits_to_float(scales[row * (K / group) + (wd * 8) / group]);
  const uint32_t word = static_cast<uint32_t>(qw[i]);
  float v[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) v[b] = static_cast<float>(static_cast<int>((word >> (4 * b)) & 15u) - 8) * s;
  OutT* dst = out + i * 8;
  if constexpr (sizeof(OutT) == 4) {
    reinterpret_cast<float4*>(dst)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(dst)[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      p[j] = static_cast<uint32_t>(float_to_half_bits(v[2 * j])) |
             (static_cast<uint32_t>(float_to_half_bits(v[2 * j + 1])) << 16);
    reinterpret_cast<uint4*>(dst)[0] = make_uint4(p[0], p[1], p[2], p[3]);
  }
}

// QEmbedding.lookup (llama_q4.py:106-119): gather + dequant one int4 row per token; tokens
// outside [0, vocab) produce zeros like the reference's per-chunk `valid` mask.
__global__ void embed_kernel(const int32_t* __restrict__ qw, const uint16_t* __restrict__ scales,
                             const int32_t* __restrict__ tokens, float* __restrict__ out, int C,
                             int64_t vocab, int64_t D, int group) {
  const int64_t words_per_row = D / 8;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= C * words_per_row) return;
  const int64_t c = i / words_per_row;
  const int64_t wd = i % words_per_row;
  const int64_t tok = tokens[c];
  float v[8];
  if (tok >= 0 && tok < vocab) {
    const float s = half_bits_to_float(scales[tok * (D / group) + (wd * 8) / group]);
    const uint32_t word = static_cast<uint32_t>(qw[tok * words_per_row + wd]);
#pragma unroll
    for (int b = 0; b < 8; ++b) v[b] = static_cast<float>(static_cast<int>((word >> (4 * b)) & 15u) - 8) * s;
  } else {
#pragma unroll
    for (int b = 0; b < 8; ++b) v[b] = 0.0f;
  }
  float4* dst = reinterpret_cast<float4*>(out + c * D + wd * 8);
  dst[0] = make_float4(v[0], v[1], v[2], v[3]);
  dst[1] = make_float4(v[4], v[5], v[6], v[7]);
}

inline unsigned blocks_for(int64_t n, int threads) {
  return static_cast<unsigned>((n + threads - 1) / threads);
}

int check_format(int64_t N, int64_t K, int group) {
  if (N <= 0 || K <= 0 || group <= 0) return Q4_ERR_SHAPE;
  if (K % 8 != 0 || group % 8 != 0 || K % group != 0) return Q4_ERR_SHAPE;
  return Q4_OK;
}

}  // namespace
}  // namespace q4

using namespace q4;

extern "C" int q4_quantize(const float* w, int32_t* qweight, uint16_t* scales, int64_t N, int64_t K,
                           int group, void* stream) {
  if (!w || !qweight || !scales) return Q4_ERR_NULL;
  if (int st = check_format(N, K, group)) return st;
  const int64_t n_groups = N * (K / group);
  const int threads = 256;
  hipLaunchKernelGGL(quantize_kernel, dim3(blocks_for(n_groups, threads)), dim3(threads), 0,
                     as_stream(stream), w, qweight, scales, N, K, group);
  return launch_status();
}

extern "C" int q4_unpack(const int32_t* qweight, uint8_t* nibbles, int64_t N, int64_t K, void* stream) {
  if (!qweight || !nibbles) return Q4_ERR_NULL;
  if (N <= 0 || K <= 0 || K % 8 != 0) return Q4_ERR_SHAPE;
  if (!aligned(nibbles, 8)) return Q4_ERR_ALIGN;
  const int64_t n_words = N * (K / 8);
  hipLaunchKernelGGL(unpack_kernel, dim3(blocks_for(n_words, 256)), dim3(256), 0, as_stream(stream),
                     qweight, nibbles, n_words);
  return launch_status();
}

extern "C" int q4_dequant(const int32_t* qweight, const uint16_t* scales, void* w, int w_dtype,
                          int64_t N, int64_t K, int group, void* stream) {
  if (!qweight || !scales || !w) return Q4_ERR_NULL;
  if (int st = check_format(N, K, group)) return st;
  if (!aligned(w, 16)) return Q4_ERR_ALIGN;
  const int64_t n_words = N * (K / 8);
  const dim3 grid(blocks_for(n_words, 256));
  if (w_dtype == Q4_F32) {
    hipLaunchKernelGGL(dequant_kernel<float>, grid, dim3(256), 0, as_stream(stream), qweight, scales,
                       static_cast<float*>(w), N, K, group);
  } else if (w_dtype == Q4_F16) {
    hipLaunchKernelGGL(dequant_kernel<uint16_t>, grid, dim3(256), 0, as_stream(stream), qweight,
                       scales, static_cast<uint16_t*>(w), N, K, group);
  } else {
    return Q4_ERR_DTYPE;
  }
  return launch_status();
}

extern "C" int q4_embed_lookup(const int32_t* qweight, const uint16_t* scales, const int32_t* tokens,
                               float* out, int C, int64_t vocab, int64_t D, int group, void* stream) {
  if (!qweight || !scales || !tokens || !out) return Q4_ERR_NULL;
  if (C <= 0) return Q4_ERR_SHAPE;
  if (int st = check_format(vocab, D, group)) return st;
  if (!aligned(out, 16)) return Q4_ERR_ALIGN;
  const int64_t n = static_cast<int64_t>(C) * (D / 8);
  hipLaunchKernelGGL(embed_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), qweight,
                     scales, tokens, out, C, vocab, D, group);
  return launch_status();
}
