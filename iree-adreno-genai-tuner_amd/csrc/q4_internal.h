// Entry points shared between the library's translation units and not part of the C ABI: the
// prefill step hands activations to its projections as fp16 (hi, lo) planes written by the
// producing kernel (store_x_planes layout), instead of fp32 rows split by a kernel of their own.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace q4 {

// q4_linear_ws's GEMM on given planes (power-of-two group).
int q4_linear_planes(const uint16_t* xh, const uint16_t* xl, int64_t M, const int32_t* qw, const uint16_t* sc,
                     float* y, const float* res, int64_t N, int64_t K, int group, hipStream_t st);
// The gate/up projection with silu(gate) * up written as the [M, N / 2] planes oh / ol (ol = oh + M N / 2)
// of the down projection; Q4_ERR_UNSUPPORTED when the shape does not take the fused tile (the caller then
// runs q4_linear_planes + silu_mul_planes).
int q4_linear_planes_swiglu(const uint16_t* xh, const uint16_t* xl, int64_t M, const int32_t* qw, const uint16_t* sc,
                            uint16_t* oh, uint16_t* ol, int64_t N, int64_t K, int group, hipStream_t st);
// rmsnorm_f32 of M rows (no row selection), written as planes.
int rmsnorm_planes(const float* x, const float* w, uint16_t* xh, uint16_t* xl, int64_t M, int64_t D, float eps,
                   hipStream_t st);
// silu_mul_f32, written as planes.
int silu_mul_planes(const float* gu, uint16_t* xh, uint16_t* xl, int64_t M, int64_t inter, hipStream_t st);
// attn_bucket for C > 1, its output written as planes.
int attn_bucket_planes(const float* q, int q_row_stride, const uint16_t* k_cache, const uint16_t* v_cache,
                       uint16_t* xh, uint16_t* xl, int C, int n_q, int n_kv, int hd, int L, const int32_t* start,
                       float scale, void* workspace, size_t workspace_bytes, hipStream_t stream);

}  // namespace q4
