// Device helpers shared by the LLM kernels (llm_kernels.hip) and the
// persistent decode-layers kernel (decode_layers.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"
#include "llm.h"

namespace sh {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// DPP lane moves within rows of 16 lanes (no LDS round trip, unlike the
// ds_bpermute behind __shfl_xor): quad_perm [1,0,3,2] = 0xB1,
// quad_perm [2,3,0,1] = 0x4E, row_ror:4 = 0x124, row_ror:8 = 0x128.
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}

// Sum over each row of 16 lanes, in every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x124>(v);
  v += dpp_f32<0x128>(v);
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x124>(v));
  v = fmaxf(v, dpp_f32<0x128>(v));
  return v;
}

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Wave-wide sum / max, the same (uniform) value in every lane.
__device__ __forceinline__ float wave_sum_rows(float v) {
  v = row16_sum(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

__device__ __forceinline__ float wave_max_rows(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// Order-preserving key of an fp32 logit with its column: larger logits give
// larger keys; among equal logits the smaller column wins (as argmax does).
__device__ __forceinline__ unsigned long long argmax_key(float v, int n) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)n);
}

// The token of batch row b: the largest of its keys over the kKeySlots slots
// of key set `keys` (token = ~ low word; out-of-vocabulary tokens read as 0).
// Called by a whole wave; the result is wave-uniform.
__device__ __forceinline__ int step_token(const unsigned long long *keys, int b, int vocab) {
  const int lane = threadIdx.x & 63;
  unsigned long long key = 0;
  if (lane < kKeySlots)
    key = __hip_atomic_load(keys + (size_t)lane * kKeyStride + b, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(key, off, 64);
    key = o > key ? o : key;
  }
  int tok = (int)(0xffffffffu - (uint32_t)(key & 0xffffffffu));
  if (tok < 0 || tok >= vocab) tok = 0;
  return __builtin_amdgcn_readfirstlane(tok);
}

// Byte offset of W[n][k] in an FP8 tiled matrix with K columns (1 KiB tiles
// of 16 rows x 64 K; 8 consecutive k of a row are contiguous).
__device__ __forceinline__ size_t fp8_tiled_offset(int n, int k, int K) {
  const int kt = k >> 6, k64 = k & 63, half = k64 >> 5, kk = k64 & 31;
  const int lane = (n & 15) + 16 * (kk >> 3);
  return ((size_t)(n >> 4) * (size_t)(K >> 6) + (size_t)kt) * 1024 + (size_t)lane * 16 +
         (size_t)(half * 8 + (kk & 7));
}

// Element offset of W[n][k] in an fp16 tiled matrix with K columns (1 KiB
// tiles of 16 rows x 32 K; 8 consecutive k of a row are contiguous).
__device__ __forceinline__ size_t f16_tiled_offset(int n, int k, int K) {
  const int kt = k >> 5, kk = k & 31;
  const int lane = (n & 15) + 16 * (kk >> 3);
  return (((size_t)(n >> 4) * (size_t)(K >> 5) + (size_t)kt) * 64 + (size_t)lane) * 8 +
         (size_t)(kk & 7);
}

__device__ __forceinline__ float gelu_tanh(float x) {
  const float c = 0.7978845608028654f;  // sqrt(2 / pi)
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

// Eight fp16 MFMA B-operand values from 8 E4M3 bytes (two dwords), exact.
__device__ __forceinline__ f16x8 e4m3x8_to_f16(uint32_t d0, uint32_t d1) {
  const f16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, false);
  const f16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, true);
  const f16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, false);
  const f16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, true);
  return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

}  // namespace sh
