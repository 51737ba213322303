// Elementwise fp32 kernels: the generated binary ops and `Process` fill
// (InstructionsToCuda.cs:58-96), saxpy (Kernel.cs:22-28) and sigmoid
// (SigmoidPerformanceTests.cs:27), plus the device-to-device byte copy behind
// sh_copy (also the HBM calibration kernel of the benchmark).
//
// All are HBM-bound streams. Layout for gfx950: 256-thread blocks (4 waves),
// each thread moves kUnroll 16-byte vectors (f32x4) whose addresses are strided by the
// block size, so every load instruction of a wave covers 1 KiB contiguous.
// All loads of a thread are issued before any math, giving 64 B in flight per
// lane; stores are non-temporal so the outputs do not evict inputs from L2.
// Grids are sized to the data (one pass, no grid-stride loop): at 2^24 floats
// that is 4096 blocks, 16 per CU.
#include <hip/hip_runtime.h>

#include "common.h"

namespace sh {
namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 4;
constexpr size_t kPerBlock = (size_t)kBlock * kUnroll;  // f32x4 units per block

// Whether this block's kPerBlock vectors all lie below n (block-uniform).
// Full blocks take a path without per-vector bounds checks: a load under a
// divergent check leaves its register pending at the join, and the compiler
// then waited for each load before issuing the next.
__device__ __forceinline__ bool full_block(size_t n) {
  return ((size_t)blockIdx.x + 1) * kPerBlock <= n;
}

struct AddOp { __device__ float operator()(float a, float b) const { return a + b; } };
struct SubOp { __device__ float operator()(float a, float b) const { return a - b; } };
struct MulOp { __device__ float operator()(float a, float b) const { return a * b; } };
struct DivOp { __device__ float operator()(float a, float b) const { return a / b; } };

// Kernel.cs:26 `a * x + y`; the product is rounded before the add (no FMA), as
// the CPU oracle computes it.
struct SaxpyOp {
  float a;
  __device__ float operator()(float x, float y) const {
#pragma clang fp contract(off)
    float p = a * x;
    return p + y;
  }
};

// SigmoidPerformanceTests.cs:27. expf is ROCm's device-library exp (<= 1 ulp);
// the add and the IEEE divide round once each, so the result stays within
// 2 ulp of the double-exp reference.
struct SigmoidOp {
  __device__ float operator()(float x) const {
    float e = expf(-x);
    return 1.0f / (1.0f + e);
  }
};

__device__ __forceinline__ f32x4 apply(const SigmoidOp &op, f32x4 v) {
  return f32x4{op(v.x), op(v.y), op(v.z), op(v.w)};
}

template <class Op>
__device__ __forceinline__ f32x4 apply2(const Op &op, f32x4 a, f32x4 b) {
  return f32x4{op(a.x, b.x), op(a.y, b.y), op(a.z, b.z), op(a.w, b.w)};
}

template <class Op>
__global__ __launch_bounds__(kBlock) void unary_kernel(const float *__restrict__ x,
                                                       float *__restrict__ y, size_t n, Op op) {
  const size_t n4 = n / 4;
  const f32x4 *x4 = reinterpret_cast<const f32x4 *>(x);
  f32x4 *y4 = reinterpret_cast<f32x4 *>(y);
  const size_t base = (size_t)blockIdx.x * kPerBlock + threadIdx.x;
  f32x4 v[kUnroll];
  if (full_block(n4)) {
#pragma unroll
    for (int u = 0; u < kUnroll; u++) v[u] = __builtin_nontemporal_load(x4 + base + (size_t)u * kBlock);
#pragma unroll
    for (int u = 0; u < kUnroll; u++)
      __builtin_nontemporal_store(apply(op, v[u]), y4 + base + (size_t)u * kBlock);
  } else {
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      size_t i = base + (size_t)u * kBlock;
      if (i < n4) v[u] = __builtin_nontemporal_load(x4 + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      size_t i = base + (size_t)u * kBlock;
      if (i < n4) __builtin_nontemporal_store(apply(op, v[u]), y4 + i);
    }
  }
  // scalar tail (n % 4 elements) in block 0
  if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
    size_t i = n4 * 4 + threadIdx.x;
    y[i] = op(x[i]);
  }
}

template <class Op>
__global__ __launch_bounds__(kBlock) void binary_kernel(const float *__restrict__ a,
                                                        const float *__restrict__ b,
                                                        float *__restrict__ out, size_t n, Op op) {
  const size_t n4 = n / 4;
  const f32x4 *a4 = reinterpret_cast<const f32x4 *>(a);
  const f32x4 *b4 = reinterpret_cast<const f32x4 *>(b);
  f32x4 *o4 = reinterpret_cast<f32x4 *>(out);
  const size_t base = (size_t)blockIdx.x * kPerBlock + threadIdx.x;
  f32x4 va[kUnroll], vb[kUnroll];
  if (full_block(n4)) {
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      va[u] = __builtin_nontemporal_load(a4 + base + (size_t)u * kBlock);
      vb[u] = __builtin_nontemporal_load(b4 + base + (size_t)u * kBlock);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++)
      __builtin_nontemporal_store(apply2(op, va[u], vb[u]), o4 + base + (size_t)u * kBlock);
  } else {
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      size_t i = base + (size_t)u * kBlock;
      if (i < n4) {
        va[u] = __builtin_nontemporal_load(a4 + i);
        vb[u] = __builtin_nontemporal_load(b4 + i);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      size_t i = base + (size_t)u * kBlock;
      if (i < n4) __builtin_nontemporal_store(apply2(op, va[u], vb[u]), o4 + i);
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
    size_t i = n4 * 4 + threadIdx.x;
    out[i] = op(a[i], b[i]);
  }
}

// Unaligned fallbacks: one element per thread.
template <class Op>
__global__ __launch_bounds__(kBlock) void unary_scalar_kernel(const float *x, float *y, size_t n,
                                                              Op op) {
  size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) y[i] = op(x[i]);
}

template <class Op>
__global__ __launch_bounds__(kBlock) void binary_scalar_kernel(const float *a, const float *b,
                                                               float *out, size_t n, Op op) {
  size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) out[i] = op(a[i], b[i]);
}

__global__ __launch_bounds__(kBlock) void fill_kernel(float value, float *__restrict__ out,
                                                      size_t n) {
  size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  size_t n4 = n / 4;
  f32x4 *o4 = reinterpret_cast<f32x4 *>(out);
  for (; i < n4; i += (size_t)gridDim.x * kBlock)
    __builtin_nontemporal_store(f32x4{value, value, value, value}, o4 + i);
  if (blockIdx.x == 0 && threadIdx.x < (n & 3)) out[n4 * 4 + threadIdx.x] = value;
}

__global__ __launch_bounds__(kBlock) void fill_scalar_kernel(float value, float *out, size_t n) {
  size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) out[i] = value;
}

__global__ __launch_bounds__(kBlock) void copy_vec_kernel(const u32x4 *__restrict__ src,
                                                           u32x4 *__restrict__ dst, size_t n16,
                                                           const uint8_t *src_b, uint8_t *dst_b,
                                                           size_t bytes) {
  const size_t base = (size_t)blockIdx.x * kPerBlock + threadIdx.x;
  u32x4 v[kUnroll];
  if (full_block(n16)) {
#pragma unroll
    for (int u = 0; u < kUnroll; u++) v[u] = __builtin_nontemporal_load(src + base + (size_t)u * kBlock);
#pragma unroll
    for (int u = 0; u < kUnroll; u++) __builtin_nontemporal_store(v[u], dst + base + (size_t)u * kBlock);
  } else {
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      size_t i = base + (size_t)u * kBlock;
      if (i < n16) v[u] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      size_t i = base + (size_t)u * kBlock;
      if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < (bytes & 15)) {
    size_t i = n16 * 16 + threadIdx.x;
    dst_b[i] = src_b[i];
  }
}

__global__ __launch_bounds__(kBlock) void copy_byte_kernel(const uint8_t *src, uint8_t *dst,
                                                            size_t bytes) {
  for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < bytes;
       i += (size_t)gridDim.x * kBlock)
    dst[i] = src[i];
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

unsigned vector_grid(size_t n) {
  size_t n4 = n / 4;
  size_t g = (n4 + kPerBlock - 1) / kPerBlock;
  return (unsigned)(g == 0 ? 1 : g);
}

unsigned scalar_grid(size_t n) { return (unsigned)((n + kBlock - 1) / kBlock); }

template <class Op>
hipError_t run_binary(hipStream_t s, const float *a, const float *b, float *out, size_t n, Op op) {
  if (aligned16(a) && aligned16(b) && aligned16(out))
    binary_kernel<<<vector_grid(n), kBlock, 0, s>>>(a, b, out, n, op);
  else
    binary_scalar_kernel<<<scalar_grid(n), kBlock, 0, s>>>(a, b, out, n, op);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_binary_f32(hipStream_t s, int op, const float *a, const float *b, float *out,
                             size_t n) {
  switch (op) {
    case SH_ADD: return run_binary(s, a, b, out, n, AddOp{});
    case SH_SUBTRACT: return run_binary(s, a, b, out, n, SubOp{});
    case SH_MULTIPLY: return run_binary(s, a, b, out, n, MulOp{});
    default: return run_binary(s, a, b, out, n, DivOp{});
  }
}

hipError_t launch_fill_f32(hipStream_t s, float value, float *out, size_t n) {
  if (aligned16(out)) {
    size_t blocks = (n / 4 + kBlock - 1) / kBlock;
    if (blocks > 8192) blocks = 8192;
    if (blocks == 0) blocks = 1;
    fill_kernel<<<(unsigned)blocks, kBlock, 0, s>>>(value, out, n);
  } else {
    fill_scalar_kernel<<<scalar_grid(n), kBlock, 0, s>>>(value, out, n);
  }
  return hipGetLastError();
}

hipError_t launch_saxpy_f32(hipStream_t s, float a, const float *x, const float *y, float *out,
                            size_t n) {
  return run_binary(s, x, y, out, n, SaxpyOp{a});
}

hipError_t launch_copy_bytes(hipStream_t s, void *dst, const void *src, size_t bytes) {
  const uint8_t *sb = static_cast<const uint8_t *>(src);
  uint8_t *db = static_cast<uint8_t *>(dst);
  if (aligned16(src) && aligned16(dst)) {
    const size_t n16 = bytes / 16;
    size_t g = (n16 + kPerBlock - 1) / kPerBlock;
    copy_vec_kernel<<<(unsigned)(g == 0 ? 1 : g), kBlock, 0, s>>>(
        reinterpret_cast<const u32x4 *>(src), reinterpret_cast<u32x4 *>(dst), n16, sb, db, bytes);
  } else {
    size_t g = (bytes + kBlock - 1) / kBlock;
    copy_byte_kernel<<<(unsigned)(g > 65536 ? 65536 : g), kBlock, 0, s>>>(sb, db, bytes);
  }
  return hipGetLastError();
}

hipError_t launch_sigmoid_f32(hipStream_t s, const float *x, float *y, size_t n) {
  if (aligned16(x) && aligned16(y))
    unary_kernel<<<vector_grid(n), kBlock, 0, s>>>(x, y, n, SigmoidOp{});
  else
    unary_scalar_kernel<<<scalar_grid(n), kBlock, 0, s>>>(x, y, n, SigmoidOp{});
  return hipGetLastError();
}

}  // namespace sh
