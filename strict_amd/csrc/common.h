// Internal declarations shared by the runtime (runtime.hip) and the kernel
// translation units. Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "strict_hip.h"

namespace sh {

// Native clang vectors (HIP's float4/uint4 are structs, which the
// nontemporal builtins and 16-byte LDS accesses do not take).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Records `message` as this thread's last error and returns `status`.
int fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps a failed HIP call to SH_ERR_HIP / SH_ERR_OUT_OF_MEMORY with its text.
int hip_fail(hipError_t err, const char *what);
void clear_error();

struct Context;
// Checks that [ptr, ptr + bytes) lies inside one tracked allocation of ctx.
int check_range(sh_ctx *ctx, const void *ptr, size_t bytes, const char *name);
hipStream_t stream_of(sh_ctx *ctx);
// The context's work buffer of at least `bytes` (grown on demand, freed by
// sh_destroy). Typed ops ordered on the context's stream share it.
int context_scratch(sh_ctx *ctx, size_t bytes, void **ptr);
int device_of(sh_ctx *ctx);
// Makes ctx's device current on the calling thread.
int enter(sh_ctx *ctx);

// ---- kernel launchers (return the hipGetLastError of the launch) ---------
hipError_t launch_binary_f32(hipStream_t s, int op, const float *a, const float *b, float *out,
                             size_t n);
hipError_t launch_fill_f32(hipStream_t s, float value, float *out, size_t n);
hipError_t launch_saxpy_f32(hipStream_t s, float a, const float *x, const float *y, float *out,
                            size_t n);
hipError_t launch_sigmoid_f32(hipStream_t s, const float *x, float *y, size_t n);
hipError_t launch_copy_bytes(hipStream_t s, void *dst, const void *src, size_t bytes);

hipError_t launch_gemm_bf16(hipStream_t s, const uint16_t *A, const uint16_t *B, uint16_t *C,
                            int M, int N, int K, int lda, int ldb, int ldc);
bool gemm_bf16_uses_mfma(int M, int N, int K, int lda, int ldb, int ldc, const void *A,
                         const void *B, const void *C);
hipError_t launch_gemm_fp8(hipStream_t s, const uint8_t *A, const float *sa, const uint8_t *Bt,
                           const float *sb, uint16_t *C, int M, int N, int K, int lda, int ldb,
                           int ldc);
bool gemm_fp8_uses_mfma(int M, int N, int K, int lda, int ldb, int ldc, const void *A,
                        const void *Bt, const void *C, const void *sb);

hipError_t launch_bgr_to_rgba_u8(hipStream_t s, const uint8_t *src, int bpp, size_t src_stride,
                                 uint32_t *dst, int width, int height);
hipError_t launch_rgb_to_bgr_u8(hipStream_t s, const uint8_t *src, uint8_t *dst, int width,
                                int height, size_t dst_stride);
hipError_t launch_brightness_u8(hipStream_t s, const uint8_t *in, uint8_t *out, size_t bytes,
                                int channels, int delta, int all_channels);
hipError_t launch_blur5_u8(hipStream_t s, const uint8_t *in, uint8_t *out, int width, int height,
                           int channels, int mode, bool fuse_brightness, int delta,
                           int all_channels);

}  // namespace sh

#define SH_HIP_TRY(expr)                                 \
  do {                                                   \
    hipError_t sh_err_ = (expr);                         \
    if (sh_err_ != hipSuccess) return ::sh::hip_fail(sh_err_, #expr); \
  } while (0)
