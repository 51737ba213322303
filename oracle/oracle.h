/*
 * CPU oracle for the Strict GPU kernel path -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain C restatement of the reference's CPU semantics (strict-lang/Strict, C#)
 * for the ops that libstrict_hip runs on the GPU. Only tests/, the smoke check
 * and bench.py's cpu_baseline leg may load this library; the product path never
 * does. Every function cites the reference file:line it restates, or says that
 * the reference has no implementation and what fixes the semantics instead.
 *
 * Compiled with -ffp-contract=off so that every float operation rounds exactly
 * where the C# source rounds.
 */
#ifndef STRICT_ORACLE_H
#define STRICT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Binary elementwise ops of the generated kernels (InstructionsToCuda.cs:58-73,
 * operator table :101-109): output[i] = first[i] OP second[i]. */
enum { OR_ADD = 0, OR_SUBTRACT = 1, OR_MULTIPLY = 2, OR_DIVIDE = 3 };
void or_binary_f32(int op, const float *first, const float *second, float *output, size_t count);

/* Scalar broadcast of the generated `Process` kernel (InstructionsToCuda.cs:79-96,
 * CSharpToCudaTranspilerTests.cs:80-87): output[i] = initialDepth. */
void or_fill_f32(float value, float *output, size_t count);

/* saxpy of Kernel.cs:22-28: out[i] = a * x[i] + y[i] (multiply and add rounded
 * separately). */
void or_saxpy_f32(float a, const float *x, const float *y, float *out, size_t n);

/* SigmoidPerformanceTests.cs:27: 1.0f / (1.0f + (float)Math.Exp(-x)), the
 * exponential in double, the rest in float. nthreads <= 1 runs serially. */
void or_sigmoid_f32(const float *x, float *y, size_t n, int nthreads);

/* Assembly.Tests/BlurPerformanceTests.cs:287-294 (AdjustPixelBrightness):
 * p' = (byte)clamp(p + delta, 0, 255) on channels 0..2 of each pixel.
 * `channels` is the bytes per pixel (3 as in the reference, or 4 for RGBA);
 * the 4th byte (alpha) passes through unless all_channels != 0. */
void or_adjust_brightness(const uint8_t *in, uint8_t *out, size_t pixels, int channels,
                          int delta, int all_channels, int nthreads);

/* Assembly.Tests/BlurPerformanceTests.cs:53-141 (ApplyBlurSingleThread,
 * BlurInteriorPixel, BlurEdgePixel): 5x5 box per channel, interior sum/25
 * truncating, border pixels average over in-bounds taps (sum/count truncating).
 * `channels` bytes per pixel, all channels blurred. Out of place. */
void or_blur5_reference(const uint8_t *in, uint8_t *out, int width, int height, int channels,
                        int nthreads);

/* Config semantics (no reference implementation; fixed by BASELINE.json
 * configs[1]): 5x5 box, clamp-to-edge coordinates, (sum + 12) / 25. */
void or_blur5_config(const uint8_t *in, uint8_t *out, int width, int height, int channels,
                     int nthreads);

/* Brightness then config blur, as two passes over a temporary image. */
void or_brightness_blur5_config(const uint8_t *in, uint8_t *out, int width, int height,
                                int channels, int delta, int all_channels, int nthreads);

/* TestPerformance's CPU modes (Strict.Compiler.Cuda.Tests/TestPerformance.cs:34-49):
 * SingleThread, SingleThreadChunks, ParallelCpu, ParallelCpuChunks. Each
 * or_perf_* call runs one mode of one workload's RunChunk(start, chunk) over
 * `iterations` indices (chunk = ChunkSize, 100 in the reference's tests) on
 * up to nthreads threads and returns the wall time in ms. */
enum {
  OR_SINGLE_THREAD = 0,
  OR_SINGLE_THREAD_CHUNKS = 1,
  OR_PARALLEL_CPU = 2,
  OR_PARALLEL_CPU_CHUNKS = 3
};
/* index n: y[n] = sigmoid(x[n]) (SigmoidPerformanceTests.cs:24-28, over an array) */
double or_perf_sigmoid(int mode, const float *x, float *y, long n, int chunk, int nthreads);
/* index n: pixel n of AdjustPixelBrightness (Assembly BlurPerformanceTests.cs:287-294) */
double or_perf_brightness(int mode, const uint8_t *in, uint8_t *out, long pixels, int channels,
                          int delta, int chunk, int nthreads);
/* index n < pixels: output pixel n of a 5x5 blur; kind 0 = reference semantics
 * (or_blur5_reference), 1 = config semantics (or_blur5_config), 2 = config blur of
 * the taps brightened by delta on channels 0..2 (the fused brightness + blur) */
double or_perf_blur5(int mode, int kind, const uint8_t *in, uint8_t *out, int width, int height,
                     int channels, int delta, long pixels, int chunk, int nthreads);
/* the same over output pixels [first, first + pixels) (index n is pixel first + n):
 * the CPU share of TestPerformance's CudaGpuAndCpu mode (TestPerformance.cs:53-61) */
double or_perf_blur5_from(int mode, int kind, const uint8_t *in, uint8_t *out, int width,
                          int height, int channels, int delta, long first, long pixels, int chunk,
                          int nthreads);
/* Cuda.Tests/BlurPerformanceTests.cs:160-169: the in-place 5-point cross /5
 * over the RGBA byte stream, indices modulo width * height * 4, chunks
 * starting below width * 4 skipped; the reference runs width * height * 100
 * (its logged counts) or * 200 (its constant, :106) iterations. */
double or_perf_cross_blur(int mode, uint8_t *image, int width, int height, long iterations,
                          int chunk, int nthreads);

/* Number formats (no reference implementation; IEEE 754 / OCP 8-bit FP spec). */
uint16_t or_f32_to_bf16(float f);   /* round to nearest even, NaN kept quiet */
float or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);    /* round to nearest even, overflow -> inf */
float or_f16_to_f32(uint16_t h);
uint8_t or_f32_to_e4m3(float f);    /* OCP E4M3 (bias 7, max 448), RNE, saturating */
float or_e4m3_to_f32(uint8_t q);

void or_f32_to_bf16_array(const float *in, uint16_t *out, size_t n);
void or_bf16_to_f32_array(const uint16_t *in, float *out, size_t n);
void or_f32_to_f16_array(const float *in, uint16_t *out, size_t n);
void or_f16_to_f32_array(const uint16_t *in, float *out, size_t n);
void or_e4m3_to_f32_array(const uint8_t *in, float *out, size_t n);

/* Per-row FP8 quantization of a [rows x cols] fp32 matrix (one scale per row):
 * scale = max|w| / 448 (1 if the row is all zero), q = e4m3(w / scale). */
void or_quantize_e4m3_rows(const float *w, int rows, int cols, uint8_t *q, float *scales,
                           int nthreads);

/* C[M,N] = A[M,K] * B[K,N] with double accumulation, all fp32 row-major
 * (bf16/fp8 operands are widened by the caller). */
void or_gemm_f32(const float *a, const float *b, float *c, int m, int n, int k, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
