/*
 * CPU oracle for the Strict GPU kernel path -- TEST INFRASTRUCTURE ONLY.
 * See oracle.h for the contract; each function cites the reference line it
 * restates. Built by oracle/Makefile with -ffp-contract=off.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <time.h>
#include <stdlib.h>
#include <string.h>

/* ---- tiny parallel-for over [0, n) in contiguous ranges ------------------ */

typedef void (*range_fn)(void *ctx, size_t begin, size_t end);

typedef struct {
  range_fn fn;
  void *ctx;
  size_t begin, end;
} range_job;

static void *range_thread(void *p) {
  range_job *job = (range_job *)p;
  job->fn(job->ctx, job->begin, job->end);
  return NULL;
}

/* Mirrors TestPerformance.cs:46-49 (Parallel.For over chunks): the range is
 * cut into nthreads contiguous chunks, each run on its own thread. */
static void parallel_for(size_t n, int nthreads, range_fn fn, void *ctx) {
  if (nthreads <= 1 || n < 2) {
    fn(ctx, 0, n);
    return;
  }
  if ((size_t)nthreads > n) nthreads = (int)n;
  pthread_t *threads = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
  range_job *jobs = (range_job *)malloc(sizeof(range_job) * (size_t)nthreads);
  size_t chunk = (n + (size_t)nthreads - 1) / (size_t)nthreads;
  int started = 0;
  for (int t = 0; t < nthreads; t++) {
    size_t b = (size_t)t * chunk, e = b + chunk;
    if (b >= n) break;
    if (e > n) e = n;
    jobs[t].fn = fn;
    jobs[t].ctx = ctx;
    jobs[t].begin = b;
    jobs[t].end = e;
    if (pthread_create(&threads[t], NULL, range_thread, &jobs[t]) != 0) {
      fn(ctx, b, e); /* no thread available: run inline */
      threads[t] = 0;
    }
    started = t + 1;
  }
  for (int t = 0; t < started; t++)
    if (threads[t]) pthread_join(threads[t], NULL);
  free(threads);
  free(jobs);
}

/* ---- generated elementwise kernels ------------------------------------- */

void or_binary_f32(int op, const float *first, const float *second, float *output,
                   size_t count) {
  /* InstructionsToCuda.cs:72 `output[idx] = first[idx] OP second[idx]`,
   * operators from GetOperatorSymbol (:101-109). */
  for (size_t i = 0; i < count; i++) {
    float a = first[i], b = second[i];
    switch (op) {
      case OR_ADD: output[i] = a + b; break;
      case OR_SUBTRACT: output[i] = a - b; break;
      case OR_MULTIPLY: output[i] = a * b; break;
      default: output[i] = a / b; break;
    }
  }
}

void or_fill_f32(float value, float *output, size_t count) {
  /* Output/InitializeDepths.cu:10 / InstructionsToCuda.cs:72 with the return
   * expression `initialDepth`. */
  for (size_t i = 0; i < count; i++) output[i] = value;
}

void or_saxpy_f32(float a, const float *x, const float *y, float *out, size_t n) {
  /* Kernel.cs:26 `out[tid] = a * x[tid] + y[tid]`, product rounded first. */
  for (size_t i = 0; i < n; i++) {
    float p = a * x[i];
    out[i] = p + y[i];
  }
}

/* ---- sigmoid ------------------------------------------------------------- */

typedef struct {
  const float *x;
  float *y;
} sigmoid_ctx;

static void sigmoid_range(void *p, size_t b, size_t e) {
  sigmoid_ctx *c = (sigmoid_ctx *)p;
  for (size_t i = b; i < e; i++) {
    /* SigmoidPerformanceTests.cs:27: -Input is a float negation, Math.Exp is
     * double, the cast back to float happens before the float add/divide. */
    float neg = -c->x[i];
    float ex = (float)exp((double)neg);
    float den = 1.0f + ex;
    c->y[i] = 1.0f / den;
  }
}

void or_sigmoid_f32(const float *x, float *y, size_t n, int nthreads) {
  sigmoid_ctx c = {x, y};
  parallel_for(n, nthreads, sigmoid_range, &c);
}

/* ---- brightness ---------------------------------------------------------- */

typedef struct {
  const uint8_t *in;
  uint8_t *out;
  int channels, delta, all_channels;
} brightness_ctx;

static void brightness_range(void *p, size_t b, size_t e) {
  brightness_ctx *c = (brightness_ctx *)p;
  int adjusted = c->channels < 3 ? c->channels : 3;
  if (c->all_channels) adjusted = c->channels;
  for (size_t px = b; px < e; px++) {
    size_t base = px * (size_t)c->channels;
    /* BlurPerformanceTests.cs:289-293: channel loop 0..2,
     * (byte)Math.Clamp(pixels[index] + delta, 0, 255). */
    for (int ch = 0; ch < c->channels; ch++) {
      int v = c->in[base + ch];
      if (ch < adjusted) {
        v += c->delta;
        if (v < 0) v = 0;
        if (v > 255) v = 255;
      }
      c->out[base + ch] = (uint8_t)v;
    }
  }
}

void or_adjust_brightness(const uint8_t *in, uint8_t *out, size_t pixels, int channels,
                          int delta, int all_channels, int nthreads) {
  brightness_ctx c = {in, out, channels, delta, all_channels};
  parallel_for(pixels, nthreads, brightness_range, &c);
}

/* ---- blur, reference semantics ----------------------------------------- */

typedef struct {
  const uint8_t *in;
  uint8_t *out;
  int width, height, channels;
} blur_ctx;

static void blur_reference_rows(void *p, size_t rb, size_t re) {
  blur_ctx *c = (blur_ctx *)p;
  const int w = c->width, h = c->height, ch = c->channels;
  const size_t stride = (size_t)w * (size_t)ch; /* :56 stride = width * 3 */
  for (size_t row = rb; row < re; row++) {
    for (int col = 0; col < w; col++) {
      size_t base = row * stride + (size_t)col * (size_t)ch;
      int interior = (int)row >= 2 && (int)row < h - 2 && col >= 2 && col < w - 2; /* :60 */
      for (int k = 0; k < ch; k++) {
        int sum = 0, count = 0;
        for (int ky = -2; ky <= 2; ky++)
          for (int kx = -2; kx <= 2; kx++) {
            int nx = col + kx, ny = (int)row + ky;
            /* :134 unsigned compare skips out-of-bounds taps (edge only) */
            if ((unsigned)nx >= (unsigned)w || (unsigned)ny >= (unsigned)h) continue;
            sum += c->in[(size_t)ny * stride + (size_t)nx * (size_t)ch + (size_t)k];
            count++;
          }
        /* interior: sum / 25 (:117); edge: sum / count (:139); both truncate.
         * For interior pixels count is always 25, so one formula covers both. */
        c->out[base + (size_t)k] = (uint8_t)(interior ? sum / 25 : sum / count);
      }
    }
  }
}

void or_blur5_reference(const uint8_t *in, uint8_t *out, int width, int height, int channels,
                        int nthreads) {
  blur_ctx c = {in, out, width, height, channels};
  /* rows in parallel as ApplyBlurParallel (:72) */
  parallel_for((size_t)height, nthreads, blur_reference_rows, &c);
}

/* ---- blur, config semantics -------------------------------------------- */

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

static void blur_config_rows(void *p, size_t rb, size_t re) {
  blur_ctx *c = (blur_ctx *)p;
  const int w = c->width, h = c->height, ch = c->channels;
  const size_t stride = (size_t)w * (size_t)ch;
  for (size_t row = rb; row < re; row++)
    for (int col = 0; col < w; col++)
      for (int k = 0; k < ch; k++) {
        int sum = 0;
        for (int ky = -2; ky <= 2; ky++) {
          int ny = clampi((int)row + ky, 0, h - 1);
          for (int kx = -2; kx <= 2; kx++) {
            int nx = clampi(col + kx, 0, w - 1);
            sum += c->in[(size_t)ny * stride + (size_t)nx * (size_t)ch + (size_t)k];
          }
        }
        c->out[row * stride + (size_t)col * (size_t)ch + (size_t)k] = (uint8_t)((sum + 12) / 25);
      }
}

void or_blur5_config(const uint8_t *in, uint8_t *out, int width, int height, int channels,
                     int nthreads) {
  blur_ctx c = {in, out, width, height, channels};
  parallel_for((size_t)height, nthreads, blur_config_rows, &c);
}

void or_brightness_blur5_config(const uint8_t *in, uint8_t *out, int width, int height,
                                int channels, int delta, int all_channels, int nthreads) {
  size_t bytes = (size_t)width * (size_t)height * (size_t)channels;
  uint8_t *tmp = (uint8_t *)malloc(bytes ? bytes : 1);
  or_adjust_brightness(in, tmp, (size_t)width * (size_t)height, channels, delta, all_channels,
                       nthreads);
  or_blur5_config(tmp, out, width, height, channels, nthreads);
  free(tmp);
}

/* ---- TestPerformance's CPU modes ----------------------------------------
 *
 * Strict.Compiler.Cuda.Tests/TestPerformance.cs:34-49 times one workload
 * `RunChunk(start, chunkSize)` four ways: SingleThread (RunChunk(i, 1) for
 * every i), SingleThreadChunks (RunChunk(i * ChunkSize, ChunkSize) for every
 * chunk), ParallelCpu (Parallel.For over i, RunChunk(i, 1)) and
 * ParallelCpuChunks (Parallel.For over chunks). The chunk functions are
 * called through a function pointer, as the C# delegate is, and are never
 * inlined into the loops. Parallel.For is restated as a pool of `nthreads`
 * threads taking ranges of indices from a shared counter (dynamic range
 * partitioning). Each run returns its wall time in ms (Stopwatch, :26-29). */

typedef void (*chunk_fn)(void *ctx, long start, long chunk);

typedef struct {
  chunk_fn fn;
  void *ctx;
  long items;  /* indices handed out: iterations, or chunks */
  long grain;  /* indices per grab */
  int chunk;   /* 0: fn(i, 1) per index; else fn(i * chunk, chunk) */
  long next;   /* shared counter (atomic) */
} perf_job;

static void run_indices(perf_job *j, long b, long e) {
  if (j->chunk)
    for (long k = b; k < e; k++) j->fn(j->ctx, k * (long)j->chunk, j->chunk);
  else
    for (long k = b; k < e; k++) j->fn(j->ctx, k, 1);
}

static void *perf_worker(void *p) {
  perf_job *j = (perf_job *)p;
  for (;;) {
    long b = __atomic_fetch_add(&j->next, j->grain, __ATOMIC_RELAXED);
    if (b >= j->items) break;
    long e = b + j->grain < j->items ? b + j->grain : j->items;
    run_indices(j, b, e);
  }
  return NULL;
}

static double now_ms(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec * 1e3 + (double)ts.tv_nsec * 1e-6;
}

__attribute__((noipa)) static double perf_run(int mode, long iterations, int chunk_size, chunk_fn fn,
                                              void *ctx, int nthreads) {
  perf_job j;
  j.fn = fn;
  j.ctx = ctx;
  j.next = 0;
  const int chunked = mode == OR_SINGLE_THREAD_CHUNKS || mode == OR_PARALLEL_CPU_CHUNKS;
  j.chunk = chunked ? chunk_size : 0;
  j.items = chunked ? iterations / chunk_size : iterations; /* :41, :48 */
  j.grain = chunked ? 16 : 4096;
  const double t0 = now_ms();
  if (mode == OR_SINGLE_THREAD || mode == OR_SINGLE_THREAD_CHUNKS || nthreads <= 1) {
    run_indices(&j, 0, j.items);
  } else {
    pthread_t *threads = (pthread_t *)calloc((size_t)nthreads, sizeof(pthread_t));
    int started = 0;
    for (int t = 0; t < nthreads; t++)
      if (pthread_create(&threads[t], NULL, perf_worker, &j) == 0) started++;
      else break;
    if (started == 0) run_indices(&j, 0, j.items);
    for (int t = 0; t < started; t++) pthread_join(threads[t], NULL);
    free(threads);
  }
  return now_ms() - t0;
}

/* SigmoidPerformanceTests.SigmoidOutput (:24-28) over the config's array:
 * element n of x -> y[n], the arithmetic of or_sigmoid_f32. */
__attribute__((noinline)) static void sigmoid_chunk(void *p, long start, long chunk) {
  sigmoid_range(p, (size_t)start, (size_t)(start + chunk));
}

double or_perf_sigmoid(int mode, const float *x, float *y, long n, int chunk, int nthreads) {
  sigmoid_ctx c = {x, y};
  return perf_run(mode, n, chunk, sigmoid_chunk, &c, nthreads);
}

/* AdjustPixelBrightness (Assembly.Tests/BlurPerformanceTests.cs:287-294),
 * one pixel per index. */
__attribute__((noinline)) static void brightness_chunk(void *p, long start, long chunk) {
  brightness_range(p, (size_t)start, (size_t)(start + chunk));
}

double or_perf_brightness(int mode, const uint8_t *in, uint8_t *out, long pixels, int channels,
                          int delta, int chunk, int nthreads) {
  brightness_ctx c = {in, out, channels, delta, 0};
  return perf_run(mode, pixels, chunk, brightness_chunk, &c, nthreads);
}

/* 5x5 blurs, one output pixel per index (pixel n = row n / width, column
 * n % width): the reference semantics of or_blur5_reference
 * (BlurPerformanceTests.cs:85-141), the config semantics of or_blur5_config,
 * and the config blur of brightened taps (the fused kernel's result). */
typedef struct {
  const uint8_t *in;
  uint8_t *out;
  int width, height, channels, delta, kind;
  long first; /* index 0 is output pixel `first` */
} blur_px_ctx;

static void blur_pixel(const blur_px_ctx *c, int row, int col) {
  const int w = c->width, h = c->height, ch = c->channels;
  const size_t stride = (size_t)w * (size_t)ch, base = (size_t)row * stride + (size_t)col * (size_t)ch;
  const int interior = row >= 2 && row < h - 2 && col >= 2 && col < w - 2;
  for (int k = 0; k < ch; k++) {
    int sum = 0, count = 0;
    for (int ky = -2; ky <= 2; ky++)
      for (int kx = -2; kx <= 2; kx++) {
        int ny = row + ky, nx = col + kx;
        if (c->kind == 0) { /* reference: in-bounds taps only */
          if ((unsigned)nx >= (unsigned)w || (unsigned)ny >= (unsigned)h) continue;
        } else {
          ny = clampi(ny, 0, h - 1);
          nx = clampi(nx, 0, w - 1);
        }
        int v = c->in[(size_t)ny * stride + (size_t)nx * (size_t)ch + (size_t)k];
        if (c->kind == 2 && k < 3) v = clampi(v + c->delta, 0, 255);
        sum += v;
        count++;
      }
    c->out[base + (size_t)k] =
        (uint8_t)(c->kind == 0 ? (interior ? sum / 25 : sum / count) : (sum + 12) / 25);
  }
}

__attribute__((noinline)) static void blur_chunk(void *p, long start, long chunk) {
  const blur_px_ctx *c = (const blur_px_ctx *)p;
  for (long n = c->first + start; n < c->first + start + chunk; n++)
    blur_pixel(c, (int)(n / c->width), (int)(n % c->width));
}

double or_perf_blur5(int mode, int kind, const uint8_t *in, uint8_t *out, int width, int height,
                     int channels, int delta, long pixels, int chunk, int nthreads) {
  return or_perf_blur5_from(mode, kind, in, out, width, height, channels, delta, 0, pixels, chunk,
                            nthreads);
}

double or_perf_blur5_from(int mode, int kind, const uint8_t *in, uint8_t *out, int width,
                          int height, int channels, int delta, long first, long pixels, int chunk,
                          int nthreads) {
  blur_px_ctx c = {in, out, width, height, channels, delta, kind, first};
  long total = (long)width * (long)height;
  if (first < 0 || first > total) return -1.0;
  if (pixels > total - first) pixels = total - first;
  return perf_run(mode, pixels, chunk, blur_chunk, &c, nthreads);
}

/* The CUDA harness's CPU blur (Strict.Compiler.Cuda.Tests/BlurPerformanceTests.cs:160-169):
 * in place over the RGBA byte stream of `size` = width * height * 4 bytes,
 * for every index n of the chunk (chunks starting below width * 4 are skipped
 * whole, :162-163):
 *   image[n % size] = (image[n % size] + image[(n - 4w) % size] + image[(n - 4) % size]
 *                      + image[(n + 4) % size] + image[(n + 4w) % size]) / 5
 * The byte accesses are relaxed atomics, so the parallel modes' overlapping
 * in-place updates (a race in the reference too) stay defined; on x86 they
 * are plain byte loads and stores. */
typedef struct {
  uint8_t *image;
  long size, w4;
} cross_ctx;

static inline int cross_ld(const cross_ctx *c, long i) {
  return __atomic_load_n(c->image + i, __ATOMIC_RELAXED);
}

__attribute__((noinline)) static void cross_blur_chunk(void *p, long start, long chunk) {
  const cross_ctx *c = (const cross_ctx *)p;
  if (start < c->w4) return;
  const long size = c->size;
  for (long n = start; n < start + chunk; n++) {
    int sum = cross_ld(c, n % size) + cross_ld(c, (n - c->w4) % size) + cross_ld(c, (n - 4) % size) +
              cross_ld(c, (n + 4) % size) + cross_ld(c, (n + c->w4) % size);
    __atomic_store_n(c->image + n % size, (uint8_t)(sum / 5), __ATOMIC_RELAXED);
  }
}

double or_perf_cross_blur(int mode, uint8_t *image, int width, int height, long iterations,
                          int chunk, int nthreads) {
  cross_ctx c = {image, (long)width * (long)height * 4, (long)width * 4};
  return perf_run(mode, iterations, chunk, cross_blur_chunk, &c, nthreads);
}

/* ---- number formats ------------------------------------------------------ */

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t or_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
  uint32_t rounding = 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)((u + rounding) >> 16);
}

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t or_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u); /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {
    /* below 2^-14: fp16 subnormal. value = a_float; units of 2^-24 */
    if (a < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
    uint32_t e = a >> 23;
    uint32_t m = (a & 0x7fffffu) | 0x800000u;
    /* value = m * 2^(e-150); want units of 2^-24: shift = 150-24 - e = 126 - e */
    uint32_t shift = 126u - e;
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  /* normal: rebias exponent 127 -> 15, keep 10 mantissa bits with RNE */
  uint32_t r = a - 0x38000000u; /* exponent - 112 */
  uint32_t q = r >> 13;
  uint32_t rem = r & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
    return sign ? -v : v;
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

float or_e4m3_to_f32(uint8_t q) {
  /* OCP OFP8 E4M3: 1 sign, 4 exponent (bias 7), 3 mantissa; S.1111.111 = NaN;
   * no infinities; max normal 0x7E = 448. */
  int s = q >> 7, e = (q >> 3) & 0xf, m = q & 7;
  float v;
  if (e == 15 && m == 7) return s ? -NAN : NAN;
  if (e == 0)
    v = ldexpf((float)m, -9); /* subnormal m/8 * 2^-6 */
  else
    v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return s ? -v : v;
}

uint8_t or_f32_to_e4m3(float f) {
  uint8_t sign = (f2u(f) >> 24) & 0x80u;
  if (isnan(f)) return (uint8_t)(sign | 0x7fu);
  float a = fabsf(f);
  if (a >= 448.0f) return (uint8_t)(sign | 0x7eu); /* saturate */
  /* Scan the 127 finite magnitudes: pick the nearest, ties to even code. */
  uint8_t best = 0;
  float best_err = INFINITY;
  for (int c = 0; c <= 0x7e; c++) {
    float v = or_e4m3_to_f32((uint8_t)c);
    float err = fabsf(v - a);
    if (err < best_err || (err == best_err && (c & 1) == 0)) {
      best = (uint8_t)c;
      best_err = err;
    }
    if (v > a) break; /* magnitudes increase with the code */
  }
  return (uint8_t)(sign | best);
}

void or_f32_to_bf16_array(const float *in, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = or_f32_to_bf16(in[i]);
}
void or_bf16_to_f32_array(const uint16_t *in, float *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = or_bf16_to_f32(in[i]);
}
void or_f32_to_f16_array(const float *in, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = or_f32_to_f16(in[i]);
}
void or_f16_to_f32_array(const uint16_t *in, float *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(in[i]);
}
void or_e4m3_to_f32_array(const uint8_t *in, float *out, size_t n) {
  float table[256];
  for (int c = 0; c < 256; c++) table[c] = or_e4m3_to_f32((uint8_t)c);
  for (size_t i = 0; i < n; i++) out[i] = table[in[i]];
}

typedef struct {
  const float *w;
  int cols;
  uint8_t *q;
  float *scales;
} quant_ctx;

static void quant_rows(void *p, size_t rb, size_t re) {
  quant_ctx *c = (quant_ctx *)p;
  for (size_t r = rb; r < re; r++) {
    const float *row = c->w + r * (size_t)c->cols;
    float amax = 0.0f;
    for (int j = 0; j < c->cols; j++) {
      float a = fabsf(row[j]);
      if (a > amax) amax = a;
    }
    float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
    c->scales[r] = scale;
    for (int j = 0; j < c->cols; j++) c->q[r * (size_t)c->cols + (size_t)j] = or_f32_to_e4m3(row[j] / scale);
  }
}

void or_quantize_e4m3_rows(const float *w, int rows, int cols, uint8_t *q, float *scales,
                           int nthreads) {
  quant_ctx c = {w, cols, q, scales};
  parallel_for((size_t)rows, nthreads, quant_rows, &c);
}

typedef struct {
  const float *a, *b;
  float *c;
  int n, k;
} gemm_ctx;

static void gemm_rows(void *p, size_t rb, size_t re) {
  gemm_ctx *g = (gemm_ctx *)p;
  double *acc = (double *)malloc(sizeof(double) * (size_t)g->n);
  for (size_t i = rb; i < re; i++) {
    for (int j = 0; j < g->n; j++) acc[j] = 0.0;
    for (int kk = 0; kk < g->k; kk++) {
      double av = g->a[i * (size_t)g->k + (size_t)kk];
      const float *brow = g->b + (size_t)kk * (size_t)g->n;
      for (int j = 0; j < g->n; j++) acc[j] += av * (double)brow[j];
    }
    for (int j = 0; j < g->n; j++) g->c[i * (size_t)g->n + (size_t)j] = (float)acc[j];
  }
  free(acc);
}

void or_gemm_f32(const float *a, const float *b, float *c, int m, int n, int k, int nthreads) {
  gemm_ctx g = {a, b, c, n, k};
  parallel_for((size_t)m, nthreads, gemm_rows, &g);
}
