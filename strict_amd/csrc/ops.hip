// Standalone decoder building blocks behind the C ABI: RMSNorm, LayerNorm,
// RoPE, SwiGLU, GELU, argmax and decode attention on caller buffers. The
// model runners fuse the same operations into their GEMV prologues and
// epilogues and into the decode-layers kernel; these entry points let a
// caller launch each one on its own buffers (and let each one be checked on
// its own).
//
// Rounding: the norms take their statistics in fp64 and RoPE its cos / sin
// in fp64 of the fp32 angle; every fp32 product and sum after that is
// rounded on its own (no contraction into FMAs), which are the rounding
// points of the oracle (oracle/llm.py).
//
// Decode attention is split-K flash decoding: grid (split, KV head, row),
// each workgroup streams its split's positions in 64-position tiles of K and
// V through LDS with a running softmax (max, sum, unnormalised V sum) per
// query head, and writes those three as a partial; a merge kernel per
// (row, head) combines the partials. The partials live in a work buffer:
// the context's (sh_attn_decode_f16) or a fixed device array
// (sh_attn_decode_f16_noalloc).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>

#include "common.h"
#include "llm_device.h"

namespace sh {
namespace {

constexpr int kT = 256;

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over the workgroup (kT threads), the same value in every thread.
__device__ __forceinline__ double block_sum_f64(double v, double *red) {
  v = wave_sum_f64(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const double r = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return r;
}

// ---- row norms -------------------------------------------------------------

// grid (rows): y = (x * inv) * g, inv = fp32(1 / sqrt(mean(x^2) + eps)).
// (x and y may be the same rows: each thread reads its values again before
// it overwrites them, after the workgroup's sum)
__global__ __launch_bounds__(kT) void rmsnorm_kernel(const float *x, const float *__restrict__ g,
                                                     float *y, int n, float eps) {
#pragma clang fp contract(off)
  __shared__ double red[4];
  const float *xr = x + (size_t)blockIdx.x * n;
  float *yr = y + (size_t)blockIdx.x * n;
  double ss = 0.0;
  for (int i = threadIdx.x; i < n; i += kT) {
    const double v = xr[i];
    ss += v * v;
  }
  ss = block_sum_f64(ss, red);
  const float inv = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
  for (int i = threadIdx.x; i < n; i += kT) yr[i] = (xr[i] * inv) * g[i];
}

// grid (rows): y = ((x - mean) * inv) * g + b, mean and variance in fp64
// (two passes), inv = fp32(1 / sqrt(var + eps)).
__global__ __launch_bounds__(kT) void layernorm_kernel(const float *x, const float *__restrict__ g,
                                                       const float *__restrict__ bias, float *y,
                                                       int n, float eps) {
#pragma clang fp contract(off)
  __shared__ double red[4];
  const float *xr = x + (size_t)blockIdx.x * n;
  float *yr = y + (size_t)blockIdx.x * n;
  double s = 0.0;
  for (int i = threadIdx.x; i < n; i += kT) s += (double)xr[i];
  const double mean = block_sum_f64(s, red) / (double)n;
  double ss = 0.0;
  for (int i = threadIdx.x; i < n; i += kT) {
    const double d = (double)xr[i] - mean;
    ss += d * d;
  }
  const double var = block_sum_f64(ss, red) / (double)n;
  const float inv = (float)(1.0 / sqrt(var + (double)eps));
  const float mf = (float)mean;
  for (int i = threadIdx.x; i < n; i += kT) yr[i] = ((xr[i] - mf) * inv) * g[i] + bias[i];
}

// ---- RoPE ------------------------------------------------------------------

// grid (rows * heads), block >= d / 2: rotate-half of x[row][head][0..d) at
// positions[row]: angle = fp32(pos) * fp32(theta^(-2i/d)), cos / sin in fp64.
__global__ void rope_kernel(float *__restrict__ x, const int *__restrict__ pos, int heads, int d,
                            float theta) {
#pragma clang fp contract(off)
  const int rh = blockIdx.x, half = d / 2, i = threadIdx.x;
  if (i >= half) return;
  const float inv_freq = (float)pow((double)theta, -2.0 * (double)i / (double)d);
  const float ang = (float)pos[rh / heads] * inv_freq;
  double sd, cd;
  sincos((double)ang, &sd, &cd);
  const float c = (float)cd, s = (float)sd;
  float *xp = x + (size_t)rh * d;
  const float x1 = xp[i], x2 = xp[i + half];
  xp[i] = x1 * c - x2 * s;
  xp[i + half] = x2 * c + x1 * s;
}

// ---- elementwise -------------------------------------------------------------

__global__ __launch_bounds__(kT) void swiglu_kernel(const float *__restrict__ gate,
                                                    const float *__restrict__ up,
                                                    float *__restrict__ out, size_t n) {
#pragma clang fp contract(off)
  for (size_t i = (size_t)blockIdx.x * kT + threadIdx.x; i < n; i += (size_t)gridDim.x * kT)
    out[i] = silu(gate[i]) * up[i];
}

__global__ __launch_bounds__(kT) void gelu_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                  size_t n) {
  for (size_t i = (size_t)blockIdx.x * kT + threadIdx.x; i < n; i += (size_t)gridDim.x * kT)
    y[i] = gelu_tanh(x[i]);
}

// ---- argmax ------------------------------------------------------------------

// Key of x[i]: larger values give larger keys, NaN the largest of all (as
// numpy's argmax, which returns the first NaN), and among equal keys the
// smaller index wins.
__device__ __forceinline__ unsigned long long argmax_key_nan(float v, int i) {
  return v != v ? (0xffffffffull << 32) | (unsigned long long)(0xffffffffu - (uint32_t)i)
                : argmax_key(v, i);
}

// grid (rows): index[row] = the first position of the row's maximum.
__global__ __launch_bounds__(kT) void argmax_kernel(const float *__restrict__ x, int n,
                                                    int32_t *__restrict__ index) {
  __shared__ unsigned long long red[4];
  const float *xr = x + (size_t)blockIdx.x * n;
  unsigned long long best = 0;
  for (int i = threadIdx.x; i < n; i += kT) {
    const unsigned long long k = argmax_key_nan(xr[i], i);
    best = k > best ? k : best;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off, 64);
    best = o > best ? o : best;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = red[0];
    for (int w = 1; w < 4; w++) k = red[w] > k ? red[w] : k;
    index[blockIdx.x] = (int32_t)(0xffffffffu - (uint32_t)(k & 0xffffffffu));
  }
}

// ---- decode attention ----------------------------------------------------------

constexpr int kTile = 64;      // positions per K / V tile
constexpr int kMaxGroup = 16;  // query heads per KV head

struct AttnOpArgs {
  const float *q;            // [B][heads][d]
  const uint16_t *k, *v;     // [B][kv_heads][max_pos][d] fp16
  const int *lengths;        // [B] positions attended: 0 .. length - 1
  float *out;                // [B][heads][d]
  float *part;               // [B][heads][splits][d + 2]: V sum, max, sum
  int heads, kv_heads, max_pos, splits, chunk;
  float scale;
};

// grid (splits, kv_heads, B): positions [s * chunk, min((s + 1) * chunk, L))
// of row b for the G = heads / kv_heads query heads of KV head kvh.
template <int kD>
__global__ __launch_bounds__(kT) void attn_op_partials_kernel(const AttnOpArgs a) {
  constexpr int kRow = kD + 8;                        // padded LDS row of K (fp16)
  constexpr int kAcc = kMaxGroup * kD / kT;           // (head, dim) pairs per thread
  constexpr int kHeadsPerWave = kMaxGroup / 4;
  __shared__ float qs[kMaxGroup][kD];
  __shared__ __attribute__((aligned(16))) _Float16 ks[kTile][kRow];
  __shared__ __attribute__((aligned(16))) _Float16 vs[kTile][kD];
  __shared__ float ps[kMaxGroup][kTile];
  __shared__ float corr[kMaxGroup];

  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int G = a.heads / a.kv_heads;
  const int L = min(a.lengths[b], a.max_pos);
  const int p0 = s * a.chunk;
  if (p0 >= L) return;  // uniform: nothing of this row in the split
  const int p1 = min(p0 + a.chunk, L);
  const int h0 = kvh * G;

  for (int i = t; i < G * kD; i += kT)
    qs[i / kD][i % kD] = a.q[((size_t)b * a.heads + h0 + i / kD) * kD + i % kD] * a.scale;

  float m_run[kHeadsPerWave], l_run[kHeadsPerWave];
#pragma unroll
  for (int j = 0; j < kHeadsPerWave; j++) {
    m_run[j] = -INFINITY;
    l_run[j] = 0.0f;
  }
  float acc[kAcc];
#pragma unroll
  for (int j = 0; j < kAcc; j++) acc[j] = 0.0f;

  const size_t row0 = ((size_t)b * a.kv_heads + kvh) * (size_t)a.max_pos;
  const uint16_t *kb = a.k + row0 * kD;
  const uint16_t *vb = a.v + row0 * kD;
  for (int pt = p0; pt < p1; pt += kTile) {
    const int n = min(kTile, p1 - pt);
    __syncthreads();  // the previous tile's LDS reads are done (and qs is written)
    // K and V rows of the tile in 16-byte vectors; rows past n re-read the
    // tile's last position (in bounds, never weighted)
    for (int vi = t; vi < kTile * kD / 8; vi += kT) {
      const int r = vi / (kD / 8), c8 = (vi % (kD / 8)) * 8;
      const size_t p = (size_t)min(pt + r, p1 - 1);
      *reinterpret_cast<u32x4 *>(&ks[r][c8]) = *reinterpret_cast<const u32x4 *>(kb + p * kD + c8);
      *reinterpret_cast<u32x4 *>(&vs[r][c8]) = *reinterpret_cast<const u32x4 *>(vb + p * kD + c8);
    }
    __syncthreads();
    // scores: wave w holds heads w, w + 4, ..; lane = position in the tile
#pragma unroll
    for (int j = 0; j < kHeadsPerWave; j++) {
      const int g = wave + 4 * j;
      if (g >= G) break;  // wave-uniform
      float dot = 0.0f;
#pragma unroll
      for (int c = 0; c < kD; c += 8) {
        const f16x8 kk = *reinterpret_cast<const f16x8 *>(&ks[lane][c]);
#pragma unroll
        for (int e = 0; e < 8; e++) dot += qs[g][c + e] * (float)kk[e];
      }
      const bool valid = lane < n;
      const float sc = valid ? dot : -INFINITY;
      const float m_new = fmaxf(m_run[j], wave_max(sc));
      const float pr = valid ? expf(sc - m_new) : 0.0f;
      const float c_old = expf(m_run[j] - m_new);  // 0 on the first tile
      l_run[j] = l_run[j] * c_old + wave_sum(pr);
      m_run[j] = m_new;
      ps[g][lane] = pr;
      if (lane == 0) corr[g] = c_old;
    }
    __syncthreads();
    // V sums: thread t owns (head, dim) pairs t, t + 256, ..
#pragma unroll
    for (int j = 0; j < kAcc; j++) {
      const int idx = t + kT * j, g = idx / kD, dd = idx % kD;
      if (g < G) {
        float sum = 0.0f;
#pragma unroll 8
        for (int p = 0; p < kTile; p++) sum += ps[g][p] * (float)vs[p][dd];
        acc[j] = acc[j] * corr[g] + sum;
      }
    }
  }
  // partials of this split
  const size_t pstride = (size_t)kD + 2;
#pragma unroll
  for (int j = 0; j < kAcc; j++) {
    const int idx = t + kT * j, g = idx / kD, dd = idx % kD;
    if (g < G)
      a.part[(((size_t)b * a.heads + h0 + g) * a.splits + s) * pstride + dd] = acc[j];
  }
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < kHeadsPerWave; j++) {
      const int g = wave + 4 * j;
      if (g < G) {
        float *pp = a.part + (((size_t)b * a.heads + h0 + g) * a.splits + s) * pstride + kD;
        pp[0] = m_run[j];
        pp[1] = l_run[j];
      }
    }
  }
}

// grid (heads, B), kD threads:
//   out = sum_j exp(m_j - M) acc_j / sum_j exp(m_j - M) l_j,  M = max_j m_j
// over the row's active splits j (rows of length <= 0: zeros).
template <int kD>
__global__ __launch_bounds__(kD) void attn_op_merge_kernel(const AttnOpArgs a) {
  const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
  const int L = min(a.lengths[b], a.max_pos);
  float *o = a.out + ((size_t)b * a.heads + h) * kD;
  if (L <= 0) {
    o[i] = 0.0f;
    return;
  }
  const int active = (L + a.chunk - 1) / a.chunk;
  const size_t pstride = (size_t)kD + 2;
  const float *pp = a.part + ((size_t)b * a.heads + h) * a.splits * pstride;
  float M = -INFINITY;
  for (int j = 0; j < active; j++) M = fmaxf(M, pp[(size_t)j * pstride + kD]);
  float num = 0.0f, den = 0.0f;
  for (int j = 0; j < active; j++) {
    const float w = expf(pp[(size_t)j * pstride + kD] - M);
    num += w * pp[(size_t)j * pstride + i];
    den += w * pp[(size_t)j * pstride + kD + 1];
  }
  o[i] = num / den;
}

// Split layout of a call: about two workgroups per CU of 256, splits of
// whole 64-position tiles.
void attn_split(int batch, int kv_heads, int max_pos, int *splits, int *chunk) {
  const long long rows = (long long)batch * kv_heads;
  const int want = (int)std::max(1LL, std::min(1024LL, (512 + rows - 1) / rows));
  int c = (max_pos + want - 1) / want;
  c = (c + kTile - 1) / kTile * kTile;
  *chunk = c;
  *splits = (max_pos + c - 1) / c;
}

size_t attn_part_bytes(int batch, int heads, int head_dim, int splits) {
  return (size_t)batch * heads * splits * (head_dim + 2) * sizeof(float);
}

int check_attn(sh_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v,
               const int32_t *lengths, float *out, int batch, int heads, int kv_heads,
               int head_dim, int max_positions) {
  if (batch < 1 || heads < 1 || kv_heads < 1 || max_positions < 1)
    return fail(SH_ERR_INVALID_ARGUMENT,
                "attention sizes must be positive (batch=%d heads=%d kv_heads=%d max_positions=%d)",
                batch, heads, kv_heads, max_positions);
  if (heads % kv_heads != 0 || heads / kv_heads > kMaxGroup)
    return fail(SH_ERR_INVALID_ARGUMENT, "heads %d must be kv_heads %d times 1..%d", heads, kv_heads,
                kMaxGroup);
  if (head_dim != 64 && head_dim != 128)
    return fail(SH_ERR_UNSUPPORTED, "attention head_dim %d (64 or 128 are built)", head_dim);
  if (max_positions > (1 << 24)) return fail(SH_ERR_INVALID_ARGUMENT, "max_positions > 2^24");
  if ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15)
    return fail(SH_ERR_INVALID_ARGUMENT, "k and v caches must be 16-byte aligned");
  const size_t qn = (size_t)batch * heads * head_dim;
  const size_t kvn = (size_t)batch * kv_heads * max_positions * head_dim;
  int rc;
  if ((rc = check_range(ctx, q, qn * 4, "q")) || (rc = check_range(ctx, k, kvn * 2, "k")) ||
      (rc = check_range(ctx, v, kvn * 2, "v")) ||
      (rc = check_range(ctx, lengths, (size_t)batch * 4, "lengths")) ||
      (rc = check_range(ctx, out, qn * 4, "out")))
    return rc;
  return SH_OK;
}

hipError_t launch_attn(hipStream_t st, AttnOpArgs a, int batch, int head_dim) {
  const dim3 grid_p(a.splits, a.kv_heads, batch), grid_m(a.heads, batch);
  if (head_dim == 64) {
    attn_op_partials_kernel<64><<<grid_p, kT, 0, st>>>(a);
    attn_op_merge_kernel<64><<<grid_m, 64, 0, st>>>(a);
  } else {
    attn_op_partials_kernel<128><<<grid_p, kT, 0, st>>>(a);
    attn_op_merge_kernel<128><<<grid_m, 128, 0, st>>>(a);
  }
  return hipGetLastError();
}

int run_attn(sh_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v,
             const int32_t *lengths, float *out, int batch, int heads, int kv_heads, int head_dim,
             int max_positions, float scale, float *part, int splits, int chunk) {
  AttnOpArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.lengths = lengths;
  a.out = out;
  a.part = part;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.max_pos = max_positions;
  a.splits = splits;
  a.chunk = chunk;
  a.scale = scale;
  const hipError_t e = launch_attn(stream_of(ctx), a, batch, head_dim);
  return e == hipSuccess ? SH_OK : hip_fail(e, "attention decode");
}

// ---- the allocation-free attention's work buffer --------------------------------

// Partials of sh_attn_decode_f16_noalloc: one array per device, held from the
// library's load until the process ends. Host code never passes `scratch`
// itself to a kernel (in host code the name is a stand-in, not a device
// address): the device address comes from hipGetSymbolAddress, once per
// device with that device current, and is kept in g_scratch_dev.
constexpr size_t kNoAllocScratchBytes = SH_ATTN_NOALLOC_MAX_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_dev[kMaxDevices] = {};

// The current device's address of `scratch` (ctx's device is current).
int noalloc_scratch(sh_ctx *ctx, void **ptr) {
  const int dev = device_of(ctx);
  if (dev < 0 || dev >= kMaxDevices) return fail(SH_ERR_NO_DEVICE, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(SH_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_dev[dev] = p;
  }
  *ptr = g_scratch_dev[dev];
  return SH_OK;
}

}  // namespace
}  // namespace sh

using namespace sh;

extern "C" {

SH_API int sh_rmsnorm_f32(sh_ctx *ctx, const float *x, const float *gain, float *y, int rows,
                          int n, float eps) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if (rows < 0 || n < 0) return fail(SH_ERR_INVALID_ARGUMENT, "negative size rows=%d n=%d", rows, n);
  if (rows == 0 || n == 0) return SH_OK;
  if (!(eps >= 0.0f)) return fail(SH_ERR_INVALID_ARGUMENT, "eps must be >= 0");
  const size_t bytes = (size_t)rows * n * 4;
  if ((rc = check_range(ctx, x, bytes, "x")) || (rc = check_range(ctx, gain, (size_t)n * 4, "gain")) ||
      (rc = check_range(ctx, y, bytes, "y")))
    return rc;
  rmsnorm_kernel<<<rows, kT, 0, stream_of(ctx)>>>(x, gain, y, n, eps);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SH_OK : hip_fail(e, "rmsnorm");
}

SH_API int sh_layernorm_f32(sh_ctx *ctx, const float *x, const float *gain, const float *bias,
                            float *y, int rows, int n, float eps) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if (rows < 0 || n < 0) return fail(SH_ERR_INVALID_ARGUMENT, "negative size rows=%d n=%d", rows, n);
  if (rows == 0 || n == 0) return SH_OK;
  if (!(eps >= 0.0f)) return fail(SH_ERR_INVALID_ARGUMENT, "eps must be >= 0");
  const size_t bytes = (size_t)rows * n * 4;
  if ((rc = check_range(ctx, x, bytes, "x")) || (rc = check_range(ctx, gain, (size_t)n * 4, "gain")) ||
      (rc = check_range(ctx, bias, (size_t)n * 4, "bias")) || (rc = check_range(ctx, y, bytes, "y")))
    return rc;
  layernorm_kernel<<<rows, kT, 0, stream_of(ctx)>>>(x, gain, bias, y, n, eps);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SH_OK : hip_fail(e, "layernorm");
}

SH_API int sh_rope_f32(sh_ctx *ctx, float *x, const int32_t *positions, int rows, int heads,
                       int head_dim, float theta) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if (rows < 0 || heads < 0) return fail(SH_ERR_INVALID_ARGUMENT, "negative size rows=%d heads=%d", rows, heads);
  if (head_dim < 2 || head_dim % 2 != 0 || head_dim > 512)
    return fail(SH_ERR_INVALID_ARGUMENT, "head_dim %d must be even and 2..512", head_dim);
  if (!(theta > 0.0f)) return fail(SH_ERR_INVALID_ARGUMENT, "theta must be positive");
  if (rows == 0 || heads == 0) return SH_OK;
  if ((long long)rows * heads > 0x7fffffffLL)
    return fail(SH_ERR_INVALID_ARGUMENT, "rows * heads exceeds 2^31 - 1");
  if ((rc = check_range(ctx, x, (size_t)rows * heads * head_dim * 4, "x")) ||
      (rc = check_range(ctx, positions, (size_t)rows * 4, "positions")))
    return rc;
  const int block = (head_dim / 2 + 63) / 64 * 64;
  rope_kernel<<<rows * heads, block, 0, stream_of(ctx)>>>(x, positions, heads, head_dim, theta);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SH_OK : hip_fail(e, "rope");
}

SH_API int sh_swiglu_f32(sh_ctx *ctx, const float *gate, const float *up, float *out, size_t n) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if (n == 0) return SH_OK;
  if ((rc = check_range(ctx, gate, n * 4, "gate")) || (rc = check_range(ctx, up, n * 4, "up")) ||
      (rc = check_range(ctx, out, n * 4, "out")))
    return rc;
  const size_t grid = std::min<size_t>((n + kT - 1) / kT, 8192);
  swiglu_kernel<<<(unsigned)grid, kT, 0, stream_of(ctx)>>>(gate, up, out, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SH_OK : hip_fail(e, "swiglu");
}

SH_API int sh_gelu_f32(sh_ctx *ctx, const float *x, float *y, size_t n) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if (n == 0) return SH_OK;
  if ((rc = check_range(ctx, x, n * 4, "x")) || (rc = check_range(ctx, y, n * 4, "y"))) return rc;
  const size_t grid = std::min<size_t>((n + kT - 1) / kT, 8192);
  gelu_kernel<<<(unsigned)grid, kT, 0, stream_of(ctx)>>>(x, y, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SH_OK : hip_fail(e, "gelu");
}

SH_API int sh_argmax_f32(sh_ctx *ctx, const float *x, int rows, int n, int32_t *index) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if (rows < 0 || n < 1) return fail(SH_ERR_INVALID_ARGUMENT, "need rows >= 0 and n >= 1 (rows=%d n=%d)", rows, n);
  if (rows == 0) return SH_OK;
  if ((rc = check_range(ctx, x, (size_t)rows * n * 4, "x")) ||
      (rc = check_range(ctx, index, (size_t)rows * 4, "index")))
    return rc;
  argmax_kernel<<<rows, kT, 0, stream_of(ctx)>>>(x, n, index);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SH_OK : hip_fail(e, "argmax");
}

SH_API int sh_attn_decode_f16(sh_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v,
                              const int32_t *lengths, float *out, int batch, int heads,
                              int kv_heads, int head_dim, int max_positions, float scale) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if ((rc = check_attn(ctx, q, k, v, lengths, out, batch, heads, kv_heads, head_dim, max_positions)))
    return rc;
  int splits = 0, chunk = 0;
  attn_split(batch, kv_heads, max_positions, &splits, &chunk);
  void *part = nullptr;
  if ((rc = context_scratch(ctx, attn_part_bytes(batch, heads, head_dim, splits), &part))) return rc;
  return run_attn(ctx, q, k, v, lengths, out, batch, heads, kv_heads, head_dim, max_positions, scale,
                  static_cast<float *>(part), splits, chunk);
}

SH_API int sh_attn_decode_f16_noalloc(sh_ctx *ctx, const float *q, const uint16_t *k,
                                      const uint16_t *v, const int32_t *lengths, float *out,
                                      int batch, int heads, int kv_heads, int head_dim,
                                      int max_positions, float scale) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if ((rc = check_attn(ctx, q, k, v, lengths, out, batch, heads, kv_heads, head_dim, max_positions)))
    return rc;
  int splits = 0, chunk = 0;
  attn_split(batch, kv_heads, max_positions, &splits, &chunk);
  const size_t need = attn_part_bytes(batch, heads, head_dim, splits);
  if (need > kNoAllocScratchBytes)
    return fail(SH_ERR_INVALID_ARGUMENT,
                "attention partials need %zu bytes, more than the %zu-byte allocation-free "
                "work buffer (batch * heads * splits * (head_dim + 2) * 4, %d splits)",
                need, kNoAllocScratchBytes, splits);
  void *part = nullptr;
  if ((rc = noalloc_scratch(ctx, &part))) return rc;
  return run_attn(ctx, q, k, v, lengths, out, batch, heads, kv_heads, head_dim, max_positions, scale,
                  static_cast<float *>(part), splits, chunk);
}

}  // extern "C"
