// FP8 GEMM: C[M,N] = bf16( sa[m] * sb[n] * sum_k e4m3(A[m,k]) * e4m3(Bt[n,k]) ),
// fp32 accumulation. A is row-major [M][K]; B arrives transposed, Bt [N][K]
// row-major (each output column's K values contiguous, the layout of a
// weight matrix W[N][K] quantized per output row); sa / sb are the fp32
// per-row / per-column scales (sh_quantize_e4m3 makes both). OCP E4M3.
// The reference has nothing for this (BASELINE's FP8 GEMM
// measurement); the decode path's prefill shape is M = 4096 tokens.
//
// MFMA kernel (M % 256 == 0, N % 256 == 0, K % 128 == 0, leading dimensions
// multiples of 16 bytes, 16-byte aligned A / Bt, 8-byte aligned C):
//  - one 256-thread workgroup per 256 x 256 tile of C; its 4 waves own
//    128 x 128 quadrants, each a 4 x 4 grid of v_mfma_scale_f32_32x32x64_f8f6f4
//    accumulators (E8M0 block scales fixed at 1: the fp32 row / column scales
//    are applied once in the epilogue);
//  - K advances in 128-byte slabs staged in LDS, double buffered (2 x 64 KiB),
//    next slab loaded during the current one's MFMAs, one barrier per slab;
//  - both operands are K-contiguous, so A rows and Bt rows are staged alike
//    (no transpose), the 16-byte chunk index XOR-swizzled by (row / 2) % 8 so
//    16-lane LDS phases hit 16 distinct bank groups;
//  - a lane's MFMA operand is 32 consecutive k of one row (two 16-byte LDS
//    reads); the hardware pairs A and B bytes by lane half and position, so
//    any k order common to both operands gives the same sum;
//  - issued as Bt x A so that each lane holds one row of C with runs of four
//    consecutive columns;
//  - XCD-grouped tile order as in the bf16 kernel.
// Every other shape takes a bounds-checked fp32 FMA kernel.
#include <hip/hip_runtime.h>

#include "common.h"

namespace sh {
namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = 256, kBN = 256, kBK = 128;  // kBK in bytes = fp8 values
constexpr int kThreads = 256;
constexpr int kLdsRow = kBK;                  // bytes per staged row
constexpr int kLdsTile = 256 * kLdsRow;       // 32 KiB per operand slab
constexpr int kLdsBytes = 4 * kLdsTile;       // 2 buffers x (A, Bt)
constexpr int kScaleOne = 127;                // E8M0 exponent of 1.0

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                                  // round to nearest even
  return u >> 16;
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_fp8_mfma_kernel(const uint8_t *__restrict__ A, const float *__restrict__ sa,
                          const uint8_t *__restrict__ Bt, const float *__restrict__ sb,
                          uint16_t *__restrict__ C, int K, int lda, int ldb, int ldc,
                          int tiles_m, int tiles_n, int grouped) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const int ntiles = tiles_m * tiles_n;
  int tile = blockIdx.x;
  int tm, tn;
  if (grouped) {
    tile = (blockIdx.x & 7) * (ntiles >> 3) + (blockIdx.x >> 3);
    const int g = tile >> 5, li = tile & 31;
    const int groups_n = tiles_n >> 3;
    tm = (g / groups_n) * 4 + (li >> 3);
    tn = (g % groups_n) * 8 + (li & 7);
  } else {
    tm = tile / tiles_n;
    tn = tile % tiles_n;
  }

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // global load roles: rows t/8 + 32i (i < 8), 16-byte chunk t%8 of the slab
  const int g_row = t >> 3, g_chunk = t & 7;
  const uint8_t *a_src = A + (size_t)(tm * kBM + g_row) * lda + g_chunk * 16;
  const uint8_t *b_src = Bt + (size_t)(tn * kBN + g_row) * ldb + g_chunk * 16;

  u32x4 ra[8], rb[8];
  auto load_slab = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 8; i++)
      ra[i] = *reinterpret_cast<const u32x4 *>(a_src + (size_t)(32 * i) * lda + kt * kBK);
#pragma unroll
    for (int i = 0; i < 8; i++)
      rb[i] = *reinterpret_cast<const u32x4 *>(b_src + (size_t)(32 * i) * ldb + kt * kBK);
  };
  auto store_slab = [&](int buf) {
    uint8_t *la = lds + buf * 2 * kLdsTile;
    uint8_t *lb = la + kLdsTile;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int r = g_row + 32 * i;
      *reinterpret_cast<u32x4 *>(la + r * kLdsRow + swz(r, g_chunk) * 16) = ra[i];
      *reinterpret_cast<u32x4 *>(lb + r * kLdsRow + swz(r, g_chunk) * 16) = rb[i];
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  const int ktiles = K / kBK;
  load_slab(0);
  store_slab(0);
  __syncthreads();

  const int frag_row = lane & 31, frag_half = lane >> 5;
  for (int kt = 0; kt < ktiles; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < ktiles) load_slab(kt + 1);
    const uint8_t *la = lds + buf * 2 * kLdsTile;
    const uint8_t *lb = la + kLdsTile;
#pragma unroll
    for (int s = 0; s < kBK / 64; s++) {
      const int c0 = 4 * s + 2 * frag_half;  // the lane's two 16-byte chunks
      i32x8 fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = wm * 128 + i * 32 + frag_row;
        const u32x4 lo = *reinterpret_cast<const u32x4 *>(la + m * kLdsRow + swz(m, c0) * 16);
        const u32x4 hi = *reinterpret_cast<const u32x4 *>(la + m * kLdsRow + swz(m, c0 + 1) * 16);
        fa[i] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int n = wn * 128 + j * 32 + frag_row;
        const u32x4 lo = *reinterpret_cast<const u32x4 *>(lb + n * kLdsRow + swz(n, c0) * 16);
        const u32x4 hi = *reinterpret_cast<const u32x4 *>(lb + n * kLdsRow + swz(n, c0 + 1) * 16);
        fb[j] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              fb[j], fa[i], acc[i][j], 0, 0, 0, kScaleOne, 0, kScaleOne);
    }
    if (kt + 1 < ktiles) store_slab(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds C row m, columns n0 + 8q + 4*half + 0..3 ----
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = tm * kBM + wm * 128 + i * 32 + frag_row;
    const float am = sa[m];
    uint16_t *crow = C + (size_t)m * ldc;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n0 = tn * kBN + wn * 128 + j * 32 + 4 * frag_half;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const f32x4 bn = *reinterpret_cast<const f32x4 *>(sb + n0 + 8 * q);
        const uint32_t p0 = f32_to_bf16_bits(acc[i][j][4 * q + 0] * am * bn[0]) |
                            (f32_to_bf16_bits(acc[i][j][4 * q + 1] * am * bn[1]) << 16);
        const uint32_t p1 = f32_to_bf16_bits(acc[i][j][4 * q + 2] * am * bn[2]) |
                            (f32_to_bf16_bits(acc[i][j][4 * q + 3] * am * bn[3]) << 16);
        *reinterpret_cast<u32x2 *>(crow + n0 + 8 * q) = u32x2{p0, p1};
      }
    }
  }
}

// ---- generic path: any shape and leading dimensions ----------------------

constexpr int kGT = 64;  // 64 x 64 tile, 256 threads, 4 x 4 outputs each

__device__ __forceinline__ float e4m3_to_f32(uint8_t q) {
  const f16x2 h = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((uint32_t)q, 1.0f, false);
  return (float)h[0];
}

__global__ __launch_bounds__(256) void gemm_fp8_generic_kernel(const uint8_t *A, const float *sa,
                                                               const uint8_t *Bt, const float *sb,
                                                               uint16_t *C, int M, int N, int K,
                                                               int lda, int ldb, int ldc) {
  __shared__ float as[16][kGT + 1];
  __shared__ float bs[16][kGT + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * kGT, n0 = blockIdx.x * kGT;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int idx = threadIdx.x; idx < 16 * kGT; idx += 256) {
      const int kk = idx & 15, rr = idx >> 4;  // 64 rows x 16 k of each operand
      const int gk = k0 + kk;
      const int gm = m0 + rr, gn = n0 + rr;
      as[kk][rr] = (gm < M && gk < K) ? e4m3_to_f32(A[(size_t)gm * lda + gk]) : 0.0f;
      bs[kk][rr] = (gn < N && gk < K) ? e4m3_to_f32(Bt[(size_t)gn * ldb + gk]) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; kk++) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++) a[i] = as[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int gm = m0 + ty * 4 + i;
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int gn = n0 + tx * 4 + j;
      if (gn < N) C[(size_t)gm * ldc + gn] = (uint16_t)f32_to_bf16_bits(acc[i][j] * sa[gm] * sb[gn]);
    }
  }
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

bool gemm_fp8_uses_mfma(int M, int N, int K, int lda, int ldb, int ldc, const void *A,
                        const void *Bt, const void *C, const void *sb) {
  return M % kBM == 0 && N % kBN == 0 && K % kBK == 0 && K > 0 && lda % 16 == 0 &&
         ldb % 16 == 0 && ldc % 4 == 0 && aligned(A, 16) && aligned(Bt, 16) && aligned(C, 8) &&
         aligned(sb, 16);
}

hipError_t launch_gemm_fp8(hipStream_t s, const uint8_t *A, const float *sa, const uint8_t *Bt,
                           const float *sb, uint16_t *C, int M, int N, int K, int lda, int ldb,
                           int ldc) {
  if (gemm_fp8_uses_mfma(M, N, K, lda, ldb, ldc, A, Bt, C, sb)) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_fp8_mfma_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return e;
    const int tiles_m = M / kBM, tiles_n = N / kBN;
    const int ntiles = tiles_m * tiles_n;
    const int grouped = (ntiles % 256 == 0 && tiles_m % 4 == 0 && tiles_n % 8 == 0) ? 1 : 0;
    gemm_fp8_mfma_kernel<<<ntiles, kThreads, kLdsBytes, s>>>(A, sa, Bt, sb, C, K, lda, ldb, ldc,
                                                            tiles_m, tiles_n, grouped);
  } else {
    dim3 grid((N + kGT - 1) / kGT, (M + kGT - 1) / kGT);
    gemm_fp8_generic_kernel<<<grid, 256, 0, s>>>(A, sa, Bt, sb, C, M, N, K, lda, ldb, ldc);
  }
  return hipGetLastError();
}

}  // namespace sh
