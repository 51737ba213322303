// Dense GEMM C[M,N] = A[M,K] * B[K,N], bf16 operands, fp32 accumulation,
// bf16 output, all row-major. The reference only holds an unused cuBLAS
// handle for this (Kernel.cs:10-11, :16); the workload is BASELINE configs[2].
//
// MFMA kernel (M % 256 == 0, N % 256 == 0, K % 64 == 0, leading dimensions
// multiples of 8 elements, 16-byte aligned operands):
//  - one 256-thread workgroup per 256 x 256 tile of C; its 4 waves own
//    128 x 128 quadrants, each a 4 x 4 grid of v_mfma_f32_32x32x16_bf16
//    accumulators (256 fp32 per lane, held in AGPRs at one wave per SIMD);
//  - K advances in 64-wide slabs staged in LDS, double buffered (2 x 64 KiB):
//    the next slab's global loads are issued before the MFMAs of the current
//    one and written to the other buffer after them, one barrier per slab;
//  - A rows and B columns are stored K-contiguous in LDS (128 B per row), the
//    16-byte chunk index XOR-swizzled by (row / 2) % 8 so that the 16-lane
//    phases of ds_read_b128 / ds_write_b128 touch 16 distinct bank groups;
//  - B arrives row-major (N contiguous): each thread loads an 8(k) x 8(n)
//    block and transposes it in registers with v_perm before the LDS store;
//  - the MFMA is issued as Bt x A so that each lane ends up holding one row
//    of C with runs of 4 consecutive columns (8-byte bf16 stores);
//  - tiles are numbered so that each of the 8 XCDs (workgroups are dealt to
//    XCDs round-robin) computes a 4 x 8 block of tiles, whose A and B slabs
//    its L2 then shares.
// Every other shape takes a bounds-checked LDS-tiled fp32 FMA kernel.
#include <hip/hip_runtime.h>

#include "common.h"

namespace sh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 256;
constexpr int kLdsRow = kBK * 2;          // bytes per staged row (64 bf16)
constexpr int kLdsTile = 256 * kLdsRow;   // 32 KiB per operand slab
constexpr int kLdsBytes = 4 * kLdsTile;   // 2 buffers x (A, Bt)

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                                  // round to nearest even
  return u >> 16;
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_mfma_kernel(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                           uint16_t *__restrict__ C, int K, int lda, int ldb, int ldc,
                           int tiles_m, int tiles_n, int grouped) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  // ---- tile of this workgroup ----
  const int ntiles = tiles_m * tiles_n;
  int tile = blockIdx.x;
  int tm, tn;
  if (grouped) {
    // workgroup b runs on XCD b % 8; give XCD x the tiles x*T/8 .. (x+1)*T/8-1,
    // laid out as 4 x 8 tile blocks
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

  // ---- global load roles ----
  // A: rows t/8 + 32i (i < 8), 16-byte chunk t%8 of the 64-wide slab
  const int a_row = t >> 3, a_chunk = t & 7;
  const uint16_t *a_src = A + (size_t)(tm * kBM + a_row) * lda + a_chunk * 8;
  // B: 8 x 8 block, k rows 8*(t%8) .. +7, n columns 8*(t/8) .. +7
  const int b_kc = t & 7, b_nc = t >> 3;
  const uint16_t *b_src = B + (size_t)(8 * b_kc) * ldb + tn * kBN + 8 * b_nc;

  u32x4 ra[8], rb[8];
  auto load_slab = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 8; i++)
      ra[i] = *reinterpret_cast<const u32x4 *>(a_src + (size_t)(32 * i) * lda + kt * kBK);
#pragma unroll
    for (int i = 0; i < 8; i++)
      rb[i] = *reinterpret_cast<const u32x4 *>(b_src + (size_t)(kt * kBK + i) * ldb);
  };
  auto store_slab = [&](int buf) {
    uint8_t *la = lds + buf * 2 * kLdsTile;
    uint8_t *lb = la + kLdsTile;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int r = a_row + 32 * i;
      *reinterpret_cast<u32x4 *>(la + r * kLdsRow + swz(r, a_chunk) * 16) = ra[i];
    }
    // transpose the 8x8 bf16 block: column j of rb -> 8 k values of n = 8*b_nc + j.
    // Odd column groups write their rows in the opposite parity order, so the
    // two 8-lane halves of each 16-lane store phase hit different bank groups.
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int jj = j ^ (b_nc & 1);
      const uint32_t sel = (jj & 1) ? 0x07060302u : 0x05040100u;
      u32x4 o;
      o.x = __builtin_amdgcn_perm(rb[1][jj >> 1], rb[0][jj >> 1], sel);
      o.y = __builtin_amdgcn_perm(rb[3][jj >> 1], rb[2][jj >> 1], sel);
      o.z = __builtin_amdgcn_perm(rb[5][jj >> 1], rb[4][jj >> 1], sel);
      o.w = __builtin_amdgcn_perm(rb[7][jj >> 1], rb[6][jj >> 1], sel);
      const int n = 8 * b_nc + jj;
      *reinterpret_cast<u32x4 *>(lb + n * kLdsRow + swz(n, b_kc) * 16) = o;
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
    for (int s = 0; s < kBK / 16; s++) {
      const int chunk = 2 * s + frag_half;
      bf16x8 fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = wm * 128 + i * 32 + frag_row;
        fa[i] = *reinterpret_cast<const bf16x8 *>(la + m * kLdsRow + swz(m, chunk) * 16);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int n = wn * 128 + j * 32 + frag_row;
        fb[j] = *reinterpret_cast<const bf16x8 *>(lb + n * kLdsRow + swz(n, chunk) * 16);
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < ktiles) store_slab(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds C row m, columns n0 + 8q + 4*half + 0..3 ----
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = tm * kBM + wm * 128 + i * 32 + frag_row;
    uint16_t *crow = C + (size_t)m * ldc;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n0 = tn * kBN + wn * 128 + j * 32 + 4 * frag_half;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t p0 = f32_to_bf16_bits(acc[i][j][4 * q + 0]) |
                            (f32_to_bf16_bits(acc[i][j][4 * q + 1]) << 16);
        const uint32_t p1 = f32_to_bf16_bits(acc[i][j][4 * q + 2]) |
                            (f32_to_bf16_bits(acc[i][j][4 * q + 3]) << 16);
        *reinterpret_cast<u32x2 *>(crow + n0 + 8 * q) = u32x2{p0, p1};
      }
    }
  }
}

// ---- generic path: any shape and leading dimensions ----------------------

constexpr int kGT = 64;  // 64 x 64 tile, 256 threads, 4 x 4 outputs each

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}

__global__ __launch_bounds__(256) void gemm_bf16_generic_kernel(const uint16_t *A,
                                                                const uint16_t *B, uint16_t *C,
                                                                int M, int N, int K, int lda,
                                                                int ldb, int ldc) {
  __shared__ float as[16][kGT + 1];
  __shared__ float bs[16][kGT + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * kGT, n0 = blockIdx.x * kGT;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int idx = threadIdx.x; idx < 16 * kGT; idx += 256) {
      const int kk = idx & 15, mm = idx >> 4;  // A tile: 64 rows x 16 k
      const int gm = m0 + mm, gk = k0 + kk;
      as[kk][mm] = (gm < M && gk < K) ? bf16_bits_to_f32(A[(size_t)gm * lda + gk]) : 0.0f;
      const int nn = idx & 63, kb = idx >> 6;  // B tile: 16 k x 64 cols
      const int gn = n0 + nn, gk2 = k0 + kb;
      bs[kb][nn] = (gn < N && gk2 < K) ? bf16_bits_to_f32(B[(size_t)gk2 * ldb + gn]) : 0.0f;
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
      if (gn < N) C[(size_t)gm * ldc + gn] = (uint16_t)f32_to_bf16_bits(acc[i][j]);
    }
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

bool gemm_bf16_uses_mfma(int M, int N, int K, int lda, int ldb, int ldc, const void *A,
                         const void *B, const void *C) {
  return M % kBM == 0 && N % kBN == 0 && K % kBK == 0 && K > 0 && lda % 8 == 0 &&
         ldb % 8 == 0 && ldc % 4 == 0 && aligned16(A) && aligned16(B) &&
         (reinterpret_cast<uintptr_t>(C) & 7) == 0;
}

hipError_t launch_gemm_bf16(hipStream_t s, const uint16_t *A, const uint16_t *B, uint16_t *C,
                            int M, int N, int K, int lda, int ldb, int ldc) {
  if (gemm_bf16_uses_mfma(M, N, K, lda, ldb, ldc, A, B, C)) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_bf16_mfma_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return e;
    const int tiles_m = M / kBM, tiles_n = N / kBN;
    const int ntiles = tiles_m * tiles_n;
    const int grouped = (ntiles % 256 == 0 && tiles_m % 4 == 0 && tiles_n % 8 == 0) ? 1 : 0;
    gemm_bf16_mfma_kernel<<<ntiles, kThreads, kLdsBytes, s>>>(A, B, C, K, lda, ldb, ldc, tiles_m,
                                                             tiles_n, grouped);
  } else {
    dim3 grid((N + kGT - 1) / kGT, (M + kGT - 1) / kGT);
    gemm_bf16_generic_kernel<<<grid, 256, 0, s>>>(A, B, C, M, N, K, lda, ldb, ldc);
  }
  return hipGetLastError();
}

}  // namespace sh
