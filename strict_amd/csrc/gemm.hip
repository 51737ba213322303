// Dense GEMM C[M,N] = A[M,K] * B[K,N], bf16 operands, fp32 accumulation,
// bf16 output, all row-major. The reference only holds an unused cuBLAS
// handle for this (Kernel.cs:10-11, :16); the workload is BASELINE configs[2].
//
// MFMA kernel (M % 256 == 0, N % 256 == 0, K % 64 == 0, leading dimensions
// multiples of 8 elements, 16-byte aligned operands):
//  - one 256-thread workgroup per 256 x 256 tile of C; its 4 waves own
//    128 x 128 quadrants, each a 4 x 4 grid of v_mfma_f32_32x32x16_bf16
//    accumulators (256 fp32 per lane, held in AGPRs at one wave per SIMD);
//  - K advances in 64-wide slabs staged in LDS, double buffered (2 x 64 KiB),
//    software-pipelined: within a slab the fragments of k-step s + 1 are read
//    while the MFMAs of step s run; the next slab goes out to the other buffer
//    during steps 2 (A rows) and 3 (B columns), and each half's global loads
//    for the slab after that are issued as soon as its staging registers are
//    written out, so they have four k-steps to arrive; one barrier per slab,
//    before the last four MFMAs, whose shadow covers the next slab's first
//    fragment reads; scheduling barriers fix the instruction order (one
//    MFMA, then the memory operations that go with it);
//  - operands are read with buffer loads: one 32-bit lane offset per operand,
//    the row and slab steps in the scalar offset (the tile's A rows and all of
//    B's rows must span < 2 GiB);
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

  // A: rows t/8 + 32i (i < 8), 16-byte chunk t%8 of the 64-wide slab;
  // B: an 8 x 8 block, k rows 8*(t%8) .. +7, n columns 8*(t/8) .. +7
  const int a_row = t >> 3, a_chunk = t & 7;
  const int b_kc = t & 7, b_nc = t >> 3;

  const __amdgpu_buffer_rsrc_t a_rs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(A + (size_t)tm * kBM * lda), (short)0, (255 * lda + K) * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t b_rs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(B + tn * kBN), (short)0, ((K - 1) * ldb + kBN) * 2, 0x00020000);
  const int a_voff = (a_row * lda + a_chunk * 8) * 2, b_voff = (8 * b_kc * ldb + 8 * b_nc) * 2;
  u32x4 ra[8], rb[8];
  auto load_a = [&](int kt, int i) {
    ra[i] = __builtin_amdgcn_raw_buffer_load_b128(a_rs, a_voff, (32 * i * lda + kt * kBK) * 2, 0);
  };
  auto load_b = [&](int kt, int i) {
    rb[i] = __builtin_amdgcn_raw_buffer_load_b128(b_rs, b_voff, (kt * kBK + i) * ldb * 2, 0);
  };
  auto store_a = [&](uint8_t *buf, int i) {
    const int r = a_row + 32 * i;
    *reinterpret_cast<u32x4 *>(buf + r * kLdsRow + swz(r, a_chunk) * 16) = ra[i];
  };
  // B's 8 x 8 block transposed: every output column needs all eight staged
  // rows, so the whole block is permuted before any of its registers is
  // reloaded
  u32x4 bt[8];
  auto transpose_b = [&]() {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int jj = j ^ (b_nc & 1);
      const uint32_t sel = (jj & 1) ? 0x07060302u : 0x05040100u;
      bt[j].x = __builtin_amdgcn_perm(rb[1][jj >> 1], rb[0][jj >> 1], sel);
      bt[j].y = __builtin_amdgcn_perm(rb[3][jj >> 1], rb[2][jj >> 1], sel);
      bt[j].z = __builtin_amdgcn_perm(rb[5][jj >> 1], rb[4][jj >> 1], sel);
      bt[j].w = __builtin_amdgcn_perm(rb[7][jj >> 1], rb[6][jj >> 1], sel);
    }
  };
  auto store_b = [&](uint8_t *buf, int j) {
    const int n = 8 * b_nc + (j ^ (b_nc & 1));
    *reinterpret_cast<u32x4 *>(buf + kLdsTile + n * kLdsRow + swz(n, b_kc) * 16) = bt[j];
  };

  // Fragment q of k-step s: q < 4 is A rows wm*128 + 32 q + (lane % 32), q >= 4
  // B columns wn*128 + 32 (q - 4) + (lane % 32); 8 k values each, k chunk
  // 2 s + lane / 32. The row swizzle (row / 2) % 8 only depends on lane % 32.
  const int frag_row = lane & 31, frag_half = lane >> 5, fsw = (frag_row >> 1) & 7;
  const int a_off = (wm * 128 + frag_row) * kLdsRow, b_off = kLdsTile + (wn * 128 + frag_row) * kLdsRow;
  bf16x8 f[2][8];
  auto read_frag = [&](bf16x8 (&fr)[8], const uint8_t *buf, int s, int q) {
    const int chunk = ((2 * s + frag_half) ^ fsw) * 16;
    const int off = q < 4 ? a_off + q * 32 * kLdsRow : b_off + (q - 4) * 32 * kLdsRow;
    fr[q] = *reinterpret_cast<const bf16x8 *>(buf + off + chunk);
  };
  // fragments are read A0, B0, B1, B2, B3, A1, A2, A3: the order the MFMAs
  // (row-major over the 4 x 4 accumulators) first need them
  constexpr int kReadOrder[8] = {0, 4, 5, 6, 7, 1, 2, 3};

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
  auto mfma = [&](const bf16x8 (&fr)[8], int k) {
    const int i = k >> 2, j = k & 3;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr[4 + j], fr[i], acc[i][j], 0, 0, 0);
  };

  const int ktiles = K / kBK;
  // prologue: slab 0 into buffer 0, slab 1 requested, step 0 fragments read
#pragma unroll
  for (int i = 0; i < 8; i++) load_a(0, i);
#pragma unroll
  for (int i = 0; i < 8; i++) load_b(0, i);
#pragma unroll
  for (int i = 0; i < 8; i++) store_a(lds, i);
  transpose_b();
#pragma unroll
  for (int j = 0; j < 8; j++) store_b(lds, j);
  const int k1 = min(1, ktiles - 1);
#pragma unroll
  for (int i = 0; i < 8; i++) load_a(k1, i);
#pragma unroll
  for (int i = 0; i < 8; i++) load_b(k1, i);
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 8; q++) read_frag(f[0], lds, 0, kReadOrder[q]);

  for (int kt = 0; kt < ktiles; kt++) {
    const uint8_t *cur = lds + (kt & 1) * 2 * kLdsTile;
    uint8_t *nxt = lds + ((kt & 1) ^ 1) * 2 * kLdsTile;
    // slab after the next one (re-reads the last slab at the end; those
    // values are never used)
    const int k2 = min(kt + 2, ktiles - 1);
    // steps 0 and 1: MFMAs of step s, reads of step s + 1
#pragma unroll
    for (int s = 0; s < 2; s++) {
#pragma unroll
      for (int k = 0; k < 16; k++) {
        mfma(f[s & 1], k);
        if (k < 8) read_frag(f[(s + 1) & 1], cur, s + 1, kReadOrder[k]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // step 2: reads of step 3, then the A half of the next slab out to LDS
    // and the A half of the slab after it requested
#pragma unroll
    for (int k = 0; k < 16; k++) {
      mfma(f[0], k);
      if (k < 8) {
        read_frag(f[1], cur, 3, kReadOrder[k]);
      } else {
        store_a(nxt, k - 8);
        load_a(k2, k - 8);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // step 3: the B half likewise, then the barrier, then the next slab's
    // step 0 fragments under the last four MFMAs
    transpose_b();
#pragma unroll
    for (int k = 0; k < 12; k++) {
      mfma(f[1], k);
      if (k < 8) {
        store_b(nxt, k);
        load_b(k2, k);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes done
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 12; k < 16; k++) {
      mfma(f[1], k);
      read_frag(f[0], nxt, 0, kReadOrder[2 * (k - 12)]);
      read_frag(f[0], nxt, 0, kReadOrder[2 * (k - 12) + 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

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
         (reinterpret_cast<uintptr_t>(C) & 7) == 0 && (int64_t)kBM * lda * 2 < (1ll << 31) &&
         (int64_t)K * ldb * 2 < (1ll << 31);
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
