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
//    software-pipelined like the bf16 kernel: the second 64-deep k-step's
//    fragments are read under the first step's MFMAs; the next slab goes out
//    to the other buffer during the slab (A rows in step 0, Bt rows in step 1)
//    and each half's loads for the slab after it are issued as soon as its
//    staging registers are free; one barrier per slab, before the last four
//    MFMAs, whose shadow covers the next slab's first fragment reads;
//    scheduling barriers fix the order; buffer loads with 32-bit lane offsets
//    (the tile's rows of A and of Bt must each span < 2 GiB);
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

  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // the epilogue's pointers are used here, so their scalar loads complete
  // before the loop: left pending, they made every wait on the LDS counter
  // at the loop's top a full lgkmcnt(0) (scalar and LDS results return out
  // of order)
  asm volatile("" ::"s"(sa), "s"(sb), "s"(C));

  // rows t/8 + 32i (i < 8), 16-byte chunk t%8 of the slab
  const int g_row = t >> 3, g_chunk = t & 7;
  const __amdgpu_buffer_rsrc_t a_rs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(A + (size_t)tm * kBM * lda), (short)0, 255 * lda + K, 0x00020000);
  const __amdgpu_buffer_rsrc_t b_rs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(Bt + (size_t)tn * kBN * ldb), (short)0, 255 * ldb + K, 0x00020000);
  const int a_voff = g_row * lda + g_chunk * 16, b_voff = g_row * ldb + g_chunk * 16;
  u32x4 ra[8], rb[8];
  auto load_a = [&](int kt, int i) {
    ra[i] = __builtin_amdgcn_raw_buffer_load_b128(a_rs, a_voff, 32 * i * lda + kt * kBK, 0);
  };
  auto load_b = [&](int kt, int i) {
    rb[i] = __builtin_amdgcn_raw_buffer_load_b128(b_rs, b_voff, 32 * i * ldb + kt * kBK, 0);
  };
  auto store_a = [&](uint8_t *buf, int i) {
    const int r = g_row + 32 * i;
    *reinterpret_cast<u32x4 *>(buf + r * kLdsRow + swz(r, g_chunk) * 16) = ra[i];
  };
  auto store_b = [&](uint8_t *buf, int i) {
    const int r = g_row + 32 * i;
    *reinterpret_cast<u32x4 *>(buf + kLdsTile + r * kLdsRow + swz(r, g_chunk) * 16) = rb[i];
  };

  // Fragment q of k-step s (q < 4: A rows wm*128 + 32 q + lane % 32; q >= 4:
  // Bt rows wn*128 + 32 (q - 4) + lane % 32): 32 bytes, chunks c0 and c0 + 1
  // with c0 = 4 s + 2 (lane / 32), read as two halves h.
  const int frag_row = lane & 31, frag_half = lane >> 5, fsw = (frag_row >> 1) & 7;
  const int a_off = (wm * 128 + frag_row) * kLdsRow, b_off = kLdsTile + (wn * 128 + frag_row) * kLdsRow;
  u32x4 f[2][8][2];
  auto read_half = [&](u32x4 (&fr)[8][2], const uint8_t *buf, int s, int q, int h) {
    const int chunk = ((4 * s + 2 * frag_half + h) ^ fsw) * 16;
    const int off = q < 4 ? a_off + q * 32 * kLdsRow : b_off + (q - 4) * 32 * kLdsRow;
    fr[q][h] = *reinterpret_cast<const u32x4 *>(buf + off + chunk);
  };
  // halves in the order the MFMAs (row-major over the 4 x 4 accumulators)
  // first need them: A0, B0, B1, B2, B3, A1, A2, A3
  constexpr int kReadOrder[8] = {0, 4, 5, 6, 7, 1, 2, 3};

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
  auto mfma = [&](const u32x4 (&fr)[8][2], int k) {
    const int i = k >> 2, j = k & 3;
    const u32x4 al = fr[i][0], ah = fr[i][1], bl = fr[4 + j][0], bh = fr[4 + j][1];
    const i32x8 fa = i32x8{(int)al.x, (int)al.y, (int)al.z, (int)al.w, (int)ah.x, (int)ah.y, (int)ah.z, (int)ah.w};
    const i32x8 fb = i32x8{(int)bl.x, (int)bl.y, (int)bl.z, (int)bl.w, (int)bh.x, (int)bh.y, (int)bh.z, (int)bh.w};
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb, fa, acc[i][j], 0, 0, 0, kScaleOne, 0,
                                                                 kScaleOne);
  };

  const int ktiles = K / kBK;
#pragma unroll
  for (int i = 0; i < 8; i++) load_a(0, i);
#pragma unroll
  for (int i = 0; i < 8; i++) load_b(0, i);
#pragma unroll
  for (int i = 0; i < 8; i++) store_a(lds, i);
#pragma unroll
  for (int i = 0; i < 8; i++) store_b(lds, i);
  const int k1 = min(1, ktiles - 1);
#pragma unroll
  for (int i = 0; i < 8; i++) load_a(k1, i);
#pragma unroll
  for (int i = 0; i < 8; i++) load_b(k1, i);
  __syncthreads();
  // in the loop's order: the loop's top waits for what both paths into it
  // have pending, so reads issued here in another order made every
  // iteration begin with a full lgkmcnt(0)
#pragma unroll
  for (int q = 0; q < 16; q++) {
    read_half(f[0], lds, 0, kReadOrder[q >> 1], q & 1);
    __builtin_amdgcn_sched_barrier(0);
  }

  for (int kt = 0; kt < ktiles; kt++) {
    const uint8_t *cur = lds + (kt & 1) * 2 * kLdsTile;
    uint8_t *nxt = lds + ((kt & 1) ^ 1) * 2 * kLdsTile;
    const int k2 = min(kt + 2, ktiles - 1);  // re-reads the last slab at the end, unused
    // step 0: MFMAs, step 1's fragments, then A rows of the next slab out
    // and the A rows of the slab after it requested
#pragma unroll
    for (int k = 0; k < 16; k++) {
      mfma(f[0], k);
      if (k < 8) {
        read_half(f[1], cur, 1, kReadOrder[k], 0);
        read_half(f[1], cur, 1, kReadOrder[k], 1);
      } else {
        store_a(nxt, k - 8);
        load_a(k2, k - 8);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // step 1: the Bt rows likewise, the barrier, then the next slab's step 0
    // fragments under the last four MFMAs
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
#pragma unroll
      for (int h = 0; h < 4; h++) {
        const int q = 4 * (k - 12) + h;
        read_half(f[0], nxt, 0, kReadOrder[q >> 1], q & 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

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
         aligned(sb, 16) && (int64_t)kBM * lda < (1ll << 31) && (int64_t)kBN * ldb < (1ll << 31);
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
