// Dense GEMM C[M,N] = A[M,K] * B[K,N], bf16 operands, fp32 accumulation,
// bf16 output, all row-major. The reference only holds an unused cuBLAS
// handle for this (Kernel.cs:10-11, :16); the workload is BASELINE configs[2].
//
// MFMA kernel (M % 256 == 0, N % 256 == 0, K % 32 == 0, leading dimensions
// multiples of 8 elements, 16-byte aligned operands):
//  - one 256-thread workgroup per 256 x 256 tile of C; its 4 waves own
//    128 x 128 quadrants, each an 8 x 8 grid of v_mfma_f32_16x16x32_bf16
//    accumulators (256 fp32 per lane, held in AGPRs at one wave per SIMD);
//  - the operands go global -> LDS directly (buffer loads with the LDS
//    destination), in 32-wide K stages, four in flight; the next stage's
//    fragments are read under a stage's MFMAs, after the next stage's
//    readiness wait and one barrier (details at the kernel);
//  - A rows are stored K-contiguous in LDS, B as it arrives (N contiguous)
//    and read through the transposing ds_read_b64_tr_b16; both XOR-swizzled
//    so that the fragment reads' lane phases touch distinct banks;
//  - the MFMA is issued as Bt x A so that each lane ends up holding one row
//    of C with runs of 4 consecutive columns (8-byte bf16 stores; 16 lanes
//    write 32 contiguous bytes of each row);
//  - tiles are numbered so that each of the 8 XCDs (workgroups are dealt to
//    XCDs round-robin) computes a 4 x 8 block of tiles, whose A and B slabs
//    its L2 then shares.
// Every other shape takes a bounds-checked LDS-tiled fp32 FMA kernel.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.h"

namespace sh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 256, kBN = 256;
constexpr int kThreads = 256;

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                                  // round to nearest even
  return u >> 16;
}

// ---- MFMA kernel -----------------------------------------------------------
// The operands go global -> LDS by buffer loads with the LDS destination (no
// staging registers, no LDS stores): K advances in 32-wide stages, four in
// flight (128 KiB), each wave issuing 8 of a stage's 32 one-KiB loads. The compiler
// does not count these loads' LDS writes against later LDS reads, so every
// stage's readiness is an explicit s_waitcnt vmcnt (this wave's loads of
// the stage done, the two later stages still in flight) plus s_barrier (the
// other waves' too), never a full vmcnt(0).
//  - A stage: 256 rows x 64 B, the 16-byte chunk c of row r stored at
//    position c ^ ((r / 4) % 4) (16-lane phases of the fragment reads hit
//    distinct banks); a load's lane l writes position l % 4 of row l / 4
//    of its 16-row block, so it fetches chunk (l % 4) ^ swizzle.
//  - B stage: 32 k rows x 512 B (N contiguous, as B is stored), chunk c of
//    k row r at position c ^ (4 (r % 4)); the MFMA's B fragments (8
//    consecutive k of one column per lane) come from pairs of transposing
//    reads (ds_read_b64_tr_b16: within 16 lanes, lane 4 i + q addresses k
//    row kb + i at column cb + 4 q, and lane j receives column cb + j at
//    rows kb .. kb + 3), whose 4-row groups the swizzle spreads over the
//    banks.
//  - A stage is one k-step of v_mfma_f32_16x16x32_bf16: each wave reads 8 A
//    fragments (16 rows x 32 k, one 16-byte read each) and 8 B fragments
//    (16 columns x 32 k, two transposing reads each) and issues 8 x 8
//    MFMAs of 16 cycles. Sustained on every SIMD, this MFMA delivers ~13 %
//    more flops than v_mfma_f32_32x32x16_bf16 under the power limit (~2.34
//    against ~2.07 PFLOP/s in register-only loops), and the kernel, which
//    was power-limited, took ~112 us against ~121-129 us with the 32x32x16
//    tiles of the same stages (launches interleaved in one process), same
//    results bit for bit; the clock it then runs at is no longer below
//    hipBLASLt's.
//  - Per stage: its 8 loads of the stage three ahead, one every kDGap
//    MFMAs from the first (issued back to back they measured ~5 % slower:
//    112 against 115-118 us), the next stage's readiness after MFMA kDBar,
//    then the next stage's 24 fragment reads one per MFMA (into the other
//    fragment set; two per MFMA measured ~9 % slower). Five stages in
//    flight (all 160 KiB of LDS) measured slower than four.
//  - The MFMAs are inline asm with AGPR accumulator operands: through the
//    builtin, the 64 four-register accumulators were shuttled between
//    AGPRs and VGPRs (~180 moves each way per stage pair) and spilled. The
//    compiler does not see these as MFMAs, so: each accumulator is rewritten
//    only 63 MFMAs after its previous write (no dependent-MFMA wait needed),
//    fragment registers are waited for by the load counters like any asm
//    input, and explicit wait states precede the epilogue's accumulator reads.
constexpr int kDK = 32;                      // K per stage
constexpr int kDStages = 4;                  // stages in flight
constexpr int kDA = kBM * kDK * 2;           // A stage bytes (16 KiB)
constexpr int kDStage = kDA + kDK * kBN * 2;  // + B (16 KiB)
constexpr int kDLdsBytes = kDStages * kDStage;
constexpr int kDBar = 39;                    // MFMAs of a stage before the next stage's readiness wait
constexpr int kDGap = 4;                     // MFMAs between a stage's loads

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
#define SH_LDS_AS __attribute__((address_space(3)))

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_mfma_kernel(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                          uint16_t *__restrict__ C, int K, int lda, int ldb, int ldc, int tiles_m,
                          int tiles_n, int grouped) {
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
  // C's pointer is used here, so its scalar load completes before the loop:
  // left pending until the epilogue, it made every wait on the LDS counter
  // at the loop's top a full lgkmcnt(0) (scalar and LDS results return out
  // of order), including the fragments the first MFMAs do not need
  asm volatile("" ::"s"(C));

  // this lane's source offsets for the wave's 4 A and 4 B loads of a stage
  int a_vo[4], b_vo[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int r = (wave * 4 + u) * 16 + (lane >> 2);
    a_vo[u] = (r * lda + (((lane & 3) ^ ((r >> 2) & 3)) * 8)) * 2;
    const int kr = (wave * 4 + u) * 2 + (lane >> 5);
    b_vo[u] = (kr * ldb + (((lane & 31) ^ (4 * (kr & 3))) * 8)) * 2;
  }
  SH_LDS_AS uint8_t *lds3 = (SH_LDS_AS uint8_t *)lds;
  // the same resources as 4-dword descriptors for the asm (base, stride 0,
  // size in bytes, the flags make_buffer_rsrc gets above)
  auto desc = [](const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
  };
  const u32x4 a_d = desc(A + (size_t)tm * kBM * lda, (uint32_t)((255 * lda + K) * 2));
  const u32x4 b_d = desc(B + tn * kBN, (uint32_t)(((K - 1) * ldb + kBN) * 2));
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds3;
  // load u (< 8) of stage kt. Inline asm: through the compiler's builtin,
  // every later LDS read that it could not tell apart from the loads' LDS
  // writes got a full vmcnt(0) wait, which emptied the pipeline; here the
  // explicit per-stage waits below are the only ones.
  auto dma = [&](int kt, int u) {
    const uint32_t m0 = lds_base + (kt % kDStages) * kDStage + (u < 4 ? 0 : kDA) + (wave * 4 + (u & 3)) * 1024;
    if (u < 4)
      asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
                   :: "v"(a_vo[u]), "s"(a_d), "s"(kt * kDK * 2), "{m0}"(m0) : "memory");
    else
      asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
                   :: "v"(b_vo[u - 4]), "s"(b_d), "s"(kt * kDK * ldb * 2), "{m0}"(m0) : "memory");
  };

  // A fragment i (< 8): rows wm 128 + 16 i + lane % 16, k 8 (lane / 16) .. + 7
  // (chunk lane / 16 of the row, swizzled by the row's (r / 4) % 4 =
  // (lane % 16) / 4)
  const int a_base = (wm * 128 + (lane & 15)) * (kDK * 2) + (((lane >> 4) ^ ((lane & 15) >> 2)) * 16);
  // B fragment j (< 8): columns wn 128 + 16 j + lane % 16, k 8 (lane / 16)
  // .. + 7 from two transposing reads (k rows + 4 h); lane 4 ti + tq of
  // 16-lane group G addresses k row 8 G + ti (+ 4 h), columns + 4 tq
  const int G = lane >> 4, ti = (lane >> 2) & 3, tq = lane & 3;
  int b_base[8];
#pragma unroll
  for (int j = 0; j < 8; j++)
    b_base[j] = kDA + (8 * G + ti) * (kBN * 2) + ((16 * wn + 2 * j + (tq >> 1)) ^ (4 * ti)) * 16 + (tq & 1) * 8;
  bf16x8 fa[2][8];
  s16x4 fb[2][8][2];
  auto read_frag = [&](int fs, const SH_LDS_AS uint8_t *st, int r) {
    // read r (< 24) of a stage in the order the MFMAs need them: A0, B0
    // (2), B1 (2), .. B7 (2), A1 .. A7
    if (r == 0 || r >= 17) {
      const int i = r == 0 ? 0 : r - 16;
      fa[fs][i] = *reinterpret_cast<const SH_LDS_AS bf16x8 *>(st + a_base + i * 16 * (kDK * 2));
    } else {
      const int j = (r - 1) >> 1, h = (r - 1) & 1;
      fb[fs][j][h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (SH_LDS_AS s16x4 *)(st + b_base[j] + 4 * h * (kBN * 2)));
    }
  };

  f32x4v acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0f;
  // MFMA k (< 64) of a stage: accumulator (k / 8, k % 8), issued as Bt x A
  // so that each lane ends up holding row lane % 16 of the 16 x 16 block,
  // columns 4 (lane / 16) .. + 3 (8-byte bf16 stores)
  auto mfma = [&](int fs, int k) {
    const int i = k >> 3, j = k & 7;
    const bf16x8 b = __builtin_bit_cast(
        bf16x8, __builtin_shufflevector(fb[fs][j][0], fb[fs][j][1], 0, 1, 2, 3, 4, 5, 6, 7));
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc[i][j]) : "v"(b), "v"(fa[fs][i]));
  };

  // this wave's loads of the oldest stage in flight done (8 loads per
  // stage; the kDStages - 2 later stages may still be in flight)
  static_assert(kDStages == 4, "stage_wait's count");
  static_assert(7 * kDGap < kDBar && 24 <= 63 - kDBar, "a stage's loads precede the wait; all reads fit");
  auto stage_wait = [] { asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); };
  const int ktiles = K / kDK;
  // prologue: stages 0 .. kDStages - 2 requested, stage 0 waited for, its fragments read
#pragma unroll
  for (int p = 0; p < kDStages - 1; p++)
#pragma unroll
    for (int u = 0; u < 8; u++) dma(min(p, ktiles - 1), u);
  stage_wait();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  // in the loop's order (A0 first): the loop's top waits for what both
  // paths into it have pending, so reads issued here in another order
  // made every iteration begin with a full wait
#pragma unroll
  for (int r = 0; r < 24; r++) {
    read_frag(0, lds3, r);
    __builtin_amdgcn_sched_barrier(0);
  }

  // stage kt on fragment set kCur: its MFMAs; the loads of stage kt + 3
  // into the buffer stage kt - 1 used (every wave has read that one: each
  // is past the previous stage's barrier); after MFMA kDBar, stage kt + 1's
  // readiness, then its fragments into the other set (re-reads the last
  // stage past the end; never used)
  auto stage = [&](auto cur_c, int kt) {
    constexpr int kCur = decltype(cur_c)::value;
    const SH_LDS_AS uint8_t *nxt = lds3 + ((kt + 1) % kDStages) * kDStage;
    const int kq = min(kt + kDStages - 1, ktiles - 1);
#pragma unroll
    for (int k = 0; k < 64; k++) {
      mfma(kCur, k);
      if (k % kDGap == 0 && k / kDGap < 8) dma(kq, k / kDGap);
      if (k == kDBar) {
        stage_wait();
        __builtin_amdgcn_s_barrier();
      }
      if (k > kDBar && k - kDBar - 1 < 24) read_frag(kCur ^ 1, nxt, k - kDBar - 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int kt = 0;
  for (; kt + 1 < ktiles; kt += 2) {
    stage(std::integral_constant<int, 0>{}, kt);
    stage(std::integral_constant<int, 1>{}, kt + 1);
  }
  if (kt < ktiles) stage(std::integral_constant<int, 0>{}, kt);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS write in flight past the end
  // the MFMAs are asm: the wait states before the accumulators are read
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int m = tm * kBM + wm * 128 + i * 16 + (lane & 15);
    uint16_t *crow = C + (size_t)m * ldc;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int n0 = tn * kBN + wn * 128 + j * 16 + 4 * (lane >> 4);
      const uint32_t p0 = f32_to_bf16_bits(acc[i][j][0]) | (f32_to_bf16_bits(acc[i][j][1]) << 16);
      const uint32_t p1 = f32_to_bf16_bits(acc[i][j][2]) | (f32_to_bf16_bits(acc[i][j][3]) << 16);
      *reinterpret_cast<u32x2 *>(crow + n0) = u32x2{p0, p1};
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
  return M % kBM == 0 && N % kBN == 0 && K % kDK == 0 && K > 0 && lda % 8 == 0 &&
         ldb % 8 == 0 && ldc % 4 == 0 && aligned16(A) && aligned16(B) &&
         (reinterpret_cast<uintptr_t>(C) & 7) == 0 && (int64_t)kBM * lda * 2 < (1ll << 31) &&
         (int64_t)K * ldb * 2 < (1ll << 31);
}

hipError_t launch_gemm_bf16(hipStream_t s, const uint16_t *A, const uint16_t *B, uint16_t *C,
                            int M, int N, int K, int lda, int ldb, int ldc) {
  if (gemm_bf16_uses_mfma(M, N, K, lda, ldb, ldc, A, B, C)) {
    const void *kfn = reinterpret_cast<const void *>(&gemm_bf16_mfma_kernel);
    const int lds_bytes = kDLdsBytes;
    hipError_t e = hipFuncSetAttribute(kfn, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
    if (e != hipSuccess) return e;
    const int tiles_m = M / kBM, tiles_n = N / kBN;
    const int ntiles = tiles_m * tiles_n;
    const int grouped = (ntiles % 256 == 0 && tiles_m % 4 == 0 && tiles_n % 8 == 0) ? 1 : 0;
    void *args[] = {(void *)&A, (void *)&B, (void *)&C, (void *)&K, (void *)&lda, (void *)&ldb, (void *)&ldc,
                    (void *)&tiles_m, (void *)&tiles_n, (void *)&grouped};
    e = hipLaunchKernel(kfn, dim3(ntiles), dim3(kThreads), args, lds_bytes, s);
    if (e != hipSuccess) return e;
  } else {
    dim3 grid((N + kGT - 1) / kGT, (M + kGT - 1) / kGT);
    gemm_bf16_generic_kernel<<<grid, 256, 0, s>>>(A, B, C, M, N, K, lda, ldb, ldc);
  }
  return hipGetLastError();
}

}  // namespace sh
