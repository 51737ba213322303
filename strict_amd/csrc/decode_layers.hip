// Persistent decode-layers kernel: all decoder layers of one Qwen3 decode
// step (FP8 weights, head_dim 128) in one cooperative launch, one workgroup
// per CU. It replaces the six kernels per layer of the per-op path (norm +
// QKV GEMV, attention, split merge, O GEMV, norm + gate/up GEMV, down GEMV).
//
// Work per layer, as items spread over the workgroups:
//   A  QKV     one 16-row tile of W_qkv each      (RMSNorm of x in every item)
//   B  attn    one (row, KV head, split) each      (q/k norm, RoPE, cache append;
//              the last split of a (row, KV head) to arrive merges the partials)
//   C  O       one 16-row tile of W_o each         (x_mid = x + W_o attn)
//   D  gate/up one gate tile + up tile pair each   (RMSNorm of x_mid, SwiGLU)
//   E  down    one 16-row tile of W_down each      (x = x_mid + W_down act)
// An item publishes its output with device-coherent stores, waits for them
// to complete, then stores the step number into its flag word; an item that
// needs it polls those flags (one wave, one vector load per poll) before
// reading. Weights and K / V do not depend on the step's activations, so they
// are requested before the wait: an item's weights when it starts, a
// workgroup's first attention item's K / V at the start of the layer (they
// then stream while the QKV items run).
// Every wait is bounded by a wall-clock limit; a timeout sets the sticky
// error word, after which every other wait fails at once, so the grid always
// drains. Items of C and E sit on workgroups 0.., those of D after them, so
// the workgroups without an o / down item prefetch gate/up and next-layer
// QKV weights while those run.
//
// With one wave per SIMD nothing hides an instruction's latency, so the item
// code avoids runtime integer division, LDS-based lane shuffles in its
// reductions (DPP within 16-lane rows instead) and single-wave serial loops.
#include <hip/hip_runtime.h>

#include "common.h"
#include "llm.h"
#include "llm_device.h"

namespace sh {
namespace {

constexpr int kT = 256;         // threads per workgroup (4 waves)
constexpr int kD = 128;         // head dim
constexpr int kAttnBatch = 10;  // 16-position block steps of K / V requested ahead
constexpr int kMaxSplits = 64;  // the merge reads one split per lane
constexpr int kPStride = kD + 4;  // floats per attention partial: acc[128], m, l, pad
constexpr int kRowsPerPass = 4;   // batch rows staged together

__device__ __forceinline__ unsigned ld_flag(const unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void st_flag(unsigned *p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Accesses to the exchange buffers (x, qkv, part, attn, act) go through
// buffer instructions with the device-scope cache policy (sc1), like the
// flags: a load never returns a stale copy held by this CU's vector cache or
// this XCD's L2, and a store is visible to every CU once it has completed.
// Offsets are bytes from the buffer start (the buffers are far below 2 GiB).
constexpr int kDeviceScope = 16;  // cache-policy bit sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t xrsrc(const void *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff,
                                           0x00020000);
}

__device__ __forceinline__ u32x4 xld16(const void *base, size_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(xrsrc(base), (int)byte_off, 0, kDeviceScope);
}

__device__ __forceinline__ float xld_f32(const float *base, size_t i) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_raw_buffer_load_b32(xrsrc(base), (int)(i * 4), 0, kDeviceScope));
}

__device__ __forceinline__ void xst_f32(float *base, size_t i, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), xrsrc(base), (int)(i * 4),
                                        0, kDeviceScope);
}

__device__ __forceinline__ void xst_u16(uint16_t *base, size_t i, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, xrsrc(base), (int)(i * 2), 0, kDeviceScope);
}

__device__ __forceinline__ void xst_u64(void *base, size_t byte_off, uint64_t v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), xrsrc(base), (int)byte_off,
                                        0, kDeviceScope);
}

// Small LDS words after the phase areas.
struct Misc {
  int ok;                               // result of the last wait
  int last;                             // this attention item merges
  float part[4][kRowsPerPass];          // per-wave partial sums of squares
};

// True once flags [f, f + n) all hold `epoch`. Wave 0 polls; the result is
// shared through LDS, so all threads return the same value.
__device__ bool wait_flags(const LayersArgs &a, const unsigned *f, int n, unsigned epoch,
                           Misc *misc) {
  if (n <= 0) return true;
  const int t = threadIdx.x, lane = t & 63;
  __syncthreads();  // every thread has read the previous wait's result
  if (t < 64) {
    const unsigned long long t0 = wall_clock64();
    int ok = 1;
    for (int it = 1;; it++) {
      int mine = 1;
      for (int i = lane; i < n; i += 64) mine &= ld_flag(f + i) == epoch ? 1 : 0;
      if (__all(mine)) break;
      if ((it & 15) == 0 && (ld_flag(a.err) != 0 || wall_clock64() - t0 > a.spin_ticks)) {
        ok = 0;
        break;
      }
    }
    if (lane == 0) {
      misc->ok = ok;
      if (!ok) atomicOr(a.err, 1u);
    }
  }
  __syncthreads();
  return misc->ok != 0;
}

// Completes this workgroup's stores, then marks the item done.
__device__ __forceinline__ void publish(unsigned *flag, unsigned epoch) {
  __builtin_amdgcn_s_waitcnt(0);  // every store of this thread has completed
  __syncthreads();
  if (threadIdx.x == 0) st_flag(flag, epoch);
}

// ---- GEMV items ----------------------------------------------------------------

// This wave's quarter of K for tile group g (kNT consecutive 16-row tiles of
// an FP8 tiled matrix with K columns): kL 16-byte loads per lane and tile.
template <int kL, int kNT>
__device__ __forceinline__ void load_weights(u32x4 (&w)[kL][kNT], const uint8_t *W, int K, int g) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = K >> 6;
#pragma unroll
  for (int u = 0; u < kL; u++)
#pragma unroll
    for (int j = 0; j < kNT; j++) {
      const size_t tile = (size_t)(g * kNT + j) * lpr + wave * kL + u;
      w[u][j] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4 *>(W + tile * 1024 + (size_t)lane * 16));
    }
}

// acc[j] (lane: column lane % 16 of batch rows 4 * (lane / 16) + r) = this
// wave's K quarter of xs (B rows, row stride `stride` fp16) times tile j.
template <int kL, int kNT>
__device__ __forceinline__ void mfma_weights(const u32x4 (&w)[kL][kNT], const _Float16 *xs,
                                             int stride, int B, f32x4 (&acc)[kNT]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int arow = lane & 15, acol = 8 * (lane >> 4);
  const int row = arow < B ? arow : 0;  // rows past B read row 0 and are never stored
#pragma unroll
  for (int j = 0; j < kNT; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kL; u++) {
    const int kbase = (wave * kL + u) * 64;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const f16x8 af = *reinterpret_cast<const f16x8 *>(xs + row * stride + kbase + 32 * h + acol);
#pragma unroll
      for (int j = 0; j < kNT; j++)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            af, e4m3x8_to_f16(w[u][j][2 * h], w[u][j][2 * h + 1]), acc[j], 0, 0, 0);
    }
  }
}

// Sums the four waves' accumulators; the result is valid in wave 0.
template <int kNT>
__device__ __forceinline__ void reduce_waves(f32x4 (&acc)[kNT], float *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < kNT; j++)
      *reinterpret_cast<f32x4 *>(red + (((wave - 1) * kNT + j) * 64 + lane) * 4) = acc[j];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int j = 0; j < kNT; j++) {
      const f32x4 r1 = *reinterpret_cast<const f32x4 *>(red + ((0 * kNT + j) * 64 + lane) * 4);
      const f32x4 r2 = *reinterpret_cast<const f32x4 *>(red + ((1 * kNT + j) * 64 + lane) * 4);
      const f32x4 r3 = *reinterpret_cast<const f32x4 *>(red + ((2 * kNT + j) * 64 + lane) * 4);
      acc[j] = (acc[j] + r1) + (r2 + r3);
    }
  }
}

// fp16 rows [B][K] of an exchange buffer (row stride ld) -> xs (row stride
// K + 8); kChunks >= K / 8 / 256 16-byte chunks per thread and row.
template <int kChunks>
__device__ void stage_f16(const uint16_t *src, int ld, int B, int K, _Float16 *xs) {
  const int c8 = K >> 3, t = threadIdx.x;
  for (int b0 = 0; b0 < B; b0 += kRowsPerPass) {
    u32x4 v[kRowsPerPass][kChunks];
#pragma unroll
    for (int r = 0; r < kRowsPerPass; r++)
#pragma unroll
      for (int j = 0; j < kChunks; j++) {
        const int c = min(t + kT * j, c8 - 1);
        v[r][j] = u32x4{0u, 0u, 0u, 0u};
        if (b0 + r < B) v[r][j] = xld16(src, ((size_t)(b0 + r) * ld + c * 8) * 2);  // uniform
      }
#pragma unroll
    for (int r = 0; r < kRowsPerPass; r++)
#pragma unroll
      for (int j = 0; j < kChunks; j++) {
        const int b = b0 + r, c = t + kT * j;
        if (b < B && c < c8) *reinterpret_cast<u32x4 *>(xs + b * (K + 8) + c * 8) = v[r][j];
      }
  }
  __syncthreads();
}

// fp32 rows [B][K] at element x_off of the exchange buffer x (row stride ld)
// -> RMSNorm with gains g -> xs (fp16, row stride K + 8). Each thread keeps
// its 4-float chunks in registers; the per-row sums of squares are combined
// across the four waves through LDS. kChunks >= K / 4 / 256.
template <int kChunks>
__device__ void stage_rms(const float *x, size_t x_off, int ld, const float *g, int B, int K,
                          float eps, _Float16 *xs, Misc *misc) {
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  const int c4 = K >> 2, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  f32x4 gv[kChunks];
#pragma unroll
  for (int j = 0; j < kChunks; j++)
    gv[j] = *reinterpret_cast<const f32x4 *>(g + min(t + kT * j, c4 - 1) * 4);
  for (int b0 = 0; b0 < B; b0 += kRowsPerPass) {
    f32x4 v[kRowsPerPass][kChunks];
#pragma unroll
    for (int r = 0; r < kRowsPerPass; r++)
#pragma unroll
      for (int j = 0; j < kChunks; j++) {
        const int c = min(t + kT * j, c4 - 1);
        v[r][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (b0 + r < B)  // uniform
          v[r][j] = __builtin_bit_cast(f32x4, xld16(x, (x_off + (size_t)(b0 + r) * ld + c * 4) * 4));
      }
#pragma unroll
    for (int r = 0; r < kRowsPerPass; r++) {
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < kChunks; j++)
        if (t + kT * j < c4)
          ss += (v[r][j][0] * v[r][j][0] + v[r][j][1] * v[r][j][1]) +
                (v[r][j][2] * v[r][j][2] + v[r][j][3] * v[r][j][3]);
      ss = wave_sum_rows(ss);
      if (lane == 0) misc->part[wave][r] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRowsPerPass; r++) {
      const int b = b0 + r;
      if (b >= B) break;
      const float ss = (misc->part[0][r] + misc->part[1][r]) + (misc->part[2][r] + misc->part[3][r]);
      const float inv = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
      for (int j = 0; j < kChunks; j++) {
        const int c = t + kT * j;
        if (c < c4) {
          const f32x4 y = v[r][j] * inv * gv[j];
          *reinterpret_cast<f16x4 *>(xs + b * (K + 8) + c * 4) =
              f16x4{(_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]};
        }
      }
    }
    __syncthreads();
  }
}

struct Lds {
  _Float16 *xs;
  float *red;
  Misc *misc;
};

// A: qkv[b][16 i + c] = scale * (W_qkv RMSNorm(x)); w holds the item's
// weights (load_weights, issued by the caller)
template <int kL>
__device__ bool qkv_item(const LayersArgs &a, const LayerPtrs &P, int i, unsigned epoch,
                         const unsigned *wait_f, int wait_n, unsigned *flag, const Lds &s,
                         const u32x4 (&w)[kL][1]) {
  const int lane = threadIdx.x & 63, col = lane & 15;
  const float sc = P.sqkv[i * 16 + col];
  __builtin_amdgcn_sched_barrier(0);
  if (!wait_flags(a, wait_f, wait_n, epoch, s.misc)) return false;
  stage_rms<(kL + 3) / 4>(a.x, 0, a.H, P.norm1, a.B, a.H, a.eps, s.xs, s.misc);
  f32x4 acc[1];
  mfma_weights<kL, 1>(w, s.xs, a.H + 8, a.B, acc);
  reduce_waves<1>(acc, s.red);
  if (threadIdx.x < 64) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int b = 4 * (lane >> 4) + r;
      if (b < a.B) xst_f32(a.qkv, (size_t)b * a.qkv_n + i * 16 + col, acc[0][r] * sc);
    }
  }
  publish(flag, epoch);
  return true;
}

// C: x_mid[b][16 i + c] = x[b][.] + scale * (W_o attn)
template <int kL>
__device__ bool o_item(const LayersArgs &a, const LayerPtrs &P, int i, unsigned epoch,
                       const unsigned *wait_f, int wait_n, unsigned *flag, const Lds &s) {
  const int lane = threadIdx.x & 63, col = lane & 15, K = a.heads * kD;
  u32x4 w[kL][1];
  load_weights<kL, 1>(w, P.wo, K, i);
  const float sc = P.so[i * 16 + col];
  __builtin_amdgcn_sched_barrier(0);
  if (!wait_flags(a, wait_f, wait_n, epoch, s.misc)) return false;
  float rv[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int b = min(4 * (lane >> 4) + r, a.B - 1);
    rv[r] = xld_f32(a.x, (size_t)b * a.H + i * 16 + col);
  }
  stage_f16<(kL + 7) / 8>(a.attn, K, a.B, K, s.xs);
  f32x4 acc[1];
  mfma_weights<kL, 1>(w, s.xs, K + 8, a.B, acc);
  reduce_waves<1>(acc, s.red);
  if (threadIdx.x < 64) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int b = 4 * (lane >> 4) + r;
      if (b < a.B) xst_f32(a.x, (size_t)(kMaxBatch + b) * a.H + i * 16 + col, rv[r] + acc[0][r] * sc);
    }
  }
  publish(flag, epoch);
  return true;
}

// D: act[b][16 p + c] = silu(scale_g * gate) * (scale_u * up) of RMSNorm(x_mid)
template <int kL>
__device__ bool up_item(const LayersArgs &a, const LayerPtrs &P, int p, unsigned epoch,
                        const unsigned *wait_f, int wait_n, unsigned *flag, const Lds &s) {
  const int lane = threadIdx.x & 63, col = lane & 15;
  u32x4 w[kL][2];
  load_weights<kL, 2>(w, P.wup, a.H, p);
  const int ng = 2 * p * 16 + col;  // tiled rows of the gate and up tiles of pair p
  const float sg = P.sup[ng], su = P.sup[ng + 16];
  __builtin_amdgcn_sched_barrier(0);
  if (!wait_flags(a, wait_f, wait_n, epoch, s.misc)) return false;
  stage_rms<(kL + 3) / 4>(a.x, (size_t)kMaxBatch * a.H, a.H, P.norm2, a.B, a.H, a.eps, s.xs, s.misc);
  f32x4 acc[2];
  mfma_weights<kL, 2>(w, s.xs, a.H + 8, a.B, acc);
  reduce_waves<2>(acc, s.red);
  if (threadIdx.x < 64) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int b = 4 * (lane >> 4) + r;
      if (b < a.B)
        xst_u16(a.act, (size_t)b * a.inter + p * 16 + col,
                f32_to_f16_bits(silu(acc[0][r] * sg) * (acc[1][r] * su)));
    }
  }
  publish(flag, epoch);
  return true;
}

// E: x[b][16 i + c] = x_mid[b][.] + scale * (W_down act)
template <int kL>
__device__ bool down_item(const LayersArgs &a, const LayerPtrs &P, int i, unsigned epoch,
                          const unsigned *wait_f, int wait_n, unsigned *flag, const Lds &s) {
  const int lane = threadIdx.x & 63, col = lane & 15, K = a.inter;
  u32x4 w[kL][1];
  load_weights<kL, 1>(w, P.wdown, K, i);
  const float sc = P.sdown[i * 16 + col];
  __builtin_amdgcn_sched_barrier(0);
  if (!wait_flags(a, wait_f, wait_n, epoch, s.misc)) return false;
  float rv[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int b = min(4 * (lane >> 4) + r, a.B - 1);
    rv[r] = xld_f32(a.x, (size_t)(kMaxBatch + b) * a.H + i * 16 + col);
  }
  stage_f16<(kL + 7) / 8>(a.act, K, a.B, K, s.xs);
  f32x4 acc[1];
  mfma_weights<kL, 1>(w, s.xs, K + 8, a.B, acc);
  reduce_waves<1>(acc, s.red);
  if (threadIdx.x < 64) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int b = 4 * (lane >> 4) + r;
      if (b < a.B) xst_f32(a.x, (size_t)b * a.H + i * 16 + col, rv[r] + acc[0][r] * sc);
    }
  }
  publish(flag, epoch);
  return true;
}

// ---- attention item -------------------------------------------------------------

// LDS of an attention item, from the start of the dynamic area.
template <int kG>
struct AttnLds {
  float qs[kG][kD];
  _Float16 knew[kD], vnew[kD];
  float scores[kG][kMaxSplitChunk];
  float red[4][kG][kD];
  float wsum[8];
  float stat[kG][2];
  float mw[kG][kMaxSplits];
  float msum[kG];
  f32x4 macc[8][kG][kD / 4];  // merge: split-group partial sums
};

constexpr int kLPP = kD / 8;     // lanes per position (8 dims each)
constexpr int kPPW = 64 / kLPP;  // positions per wave step
constexpr int kPPB = 4 * kPPW;   // positions per block step

struct AttnKV {
  f16x8 k8[kAttnBatch], v8[kAttnBatch];
};

// K / V of the first kAttnBatch block steps of item `item`, clamped into the
// cache (positions past the context are loaded and never used).
__device__ __forceinline__ void attn_prefetch(const LayersArgs &a, const LayerPtrs &P, int item,
                                              AttnKV &kv) {
  const int splits = a.splits, kvn = a.kv_heads;
  const int s = item % splits, kvh = (item / splits) % kvn, b = item / (splits * kvn);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int chunk = a.chunk, p0 = s * chunk;
  const int cap = min(chunk, a.max_pos - p0);
  const size_t cache_base = ((size_t)b * kvn + kvh) * (size_t)a.max_pos * kD;
  const int seg = lane % kLPP, sub = lane / kLPP;
  const uint16_t *kbase = P.kcache + cache_base + seg * 8;
  const uint16_t *vbase = P.vcache + cache_base + seg * 8;
  const int last = max(cap, 1) - 1;
#pragma unroll
  for (int u = 0; u < kAttnBatch; u++) {
    const int p = min(p0 + min(u * kPPB + wave * kPPW + sub, last), a.max_pos - 1);
    kv.k8[u] = *reinterpret_cast<const f16x8 *>(kbase + (size_t)p * kD);
    kv.v8[u] = *reinterpret_cast<const f16x8 *>(vbase + (size_t)p * kD);
  }
}

// B: item = (b, KV head, split), its K / V requested by attn_prefetch.
// Scores positions [p0, p0 + chunk) of the context for the kG query heads
// of the KV head (Qwen3: RMSNorm of q and of the new k over the head, RoPE
// rotate-half at this step's position; the split holding it appends the new
// k / v to the cache), writes the partial (unnormalised V sum, max, sum) per
// head, then counts its arrival. The split that arrives last merges all
// partials of the (b, KV head):
//   out = sum_j exp(m_j - M) acc_j / sum_j exp(m_j - M) l_j,  M = max_j m_j.
template <int kG>
__device__ bool attn_item(const LayersArgs &a, const LayerPtrs &P, int l, int item,
                          unsigned epoch, const unsigned *fA, unsigned *fB, uint8_t *smem,
                          Misc *misc, AttnKV &kv) {
  AttnLds<kG> &S = *reinterpret_cast<AttnLds<kG> *>(smem);
  const int splits = a.splits, kvn = a.kv_heads;
  const int s = item % splits, kvh = (item / splits) % kvn, b = item / (splits * kvn);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int chunk = a.chunk, p0 = s * chunk;
  const int cap = min(chunk, a.max_pos - p0);  // <= 0 for splits past the cache
  const size_t cache_base = ((size_t)b * kvn + kvh) * (size_t)a.max_pos * kD;
  const int seg = lane % kLPP, sub = lane / kLPP;
  const uint16_t *kbase = P.kcache + cache_base + seg * 8;
  const uint16_t *vbase = P.vcache + cache_base + seg * 8;

  // this KV head's q, k and v tiles of the QKV items
  const int tq = kvh * kG * (kD / 16);
  const int tk = (a.heads * kD + kvh * kD) / 16, tv = ((a.heads + kvn) * kD + kvh * kD) / 16;
  if (!wait_flags(a, fA + tq, kG * (kD / 16), epoch, misc) ||
      !wait_flags(a, fA + tk, kD / 16, epoch, misc) || !wait_flags(a, fA + tv, kD / 16, epoch, misc))
    return false;

  const int L = a.pos[b] + 1;  // context including the new token
  const int active = (L + chunk - 1) / chunk;
  const bool live = s < active && cap > 0 && L <= a.max_pos;
  const int h0 = kvh * kG;
  if (live) {
    const size_t qrow = (size_t)b * a.qkv_n;
    const int gq = t / kD, iq = t % kD, half = kD / 2, fi = iq % half;
    const bool q_thread = t < kG * kD;
    const int p1 = min(L, p0 + chunk), np = p1 - p0, pos = L - 1;
    const bool kv_thread = p1 == L && t < kD;
    float qv = xld_f32(a.qkv, qrow + (h0 + min(gq, kG - 1)) * kD + iq);
    float knv = xld_f32(a.qkv, qrow + a.heads * kD + kvh * kD + iq);
    const float vv = xld_f32(a.qkv, qrow + (a.heads + kvn) * kD + kvh * kD + iq);
    const float qn = P.q_norm[iq], kn = P.k_norm[iq];
    const float cs = a.rope[(size_t)b * kD + fi], sn = a.rope[(size_t)b * kD + half + fi];
    if (!q_thread) qv = 0.0f;
    if (!kv_thread) knv = 0.0f;
    // RMSNorm over each head (kD / 64 waves per head), then RoPE
    {
      constexpr int kWavesPerHead = kD / 64;
      const float qss = wave_sum_rows(qv * qv), kss = wave_sum_rows(knv * knv);
      if (lane == 0) {
        S.wsum[wave] = qss;
        S.wsum[4 + wave] = kss;
      }
      __syncthreads();
      if (q_thread) {
        float ss = 0.0f;
#pragma unroll
        for (int w = 0; w < kWavesPerHead; w++) ss += S.wsum[gq * kWavesPerHead + w];
        qv = qv * (1.0f / sqrtf(ss / kD + a.eps)) * qn;
      }
      if (kv_thread) {
        float ss = 0.0f;
#pragma unroll
        for (int w = 0; w < kWavesPerHead; w++) ss += S.wsum[4 + w];
        knv = knv * (1.0f / sqrtf(ss / kD + a.eps)) * kn;
      }
      if (q_thread) S.red[2][gq][iq] = qv;
      if (kv_thread) S.red[3][0][iq] = knv;
      __syncthreads();
      if (q_thread) {
        const float other = S.red[2][gq][iq < half ? iq + half : iq - half];
        qv = iq < half ? qv * cs - other * sn : qv * cs + other * sn;
      }
      if (kv_thread) {
        const float other = S.red[3][0][iq < half ? iq + half : iq - half];
        knv = iq < half ? knv * cs - other * sn : knv * cs + other * sn;
      }
    }
    if (q_thread) S.qs[gq][iq] = qv * a.scale;
    if (kv_thread) {
      const _Float16 k16 = (_Float16)knv, v16 = (_Float16)vv;
      S.knew[iq] = k16;
      S.vnew[iq] = v16;
      P.kcache[cache_base + (size_t)pos * kD + iq] = __builtin_bit_cast(uint16_t, k16);
      P.vcache[cache_base + (size_t)pos * kD + iq] = __builtin_bit_cast(uint16_t, v16);
    }
    __syncthreads();

    float q8[kG][8];
#pragma unroll
    for (int g = 0; g < kG; g++)
#pragma unroll
      for (int e = 0; e < 8; e++) q8[g][e] = S.qs[g][seg * 8 + e];
#pragma unroll
    for (int u = 0; u < kAttnBatch; u++) {  // the new token's K / V
      const int pi = u * kPPB + wave * kPPW + sub;
      if (pi < np && p0 + pi == pos) {
        kv.k8[u] = *reinterpret_cast<const f16x8 *>(&S.knew[seg * 8]);
        kv.v8[u] = *reinterpret_cast<const f16x8 *>(&S.vnew[seg * 8]);
      }
    }

    // scores: a position's 16 lanes are one DPP row
    for (int base = 0; base < np; base += kAttnBatch * kPPB) {
      if (base > 0) {
#pragma unroll
        for (int u = 0; u < kAttnBatch; u++) {
          const int pi = base + u * kPPB + wave * kPPW + sub, p = p0 + pi;
          kv.k8[u] = f16x8{};
          if (pi < np)
            kv.k8[u] = p == pos ? *reinterpret_cast<const f16x8 *>(&S.knew[seg * 8])
                                : *reinterpret_cast<const f16x8 *>(kbase + (size_t)p * kD);
        }
      }
#pragma unroll
      for (int u = 0; u < kAttnBatch; u++) {
        const int pi = base + u * kPPB + wave * kPPW + sub;
#pragma unroll
        for (int g = 0; g < kG; g++) {
          float d = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; e++) d += q8[g][e] * (float)kv.k8[u][e];
          d = row16_sum(d);
          if (seg == 0 && pi < np) S.scores[g][pi] = d;
        }
      }
    }
    __syncthreads();

    // softmax statistics (wave g for head g)
    if (wave < kG) {
      const int g = wave;
      float m = -INFINITY;
      for (int i = lane; i < np; i += 64) m = fmaxf(m, S.scores[g][i]);
      m = wave_max_rows(m);
      float lsum = 0.0f;
      for (int i = lane; i < np; i += 64) {
        const float e = expf(S.scores[g][i] - m);
        S.scores[g][i] = e;
        lsum += e;
      }
      lsum = wave_sum_rows(lsum);
      if (lane == 0) {
        S.stat[g][0] = m;
        S.stat[g][1] = lsum;
      }
    }
    __syncthreads();

    // unnormalised V sums
    float acc[kG][8];
#pragma unroll
    for (int g = 0; g < kG; g++)
#pragma unroll
      for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;
    for (int base = 0; base < np; base += kAttnBatch * kPPB) {
      if (base > 0) {
#pragma unroll
        for (int u = 0; u < kAttnBatch; u++) {
          const int pi = base + u * kPPB + wave * kPPW + sub, p = p0 + pi;
          kv.v8[u] = f16x8{};
          if (pi < np)
            kv.v8[u] = p == pos ? *reinterpret_cast<const f16x8 *>(&S.vnew[seg * 8])
                                : *reinterpret_cast<const f16x8 *>(vbase + (size_t)p * kD);
        }
      }
#pragma unroll
      for (int u = 0; u < kAttnBatch; u++) {
        const int pi = base + u * kPPB + wave * kPPW + sub;
        if (pi < np) {
#pragma unroll
          for (int g = 0; g < kG; g++) {
            const float wgt = S.scores[g][pi];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] += wgt * (float)kv.v8[u][e];
          }
        }
      }
    }
#pragma unroll
    for (int g = 0; g < kG; g++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        float v = acc[g][e];
#pragma unroll
        for (int off = kLPP; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
        acc[g][e] = v;
      }
    if (sub == 0) {
#pragma unroll
      for (int g = 0; g < kG; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) S.red[wave][g][seg * 8 + e] = acc[g][e];
    }
    __syncthreads();
    if (t < kG * kD) {
      const int g = t / kD, i = t % kD;
      const size_t pp = (((size_t)b * a.heads + h0 + g) * splits + s) * kPStride;
      xst_f32(a.part, pp + i, S.red[0][g][i] + S.red[1][g][i] + S.red[2][g][i] + S.red[3][g][i]);
      if (i == 0) {
        const uint64_t ml = (uint64_t)__builtin_bit_cast(uint32_t, S.stat[g][0]) |
                            ((uint64_t)__builtin_bit_cast(uint32_t, S.stat[g][1]) << 32);
        xst_u64(a.part, (pp + kD) * 4, ml);
      }
    }
  }

  // arrival; every split of the (b, KV head) counts, live or not
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    unsigned *cnt = a.counters + ((size_t)l * kMaxBatch + b) * kvn + kvh;
    const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    misc->last = (old + 1) % (unsigned)splits == 0 ? 1 : 0;
  }
  __syncthreads();
  if (!misc->last) return true;

  // merge (active <= splits <= kMaxSplits): every thread requests its split
  // group's 16-byte columns and waves g < kG the split statistics together;
  // then the split weights per head (wave g) and the weighted sums
  {
    constexpr int kQuads = kD / 4;               // 16-byte column groups per head
    constexpr int kGroups = kT / (kG * kQuads);  // split groups (4 for kG = 2, 8 for kG = 1)
    constexpr int kPer = kMaxSplits / kGroups;   // splits per group at most
    const int g = t / (kGroups * kQuads), rem = t % (kGroups * kQuads);
    const int q = rem % kQuads, sg = rem / kQuads;
    const size_t base = ((size_t)b * a.heads + h0 + g) * splits * kPStride;
    const int n_my = (active - sg + kGroups - 1) / kGroups;  // splits sg, sg + kGroups, ...
    f32x4 xv[kPer];
#pragma unroll
    for (int u = 0; u < kPer; u++) {
      const int j = min(sg + u * kGroups, active - 1);  // unused slots reload a valid split
      xv[u] = __builtin_bit_cast(f32x4, xld16(a.part, (base + (size_t)j * kPStride + q * 4) * 4));
    }
    if (wave < kG) {
      const size_t pw = ((size_t)b * a.heads + h0 + wave) * splits * kPStride;
      const int j = min(lane, active - 1);
      float mj = xld_f32(a.part, pw + (size_t)j * kPStride + kD);
      float lj = xld_f32(a.part, pw + (size_t)j * kPStride + kD + 1);
      if (lane >= active) {
        mj = -INFINITY;
        lj = 0.0f;
      }
      const float M = wave_max_rows(mj);
      const float wj = lane < active ? expf(mj - M) : 0.0f;
      const float lw = wave_sum_rows(wj * lj);
      S.mw[wave][lane] = wj;
      if (lane == 0) S.msum[wave] = lw;
    }
    __syncthreads();
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kPer; u++)
      if (u < n_my) sum += S.mw[g][sg + u * kGroups] * xv[u];
    S.macc[sg][g][q] = sum;
    __syncthreads();
    if (sg == 0) {
      f32x4 v = S.macc[0][g][q];
#pragma unroll
      for (int k = 1; k < kGroups; k++) v += S.macc[k][g][q];
      const float inv = 1.0f / S.msum[g];
      const uint64_t packed = (uint64_t)f32_to_f16_bits(v[0] * inv) |
                              ((uint64_t)f32_to_f16_bits(v[1] * inv) << 16) |
                              ((uint64_t)f32_to_f16_bits(v[2] * inv) << 32) |
                              ((uint64_t)f32_to_f16_bits(v[3] * inv) << 48);
      xst_u64(a.attn, ((size_t)b * a.heads * kD + (h0 + g) * kD + q * 4) * 2, packed);
    }
  }
  publish(fB + b * kvn + kvh, epoch);
  return true;
}

// ---- the kernel ----------------------------------------------------------------

template <int kG, int kLA, int kLC, int kLD, int kLE>
__global__ __launch_bounds__(kT, 1) void decode_layers_kernel(const LayersArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  Misc *misc = reinterpret_cast<Misc *>(smem + a.lds_misc);
  const int B = a.B, H = a.H;
  Lds lds;
  lds.xs = reinterpret_cast<_Float16 *>(smem);
  const int kmax = max(H, max(a.heads * kD, a.inter));
  const size_t xs_max = ((size_t)B * (kmax + 8) * 2 + 15) / 16 * 16;
  lds.red = reinterpret_cast<float *>(smem + xs_max);
  lds.misc = misc;

  const unsigned epoch = *a.epoch;
  const int G = gridDim.x, w = blockIdx.x;
  const int nA = a.qkv_n / 16, nB = B * a.kv_heads * a.splits, nC = H / 16;
  const int nD = a.inter / 16, nE = H / 16;
  AttnKV kv;
  u32x4 wa[kLA][1];  // this workgroup's first QKV item's weights
  if (w < nA) load_weights<kLA, 1>(wa, a.layers[0].wqkv, H, w);
  for (int l = 0; l < a.n_layers; l++) {
    const LayerPtrs P = a.layers[l];
    unsigned *F = a.flags + (size_t)l * a.flags_per_layer;
    const unsigned *prevE = a.flags + (size_t)(l > 0 ? l - 1 : 0) * a.flags_per_layer + a.fE;
    if (w < nB) attn_prefetch(a, P, w, kv);  // streams while the QKV items run
    for (int i = w; i < nA; i += G) {
      if (i != w) load_weights<kLA, 1>(wa, P.wqkv, H, i);
      if (!qkv_item<kLA>(a, P, i, epoch, prevE, l > 0 ? nE : 0, F + i, lds, wa)) return;
    }
    for (int i = w; i < nB; i += G) {
      if (i != w) attn_prefetch(a, P, i, kv);
      if (!attn_item<kG>(a, P, l, i, epoch, F, F + a.fB, smem, misc, kv)) return;
    }
    for (int i = w; i < nC; i += G)
      if (!o_item<kLC>(a, P, i, epoch, F + a.fB, B * a.kv_heads, F + a.fC + i, lds)) return;
    for (int i = (w + G - nC % G) % G; i < nD; i += G)
      if (!up_item<kLD>(a, P, i, epoch, F + a.fC, nC, F + a.fD + i, lds)) return;
    // the next layer's first QKV weights, before the down items wait
    if (l + 1 < a.n_layers && w < nA) load_weights<kLA, 1>(wa, a.layers[l + 1].wqkv, H, w);
    for (int i = w; i < nE; i += G)
      if (!down_item<kLE>(a, P, i, epoch, F + a.fD, nD, F + a.fE + i, lds)) return;
  }
}

// (kG, loads per lane of qkv / o / gate-up / down items) per supported shape
#define SH_LAYERS_SHAPES(X) \
  X(2, 4, 8, 4, 12)  /* hidden 1024, 16 x 128 query heads, 8 KV heads, inter 3072 */ \
  X(2, 1, 2, 1, 3)   /* hidden 256, 4 x 128 query heads, 2 KV heads, inter 768 */

struct Shape {
  int g, la, lc, ld, le;
};

Shape shape_of(int H, int heads, int kv_heads, int inter) {
  return Shape{kv_heads > 0 ? heads / kv_heads : 0, H / 256, heads * kD / 256, H / 256, inter / 256};
}

const void *kernel_for(const Shape &s) {
#define SH_MATCH(G, LA, LC, LD, LE)                                               \
  if (s.g == G && s.la == LA && s.lc == LC && s.ld == LD && s.le == LE)           \
    return reinterpret_cast<const void *>(&decode_layers_kernel<G, LA, LC, LD, LE>);
  SH_LAYERS_SHAPES(SH_MATCH)
#undef SH_MATCH
  return nullptr;
}

size_t attn_lds(int g) {
  return g == 1 ? sizeof(AttnLds<1>) : sizeof(AttnLds<2>);
}

}  // namespace

bool decode_layers_supported(int H, int heads, int kv_heads, int head_dim, int inter) {
  if (head_dim != kD || kv_heads <= 0 || heads % kv_heads != 0) return false;
  if (H % 256 || (heads * kD) % 256 || inter % 256 || H > 4096) return false;
  return kernel_for(shape_of(H, heads, kv_heads, inter)) != nullptr;
}

size_t decode_layers_lds(int B, int H, int heads, int inter, int *misc_offset) {
  int kmax = H;
  if (heads * kD > kmax) kmax = heads * kD;
  if (inter > kmax) kmax = inter;
  const size_t xs_max = ((size_t)B * (kmax + 8) * 2 + 15) / 16 * 16;
  size_t end = xs_max + 3 * 2 * 64 * 4 * sizeof(float);  // + wave-reduction area
  const size_t attn = attn_lds(2);
  if (attn > end) end = attn;
  end = (end + 15) / 16 * 16;
  *misc_offset = (int)end;
  return end + sizeof(Misc);
}

hipError_t decode_layers_occupancy(const LayersArgs &a, size_t lds, int *blocks_per_cu) {
  const void *k = kernel_for(shape_of(a.H, a.heads, a.kv_heads, a.inter));
  if (!k) return hipErrorInvalidValue;
  hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k, kT, lds);
}

hipError_t launch_decode_layers(hipStream_t s, const LayersArgs &a, int grid, size_t lds) {
  const void *k = kernel_for(shape_of(a.H, a.heads, a.kv_heads, a.inter));
  if (!k) return hipErrorInvalidValue;
  void *args[] = {const_cast<LayersArgs *>(&a)};
  return hipLaunchCooperativeKernel(k, dim3(grid), dim3(kT), args, (unsigned)lds, s);
}

}  // namespace sh
