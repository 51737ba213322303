// Kernels of the LLM decode path (BASELINE configs[3] GPT-2 small fp16 and
// configs[4] Qwen3-0.6B-shaped FP8): weight quantization / tiling, a fused
// batched GEMV on MFMA, split-K decode attention and the embedding gather.
// The reference has no implementation of any of these (SURVEY rows a14-a16
// of the hot path are defined by BASELINE.json only).
//
// Weight layout ("tiled"): a linear layer W[N][K] (N outputs, K inputs) is
// stored as 1 KiB tiles of 16 rows, tiles of one row group consecutive along
// K. Within a tile, lane l of a wave owns 16 bytes: the 8-element K runs
//   W[n0 + l%16][k0 + 8*(l/16) + e], e = 0..7
// that a v_mfma_f32_16x16x32_f16 B operand holds. An FP8 tile spans 64 K
// values (two MFMA k-steps: bytes 0-7 step 0, bytes 8-15 step 1); an fp16
// tile spans 32 K values. One 16-byte load per lane then feeds the MFMA and a
// wave reads each tile as 1 KiB contiguous.
//
// FP8 is OCP E4M3 (bias 7, max 448, no infinities), one fp32 scale per output
// row: W ~= e4m3(q) * scale[n]. E4M3 values are exact in fp16, so the GEMV's
// products x * q are exact and the scale is applied once to the fp32 sum.
#include <hip/hip_runtime.h>

#include "common.h"
#include "llm.h"
#include "llm_device.h"

namespace sh {
namespace {

typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;

// ---- number formats ---------------------------------------------------------

// fp32 -> OCP E4M3, round to nearest even, saturating to +-448 (NaN -> 0x7f).
__device__ __forceinline__ uint8_t f32_to_e4m3(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x7f;       // NaN
  if (a >= 0x43E00000u) return sign | 0x7e;  // >= 448 (and inf): saturate
  const int e = (int)(a >> 23) - 127;
  if (e < -6) {
    // subnormal range of E4M3: value = m * 2^-9, m = 0..7 (m = 8 rounds up to
    // the smallest normal 0x08)
    const float av = __builtin_bit_cast(float, a);
    const float m = av * 512.0f;  // exact scaling by a power of two
    const float r = __builtin_rintf(m);  // round half to even
    return sign | (uint8_t)r;
  }
  // normal: keep 3 mantissa bits, RNE on the 20 dropped bits
  uint32_t mant = a & 0x7fffffu;
  uint32_t q = ((uint32_t)(e + 7) << 3) | (mant >> 20);
  const uint32_t rest = mant & 0xfffffu;
  if (rest > 0x80000u || (rest == 0x80000u && (q & 1u))) q += 1;  // may carry into exponent
  if (q > 0x7e) q = 0x7e;  // 464 and up round to 448 after saturation
  return sign | (uint8_t)q;
}

// ---- tiled offsets -------------------------------------------------------

// Source row of tiled row n when the layer is a gate/up pair stored with its
// 16-row tiles interleaved (gate tile p, up tile p, ...): logical input is
// [gate (I rows); up (I rows)].
__device__ __forceinline__ int pair_source_row(int n, int interleave_rows) {
  if (interleave_rows == 0) return n;
  const int tile = n >> 4, p = tile >> 1;
  return (tile & 1) ? interleave_rows + 16 * p + (n & 15) : 16 * p + (n & 15);
}

// ---- quantization / tiling kernels --------------------------------------

// One wave per output row: scale = max|w| / 448 (1 when the row is zero),
// q = e4m3(w / scale), written in the tiled layout (or row-major).
__global__ __launch_bounds__(kThreads) void quantize_e4m3_kernel(
    const float *__restrict__ w, int N, int K, int interleave_rows, uint8_t *__restrict__ q,
    float *__restrict__ scales, int tiled) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (n >= N) return;
  const float *row = w + (size_t)pair_source_row(n, interleave_rows) * K;
  float amax = 0.0f;
  for (int k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(row[k]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
  if (lane == 0) scales[n] = scale;
  for (int k = lane; k < K; k += 64)
    q[tiled ? fp8_tiled_offset(n, k, K) : (size_t)n * K + k] = f32_to_e4m3(row[k] / scale);
}

// Row-major E4M3 bytes -> tiled layout.
__global__ __launch_bounds__(kThreads) void pack_e4m3_tiles_kernel(const uint8_t *__restrict__ q,
                                                                   int N, int K,
                                                                   uint8_t *__restrict__ out) {
  const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= (size_t)N * K) return;
  const int n = (int)(i / K), k = (int)(i % K);
  out[fp8_tiled_offset(n, k, K)] = q[i];
}

// fp32 [N][K] -> fp16 tiled (round to nearest even).
__global__ __launch_bounds__(kThreads) void tile_f16_kernel(const float *__restrict__ w, int N,
                                                            int K, int interleave_rows,
                                                            uint16_t *__restrict__ out) {
  const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= (size_t)N * K) return;
  const int n = (int)(i / K), k = (int)(i % K);
  out[f16_tiled_offset(n, k, K)] = f32_to_f16_bits(w[(size_t)pair_source_row(n, interleave_rows) * K + k]);
}

// Counter-based N(mean, std) fill: SplitMix64 of (seed, index) -> two
// uniforms -> Box-Muller. Used for synthetic weights.
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__global__ __launch_bounds__(kThreads) void fill_normal_kernel(float *__restrict__ out, size_t n,
                                                               uint64_t seed, float mean,
                                                               float stddev) {
  const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const uint64_t r = splitmix64(seed * 0x100000001B3ull + i);
  const float u1 = ((float)(uint32_t)(r >> 40) + 0.5f) * (1.0f / 16777216.0f);  // (0, 1)
  const float u2 = (float)((uint32_t)r & 0xffffffu) * (1.0f / 16777216.0f);
  const float z = sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
  out[i] = mean + stddev * z;
}

__global__ __launch_bounds__(kThreads) void fill_f32_kernel(float *out, size_t n, float v) {
  const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) out[i] = v;
}

__global__ __launch_bounds__(kThreads) void f32_to_f16_kernel(const float *in, uint16_t *out,
                                                              size_t n) {
  const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) out[i] = f32_to_f16_bits(in[i]);
}

// ---- GEMV ---------------------------------------------------------------

// Stages the MFMA A operand (activations of B rows, fp16, row stride K + 8
// elements so that the 16 rows of a 16-lane LDS phase fall in 16 distinct
// bank groups) from fp16 activations or from the fp32 residual stream after
// RMSNorm / LayerNorm. Split in two so that the caller can issue its weight
// loads in between: issue() starts the first kStage 16-byte loads of this
// thread (activation rows, then gamma / beta), finish() stores them to LDS,
// loads any remainder, and for the norms takes the statistics (one wave per
// row) from an fp32 copy of the rows in LDS (`xf`, gamma / beta after it).
constexpr int kStage = 4;

template <int kPro>
struct Stager {
  u32x4 v[kStage];
  int total = 0, c4 = 0, rows4 = 0;

  __device__ __forceinline__ u32x4 load_item(const GemvArgs &a, int i) const {
    if (kPro == kProNone) {
      const int chunks = a.K / 8, b = i / chunks, c = i - b * chunks;
      return *reinterpret_cast<const u32x4 *>(a.act + (size_t)b * a.act_ld + c * 8);
    }
    if (i < rows4) {
      const int b = i / c4, c = i - b * c4;
      return *reinterpret_cast<const u32x4 *>(a.x + (size_t)b * a.x_ld + c * 4);
    }
    if (i < rows4 + c4) return *reinterpret_cast<const u32x4 *>(a.gamma + (i - rows4) * 4);
    return *reinterpret_cast<const u32x4 *>(a.beta + (i - rows4 - c4) * 4);
  }

  __device__ __forceinline__ void store_item(const GemvArgs &a, int i, u32x4 val, _Float16 *xs,
                                             float *xf) const {
    if (kPro == kProNone) {
      const int chunks = a.K / 8, b = i / chunks, c = i - b * chunks;
      *reinterpret_cast<u32x4 *>(xs + b * (a.K + 8) + c * 8) = val;
    } else {
      *reinterpret_cast<u32x4 *>(xf + (size_t)i * 4) = val;
    }
  }

  __device__ __forceinline__ void issue(const GemvArgs &a) {
    const int t = threadIdx.x;
    if (kPro == kProNone) {
      total = a.B * (a.K / 8);
    } else {
      c4 = a.K / 4;
      rows4 = a.B * c4;
      total = rows4 + (kPro == kProLayer ? 2 : 1) * c4;
    }
#pragma unroll
    for (int u = 0; u < kStage; u++) {
      const int i = u * kThreads + t;
      if (i < total) v[u] = load_item(a, i);
    }
  }

  __device__ void finish(const GemvArgs &a, _Float16 *xs, float *red, float *xf) {
    const int K = a.K, B = a.B, stride = K + 8;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
#pragma unroll
    for (int u = 0; u < kStage; u++) {
      const int i = u * kThreads + t;
      if (i < total) store_item(a, i, v[u], xs, xf);
    }
    for (int i = kStage * kThreads + t; i < total; i += kThreads) store_item(a, i, load_item(a, i), xs, xf);
    __syncthreads();
    if (kPro == kProNone) return;
    const float *gs = xf + (size_t)B * K, *bs = gs + K;
    // statistics: wave w handles rows w, w + 4, ...; red[8 + b] = mean,
    // red[8 + kMaxBatch + b] = 1 / sqrt(var + eps)
    for (int b = wave; b < B; b += 4) {
      const float *row = xf + (size_t)b * K;
      float mean = 0.0f;
      if (kPro == kProLayer) {
        float sm = 0.0f;
        for (int k = lane; k < K; k += 64) sm += row[k];
        mean = wave_sum(sm) / (float)K;
      }
      float ss = 0.0f;
      for (int k = lane; k < K; k += 64) {
        const float d = row[k] - mean;
        ss += d * d;
      }
      ss = wave_sum(ss);
      if (lane == 0) {
        red[8 + b] = mean;
        red[8 + kMaxBatch + b] = 1.0f / sqrtf(ss / (float)K + a.eps);
      }
    }
    __syncthreads();
    for (int i = t; i < B * K; i += kThreads) {
      const int b = i / K, k = i - b * K;
      float y = (xf[i] - red[8 + b]) * red[8 + kMaxBatch + b] * gs[k];
      if (kPro == kProLayer) y += bs[k];
      xs[b * stride + k] = (_Float16)y;
    }
    __syncthreads();
  }
};

// A workgroup handles kNT row tiles (two for the gate/up pair) at a time,
// grid-striding over tile groups; its 4 waves split K in four and the partial
// 16x16 accumulators are summed in LDS, wave 0 running the epilogue.
// The first batch of weight loads is issued before the activation prologue
// (the weights do not depend on it), so the two memory round trips overlap.
template <int kW, int kPro, int kEpi, int kU>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int kNT = kEpi == kEpiSwiGLU ? 2 : 1;
  constexpr int kKPerLoad = kW == kWeightFp8 ? 64 : 32;
  // kU: 16-byte weight loads per lane per batch (per tile of a pair); the host
  // picks it dividing the wave's loads, so every batch is full and its loads
  // are unconditional
  const int K = a.K, B = a.B;
  const int stride = K + 8;
  _Float16 *xs = reinterpret_cast<_Float16 *>(smem);
  float *red = reinterpret_cast<float *>(smem + (size_t)B * stride * 2);  // 4*2*64*4 floats
  float *xf = red + 4 * 2 * 64 * 4;  // norm prologue: fp32 rows, gamma, beta

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int loads_per_row = K / kKPerLoad;  // 16-byte lane loads per tile row group
  const int per_wave = loads_per_row / 4;
  const int c0 = wave * per_wave;
  const int groups = a.N / (16 * kNT);
  const int g_first = blockIdx.x;
  const int g_step = gridDim.x;
  const int arow = lane & 15, acol = 8 * (lane >> 4);
  const bool arow_valid = arow < B;

  u32x4 wv[kU][kNT];
  auto load_into = [&](u32x4 (&r)[kU][kNT], int g, int c) {
#pragma unroll
    for (int u = 0; u < kU; u++)
#pragma unroll
      for (int j = 0; j < kNT; j++) {
        const size_t tile = (size_t)(g * kNT + j) * loads_per_row + (c + u);
        r[u][j] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4 *>(a.w + tile * 1024 + (size_t)lane * 16));
      }
  };
  auto load_batch = [&](int g, int c) { load_into(wv, g, c); };
  auto mul_from = [&](const u32x4 (&r)[kU][kNT], int c, f32x4 (&acc)[kNT]) {
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int kbase = (c + u) * kKPerLoad;
#pragma unroll
      for (int h = 0; h < kKPerLoad / 32; h++) {
        f16x8 af = {};
        if (arow_valid)
          af = *reinterpret_cast<const f16x8 *>(xs + arow * stride + kbase + 32 * h + acol);
#pragma unroll
        for (int j = 0; j < kNT; j++) {
          f16x8 bf;
          if (kW == kWeightFp8) {
            bf = e4m3x8_to_f16(r[u][j][2 * h], r[u][j][2 * h + 1]);
          } else {
            bf = __builtin_bit_cast(f16x8, r[u][j]);
          }
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc[j], 0, 0, 0);
        }
      }
    }
  };
  auto mul_batch = [&](int c, f32x4 (&acc)[kNT]) { mul_from(wv, c, acc); };

  unsigned long long best[4] = {0, 0, 0, 0};  // logits: running argmax keys per b row
  // lane holds column n = tile row (lane % 16) for batch rows 4*(lane/16) + r
  auto epilogue = [&](int g, const f32x4 (&y)[kNT]) {
    const int col = lane & 15;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int b = 4 * (lane >> 4) + r;
      if (b >= B) continue;
      if (kEpi == kEpiSwiGLU) {
        const int ng = (g * 2) * 16 + col, nu = ng + 16;  // tiled rows of gate / up
        float gv = y[0][r], uv = y[kNT - 1][r];
        if (a.scale) { gv *= a.scale[ng]; uv *= a.scale[nu]; }
        if (a.bias) { gv += a.bias[ng]; uv += a.bias[nu]; }
        const int n = g * 16 + col;  // output column
        a.out16[(size_t)b * a.out_ld + n] = f32_to_f16_bits(silu(gv) * uv);
      } else {
        const int n = g * 16 + col;
        float v = y[0][r];
        if (a.scale) v *= a.scale[n];
        if (a.bias) v += a.bias[n];
        if (kEpi == kEpiStore) {
          a.out[(size_t)b * a.out_ld + n] = v;
        } else if (kEpi == kEpiResidual) {
          a.out[(size_t)b * a.out_ld + n] += v;
        } else if (kEpi == kEpiGelu) {
          a.out16[(size_t)b * a.out_ld + n] = f32_to_f16_bits(gelu_tanh(v));
        } else {  // logits
          if (n < a.n_valid) {
            a.out[(size_t)b * a.out_ld + n] = v;
            const unsigned long long key = argmax_key(v, n);
            best[r] = key > best[r] ? key : best[r];
          }
        }
      }
    }
  };

  // activation loads, then the first weight batch (independent of them),
  // then the prologue: waiting on the activations does not wait on weights
  Stager<kPro> stager;
  stager.issue(a);
  if (g_first < groups) load_batch(g_first, c0);
  __builtin_amdgcn_sched_barrier(0);  // keep every load above ahead of their uses
  stager.finish(a, xs, red, xf);

  for (int g = g_first; g < groups; g += g_step) {
    f32x4 acc[kNT];
#pragma unroll
    for (int j = 0; j < kNT; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int c = c0; c < c0 + per_wave; c += kU) {
      if (g != g_first || c != c0) load_batch(g, c);
      mul_batch(c, acc);
    }
#pragma unroll
    for (int j = 0; j < kNT; j++)
      *reinterpret_cast<f32x4 *>(red + ((wave * kNT + j) * 64 + lane) * 4) = acc[j];
    __syncthreads();
    if (wave == 0) {
      f32x4 y[kNT];
#pragma unroll
      for (int j = 0; j < kNT; j++) {
        y[j] = *reinterpret_cast<const f32x4 *>(red + (j * 64 + lane) * 4);
#pragma unroll
        for (int w = 1; w < 4; w++)
          y[j] += *reinterpret_cast<const f32x4 *>(red + ((w * kNT + j) * 64 + lane) * 4);
      }
      epilogue(g, y);
    }
    __syncthreads();
  }

  if (kEpi == kEpiLogits && wave == 0) {
    // reduce the running keys over the 16 columns held by each lane group
#pragma unroll
    for (int r = 0; r < 4; r++) {
      unsigned long long k = best[r];
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) {
        const unsigned long long o = __shfl_xor(k, off, 64);
        k = o > k ? o : k;
      }
      const int b = 4 * (lane >> 4) + r;
      // this workgroup's slot; most workgroups finish below its running
      // maximum: read it first and only those above it update
      unsigned long long *slot = a.argmax + (blockIdx.x % kKeySlots) * kKeyStride + b;
      if ((lane & 15) == 0 && b < B && k != 0 &&
          k > __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
        atomicMax(slot, k);
    }
  }
}

// ---- decode attention ------------------------------------------------------

// Positions per split: a fixed size for the model (multiple of 16, at least
// 16) chosen by the host from max_positions and the split count, so that a
// workgroup's K / V addresses depend on its block index only and can be
// requested before the context length is known.
// grid (splits, kv_heads, B); one workgroup scores positions [p0, p1) of one
// KV head for its kG query heads, keeps (max, sum, unnormalised V sum) per
// head, and the last workgroup of the (b, kv head) to finish merges all
// splits. Qwen3 (kQwen): q and the new k get RMSNorm over the head and RoPE
// (rotate-half) at position L-1 here; the workgroup whose split holds L-1
// also appends the new k / v to the cache.
//
// Lane layout: kLPP = d/8 lanes per position, each holding 8 dims (16 bytes
// of fp16 K or V); a wave covers kPPW positions per load. Every K (then V)
// load of a thread for up to kBatch positions is issued before any is used.
template <int kD, int kG, bool kQwen>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(const AttnArgs a) {
  constexpr int kLPP = kD / 8;        // lanes per position (8 dims each)
  constexpr int kPPW = 64 / kLPP;     // positions per wave step
  constexpr int kPPB = 4 * kPPW;      // positions per block step
  constexpr int kBatch = 8;           // block steps whose loads are in flight together
  constexpr int kMaxSplits = 64;
  __shared__ float qs[kG][kD];
  __shared__ _Float16 knew[kD], vnew[kD];
  __shared__ float scores[kG][kMaxSplitChunk];
  __shared__ float red[4][kG][kD];
  __shared__ float wsum[8];
  __shared__ float stat[kG][2];

  const int b = blockIdx.z, kvh = blockIdx.y, s = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int chunk = a.chunk;
  // the host sizes `splits` x `chunk` to cover max_pos with chunk <=
  // kMaxSplitChunk and splits <= kMaxSplits; anything else would overrun LDS
  if (chunk > kMaxSplitChunk || chunk < 16 || a.splits > kMaxSplits) return;
  const int p0 = s * chunk;
  if (p0 >= a.max_pos) return;
  const float *qkv = a.qkv + (size_t)b * a.qkv_ld;
  const size_t cache_base = ((size_t)b * a.kv_heads + kvh) * (size_t)a.max_pos * kD;
  const int seg = lane % kLPP, sub = lane / kLPP;
  const uint16_t *kbase = a.kcache + cache_base + seg * 8;
  const uint16_t *vbase = a.vcache + cache_base + seg * 8;
  const int gq = t / kD, iq = t % kD;
  const bool q_thread = t < kG * kD;
  const int half = kD / 2, fi = iq % half;

  // Issue order: the position, this step's q / k / v, norm gains and RoPE,
  // then K and V of the first kBatch block steps of the split (addresses
  // from the block index only; positions past the context are loaded from
  // the allocated cache and discarded). Vector-memory counters retire in
  // issue order, so using the position and q waits only for what precedes
  // them while K / V stay in flight through the q prologue.
  // (unconditional loads at clamped in-bounds indices: no load sits in a
  // branch, so the compiler cannot pull a conversion of it, and the wait it
  // needs, ahead of the K / V loads below)
  const int L = a.pos[b] + 1;  // context including the new token
  const bool may_hold_new = t < kD;
  float qv = qkv[(kvh * kG + min(gq, kG - 1)) * kD + iq];
  float kv = qkv[a.heads * kD + kvh * kD + iq];
  float vv = qkv[(a.heads + a.kv_heads) * kD + kvh * kD + iq];
  float qn = 1.0f, kn = 1.0f, cs = 1.0f, sn = 0.0f;
  if (kQwen) {
    qn = a.q_norm[iq];
    kn = a.k_norm[iq];
    cs = a.rope[(size_t)b * kD + fi];
    sn = a.rope[(size_t)b * kD + half + fi];
  }
  // positions of this split inside the cache; slots past them reload its
  // last position (unconditional loads: no register merge forces a wait)
  const int cap = min(chunk, a.max_pos - p0);
  f16x8 k8[kBatch], v8[kBatch];
#pragma unroll
  for (int u = 0; u < kBatch; u++) {
    const int pi = min(u * kPPB + wave * kPPW + sub, cap - 1);
    k8[u] = *reinterpret_cast<const f16x8 *>(kbase + (size_t)(p0 + pi) * kD);
    v8[u] = *reinterpret_cast<const f16x8 *>(vbase + (size_t)(p0 + pi) * kD);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep every load above ahead of their uses

  const int active = (L + chunk - 1) / chunk;
  if (s >= active || L > a.max_pos) return;
  const int p1 = min(L, p0 + chunk), np = p1 - p0;
  const int pos = L - 1;
  const bool holds_new = p1 == L;
  const bool kv_thread = holds_new && may_hold_new;
  if (!q_thread) qv = 0.0f;
  if (!kv_thread) kv = vv = 0.0f;

  // ---- q (and the new k / v) ----
  {
    if (kQwen) {
      // RMSNorm over each head: wave sums, then the kD / 64 waves of a head
      // combined through LDS (q heads use waves 0..; k uses the first kD/64)
      constexpr int kWavesPerHead = kD / 64;
      const float qss = wave_sum(qv * qv);
      const float kss = wave_sum(kv * kv);
      if (lane == 0) {
        wsum[wave] = qss;
        wsum[4 + wave] = kss;
      }
      __syncthreads();
      if (q_thread) {
        float ss = 0.0f;
#pragma unroll
        for (int w = 0; w < kWavesPerHead; w++) ss += wsum[gq * kWavesPerHead + w];
        qv = qv * (1.0f / sqrtf(ss / kD + a.eps)) * qn;
      }
      if (kv_thread) {
        float ss = 0.0f;
#pragma unroll
        for (int w = 0; w < kWavesPerHead; w++) ss += wsum[4 + w];
        kv = kv * (1.0f / sqrtf(ss / kD + a.eps)) * kn;
      }
      if (q_thread) red[2][gq][iq] = qv;
      if (kv_thread) red[3][0][iq] = kv;
      __syncthreads();
      if (q_thread) {
        const float other = red[2][gq][iq < half ? iq + half : iq - half];
        qv = iq < half ? qv * cs - other * sn : qv * cs + other * sn;
      }
      if (kv_thread) {
        const float other = red[3][0][iq < half ? iq + half : iq - half];
        kv = iq < half ? kv * cs - other * sn : kv * cs + other * sn;
      }
    }
    if (q_thread) qs[gq][iq] = qv * a.scale;
    if (kv_thread) {
      const _Float16 k16 = (_Float16)kv, v16 = (_Float16)vv;
      knew[iq] = k16;
      vnew[iq] = v16;
      a.kcache[cache_base + (size_t)pos * kD + iq] = __builtin_bit_cast(uint16_t, k16);
      a.vcache[cache_base + (size_t)pos * kD + iq] = __builtin_bit_cast(uint16_t, v16);
    }
    __syncthreads();
  }

  float q8[kG][8];
#pragma unroll
  for (int g = 0; g < kG; g++)
#pragma unroll
    for (int e = 0; e < 8; e++) q8[g][e] = qs[g][seg * 8 + e];
#pragma unroll
  for (int u = 0; u < kBatch; u++) {  // the new token's K / V, computed above
    const int pi = u * kPPB + wave * kPPW + sub;
    if (pi < np && p0 + pi == pos) {
      k8[u] = *reinterpret_cast<const f16x8 *>(&knew[seg * 8]);
      v8[u] = *reinterpret_cast<const f16x8 *>(&vnew[seg * 8]);
    }
  }

  // ---- scores ----
  for (int base = 0; base < np; base += kBatch * kPPB) {
    if (base > 0) {
#pragma unroll
      for (int u = 0; u < kBatch; u++) {
        const int pi = base + u * kPPB + wave * kPPW + sub;
        const int p = p0 + pi;
        k8[u] = f16x8{};
        if (pi < np)
          k8[u] = p == pos ? *reinterpret_cast<const f16x8 *>(&knew[seg * 8])
                           : *reinterpret_cast<const f16x8 *>(kbase + (size_t)p * kD);
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; u++) {
      const int pi = base + u * kPPB + wave * kPPW + sub;
#pragma unroll
      for (int g = 0; g < kG; g++) {
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) d += q8[g][e] * (float)k8[u][e];
#pragma unroll
        for (int off = kLPP / 2; off >= 1; off >>= 1) d += __shfl_xor(d, off, 64);
        if (seg == 0 && pi < np) scores[g][pi] = d;
      }
    }
  }
  __syncthreads();

  // ---- softmax statistics (wave g for head g) ----
  if (wave < kG) {
    const int g = wave;
    float m = -INFINITY;
    for (int i = lane; i < np; i += 64) m = fmaxf(m, scores[g][i]);
    m = wave_max(m);
    float l = 0.0f;
    for (int i = lane; i < np; i += 64) {
      const float e = expf(scores[g][i] - m);
      scores[g][i] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      stat[g][0] = m;
      stat[g][1] = l;
    }
  }
  __syncthreads();

  // ---- unnormalised V sums ----
  float acc[kG][8];
#pragma unroll
  for (int g = 0; g < kG; g++)
#pragma unroll
    for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;
  for (int base = 0; base < np; base += kBatch * kPPB) {
    if (base > 0) {
#pragma unroll
      for (int u = 0; u < kBatch; u++) {
        const int pi = base + u * kPPB + wave * kPPW + sub;
        const int p = p0 + pi;
        v8[u] = f16x8{};
        if (pi < np)
          v8[u] = p == pos ? *reinterpret_cast<const f16x8 *>(&vnew[seg * 8])
                           : *reinterpret_cast<const f16x8 *>(vbase + (size_t)p * kD);
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; u++) {
      const int pi = base + u * kPPB + wave * kPPW + sub;
      if (pi < np) {
#pragma unroll
        for (int g = 0; g < kG; g++) {
          const float w = scores[g][pi];
#pragma unroll
          for (int e = 0; e < 8; e++) acc[g][e] += w * (float)v8[u][e];
        }
      }
    }
  }
  // across the position groups of the wave, then across waves
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
      for (int e = 0; e < 8; e++) red[wave][g][seg * 8 + e] = acc[g][e];
  }
  __syncthreads();

  const int h0 = kvh * kG;
  if (active == 1) {  // one split: normalise and write the head output directly
    if (t < kG * kD) {
      const int g = t / kD, i = t % kD;
      const float v = red[0][g][i] + red[1][g][i] + red[2][g][i] + red[3][g][i];
      a.out[(size_t)b * a.out_ld + (h0 + g) * kD + i] = f32_to_f16_bits(v / stat[g][1]);
    }
    return;
  }

  // ---- partials: merged by attn_merge_kernel after this kernel ends (a
  // kernel boundary publishes them to every XCD's L2 without per-workgroup
  // device-scope fences, which write back and invalidate the whole L2) ----
  const size_t pstride = (size_t)kD + 2;
  if (t < kG * kD) {
    const int g = t / kD, i = t % kD;
    float *pp = a.part + (((size_t)b * a.heads + h0 + g) * a.splits + s) * pstride;
    pp[i] = red[0][g][i] + red[1][g][i] + red[2][g][i] + red[3][g][i];
    if (i == 0) {
      pp[kD] = stat[g][0];
      pp[kD + 1] = stat[g][1];
    }
  }
}

// grid (heads, B), kD threads: combines the split partials of one head,
//   out = sum_j exp(m_j - M) acc_j / sum_j exp(m_j - M) l_j,  M = max_j m_j.
// Heads whose context fitted one split were written by the attention kernel.
template <int kD>
__global__ __launch_bounds__(kD) void attn_merge_kernel(const AttnArgs a) {
  constexpr int kMaxSplits = 64;
  __shared__ float w[kMaxSplits];
  __shared__ float lsum[kD / 64];
  const int b = blockIdx.y, h = blockIdx.x, i = threadIdx.x, lane = i & 63;
  const int L = a.pos[b] + 1;
  const int active = (L + a.chunk - 1) / a.chunk;
  if (active <= 1 || active > kMaxSplits || L > a.max_pos) return;
  const size_t pstride = (size_t)kD + 2;
  const float *pp = a.part + ((size_t)b * a.heads + h) * a.splits * pstride;
  // split statistics: thread j < active holds (m_j, l_j)
  const float mj = i < active ? pp[(size_t)i * pstride + kD] : -INFINITY;
  const float lj = i < active ? pp[(size_t)i * pstride + kD + 1] : 0.0f;
  float M = wave_max(mj);
  if (kD > 64) {  // splits never exceed 64: lanes of wave 0 hold them all
    __shared__ float m0;
    if (i == 0) m0 = M;
    __syncthreads();
    M = m0;
  }
  const float wj = i < active ? expf(mj - M) : 0.0f;
  if (i < kMaxSplits) w[i] = wj;
  const float lw = wave_sum(wj * lj);
  if (lane == 0) lsum[i >> 6] = lw;
  __syncthreads();
  float ltot = 0.0f;
#pragma unroll
  for (int k = 0; k < kD / 64; k++) ltot += lsum[k];
  // every split's column value in one batch of loads (active <= 64)
  float x[kMaxSplits];
#pragma unroll
  for (int u = 0; u < kMaxSplits; u++) x[u] = u < active ? pp[(size_t)u * pstride + i] : 0.0f;
  float v = 0.0f;
#pragma unroll
  for (int u = 0; u < kMaxSplits; u++)
    if (u < active) v += w[u] * x[u];
  a.out[(size_t)b * a.out_ld + h * kD + i] = f32_to_f16_bits(v / ltot);
}

// ---- row norm ----------------------------------------------------------------

// grid (B): fp16 out[b] = RMSNorm / LayerNorm of the fp32 row x[b] (the final
// norm before the LM head, done once instead of in every head workgroup).
template <int kPro>
__global__ __launch_bounds__(kThreads) void norm_rows_kernel(const GemvArgs a) {
  constexpr int kPer = 16;  // K <= 4096
  __shared__ float red[4];
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float *x = a.x + (size_t)b * a.x_ld;
  float v[kPer], g[kPer], be[kPer];
#pragma unroll
  for (int u = 0; u < kPer; u++) {
    const int k = u * kThreads + t;
    v[u] = k < a.K ? x[k] : 0.0f;
    g[u] = k < a.K ? a.gamma[k] : 0.0f;
    be[u] = (kPro == kProLayer && k < a.K) ? a.beta[k] : 0.0f;
  }
  float mean = 0.0f;
  if (kPro == kProLayer) {
    float sm = 0.0f;
#pragma unroll
    for (int u = 0; u < kPer; u++) sm += v[u];
    sm = wave_sum(sm);
    if (lane == 0) red[wave] = sm;
    __syncthreads();
    mean = (red[0] + red[1] + red[2] + red[3]) / (float)a.K;
    __syncthreads();
  }
  float ss = 0.0f;
#pragma unroll
  for (int u = 0; u < kPer; u++) {
    const int k = u * kThreads + t;
    const float d = k < a.K ? v[u] - mean : 0.0f;
    ss += d * d;
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)a.K + a.eps);
#pragma unroll
  for (int u = 0; u < kPer; u++) {
    const int k = u * kThreads + t;
    if (k < a.K) {
      float y = (v[u] - mean) * inv * g[u];
      if (kPro == kProLayer) y += be[u];
      a.out16[(size_t)b * a.out_ld + k] = f32_to_f16_bits(y);
    }
  }
}

// ---- embedding -------------------------------------------------------------

// grid (B): reads the token of row b from its argmax keys (the largest over
// the slots; the host writes prompt tokens as keys too), records it in the
// history, clears row b of the key set this step's LM head writes (the one it
// read, or the other set after a decode-layers kernel step), advances the
// row's position and writes the fp32
// residual stream: Qwen3 dequantises the tied FP8 head row, GPT-2 adds the
// fp16 token (tied head) and position rows.
__global__ __launch_bounds__(kThreads) void embed_kernel(const EmbedArgs a) {
  const int b = blockIdx.x, t = threadIdx.x;
  __shared__ int tok_s, pos_s;
  if (t < 64) {  // wave 0: the largest key over the slots, which it clears
    unsigned long long key = 0;
    if (t < kKeySlots) {
      key = a.keys[t * kKeyStride + b];
      a.keys_clear[t * kKeyStride + b] = 0;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const unsigned long long o = __shfl_xor(key, off, 64);
      key = o > key ? o : key;
    }
    if (t == 0) {
      int tok = (int)(0xffffffffu - (uint32_t)(key & 0xffffffffu));
      if (tok < 0 || tok >= a.vocab) tok = 0;
      const int pos = a.lens[b];
      tok_s = tok;
      pos_s = pos;
      if (pos < a.hist_len) a.hist[(size_t)b * a.hist_len + pos] = tok;
      if (a.epoch && b == 0) a.epoch[0] += 1u;
      a.pos[b] = pos;
      a.lens[b] = pos + 1;
    }
  }
  __syncthreads();
  const int tok = tok_s, pos = pos_s;
  if (a.rope && t < a.half) {  // RoPE of this step's position, shared by all layers
    float sn, cs;
    sincosf((float)pos * a.inv_freq[t], &sn, &cs);
    a.rope[(size_t)b * 2 * a.half + t] = cs;
    a.rope[(size_t)b * 2 * a.half + a.half + t] = sn;
  }
  float *x = a.x + (size_t)b * a.x_ld;
  for (int k = t; k < a.K; k += kThreads) {
    float v;
    if (a.fp8_head) {
      const uint8_t q = a.head8[fp8_tiled_offset(tok, k, a.K)];
      const f16x2 h = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((uint32_t)q, 1.0f, false);
      v = (float)h[0] * a.head_scale[tok];
    } else {
      v = f16_bits_to_f32(a.head16[f16_tiled_offset(tok, k, a.K)]);
      if (a.wpe) v += f16_bits_to_f32(a.wpe[(size_t)min(pos, a.max_pos - 1) * a.K + k]);
    }
    x[k] = v;
  }
}

size_t gemv_lds_bytes(const GemvArgs &a, int pro) {
  size_t lds = (size_t)a.B * (a.K + 8) * 2 + 4 * 2 * 64 * 4 * sizeof(float);
  if (pro != kProNone) lds += (size_t)a.B * a.K * 4 + 2 * (size_t)a.K * 4;
  return lds;
}

template <int kW, int kPro, int kEpi, int kU>
hipError_t launch_gemv_t(hipStream_t s, const GemvArgs &a, int grid) {
  gemv_kernel<kW, kPro, kEpi, kU><<<grid, kThreads, gemv_lds_bytes(a, kPro), s>>>(a);
  return hipGetLastError();
}

template <int kW, int kPro, int kEpi>
hipError_t launch_gemv_u(hipStream_t s, const GemvArgs &a, int grid, int u) {
  switch (u) {
    case 8: return launch_gemv_t<kW, kPro, kEpi, 8>(s, a, grid);
    case 6: return launch_gemv_t<kW, kPro, kEpi, 6>(s, a, grid);
    case 4: return launch_gemv_t<kW, kPro, kEpi, 4>(s, a, grid);
    case 2: return launch_gemv_t<kW, kPro, kEpi, 2>(s, a, grid);
    default: return launch_gemv_t<kW, kPro, kEpi, 1>(s, a, grid);
  }
}

// The (weights, prologue, epilogue) combinations the runners and
// sh_gemv_w8a16 use; anything else is rejected.
#define SH_GEMV_COMBOS(X)                \
  X(kWeightFp8, kProNone, kEpiStore)     \
  X(kWeightFp8, kProNone, kEpiResidual)  \
  X(kWeightFp8, kProNone, kEpiLogits)    \
  X(kWeightFp8, kProRms, kEpiStore)      \
  X(kWeightFp8, kProRms, kEpiSwiGLU)     \
  X(kWeightFp16, kProNone, kEpiStore)    \
  X(kWeightFp16, kProNone, kEpiResidual) \
  X(kWeightFp16, kProNone, kEpiLogits)   \
  X(kWeightFp16, kProLayer, kEpiStore)   \
  X(kWeightFp16, kProLayer, kEpiGelu)

template <int kW, int kPro, int kEpi>
hipError_t allow_large_lds() {
  const void *fns[5] = {reinterpret_cast<const void *>(&gemv_kernel<kW, kPro, kEpi, 1>),
                        reinterpret_cast<const void *>(&gemv_kernel<kW, kPro, kEpi, 2>),
                        reinterpret_cast<const void *>(&gemv_kernel<kW, kPro, kEpi, 4>),
                        reinterpret_cast<const void *>(&gemv_kernel<kW, kPro, kEpi, 6>),
                        reinterpret_cast<const void *>(&gemv_kernel<kW, kPro, kEpi, 8>)};
  for (const void *f : fns) {
    const hipError_t e =
        hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

unsigned blocks_for(size_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

}  // namespace

hipError_t launch_gemv(hipStream_t s, const GemvArgs &a_in, int weight_type, int pro, int epi,
                       int max_grid) {
  GemvArgs a = a_in;
  const int groups = a.N / (16 * (epi == kEpiSwiGLU ? 2 : 1));
  // split K over the 4 waves of a workgroup, one tile group per workgroup
  // (grid-striding past max_grid)
  int grid = groups;
  if (max_grid > 0 && grid > max_grid) grid = max_grid;
  const int per_wave = a.K / (weight_type == kWeightFp8 ? 64 : 32) / 4;
  // the deepest batch that divides the wave's share (small K: down to 1)
  if (per_wave < 1) return hipErrorInvalidValue;  // callers check K alignment first
  const int u = per_wave % 8 == 0   ? 8
                : per_wave % 6 == 0 ? 6
                : per_wave % 4 == 0 ? 4
                : per_wave % 2 == 0 ? 2
                                    : 1;
#define SH_DISPATCH(W, P, E) \
  if (weight_type == W && pro == P && epi == E) return launch_gemv_u<W, P, E>(s, a, grid, u);
  SH_GEMV_COMBOS(SH_DISPATCH)
#undef SH_DISPATCH
  return hipErrorInvalidValue;
}

hipError_t launch_attention_partials(hipStream_t s, const AttnArgs &a, int head_dim, int group,
                                     bool qwen, dim3 grid);

hipError_t prepare_gemv_kernels() {
  hipError_t e = hipSuccess;
#define SH_ALLOW(W, P, E) \
  if (e == hipSuccess) e = allow_large_lds<W, P, E>();
  SH_GEMV_COMBOS(SH_ALLOW)
#undef SH_ALLOW
  return e;
}

hipError_t launch_attention(hipStream_t s, const AttnArgs &a, int head_dim, int group, bool qwen,
                            int batch) {
  dim3 grid(a.splits, a.kv_heads, batch);
  hipError_t e = launch_attention_partials(s, a, head_dim, group, qwen, grid);
  if (e != hipSuccess || a.splits == 1) return e;
  dim3 mgrid(a.heads, batch);
  if (head_dim == 128)
    attn_merge_kernel<128><<<mgrid, 128, 0, s>>>(a);
  else
    attn_merge_kernel<64><<<mgrid, 64, 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_attention_partials(hipStream_t s, const AttnArgs &a, int head_dim, int group,
                                     bool qwen, dim3 grid) {
  if (head_dim == 128 && group == 2 && qwen)
    attn_decode_kernel<128, 2, true><<<grid, kThreads, 0, s>>>(a);
  else if (head_dim == 128 && group == 1 && qwen)
    attn_decode_kernel<128, 1, true><<<grid, kThreads, 0, s>>>(a);
  else if (head_dim == 64 && group == 1 && !qwen)
    attn_decode_kernel<64, 1, false><<<grid, kThreads, 0, s>>>(a);
  else if (head_dim == 128 && group == 1 && !qwen)
    attn_decode_kernel<128, 1, false><<<grid, kThreads, 0, s>>>(a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_norm_rows(hipStream_t s, const GemvArgs &a, int pro) {
  if (a.K > 16 * kThreads) return hipErrorInvalidValue;
  if (pro == kProLayer)
    norm_rows_kernel<kProLayer><<<a.B, kThreads, 0, s>>>(a);
  else
    norm_rows_kernel<kProRms><<<a.B, kThreads, 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_embed(hipStream_t s, const EmbedArgs &a, int batch) {
  embed_kernel<<<batch, kThreads, 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_quantize_e4m3_tiled(hipStream_t s, const float *w, int N, int K,
                                      int interleave_rows, uint8_t *q, float *scales,
                                      bool tiled) {
  quantize_e4m3_kernel<<<(N + 3) / 4, kThreads, 0, s>>>(w, N, K, interleave_rows, q, scales,
                                                        tiled ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_pack_e4m3_tiles(hipStream_t s, const uint8_t *q, int N, int K, uint8_t *out) {
  if ((size_t)N * K) pack_e4m3_tiles_kernel<<<blocks_for((size_t)N * K), kThreads, 0, s>>>(q, N, K, out);
  return hipGetLastError();
}

hipError_t launch_tile_f16(hipStream_t s, const float *w, int N, int K, int interleave_rows,
                           uint16_t *out) {
  tile_f16_kernel<<<blocks_for((size_t)N * K), kThreads, 0, s>>>(w, N, K, interleave_rows, out);
  return hipGetLastError();
}

hipError_t launch_fill_normal(hipStream_t s, float *out, size_t n, uint64_t seed, float mean,
                              float stddev) {
  if (n) fill_normal_kernel<<<blocks_for(n), kThreads, 0, s>>>(out, n, seed, mean, stddev);
  return hipGetLastError();
}

hipError_t launch_fill_value(hipStream_t s, float *out, size_t n, float v) {
  if (n) fill_f32_kernel<<<blocks_for(n), kThreads, 0, s>>>(out, n, v);
  return hipGetLastError();
}

hipError_t launch_f32_to_f16(hipStream_t s, const float *in, uint16_t *out, size_t n) {
  if (n) f32_to_f16_kernel<<<blocks_for(n), kThreads, 0, s>>>(in, out, n);
  return hipGetLastError();
}

}  // namespace sh
