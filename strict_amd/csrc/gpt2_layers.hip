// Persistent GPT-2 layers kernel: all decoder layers of one GPT-2 decode
// step at batch 1 (fp16 weights, head_dim 64, LayerNorm, biases, GELU) in one
// launch, one workgroup per CU, all resident together. It replaces the five
// kernels per layer of the per-op path (LayerNorm + QKV GEMV, attention,
// O GEMV + residual, LayerNorm + fc GEMV + GELU, proj GEMV + residual), each
// ~3-6 us whatever its size, with exchanges between workgroups of ~1-1.5 us.
//
// Work per layer, as items spread over the workgroups:
//   A  QKV   one 16-row tile of W_qkv each      (LayerNorm of x in every item)
//   B  attn  one (head, split) each             (cache append, partial softmax)
//   C  O     one 16-row tile of W_o each        (merges the splits of every
//                                                head, x_mid = x + W_o attn + b)
//   D  fc    one 16-row tile of W_fc each       (LayerNorm of x_mid, GELU)
//   E  proj  one 16-row tile of W_proj each     (x = x_mid + W_proj act + b)
// and, on steps with logits, after the last layer:
//   H  head  16-row tiles of the LM head          (final LayerNorm, logits,
//                                                  greedy argmax)
//
// Items: A on workgroups 0.., C and E on 0.., D after the C range, B on the
// last workgroups; at most one item per workgroup and phase. Exchange:
// exchange.h (tagged cells, bounded waits). Weights and K / V do not depend
// on the step's activations: each workgroup requests the next layer's QKV
// weights and K / V after its last item of a layer, and an item's other
// weights when it starts, so they arrive while earlier phases run.
//
// Rounding points follow the per-op path and the oracle: LayerNorm
// statistics in fp32 over the row, its output fp16 (the MFMA A operand);
// q, k, v fp32 from the QKV GEMV, k and v stored fp16 in the cache; q scaled
// by 1 / sqrt(64) in fp32; scores, softmax and the V sums in fp32, the
// merged attention output fp16; residual stream fp32; GELU output fp16.
#include <hip/hip_runtime.h>

#include "common.h"

#ifdef SH_GPT2_TRACE
// Diagnostic builds only (-DSH_GPT2_TRACE): wall-clock marks per workgroup
// and layer: slots 0..4 the ends of its A..E items, 5..9 the ends of their
// waits, 10 the kernel's start (layer 0), 11 the head's end (layer 0),
// 12..15 the ends of the attention item's q / k / v staging, scores,
// softmax and V sums; layer 15 slot 15: the XCD the workgroup ran on;
// layer n_layers slot 0: the end of the LM head's final-LayerNorm wait.
constexpr int kTrWgs = 256, kTrLayers = 16, kTrSlots = 16;
__device__ unsigned long long g_gpt2_trace[kTrWgs][kTrLayers][kTrSlots];
#define SH_G2MARK(l, slot)                                                              \
  do {                                                                                   \
    if (threadIdx.x == 0 && blockIdx.x < kTrWgs && (l) < kTrLayers)                     \
      g_gpt2_trace[blockIdx.x][l][slot] = wall_clock64();                               \
  } while (0)
#else
#define SH_G2MARK(l, slot) ((void)0)
#endif
#define SH_G2WAIT(l, p) SH_G2MARK(l, 5 + (p))

#include "exchange.h"
#include "llm.h"
#include "llm_device.h"

namespace sh {
namespace {

using namespace xchg;

constexpr int kT = 256;     // threads per workgroup (4 waves)
constexpr int kHd = 64;     // head dim
constexpr int kMaxChunk = 256;  // positions per split (one per thread)
constexpr int kVJ = kMaxChunk / 32;  // V rows per thread
// Wall-clock ticks (100 MHz) the fc workgroups wait before requesting the
// next layer's K / V and QKV weights (see the layer loop).
constexpr unsigned long long kPrefetchDelay = 125;

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));


struct LayerP {
  const SH_XGLOBAL uint16_t *wqkv, *wo, *wfc, *wproj;
  const SH_XGLOBAL float *bqkv, *bo, *bfc, *bproj;
  const SH_XGLOBAL float *ln1_g, *ln1_b, *ln2_g, *ln2_b;
  SH_XGLOBAL uint16_t *kcache, *vcache;
};

__device__ __forceinline__ LayerP layer_p(const Gpt2Args &a, int l) {
  const SH_XCONST Gpt2LayerPtrs &p = cnst(a.layers)[l];
  return LayerP{gbl(p.wqkv),  gbl(p.wo),    gbl(p.wfc),   gbl(p.wproj), gbl(p.bqkv),
                gbl(p.bo),    gbl(p.bfc),   gbl(p.bproj), gbl(p.ln1_g), gbl(p.ln1_b),
                gbl(p.ln2_g), gbl(p.ln2_b), gbl(p.kcache), gbl(p.vcache)};
}

// LDS of a workgroup (one batch row).
struct Lds {
  alignas(16) _Float16 xs[4096 + 8];  // the MFMA A operand row (fp16)
  alignas(16) float red[3][64][4];    // waves 1..3's accumulators
  float part[2][4];                   // per-wave LayerNorm statistics (means, squared deviations)
  Votes votes;
  // attention
  alignas(16) float q[kHd];
  alignas(16) _Float16 knew[kHd];
  alignas(16) _Float16 vnew[kHd];
  float p[kMaxChunk];
  float wmax[4], wl[4];
  alignas(16) float pv[4][kHd];
};

// ---- GEMV items ----------------------------------------------------------------

// This wave's quarter of K for 16-row tile g of an fp16 tiled matrix with K
// columns (1 KiB tiles of 16 rows x 32 K): kL 16-byte loads per lane (those
// of u in [kU0, kU1)).
template <int kL, int kU0 = 0, int kU1 = kL>
__device__ __forceinline__ void load_weights(u32x4 (&w)[kL], const SH_XGLOBAL uint16_t *W, int K, int g) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tiles = K >> 5;
#pragma unroll
  for (int u = kU0; u < kU1; u++) {
    const size_t tile = (size_t)g * tiles + wave * kL + u;
    w[u] = __builtin_nontemporal_load(reinterpret_cast<const SH_XGLOBAL u32x4 *>(
        reinterpret_cast<const SH_XGLOBAL uint8_t *>(W) + tile * 1024 + (size_t)lane * 16));
  }
}

// This wave's K quarter of row 0 of xs times the tile (lanes 0..15 of the
// result's r = 0 hold the 16 columns; every A row reads row 0).
template <int kL>
__device__ __forceinline__ f32x4 mfma_weights(const u32x4 (&w)[kL], const _Float16 *xs) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const _Float16 *xrow = xs + wave * kL * 32 + 8 * (lane >> 4);
  constexpr int kCh = kL < 4 ? kL : 4;  // independent accumulator chains
  f32x4 part[kCh];
#pragma unroll
  for (int c = 0; c < kCh; c++) part[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kL; u++) {
    const f16x8 af = *reinterpret_cast<const f16x8 *>(xrow + u * 32);
    part[u % kCh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, __builtin_bit_cast(f16x8, w[u]),
                                                          part[u % kCh], 0, 0, 0);
  }
  f32x4 acc = part[0];
#pragma unroll
  for (int c = 1; c < kCh; c++) acc += part[c];
  return acc;
}

// Sums the four waves' accumulators; the result is valid in wave 0.
__device__ __forceinline__ f32x4 reduce_waves(f32x4 acc, Lds &S) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave > 0) *reinterpret_cast<f32x4 *>(S.red[wave - 1][lane]) = acc;
  lds_barrier();
  if (wave == 0) {
    const f32x4 r1 = *reinterpret_cast<const f32x4 *>(S.red[0][lane]);
    const f32x4 r2 = *reinterpret_cast<const f32x4 *>(S.red[1][lane]);
    const f32x4 r3 = *reinterpret_cast<const f32x4 *>(S.red[2][lane]);
    acc = (acc + r1) + (r2 + r3);
  }
  return acc;
}

// The 4-value chunks of a K-value row a thread stages: wave w holds those of
// its K quarter, [w K / 16, (w + 1) K / 16), lane l the chunks w K / 16 + l +
// 64 j. That is the quarter of xs the wave's MFMAs read (mfma_weights), so a
// GEMV item needs no workgroup barrier between staging and its MFMAs: a
// wave's LDS reads follow its own writes in order.
__device__ __forceinline__ int stage_chunk(int K, int j) {
  return (threadIdx.x >> 6) * (K >> 4) + (threadIdx.x & 63) + 64 * j;
}
__device__ __forceinline__ bool stage_chunk_ok(int K, int j) {
  return (threadIdx.x & 63) + 64 * j < (K >> 4);
}

// The 2-value pairs of a K-value row stage_ln stages: wave w holds those of
// its K quarter, [w K / 8, (w + 1) K / 8), lane l the pairs w K / 8 + l +
// 64 i (the same quarter of xs as stage_chunk). A pair is two adjacent
// cells, so a wave's poll of its pairs i is one lane-contiguous 16-byte load,
// which reaches memory as the fewest line requests.
__device__ __forceinline__ int stage_pair(int K, int i) {
  return (threadIdx.x >> 6) * (K >> 3) + (threadIdx.x & 63) + 64 * i;
}
__device__ __forceinline__ bool stage_pair_ok(int K, int i) {
  return (threadIdx.x & 63) + 64 * i < (K >> 3);
}

// The first layer's input row straight from the embedding tables: row `tok`
// of the tied head (fp16 tiled) plus the position row `wpe_row`, summed in
// fp32 (the per-op path's embed kernel does the same sum).
struct Emb {
  int tok = -1;  // < 0: the row comes from cells
  const SH_XGLOBAL uint16_t *wte = nullptr, *wpe_row = nullptr;
};

// Values k, k + 1 of the embedded row (k even).
__device__ __forceinline__ f32x2 emb2(const Emb &e, int k, int K) {
  const uint32_t t = *reinterpret_cast<const SH_XGLOBAL uint32_t *>(e.wte + f16_tiled_offset(e.tok, k, K));
  const uint32_t p = *reinterpret_cast<const SH_XGLOBAL uint32_t *>(e.wpe_row + k);
  return f32x2{f16_bits_to_f32((uint16_t)t) + f16_bits_to_f32((uint16_t)p),
               f16_bits_to_f32((uint16_t)(t >> 16)) + f16_bits_to_f32((uint16_t)(p >> 16))};
}

__device__ __forceinline__ float emb1(const Emb &e, int k, int K) {
  return f16_bits_to_f32(e.wte[f16_tiled_offset(e.tok, k, K)]) + f16_bits_to_f32(e.wpe_row[k]);
}

// LayerNorm of the fp32 row x (K values: cells tagged `tag`, or the embedded
// row e when e.tok >= 0) with gains g and biases b -> xs (fp16). A thread
// holds the 2-value pairs stage_pair(K, i), i < 2 kC (kC >= K / 1024).
// kLocal: the caller's waves read only their own K quarter of xs, so no
// barrier follows the stores.
template <int kC, bool kLocal>
__device__ __forceinline__ bool stage_ln(const Gpt2Args &a, const uint64_t *xc, const Emb &e,
                                         unsigned tag, const SH_XGLOBAL float *g,
                                         const SH_XGLOBAL float *bta, int K, Lds &S) {
  constexpr int kP = 2 * kC;
  const int c2 = K >> 1;
  f32x2 gv[kP], bv[kP], v[kP];
#pragma unroll
  for (int i = 0; i < kP; i++) {
    const int c = min(stage_pair(K, i), c2 - 1);
    gv[i] = *reinterpret_cast<const SH_XGLOBAL f32x2 *>(g + c * 2);
    bv[i] = *reinterpret_cast<const SH_XGLOBAL f32x2 *>(bta + c * 2);
  }
  bool ok = true;
  if (e.tok >= 0) {
#pragma unroll
    for (int i = 0; i < kP; i++) v[i] = emb2(e, min(stage_pair(K, i), c2 - 1) * 2, K);
  } else {
    uint64_t cv[kP * 2];
    uint64_t mask = 0;
#pragma unroll
    for (int i = 0; i < kP; i++)
      if (stage_pair_ok(K, i)) mask |= 3ull << (i * 2);
    ok = spin_pairs(a, xc, [&](int k) { return (size_t)min(stage_pair(K, k >> 1), c2 - 1) * 2 + (k & 1); },
                    mask, tag, cv);
#pragma unroll
    for (int i = 0; i < kP; i++) v[i] = f32x2{cell_f32(cv[2 * i]), cell_f32(cv[2 * i + 1])};
  }
  // Statistics in one exchange between the waves: each wave's mean and sum
  // of squared deviations over its K / 4 values, merged as
  //   mean = sum_w mean_w / 4,  M2 = sum_w M2_w + (K / 4) sum_w (mean_w - mean)^2
  // (exact in real arithmetic, as stable as two passes over the row); the
  // waits' vote shares that barrier.
  const int vpar = vote_cast(!ok, &S.votes);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float nw = (float)(K >> 2);
  float sm = 0.0f;
#pragma unroll
  for (int i = 0; i < kP; i += 2) {
    const float s0 = stage_pair_ok(K, i) ? v[i][0] + v[i][1] : 0.0f;
    const float s1 = stage_pair_ok(K, i + 1) ? v[i + 1][0] + v[i + 1][1] : 0.0f;
    sm += s0 + s1;
  }
  const float mw = wave_sum_rows(sm) / nw;
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kP; i += 2) {
    const f32x2 d0 = v[i] - mw, d1 = v[i + 1] - mw;
    const float s0 = stage_pair_ok(K, i) ? d0[0] * d0[0] + d0[1] * d0[1] : 0.0f;
    const float s1 = stage_pair_ok(K, i + 1) ? d1[0] * d1[0] + d1[1] * d1[1] : 0.0f;
    ss += s0 + s1;
  }
  ss = wave_sum_rows(ss);
  if (lane == 0) {
    S.part[0][wave] = mw;
    S.part[1][wave] = ss;
  }
  lds_barrier();
  if (!waits_done(a, vote_seen(vpar, &S.votes))) return false;
  const float mean = ((S.part[0][0] + S.part[0][1]) + (S.part[0][2] + S.part[0][3])) * 0.25f;
  const float e0 = S.part[0][0] - mean, e1 = S.part[0][1] - mean, e2 = S.part[0][2] - mean,
              e3 = S.part[0][3] - mean;
  const float m2 = ((S.part[1][0] + S.part[1][1]) + (S.part[1][2] + S.part[1][3])) +
                   nw * ((e0 * e0 + e1 * e1) + (e2 * e2 + e3 * e3));
  const float inv = 1.0f / sqrtf(m2 / (float)K + a.eps);
#pragma unroll
  for (int i = 0; i < kP; i++) {
    const int c = stage_pair(K, i);
    if (stage_pair_ok(K, i)) {
      const f32x2 y = (v[i] - mean) * inv * gv[i] + bv[i];
      *reinterpret_cast<f16x2 *>(S.xs + c * 2) = f16x2{(_Float16)y[0], (_Float16)y[1]};
    }
  }
  if (!kLocal) lds_barrier();
  return true;
}

// fp16 row of K values packed two per cell (tagged `tag`) -> xs. A thread
// holds the two-cell chunks stage_chunk(K, j), j < kC; the caller's waves
// read only their own K quarter of xs.
template <int kC>
__device__ __forceinline__ bool stage_f16(const Gpt2Args &a, const uint64_t *cells, unsigned tag,
                                          int K, Lds &S) {
  const int c4 = K >> 2;
  uint64_t cv[kC * 2];
  uint64_t mask = 0;
#pragma unroll
  for (int j = 0; j < kC; j++)
    if (stage_chunk_ok(K, j)) mask |= 3ull << (j * 2);
  const bool ok = spin_pairs(
      a, cells, [&](int k) { return (size_t)min(stage_chunk(K, k >> 1), c4 - 1) * 2 + (k & 1); }, mask, tag, cv);
  wave_waits_ok(a, ok);  // no vote (no barrier): see wave_waits_ok
#pragma unroll
  for (int j = 0; j < kC; j++) {
    const int c = stage_chunk(K, j);
    if (stage_chunk_ok(K, j))
      *reinterpret_cast<u32x2 *>(S.xs + c * 4) = u32x2{(uint32_t)cv[2 * j], (uint32_t)cv[2 * j + 1]};
  }
  return true;
}

// A: qkv[16 i + c] = W_qkv LayerNorm(x) + b; w holds the item's weights;
// local: every consumer of the cells runs on this XCD (cst)
template <int kLH>
__device__ __forceinline__ bool qkv_item(const Gpt2Args &a, const LayerP &P, int l, int i, unsigned ep,
                                         const Emb &e, Lds &S, const u32x4 (&w)[kLH], bool local) {
  const int lane = threadIdx.x & 63, col = lane & 15;
  const float bias = P.bqkv[i * 16 + col];
  __builtin_amdgcn_sched_barrier(0);
  if (!stage_ln<(kLH * 128 + 1023) / 1024, true>(a, a.x0c, l == 0 ? e : Emb{}, tag_of(ep, l - 1),
                                            P.ln1_g, P.ln1_b, a.H, S))
    return false;
  SH_G2WAIT(l, 0);
  f32x4 acc = reduce_waves(mfma_weights<kLH>(w, S.xs), S);
  if (threadIdx.x < 16) cst(a.qkvc, (size_t)i * 16 + col, bits_of(acc[0] + bias), tag_of(ep, l), local);
  SH_G2MARK(l, 0);
  return true;
}

// K / V rows of attention item (head h, split s), requested ahead of the
// item. Thread t = 4 g + q holds dims 16 q .. 16 q + 15 of the K rows p0 + g
// + 64 m, m < 4 (k[2 m], k[2 m + 1]: a quarter of each dot product, the
// four quarters summed across the lane quad), and, for dims 8 (t % 8) ..,
// the V rows p0 + t / 8 + 32 j. Positions are clamped to the cached ones
// (before this step's token, which the item substitutes from its cells).
struct AttnKV {
  u32x4 k[8];
  u32x4 v[kVJ];
};

__device__ __forceinline__ void attn_prefetch(const Gpt2Args &a, const LayerP &P, int item, int L,
                                              AttnKV &kv) {
  const int h = item / kGpt2Splits, s = item % kGpt2Splits, t = threadIdx.x;
  const int p0 = s * a.chunk, last = max(min(L - 2, p0 + a.chunk - 1), 0);
  const SH_XGLOBAL uint16_t *kb = P.kcache + (size_t)h * a.max_pos * kHd;
  const SH_XGLOBAL uint16_t *vb = P.vcache + (size_t)h * a.max_pos * kHd;
  const int kq = t & 3, kg = t >> 2;
#pragma unroll
  for (int m = 0; m < 4; m++) {
    const int pk = min(p0 + kg + 64 * m, last);
#pragma unroll
    for (int hh = 0; hh < 2; hh++)
      kv.k[2 * m + hh] = *reinterpret_cast<const SH_XGLOBAL u32x4 *>(kb + (size_t)pk * kHd + 16 * kq + 8 * hh);
  }
  const int d8 = t & 7, pg = t >> 3;
#pragma unroll
  for (int j = 0; j < kVJ; j++) {
    const int pv = min(p0 + pg + 32 * j, last);
    kv.v[j] = *reinterpret_cast<const SH_XGLOBAL u32x4 *>(vb + (size_t)pv * kHd + 8 * d8);
  }
}


// x + x of lane l ^ kX (kX 16 or 32) in every lane: v_permlane16_swap /
// v_permlane32_swap exchange the odd and even 16-lane rows / the halves of
// two registers, so on two copies of x their sum is the pair sum. Inline
// asm with two read-write operands: through the compiler's builtins, the
// two results of a swap of one value were folded into one (x' + x'). The
// s_nop covers the wait states between the copy and the swap.
template <int kX>
__device__ __forceinline__ float add_lane_swap(float x) {
  unsigned u = __builtin_bit_cast(unsigned, x), v = u;
  if (kX == 16)
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(u), "+v"(v));
  else
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(u), "+v"(v));
  return __builtin_bit_cast(float, u) + __builtin_bit_cast(float, v);
}

// B: item = (head h, split s): positions [p0, min(p0 + chunk, L)) of the
// context. Appends the new token's k / v to the cache when the split holds
// it, writes the partial (unnormalised V sum, max, sum) as cells. Splits past
// the context write nothing.
__device__ __forceinline__ bool attn_item(const Gpt2Args &a, const LayerP &P, int l, int item,
                                          unsigned ep, int L, Lds &S, AttnKV &kv) {
  const int h = item / kGpt2Splits, s = item % kGpt2Splits;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int p0 = s * a.chunk;
  if (p0 >= L) return true;  // uniform
  const int np = min(a.chunk, L - p0), pos = L - 1;
  const bool holds_new = p0 + np == L;
  const unsigned tag = tag_of(ep, l);
  {  // q, the new k and the new v as 96 cell pairs (one 16-byte load each):
     // thread t < 96 holds dims 2 (t % 32), + 1 of part t / 32 (q, k, v)
    const int pr = min(t, 95), part = pr >> 5, d = 2 * (pr & 31);
    const size_t cell = (size_t)part * a.H + (size_t)h * kHd + d;
    uint64_t cv[2];
    const bool ok = spin_pairs(a, a.qkvc, [&](int) { return cell; }, t < 96 ? 3ull : 0ull, tag, cv);
    if (!waits_ok(a, ok, &S.votes)) return false;
    SH_G2WAIT(l, 1);
    const float v0 = cell_f32(cv[0]), v1 = cell_f32(cv[1]);
    if (t < 32) {
      S.q[d] = v0 * a.scale;
      S.q[d + 1] = v1 * a.scale;
    } else if (t < 96) {
      const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
      _Float16 *dst = t < 64 ? S.knew : S.vnew;
      dst[d] = h0;
      dst[d + 1] = h1;
      if (holds_new) {
        SH_XGLOBAL uint16_t *c = (t < 64 ? P.kcache : P.vcache) + ((size_t)h * a.max_pos + pos) * kHd + d;
        *reinterpret_cast<SH_XGLOBAL uint32_t *>(c) =
            (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
      }
    }
  }
  lds_barrier();
  SH_G2MARK(l, 12);
  // scores: thread t = 4 g + q sums dims 16 q .. 16 q + 15 of positions
  // g + 64 m, m < 4 (four independent chains, q read from LDS once); the
  // quad's lanes then add their quarters (DPP), and thread t keeps the
  // score of position g + 64 q. The new token's K first replaces the cache
  // copy in the registers of the quad that holds it.
  const int kq = t & 3, kg = t >> 2;
  f32x4 qr[4];
#pragma unroll
  for (int i = 0; i < 4; i++) qr[i] = *reinterpret_cast<const f32x4 *>(&S.q[16 * kq + 4 * i]);
  const int pn = pos - p0;  // the new token's index in the split (when holds_new)
  if (holds_new) {          // uniform
    // selects on every m (a branch per m became a dynamic register index,
    // which put kv in scratch memory)
    const u32x4 kn[2] = {*reinterpret_cast<const u32x4 *>(&S.knew[16 * kq]),
                         *reinterpret_cast<const u32x4 *>(&S.knew[16 * kq + 8])};
#pragma unroll
    for (int m = 0; m < 4; m++) {
      const bool hit = kg + 64 * m == pn;
#pragma unroll
      for (int hh = 0; hh < 2; hh++) kv.k[2 * m + hh] = hit ? kn[hh] : kv.k[2 * m + hh];
    }
  }
  float s4[4];
#pragma unroll
  for (int m = 0; m < 4; m++) {
    float acc = 0.0f;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      const f16x8 kr = __builtin_bit_cast(f16x8, kv.k[2 * m + hh]);
#pragma unroll
      for (int e = 0; e < 8; e++) acc += qr[2 * hh + e / 4][e % 4] * (float)kr[e];
    }
    s4[m] = acc;
  }
#pragma unroll
  for (int m = 0; m < 4; m++) {
    s4[m] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s4[m]), 0xB1, 0xf, 0xf, false));
    s4[m] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s4[m]), 0x4E, 0xf, 0xf, false));
  }
  const int pi_own = kg + 64 * kq;  // this thread's position in the split
  float sc = kq == 0 ? s4[0] : kq == 1 ? s4[1] : kq == 2 ? s4[2] : s4[3];
  sc = pi_own < np ? sc : -INFINITY;
  float m = wave_max_rows(sc);
  if (lane == 0) S.wmax[wave] = m;
  lds_barrier();
  SH_G2MARK(l, 13);
  m = fmaxf(fmaxf(S.wmax[0], S.wmax[1]), fmaxf(S.wmax[2], S.wmax[3]));
  const float e = pi_own < np ? expf(sc - m) : 0.0f;
  S.p[pi_own] = e;
  const float ls = wave_sum_rows(e);
  if (lane == 0) S.wl[wave] = ls;
  lds_barrier();
  SH_G2MARK(l, 14);
  const float lsum = (S.wl[0] + S.wl[1]) + (S.wl[2] + S.wl[3]);
  // V sums: thread (d8 = t % 8, pg = t / 8) over positions pg + 32 j
  // (p = 0 past the split's end); the new token's V from LDS
  const int d8 = t & 7, pg = t >> 3;
  const u32x4 vnw = *reinterpret_cast<const u32x4 *>(&S.vnew[8 * d8]);
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kVJ; j++) {
    const int pi = pg + 32 * j;
    const float pw = S.p[pi];
    const f16x8 vr = __builtin_bit_cast(f16x8, p0 + pi == pos ? vnw : kv.v[j]);
#pragma unroll
    for (int q = 0; q < 8; q++) o[q] += pw * (float)vr[q];
  }
  // sum over pg: lanes l, l ^ 8, l ^ 16, l ^ 32 share d8 within a wave
  // (DPP row_ror:8 within 16-lane rows, then the gfx950 row / half swaps)
#pragma unroll
  for (int q = 0; q < 8; q++) {
    o[q] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, o[q]), 0x128, 0xf, 0xf, false));
    o[q] = add_lane_swap<16>(o[q]);
    o[q] = add_lane_swap<32>(o[q]);
  }
  if (lane < 8) {
#pragma unroll
    for (int q = 0; q < 8; q++) S.pv[wave][8 * lane + q] = o[q];
  }
  lds_barrier();
  SH_G2MARK(l, 15);
  const size_t pp = ((size_t)h * kGpt2Splits + s) * kGpt2PStride;
  if (t < kHd) {
    const float v = (S.pv[0][t] + S.pv[1][t]) + (S.pv[2][t] + S.pv[3][t]);
    cst(a.partc, pp + t, bits_of(v), tag);
  } else if (t == kHd) {
    cst(a.partc, pp + kHd, bits_of(m), tag);
  } else if (t == kHd + 1) {
    cst(a.partc, pp + kHd + 1, bits_of(lsum), tag);
  }
  SH_G2MARK(l, 1);
  return true;
}

// The attention output of every head (the splits merged, fp16) -> xs: a
// thread computes the dim pairs wave H / 4 + 2 (lane + 64 j), j < kC2, of
// the H = heads * 64 (the wave's K quarter of the O item's MFMAs, so no
// barrier follows), over the first kNS splits (the active ones, ns <= kNS;
// the polls load only those: every poll of a wait reloads all of its
// cells). A pair's two acc cells and its split's (max, sum) cells are each
// one 16-byte load (partials start at even cells, 68 apart).
template <int kC, int kNS>
__device__ __forceinline__ bool stage_attn_n(const Gpt2Args &a, unsigned tag, int ns, Lds &S) {
  const int lane = threadIdx.x & 63, q2 = a.H >> 3, base = (threadIdx.x >> 6) * (a.H >> 2);
  constexpr int kC2 = (kC + 1) / 2;
  constexpr int kN = kC2 * kNS * 4;
  uint64_t cv[kN];
  uint64_t mask = 0;
#pragma unroll
  for (int j = 0; j < kC2; j++)
#pragma unroll
    for (int s = 0; s < kNS; s++)
      if (s < ns && lane + 64 * j < q2) mask |= 15ull << ((j * kNS + s) * 4);
  const bool ok = spin_pairs(a, a.partc,
                             [&](int k) {
                               const int j = k / (kNS * 4), s = (k / 4) % kNS, f = k % 4;
                               const int idx = base + 2 * min(lane + 64 * j, q2 - 1), h = idx >> 6, d = idx & 63;
                               const size_t pp = ((size_t)h * kGpt2Splits + min(s, ns - 1)) * kGpt2PStride;
                               return pp + (f == 0 ? d : kHd);
                             },
                             mask, tag, cv);
  wave_waits_ok(a, ok);  // no vote (no barrier): see wave_waits_ok
#pragma unroll
  for (int j = 0; j < kC2; j++) {
    if (lane + 64 * j >= q2) continue;
    const int idx = base + 2 * (lane + 64 * j);
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < kNS; s++)
      if (s < ns) M = fmaxf(M, cell_f32(cv[(j * kNS + s) * 4 + 2]));
    float num0 = 0.0f, num1 = 0.0f, den = 0.0f;
#pragma unroll
    for (int s = 0; s < kNS; s++)
      if (s < ns) {
        const int k = (j * kNS + s) * 4;
        const float f = expf(cell_f32(cv[k + 2]) - M);
        num0 += f * cell_f32(cv[k]);
        num1 += f * cell_f32(cv[k + 1]);
        den += f * cell_f32(cv[k + 3]);
      }
    S.xs[idx] = (_Float16)(num0 / den);
    S.xs[idx + 1] = (_Float16)(num1 / den);
  }
  return true;
}

template <int kC>
__device__ __forceinline__ bool stage_attn(const Gpt2Args &a, unsigned tag, int L, Lds &S) {
  const int ns = (L + a.chunk - 1) / a.chunk;  // uniform
  if (ns == 1) return stage_attn_n<kC, 1>(a, tag, ns, S);
  if (ns == 2) return stage_attn_n<kC, 2>(a, tag, ns, S);
  return stage_attn_n<kC, kGpt2Splits>(a, tag, ns, S);
}

// C: x_mid[16 i + c] = x[.] + W_o attn + b
template <int kLH>
__device__ __forceinline__ bool o_item(const Gpt2Args &a, const LayerP &P, int l, int i, unsigned ep,
                                       int L, const Emb &e, Lds &S) {
  const int lane = threadIdx.x & 63, col = lane & 15;
  u32x4 w[kLH];
  load_weights<kLH>(w, P.wo, a.H, i);
  const float bias = P.bo[i * 16 + col];
  const size_t cell = (size_t)i * 16 + col;
  uint64_t rc = cld(a.x0c, cell);  // the residual (layer 0: the embedded row)
  const float x0 = l == 0 ? emb1(e, (int)cell, a.H) : 0.0f;
  __builtin_amdgcn_sched_barrier(0);
  if (!stage_attn<(kLH * 128 + 255) / 256>(a, tag_of(ep, l), L, S)) return false;
  SH_G2WAIT(l, 2);
  const f32x4 acc = reduce_waves(mfma_weights<kLH>(w, S.xs), S);
  if (threadIdx.x < 16) {
    float x = x0;
    if (l > 0) {
      if (!finish_cell(a, a.x0c, cell, tag_of(ep, l - 1), rc)) atomicOr(a.err, 1u);
      x = cell_f32(rc);
    }
    cst(a.x1c, cell, bits_of(x + (acc[0] + bias)), tag_of(ep, l));
  }
  asm volatile("" ::"v"(rc));  // the residual load retires here in every thread
  SH_G2MARK(l, 2);
  return true;
}

// D: act[16 i + c] = gelu(W_fc LayerNorm(x_mid) + b), fp16, two per cell
template <int kLH>
__device__ __forceinline__ bool fc_item(const Gpt2Args &a, const LayerP &P, int l, int i, unsigned ep,
                                        Lds &S) {
  const int lane = threadIdx.x & 63, col = lane & 15;
  u32x4 w[kLH];
  load_weights<kLH>(w, P.wfc, a.H, i);
  const float bias = P.bfc[i * 16 + col];
  __builtin_amdgcn_sched_barrier(0);
  if (!stage_ln<(kLH * 128 + 1023) / 1024, true>(a, a.x1c, Emb{}, tag_of(ep, l), P.ln2_g, P.ln2_b, a.H, S))
    return false;
  SH_G2WAIT(l, 3);
  const f32x4 acc = reduce_waves(mfma_weights<kLH>(w, S.xs), S);
  if (threadIdx.x < 64) {
    const uint32_t hv = f32_to_f16_bits(gelu_tanh(acc[0] + bias));
    const uint32_t nb = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hv, 0xB1, 0xf, 0xf, false);
    if (threadIdx.x < 16 && (col & 1) == 0)
      cst(a.actc, ((size_t)i * 16 + col) / 2, hv | (nb << 16), tag_of(ep, l));
  }
  SH_G2MARK(l, 3);
  return true;
}

// E: x[16 i + c] = x_mid[.] + W_proj act + b (w: the item's weights, requested
// by the caller); the last layer also writes x to the plain buffer x_in (the
// model's residual-stream tensor)
template <int kLH, int kLI>
__device__ __forceinline__ bool proj_item(const Gpt2Args &a, const LayerP &P, int l, int i, unsigned ep,
                                          Lds &S, const u32x4 (&w)[kLI]) {
  const int lane = threadIdx.x & 63, col = lane & 15;
  const float bias = P.bproj[i * 16 + col];
  const size_t cell = (size_t)i * 16 + col;
  const unsigned tag = tag_of(ep, l);
  uint64_t rc = cld(a.x1c, cell);
  __builtin_amdgcn_sched_barrier(0);
  if (!stage_f16<(kLI * 128 + 1023) / 1024>(a, a.actc, tag, a.inter, S)) return false;
  SH_G2WAIT(l, 4);
  const f32x4 acc = reduce_waves(mfma_weights<kLI>(w, S.xs), S);
  if (threadIdx.x < 16) {
    if (!finish_cell(a, a.x1c, cell, tag, rc)) atomicOr(a.err, 1u);
    const float v = cell_f32(rc) + (acc[0] + bias);
    if (l + 1 == a.n_layers) gbl(a.x_in)[cell] = v;
    cst(a.x0c, cell, bits_of(v), tag);
  }
  asm volatile("" ::"v"(rc));
  SH_G2MARK(l, 4);
  return true;
}

// H (steps with logits): the final LayerNorm of x, then the LM head. Wave v
// of workgroup w owns the 16-row tiles j = w + G v, w + G v + 4 G, ..; a
// tile's 16 KiB x (H / 32) of weights stream through 4 H / 128 loads per
// lane, the next tile's requested while the current one is multiplied. The
// logits are written, and each wave folds its argmax keys into its slot.
template <int kLH>
__device__ __forceinline__ void head_load(u32x4 (&w)[4 * kLH], const Gpt2Args &a, int j) {
  const int lane = threadIdx.x & 63, jj = min(j, a.head_tiles - 1);  // past the end: unused
  const SH_XGLOBAL uint8_t *W = reinterpret_cast<const SH_XGLOBAL uint8_t *>(gbl(a.head_w));
#pragma unroll
  for (int u = 0; u < 4 * kLH; u++)
    w[u] = __builtin_nontemporal_load(reinterpret_cast<const SH_XGLOBAL u32x4 *>(
        W + ((size_t)jj * 4 * kLH + u) * 1024 + (size_t)lane * 16));
}

template <int kLH>
__device__ __forceinline__ bool head_phase(const Gpt2Args &a, unsigned ep, Lds &S,
                                           u32x4 (&wb)[2][4 * kLH]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, G = gridDim.x, w = blockIdx.x;
  const int first = w + G * wave, step = 4 * G, nT = a.head_tiles;
  if (!stage_ln<(kLH * 128 + 1023) / 1024, false>(a, a.x0c, Emb{}, tag_of(ep, a.n_layers - 1),
                                            gbl(a.final_g), gbl(a.final_b), a.H, S))
    return false;
  SH_G2MARK(a.n_layers, 0);
  const _Float16 *xrow = S.xs + 8 * (lane >> 4);
  unsigned long long best = 0;
  auto tile = [&](const u32x4 (&wt)[4 * kLH], int j) {
    f32x4 part[4];
#pragma unroll
    for (int c = 0; c < 4; c++) part[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4 * kLH; u++)
      part[u % 4] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          *reinterpret_cast<const f16x8 *>(xrow + u * 32), __builtin_bit_cast(f16x8, wt[u]), part[u % 4], 0, 0, 0);
    const f32x4 acc = (part[0] + part[1]) + (part[2] + part[3]);
    const int n = j * 16 + (lane & 15);
    if (lane < 16 && n < a.n_valid) {
      gbl(a.logits)[n] = acc[0];
      const unsigned long long key = argmax_key(acc[0], n);
      best = key > best ? key : best;
    }
  };
  for (int j = first; j < nT; j += 2 * step) {
    head_load<kLH>(wb[1], a, j + step);
    tile(wb[0], j);
    head_load<kLH>(wb[0], a, j + 2 * step);
    if (j + step < nT) tile(wb[1], j + step);
  }
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off, 64);
    best = o > best ? o : best;
  }
  unsigned long long *slot =
      a.keys + (size_t)(ep & 1) * kKeySet + ((w * 4 + wave) % kKeySlots) * kKeyStride;
  if (lane == 0 && best != 0 &&
      best > __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
    atomicMax(slot, best);
  return true;
}

// The step's bookkeeping, by workgroup 0 after its last item: the step
// number, the row's length and position, the history entry, and the key set
// this step read cleared for the next step's LM head. Every workgroup with an
// item has read the epoch word, lens and (QKV items) the keys by then: it read
// them first, and its items' cells carry the step's tag, its context or its
// token, while workgroup 0's last item waited, through each layer's chain of
// exchanges, on cells that depend on every item of the step. (A workgroup
// with no item that read the words after this would wait on tags no one
// writes: its wait times out and sets err.)
__device__ __forceinline__ void finish_step(const Gpt2Args &a, unsigned ep0, int pos, int tok) {
  const int t = threadIdx.x;
  if (t < kKeySlots) gbl(a.keys)[(size_t)(ep0 & 1) * kKeySet + (size_t)t * kKeyStride] = 0ull;
  if (t == 0) {
    if (pos < a.hist_len) gbl(a.hist)[pos] = tok;
    gbl(a.pos)[0] = pos;
    gbl(a.lens)[0] = pos + 1;
    gbl(a.epoch)[0] = ep0 + 1;
  }
}

template <int kLH, int kLI>
__global__ __launch_bounds__(kT, 1) void gpt2_layers_kernel(const Gpt2Args a) {
  __shared__ Lds S;
  if (threadIdx.x < 4) S.votes.par[threadIdx.x] = 0;
  lds_barrier();
  SH_G2MARK(0, 10);
  // The step: number ep (the epoch word holds the previous one), position
  // pos = lens[0]; its token is read from the previous step's key set by the
  // workgroups with QKV items (the O items are among them), which embed it.
  // These words change only in finish_step, after every workgroup has read
  // them (see there), so atomic loads, read once: no reload can see the new
  // values.
  const unsigned ep0 = __builtin_amdgcn_readfirstlane(
      __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const unsigned ep = ep0 + 1;
  const int pos = __builtin_amdgcn_readfirstlane(
      __hip_atomic_load(a.lens, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const int L = pos + 1;  // context including this step's token
  const int G = gridDim.x, w = blockIdx.x;
  const int nA = a.qkv_n / 16, nB = a.heads * kGpt2Splits, nC = a.H / 16, nD = a.inter / 16;
  // this workgroup's QKV tile (qa) and attention item (bi), when >= 0: by
  // default the QKV tiles on workgroups 0.. and the attention items on the
  // last ones; XCD-local (a.xcd): the workgroup on XCD x (XCC_ID) with rank
  // j = w / 8 runs for head x (j < 12) and head x + 8 (12 <= j < 24) their
  // 12 QKV tiles (q, k, v: 4 each), and their splits on j = 24 .. 27 and
  // 28 .. 31, so the q / k / v cells never leave the XCD. Workgroups go to
  // the XCDs round robin from an XCD that varies between launches, so an
  // XCD holds one residue class of w mod 8 and (XCD, w / 8) names every
  // role once.
  const bool xl = a.xcd != 0;
  int qa = w < nA ? w : -1, bi = w - (G - nB);
  if (xl) {
    constexpr int kT4 = kHd / 16, kT12 = 3 * kT4;  // tiles per head: of q (k, v); of all three
    const unsigned xcc = xcc_id();
    const int x = (int)(xcc & 7), j = w >> 3;
    const int hq = j < kT12 ? x : (j < 2 * kT12 ? x + 8 : a.heads), t = j % kT12;
    qa = hq < a.heads ? (t / kT4) * a.heads * kT4 + hq * kT4 + t % kT4 : -1;
    const int jb = j - 2 * kT12, hb = jb < kGpt2Splits ? x : x + 8;
    bi = jb >= 0 && hb < a.heads ? hb * kGpt2Splits + jb % kGpt2Splits : -1;
    if (threadIdx.x == 0 && xcc >= 8) atomicOr(a.err, 2u);  // every wait then fails
  }
#ifdef SH_GPT2_TRACE
  if (threadIdx.x == 0 && w < kTrWgs) g_gpt2_trace[w][kTrLayers - 1][kTrSlots - 1] = xcc_id();
#endif
  Emb emb;
  if (qa >= 0 || w < nC || w == 0) {
    emb.tok = step_token(a.keys + (size_t)(ep0 & 1) * kKeySet, 0, a.vocab);
    emb.wte = gbl(a.head_w);
    emb.wpe_row = gbl(a.wpe) + (size_t)min(pos, a.max_pos - 1) * a.H;
  }
  const bool hasD = w >= nC && w < nC + nD;
  AttnKV kv;
  u32x4 wa[kLH];
  if (qa >= 0) load_weights<kLH>(wa, layer_p(a, 0).wqkv, a.H, qa);
  if (bi >= 0) attn_prefetch(a, layer_p(a, 0), bi, L, kv);
  for (int l = 0; l < a.n_layers; l++) {
    const LayerP P = layer_p(a, l);
    const bool next = l + 1 < a.n_layers;
    if (qa >= 0 && !qkv_item<kLH>(a, P, l, qa, ep, emb, S, wa, xl)) return;
    if (bi >= 0) {
      if (!attn_item(a, P, l, bi, ep, L, S, kv)) return;
      if (next && !hasD) attn_prefetch(a, layer_p(a, l + 1), bi, L, kv);
    }
    // Workgroups with O and proj items request the proj weights (96 KiB at
    // GPT-2 small) and the next QKV weights before the O item: nothing then
    // stands between the proj and next QKV items' polls and their data
    // (loads complete in issue order). Measured: 24 / 96 / 24 KiB before the
    // O / proj / next QKV polls (proj weights at the proj item) 5,014
    // tok/s; 120 / 24 / 0 KiB 5,173; 72 / 72 / 0 KiB 5,095.
    u32x4 wp[kLI];
    if (w < nC) {
      load_weights<kLI>(wp, P.wproj, a.inter, w);
      if (next && qa >= 0) load_weights<kLH>(wa, layer_p(a, l + 1).wqkv, a.H, qa);
    }
    if (w < nC && !o_item<kLH>(a, P, l, w, ep, L, emb, S)) return;
    if (hasD) {
      if (!fc_item<kLH>(a, P, l, w - nC, ep, S)) return;
      if (next) {
        // the fc workgroups hold their requests back ~1.25 us (wall clock,
        // 100 MHz): issued right after the item, the burst coincided with
        // the proj items' polls for the fc results. Measured, one box:
        // delays of 0.25 / 0.5 / 1 / 1.5 / 2 / 3 us: 0.1548 -> 0.1526 /
        // 0.1526 / 0.1515 / 0.1511 / 0.1530 / 0.1597 ms per step.
        const unsigned long long t0 = wall_clock64();
        while (wall_clock64() - t0 < kPrefetchDelay) __builtin_amdgcn_s_sleep(1);
        if (bi >= 0) attn_prefetch(a, layer_p(a, l + 1), bi, L, kv);
        if (qa >= 0) load_weights<kLH>(wa, layer_p(a, l + 1).wqkv, a.H, qa);
      }
    }
    if (w < nC) {
      if (!proj_item<kLH, kLI>(a, P, l, w, ep, S, wp)) return;
    }
    if (next && qa >= 0 && w >= nC + nD) load_weights<kLH>(wa, layer_p(a, l + 1).wqkv, a.H, qa);
  }
  if (a.head_on) {
    u32x4 wb[2][4 * kLH];
    head_load<kLH>(wb[0], a, w + G * (threadIdx.x >> 6));  // before the final norm's wait
    if (!head_phase<kLH>(a, ep, S, wb)) return;
    SH_G2MARK(0, 11);
  }
  if (w == 0) finish_step(a, ep0, pos, emb.tok);
}

// (loads per lane for K = hidden, K = intermediate) per supported shape
#define SH_GPT2_SHAPES(X) \
  X(6, 24) /* GPT-2 small: hidden 768, intermediate 3072 */ \
  X(2, 4)  /* hidden 256, intermediate 512 */

const void *gpt2_kernel_for(int H, int inter) {
#define SH_MATCH(LH, LI) \
  if (H == LH * 128 && inter == LI * 128) return reinterpret_cast<const void *>(&gpt2_layers_kernel<LH, LI>);
  SH_GPT2_SHAPES(SH_MATCH)
#undef SH_MATCH
  return nullptr;
}

}  // namespace

bool gpt2_layers_supported(int layers, int H, int heads, int head_dim, int inter, int max_pos,
                           int grid) {
  if (layers < 1 || layers > kMaxDecodeLayers || head_dim != kHd || heads * kHd != H) return false;
  if (!gpt2_kernel_for(H, inter)) return false;
  if (max_pos < 1 || gpt2_layers_chunk(max_pos) > kMaxChunk) return false;
  // at most one item per workgroup and phase; the attention items on the
  // last workgroups
  const int nA = 3 * H / 16, nB = heads * kGpt2Splits, nC = H / 16, nD = inter / 16;
  return nA <= grid && nB <= grid && nC + nD <= grid;
}

int gpt2_layers_chunk(int max_pos) {
  return ((max_pos + kGpt2Splits - 1) / kGpt2Splits + 15) / 16 * 16;
}

bool gpt2_layers_xcd_ok(const Gpt2Args &a, int grid) {
  // 2 heads per XCD at most, each with 12 QKV tiles and kGpt2Splits splits
  return grid % 8 == 0 && a.heads <= 16 && a.qkv_n == 3 * a.heads * kHd && a.H == a.heads * kHd &&
         2 * (3 * kHd / 16 + kGpt2Splits) <= grid / 8 && a.qkv_n / 16 <= grid &&
         a.heads * kGpt2Splits <= grid;
}

size_t gpt2_layers_partial_cells(int heads) { return (size_t)heads * kGpt2Splits * kGpt2PStride; }

hipError_t gpt2_layers_occupancy(const Gpt2Args &a, int *blocks_per_cu) {
  const void *k = gpt2_kernel_for(a.H, a.inter);
  if (!k) return hipErrorInvalidValue;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k, kT, 0);
}

#ifdef SH_GPT2_TRACE
hipError_t gpt2_layers_trace(void *dst, size_t bytes) {
  if (bytes > sizeof(g_gpt2_trace)) bytes = sizeof(g_gpt2_trace);
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_gpt2_trace), bytes, 0, hipMemcpyDeviceToHost);
}
#endif

hipError_t launch_gpt2_layers(hipStream_t s, const Gpt2Args &a, int grid) {
  const void *k = gpt2_kernel_for(a.H, a.inter);
  if (!k) return hipErrorInvalidValue;
  void *args[] = {const_cast<Gpt2Args *>(&a)};
  return hipLaunchKernel(k, dim3(grid), dim3(kT), args, 0, s);
}

}  // namespace sh
