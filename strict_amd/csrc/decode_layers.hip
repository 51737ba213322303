// Persistent decode-layers kernel: all decoder layers of one Qwen3 decode
// step (FP8 weights, head_dim 128) in one launch, one workgroup per CU, all
// resident together. It replaces the six kernels per layer of the per-op path (norm +
// QKV GEMV, attention, split merge, O GEMV, norm + gate/up GEMV, down GEMV).
//
// Work per layer, as items spread over the workgroups:
//   A  QKV     one 16-row tile of W_qkv each      (RMSNorm of x in every item)
//   B  attn    one (row, KV head, split) each      (q/k norm, RoPE, cache append)
//   M  merge   one (row, query head, dim quarter) (combines the split partials)
//   C  O       one 16-row tile of W_o each         (x_mid = x + W_o attn)
//   D  gate/up one gate tile + up tile pair each   (RMSNorm of x_mid, SwiGLU)
//   E  down    one 16-row tile of W_down each      (x = x_mid + W_down act)
// and, on steps with logits, after the last layer:
//   H  head    16-row tiles of the LM head          (final RMSNorm, logits, argmax)
//
// Exchange between workgroups: every value an item hands on travels in an
// 8-byte cell of device memory, payload in the low word and the
// producing (step, layer) tag in the high word, written by one 8-byte (or
// 16-byte, two-cell) store. A consumer loads the cells it needs until each
// carries the tag it expects. The data is its own completion flag: a
// producer never waits for its stores to complete, and a consumer needs one
// memory round trip once the data has landed (a flag word would cost the
// producer's store-completion wait, the flag poll and then the data read).
// Every cell load is a relaxed 64-bit agent-scope atomic, and so is every
// cell store except the XCD-local ones (cst1): the memory model keeps those
// coherent across the XCDs' separate L2 caches (measured here: ~0.35-0.45
// us from a store to another XCD's poll seeing it, against ~0.55-0.63 us
// through uncached memory), and the compiler neither hoists such a load out
// of a spin loop nor waits after each one. The XCD-local stores (workgroup
// scope) stay in the producer's XCD L2, where the polls of that XCD's CUs
// find them sooner.
//
// Weights and K / V do not depend on the step's activations, so each
// workgroup requests them for its next items right after it has finished
// polling for the current one (the loads then arrive while the previous
// phase's producers run). Loads complete in issue order, so a poll issued
// after a bulk request returns no earlier than that request: requests are
// placed where the workgroup's next poll is at least one exchange away.
//
// Every wait is bounded by a wall-clock limit; a timeout sets the sticky
// error word, after which every other wait fails at once, so the grid always
// drains. Items of C and E sit on workgroups 0.., those of D after them and
// the merge items on the last workgroups.
//
// Rounding: this file is compiled without floating-point contraction
// (-ffp-contract=off) and writes each fused multiply-add it wants as fmaf, so
// every instantiation (batch 1, small batch, large batch) rounds the same
// way and a row of a batched step equals its batch-1 step bit for bit.
//
// With one wave per SIMD nothing hides an instruction's latency, so the item
// code avoids runtime integer division, LDS-based lane shuffles in its
// reductions (DPP within 16-lane rows instead) and single-wave serial loops.
#include <type_traits>
#include <hip/hip_runtime.h>

#include "common.h"
#include "exchange.h"
#include "llm.h"
#include "llm_device.h"

namespace sh {
namespace {

constexpr int kT = 256;         // threads per workgroup (4 waves)
constexpr int kD = 128;         // head dim
constexpr int kMaxSplits = 64;  // splits per (row, KV head) a merge item combines
// batch rows staged together (each pass is one round of cell polls): 1 at
// batch 1, 4 up to batch 4, 8 above
constexpr int kMaxRowsPerPass = 8;
// Wall-clock ticks (100 MHz) the batch-1 gate/up-only workgroups wait before
// requesting the next layer's K / V and QKV weights (see the layer loop).
constexpr unsigned long long kPrefetchDelay = 35;
constexpr int kSmallBatchRows = 4;

// Pointers the kernel reads from its argument table (LayerPtrs) are generic;
// loads through them compile to flat instructions, which also count against
// the LDS wait counter, so every LDS wait would wait for outstanding weight
// and K / V requests too. The kernel casts them to the global address space.
#define SH_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ SH_GLOBAL T *gbl(T *p) {
  return (SH_GLOBAL T *)p;
}

// Tables that the host or an earlier kernel of the step writes and this
// kernel only reads (the layer pointer table, the rows' positions, the
// step's epoch) are read through the constant address space: uniform reads
// of it become scalar loads, which complete on their own counter. Read as
// global memory they were vector loads, queued behind every weight and K / V
// request outstanding, and each layer's first use of a layer pointer waited
// for all of them.
#define SH_CONST __attribute__((address_space(4)))
template <class T>
__device__ __forceinline__ const SH_CONST T *cnst(const T *p) {
  return (const SH_CONST T *)p;
}

// One layer's pointers in the global address space.
struct LayerG {
  const SH_GLOBAL uint8_t *wqkv, *wo, *wup, *wdown;
  const SH_GLOBAL float *sqkv, *so, *sup, *sdown;
  const SH_GLOBAL float *norm1, *norm2, *q_norm, *k_norm;
  SH_GLOBAL uint16_t *kcache, *vcache;
};

// Layer l's pointers, read from the table with scalar loads.
__device__ __forceinline__ LayerG layer_g(const LayersArgs &a, int l) {
  const SH_CONST LayerPtrs &p = cnst(a.layers)[l];
  return LayerG{gbl(p.wqkv),   gbl(p.wo),     gbl(p.wup),    gbl(p.wdown), gbl(p.sqkv),
                gbl(p.so),     gbl(p.sup),    gbl(p.sdown),  gbl(p.norm1), gbl(p.norm2),
                gbl(p.q_norm), gbl(p.k_norm), gbl(p.kcache), gbl(p.vcache)};
}

// ---- exchange cells ------------------------------------------------------------

// Tag of the values layer l of step `epoch` produces (epoch >= 1, l < 63, so
// never 0, the value of never-written cells).
__device__ __forceinline__ unsigned tag_of(unsigned epoch, int l) {
  return epoch * 64u + (unsigned)l + 1u;
}

__device__ __forceinline__ uint64_t cld(const uint64_t *base, size_t cell) {
  return __hip_atomic_load(base + cell, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned ld_err(const unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cell stores are relaxed agent-scope atomics (global stores with the
// device-scope cache policy): once complete they are visible to every CU.
// `local`: a workgroup-scope store instead, which lands in the XCD's L2 and
// stays there; the agent-scope polls of the same XCD's CUs see it (one hop
// ~0.22 us against ~0.4-0.53 us measured in a ping-pong between workgroups),
// those of other XCDs do not until the kernel ends. Only for cells whose
// every consumer runs on the producer's XCD.
__device__ __forceinline__ void cst1(uint64_t *base, size_t cell, uint32_t v, unsigned tag,
                                     bool local = false) {
  const uint64_t c = (uint64_t)v | ((uint64_t)tag << 32);
  if (local)
    __hip_atomic_store(base + cell, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else
    __hip_atomic_store(base + cell, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void cst2(uint64_t *base, size_t cell, uint32_t v0, uint32_t v1,
                                     unsigned tag, bool local = false) {
  cst1(base, cell, v0, tag, local);
  cst1(base, cell + 1, v1, tag, local);
}

// The XCD this wave runs on (hardware register XCC_ID).
__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xf;
}

__device__ __forceinline__ float f32_of(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t bits_of(float f) { return __builtin_bit_cast(uint32_t, f); }

// Loads the cells base[at(k)], k < kN, until each one with bit k of mask
// set carries `tag`; c[k] receives them (payload in the low word). at(k)
// must name a valid cell for every k (callers clamp the unused ones onto
// used cells, so the loads need no branches). False when the wait exceeded
// the limit or another wait has failed.
template <int kN, class At>
__device__ __forceinline__ bool spin_cells(const LayersArgs &a, const uint64_t *base, At at,
                                           uint64_t mask, unsigned tag, uint64_t (&c)[kN]) {
  unsigned long long t0 = 0;
  for (int it = 0;; it++) {
#pragma unroll
    for (int k = 0; k < kN; k++) c[k] = cld(base, at(k));
    bool ok = true;
#pragma unroll
    for (int k = 0; k < kN; k++) ok = ok && ((mask >> k & 1) == 0 || (uint32_t)(c[k] >> 32) == tag);
    if (ok) return true;
    if (it == 0) {
      t0 = wall_clock64();
    } else if ((it & 7) == 0 && (ld_err(a.err) != 0 || wall_clock64() - t0 > a.spin_ticks)) {
      return false;
    }
#if defined(SH_POLL_SLEEP) && SH_POLL_SLEEP > 0
    __builtin_amdgcn_s_sleep(SH_POLL_SLEEP);
#endif
  }
}

// spin_cells over cells taken two at a time (one 16-byte load each, with
// the agent-scope cache policy of cld): at(k) for even k must be even, and
// cell k + 1 is at(k) + 1 (at is called for even k only). Polls of adjacent
// cells this way send half the line requests to memory.
template <int kN, class At>
__device__ __forceinline__ bool spin_pairs(const LayersArgs &a, const uint64_t *base, At at,
                                           uint64_t mask, unsigned tag, uint64_t (&c)[kN]) {
  static_assert(kN % 2 == 0, "pairs of cells");
  const __amdgpu_buffer_rsrc_t rs = xchg::cell_rsrc(base);
  unsigned long long t0 = 0;
  for (int it = 0;; it++) {
    // compiler barriers: a new load each round, every load issued before
    // the checks (ordinary loads are otherwise moved into the branches of
    // the checks, one round trip after another)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int k = 0; k < kN; k += 2) xchg::cld2(rs, at(k), c[k], c[k + 1]);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    bool ok = true;
#pragma unroll
    for (int k = 0; k < kN; k++) ok &= ((mask >> k & 1) == 0) | ((uint32_t)(c[k] >> 32) == tag);
    if (ok) return true;
    if (it == 0) {
      t0 = wall_clock64();
    } else if ((it & 7) == 0 && (ld_err(a.err) != 0 || wall_clock64() - t0 > a.spin_ticks)) {
      return false;
    }
  }
}

__device__ __forceinline__ float cell_f32(uint64_t c) { return __builtin_bit_cast(float, (uint32_t)c); }

// One cell already requested as `c`: polls it again until it carries `tag`.
__device__ __forceinline__ bool finish_cell(const LayersArgs &a, const uint64_t *base, size_t cell,
                                            unsigned tag, uint64_t &c) {
  unsigned long long t0 = 0;
  for (int it = 0; (uint32_t)(c >> 32) != tag; it++) {
    if (it == 0) {
      t0 = wall_clock64();
    } else if ((it & 7) == 0 && (ld_err(a.err) != 0 || wall_clock64() - t0 > a.spin_ticks)) {
      return false;
    }
    c = cld(base, cell);
  }
  return true;
}

#ifdef SH_DECODE_TRACE
constexpr int kTraceWgs = 256, kTraceLayers = 32, kTraceSlots = 24;
#endif

// Small LDS words after the phase areas.
struct Misc {
  float part[4][kSmallBatchRows];  // per-wave partial sums of squares, rows 0..3 of a pass
  int vote[2][4];                  // per-wave votes of block_any (two alternating sets)
  int par[4];                      // each wave's current vote set
  float part_hi[4][kMaxRowsPerPass - kSmallBatchRows];  // rows 4.. of a pass
  float inv[kMaxBatch];  // post-scaled staging, batched variants: each row's RMSNorm scale
#ifdef SH_DECODE_TRACE
  unsigned long long t_wait;                          // when the last wait ended
  unsigned long long tr[2][kTraceLayers][kTraceSlots];  // this workgroup's timeline
#endif
};

// Workgroup barrier for LDS traffic only. __syncthreads() is a release /
// acquire fence plus s_barrier, and the fence makes a wave wait for every
// global store it has issued (cell stores, cache appends) before the
// barrier; nothing in this kernel reads back through global memory what
// another wave of its workgroup wrote, so only LDS needs to be complete.
// The signal fences keep the compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left alone
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// True in every thread when p holds in any thread (a barrier). Each wave
// votes in one of two sets, alternating per call (its parity lives in its
// own LDS word): a wave that runs ahead to the next call writes the other
// set, and one two calls ahead has passed a barrier that every wave reaches
// only after reading this call's votes.
__device__ __forceinline__ bool block_any(bool p, Misc *misc) {
  const int wave = threadIdx.x >> 6;
  const int par = misc->par[wave];
  const bool v = __any(p ? 1 : 0) != 0;
  if ((threadIdx.x & 63) == 0) {
    misc->vote[par][wave] = v ? 1 : 0;
    misc->par[wave] = par ^ 1;
  }
  lds_barrier();
  const int *vt = misc->vote[par];
  return (vt[0] | vt[1] | vt[2] | vt[3]) != 0;
}

// block_any in two halves around a barrier that the caller places (a
// wait's outcome can then share the barrier of values exchanged anyway):
// vote_cast before the barrier, vote_seen with its result after it.
__device__ __forceinline__ int vote_cast(bool p, Misc *misc) {
  const int wave = threadIdx.x >> 6;
  const int par = misc->par[wave];
  const bool v = __any(p ? 1 : 0) != 0;
  if ((threadIdx.x & 63) == 0) {
    misc->vote[par][wave] = v ? 1 : 0;
    misc->par[wave] = par ^ 1;
  }
  return par;
}
__device__ __forceinline__ bool vote_seen(int par, const Misc *misc) {
  const int *vt = misc->vote[par];
  return (vt[0] | vt[1] | vt[2] | vt[3]) != 0;
}

// After a vote on failed waits (block-uniform `failed`): marks the error
// and returns false if any wait failed.
__device__ __forceinline__ bool waits_done(const LayersArgs &a, bool failed, Misc *misc) {
  if (failed) {
    if (threadIdx.x == 0) atomicOr(a.err, 1u);
    return false;
  }
#ifdef SH_DECODE_TRACE
  if (threadIdx.x == 0) misc->t_wait = wall_clock64();
#endif
  return true;
}

// Marks the error when a wait of this wave failed (no vote: the caller goes
// on either way).
__device__ __forceinline__ void wave_waits_ok(const LayersArgs &a, bool ok, Misc *misc) {
  if (__any(ok ? 0 : 1) && (threadIdx.x & 63) == 0) atomicOr(a.err, 1u);
#ifdef SH_DECODE_TRACE
  if (threadIdx.x == 0) misc->t_wait = wall_clock64();
#endif
}

// Every thread's wait succeeded (block-uniform); otherwise marks the error.
__device__ __forceinline__ bool waits_ok(const LayersArgs &a, bool ok, Misc *misc) {
  if (block_any(!ok, misc)) {
    if (threadIdx.x == 0) atomicOr(a.err, 1u);
    return false;
  }
#ifdef SH_DECODE_TRACE
  if (threadIdx.x == 0) misc->t_wait = wall_clock64();
#endif
  return true;
}

#ifdef SH_DECODE_TRACE
// Timeline of one step (diagnostic builds only), kept in LDS during the step
// and written out when the kernel ends: per workgroup and layer, tr[0] holds
// each phase's start (even slots 0..8: QKV, attention, O, gate/up, down),
// end (odd slots), the end of its wait (10..14), the merge end (15) and the
// ends of the workgroup's first eight attention items (16..23); tr[1]
// holds marks inside items: QKV 0..3 (staged, MFMA, reduced, stored), down
// 4..7, attention 8..13 (q/k/v polled, RoPE, scores, softmax, V sums,
// stored), merge 14..15 (polled, stored), and the end of each phase's items
// on this workgroup (all of them, not only the first): 16 QKV, 17
// attention, 18 merge, 19 O, 20 gate/up, 21 down; 22 an attention item's
// start (with 8..13, the workgroup's last item's); at layer n_layers, 0 the
// end of the LM head's final-RMSNorm wait and 1 the workgroup's end.
__device__ unsigned long long g_decode_trace[2][kTraceWgs][kTraceLayers][kTraceSlots];
__device__ __forceinline__ void trace_mark(Misc *misc, int set, int l, int slot) {
  if (threadIdx.x == 0 && l < kTraceLayers) misc->tr[set][l][slot] = wall_clock64();
}
#define SH_MARK(misc, l, slot) trace_mark(misc, 1, l, slot)
#define SH_TRACE(misc, l, slot) trace_mark(misc, 0, l, slot)
#define SH_TRACE_WAIT(l, ph, misc)                                                 \
  do {                                                                             \
    if (threadIdx.x == 0 && (l) < kTraceLayers) (misc)->tr[0][l][10 + (ph)] = (misc)->t_wait; \
  } while (0)
#else
#define SH_TRACE(misc, l, slot) ((void)0)
#define SH_MARK(misc, l, slot) ((void)0)
#define SH_TRACE_WAIT(l, ph, misc) ((void)0)
#endif

// ---- GEMV items ----------------------------------------------------------------

// This wave's quarter of K for tile group g (kNT consecutive 16-row tiles of
// an FP8 tiled matrix with K columns): kL 16-byte loads per lane and tile.
template <int kL, int kNT>
__device__ __forceinline__ void load_weights(u32x4 (&w)[kL][kNT], const SH_GLOBAL uint8_t *W, int K, int g) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = K >> 6;
#pragma unroll
  for (int u = 0; u < kL; u++)
#pragma unroll
    for (int j = 0; j < kNT; j++) {
      const size_t tile = (size_t)(g * kNT + j) * lpr + wave * kL + u;
      w[u][j] = __builtin_nontemporal_load(
          reinterpret_cast<const SH_GLOBAL u32x4 *>(W + tile * 1024 + (size_t)lane * 16));
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
  // independent accumulator chains (MFMA k-step s on chain s % kCh), so
  // consecutive MFMAs do not wait for each other's results
  constexpr int kCh = kNT == 1 ? 4 : 2;
  f32x4 part[kCh][kNT];
#pragma unroll
  for (int c = 0; c < kCh; c++)
#pragma unroll
    for (int j = 0; j < kNT; j++) part[c][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // activation fragments are read kG4 k-steps at a time, all before their
  // MFMAs, so the LDS latency is paid once per group rather than per step
  constexpr int kG4 = kL < 4 ? kL : 4;
  static_assert(kL % kG4 == 0, "k-step groups");
  const _Float16 *xrow = xs + row * stride + wave * kL * 64 + acol;
#pragma unroll
  for (int u0 = 0; u0 < kL; u0 += kG4) {
    f16x8 af[kG4][2];
#pragma unroll
    for (int v = 0; v < kG4; v++)
#pragma unroll
      for (int h = 0; h < 2; h++)
        af[v][h] = *reinterpret_cast<const f16x8 *>(xrow + (u0 + v) * 64 + 32 * h);
#pragma unroll
    for (int v = 0; v < kG4; v++) {
      const int u = u0 + v;
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int j = 0; j < kNT; j++)
          part[(2 * u + h) % kCh][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              af[v][h], e4m3x8_to_f16(w[u][j][2 * h], w[u][j][2 * h + 1]), part[(2 * u + h) % kCh][j],
              0, 0, 0);
    }
  }
#pragma unroll
  for (int j = 0; j < kNT; j++) {
    f32x4 sum = part[0][j];
#pragma unroll
    for (int c = 1; c < kCh; c++) sum += part[c][j];
    acc[j] = sum;
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
  lds_barrier();
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

// The 4-value chunks of a K-value row a thread stages: wave w holds the
// chunks of its K quarter, [w K / 16, (w + 1) K / 16), lane l the chunks
// w K / 16 + l + 64 j. That is the quarter of xs the wave's MFMAs read
// (mfma_weights), so a GEMV item needs no workgroup barrier between staging
// and its MFMAs: a wave's LDS reads follow its own writes in order.
__device__ __forceinline__ int stage_chunk(int K, int j) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  return wave * (K >> 4) + lane + 64 * j;
}
__device__ __forceinline__ bool stage_chunk_ok(int K, int j) {
  return (threadIdx.x & 63) + 64 * j < (K >> 4);
}

// The first layer's input of a batch-1 step that embeds its own token
// (LayersArgs::fold): row `tok` of the tied FP8 head times its scale, each
// value converted as the embed kernel converts it (E4M3 -> fp16 -> fp32,
// then the scale).
struct EmbQ {
  int tok = -1;  // < 0: the input comes from x_in (the embed kernel's) or cells
  const SH_GLOBAL uint8_t *head8 = nullptr;
  float scale = 0.0f;
};

__device__ __forceinline__ float embq1(const EmbQ &e, int k, int K) {
  const uint8_t q = e.head8[fp8_tiled_offset(e.tok, k, K)];
  return (float)__builtin_amdgcn_cvt_scalef32_pk_f16_fp8((uint32_t)q, 1.0f, false)[0] * e.scale;
}

// The 2-value pairs of a K-value row stage_rms stages: wave w holds the
// pairs of its K quarter, [w K / 8, (w + 1) K / 8), lane l the pairs
// w K / 8 + l + 64 i, i < kP (kP >= K / 512). As with stage_chunk, that is
// the quarter of xs the wave's MFMAs read. A pair is two adjacent cells, so
// a wave's poll of its pairs i is one lane-contiguous 16-byte load, which
// reaches memory as the fewest line requests (measured over 1,024 cells, 64
// producer x 192 consumer workgroups: 1.46 us per exchange, against 1.59 us
// with two 16-byte loads of four adjacent cells per lane).
__device__ __forceinline__ int stage_pair(int K, int i) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  return wave * (K >> 3) + lane + 64 * i;
}
__device__ __forceinline__ bool stage_pair_ok(int K, int i) {
  return (threadIdx.x & 63) + 64 * i < (K >> 3);
}

// Values k, k + 1 of the embedded token (k even: two contiguous bytes of the tile).
__device__ __forceinline__ f32x2 embq2(const EmbQ &e, int k, int K) {
  const uint32_t q = *reinterpret_cast<const SH_GLOBAL uint16_t *>(e.head8 + fp8_tiled_offset(e.tok, k, K));
  const f16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q, 1.0f, false);
  return f32x2{(float)lo[0] * e.scale, (float)lo[1] * e.scale};
}

// Rows [B][K] of fp32 x -> RMSNorm with gains g -> xs (fp16, row stride
// K + 8), kRows rows per pass. kPost: xs holds x * g only, and the items
// apply each row's scale 1 / rms to their GEMV results (row_inv); at batch
// 1 the staging then needs no barrier (each wave reads only its own K
// quarter of xs, and the sums of squares are read after the item's
// cross-wave reduction). The rows come from cells xc tagged `tag` or,
// for the first layer, from the plain buffer xp the embedding kernel wrote
// before this launch or (batch 1, e.tok >= 0) from the embedding table. Each
// thread keeps its 2-value pairs (stage_pair, 2 kChunks of them) in
// registers; the per-row sums of squares are combined across the four waves
// through LDS. kChunks >= K / 1024. kLocal: the caller's waves read only
// their own K quarter of xs, so no barrier follows the stores.
template <int kChunks, int kRowsMax, bool kLocal, bool kPost = false>
__device__ __forceinline__ bool stage_rms(const LayersArgs &a, const uint64_t *xc, const float *xp, unsigned tag,
                          const SH_GLOBAL float *g, int K, _Float16 *xs, Misc *misc,
                          const EmbQ &e = EmbQ{}) {
  constexpr int kP = 2 * kChunks;  // pairs per thread and row
  // rows per pass: at most kRowsMax, and at most 64 cells per thread
  constexpr int kRows = kRowsMax * kP * 2 <= 64 ? kRowsMax : 64 / (kP * 2);
  constexpr int kN = kRows * kP * 2;
  static_assert(kN <= 64, "cells per thread");
  const int B = kRows == 1 ? 1 : a.B, c2 = K >> 1, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  f32x2 gv[kP];
#pragma unroll
  for (int i = 0; i < kP; i++)
    gv[i] = *reinterpret_cast<const SH_GLOBAL f32x2 *>(g + min(stage_pair(K, i), c2 - 1) * 2);
  for (int b0 = 0; b0 < B; b0 += kRows) {
    f32x2 v[kRows][kP];
    bool ok = true;
    if (kRowsMax == 1 && e.tok >= 0) {
#pragma unroll
      for (int i = 0; i < kP; i++) v[0][i] = embq2(e, min(stage_pair(K, i), c2 - 1) * 2, K);
    } else if (xp) {
#pragma unroll
      for (int r = 0; r < kRows; r++)
#pragma unroll
        for (int i = 0; i < kP; i++) {
          const int c = min(stage_pair(K, i), c2 - 1), b = min(b0 + r, B - 1);
          v[r][i] = *reinterpret_cast<const f32x2 *>(xp + (size_t)b * K + c * 2);
        }
    } else {
      // cells of pair (r, i): row b0 + r, values 2 c, 2 c + 1, c =
      // stage_pair(K, i) (rows past B and pairs past the wave's quarter
      // re-read valid ones)
      uint64_t cv[kN];
      uint64_t mask = 0;
#pragma unroll
      for (int r = 0; r < kRows; r++)
#pragma unroll
        for (int i = 0; i < kP; i++)
          if (b0 + r < B && stage_pair_ok(K, i)) mask |= 3ull << ((r * kP + i) * 2);
      ok = spin_pairs(a, xc,
                      [&](int k) {
                        const int r = k / (kP * 2), i = (k / 2) % kP, e = k % 2;
                        return (size_t)min(b0 + r, B - 1) * K + min(stage_pair(K, i), c2 - 1) * 2 + e;
                      },
                      mask, tag, cv);
#pragma unroll
      for (int r = 0; r < kRows; r++)
#pragma unroll
        for (int i = 0; i < kP; i++) {
          const int k = (r * kP + i) * 2;
          v[r][i] = f32x2{cell_f32(cv[k]), cell_f32(cv[k + 1])};
        }
    }
    // at batch 1 the waits' vote shares the barrier of the sums of squares
    // (the batched variants vote first: their kernels measured ~1 % slower
    // with the shared barrier)
    // (post-scaled at batch 1: no vote and no barrier, see wave_waits_ok)
    constexpr bool kFree = kPost && kRowsMax == 1;
    int vpar = 0;
    if constexpr (kFree) {
      wave_waits_ok(a, ok, misc);
    } else if constexpr (kRowsMax == 1) {
      vpar = vote_cast(!ok, misc);
    } else {
      if (!waits_ok(a, ok, misc)) return false;
    }
#pragma unroll
    for (int r = 0; r < kRows; r++) {
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < kP; i += 2) {
        const float s0 = stage_pair_ok(K, i) ? fmaf(v[r][i][0], v[r][i][0], v[r][i][1] * v[r][i][1]) : 0.0f;
        const float s1 =
            stage_pair_ok(K, i + 1) ? fmaf(v[r][i + 1][0], v[r][i + 1][0], v[r][i + 1][1] * v[r][i + 1][1]) : 0.0f;
        ss += s0 + s1;
      }
      ss = wave_sum_rows(ss);
      if (lane == 0) {
        if (r < kSmallBatchRows) misc->part[wave][r] = ss;
        else misc->part_hi[wave][r - kSmallBatchRows] = ss;
      }
    }
    if constexpr (!kFree) {
      lds_barrier();
      if constexpr (kRowsMax == 1) {
        if (!waits_done(a, vote_seen(vpar, misc), misc)) return false;
      }
    }
#pragma unroll
    for (int r = 0; r < kRows; r++) {
      const int b = b0 + r;
      if (b >= B) break;
      float inv = 1.0f;
      if constexpr (!kFree) {
        const float(&pr)[4][kSmallBatchRows] = *reinterpret_cast<const float(*)[4][kSmallBatchRows]>(
            r < kSmallBatchRows ? &misc->part[0][r] : &misc->part_hi[0][r - kSmallBatchRows]);
        const float ss = (pr[0][0] + pr[1][0]) + (pr[2][0] + pr[3][0]);
        inv = 1.0f / sqrtf(ss / (float)K + a.eps);
        if (kPost && threadIdx.x == 0) misc->inv[b] = inv;
      }
#pragma unroll
      for (int i = 0; i < kP; i++) {
        const int c = stage_pair(K, i);
        if (stage_pair_ok(K, i)) {
          const f32x2 y = kPost ? v[r][i] * gv[i] : v[r][i] * inv * gv[i];
          *reinterpret_cast<f16x2 *>(xs + b * (K + 8) + c * 2) = f16x2{(_Float16)y[0], (_Float16)y[1]};
        }
      }
    }
    // the next pass's sums reuse misc->part; with kLocal, the MFMAs read
    // only this wave's stores
    if (!kLocal || b0 + kRows < B) lds_barrier();
  }
  return true;
}

// Rows [B][K] of fp16 values packed two per cell (K / 2 cells per row,
// tagged `tag`) -> xs (row stride K + 8), kRows rows per pass. A thread
// stages the two-cell chunks stage_chunk(K, j), j < kChunks (kChunks >=
// K / 1024). kLocal as for stage_rms.
template <int kChunks, int kRowsMax, bool kLocal>
__device__ __forceinline__ bool stage_f16(const LayersArgs &a, const uint64_t *cells, unsigned tag, int K,
                          _Float16 *xs, Misc *misc) {
  // rows per pass: at most kRowsMax, and at most 64 cells per thread
  constexpr int kRows = kRowsMax * kChunks * 2 <= 64 ? kRowsMax : 64 / (kChunks * 2);
  constexpr int kN = kRows * kChunks * 2;
  static_assert(kN <= 64, "cells per thread");
  const int B = kRows == 1 ? 1 : a.B, c4 = K >> 2, row_cells = K >> 1;
  for (int b0 = 0; b0 < B; b0 += kRows) {
    // cells of chunk (r, j): row b0 + r, cells 2 c, 2 c + 1, c = stage_chunk(K, j)
    uint64_t cv[kN];
    uint64_t mask = 0;
#pragma unroll
    for (int r = 0; r < kRows; r++)
#pragma unroll
      for (int j = 0; j < kChunks; j++)
        if (b0 + r < B && stage_chunk_ok(K, j)) mask |= 3ull << ((r * kChunks + j) * 2);
    const bool ok = spin_pairs(a, cells,
                               [&](int k) {
                                 const int r = k / (kChunks * 2), j = (k / 2) % kChunks, e = k % 2;
                                 return (size_t)min(b0 + r, B - 1) * row_cells +
                                        min(stage_chunk(K, j), c4 - 1) * 2 + e;
                               },
                               mask, tag, cv);
    if constexpr (kLocal) {
      // No vote, so no barrier: each wave stages and then reads only its
      // own quarter of xs (every pass's rows), and the item's next barrier
      // (the cross-wave sum) follows its MFMAs. A wave whose wait failed
      // marks the error and goes on with what it loaded, so every wave
      // reaches that barrier, and the host reports the step as failed.
      wave_waits_ok(a, ok, misc);
    } else if (!waits_ok(a, ok, misc)) {
      return false;
    }
#pragma unroll
    for (int r = 0; r < kRows; r++)
#pragma unroll
      for (int j = 0; j < kChunks; j++) {
        const int b = b0 + r, c = stage_chunk(K, j), k = (r * kChunks + j) * 2;
        if (b < B && stage_chunk_ok(K, j))
          *reinterpret_cast<u32x2 *>(xs + b * (K + 8) + c * 4) = u32x2{(uint32_t)cv[k], (uint32_t)cv[k + 1]};
      }
  }
  if (!kLocal) lds_barrier();
  return true;
}

struct Lds {
  _Float16 *xs;
  float *red;
  Misc *misc;
};

// Rows per lane group of an MFMA output (acc[r] is row 4 (lane / 16) + r):
// the batch-1 variants (kRows == 1, chosen only for B == 1) only ever have
// row 0, and their staging and MFMA code takes B as the constant 1.
template <int kRows>
constexpr int kOutRows = kRows == 1 ? 1 : 4;

// Requests x[b][col] of the four batch rows b = 4 (lane / 16) + r this
// lane's accumulator holds (used in wave 0): the cells (checked by
// finish_residual), and for the first layer's O item the plain input xp.
// Every thread loads its cells, without a branch: a load under a branch
// made the compiler wait for all outstanding requests (the item's weights)
// before the poll that follows.
template <int kR>
__device__ __forceinline__ void request_residual(const LayersArgs &a, const uint64_t *xc,
                                                 const float *xp, int col, float (&rv)[4],
                                                 uint64_t (&rc)[4], const EmbQ &e = EmbQ{}) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int b = min(4 * (lane >> 4) + r, a.B - 1);
    rc[r] = r < kR ? cld(xc, (size_t)b * a.H + col) : 0ull;  // rows past kR: unused
    rv[r] = 0.0f;
  }
  if (kR == 1 && e.tok >= 0) {
    rv[0] = embq1(e, col, a.H);
  } else if (xp) {
#pragma unroll
    for (int r = 0; r < kR; r++) {
      const int b = min(4 * (lane >> 4) + r, a.B - 1);
      rv[r] = gbl(xp)[(size_t)b * a.H + col];
    }
  }
}

// The residual cells of request_residual carry `tag` (they were produced a
// phase before the current inputs, so this normally returns at once).
template <int kR>
__device__ __forceinline__ bool finish_residual(const LayersArgs &a, const uint64_t *xc, int col,
                                                unsigned tag, float (&rv)[4], uint64_t (&rc)[4]) {
  const int lane = threadIdx.x & 63;
  bool ok = true;
#pragma unroll
  for (int r = 0; r < kR; r++) {
    const int b = min(4 * (lane >> 4) + r, a.B - 1);
    ok = ok && finish_cell(a, xc, (size_t)b * a.H + col, tag, rc[r]);
    rv[r] = f32_of((uint32_t)rc[r]);
  }
  if (!ok) atomicOr(a.err, 1u);  // consumers of this item then fail their waits
  return ok;
}

// Marks loaded cells as used. A load whose result no path consumes leaves
// its destination registers pending at the join, and the compiler then
// waits for every outstanding request (the next layer's K / V) before the
// registers' next write.
__device__ __forceinline__ void consume_cells(const uint64_t (&c)[4]) {
  asm volatile("" ::"v"(c[0]), "v"(c[1]), "v"(c[2]), "v"(c[3]));
}

// A: qkv[b][16 i + c] = scale * (W_qkv RMSNorm(x)); w holds the item's
// weights (load_weights, issued by the caller); local: every consumer of the
// cells runs on this XCD (cst1)
// The RMSNorm scale of row b of a post-scaled staging (stage_rms kPost),
// for the items' results: at batch 1 from the four waves' sums of squares
// (read after the item's cross-wave reduction), in the batched variants as
// the staging stored it. The same expression as stage_rms's own.
template <int kRows>
__device__ __forceinline__ float row_inv(const LayersArgs &a, const Misc *misc, int b) {
  if constexpr (kRows == 1) {
    const float ss = (misc->part[0][0] + misc->part[1][0]) + (misc->part[2][0] + misc->part[3][0]);
    return 1.0f / sqrtf(ss / (float)a.H + a.eps);
  } else {
    return misc->inv[b];
  }
}

template <int kL, int kRows>
__device__ __forceinline__ bool qkv_item(const LayersArgs &a, const LayerG &P, int l, int i, unsigned ep,
                         const Lds &s, const u32x4 (&w)[kL][1], bool reuse, bool local,
                         const EmbQ &e) {
  const int lane = threadIdx.x & 63, col = lane & 15;
  const float sc = P.sqkv[i * 16 + col];
  __builtin_amdgcn_sched_barrier(0);
  // reuse: the workgroup's previous item staged this layer's rows already
  // (each wave reads only its own K quarter of them); the barrier keeps
  // this item's reduction writes behind the previous one's reads
  if (reuse)
    lds_barrier();
  else if (!stage_rms<(kL + 3) / 4, kRows, true, true>(a, a.x0c, l == 0 ? a.x_in : nullptr, tag_of(ep, l - 1),
                                                 P.norm1, a.H, s.xs, s.misc, l == 0 ? e : EmbQ{}))
    return false;
  SH_MARK(s.misc, l, 0);
  f32x4 acc[1];
  mfma_weights<kL, 1>(w, s.xs, a.H + 8, kRows == 1 ? 1 : a.B, acc);
  SH_MARK(s.misc, l, 1);
  reduce_waves<1>(acc, s.red);
  SH_MARK(s.misc, l, 2);
  if (threadIdx.x < 64) {
    const unsigned tag = tag_of(ep, l);
#pragma unroll
    for (int r = 0; r < kOutRows<kRows>; r++) {
      const int b = 4 * (lane >> 4) + r;
      if (b < a.B)
        cst1(a.qkvc, (size_t)b * a.qkv_n + i * 16 + col, bits_of(acc[0][r] * row_inv<kRows>(a, s.misc, b) * sc),
             tag, local);
    }
  }
  SH_MARK(s.misc, l, 3);
  return true;
}

// C: x_mid[b][16 i + c] = x[b][.] + scale * (W_o attn)
template <int kL, int kRows>
__device__ __forceinline__ bool o_item(const LayersArgs &a, const LayerG &P, int l, int i, unsigned ep,
                       const Lds &s, const EmbQ &e) {
  const int lane = threadIdx.x & 63, col = lane & 15, K = a.heads * kD;
  u32x4 w[kL][1];
  load_weights<kL, 1>(w, P.wo, K, i);
  const float sc = P.so[i * 16 + col];
  float rv[4];
  uint64_t rc[4];
  request_residual<kOutRows<kRows>>(a, a.x0c, l == 0 ? a.x_in : nullptr, i * 16 + col, rv, rc,
                                    l == 0 ? e : EmbQ{});
  __builtin_amdgcn_sched_barrier(0);
  if (!stage_f16<(kL + 3) / 4, kRows, true>(a, a.attnc, tag_of(ep, l), K, s.xs, s.misc)) return false;
  f32x4 acc[1];
  mfma_weights<kL, 1>(w, s.xs, K + 8, kRows == 1 ? 1 : a.B, acc);
  reduce_waves<1>(acc, s.red);
  if (threadIdx.x < 64) {
    if (l > 0) finish_residual<kOutRows<kRows>>(a, a.x0c, i * 16 + col, tag_of(ep, l - 1), rv, rc);
    else consume_cells(rc);  // unused at the first layer, but the loads must retire here
    const unsigned tag = tag_of(ep, l);
#pragma unroll
    for (int r = 0; r < kOutRows<kRows>; r++) {
      const int b = 4 * (lane >> 4) + r;
      if (b < a.B) cst1(a.x1c, (size_t)b * a.H + i * 16 + col, bits_of(fmaf(acc[0][r], sc, rv[r])), tag);
    }
  }
  return true;
}

// D: act[b][16 p + c] = silu(scale_g * gate) * (scale_u * up) of RMSNorm(x_mid),
// two adjacent columns per cell
template <int kL, int kRows>
__device__ __forceinline__ bool up_item(const LayersArgs &a, const LayerG &P, int l, int p, unsigned ep,
                        const Lds &s) {
  const int lane = threadIdx.x & 63, col = lane & 15;
  u32x4 w[kL][2];
  load_weights<kL, 2>(w, P.wup, a.H, p);
  const int ng = 2 * p * 16 + col;  // tiled rows of the gate and up tiles of pair p
  const float sg = P.sup[ng], su = P.sup[ng + 16];
  __builtin_amdgcn_sched_barrier(0);
  if (!stage_rms<(kL + 3) / 4, kRows, true, true>(a, a.x1c, nullptr, tag_of(ep, l), P.norm2, a.H, s.xs, s.misc))
    return false;
  f32x4 acc[2];
  mfma_weights<kL, 2>(w, s.xs, a.H + 8, kRows == 1 ? 1 : a.B, acc);
  reduce_waves<2>(acc, s.red);
  if (threadIdx.x < 64) {
    const unsigned tag = tag_of(ep, l);
#pragma unroll
    for (int r = 0; r < kOutRows<kRows>; r++) {
      const int b = 4 * (lane >> 4) + r;
      const float inv = row_inv<kRows>(a, s.misc, b);
      const uint32_t h = f32_to_f16_bits(silu(acc[0][r] * inv * sg) * (acc[1][r] * inv * su));
      const uint32_t nb = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)h, 0xB1, 0xf, 0xf, false);
      if (b < a.B && (col & 1) == 0)
        cst1(a.actc, (size_t)b * (a.inter / 2) + (p * 16 + col) / 2, h | (nb << 16), tag);
    }
  }
  return true;
}

// E: x[b][16 i + c] = x_mid[b][.] + scale * (W_down act); the last layer
// writes the plain buffer the final norm reads
// w holds the item's weights (requested by the caller).
template <int kL, int kRows>
__device__ __forceinline__ bool down_item(const LayersArgs &a, const LayerG &P, int l, int i, unsigned ep,
                          const Lds &s, const u32x4 (&w)[kL][1]) {
  const int lane = threadIdx.x & 63, col = lane & 15, K = a.inter;
  const float sc = P.sdown[i * 16 + col];
  const unsigned tag = tag_of(ep, l);
  float rv[4];
  uint64_t rc[4];
  request_residual<kOutRows<kRows>>(a, a.x1c, nullptr, i * 16 + col, rv, rc);
  __builtin_amdgcn_sched_barrier(0);
  if (!stage_f16<(kL + 3) / 4, kRows, true>(a, a.actc, tag, K, s.xs, s.misc)) return false;
  SH_MARK(s.misc, l, 4);
  f32x4 acc[1];
  mfma_weights<kL, 1>(w, s.xs, K + 8, kRows == 1 ? 1 : a.B, acc);
  SH_MARK(s.misc, l, 5);
  reduce_waves<1>(acc, s.red);
  SH_MARK(s.misc, l, 6);
  if (threadIdx.x < 64) {
    finish_residual<kOutRows<kRows>>(a, a.x1c, i * 16 + col, tag, rv, rc);
    const bool last = l + 1 == a.n_layers;
#pragma unroll
    for (int r = 0; r < kOutRows<kRows>; r++) {
      const int b = 4 * (lane >> 4) + r;
      const float v = fmaf(acc[0][r], sc, rv[r]);
      if (b < a.B) {
        // the last layer also writes the plain buffer the separate final
        // norm reads (steps whose LM head runs outside this kernel)
        if (last) gbl(a.x_in)[(size_t)b * a.H + i * 16 + col] = v;
        cst1(a.x0c, (size_t)b * a.H + i * 16 + col, bits_of(v), tag);
      }
    }
  }
  SH_MARK(s.misc, l, 7);
  return true;
}

// ---- attention and merge items -------------------------------------------------

constexpr int kPStride = kD + 4;  // cells per attention partial: acc[128], m, l, pad

// Attention works on blocks of kBlk positions: the scores as q (heads as
// MFMA rows) times K^T (positions as columns), ten 16-position tiles per
// block, tiles w, w + 4, w + 8 on wave w; the V sums as P (fp16, heads as
// rows) times V, five 32-position steps per block, output dims
// [32 w, 32 w + 32) on wave w. The MFMA operands hold 8 consecutive values
// of the contracted index per lane, so this kernel keeps V transposed per
// KV head: vcache[b][kv_head][d][vt_stride] (positions contiguous).
constexpr int kBlk = 160;
constexpr int kKT = 3;           // K tiles of a block per wave
constexpr int kVS = kBlk / 32;   // V steps of a block

// LDS of an attention item, from the start of the dynamic area.
template <int kG>
struct AttnLds {
  float qs[kG][kD];  // this row's normed, rotated, scaled q of the KV head's query heads
  alignas(16) _Float16 knew[kD];
  _Float16 vnew[kD];
  float scores[kG][kMaxSplitChunk];
  alignas(16) _Float16 p[kG][kMaxSplitChunk + kBlk];  // probabilities, zero up to whole blocks
  float wmax[4][kG], wl[4][kG];
  float sdump[4][kG][64];  // where the score stores of lanes without a score go
};

// LDS of a merge item.
// Merge items per (row, query head). Measured at batch 1: 4 parts +1.6 %
// tokens/s over 1 part (each item polls a quarter of the partials); 8 parts
// -3.7 % against 4.
constexpr int kMergeParts = 4;

struct MergeLds {
  float gm[kT];             // per split group: max m_j of its active splits
  float part[4][kT][3];     // per wave: column pair's two sums and the l sum
};

// LDS of a merge run (all kMergeParts parts of a head in one item).
struct MergeRunLds {
  float gm[kT];
  float part[kMergeParts][4][16][3];  // per part and wave, as MergeLds::part
};

// K and V^T registers of one block (the first block of an item is
// requested ahead by attn_prefetch): k[tt][kk] holds K[position 16 (w +
// 4 tt) + lane % 16][32 kk + 8 (lane / 16) ..], v[nt][ks] holds
// V^T[dim 32 w + 16 nt + lane % 16][positions 32 ks + 8 (lane / 16) ..].
struct AttnKV {
  f16x8 k[kKT][4];
  f16x8 v[2][kVS];
};

// Positions are clamped to the split's own range, [pb, pe_k) of the K
// cache and [pb, pe_v) of V^T: positions past the split re-read its last
// ones (already requested) instead of fetching the next split's.
__device__ __forceinline__ void attn_load_k(const SH_GLOBAL uint16_t *kb, int pb, int pe_k, AttnKV &kv) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int tt = 0; tt < kKT; tt++) {
    const int p = min(pb + 16 * (wave + 4 * tt) + r, pe_k - 1);
#pragma unroll
    for (int kk = 0; kk < 4; kk++)
      kv.k[tt][kk] = *reinterpret_cast<const SH_GLOBAL f16x8 *>(kb + (size_t)p * kD + 32 * kk + 8 * grp);
  }
}

__device__ __forceinline__ void attn_load_v(const LayersArgs &a, const SH_GLOBAL uint16_t *vtb, int pb,
                                            int pe_v, AttnKV &kv) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int nt = 0; nt < 2; nt++) {
    const SH_GLOBAL uint16_t *row = vtb + (size_t)(32 * wave + 16 * nt + r) * a.vt_stride;
#pragma unroll
    for (int ks = 0; ks < kVS; ks++) {
      const int p = min(pb + 32 * ks + 8 * grp, pe_v - 8);
      kv.v[nt][ks] = *reinterpret_cast<const SH_GLOBAL f16x8 *>(row + p);
    }
  }
}

// The split's ends: the K cache holds max_pos positions, a V^T row
// vt_stride (both ends multiples of 16 or max_pos, so 8-position V loads
// stay aligned).
__device__ __forceinline__ int split_end_k(const LayersArgs &a, int s) {
  return min(s * a.chunk + a.chunk, a.max_pos);
}
__device__ __forceinline__ int split_end_v(const LayersArgs &a, int s) {
  return min(s * a.chunk + a.chunk, a.vt_stride);
}

// Requests K / V^T of the first block of attention item `item`.
__device__ __forceinline__ void attn_prefetch(const LayersArgs &a, const LayerG &P, int item,
                                              AttnKV &kv) {
  const int splits = a.splits, kvn = a.kv_heads;
  const int s = item % splits, kvh = (item / splits) % kvn, b = item / (splits * kvn);
  const size_t kv_row = (size_t)b * kvn + kvh;
  const int p0 = s * a.chunk;
  attn_load_k(P.kcache + kv_row * a.max_pos * kD, min(p0, a.max_pos - 1), split_end_k(a, s), kv);
  attn_load_v(a, P.vcache + kv_row * kD * a.vt_stride, p0, split_end_v(a, s), kv);
}

// ---- K / V^T of a run's next attention item, staged in LDS -------------
// Within a workgroup's run of attention items, each item requests its
// successor's first block global -> LDS directly (buffer loads with the LDS
// destination, inline asm, so the compiler neither waits for them nor
// counts them) once its own block is in registers, and the successor copies
// it from LDS into the registers attn_load_k / attn_load_v would fill. The
// area overlays the GEMV staging, idle during the attention phase, after
// the item's own LDS.
//  - K: kBlk positions x 256 B, position p's 16-byte chunk c at chunk c ^ (p
//    % 16) (16 lanes reading one chunk of 16 consecutive positions hit
//    distinct banks); 40 loads of 4 positions.
//  - V^T: kD rows (dims) x kBlk positions (320 B), chunk c of row d at c ^
//    ((d / 4) % 4); 40 loads of 64 chunks.
// Positions are clamped as the register path clamps them, so the values
// are the same. Items past the context request nothing.
constexpr int kStageRun = 8;  // shortest run whose items stage their successor's block
constexpr int kStageOff = (int)((sizeof(AttnLds<2>) + 1023) / 1024 * 1024);
constexpr int kStageK = kBlk * kD * 2;       // 40 KiB
constexpr int kStageBytes = 2 * kStageK;     // + V^T
constexpr int kStageLoads = kStageK / 1024;  // per operand: 40
static_assert(kBlk % 4 == 0 && (kD * kBlk * 2) % 1024 == 0 && kStageLoads % 4 == 0, "stage layout");
static_assert(kBlk / 8 % 4 == 0, "V^T chunk swizzle stays in the row");

__device__ __forceinline__ void attn_stage_issue(const LayersArgs &a, const LayerG &P, int item,
                                                 uint8_t *smem) {
  const int splits = a.splits, kvn = a.kv_heads;
  const int s = item % splits, kvh = (item / splits) % kvn, b = item / (splits * kvn);
  const int p0 = s * a.chunk, L = cnst(a.pos)[b] + 1;
  if (p0 >= L || p0 >= a.max_pos || L > a.max_pos) return;  // uniform: an item past the context
  const size_t kv_row = (size_t)b * kvn + kvh;
  const int pe_k = split_end_k(a, s), pe_v = split_end_v(a, s);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  auto desc = [](uint64_t x, uint32_t bytes) {
    return u32x4{(uint32_t)x, (uint32_t)(x >> 32) & 0xffffu, bytes, 0x00020000u};
  };
  const u32x4 kd = desc((uint64_t)(uintptr_t)(P.kcache + kv_row * a.max_pos * kD), (uint32_t)a.max_pos * kD * 2);
  const u32x4 vd = desc((uint64_t)(uintptr_t)(P.vcache + kv_row * kD * a.vt_stride), (uint32_t)kD * a.vt_stride * 2);
  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)smem + kStageOff;
  constexpr int kPer = kStageLoads / 4;  // loads per wave per operand
#pragma unroll
  for (int j = 0; j < kPer; j++) {
    const int u = wave * kPer + j;
    const int pos = 4 * u + (lane >> 4);
    const int pc = min(p0 + pos, pe_k - 1);
    const int vo = pc * kD * 2 + (((lane & 15) ^ (pos & 15)) * 16);
    const uint32_t m0 = base + u * 1024;
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(vo), "s"(kd), "{m0}"(m0) : "memory");
  }
#pragma unroll
  for (int j = 0; j < kPer; j++) {
    const int u = wave * kPer + j;
    const int f = 64 * u + lane, d = f / (kBlk / 8), c = f % (kBlk / 8);
    const int pv = min(p0 + 8 * (c ^ ((d >> 2) & 3)), pe_v - 8);
    const int vo = (d * a.vt_stride + pv) * 2;
    const uint32_t m0 = base + kStageK + u * 1024;
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(vo), "s"(vd), "{m0}"(m0) : "memory");
  }
}

// Uses every register of kv, so the compiler waits here for the loads that
// filled them: a load still pending on some path where paths join makes it
// wait for all loads (vmcnt(0)) at the next register it reuses, staging
// loads included.
__device__ __forceinline__ void attn_kv_ready(const AttnKV &kv) {
#pragma unroll
  for (int tt = 0; tt < kKT; tt++)
    asm volatile("" ::"v"(kv.k[tt][0]), "v"(kv.k[tt][1]), "v"(kv.k[tt][2]), "v"(kv.k[tt][3]));
#pragma unroll
  for (int nt = 0; nt < 2; nt++)
#pragma unroll
    for (int ks = 0; ks < kVS; ks++) asm volatile("" ::"v"(kv.v[nt][ks]));
}

// The staged block into the registers of attn_load_k / attn_load_v (item
// positions from p0, the split's K end pe_k).
__device__ __forceinline__ void attn_stage_read(const uint8_t *smem, int p0, int pe_k, AttnKV &kv) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, grp = lane >> 4;
  const uint8_t *st = smem + kStageOff;
#pragma unroll
  for (int tt = 0; tt < kKT; tt++) {
    const int pos = min(16 * (wave + 4 * tt) + r, pe_k - 1 - p0);
#pragma unroll
    for (int kk = 0; kk < 4; kk++)
      kv.k[tt][kk] = *reinterpret_cast<const f16x8 *>(st + pos * kD * 2 + (((4 * kk + grp) ^ (pos & 15)) * 16));
  }
#pragma unroll
  for (int nt = 0; nt < 2; nt++) {
    const int d = 32 * wave + 16 * nt + r;
#pragma unroll
    for (int ks = 0; ks < kVS; ks++)
      kv.v[nt][ks] = *reinterpret_cast<const f16x8 *>(
          st + kStageK + (d * (kBlk / 8) + ((4 * ks + grp) ^ ((d >> 2) & 3))) * 16);
  }
}

// The new token's k (wave 2) or v (wave 3) values e0, e0 + 1 into the
// cache: K row `pos`, V^T column `pos`.
__device__ __forceinline__ void append_new(const LayersArgs &a, SH_GLOBAL uint16_t *kb, SH_GLOBAL uint16_t *vtb,
                                           int pos, int wave, int e0, _Float16 x0, _Float16 x1) {
  const uint16_t u0 = __builtin_bit_cast(uint16_t, x0), u1 = __builtin_bit_cast(uint16_t, x1);
  if (wave == 2) {
    *reinterpret_cast<SH_GLOBAL uint32_t *>(kb + (size_t)pos * kD + e0) = (uint32_t)u0 | ((uint32_t)u1 << 16);
  } else {
    vtb[(size_t)e0 * a.vt_stride + pos] = u0;
    vtb[(size_t)(e0 + 1) * a.vt_stride + pos] = u1;
  }
}

// B: item = (b, KV head, split), its first K / V^T block requested by
// attn_prefetch. Scores positions [p0, p0 + chunk) of the context for the
// kG query heads of the KV head (Qwen3: RMSNorm of q and of the new k over
// the head, RoPE rotate-half at this step's position; the split holding it
// appends the new k / v to the cache) and writes the partial (unnormalised
// V sum, max, sum) of each head as cells (local: every consumer of them
// runs on this XCD, cst1). Splits past the context write nothing. `runs`:
// the workgroup runs several items (staged: this item's
// first block was staged in LDS by the previous one; next: the item whose
// block this one stages, or -1). With `reuse`, the workgroup's previous
// item was the split
// before this one of the same (row, KV head): its normed, rotated q and new
// k / v are still in LDS, so this item neither polls the cells nor
// normalises again (the values, and so the arithmetic, are the same).
// kRope: this step's RoPE factors of the lane's two frequencies arrive in
// rcs / rsn (batch 1 with the embedding inside the kernel) instead of from
// the embed kernel's table.
struct NoRequest {
  __device__ void operator()() const {}
};

// after_poll: requests issued once the item's q / k / v cells have arrived
// (batch 1: the down weights of a workgroup with a down item)
template <int kG, bool kRope = false, class AfterPoll = NoRequest>
__device__ __forceinline__ bool attn_item(const LayersArgs &a, const LayerG &P, int l, int item, unsigned ep,
                          uint8_t *smem, Misc *misc, AttnKV &kv, bool runs, bool reuse, bool staged,
                          int next, bool local, f32x2 rcs = f32x2{}, f32x2 rsn = f32x2{},
                          AfterPoll &&after_poll = AfterPoll{}) {
  static_assert((kG + 2) * kD / 2 <= kT, "one pair of q / k / v cells per thread");
  static_assert(kG <= 4, "MFMA rows 0..3 of lanes 0..15 hold the heads");
  AttnLds<kG> &S = *reinterpret_cast<AttnLds<kG> *>(smem);
  SH_MARK(misc, l, 22);
  const int splits = a.splits, kvn = a.kv_heads;
  const int s = item % splits, kvh = (item / splits) % kvn, b = item / (splits * kvn);
  // wave through readfirstlane: the compiler then treats conditions on it
  // as uniform (scalar branches, no exec masks between MFMA chains)
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), r = lane & 15,
            grp = lane >> 4;
  const int chunk = a.chunk, p0 = s * chunk;
  const int cap = min(chunk, a.max_pos - p0);  // <= 0 for splits past the cache
  const size_t kv_row = (size_t)b * kvn + kvh;
  SH_GLOBAL uint16_t *kb = P.kcache + kv_row * a.max_pos * kD;
  SH_GLOBAL uint16_t *vtb = P.vcache + kv_row * kD * a.vt_stride;

  const int L = cnst(a.pos)[b] + 1;  // context including the new token
  const int active = (L + chunk - 1) / chunk;
  if (s >= active || cap <= 0 || L > a.max_pos) {  // uniform
    after_poll();
    // the next item's block is staged all the same; with none, a block
    // staged for this one lands before the phase ends
    if (next >= 0)
      attn_stage_issue(a, P, next, smem);
    else if (staged)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return true;
  }
  const int h0 = kvh * kG;
  const unsigned tag = tag_of(ep, l);
  const int p1 = min(L, p0 + chunk), np = p1 - p0, pos = L - 1;
  const bool holds_new = p1 == L;  // this split holds the new token (S.knew / S.vnew)
  // Each wave holds one head as a pair of cells per lane: waves 0 and 1 the
  // query heads h0 and h0 + 1, wave 2 the new k, wave 3 the new v; lane j
  // values e0 = 2 j and 2 j + 1. The RMSNorm of a head is a wave sum, and
  // RoPE's rotate-half partner of index e (e +- 64) sits in lane j +- 32.
  // This step's norm gains and RoPE factors are requested before the wait.
  static_assert(kG == 2 && (kG + 2) * kD / 2 == kT, "one head per wave");
  const int e0 = 2 * lane, fe = e0 & (kD / 2 - 1);
  if (!reuse) {
    const SH_GLOBAL float *gain = wave == 2 ? P.k_norm : P.q_norm;
    const f32x2 g = *reinterpret_cast<const SH_GLOBAL f32x2 *>(gain + e0);
    const f32x2 cs = kRope ? rcs : *reinterpret_cast<const SH_GLOBAL f32x2 *>(gbl(a.rope) + (size_t)b * kD + fe);
    const f32x2 sn = kRope ? rsn
                           : *reinterpret_cast<const SH_GLOBAL f32x2 *>(gbl(a.rope) + (size_t)b * kD + kD / 2 + fe);
    float v0, v1;
    {
      const size_t qrow = (size_t)b * a.qkv_n;
      size_t cell;
      if (wave < 2) cell = qrow + (size_t)(h0 + wave) * kD + e0;
      else if (wave == 2) cell = qrow + (size_t)a.heads * kD + kvh * kD + e0;
      else cell = qrow + (size_t)(a.heads + kvn) * kD + kvh * kD + e0;
      uint64_t cv[2];
      // one 16-byte load per lane at batch 1; the batched variants measured
      // ~1 % slower that way (b=4, with the merge polls below), so they keep
      // 8-byte loads here and in merge_run
      bool ok;
      if constexpr (kRope)
        ok = spin_pairs(a, a.qkvc, [&](int k) { return cell + k; }, 3ull, tag, cv);
      else
        ok = spin_cells(a, a.qkvc, [&](int k) { return cell + k; }, 3ull, tag, cv);
      // batch 1: no vote (see wave_waits_ok); every wave reaches the
      // barrier after the q / k / v stores below
      if constexpr (kRope)
        wave_waits_ok(a, ok, misc);
      else if (!waits_ok(a, ok, misc))
        return false;
      after_poll();
      SH_MARK(misc, l, 8);
      v0 = cell_f32(cv[0]);
      v1 = cell_f32(cv[1]);
    }
    if (wave < 3) {  // q heads and k: RMSNorm over the head, then RoPE
      const float ss = wave_sum_rows(fmaf(v0, v0, v1 * v1));
      const float inv = 1.0f / sqrtf(ss / kD + a.eps);
      v0 = v0 * inv * g.x;
      v1 = v1 * inv * g.y;
      const float o0 = __shfl_xor(v0, 32, 64), o1 = __shfl_xor(v1, 32, 64);
      if (lane < 32) {
        v0 = fmaf(v0, cs.x, -(o0 * sn.x));
        v1 = fmaf(v1, cs.y, -(o1 * sn.y));
      } else {
        v0 = fmaf(v0, cs.x, o0 * sn.x);
        v1 = fmaf(v1, cs.y, o1 * sn.y);
      }
    }
    if (wave < 2) {
      *reinterpret_cast<f32x2 *>(&S.qs[wave][e0]) = f32x2{v0 * a.scale, v1 * a.scale};
    } else {  // the new k / v, kept for the run's split that holds the new token
      const _Float16 h0v = (_Float16)v0, h1v = (_Float16)v1;
      _Float16 *nw = wave == 2 ? S.knew : S.vnew;
      nw[e0] = h0v;
      nw[e0 + 1] = h1v;
      if (holds_new) append_new(a, kb, vtb, pos, wave, e0, h0v, h1v);
    }
  } else if (holds_new && wave >= 2) {
    const _Float16 *nw = wave == 2 ? S.knew : S.vnew;
    append_new(a, kb, vtb, pos, wave, e0, nw[e0], nw[e0 + 1]);
  }
  lds_barrier();
  SH_MARK(misc, l, 9);
  // this item's first block, staged in LDS by the previous item, into kv;
  // the next item's block is requested below, after every load this item
  // waits for (loads complete in issue order; this item's further blocks, if
  // any, wait for it)
  if (staged) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's staging loads done
    __builtin_amdgcn_s_barrier();                      // and every wave's
    attn_stage_read(smem, p0, split_end_k(a, s), kv);
    lds_barrier();  // all reads of the area done before it is written again
  }

  // q as the MFMA A operand: row lane % 16 = head (zero past kG), k = 32 kk + 8 (lane / 16)
  // (read unconditionally from a clamped row, then selected: a conditional
  // read compiles to one branch and one LDS wait per element)
  f16x8 qa[4];
  {
    const float *qrow = &S.qs[min(r, kG - 1)][8 * grp];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const f32x4 lo = *reinterpret_cast<const f32x4 *>(qrow + 32 * kk);
      const f32x4 hi = *reinterpret_cast<const f32x4 *>(qrow + 32 * kk + 4);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        qa[kk][e] = r < kG ? (_Float16)lo[e] : (_Float16)0.0f;
        qa[kk][e + 4] = r < kG ? (_Float16)hi[e] : (_Float16)0.0f;
      }
    }
  }
  // (after the q reads: a wait the compiler places before them would
  // otherwise wait for the staging loads)
  if (runs) {
    if (!staged) attn_kv_ready(kv);
    // every load the compiler counts completes here, on every path (it
    // applies a wait it sees to its own count), so no later wait it places
    // for one of them also waits for the staging loads
    __builtin_amdgcn_s_waitcnt(0);
    if (next >= 0) attn_stage_issue(a, P, next, smem);
  }
  const int nblk = (np + kBlk - 1) / kBlk;

  // scores: lanes 0..15 of a tile's result hold heads 0..3 of its 16
  // positions; each lane keeps the max of the scores it stores. The new
  // token's K replaces the cache copy in its lane's registers before a
  // block's MFMAs (a fix-up between the tiles' MFMAs split them into basic
  // blocks, and the tiles' chains ran one after another), the tiles have
  // their own accumulators, and lanes without a score store it to a dump
  // area (no branch around the stores).
  float M[kG], lsum[kG];
#pragma unroll
  for (int g = 0; g < kG; g++) M[g] = -INFINITY;
  for (int bb = 0; bb < nblk; bb++) {
    const int pb = p0 + bb * kBlk;
    if (bb > 0) attn_load_k(kb, pb, split_end_k(a, s), kv);
    const int pn = pos - pb;  // the new token's index in this block
    if (holds_new && pn >= 0 && pn < kBlk) {  // uniform
      const bool mine = r == (pn & 15);
#pragma unroll
      for (int tt = 0; tt < kKT; tt++)
        if ((pn >> 4) == wave + 4 * tt) {  // uniform
#pragma unroll
          for (int kk = 0; kk < 4; kk++) {
            const f16x8 kn = *reinterpret_cast<const f16x8 *>(&S.knew[32 * kk + 8 * grp]);
            kv.k[tt][kk] = mine ? kn : kv.k[tt][kk];
          }
        }
    }
    // every wave runs kKT tiles; a tile past the block (waves 2 and 3's
    // last) scores clamped rows that nothing stores or counts
    // (the tiles' chains interleaved: each MFMA waits for its chain's last)
    f32x4 acc[kKT];
#pragma unroll
    for (int tt = 0; tt < kKT; tt++) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; kk++)
#pragma unroll
      for (int tt = 0; tt < kKT; tt++)
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[kk], kv.k[tt][kk], acc[tt], 0, 0, 0);
#pragma unroll
    for (int tt = 0; tt < kKT; tt++) {
      const int tile = wave + 4 * tt;
      const int pi = bb * kBlk + 16 * tile + lane;
      const bool valid = tile < kBlk / 16 && lane < 16 && pi < np;
#pragma unroll
      for (int g = 0; g < kG; g++) {
        float *dst = valid ? &S.scores[g][pi] : &S.sdump[wave][g][lane];
        *dst = acc[tt][g];
        M[g] = fmaxf(M[g], valid ? acc[tt][g] : -INFINITY);
      }
    }
  }
#pragma unroll
  for (int g = 0; g < kG; g++) {
    M[g] = wave_max_rows(M[g]);
    if (lane == 0) S.wmax[wave][g] = M[g];
  }
  lds_barrier();
  SH_MARK(misc, l, 10);

  // softmax statistics per head over the np scores; P = exp(s - M) in fp16,
  // zero up to whole blocks, and l = the sum of those fp16 values
  {
#pragma unroll
    for (int g = 0; g < kG; g++) {
      M[g] = fmaxf(fmaxf(S.wmax[0][g], S.wmax[1][g]), fmaxf(S.wmax[2][g], S.wmax[3][g]));
      lsum[g] = 0.0f;
    }
    for (int i = t; i < nblk * kBlk; i += kT) {
      const int ic = min(i, np - 1);
#pragma unroll
      for (int g = 0; g < kG; g++) {
        const float ev = expf(S.scores[g][ic] - M[g]);
        const _Float16 e = i < np ? (_Float16)ev : (_Float16)0.0f;
        S.p[g][i] = e;
        lsum[g] += (float)e;
      }
    }
#pragma unroll
    for (int g = 0; g < kG; g++) {
      lsum[g] = wave_sum_rows(lsum[g]);
      if (lane == 0) S.wl[wave][g] = lsum[g];
    }
    lds_barrier();
#pragma unroll
    for (int g = 0; g < kG; g++) lsum[g] = (S.wl[0][g] + S.wl[1][g]) + (S.wl[2][g] + S.wl[3][g]);
  }
  SH_MARK(misc, l, 11);

  // V sums: wave w owns dims [32 w, 32 w + 32); vn = the new token's V at
  // this lane's two dims (substituted by selects, not per-element branches)
  f32x4 oacc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  const _Float16 vn[2] = {S.vnew[32 * wave + r], S.vnew[32 * wave + 16 + r]};
  for (int bb = 0; bb < nblk; bb++) {
    const int pb = p0 + bb * kBlk;
    if (bb > 0) attn_load_v(a, vtb, pb, split_end_v(a, s), kv);
#pragma unroll
    for (int ks = 0; ks < kVS; ks++) {
      const int q0 = pb + 32 * ks + 8 * grp;
      if (holds_new && pos >= q0 && pos < q0 + 8) {  // the new token's V
        const int e0 = pos - q0;
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
          for (int e = 0; e < 8; e++) kv.v[nt][ks][e] = e == e0 ? vn[nt] : kv.v[nt][ks][e];
      }
      const f16x8 pr = *reinterpret_cast<const f16x8 *>(&S.p[min(r, kG - 1)][bb * kBlk + 32 * ks + 8 * grp]);
      const f16x8 pa = r < kG ? pr : f16x8{};
#pragma unroll
      for (int nt = 0; nt < 2; nt++) oacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, kv.v[nt][ks], oacc[nt], 0, 0, 0);
    }
  }
  SH_MARK(misc, l, 12);
  // lanes 0..15: oacc[nt][g] = sum_p P[g][p] V[p][32 w + 16 nt + lane]
  if (lane < 16) {
#pragma unroll
    for (int g = 0; g < kG; g++) {
      const size_t pp = (((size_t)b * a.heads + h0 + g) * splits + s) * kPStride;
#pragma unroll
      for (int nt = 0; nt < 2; nt++)
        cst1(a.partc, pp + 32 * wave + 16 * nt + lane, bits_of(oacc[nt][g]), tag, local);
    }
  }
  if (t < kG) {
    const size_t pp = (((size_t)b * a.heads + h0 + t) * splits + s) * kPStride;
    cst2(a.partc, pp + kD, bits_of(M[t]), bits_of(lsum[t]), tag, local);
  }
  SH_MARK(misc, l, 13);
  return true;
}

// M: item = (row, query head, part): combines the partials of the active
// splits (at most kSP),
//   out = sum_j exp(m_j - M) acc_j / sum_j exp(m_j - M) l_j,  M = max_j m_j,
// for dims [32 part, 32 part + 32) of the head (a head's merge is spread
// over kMergeParts workgroups, each polling a quarter of the head's
// partials), written as fp16 pairs. Thread t = (split group sg, column pair
// q) combines its splits sg, sg + kGroups, .. against their own max M_g;
// then each column pair rescales the groups: with M = max_g M_g,
//   out = sum_g exp(M_g - M) S_g / sum_g exp(M_g - M) L_g.
template <int kSP>
__device__ __forceinline__ bool merge_item(const LayersArgs &a, int l, int item, unsigned ep,
                                           uint8_t *smem, Misc *misc) {
  constexpr int kPairs = kD / kMergeParts / 2;  // column pairs per item
  constexpr int kGroups = kT / kPairs;           // split groups
  static_assert(kSP % kGroups == 0 && kSP <= kMaxSplits && kSP <= 64, "splits per merge");
  constexpr int kPer = kSP / kGroups;  // splits per thread
  MergeLds &S = *reinterpret_cast<MergeLds *>(smem);
  const int part = item % kMergeParts, hb = item / kMergeParts;
  const int h = hb % a.heads, b = hb / a.heads;
  const int t = threadIdx.x, q = t % kPairs, sg = t / kPairs;
  const int L = cnst(a.pos)[b] + 1;
  const int active = min((L + a.chunk - 1) / a.chunk, a.splits);
  const size_t base = ((size_t)b * a.heads + h) * a.splits * kPStride;
  const int col = kD / kMergeParts * part + 2 * q;  // this thread's column pair
  const unsigned tag = tag_of(ep, l);
  // cells 4 k .. 4 k + 3 of split sg + kGroups k: its two columns, then (m, l)
  uint64_t mask = 0;
#pragma unroll
  for (int k = 0; k < kPer; k++)
    if (sg + kGroups * k < active) mask |= 15ull << (4 * k);
  uint64_t cv[4 * kPer];
  const bool ok = spin_pairs(a, a.partc,
                             [&](int k) {
                               const int j = min(sg + kGroups * (k / 4), active - 1);
                               return base + (size_t)j * kPStride +
                                      ((k & 2) ? kD + (k & 1) : col + (k & 1));
                             },
                             mask, tag, cv);
  wave_waits_ok(a, ok, misc);  // no vote: every wave reaches the barrier below
  SH_MARK(misc, l, 14);
  float mg = -INFINITY;
#pragma unroll
  for (int k = 0; k < kPer; k++)
    if (sg + kGroups * k < active) mg = fmaxf(mg, cell_f32(cv[4 * k + 2]));
  float s0 = 0.0f, s1 = 0.0f, lg = 0.0f;
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    if (sg + kGroups * k < active) {
      const float wj = expf(cell_f32(cv[4 * k + 2]) - mg);
      s0 = fmaf(wj, cell_f32(cv[4 * k]), s0);
      s1 = fmaf(wj, cell_f32(cv[4 * k + 1]), s1);
      lg = fmaf(wj, cell_f32(cv[4 * k + 3]), lg);
    }
  }
  if (q == 0) S.gm[sg] = mg;  // -inf for a group without active splits (its sums are 0)
  lds_barrier();
  // every thread rescales its group's sums by exp(M_g - M); the groups of a
  // wave (sg = 4 wave .. 4 wave + 3, lanes q + 16 i) sum by lane exchanges
  float M = -INFINITY;
#pragma unroll
  for (int g = 0; g < kGroups; g++) M = fmaxf(M, S.gm[g]);  // finite: split 0 is active
  const float wg = mg == -INFINITY ? 0.0f : expf(mg - M);
  s0 *= wg;
  s1 *= wg;
  lg *= wg;
  static_assert(kPairs == 16 && kGroups == 16, "four split groups per wave");
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    s0 += __shfl_xor(s0, off, 64);
    s1 += __shfl_xor(s1, off, 64);
    lg += __shfl_xor(lg, off, 64);
  }
  const int wave = t >> 6;
  if ((t & 63) < kPairs) {
    S.part[wave][q][0] = s0;
    S.part[wave][q][1] = s1;
    S.part[wave][q][2] = lg;
  }
  lds_barrier();
  if (t < kPairs) {
    float v0 = 0.0f, v1 = 0.0f, lsum = 0.0f;
#pragma unroll
    for (int w4 = 0; w4 < 4; w4++) {
      v0 += S.part[w4][q][0];
      v1 += S.part[w4][q][1];
      lsum += S.part[w4][q][2];
    }
    const float inv = 1.0f / lsum;
    const uint32_t packed = (uint32_t)f32_to_f16_bits(v0 * inv) |
                            ((uint32_t)f32_to_f16_bits(v1 * inv) << 16);
    cst1(a.attnc, (size_t)(b * a.heads + h) * (kD / 2) + col / 2, packed, tag);
  }
  SH_MARK(misc, l, 15);
  lds_barrier();  // the next item reuses the LDS
  return true;
}

// M, all kMergeParts parts of (row, query head) hb in one item (the
// batched variants): one round of polls for every part's cells, the
// split maxima and l sums combined once, then each part's arithmetic
// exactly as merge_item's (so the results are the same bit for bit).
template <int kSP>
__device__ __forceinline__ bool merge_run(const LayersArgs &a, int l, int hb, unsigned ep, uint8_t *smem,
                                          Misc *misc) {
  constexpr int kPairs = kD / kMergeParts / 2, kGroups = kT / kPairs, kPer = kSP / kGroups;
  constexpr int kC = 2 + 2 * kMergeParts;  // cells per split: (m, l), then each part's column pair
  static_assert(kPer * kC <= 64 && kPairs == 16 && kGroups == 16, "cells per thread");
  MergeRunLds &S = *reinterpret_cast<MergeRunLds *>(smem);
  const int h = hb % a.heads, b = hb / a.heads;
  const int t = threadIdx.x, q = t % kPairs, sg = t / kPairs;
  const int L = cnst(a.pos)[b] + 1;
  const int active = min((L + a.chunk - 1) / a.chunk, a.splits);
  const size_t base = ((size_t)b * a.heads + h) * a.splits * kPStride;
  const unsigned tag = tag_of(ep, l);
  uint64_t mask = 0;
#pragma unroll
  for (int k = 0; k < kPer; k++)
    if (sg + kGroups * k < active) mask |= ((1ull << kC) - 1) << (kC * k);
  uint64_t cv[kPer * kC];
  const bool ok = spin_cells(a, a.partc,
                             [&](int c) {
                               const int k = c / kC, r = c % kC;
                               const int j = min(sg + kGroups * k, active - 1);
                               const int p = (r - 2) >> 1;
                               return base + (size_t)j * kPStride +
                                      (r < 2 ? kD + r : kD / kMergeParts * p + 2 * q + ((r - 2) & 1));
                             },
                             mask, tag, cv);
  if (!waits_ok(a, ok, misc)) return false;
  SH_MARK(misc, l, 14);
  float mg = -INFINITY;
#pragma unroll
  for (int k = 0; k < kPer; k++)
    if (sg + kGroups * k < active) mg = fmaxf(mg, cell_f32(cv[kC * k]));
  float s0[kMergeParts], s1[kMergeParts], lg = 0.0f;
#pragma unroll
  for (int p = 0; p < kMergeParts; p++) s0[p] = s1[p] = 0.0f;
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    if (sg + kGroups * k < active) {
      const float wj = expf(cell_f32(cv[kC * k]) - mg);
#pragma unroll
      for (int p = 0; p < kMergeParts; p++) {
        s0[p] = fmaf(wj, cell_f32(cv[kC * k + 2 + 2 * p]), s0[p]);
        s1[p] = fmaf(wj, cell_f32(cv[kC * k + 3 + 2 * p]), s1[p]);
      }
      lg = fmaf(wj, cell_f32(cv[kC * k + 1]), lg);
    }
  }
  if (q == 0) S.gm[sg] = mg;
  lds_barrier();
  float M = -INFINITY;
#pragma unroll
  for (int g = 0; g < kGroups; g++) M = fmaxf(M, S.gm[g]);
  const float wg = mg == -INFINITY ? 0.0f : expf(mg - M);
  lg *= wg;
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) lg += __shfl_xor(lg, off, 64);
  const int wave = t >> 6;
#pragma unroll
  for (int p = 0; p < kMergeParts; p++) {
    float x0 = s0[p] * wg, x1 = s1[p] * wg;
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      x0 += __shfl_xor(x0, off, 64);
      x1 += __shfl_xor(x1, off, 64);
    }
    if ((t & 63) < kPairs) {
      S.part[p][wave][q][0] = x0;
      S.part[p][wave][q][1] = x1;
      S.part[p][wave][q][2] = lg;
    }
  }
  lds_barrier();
  if (t < kPairs * kMergeParts) {
    const int p = t / kPairs, qq = t % kPairs;
    float v0 = 0.0f, v1 = 0.0f, lsum = 0.0f;
#pragma unroll
    for (int w4 = 0; w4 < 4; w4++) {
      v0 += S.part[p][w4][qq][0];
      v1 += S.part[p][w4][qq][1];
      lsum += S.part[p][w4][qq][2];
    }
    const float inv = 1.0f / lsum;
    const uint32_t packed = (uint32_t)f32_to_f16_bits(v0 * inv) |
                            ((uint32_t)f32_to_f16_bits(v1 * inv) << 16);
    cst1(a.attnc, (size_t)(b * a.heads + h) * (kD / 2) + (kD / kMergeParts * p + 2 * qq) / 2, packed, tag);
  }
  SH_MARK(misc, l, 15);
  lds_barrier();  // the next item reuses the LDS
  return true;
}

// ---- the kernel ----------------------------------------------------------------

// H (steps with logits): logits[b][n] = head_scale[n] * (W_head
// RMSNorm(x; final_g))[b][n] for the 16-row tiles j = w, w + G, .. of this
// workgroup, each wave taking every fourth of them over the whole K (kLH
// 16-byte loads per lane and tile), the next tile's weights requested while
// the current one is multiplied; the running argmax keys go to the wave's
// slot of keys (read first, atomicMax only when larger).
template <int kLA, int kRows>
__device__ __forceinline__ bool head_phase(const LayersArgs &a, unsigned ep, const Lds &s) {
  constexpr int kLH = 4 * kLA;  // K / 64
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, G = gridDim.x, w = blockIdx.x;
  const int nT = a.head_tiles, H = a.H, B = kRows == 1 ? 1 : a.B;
  const SH_GLOBAL uint8_t *W = gbl(a.head_w);
  const int first = w + G * wave, step = 4 * G;
  u32x4 wb[2][kLH];
  float sc[2];
  auto load_tile = [&](u32x4 (&dst)[kLH], float &scale, int j) {
    const int jj = min(j, nT - 1);  // past the end: the last tile again, never used
#pragma unroll
    for (int u = 0; u < kLH; u++)
      dst[u] = __builtin_nontemporal_load(reinterpret_cast<const SH_GLOBAL u32x4 *>(
          W + ((size_t)jj * kLH + u) * 1024 + (size_t)lane * 16));
    scale = gbl(a.head_scale)[jj * 16 + (lane & 15)];
  };
  if (first < nT) load_tile(wb[0], sc[0], first);
  __builtin_amdgcn_sched_barrier(0);
  if (!stage_rms<(kLA + 3) / 4, kRows, false>(a, a.x0c, nullptr, tag_of(ep, a.n_layers - 1), gbl(a.final_g),
                                       H, s.xs, s.misc))
    return false;
  SH_MARK(s.misc, a.n_layers, 0);  // the final RMSNorm's input has arrived
  const int arow = lane & 15, acol = 8 * (lane >> 4);
  const _Float16 *xrow = s.xs + (arow < B ? arow : 0) * (H + 8) + acol;
  unsigned long long best[4] = {0, 0, 0, 0};
  auto tile = [&](const u32x4 (&wt)[kLH], float scale, int j) {
    constexpr int kCh = 4;
    f32x4 part[kCh];
#pragma unroll
    for (int c = 0; c < kCh; c++) part[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kLH; u++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const f16x8 af = *reinterpret_cast<const f16x8 *>(xrow + u * 64 + 32 * h);
        part[(2 * u + h) % kCh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            af, e4m3x8_to_f16(wt[u][2 * h], wt[u][2 * h + 1]), part[(2 * u + h) % kCh], 0, 0, 0);
      }
    const f32x4 acc = (part[0] + part[1]) + (part[2] + part[3]);
    const int n = j * 16 + (lane & 15);
#pragma unroll
    for (int r = 0; r < kOutRows<kRows>; r++) {
      const int b = 4 * (lane >> 4) + r;
      if (b < B && n < a.n_valid) {
        const float v = acc[r] * scale;
        gbl(a.logits)[(size_t)b * a.logits_ld + n] = v;
        const unsigned long long key = argmax_key(v, n);
        best[r] = key > best[r] ? key : best[r];
      }
    }
  };
  for (int j = first; j < nT; j += 2 * step) {
    load_tile(wb[1], sc[1], j + step);
    tile(wb[0], sc[0], j);
    load_tile(wb[0], sc[0], j + 2 * step);
    if (j + step < nT) tile(wb[1], sc[1], j + step);
  }
#pragma unroll
  for (int r = 0; r < kOutRows<kRows>; r++) {
    unsigned long long k = best[r];
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) {
      const unsigned long long o = __shfl_xor(k, off, 64);
      k = o > k ? o : k;
    }
    const int b = 4 * (lane >> 4) + r;
    unsigned long long *slot = a.keys + ((w * 4 + wave) % kKeySlots) * kKeyStride + b;
    if ((lane & 15) == 0 && b < B && k != 0 &&
        k > __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      atomicMax(slot, k);
  }
  return true;
}

// Runs f(i) for this workgroup's items i = first, first + G, .. < n. With
// kOne the host has checked that every phase has at most G items, so there
// is at most one: no loop, whose preheader would make the compiler wait for
// every outstanding request (it flushes the load counter ahead of a loop
// that uses values loaded before it), including the weights and K / V
// requested ahead. False when an item failed.
template <bool kOne, class F>
__device__ __forceinline__ bool for_items(int first, int n, int G, F &&f) {
  if constexpr (kOne) {
    return first < n ? f(first) : true;
  } else {
    for (int i = first; i < n; i += G)
      if (!f(i)) return false;
    return true;
  }
}

// Active attention splits of row b: those within its context (none for a
// row past the cache), the splits an attention item does work for.
__device__ __forceinline__ int attn_active(const LayersArgs &a, int b) {
  const int L = cnst(a.pos)[b] + 1;
  return L > a.max_pos ? 0 : min((L + a.chunk - 1) / a.chunk, a.splits);
}

// Items first .. end - 1 in order (kOne: at most one).
template <bool kOne, typename F>
__device__ __forceinline__ bool for_run(int first, int end, F &&f) {
  if constexpr (kOne) {
    return first < end ? f(first) : true;
  } else {
    for (int i = first; i < end; i++)
      if (!f(i)) return false;
    return true;
  }
}

template <int kG, int kLA, int kLC, int kLD, int kLE, int kSP, int kRows, bool kOne>
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

  if (threadIdx.x < 4) misc->par[threadIdx.x] = 0;
#ifdef SH_DECODE_TRACE
  for (int i = threadIdx.x; i < 2 * kTraceLayers * kTraceSlots; i += kT)
    (&misc->tr[0][0][0])[i] = 0;
#endif
  lds_barrier();
  // The step number: the embed kernel advanced the epoch word before this
  // launch, or, at batch 1 (kOne), where this launch is the step's only one,
  // it reads the previous number and workgroup 0 stores the new one after
  // its last item. kOne also reads the step's position (a.pos points at the
  // row lengths, which only that last act of workgroup 0 changes, after
  // every item that reads them), the token from key set keys_in, and
  // computes this lane's RoPE factors once for all layers.
  unsigned ep;
  EmbQ emb;
  int pos0 = 0;
  f32x2 rcs{}, rsn{};
  if constexpr (kOne) {
    ep = __builtin_amdgcn_readfirstlane(
             __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) + 1u;
    pos0 = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(a.lens, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    emb.tok = step_token(a.keys_in, 0, a.vocab);
    emb.head8 = gbl(a.head_w);
    emb.scale = gbl(a.head_scale)[emb.tok];
    const int fe = (2 * (threadIdx.x & 63)) & (kD / 2 - 1);  // attn_item's frequency pair
    float s0, c0, s1, c1;
    sincosf((float)pos0 * gbl(a.inv_freq)[fe], &s0, &c0);
    sincosf((float)pos0 * gbl(a.inv_freq)[fe + 1], &s1, &c1);
    rcs = f32x2{c0, c1};
    rsn = f32x2{s0, s1};
  } else {
    ep = *cnst(a.epoch);
  }
  const int G = gridDim.x, w = blockIdx.x;
  const int nA = a.qkv_n / 16, nB = B * a.kv_heads * a.splits, nM = B * a.heads * kMergeParts;
  const int nC = H / 16, nD = a.inter / 16, nE = H / 16;
  const int d0 = (w + G - nC % G) % G;  // this workgroup's first gate/up item
  // XCD-local placement (batch 1, a.xcd): the workgroup on XCD h (XCC_ID)
  // with rank j = w / 8 runs KV head h's j-th QKV tile (its kG query heads'
  // q tiles, then its k, then its v tiles), its split j and, on the last
  // kG * kMergeParts ranks, its query heads' merge items: the QKV ->
  // attention and attention -> merge cells never leave the XCD. Workgroups
  // go to the XCDs round robin from an XCD that varies between launches
  // (measured: w on XCD w % 8 in a fresh process, on (w + 7) % 8 after
  // other launches), so an XCD holds one residue class of w mod 8 and
  // (XCD, w / 8) names every role once.
  const bool xl = kOne && a.xcd != 0;
  const unsigned xcc = xl ? xcc_id() : 0u;
  const int xh = (int)(xcc & 7), xj = w >> 3, xw = G >> 3;
  constexpr int kTiles = kD / 16;  // 16-row tiles per head
  const int xq = xj < kG * kTiles ? xh * kG * kTiles + xj
                 : xj < (kG + 1) * kTiles ? a.heads * kTiles + xh * kTiles + (xj - kG * kTiles)
                                          : (a.heads + a.kv_heads) * kTiles + xh * kTiles +
                                                (xj - (kG + 1) * kTiles);
  const int xm = xj >= xw - kG * kMergeParts ? xh * kG * kMergeParts + (xj - (xw - kG * kMergeParts)) : nM;
  const int m0 = xl ? xm : G - 1 - w;  // its first merge item
  if (xl && threadIdx.x == 0 && xcc >= 8) atomicOr(a.err, 2u);  // every wait then fails at once
  const bool hasC = w < nC;
  // attention items: workgroup w runs items [bA, eA), one at batch 1; at
  // larger batches a contiguous run of the active items (splits within
  // their row's context), i.e. consecutive splits of one (row, KV head),
  // whose items after the first reuse its q / k / v preparation. Only active
  // items are counted, so every workgroup gets the same number of them (a
  // split past the context costs nothing); bA / eA then index the active
  // items and item_of maps such an index to its item.
  // (the small-batch variant; the large-batch one partitions all items,
  // which keeps each run within half of a (row, KV head)'s splits: counting
  // only active items there measured 3.471 -> 3.534 ms at b=16)
  constexpr bool kAct = !kOne && kRows <= kSmallBatchRows;
  int nAct = nB;
  if constexpr (kAct) {
    nAct = 0;
    for (int b = 0; b < B; b++) nAct += attn_active(a, b) * a.kv_heads;
  }
  int bA = kOne ? (xl ? xh * a.splits + xj : w) : (int)((int64_t)w * nAct / G);
  int eA = kOne ? min(bA + 1, nB) : (int)((int64_t)(w + 1) * nAct / G);
  if constexpr (!kOne && !kAct) {
    // large-batch variant: when the grid divides into the (row, KV head)
    // pairs, each pair's workgroups split its active splits evenly (runs
    // stay within one pair, and no workgroup gets the pair's inactive ones)
    const int np = B * a.kv_heads;
    if (G % np == 0) {
      const int q = G / np, pr = w / q, part = w % q;
      const int act = attn_active(a, pr / a.kv_heads);
      bA = pr * a.splits + part * act / q;
      eA = pr * a.splits + (part + 1) * act / q;
    }
  }
  // a position in the active items: row b, KV head kvh, split s of the
  // row's act active ones (walked forward one item at a time: the row scan
  // runs once per run and at row changes)
  struct ActPos {
    int b, kvh, s, act;
  };
  auto act_at = [&](int k) {
    ActPos p{0, 0, 0, 0};
    if (kOne || !kAct) return p;
    for (; p.b < B; p.b++) {
      p.act = attn_active(a, p.b);
      const int n = p.act * a.kv_heads;
      if (k < n) break;
      k -= n;
    }
    if (p.act > 0) {
      p.kvh = k / p.act;
      p.s = k % p.act;
    }
    return p;
  };
  auto act_next = [&](ActPos p) {
    if (++p.s < p.act) return p;
    p.s = 0;
    if (++p.kvh < a.kv_heads) return p;
    p.kvh = 0;
    do {
      ++p.b;
    } while (p.b < B && (p.act = attn_active(a, p.b)) == 0);
    return p;
  };
  auto item_at = [&](const ActPos &p) { return (p.b * a.kv_heads + p.kvh) * a.splits + p.s; };
  auto item_of = [&](int k) { return kOne ? k : (kAct ? item_at(act_at(k)) : k); };
  // the run's first K / V block requested into registers a phase ahead (in
  // the previous layer's gate/up or down phase); the large-batch variant
  // instead stages it in LDS when the attention phase starts (its cell poll
  // covers the load), so no K / V registers are live through the GEMV
  // phases, whose staging passes then hold 8 rows
  constexpr bool kPre = kRows <= kSmallBatchRows;
  // QKV items: every G-th from w; in the large-batch variant two
  // consecutive tiles per workgroup [bQ, eQ) on one staged input, so each
  // input row is read by half as many workgroups
  const int gQ = kPre ? G : min(G, (nA + 1) / 2);
  const int bQ = kPre ? (xl ? xq : w) : (w < gQ ? (int)((int64_t)w * nA / gQ) : nA);
  const int eQ = kPre ? nA : (w < gQ ? (int)((int64_t)(w + 1) * nA / gQ) : nA);
  const bool hasQ = bQ < eQ;
  AttnKV kv;
  u32x4 wa[kLA][1];  // this workgroup's first QKV item's weights
  if (hasQ) load_weights<kLA, 1>(wa, layer_g(a, 0).wqkv, H, bQ);
  if (kPre && bA < eA) attn_prefetch(a, layer_g(a, 0), item_of(bA), kv);
  for (int l = 0; l < a.n_layers; l++) {
    const LayerG P = layer_g(a, l);
    const bool next = l + 1 < a.n_layers;
    u32x4 wd[kLE][1];  // this workgroup's down item's weights
    auto qkv_one = [&](int i) {
      if (i != bQ) load_weights<kLA, 1>(wa, P.wqkv, H, i);
      if (i == bQ) SH_TRACE(misc, l, 0);
      if (!qkv_item<kLA, kRows>(a, P, l, i, ep, lds, wa, !kPre && i != bQ, xl, emb)) return false;
      if (i == bQ) { SH_TRACE(misc, l, 1); SH_TRACE_WAIT(l, 0, misc); }
      return true;
    };
    if (kPre ? !for_items<kOne>(bQ, nA, G, qkv_one) : !for_run<false>(bQ, eQ, qkv_one)) return;
    SH_MARK(misc, l, 16);
    // the run's first block was requested into registers before the phase;
    // in runs of kStageRun items or more every later one is staged in LDS by
    // the item before it, in shorter ones requested when its item starts
    // (two copies of the loop: where paths with and without staging join,
    // the compiler's waits for the register path's loads would also wait
    // for staging loads)
    auto attn_run = [&](auto stg_c) {
      constexpr bool kStg = decltype(stg_c)::value;
      if (kStg && !kPre && bA < eA) {
        lds_barrier();  // every wave is past the previous phase's LDS reads
        attn_stage_issue(a, P, item_of(bA), smem);
      }
      ActPos cur{0, 0, 0, 0};
      if constexpr (kAct) cur = act_at(bA);
      return for_run<kOne>(bA, eA, [&](int k) {
        ActPos nxt{0, 0, 0, 0};
        int i = k;
        if constexpr (kAct) {
          nxt = act_next(cur);
          i = item_at(cur);
          cur = nxt;
        }
        if ((k != bA || !kPre) && !kStg) attn_prefetch(a, P, i, kv);
        if (k == bA) SH_TRACE(misc, l, 2);
        const bool reuse = !kOne && k != bA && i % a.splits != 0;
        const int nx = kStg && k + 1 < eA ? (kOne || kAct ? item_at(nxt) : k + 1) : -1;
        const bool staged = kStg && (k != bA || !kPre);
        if (!attn_item<kG, kOne>(a, P, l, i, ep, smem, misc, kv, kStg, reuse, staged, nx, xl, rcs, rsn,
                                 [&] {
                                   if (kOne && w < nE) load_weights<kLE, 1>(wd, P.wdown, a.inter, w);
                                 }))
          return false;
        if (k == bA) { SH_TRACE(misc, l, 3); SH_TRACE_WAIT(l, 1, misc); }
        if (k - bA < 8) SH_TRACE(misc, l, 16 + (k - bA));  // the run's first eight items' ends
        return true;
      });
    };
    if (!kOne && eA - bA >= kStageRun) {
      if (!attn_run(std::integral_constant<bool, true>())) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no staging load lands after the exit
        return;
      }
    } else if (!attn_run(std::integral_constant<bool, false>())) {
      return;
    }
    SH_MARK(misc, l, 17);
    // merge items: a part of a head each at batch 1; in the batched variants
    // a whole head each (one round of polls instead of kMergeParts in turn)
    if constexpr (kRows == 1) {
      if (!for_items<kOne>(m0, nM, G, [&](int j) {
            if (!merge_item<kSP>(a, l, j, ep, smem, misc)) return false;
            if (j == m0) SH_TRACE(misc, l, 15);
            return true;
          }))
        return;
    } else if (!for_items<false>(m0, nM / kMergeParts, G, [&](int j) {
                 if (!merge_run<kSP>(a, l, j, ep, smem, misc)) return false;
                 if (j == m0) SH_TRACE(misc, l, 15);
                 return true;
               })) {
      return;
    }
    SH_MARK(misc, l, 18);
    // O, gate/up and down items request their weights when they start: at
    // batch 1 each workgroup's previous item is then a phase or more behind
    // Workgroups with an O item request their down item's weights before
    // it, so the windows before the O item's and the down item's polls
    // carry 80 and 64 KiB of requests (with the down weights after the O
    // item: 32 and 112 KiB, and the down items' polls came last).
    // (batch 1: requested inside the workgroup's attention item, once its q
    // / k / v cells have arrived, or here if it has none)
    if ((!kOne || !(bA < eA)) && w < nE) load_weights<kLE, 1>(wd, P.wdown, a.inter, w);
    if (!for_items<kOne>(w, nC, G, [&](int i) {
          if (i == w) SH_TRACE(misc, l, 4);
          if (!o_item<kLC, kRows>(a, P, l, i, ep, lds, emb)) return false;
          if (i == w) { SH_TRACE(misc, l, 5); SH_TRACE_WAIT(l, 2, misc); }
          return true;
        }))
      return;
    SH_MARK(misc, l, 19);
    // The next layer's K / V and QKV weights: on workgroups with an O item
    // while the gate/up items run, on the others after their gate/up item.
    // Loads complete in issue order, and a wave also stalls at issuing a
    // bulk request while the memory pipeline is backed up: both belong
    // where the workgroup waits at least an exchange anyway. (Right after
    // the attention item, the K / V delayed the O items' polls; between the
    // down item's wait and its MFMAs, their issue stalled the down item by
    // ~2 us; on the workgroups with only a gate/up item, right after the
    // attention item, the burst slowed the merge and O items' polls.)
    if (hasC && next) {
      if (kPre && bA < eA) attn_prefetch(a, layer_g(a, l + 1), item_of(bA), kv);
      // (batch 1: the QKV weights after the down item, below)
      if (hasQ && !kOne) load_weights<kLA, 1>(wa, layer_g(a, l + 1).wqkv, H, bQ);
    }
    if (!for_items<kOne>(d0, nD, G, [&](int i) {
          if (i == d0) SH_TRACE(misc, l, 6);
          if (!up_item<kLD, kRows>(a, P, l, i, ep, lds)) return false;
          if (i == d0) { SH_TRACE(misc, l, 7); SH_TRACE_WAIT(l, 3, misc); }
          return true;
        }))
      return;
    SH_MARK(misc, l, 20);
    if (!hasC && next) {
      if constexpr (kOne) {
        // batch 1: these 192 workgroups hold their requests back for ~0.35 us
        // (wall clock, 100 MHz): issued right after the item, the burst (15
        // MiB) coincided with the O / down workgroups' K / V and the down
        // items' polls. Measured, one box each: delays of 0.25 / 0.35 / 0.5
        // / 0.7 us 0.4077 -> 0.4020 / 0.4024 / 0.4029 / 0.4037 ms per step;
        // 0.1 and 0.15 us and 1 us neutral or slower, 1.5 us 0.4114 ->
        // 0.4265; waiting for the item's cell stores instead, neutral.
        const unsigned long long t0 = wall_clock64();
        while (wall_clock64() - t0 < kPrefetchDelay) __builtin_amdgcn_s_sleep(1);
      }
      if (kPre && bA < eA) attn_prefetch(a, layer_g(a, l + 1), item_of(bA), kv);
      if (hasQ) load_weights<kLA, 1>(wa, layer_g(a, l + 1).wqkv, H, bQ);
    }
    if (!for_items<kOne>(w, nE, G, [&](int i) {
          if (i == w) SH_TRACE(misc, l, 8);
          if (i != w) load_weights<kLE, 1>(wd, P.wdown, a.inter, i);
          if (!down_item<kLE, kRows>(a, P, l, i, ep, lds, wd)) return false;
          if (i == w) { SH_TRACE(misc, l, 9); SH_TRACE_WAIT(l, 4, misc); }
          return true;
        }))
      return;
    SH_MARK(misc, l, 21);
    // batch 1, workgroups with O and down items: the next QKV weights (16
    // KiB) after the down item, so the down item's poll waits only behind
    // the K / V (0.4082 -> 0.4071 ms per step against both after the O item)
    if (kOne && hasC && next && hasQ) load_weights<kLA, 1>(wa, layer_g(a, l + 1).wqkv, H, bQ);
  }
  if (a.head_on && !head_phase<kLA, kRows>(a, ep, lds)) return;
  SH_MARK(misc, a.n_layers, 1);
  // kOne: the step's bookkeeping, by workgroup 0 after its last item. Every
  // workgroup has read the epoch word, the lengths and key set keys_in by
  // then: it read them first, and its items' cells carry the step's tag,
  // position or token, while workgroup 0's last item (its head tiles or its
  // last down item) waited, through the layers' chains of exchanges, on
  // cells that depend on every item of the step.
  if constexpr (kOne) {
    if (w == 0) {
      if (threadIdx.x < kKeySlots) gbl(a.keys_in)[(size_t)threadIdx.x * kKeyStride] = 0ull;
      if (threadIdx.x == 0) {
        if (pos0 < a.hist_len) gbl(a.hist)[pos0] = emb.tok;
        gbl(a.pos_out)[0] = pos0;
        gbl(a.lens)[0] = pos0 + 1;
        gbl(a.epoch)[0] = ep;
      }
    }
  }
#ifdef SH_DECODE_TRACE
  lds_barrier();
  if (w < kTraceWgs)
    for (int i = threadIdx.x; i < 2 * kTraceLayers * kTraceSlots; i += kT) {
      const int set = i / (kTraceLayers * kTraceSlots), rem = i % (kTraceLayers * kTraceSlots);
      g_decode_trace[set][w][rem / kTraceSlots][rem % kTraceSlots] = (&misc->tr[0][0][0])[i];
    }
#endif
}

// (kG, loads per lane of qkv / o / gate-up / down items, most splits per
// (row, KV head)) per supported shape; each in a batch-1 variant (one row
// per staging pass) and a variant for larger batches (four rows per pass)
#define SH_LAYERS_SHAPES(X) \
  X(2, 4, 8, 4, 12, 32)  /* hidden 1024, 16 x 128 query heads, 8 KV heads, inter 3072 */ \
  X(2, 1, 2, 1, 3, 64)   /* hidden 256, 4 x 128 query heads, 2 KV heads, inter 768 */

struct Shape {
  int g, la, lc, ld, le;
};

Shape shape_of(int H, int heads, int kv_heads, int inter) {
  return Shape{kv_heads > 0 ? heads / kv_heads : 0, H / 256, heads * kD / 256, H / 256, inter / 256};
}

// The kernel for a shape and batch (batch 0: the batch-1 variant; `one`: at
// most one item per workgroup in every phase), and the shape's split limit.
const void *kernel_for(const Shape &s, int batch, bool one, int *max_splits) {
#define SH_MATCH(G, LA, LC, LD, LE, SP)                                                            \
  if (s.g == G && s.la == LA && s.lc == LC && s.ld == LD && s.le == LE) {                          \
    if (max_splits) *max_splits = SP;                                                              \
    if (batch > kSmallBatchRows)                                                                   \
      return reinterpret_cast<const void *>(                                                       \
          &decode_layers_kernel<G, LA, LC, LD, LE, SP, kMaxRowsPerPass, false>);                   \
    if (batch > 1)                                                                                 \
      return reinterpret_cast<const void *>(                                                       \
          &decode_layers_kernel<G, LA, LC, LD, LE, SP, kSmallBatchRows, false>);                   \
    return one ? reinterpret_cast<const void *>(&decode_layers_kernel<G, LA, LC, LD, LE, SP, 1, true>) \
               : reinterpret_cast<const void *>(&decode_layers_kernel<G, LA, LC, LD, LE, SP, 1, false>); \
  }
  SH_LAYERS_SHAPES(SH_MATCH)
#undef SH_MATCH
  return nullptr;
}

// Every phase of a launch with `grid` workgroups has at most one item per
// workgroup.
bool one_item_each(const LayersArgs &a, int grid) {
  const int n[] = {a.qkv_n / 16, a.B * a.kv_heads * a.splits, a.B * a.heads * kMergeParts, a.H / 16,
                   a.inter / 16};
  for (int k : n)
    if (k > grid) return false;
  return true;
}

size_t attn_lds(int g) {
  return g == 1 ? sizeof(AttnLds<1>) : sizeof(AttnLds<2>);
}

}  // namespace

bool decode_layers_folds_embed(const LayersArgs &a, int grid) {
  // kernel_for's choice of the batch-1 instantiation (kOne)
  return a.B == 1 && one_item_each(a, grid);
}

bool decode_layers_xcd_ok(const LayersArgs &a, int grid) {
  if (a.B != 1 || grid % 8 != 0 || a.kv_heads != 8 || a.heads % a.kv_heads != 0) return false;
  const int per = grid / 8, g = a.heads / a.kv_heads;
  return a.splits == per && (g + 2) * (kD / 16) == per && g * kMergeParts <= per &&
         a.qkv_n == (a.heads + 2 * a.kv_heads) * kD && one_item_each(a, grid);
}

bool decode_layers_supported(int layers, int H, int heads, int kv_heads, int head_dim, int inter) {
  if (layers < 1 || layers > kMaxDecodeLayers) return false;
  if (head_dim != kD || kv_heads <= 0 || heads % kv_heads != 0) return false;
  if (H % 256 || (heads * kD) % 256 || inter % 256 || H > 4096) return false;
  return kernel_for(shape_of(H, heads, kv_heads, inter), 1, false, nullptr) != nullptr;
}

int decode_layers_max_splits(int H, int heads, int kv_heads, int inter) {
  int sp = 0;
  return kernel_for(shape_of(H, heads, kv_heads, inter), 1, false, &sp) ? sp : 0;
}

size_t decode_layers_lds(int B, int H, int heads, int inter, int *misc_offset) {
  int kmax = H;
  if (heads * kD > kmax) kmax = heads * kD;
  if (inter > kmax) kmax = inter;
  const size_t xs_max = ((size_t)B * (kmax + 8) * 2 + 15) / 16 * 16;
  size_t end = xs_max + 3 * 2 * 64 * 4 * sizeof(float);  // + wave-reduction area
  const size_t attn = attn_lds(2);
  if (attn > end) end = attn;
  if ((size_t)kStageOff + kStageBytes > end) end = (size_t)kStageOff + kStageBytes;  // staged K / V^T
  if (sizeof(MergeLds) > end) end = sizeof(MergeLds);
  if (sizeof(MergeRunLds) > end) end = sizeof(MergeRunLds);
  end = (end + 15) / 16 * 16;
  *misc_offset = (int)end;
  return end + sizeof(Misc);
}

size_t decode_layers_partial_cells(int heads) { return (size_t)kMaxBatch * heads * kMaxSplits * kPStride; }

hipError_t decode_layers_occupancy(const LayersArgs &a, size_t lds, int *blocks_per_cu) {
  const Shape sh = shape_of(a.H, a.heads, a.kv_heads, a.inter);
  int least = 1 << 30;
  // every variant: batch 1 (one item each / not), up to kSmallBatchRows, larger
  const int batch_of[4] = {1, 1, kSmallBatchRows, kMaxBatch};
  for (int v = 0; v < 4; v++) {
    const void *k = kernel_for(sh, batch_of[v], v == 0, nullptr);
    if (!k) return hipErrorInvalidValue;
    hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    int n = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kT, lds);
    if (e != hipSuccess) return e;
    if (n < least) least = n;
  }
  *blocks_per_cu = least;
  return hipSuccess;
}

#ifdef SH_DECODE_TRACE
hipError_t decode_layers_trace(void *dst, size_t bytes) {
  if (bytes > sizeof(g_decode_trace)) bytes = sizeof(g_decode_trace);
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_decode_trace), bytes, 0, hipMemcpyDeviceToHost);
}
#endif

hipError_t launch_decode_layers(hipStream_t s, const LayersArgs &a, int grid, size_t lds,
                                bool cooperative) {
  const void *k = kernel_for(shape_of(a.H, a.heads, a.kv_heads, a.inter), a.B, one_item_each(a, grid), nullptr);
  if (!k) return hipErrorInvalidValue;
  void *args[] = {const_cast<LayersArgs *>(&a)};
  if (cooperative) return hipLaunchCooperativeKernel(k, dim3(grid), dim3(kT), args, (unsigned)lds, s);
  return hipLaunchKernel(k, dim3(grid), dim3(kT), args, (unsigned)lds, s);
}

}  // namespace sh
