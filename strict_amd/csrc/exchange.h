// Exchange between the workgroups of a persistent kernel: values handed on
// within a launch travel in 8-byte cells of device memory, payload in the
// low word and the producing (step, layer) tag in the high word. A consumer
// loads the cells it needs until each carries the tag it expects, so the data
// is its own completion flag. Every cell load is a relaxed 64-bit
// agent-scope atomic, and so is every cell store except the XCD-local ones
// (cst with `local`): the memory model keeps those coherent across the
// XCDs' separate L2 caches. Every wait is bounded by a wall-clock limit; a timeout
// sets the sticky error word, after which every other wait gives up at once,
// so the grid always drains.
//
// The helpers take the kernel's argument struct, which must provide
// `unsigned *err` and `unsigned long long spin_ticks`.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sh {
namespace xchg {

#define SH_XGLOBAL __attribute__((address_space(1)))
#define SH_XCONST __attribute__((address_space(4)))

// Pointers cast to the global address space: loads through generic pointers
// compile to flat instructions, which also count against the LDS wait
// counter (every LDS wait would then wait for outstanding global requests).
template <class T>
__device__ __forceinline__ SH_XGLOBAL T *gbl(T *p) {
  return (SH_XGLOBAL T *)p;
}

// Tables written before the launch and only read by it, through the constant
// address space: uniform reads become scalar loads on their own counter.
template <class T>
__device__ __forceinline__ const SH_XCONST T *cnst(const T *p) {
  return (const SH_XCONST T *)p;
}

// Tag of the values layer l of step `epoch` produces (epoch >= 1, l < 63,
// so never 0, the value of never-written cells).
__device__ __forceinline__ unsigned tag_of(unsigned epoch, int l) {
  return epoch * 64u + (unsigned)l + 1u;
}

__device__ __forceinline__ uint64_t cld(const uint64_t *base, size_t cell) {
  return __hip_atomic_load(base + cell, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef unsigned xu32x4 __attribute__((ext_vector_type(4)));

// Buffer resource over a cell array for cld2 (byte offsets below 2 GiB).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t cell_rsrc(const uint64_t *base) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff, 0x00020000);
}

// Cells `cell` and `cell + 1` (cell even) in one 16-byte load with cld's
// agent-scope cache policy (sc1). Each cell is written by one 8-byte (or
// two-cell 16-byte) store, so each half holds a cell as a store left it,
// and each is checked for its tag on its own. A wave's poll of adjacent
// cells this way sends half the line requests of 8-byte loads: measured
// over 1,024 cells, 64 producer x 192 consumer workgroups, 1.45-1.59 us
// per exchange against 1.76 us with four adjacent 8-byte cells per lane.
// Loads of this kind are ordinary loads to the compiler, so the spin loops
// that issue them keep a compiler barrier in each round.
__device__ __forceinline__ void cld2(__amdgpu_buffer_rsrc_t rs, size_t cell, uint64_t &c0, uint64_t &c1) {
  const xu32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(cell * 8), 0, 16 /* sc1 */);
  c0 = (uint64_t)v.x | ((uint64_t)v.y << 32);
  c1 = (uint64_t)v.z | ((uint64_t)v.w << 32);
}

// `local`: a workgroup-scope store instead, which lands in the XCD's L2 and
// stays there; agent-scope loads on the same XCD see it (a hop ~0.22 us
// against ~0.4-0.53 us, measured in a ping-pong between workgroups), those
// on other XCDs do not until the kernel ends. Only for cells whose every
// consumer runs on the producer's XCD.
__device__ __forceinline__ void cst(uint64_t *base, size_t cell, uint32_t v, unsigned tag,
                                    bool local = false) {
  const uint64_t c = (uint64_t)v | ((uint64_t)tag << 32);
  if (local)
    __hip_atomic_store(base + cell, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else
    __hip_atomic_store(base + cell, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The XCD this wave runs on (hardware register XCC_ID).
__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xf;
}

__device__ __forceinline__ float cell_f32(uint64_t c) { return __builtin_bit_cast(float, (uint32_t)c); }
__device__ __forceinline__ uint32_t bits_of(float f) { return __builtin_bit_cast(uint32_t, f); }

template <class A>
__device__ __forceinline__ unsigned ld_err(const A &a) {
  return __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Loads base[at(k)], k < kN, until each one with bit k of mask set carries
// `tag`; c[k] receives them. at(k) must name a valid cell for every k
// (unused ones clamped onto used cells, so the loads need no branch). False
// when the wait exceeded the limit or another wait has failed.
template <int kN, class A, class At>
__device__ __forceinline__ bool spin_cells(const A &a, const uint64_t *base, At at, uint64_t mask,
                                           unsigned tag, uint64_t (&c)[kN]) {
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
    } else if ((it & 7) == 0 && (ld_err(a) != 0 || wall_clock64() - t0 > a.spin_ticks)) {
      return false;
    }
  }
}

// spin_cells over cells taken two at a time (cld2): at(k) for even k must be
// even, and cell k + 1 is at(k) + 1 (at is called for even k only).
template <int kN, class A, class At>
__device__ __forceinline__ bool spin_pairs(const A &a, const uint64_t *base, At at, uint64_t mask,
                                           unsigned tag, uint64_t (&c)[kN]) {
  static_assert(kN % 2 == 0, "pairs of cells");
  const __amdgpu_buffer_rsrc_t rs = cell_rsrc(base);
  unsigned long long t0 = 0;
  for (int it = 0;; it++) {
    // compiler barriers: a new load each round, every load issued before
    // the checks (ordinary loads are otherwise moved into the branches of
    // the checks, one round trip after another)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int k = 0; k < kN; k += 2) cld2(rs, at(k), c[k], c[k + 1]);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    bool ok = true;
#pragma unroll
    for (int k = 0; k < kN; k++) ok &= ((mask >> k & 1) == 0) | ((uint32_t)(c[k] >> 32) == tag);
    if (ok) return true;
    if (it == 0) {
      t0 = wall_clock64();
    } else if ((it & 7) == 0 && (ld_err(a) != 0 || wall_clock64() - t0 > a.spin_ticks)) {
      return false;
    }
  }
}

// One cell already requested as `c`: polls it again until it carries `tag`.
template <class A>
__device__ __forceinline__ bool finish_cell(const A &a, const uint64_t *base, size_t cell,
                                            unsigned tag, uint64_t &c) {
  unsigned long long t0 = 0;
  for (int it = 0; (uint32_t)(c >> 32) != tag; it++) {
    if (it == 0) {
      t0 = wall_clock64();
    } else if ((it & 7) == 0 && (ld_err(a) != 0 || wall_clock64() - t0 > a.spin_ticks)) {
      return false;
    }
    c = cld(base, cell);
  }
  return true;
}

// Workgroup barrier for LDS traffic only (vmcnt left alone): a
// __syncthreads() fence would make each wave wait for every global store it
// issued (cell stores) before the barrier.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Votes of block_any: two alternating sets, each wave's parity in its own
// word (a wave that runs ahead writes the other set).
struct Votes {
  int vote[2][4];
  int par[4];
};

// block_any in two halves around a barrier that the caller places (a
// wait's outcome can then share the barrier of values exchanged anyway):
// vote_cast before the barrier, vote_seen with its result after it.
__device__ __forceinline__ int vote_cast(bool p, Votes *v) {
  const int wave = threadIdx.x >> 6;
  const int par = v->par[wave];
  const bool any = __any(p ? 1 : 0) != 0;
  if ((threadIdx.x & 63) == 0) {
    v->vote[par][wave] = any ? 1 : 0;
    v->par[wave] = par ^ 1;
  }
  return par;
}
__device__ __forceinline__ bool vote_seen(int par, const Votes *v) {
  const int *vt = v->vote[par];
  return (vt[0] | vt[1] | vt[2] | vt[3]) != 0;
}

// True in every thread when p holds in any thread (a barrier; 4 waves).
__device__ __forceinline__ bool block_any(bool p, Votes *v) {
  const int par = vote_cast(p, v);
  lds_barrier();
  return vote_seen(par, v);
}

// After a vote on failed waits (workgroup-uniform `failed`): marks the
// sticky error and returns false if any wait failed.
template <class A>
__device__ __forceinline__ bool waits_done(const A &a, bool failed) {
  if (failed) {
    if (threadIdx.x == 0) atomicOr(a.err, 1u);
    return false;
  }
  return true;
}

// For a wave that stages and then reads only its own part of the LDS before
// the workgroup's next barrier: marks the sticky error when a wait of this
// wave failed, without a vote (and its barrier). The caller goes on with
// what it loaded either way, so every wave still reaches the next barrier,
// and the host reports the step as failed.
template <class A>
__device__ __forceinline__ void wave_waits_ok(const A &a, bool ok) {
  if (__any(ok ? 0 : 1) && (threadIdx.x & 63) == 0) atomicOr(a.err, 1u);
}

// Every thread's wait succeeded (workgroup-uniform); otherwise marks the
// sticky error.
template <class A>
__device__ __forceinline__ bool waits_ok(const A &a, bool ok, Votes *v) {
  return waits_done(a, block_any(!ok, v));
}

}  // namespace xchg
}  // namespace sh
