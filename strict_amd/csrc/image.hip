// Image kernels on interleaved 8-bit pixels: AdjustBrightness
// (Assembly.Tests/BlurPerformanceTests.cs:287-294) and the 5x5 box blur in
// both semantics (config: clamp-to-edge, (sum + 12) / 25; reference:
// BlurInteriorPixel / BlurEdgePixel at :85-141, in-bounds taps, sum / count),
// plus brightness fused into the blur's row loads.
//
// RGBA fast path (channels == 4, width % 4 == 0, 16-byte aligned buffers): a
// register-streaming kernel in which each wave walks down a column strip
// (described above the kernel). Any other shape takes a direct kernel (one
// pixel per thread, taps read through the cache), which is exact for every
// channel count and mode.
#include <hip/hip_runtime.h>

#include "common.h"
#include "swar.h"

#include <cstdlib>

namespace sh {
namespace {

constexpr int kBlock = 256;

// ---------------------------------------------------------------------------
// Brightness: 16-byte vectors, 4 per thread.
// ---------------------------------------------------------------------------

constexpr int kBrUnroll = 4;

__device__ __forceinline__ u32x4 brighten16(u32x4 v, uint32_t mag, bool neg, uint32_t mask) {
  v.x = brighten_u8x4(v.x, mag, neg, mask);
  v.y = brighten_u8x4(v.y, mag, neg, mask);
  v.z = brighten_u8x4(v.z, mag, neg, mask);
  v.w = brighten_u8x4(v.w, mag, neg, mask);
  return v;
}

__global__ __launch_bounds__(kBlock) void brightness_vec_kernel(const uint8_t *in, uint8_t *out,
                                                                size_t bytes, uint32_t mag,
                                                                int negative, uint32_t mask) {
  const size_t n16 = bytes / 16;
  const u32x4 *in4 = reinterpret_cast<const u32x4 *>(in);
  u32x4 *out4 = reinterpret_cast<u32x4 *>(out);
  const size_t base = (size_t)blockIdx.x * kBlock * kBrUnroll + threadIdx.x;
  u32x4 v[kBrUnroll];
  // full blocks without per-vector bounds checks (a load under a divergent
  // check can make the compiler wait for it before the next one)
  if (((size_t)blockIdx.x + 1) * kBlock * kBrUnroll <= n16) {
#pragma unroll
    for (int u = 0; u < kBrUnroll; u++) v[u] = __builtin_nontemporal_load(in4 + base + (size_t)u * kBlock);
#pragma unroll
    for (int u = 0; u < kBrUnroll; u++)
      __builtin_nontemporal_store(brighten16(v[u], mag, negative != 0, mask), out4 + base + (size_t)u * kBlock);
  } else {
#pragma unroll
    for (int u = 0; u < kBrUnroll; u++) {
      size_t i = base + (size_t)u * kBlock;
      if (i < n16) v[u] = __builtin_nontemporal_load(in4 + i);
    }
#pragma unroll
    for (int u = 0; u < kBrUnroll; u++) {
      size_t i = base + (size_t)u * kBlock;
      if (i < n16) __builtin_nontemporal_store(brighten16(v[u], mag, negative != 0, mask), out4 + i);
    }
  }
  // byte tail; the 16-byte units start on pixel boundaries when channels == 4,
  // and for channels < 4 every byte is adjusted, so the mask byte index is i % 4.
  if (blockIdx.x == 0 && threadIdx.x < (bytes & 15)) {
    size_t i = n16 * 16 + threadIdx.x;
    uint32_t m = (mask >> (8 * (i & 3))) & 0xffu;
    out[i] = (uint8_t)brighten_u8x4(in[i], mag & 0xffu, negative != 0, m);
  }
}

__global__ __launch_bounds__(kBlock) void brightness_byte_kernel(const uint8_t *in, uint8_t *out,
                                                                 size_t bytes, int channels,
                                                                 int delta, int all_channels) {
  size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= bytes) return;
  int ch = (int)(i % (size_t)channels);
  int v = in[i];
  if (all_channels || ch < 3) v = min(255, max(0, v + delta));
  out[i] = (uint8_t)v;
}

// ---------------------------------------------------------------------------
// Blur, RGBA streaming kernel.
//
// One wave owns a column strip of kStripPx output pixels and kR output rows.
// Lane l holds the 16-byte chunk of pixels [x0 + 4l, x0 + 4l + 4) of each
// input row (each wave row is 1 KiB, aligned); lanes 0 and 63 also load the
// two pixels left and right of the strip (8 bytes each). Neighbouring columns
// cross lanes by DPP lane moves, no LDS.
// The wave walks down its strip one input row per step: the row is split
// into 16-bit lanes (R|B and G|A words) and added to the 5-row column sums
// (the halo pixels' sums alongside), the row leaving the window is
// subtracted, and the 5-pixel horizontal sum of the column sums is the
// 25-tap box sum of the output row two rows up. Rows are requested five
// steps ahead into a 5-slot ring of raw loads and kept, expanded, in a
// 5-slot ring of the window's rows; the loop is unrolled so the slots are
// static.
// ---------------------------------------------------------------------------

constexpr int kStripPx = 256;  // 64 lanes x 4 pixels
// threads per workgroup of the streaming blur: consecutive waves take
// consecutive strips of a band, so 8 waves on one CU sweep half of a band's
// 16 KiB rows together. Against 256 threads, launches interleaved in one
// process over 1 GiB of rotating buffers: 26.05 against 26.6 us (fused 26.4
// against 26.9); 1024 (a whole band per CU) 27.2, 64 and 128 27.2-27.5. A
// copy with the same rows, bands and sweep directions and no arithmetic
// took 24.7 (512) and 26.2 us (256), a flat copy of the same bytes 22.5 us:
// the gap to the copy is this access pattern, not the arithmetic.
constexpr int kBlurBlock = 512;

// SWAR brightness on packed RGBA words (direct kernel and byte paths).
struct Brightness {
  uint32_t mag, mask;
  bool negative, enabled;
  __device__ __forceinline__ uint32_t operator()(uint32_t p) const {
    return enabled ? brighten_u8x4(p, mag, negative, mask) : p;
  }
};

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef int16_t i16x2 __attribute__((ext_vector_type(2)));

// Brightness of the streaming kernel, applied to 16-bit lanes (values 0..255):
// kFuse 1 adds, min 255; kFuse 2 adds the two's complement, max 0 as signed.
// d_lo / d_hi hold delta per lane of the R|B and G|A words (0 for a channel
// left unchanged).
template <int kFuse>
__device__ __forceinline__ uint32_t brighten_lanes(uint32_t w, uint32_t d) {
  if (kFuse == 0) return w;
  const u16x2 sum = __builtin_bit_cast(u16x2, w) + __builtin_bit_cast(u16x2, d);
  if (kFuse == 1) return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(sum, u16x2{255, 255}));
  return __builtin_bit_cast(
      uint32_t, __builtin_elementwise_max(__builtin_bit_cast(i16x2, sum), i16x2{0, 0}));
}

// Whole-wave lane shifts by DPP (GFX9 wave_shr:1 / wave_shl:1): lane i gets
// lane i-1 (from_left) or lane i+1 (from_right); lane 0 (from_left) / lane
// 63 (from_right), which have no such neighbour, get `edge` (DPP with
// bound_ctrl off keeps the old value in a lane whose source is out of range)
__device__ __forceinline__ uint32_t from_left(uint32_t v, uint32_t edge) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)edge, (int)v, 0x138, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t from_right(uint32_t v, uint32_t edge) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)edge, (int)v, 0x130, 0xf, 0xf, false);
}

struct StreamArgs {
  const uint32_t *in;
  uint32_t *out;
  int width, height, strips_x, total_waves, xcd_blocks;
  uint32_t d_lo, d_hi;  // brightness deltas per 16-bit lane (R|B, G|A)
};

// Bytes of one output pixel from its 25-tap sums (lo word R|B, hi word G|A,
// each lane < 6400; in config mode the lanes already carry the +12 rounding
// bias). floor(s / 25) = (s * 671089) >> 24 exactly for s < 6400: 671089 /
// 2^24 exceeds 1/25 by < 2.2e-8, the product fits 32 bits and the quotient is
// its top byte, which v_perm gathers.
template <int kMode>
__device__ __forceinline__ uint32_t finish_pixel(uint32_t vl, uint32_t vh, uint32_t count) {
  if (kMode == SH_BLUR_CONFIG || count == 25) {
    const uint32_t r = __umul24(vl & 0xffffu, 671089u);
    const uint32_t b = __umul24(vl >> 16, 671089u);
    const uint32_t g = __umul24(vh & 0xffffu, 671089u);
    const uint32_t a = __umul24(vh >> 16, 671089u);
    const uint32_t rg = __builtin_amdgcn_perm(g, r, 0x0c0c0703u);
    const uint32_t ba = __builtin_amdgcn_perm(a, b, 0x07030c0cu);
    return rg | ba;
  }
  const uint32_t c0 = (vl & 0xffffu) / count, c2 = (vl >> 16) / count;
  const uint32_t c1 = (vh & 0xffffu) / count, c3 = (vh >> 16) / count;
  return c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
}

// One input row for this lane (a cached load: the band above and below read
// the same halo rows). The row index is wave-uniform (scalar), so the
// row address is scalar and each lane adds its column offset. Lanes whose
// chunk lies outside the image load a valid chunk nobody uses (the edge fix-up
// in hsum supplies the clamped or zero taps instead).

// This lane's 4 pixels of one input row as 16-bit lanes, brightened (kFuse);
// reference mode: rows outside the image contribute nothing.
template <int kMode, int kFuse>
__device__ __forceinline__ void expand_row(const u32x4 v, int y, int height, uint32_t e[8],
                                           uint32_t d_lo, uint32_t d_hi) {
  if (kMode == SH_BLUR_REFERENCE && (y < 0 || y >= height)) {
#pragma unroll
    for (int k = 0; k < 8; k++) e[k] = 0;
    return;
  }
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    e[2 * k] = brighten_lanes<kFuse>(__builtin_amdgcn_perm(0u, w[k], 0x0c020c00u), d_lo);
    e[2 * k + 1] = brighten_lanes<kFuse>(__builtin_amdgcn_perm(0u, w[k], 0x0c030c01u), d_hi);
  }
}

// Input rows y0 - 2 .. y0 + kR + 1 are loaded once per wave (kR + 4 loads
// for kR output rows), each 5 steps before its use. Loads and stores sit
// under no branch (clamped rows, buffer stores whose dropped lanes point
// past the resource), so the compiler's waits count them exactly and keep
// ~4 rows in flight; with branches around the halo loads and the stores it
// waited for all but ~5 operations, about one row. The halo rows are shared
// with the neighbouring bands through L2: odd bands sweep upwards, so two
// neighbours reach their shared rows together (both at the start or both at
// the end of the sweep; a band's bottom halo read at the end of a downward
// sweep would be long evicted from L2 by the time the band below started).
template <int kMode, int kFuse, int kR>
__global__ __launch_bounds__(kBlurBlock) void blur_rgba_rows_kernel(const StreamArgs a) {
  constexpr int kQ = 5;  // the window's rows
  // rows requested ahead of their use (7 and 9 measured slower: their
  // registers drop the kernel to 3 waves per SIMD)
  constexpr int kL = 5;
  int b = blockIdx.x;
  if (a.xcd_blocks) b = (b & 7) * a.xcd_blocks + (b >> 3);
  const int lane = threadIdx.x & 63;
  const int wi = b * (kBlurBlock / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wi >= a.total_waves) return;
  const int sx = wi % a.strips_x, band = wi / a.strips_x;
  const int x0 = sx * kStripPx;
  const int cx = x0 + 4 * lane;
  const int lx = min(cx, a.width - 4);
  const bool left_edge = cx == 0;
  const bool right_edge = cx + 4 == a.width;
  // halo pixels: lane 0 the two left of the strip, lane 63 the two right of it
  const int hx = lane == 0 ? max(x0 - 2, 0) : min(x0 + kStripPx, a.width - 2);
  const int y0 = band * kR;
  // load j of the sweep reads row ys + dy * j
  const int dy = (band & 1) ? -1 : 1;
  const int ys = (band & 1) ? y0 + kR + 1 : y0 - 2;
  // stores through a buffer resource over this band's output rows: lanes
  // past the image's right edge and rows past its bottom get an offset
  // beyond the resource, which the hardware drops, so no branch guards them.
  // The whole offset (lane + row) is the per-lane one and the scalar offset
  // is the constant 0: with the row in a scalar offset register the compiler
  // inserts no wait state between a 16-byte store and the next write of its
  // data registers (the ISA documents none for that form), and on gfx950
  // such a store has then, now and then, taken the overwritten value in
  // lanes 12..15 of each row of 16 lanes (bank 3) of its first register.
  const bool writer = cx < a.width;
  const int out_rows = min(kR, a.height - y0);
  const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      a.out + (size_t)y0 * (size_t)a.width, 0, out_rows * a.width * 4, 0x00020000);
  // per-lane part of a store's offset (2^31 and above: past the resource)
  const uint32_t out_lane = writer ? (uint32_t)cx * 4u : 0x80000000u;
  // loads through a buffer resource over the rows this band reads (clamped
  // into the image): the row's offset is a scalar, the lane's a constant,
  // so a row costs no vector address arithmetic
  const int yb = max(y0 - 2, 0), ye = min(y0 + kR + 2, a.height);
  const __amdgpu_buffer_rsrc_t in_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t *>(a.in) + (size_t)yb * (size_t)a.width, 0, (ye - yb) * a.width * 4,
      0x00020000);
  // a wave that does not touch the image's left or right edge skips the
  // edge rule (a wave-uniform branch around eight selects per row)
  const bool edge_wave = x0 == 0 || x0 + kStripPx >= a.width;

  int cxk[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int x = cx + k;
    cxk[k] = min(x + 2, a.width - 1) - max(x - 2, 0) + 1;
  }
  const uint32_t bias = kMode == SH_BLUR_CONFIG ? 0x000c000cu : 0u;
  uint32_t vs[8], hs[4];
#pragma unroll
  for (int k = 0; k < 8; k++) vs[k] = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) hs[k] = 0;

  // every lane loads, so the loads' count is fixed (no branch); lanes 1..62
  // read lane 0's two pixels (one address for the whole group: all 64 lanes
  // at their own addresses measured 0.8 us slower)
  const int hxl = lane == 63 ? hx : __builtin_amdgcn_readfirstlane(hx);
  auto row_offset = [&](int y) -> int {
    const int cy = min(max(y, 0), a.height - 1);
    return __builtin_amdgcn_readfirstlane((cy - yb) * a.width * 4);
  };
  auto load_row = [&](int y) -> u32x4 {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(in_rsrc, lx * 4,
                                                                           row_offset(y), 0));
  };
  auto load_halo = [&](int y) -> u32x2 {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(in_rsrc, hxl * 4,
                                                                          row_offset(y), 0));
  };
  auto expand_halo = [&](const u32x2 v, int y, uint32_t e[4]) {
    if (kMode == SH_BLUR_REFERENCE && (y < 0 || y >= a.height)) {
#pragma unroll
      for (int k = 0; k < 4; k++) e[k] = 0;
      return;
    }
    const uint32_t w[2] = {v.x, v.y};
#pragma unroll
    for (int k = 0; k < 2; k++) {
      e[2 * k] = brighten_lanes<kFuse>(__builtin_amdgcn_perm(0u, w[k], 0x0c020c00u), a.d_lo);
      e[2 * k + 1] = brighten_lanes<kFuse>(__builtin_amdgcn_perm(0u, w[k], 0x0c030c01u), a.d_hi);
    }
  };

  // raw[j % 5]: row j's load in flight (requested 5 steps before its use);
  // ex[j % 5]: row j expanded to 16-bit lanes, kept until it leaves the
  // window 5 steps later (re-expanding the leaving row cost ~20 of the ~140
  // vector instructions per row, and the kernel is bound by them)
  u32x4 raw[kL];
  u32x2 hraw[kL];
  uint32_t ex[kQ][8], exh[kQ][4];
#pragma unroll
  for (int i = 0; i < kL && i < kR + 4; i++) {
    raw[i] = load_row(ys + dy * i);
    hraw[i] = load_halo(ys + dy * i);
  }
#pragma unroll
  for (int i = 0; i < kR + 4; i++) {
    uint32_t e[8], eh[4];
    expand_row<kMode, kFuse>(raw[i % kL], ys + dy * i, a.height, e, a.d_lo, a.d_hi);
    expand_halo(hraw[i % kL], ys + dy * i, eh);
    if (i + kL < kR + 4) {  // the slot is free: request the row kL steps ahead
      raw[i % kL] = load_row(ys + dy * (i + kL));
      hraw[i % kL] = load_halo(ys + dy * (i + kL));
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      vs[k] += e[k];
      if (i >= kQ) vs[k] -= ex[i % kQ][k];
      ex[i % kQ][k] = e[k];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      hs[k] += eh[k];
      if (i >= kQ) hs[k] -= exh[i % kQ][k];
      exh[i % kQ][k] = eh[k];
    }
    if (i >= 4) {
      const int y = ys + dy * (i - 2), row = y - y0;  // the window's centre row
      // columns cx-2, cx-1 and cx+4, cx+5: neighbours' sums, the halo sums
      // at the strip's ends, the edge rule at the image's
      uint32_t lo[8], hi[8];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        lo[k + 2] = vs[2 * k];
        hi[k + 2] = vs[2 * k + 1];
      }
      // (the lane moves run in every lane first: a move under a branch would
      // read an inactive neighbour)
      // (lane 0 and lane 63 take the halo sums in the same DPP moves)
      lo[0] = from_left(lo[4], hs[0]);
      lo[1] = from_left(lo[5], hs[2]);
      hi[0] = from_left(hi[4], hs[1]);
      hi[1] = from_left(hi[5], hs[3]);
      lo[6] = from_right(lo[2], hs[0]);
      lo[7] = from_right(lo[3], hs[2]);
      hi[6] = from_right(hi[2], hs[1]);
      hi[7] = from_right(hi[3], hs[3]);
      if (!edge_wave) {
      } else if (kMode == SH_BLUR_CONFIG) {
        lo[0] = left_edge ? lo[2] : lo[0];
        lo[1] = left_edge ? lo[2] : lo[1];
        hi[0] = left_edge ? hi[2] : hi[0];
        hi[1] = left_edge ? hi[2] : hi[1];
        lo[6] = right_edge ? lo[5] : lo[6];
        lo[7] = right_edge ? lo[5] : lo[7];
        hi[6] = right_edge ? hi[5] : hi[6];
        hi[7] = right_edge ? hi[5] : hi[7];
      } else {
        lo[0] = left_edge ? 0u : lo[0];
        lo[1] = left_edge ? 0u : lo[1];
        hi[0] = left_edge ? 0u : hi[0];
        hi[1] = left_edge ? 0u : hi[1];
        lo[6] = right_edge ? 0u : lo[6];
        lo[7] = right_edge ? 0u : lo[7];
        hi[6] = right_edge ? 0u : hi[6];
        hi[7] = right_edge ? 0u : hi[7];
      }
      uint32_t h[8];
#pragma unroll
      for (int part = 0; part < 2; part++) {
        const uint32_t *q = part ? hi : lo;
        const uint32_t u34 = q[3] + q[4];
        const uint32_t s = q[2] + u34, t = u34 + q[5];
        h[0 + part] = s + q[0] + q[1] + bias;
        h[2 + part] = s + q[1] + q[5] + bias;
        h[4 + part] = t + q[2] + q[6] + bias;
        h[6 + part] = t + q[6] + q[7] + bias;
      }
      {
        const uint32_t ry = kMode == SH_BLUR_CONFIG
                                ? 5u
                                : (uint32_t)(min(y + 2, a.height - 1) - max(y - 2, 0) + 1);
        u32x4 o;
        o.x = finish_pixel<kMode>(h[0], h[1], ry * cxk[0]);
        o.y = finish_pixel<kMode>(h[2], h[3], ry * cxk[1]);
        o.z = finish_pixel<kMode>(h[4], h[5], ry * cxk[2]);
        o.w = finish_pixel<kMode>(h[6], h[7], ry * cxk[3]);
        // rows past the image's bottom land past the resource's end too
        __builtin_amdgcn_raw_buffer_store_b128(
            o, out_rsrc, (int)(out_lane + (uint32_t)(row * a.width * 4)), 0, 2);  // 2: nt
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Layout adapters (bitmap BGR(A) <-> the blur test's RGBA / RGB byte images).
// One pixel per thread, rows by blockIdx.y: byte gathers, one 4-byte store
// per pixel on the RGBA side.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void bgr_to_rgba_kernel(const uint8_t *__restrict__ src, int bpp,
                                                             size_t src_stride,
                                                             uint32_t *__restrict__ dst, int width) {
  const int x = blockIdx.x * kBlock + threadIdx.x, y = blockIdx.y;
  if (x >= width) return;
  const uint8_t *p = src + (size_t)y * src_stride + (size_t)x * bpp;
  dst[(size_t)y * width + x] = (uint32_t)p[2] | ((uint32_t)p[1] << 8) | ((uint32_t)p[0] << 16);
}

__global__ __launch_bounds__(kBlock) void rgb_to_bgr_kernel(const uint8_t *__restrict__ src,
                                                            uint8_t *__restrict__ dst, int width,
                                                            size_t dst_stride) {
  const int x = blockIdx.x * kBlock + threadIdx.x, y = blockIdx.y;
  if (x >= width) return;
  const uint8_t *p = src + ((size_t)y * width + x) * 3;
  uint8_t *q = dst + (size_t)y * dst_stride + (size_t)x * 3;
  q[0] = p[2];
  q[1] = p[1];
  q[2] = p[0];
}

// ---------------------------------------------------------------------------
// Blur, direct kernel for any channel count / width (one pixel per thread).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void blur_direct_kernel(const uint8_t *__restrict__ in,
                                                             uint8_t *__restrict__ out, int width,
                                                             int height, int channels, int mode,
                                                             int fuse, int delta,
                                                             int all_channels) {
  const long long pix = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (pix >= (long long)width * height) return;
  const int x = (int)(pix % width), y = (int)(pix / width);
  const size_t stride = (size_t)width * channels;
  for (int ch = 0; ch < channels; ch++) {
    const bool adjust = fuse && (all_channels || ch < 3);
    int sum = 0, count = 0;
    for (int ky = -2; ky <= 2; ky++) {
      int ny = y + ky;
      if (mode == SH_BLUR_CONFIG) {
        ny = min(max(ny, 0), height - 1);
      } else if (ny < 0 || ny >= height) {
        continue;
      }
      for (int kx = -2; kx <= 2; kx++) {
        int nx = x + kx;
        if (mode == SH_BLUR_CONFIG) {
          nx = min(max(nx, 0), width - 1);
        } else if (nx < 0 || nx >= width) {
          continue;
        }
        int v = in[(size_t)ny * stride + (size_t)nx * channels + ch];
        if (adjust) v = min(255, max(0, v + delta));
        sum += v;
        count++;
      }
    }
    const int r = mode == SH_BLUR_CONFIG ? (sum + 12) / 25 : sum / count;
    out[(size_t)y * stride + (size_t)x * channels + ch] = (uint8_t)r;
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

Brightness make_brightness(bool enabled, int channels, int delta, int all_channels) {
  Brightness br;
  br.enabled = enabled;
  br.negative = delta < 0;
  const uint32_t m = (uint32_t)(delta < 0 ? -delta : delta);
  br.mag = m * 0x01010101u;
  br.mask = (channels == 4 && !all_channels) ? 0x00ffffffu : 0xffffffffu;
  return br;
}

// Output rows per wave: 16 make 16 x 256 = 4096 waves on 4096 x 4096, one
// round at 4 waves per SIMD (measured 29.1 us against 31.3 us with 8 rows,
// two rounds).
constexpr int kBlurRows = 16;

template <int kMode, int kR>
void launch_rows_fuse(hipStream_t s, const StreamArgs &a, int fuse) {
  const int blocks = a.xcd_blocks * 8;
  if (fuse == 1)
    blur_rgba_rows_kernel<kMode, 1, kR><<<blocks, kBlurBlock, 0, s>>>(a);
  else if (fuse == 2)
    blur_rgba_rows_kernel<kMode, 2, kR><<<blocks, kBlurBlock, 0, s>>>(a);
  else
    blur_rgba_rows_kernel<kMode, 0, kR><<<blocks, kBlurBlock, 0, s>>>(a);
}

template <int kRowsPerWave>
void launch_blur_stream(hipStream_t s, const uint32_t *in, uint32_t *out, int width, int height,
                        int mode, bool fuse, int delta, int all_channels) {
  StreamArgs a;
  a.in = in;
  a.out = out;
  a.width = width;
  a.height = height;
  a.strips_x = (width + kStripPx - 1) / kStripPx;
  const int bands = (height + kRowsPerWave - 1) / kRowsPerWave;
  a.total_waves = a.strips_x * bands;
  // padded to a multiple of 8 workgroups (the extra waves exit at once) so
  // that every XCD gets an equal contiguous range of bands
  const int blocks = ((a.total_waves + kBlurBlock / 64 - 1) / (kBlurBlock / 64) + 7) / 8 * 8;
  a.xcd_blocks = blocks / 8;
  int f = 0;
  a.d_lo = a.d_hi = 0;
  if (fuse && delta != 0) {
    f = delta > 0 ? 1 : 2;
    const uint32_t d = (uint32_t)(uint16_t)(int16_t)delta;  // lane value, two's complement
    a.d_lo = d | (d << 16);                                 // R and B
    a.d_hi = d | (all_channels ? d << 16 : 0u);             // G, and A only if asked
  }
  if (mode == SH_BLUR_CONFIG)
    launch_rows_fuse<SH_BLUR_CONFIG, kRowsPerWave>(s, a, f);
  else
    launch_rows_fuse<SH_BLUR_REFERENCE, kRowsPerWave>(s, a, f);
}

}  // namespace

hipError_t launch_brightness_u8(hipStream_t s, const uint8_t *in, uint8_t *out, size_t bytes,
                                int channels, int delta, int all_channels) {
  if (aligned16(in) && aligned16(out)) {
    const Brightness br = make_brightness(true, channels, delta, all_channels);
    const size_t per_block = (size_t)kBlock * kBrUnroll;
    size_t grid = (bytes / 16 + per_block - 1) / per_block;
    if (grid == 0) grid = 1;
    brightness_vec_kernel<<<(unsigned)grid, kBlock, 0, s>>>(in, out, bytes, br.mag,
                                                            br.negative ? 1 : 0, br.mask);
  } else {
    brightness_byte_kernel<<<(unsigned)((bytes + kBlock - 1) / kBlock), kBlock, 0, s>>>(
        in, out, bytes, channels, delta, all_channels);
  }
  return hipGetLastError();
}

hipError_t launch_blur5_u8(hipStream_t s, const uint8_t *in, uint8_t *out, int width, int height,
                           int channels, int mode, bool fuse, int delta, int all_channels) {
  if (channels == 4 && width % 4 == 0 && aligned16(in) && aligned16(out)) {
    const uint32_t *in32 = reinterpret_cast<const uint32_t *>(in);
    uint32_t *out32 = reinterpret_cast<uint32_t *>(out);
    launch_blur_stream<kBlurRows>(s, in32, out32, width, height, mode, fuse, delta, all_channels);
  } else {
    const long long pixels = (long long)width * height;
    blur_direct_kernel<<<(unsigned)((pixels + kBlock - 1) / kBlock), kBlock, 0, s>>>(
        in, out, width, height, channels, mode, fuse ? 1 : 0, delta, all_channels);
  }
  return hipGetLastError();
}

hipError_t launch_bgr_to_rgba_u8(hipStream_t s, const uint8_t *src, int bpp, size_t src_stride,
                                 uint32_t *dst, int width, int height) {
  if (width > 0 && height > 0)
    bgr_to_rgba_kernel<<<dim3((width + kBlock - 1) / kBlock, height), kBlock, 0, s>>>(
        src, bpp, src_stride, dst, width);
  return hipGetLastError();
}

hipError_t launch_rgb_to_bgr_u8(hipStream_t s, const uint8_t *src, uint8_t *dst, int width,
                                int height, size_t dst_stride) {
  if (width > 0 && height > 0)
    rgb_to_bgr_kernel<<<dim3((width + kBlock - 1) / kBlock, height), kBlock, 0, s>>>(
        src, dst, width, dst_stride);
  return hipGetLastError();
}

}  // namespace sh
