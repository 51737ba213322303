// Image kernels on interleaved 8-bit pixels: AdjustBrightness
// (Assembly.Tests/BlurPerformanceTests.cs:287-294) and the 5x5 box blur in
// both semantics (config: clamp-to-edge, (sum + 12) / 25; reference:
// BlurInteriorPixel / BlurEdgePixel at :85-141, in-bounds taps, sum / count),
// plus brightness fused into the blur's tile load.
//
// RGBA fast path (channels == 4, width % 4 == 0, 16-byte aligned buffers):
//  - a workgroup of 256 threads owns a 256 x 32 pixel output tile and stages
//    the (256 + 8) x (32 + 4) input pixels (halo included, coordinates clamped
//    or zero-padded by mode) in LDS with 16-byte global loads, all issued
//    before the barrier;
//  - each thread then produces a 4 x 8 block of output pixels: the four
//    channels are split into two words of 16-bit lanes (R|B and G|A), the
//    horizontal 5-sums slide along the row and the vertical 5-sums slide
//    down the 12 staged rows; a 25-tap sum (<= 6375) fits a 16-bit lane;
//  - each output row of a thread is one 16-byte store.
//  - Workgroup ids are remapped so that each XCD (ids round-robin over 8 XCDs)
//    gets a contiguous band of tiles: the halo rows a tile shares with its
//    neighbours then hit the same L2.
// Any other shape takes a direct kernel (one pixel per thread, taps read
// through the cache), which is exact for every channel count and mode.
#include <hip/hip_runtime.h>

#include "common.h"
#include "swar.h"

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
// Blur, RGBA tile kernel.
// ---------------------------------------------------------------------------

constexpr int kTileW = 256;             // output pixels per tile row
constexpr int kTileH = 32;              // output rows per tile
constexpr int kLdsW = kTileW + 8;       // staged columns: x0 - 4 .. x0 + 259
constexpr int kLdsH = kTileH + 4;       // staged rows: y0 - 2 .. y0 + 33
constexpr int kChunksPerRow = kLdsW / 4;
constexpr int kRowsPerThread = 8;       // 256 threads = 64 column groups x 4 row groups

struct Brightness {
  uint32_t mag, mask;
  bool negative, enabled;
  __device__ __forceinline__ uint32_t operator()(uint32_t p) const {
    return enabled ? brighten_u8x4(p, mag, negative, mask) : p;
  }
};

template <int kMode>
__global__ __launch_bounds__(kBlock) void blur_rgba_tile_kernel(const uint32_t *__restrict__ in,
                                                                uint32_t *__restrict__ out,
                                                                int width, int height,
                                                                int tiles_x, int tiles_total,
                                                                Brightness br) {
  __shared__ __attribute__((aligned(16))) uint32_t tile[kLdsH][kLdsW];

  // XCD-aware tile order: blocks b, b+8, b+16 ... run on one XCD; give that
  // XCD a contiguous run of row-major tiles.
  int b = blockIdx.x;
  int t = b;
  if ((tiles_total & 7) == 0) t = (b & 7) * (tiles_total >> 3) + (b >> 3);
  const int tx = t % tiles_x, ty = t / tiles_x;
  const int x0 = tx * kTileW, y0 = ty * kTileH;

  // ---- stage input + halo ----
  for (int idx = threadIdx.x; idx < kLdsH * kChunksPerRow; idx += kBlock) {
    const int r = idx / kChunksPerRow, j = idx - r * kChunksPerRow;
    const int gy = y0 - 2 + r;
    const int gx = x0 - 4 + 4 * j;
    u32x4 v;
    const bool row_in = gy >= 0 && gy < height;
    if (kMode == SH_BLUR_CONFIG) {
      const int cy = min(max(gy, 0), height - 1);
      const uint32_t *row = in + (size_t)cy * width;
      if (gx >= 0 && gx + 3 < width) {
        v = *reinterpret_cast<const u32x4 *>(row + gx);
      } else {  // chunk fully left or right of the image (width % 4 == 0)
        const uint32_t p = row[gx < 0 ? 0 : width - 1];
        v = u32x4{p, p, p, p};
      }
      v.x = br(v.x); v.y = br(v.y); v.z = br(v.z); v.w = br(v.w);
    } else {
      if (row_in && gx >= 0 && gx + 3 < width) {
        v = *reinterpret_cast<const u32x4 *>(in + (size_t)gy * width + gx);
        v.x = br(v.x); v.y = br(v.y); v.z = br(v.z); v.w = br(v.w);
      } else {
        v = u32x4{0, 0, 0, 0};  // out-of-bounds taps add nothing
      }
    }
    *reinterpret_cast<u32x4 *>(&tile[r][4 * j]) = v;
  }
  __syncthreads();

  // ---- 4 x 8 output block per thread ----
  const int cg = threadIdx.x & 63;       // column group: pixels 4*cg .. 4*cg+3
  const int rg = threadIdx.x >> 6;       // row group: rows 8*rg .. 8*rg+7
  const int ox = x0 + 4 * cg;
  const int oy0 = y0 + kRowsPerThread * rg;
  if (ox >= width || oy0 >= height) return;

  // horizontal sums, two 16-bit-lane words (R|B, G|A) per output pixel
  uint32_t hs[kRowsPerThread + 4][4][2];
#pragma unroll
  for (int rr = 0; rr < kRowsPerThread + 4; rr++) {
    const uint32_t *row = &tile[kRowsPerThread * rg + rr][4 * cg];
    // staged cols 4cg+2 .. 4cg+9 feed output pixels 4cg+4 .. 4cg+7
    const u32x2 a = *reinterpret_cast<const u32x2 *>(row + 2);
    const u32x4 m = *reinterpret_cast<const u32x4 *>(row + 4);
    const u32x2 c = *reinterpret_cast<const u32x2 *>(row + 8);
    const uint32_t p[8] = {a.x, a.y, m.x, m.y, m.z, m.w, c.x, c.y};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      lo[k] = p[k] & 0x00ff00ffu;
      hi[k] = (p[k] >> 8) & 0x00ff00ffu;
    }
    uint32_t sl = lo[0] + lo[1] + lo[2] + lo[3] + lo[4];
    uint32_t sh = hi[0] + hi[1] + hi[2] + hi[3] + hi[4];
    hs[rr][0][0] = sl;
    hs[rr][0][1] = sh;
#pragma unroll
    for (int k = 1; k < 4; k++) {
      sl += lo[k + 4] - lo[k - 1];
      sh += hi[k + 4] - hi[k - 1];
      hs[rr][k][0] = sl;
      hs[rr][k][1] = sh;
    }
  }

  // per-pixel tap counts for the reference mode's border pixels
  int cx[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int x = ox + k;
    cx[k] = min(x + 2, width - 1) - max(x - 2, 0) + 1;
  }

#pragma unroll
  for (int r = 0; r < kRowsPerThread; r++) {
    const int y = oy0 + r;
    if (y >= height) break;
    const int ry = min(y + 2, height - 1) - max(y - 2, 0) + 1;
    uint32_t res[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t vl = hs[r][k][0] + hs[r + 1][k][0] + hs[r + 2][k][0] + hs[r + 3][k][0] +
                          hs[r + 4][k][0];
      const uint32_t vh = hs[r][k][1] + hs[r + 1][k][1] + hs[r + 2][k][1] + hs[r + 3][k][1] +
                          hs[r + 4][k][1];
      uint32_t c0 = vl & 0xffffu, c2 = vl >> 16, c1 = vh & 0xffffu, c3 = vh >> 16;
      if (kMode == SH_BLUR_CONFIG) {
        c0 = div25(c0 + 12); c1 = div25(c1 + 12); c2 = div25(c2 + 12); c3 = div25(c3 + 12);
      } else {
        const uint32_t cnt = (uint32_t)(ry * cx[k]);
        if (cnt == 25) {
          c0 = div25(c0); c1 = div25(c1); c2 = div25(c2); c3 = div25(c3);
        } else {
          c0 /= cnt; c1 /= cnt; c2 /= cnt; c3 /= cnt;
        }
      }
      res[k] = c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
    }
    *reinterpret_cast<u32x4 *>(out + (size_t)y * width + ox) =
        u32x4{res[0], res[1], res[2], res[3]};
  }
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
    const int tiles_x = (width + kTileW - 1) / kTileW;
    const int tiles_y = (height + kTileH - 1) / kTileH;
    const int total = tiles_x * tiles_y;
    const Brightness br = make_brightness(fuse, channels, delta, all_channels);
    const uint32_t *in32 = reinterpret_cast<const uint32_t *>(in);
    uint32_t *out32 = reinterpret_cast<uint32_t *>(out);
    if (mode == SH_BLUR_CONFIG)
      blur_rgba_tile_kernel<SH_BLUR_CONFIG>
          <<<total, kBlock, 0, s>>>(in32, out32, width, height, tiles_x, total, br);
    else
      blur_rgba_tile_kernel<SH_BLUR_REFERENCE>
          <<<total, kBlock, 0, s>>>(in32, out32, width, height, tiles_x, total, br);
  } else {
    const long long pixels = (long long)width * height;
    blur_direct_kernel<<<(unsigned)((pixels + kBlock - 1) / kBlock), kBlock, 0, s>>>(
        in, out, width, height, channels, mode, fuse ? 1 : 0, delta, all_channels);
  }
  return hipGetLastError();
}

}  // namespace sh
