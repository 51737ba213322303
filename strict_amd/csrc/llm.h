// Internal interface between the LLM decode kernels (llm_kernels.hip) and the
// model runner (llm.hip). Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace sh {

constexpr int kMaxBatch = 16;        // rows of the GEMV's MFMA A operand
constexpr int kMaxSplitChunk = 1024; // positions one attention workgroup may score
// Greedy argmax keys of the LM head, [kKeySlots][kKeyStride]: key of row b in
// slot s at keys[s * kKeyStride + b]; the row's token is the largest key over
// its slots. Workgroups finishing the head together spread their atomicMax
// over the slots (slot rows 256 bytes apart, on lines of their own): 2048
// workgroups on one address serialised ~9 ns each, 19 us of a GPT-2 head
// that streams its weights in 14 us.
constexpr int kKeySlots = 32;
constexpr int kKeyStride = 32;
static_assert(kKeyStride >= kMaxBatch, "a slot row holds every batch row");
// The model holds two such key sets of kKeySet keys each. A persistent
// layers kernel (one launch per step) of step number e reads this step's
// tokens from set (e - 1) & 1, its LM head writes set e & 1, and its
// workgroup 0 clears set (e - 1) & 1 after its last item (every workgroup
// has read the tokens by then), ready for step e + 1's head. The per-op path
// reads, clears and writes the set of the current step number, which it does
// not advance.
constexpr int kKeySet = kKeySlots * kKeyStride;

enum { kWeightFp8 = 0, kWeightFp16 = 1 };
enum { kProNone = 0, kProRms = 1, kProLayer = 2 };
enum { kEpiStore = 0, kEpiResidual = 1, kEpiSwiGLU = 2, kEpiGelu = 3, kEpiLogits = 4 };

// y[b][n] = (sum_k A[b][k] * W[n][k]) * scale[n] + bias[n], then the epilogue.
// A is fp16 activations (`act`, kProNone) or the fp32 residual stream `x`
// normalised per row (RMSNorm: x / sqrt(mean(x^2) + eps) * gamma; LayerNorm:
// (x - mean) / sqrt(var + eps) * gamma + beta), rounded to fp16.
struct GemvArgs {
  const uint8_t *w = nullptr;   // tiled weights, N rows (multiple of 16)
  const float *scale = nullptr; // per-row FP8 scales, or nullptr
  const float *bias = nullptr;  // per-row bias, or nullptr
  const float *x = nullptr;     // fp32 input rows (kProRms / kProLayer)
  int x_ld = 0;
  const uint16_t *act = nullptr;  // fp16 input rows (kProNone)
  int act_ld = 0;
  const float *gamma = nullptr, *beta = nullptr;
  float eps = 0.0f;
  int B = 0, K = 0, N = 0;
  int n_valid = 0;  // logits: columns >= n_valid are padding
  float *out = nullptr;      // fp32 output / residual rows
  uint16_t *out16 = nullptr; // fp16 output rows (SwiGLU, GELU)
  int out_ld = 0;
  unsigned long long *argmax = nullptr;  // logits: [kKeySlots][kKeyStride] argmax keys (atomicMax)
};

struct AttnArgs {
  const float *qkv = nullptr;  // [B][qkv_ld] fp32: q (heads*d) | k (kv_heads*d) | v
  int qkv_ld = 0;
  uint16_t *kcache = nullptr, *vcache = nullptr;  // this layer: [B][kv_heads][max_pos][d] fp16
  int max_pos = 0;
  const int *pos = nullptr;  // [B] position of the new token (= tokens already cached)
  const float *q_norm = nullptr, *k_norm = nullptr;  // Qwen3 per-head RMSNorm gains [d]
  float eps = 0.0f;
  const float *rope = nullptr;      // Qwen3 RoPE of this step: [B][2][d/2] (cos, sin)
  float scale = 1.0f;               // 1 / sqrt(d)
  int heads = 0, kv_heads = 0;
  int splits = 1;                   // grid.x
  int chunk = 16;                   // positions per split (multiple of 16)
  float *part = nullptr;            // [B][heads][splits][d + 2]
  int *counters = nullptr;          // [B][kv_heads], zero between launches
  uint16_t *out = nullptr;          // [B][out_ld] fp16 head outputs
  int out_ld = 0;
};

struct EmbedArgs {
  unsigned long long *keys = nullptr;  // [kKeySlots][kKeyStride] argmax keys (token = ~low word)
  unsigned long long *keys_clear = nullptr;  // key set whose row b the kernel zeroes for
                                             // this step's LM head (may be `keys`)
  int *lens = nullptr;                 // [B] tokens cached so far (advanced here)
  int *pos = nullptr;                  // [B] position of this step's token (written here)
  int *hist = nullptr;                 // [B][hist_len] token history
  int hist_len = 0;
  float *x = nullptr;                  // [B][x_ld] fp32 residual stream
  int x_ld = 0, K = 0, vocab = 0, max_pos = 0;
  int fp8_head = 0;
  const uint8_t *head8 = nullptr;      // FP8 tiled head (Qwen3, tied embedding)
  const float *head_scale = nullptr;
  const uint16_t *head16 = nullptr;    // fp16 tiled head (GPT-2, tied wte)
  const uint16_t *wpe = nullptr;       // GPT-2 positions [max_pos][K] fp16
  const float *inv_freq = nullptr;     // Qwen3 RoPE inverse frequencies [half]
  float *rope = nullptr;               // [B][2][half]: cos, sin of pos * inv_freq
  int half = 0;
  unsigned *epoch = nullptr;           // step counter of the decode-layers kernel (+1 here)
};

// ---- persistent decode-layers kernel (Qwen3, FP8 weights, head_dim 128) ----

// Device pointers of one layer, read by the kernel from a device array.
struct LayerPtrs {
  const uint8_t *wqkv, *wo, *wup, *wdown;  // FP8 tiled (gate/up tiles interleaved)
  const float *sqkv, *so, *sup, *sdown;    // per-row scales
  const float *norm1, *norm2, *q_norm, *k_norm;
  uint16_t *kcache;  // [max_batch][kv_heads][max_pos][128] fp16
  uint16_t *vcache;  // transposed: [max_batch][kv_heads][128][vt_stride] fp16
};

// Everything the kernel hands between workgroups within a step travels in
// 8-byte cells of device memory (payload word, then the producing
// step and layer's tag word; see decode_layers.hip). Cell buffers:
//   x0c   [kMaxBatch][H]          layer output x (fp32), read by the next layer
//   x1c   [kMaxBatch][H]          x_mid after attention (fp32)
//   qkvc  [kMaxBatch][qkv_n]      q | k | v (fp32)
//   partc [kMaxBatch][heads][64][132] attention partials (acc[128], max, sum)
//   attnc [kMaxBatch][heads * 64] merged attention output, two fp16 per cell
//   actc  [kMaxBatch][inter / 2]  SwiGLU output, two fp16 per cell
constexpr int kMaxDecodeLayers = 63;  // tags hold the layer in 6 bits
struct LayersArgs {
  const LayerPtrs *layers = nullptr;  // [n_layers]
  int n_layers = 0, B = 0, H = 0, heads = 0, kv_heads = 0, inter = 0, qkv_n = 0;
  int max_pos = 0, splits = 1, chunk = 16;
  int vt_stride = 0;                   // positions per V^T cache row: max_pos rounded up to 16
  float eps = 1e-6f, scale = 1.0f;     // RMSNorm epsilon, attention 1 / sqrt(d)
  const int *pos = nullptr;            // [B] this step's position (embed kernel; at
                                       // batch 1, the row lengths, which the kernel advances)
  const float *rope = nullptr;         // [B][128]: cos | sin (embed kernel)
  unsigned *epoch = nullptr;           // this step's number (embed kernel; at batch 1,
                                       // the previous one, which the kernel advances)
  // batch 1 (one item per workgroup and phase; decode_layers_folds_embed):
  // the kernel is the step's only launch. It reads the token from key set
  // keys_in, embeds it (row of the tied FP8 head times its scale), computes
  // RoPE's factors from inv_freq, and its workgroup 0 stores the step
  // number, the row's length, position (pos_out) and history entry after
  // its last item and clears keys_in's row 0
  unsigned long long *keys_in = nullptr;
  int *lens = nullptr, *pos_out = nullptr, *hist = nullptr;
  int hist_len = 0, vocab = 0;
  const float *inv_freq = nullptr;
  float *x_in = nullptr;               // [kMaxBatch][H] plain fp32: first layer's input
                                       // (embed kernel), last layer's output
  uint64_t *x0c = nullptr, *x1c = nullptr, *qkvc = nullptr, *partc = nullptr;
  uint64_t *attnc = nullptr, *actc = nullptr;
  unsigned *err = nullptr;             // set when a wait timed out (sticky); bit 1: an
                                       // XCD id outside 0..7 in XCD-local mode
  unsigned long long spin_ticks = 0;   // wall-clock ticks a wait may take
  int lds_misc = 0;                    // byte offset of the small LDS scratch words
  // batch 1: KV head h's QKV, attention and merge items on the workgroups
  // of XCD h, their cells stored into that XCD's L2 (decode_layers_xcd_ok
  // must hold)
  int xcd = 0;
  // final RMSNorm + LM head inside the kernel (steps with logits; head_on 0:
  // the kernel ends with the last layer)
  int head_on = 0;
  const uint8_t *head_w = nullptr;     // FP8 tiled [head_tiles * 16][H]
  const float *head_scale = nullptr;   // per row
  const float *final_g = nullptr;      // final RMSNorm gains [H]
  int head_tiles = 0, n_valid = 0;     // 16-row tiles; columns that are real tokens
  float *logits = nullptr;             // [B][logits_ld]
  int logits_ld = 0;
  unsigned long long *keys = nullptr;  // [kKeySlots][kKeyStride] the key set this step's LM
                                       // head writes (row b zeroed by the embed kernel)
};

// Model shapes the kernel is instantiated for (16-byte weight loads per lane
// of the qkv, o, gate/up and down items) and the query heads per KV head.
// Returns false for any other shape (the runner then keeps per-op kernels).
bool decode_layers_supported(int layers, int H, int heads, int kv_heads, int head_dim, int inter);
// Whether the launch of a at `grid` workgroups runs the batch-1 kernel, which
// embeds the step's token itself (LayersArgs::keys_in ..).
bool decode_layers_folds_embed(const LayersArgs &a, int grid);
// Whether a (batch 1, `grid` workgroups) fits the XCD-local placement: eight
// KV heads, one per XCD, each with grid / 8 QKV tiles (its query heads' q,
// its k and v) and grid / 8 attention splits.
bool decode_layers_xcd_ok(const LayersArgs &a, int grid);
// Most attention splits per (row, KV head) the shape's kernel merges.
int decode_layers_max_splits(int H, int heads, int kv_heads, int inter);
// Cells of the attention-partial buffer partc.
size_t decode_layers_partial_cells(int heads);
size_t decode_layers_lds(int B, int H, int heads, int inter, int *misc_offset);
// Workgroups of the kernel resident per CU with `lds` bytes of LDS (>= 1 to use it).
hipError_t decode_layers_occupancy(const LayersArgs &a, size_t lds, int *blocks_per_cu);
#ifdef SH_DECODE_TRACE
// Diagnostic builds: copies the last step's phase timeline to the host.
hipError_t decode_layers_trace(void *dst, size_t bytes);
#endif
// Launch on stream s. The kernel needs all `grid` workgroups resident
// together. cooperative: HIP's cooperative launch, which guarantees it (and
// runs on a queue of its own, ~11 us to switch to and from it, ~20 us between
// two cooperative launches). Otherwise an ordinary launch: grid is at most one
// workgroup per CU of an occupancy >= 1 and stream order has drained this
// stream's earlier work, so the workgroups are resident together unless other
// streams or processes hold the CUs; then a wait times out, sets `err`, every
// later wait gives up at once and the kernel ends with the step reported failed.
hipError_t launch_decode_layers(hipStream_t s, const LayersArgs &a, int grid, size_t lds,
                                bool cooperative);

// ---- persistent GPT-2 layers kernel (fp16 weights, head_dim 64, batch 1) ----

// Device pointers of one GPT-2 layer, read by the kernel from a device array.
struct Gpt2LayerPtrs {
  const uint16_t *wqkv, *wo, *wfc, *wproj;  // fp16 tiled
  const float *bqkv, *bo, *bfc, *bproj;     // biases
  const float *ln1_g, *ln1_b, *ln2_g, *ln2_b;
  uint16_t *kcache, *vcache;                // [max_batch][heads][max_pos][64] fp16 (row 0)
};
constexpr int kGpt2Splits = 4;    // attention splits per head
constexpr int kGpt2PStride = 68;  // cells per attention partial: acc[64], max, sum, pad
// Cell buffers (exchange.h): x0c [H] layer output, x1c [H] x_mid, qkvc [3 H],
// partc [heads][4][68] attention partials, actc [inter / 2] GELU output (two
// fp16 per cell).
struct Gpt2Args {
  const Gpt2LayerPtrs *layers = nullptr;  // [n_layers]
  int n_layers = 0, H = 0, heads = 0, inter = 0, qkv_n = 0, max_pos = 0;
  int chunk = 16;                    // positions per attention split
  float eps = 1e-5f, scale = 0.125f;  // LayerNorm epsilon, attention 1 / sqrt(64)
  // the step's embedding and bookkeeping (the kernel is the step's only
  // launch): the token from key set (epoch) & 1, the position lens[0]; at the
  // end workgroup 0 stores epoch + 1, lens[0] + 1, pos[0] and the history
  // entry, and clears that key set
  unsigned *epoch = nullptr;         // steps run so far (this step is epoch + 1)
  int *lens = nullptr;               // [1] tokens cached so far
  int *pos = nullptr;                // [1] this step's position (written at the end)
  int *hist = nullptr;               // [hist_len] token history
  int hist_len = 0, vocab = 0;
  const uint16_t *wpe = nullptr;     // positions [max_pos][H] fp16 (token rows: head_w)
  float *x_in = nullptr;             // [H] last layer's output
  uint64_t *x0c = nullptr, *x1c = nullptr, *qkvc = nullptr, *partc = nullptr, *actc = nullptr;
  unsigned *err = nullptr;           // set when a wait timed out (sticky); bit 1: an
                                     // XCD id outside 0..7 in XCD-local mode
  unsigned long long spin_ticks = 0;  // wall-clock ticks a wait may take
  // head h's QKV tiles and attention splits on the workgroups of XCD h % 8,
  // the q / k / v cells stored into that XCD's L2 (gpt2_layers_xcd_ok must
  // hold)
  int xcd = 0;
  // final LayerNorm + LM head inside the kernel (steps with logits)
  int head_on = 0;
  const uint16_t *head_w = nullptr;  // fp16 tiled [head_tiles * 16][H] (tied embedding)
  const float *final_g = nullptr, *final_b = nullptr;
  int head_tiles = 0, n_valid = 0;   // 16-row tiles; columns that are real tokens
  float *logits = nullptr;           // [logits_ld]
  unsigned long long *keys = nullptr;  // [2][kKeySet] the two greedy argmax key sets
};
// Shapes the kernel is built for (GPT-2 small and a reduced test shape),
// max_pos <= 1024, and a grid of `grid` workgroups holding every phase's items.
bool gpt2_layers_supported(int layers, int H, int heads, int head_dim, int inter, int max_pos,
                           int grid);
int gpt2_layers_chunk(int max_pos);
// Whether the XCD-local placement fits: with `grid` workgroups, grid / 8 per
// XCD, the heads h and h + 8 of XCD h % 8 with their QKV tiles and splits.
bool gpt2_layers_xcd_ok(const Gpt2Args &a, int grid);
size_t gpt2_layers_partial_cells(int heads);
hipError_t gpt2_layers_occupancy(const Gpt2Args &a, int *blocks_per_cu);
// Ordinary launch on stream s; needs its `grid` workgroups resident together
// (one per CU), as the Qwen3 decode-layers kernel.
hipError_t launch_gpt2_layers(hipStream_t s, const Gpt2Args &a, int grid);
#ifdef SH_GPT2_TRACE
// Diagnostic builds: the last step's marks, [256][16][12] wall-clock ticks.
hipError_t gpt2_layers_trace(void *dst, size_t bytes);
#endif

// Lets every GEMV instantiation use up to 160 KiB of dynamic LDS (current device).
hipError_t prepare_gemv_kernels();
hipError_t launch_gemv(hipStream_t s, const GemvArgs &a, int weight_type, int pro, int epi,
                       int max_grid);
hipError_t launch_attention(hipStream_t s, const AttnArgs &a, int head_dim, int group, bool qwen,
                            int batch);
hipError_t launch_embed(hipStream_t s, const EmbedArgs &a, int batch);
// fp16 out16[b] = norm(x[b]) (pro = kProRms or kProLayer), K <= 4096.
hipError_t launch_norm_rows(hipStream_t s, const GemvArgs &a, int pro);
hipError_t launch_quantize_e4m3_tiled(hipStream_t s, const float *w, int N, int K,
                                      int interleave_rows, uint8_t *q, float *scales,
                                      bool tiled);
hipError_t launch_pack_e4m3_tiles(hipStream_t s, const uint8_t *q, int N, int K, uint8_t *out);
hipError_t launch_tile_f16(hipStream_t s, const float *w, int N, int K, int interleave_rows,
                           uint16_t *out);
hipError_t launch_fill_normal(hipStream_t s, float *out, size_t n, uint64_t seed, float mean,
                              float stddev);
hipError_t launch_fill_value(hipStream_t s, float *out, size_t n, float v);
hipError_t launch_f32_to_f16(hipStream_t s, const float *in, uint16_t *out, size_t n);

}  // namespace sh
