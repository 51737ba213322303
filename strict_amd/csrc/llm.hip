// LLM model runner behind sh_llm_*: owns the weights, KV cache and work
// buffers of one decoder on a context's device and enqueues a decode step as
//   embed -> per layer [norm+QKV GEMV, attention, O GEMV + residual,
//                       norm+up GEMV (SwiGLU / GELU), down GEMV + residual]
//         -> final norm + LM head GEMV with argmax
// on the context's stream. Every per-step quantity (tokens, positions, argmax
// keys) lives in device memory, so a step of the per-op path is captured once
// per batch size as a HIP graph and replayed. With the decode-layers kernel
// a step is two eager launches, embed and the layers kernel, which also runs
// the final norm and LM head (not captured: with STRICT_HIP_LLM_COOP=1 the
// layers kernel is a cooperative launch, which stream capture does not take).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "common.h"
#include "llm.h"

using namespace sh;

namespace {

struct Linear {
  uint8_t *w = nullptr;  // tiled (FP8 bytes or fp16)
  float *scale = nullptr;
  float *bias = nullptr;
  int N = 0, K = 0;          // N = rows as stored (gate/up: 2 * intermediate)
  int interleave = 0;        // gate/up: intermediate (tiles interleaved), else 0
  size_t w_bytes = 0;
};

struct Layer {
  float *norm1_g = nullptr, *norm1_b = nullptr, *norm2_g = nullptr, *norm2_b = nullptr;
  float *q_norm = nullptr, *k_norm = nullptr;
  Linear qkv, o, up, down;
  uint16_t *kcache = nullptr, *vcache = nullptr;
};

// Splits of the context per (sequence, KV head): about 512 workgroups in all
// (two per CU; at the Qwen3 shape and b = 1, 64 splits of <= 80 positions up
// to 5120 tokens, so each workgroup's K and V fit one batch of loads issued
// together), at least enough that no split exceeds kMaxSplitChunk positions,
// at most 64 (the merge kernel's limit).
// Splits per (row, KV head) of the per-op attention kernel: as few as keep a
// split within kMaxSplitChunk positions. Each kernel of a per-op step costs
// ~4-6 us whatever its size (measured on GPT-2's step), so one split per
// head up to 1024 positions, which writes the head's output directly, beats
// many short splits plus the merge kernel they need.
int attention_splits(int batch, int kv_heads, int max_pos) {
  (void)batch;
  (void)kv_heads;
  const int s = (max_pos + kMaxSplitChunk - 1) / kMaxSplitChunk;
  return s < 1 ? 1 : s;
}

}  // namespace

struct sh_llm {
  sh_ctx *ctx = nullptr;
  sh_llm_config cfg{};
  bool qwen = true;
  int wtype = kWeightFp8;
  int qkv_n = 0, vocab_pad = 0;
  std::vector<void *> allocs;
  std::vector<Layer> layers;
  Linear head;
  float *final_g = nullptr, *final_b = nullptr;
  uint16_t *wpe = nullptr;
  float *inv_freq = nullptr;
  // per-step state
  float *x = nullptr, *qkv = nullptr, *logits = nullptr, *part = nullptr, *rope = nullptr;
  uint16_t *attn = nullptr, *act = nullptr;
  int *counters = nullptr, *lens = nullptr, *pos = nullptr, *hist = nullptr;
  unsigned long long *keys = nullptr;
  int batch = 0, splits = 1, chunk = 16, steps_done = 0;
  uint16_t *hnorm = nullptr;  // final-norm output rows (fp16) fed to the LM head
  size_t kv_layer_elems = 0;
  hipGraphExec_t graph[2] = {nullptr, nullptr};
  int graph_batch[2] = {-1, -1};
  unsigned long long *graph_keys[2] = {nullptr, nullptr};  // key set a graph was captured on
  bool use_graphs = true;  // STRICT_HIP_LLM_GRAPHS=0: enqueue every step eagerly
  // persistent decode-layers kernel (Qwen3 shapes it is built for;
  // STRICT_HIP_LLM_LAYERS=0 keeps the per-op kernels)
  bool layers_kernel = false;
  bool head_in_layers = false;  // final norm + LM head inside the layers kernel
  bool coop_layers = false;     // cooperative launch of the layers kernel
  LayersArgs la{};
  int layers_grid = 0;
  size_t layers_lds = 0;
  unsigned *epoch = nullptr;
  // the device's step number (*epoch), mirrored: one more per step of a
  // layers kernel; its parity selects the current key set
  unsigned epoch_host = 0;
  bool xcd_off = false;  // a step failed in XCD-local placement: none (either layers
                         // kernel) from the next reset on
  // persistent GPT-2 layers kernel (batch 1; other batches keep the per-op
  // kernels, which share its cache layout)
  bool gpt2_kernel = false;
  Gpt2Args ga{};
  int gpt2_grid = 0;
};

namespace {

int llm_alloc(sh_llm *m, size_t bytes, void **p) {
  *p = nullptr;
  if (bytes == 0) return SH_OK;
  SH_HIP_TRY(hipMalloc(p, bytes));
  m->allocs.push_back(*p);
  // registered with the context so that sh_upload / sh_download / typed ops
  // accept the model's tensors
  int rc = sh_register_external(m->ctx, *p, bytes);
  if (rc != SH_OK) return rc;
  SH_HIP_TRY(hipMemsetAsync(*p, 0, bytes, stream_of(m->ctx)));
  return SH_OK;
}

template <class T>
int alloc_n(sh_llm *m, size_t n, T **p) {
  void *v = nullptr;
  int rc = llm_alloc(m, n * sizeof(T), &v);
  *p = static_cast<T *>(v);
  return rc;
}

int alloc_linear(sh_llm *m, Linear &l, int N, int K, int interleave, bool bias) {
  l.N = N;
  l.K = K;
  l.interleave = interleave;
  l.w_bytes = (size_t)N * K * (m->wtype == kWeightFp8 ? 1 : 2);
  int rc = llm_alloc(m, l.w_bytes, reinterpret_cast<void **>(&l.w));
  if (rc == SH_OK && m->wtype == kWeightFp8) rc = alloc_n(m, (size_t)N, &l.scale);
  if (rc == SH_OK && bias) rc = alloc_n(m, (size_t)N, &l.bias);
  return rc;
}

int fill(sh_llm *m, float *p, size_t n, float v) {
  if (!p) return SH_OK;
  const hipError_t e = launch_fill_value(stream_of(m->ctx), p, n, v);
  return e == hipSuccess ? SH_OK : hip_fail(e, "fill");
}

// Quantizes / tiles a device fp32 [N][K] matrix (logical order) into `l`.
int store_linear(sh_llm *m, Linear &l, const float *w) {
  hipStream_t s = stream_of(m->ctx);
  hipError_t e = m->wtype == kWeightFp8
                     ? launch_quantize_e4m3_tiled(s, w, l.N, l.K, l.interleave, l.w, l.scale, true)
                     : launch_tile_f16(s, w, l.N, l.K, l.interleave, reinterpret_cast<uint16_t *>(l.w));
  return e == hipSuccess ? SH_OK : hip_fail(e, "storing a linear layer");
}

Linear *find_linear(sh_llm *m, const std::string &name, int layer) {
  if (name == "head") return &m->head;
  if (layer < 0 || layer >= (int)m->layers.size()) return nullptr;
  Layer &L = m->layers[layer];
  if (name == "qkv") return &L.qkv;
  if (name == "o") return &L.o;
  if (name == (m->qwen ? "gate_up" : "fc")) return &L.up;
  if (name == (m->qwen ? "down" : "proj")) return &L.down;
  return nullptr;
}

// The key set of the current step number: the one the next step reads its
// tokens from, and the one the last step's LM head wrote.
unsigned long long *key_set(sh_llm *m, unsigned ahead = 0) {
  return m->keys + (size_t)((m->epoch_host + ahead) & 1u) * kKeySet;
}

int enqueue_step(sh_llm *m, bool logits) {
  const sh_llm_config &c = m->cfg;
  hipStream_t s = stream_of(m->ctx);
  const int B = m->batch, H = c.hidden, d = c.head_dim;
  const int pro = m->qwen ? kProRms : kProLayer;

  const bool gpt2_layers = m->gpt2_kernel && B == 1;
  // keys this step reads its tokens from and its LM head writes: a layers
  // kernel step advances the step number, so the head writes the other set
  unsigned long long *keys_in = key_set(m);
  unsigned long long *keys_out = key_set(m, m->layers_kernel || gpt2_layers ? 1 : 0);
  if (gpt2_layers) {
    // the GPT-2 layers kernel embeds the token itself: one launch per step
    m->ga.head_on = logits ? 1 : 0;
    SH_HIP_TRY(launch_gpt2_layers(s, m->ga, m->gpt2_grid));
    m->epoch_host++;
    return SH_OK;
  }
  EmbedArgs e;
  e.keys = keys_in;
  e.keys_clear = keys_out;
  e.lens = m->lens;
  e.pos = m->pos;
  e.hist = m->hist;
  e.hist_len = c.max_positions;
  e.x = m->x;
  e.x_ld = H;
  e.K = H;
  e.vocab = c.vocab;
  e.max_pos = c.max_positions;
  e.fp8_head = m->qwen ? 1 : 0;
  e.head8 = m->head.w;
  e.head_scale = m->head.scale;
  e.head16 = reinterpret_cast<const uint16_t *>(m->head.w);
  e.wpe = m->wpe;
  e.inv_freq = m->inv_freq;
  e.rope = m->rope;
  e.half = d / 2;
  float *x_final = m->x;  // the layers kernel reads and writes m->x too
  if (m->layers_kernel) e.epoch = m->epoch;
  // at batch 1 the decode-layers kernel embeds the token itself (one launch)
  const bool fold = m->layers_kernel && decode_layers_folds_embed(m->la, m->layers_grid);
  if (!fold) SH_HIP_TRY(launch_embed(s, e, B));

  if (m->layers_kernel) {
    LayersArgs &la = m->la;
    la.head_on = logits && m->head_in_layers ? 1 : 0;
    la.keys = keys_out;
    la.keys_in = keys_in;
    la.pos = fold ? m->lens : m->pos;  // at batch 1 the kernel reads (and advances) the lengths
    SH_HIP_TRY(launch_decode_layers(s, la, m->layers_grid, m->layers_lds, m->coop_layers));
    m->epoch_host++;
  }
  for (Layer &L : m->layers) {
    if (m->layers_kernel) break;  // every layer ran in the kernel above
    GemvArgs g;
    g.w = L.qkv.w;
    g.scale = L.qkv.scale;
    g.bias = L.qkv.bias;
    g.x = m->x;
    g.x_ld = H;
    g.gamma = L.norm1_g;
    g.beta = L.norm1_b;
    g.eps = c.norm_eps;
    g.B = B;
    g.K = H;
    g.N = L.qkv.N;
    g.out = m->qkv;
    g.out_ld = m->qkv_n;
    SH_HIP_TRY(launch_gemv(s, g, m->wtype, pro, kEpiStore, 0));

    AttnArgs a;
    a.qkv = m->qkv;
    a.qkv_ld = m->qkv_n;
    a.kcache = L.kcache;
    a.vcache = L.vcache;
    a.max_pos = c.max_positions;
    a.pos = m->pos;
    a.q_norm = L.q_norm;
    a.k_norm = L.k_norm;
    a.eps = c.norm_eps;
    a.rope = m->rope;
    a.scale = 1.0f / std::sqrt((float)d);
    a.heads = c.heads;
    a.kv_heads = c.kv_heads;
    a.splits = m->splits;
    a.chunk = m->chunk;
    a.part = m->part;
    a.counters = m->counters;
    a.out = m->attn;
    a.out_ld = c.heads * d;
    SH_HIP_TRY(launch_attention(s, a, d, c.heads / c.kv_heads, m->qwen, B));

    GemvArgs o;
    o.w = L.o.w;
    o.scale = L.o.scale;
    o.bias = L.o.bias;
    o.act = m->attn;
    o.act_ld = c.heads * d;
    o.B = B;
    o.K = c.heads * d;
    o.N = L.o.N;
    o.out = m->x;
    o.out_ld = H;
    SH_HIP_TRY(launch_gemv(s, o, m->wtype, kProNone, kEpiResidual, 0));

    GemvArgs u;
    u.w = L.up.w;
    u.scale = L.up.scale;
    u.bias = L.up.bias;
    u.x = m->x;
    u.x_ld = H;
    u.gamma = L.norm2_g;
    u.beta = L.norm2_b;
    u.eps = c.norm_eps;
    u.B = B;
    u.K = H;
    u.N = L.up.N;
    u.out16 = m->act;
    u.out_ld = c.intermediate;
    SH_HIP_TRY(launch_gemv(s, u, m->wtype, pro, m->qwen ? kEpiSwiGLU : kEpiGelu, 0));

    GemvArgs dn;
    dn.w = L.down.w;
    dn.scale = L.down.scale;
    dn.bias = L.down.bias;
    dn.act = m->act;
    dn.act_ld = c.intermediate;
    dn.B = B;
    dn.K = c.intermediate;
    dn.N = L.down.N;
    dn.out = m->x;
    dn.out_ld = H;
    SH_HIP_TRY(launch_gemv(s, dn, m->wtype, kProNone, kEpiResidual, 0));
  }

  if (logits && !(m->layers_kernel && m->head_in_layers)) {
    GemvArgs nrm;
    nrm.x = x_final;
    nrm.x_ld = H;
    nrm.gamma = m->final_g;
    nrm.beta = m->final_b;
    nrm.eps = c.norm_eps;
    nrm.B = B;
    nrm.K = H;
    nrm.out16 = m->hnorm;
    nrm.out_ld = H;
    SH_HIP_TRY(launch_norm_rows(s, nrm, pro));
    GemvArgs h;
    h.w = m->head.w;
    h.scale = m->head.scale;
    h.act = m->hnorm;
    h.act_ld = H;
    h.B = B;
    h.K = H;
    h.N = m->head.N;
    h.n_valid = c.vocab;
    h.out = m->logits;
    h.out_ld = m->vocab_pad;
    h.argmax = keys_out;
    // grid-striding over the head's tiles (one tile per workgroup ran the
    // fp16 GPT-2 head at 2 TB/s)
    SH_HIP_TRY(launch_gemv(s, h, m->wtype, kProNone, kEpiLogits, 2048));
  }
  return SH_OK;
}

// Sets up the decode-layers kernel when the model's shape and the device
// allow it; otherwise the per-op kernels stay in use.
int setup_layers_kernel(sh_llm *m) {
  const sh_llm_config &c = m->cfg;
  const char *env = getenv("STRICT_HIP_LLM_LAYERS");
  if (env && env[0] == '0') return SH_OK;
  if (!m->qwen ||
      !decode_layers_supported(c.layers, c.hidden, c.heads, c.kv_heads, c.head_dim,
                               c.intermediate))
    return SH_OK;
  const int dev = device_of(m->ctx);
  int coop = 0, cus = 0, clock_khz = 0;
  SH_HIP_TRY(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
  SH_HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  SH_HIP_TRY(hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeWallClockRate, dev));
  if (!coop || cus <= 0 || clock_khz <= 0) return SH_OK;
  LayersArgs &a = m->la;
  a.n_layers = c.layers;
  a.H = c.hidden;
  a.heads = c.heads;
  a.kv_heads = c.kv_heads;
  a.inter = c.intermediate;
  a.qkv_n = m->qkv_n;
  a.max_pos = c.max_positions;
  a.vt_stride = (c.max_positions + 15) / 16 * 16;
  a.eps = c.norm_eps;
  a.scale = 1.0f / std::sqrt((float)c.head_dim);
  a.pos = m->pos;
  a.rope = m->rope;
  // what the batch-1 kernel reads and writes in place of the embed kernel
  a.lens = m->lens;
  a.pos_out = m->pos;
  a.hist = m->hist;
  a.hist_len = c.max_positions;
  a.vocab = c.vocab;
  a.inv_freq = m->inv_freq;
  a.spin_ticks = (unsigned long long)clock_khz * 50;  // 50 ms per wait
  // the kernel's merge limit must leave splits of at most kMaxSplitChunk positions
  const int max_sp = decode_layers_max_splits(c.hidden, c.heads, c.kv_heads, c.intermediate);
  if ((c.max_positions + kMaxSplitChunk - 1) / kMaxSplitChunk > max_sp) return SH_OK;
  int misc = 0;
  const size_t lds = decode_layers_lds(c.max_batch, c.hidden, c.heads, c.intermediate, &misc);
  int per_cu = 0;
  SH_HIP_TRY(decode_layers_occupancy(a, lds, &per_cu));
  if (per_cu < 1) return SH_OK;
  int rc;
  const size_t MB = kMaxBatch;
  // ordinary device memory: every access to these is an agent-scope atomic,
  // which the memory model keeps coherent across the XCDs' separate L2s
  if ((rc = alloc_n(m, MB * c.hidden, &a.x0c)) || (rc = alloc_n(m, MB * c.hidden, &a.x1c)) ||
      (rc = alloc_n(m, MB * m->qkv_n, &a.qkvc)) ||
      (rc = alloc_n(m, decode_layers_partial_cells(c.heads), &a.partc)) ||
      (rc = alloc_n(m, MB * c.heads * c.head_dim / 2, &a.attnc)) ||
      (rc = alloc_n(m, MB * c.intermediate / 2, &a.actc)) || (rc = alloc_n(m, 64, &a.err)) ||
      (rc = alloc_n(m, 64, &m->epoch)))
    return rc;
  a.x_in = m->x;
  LayerPtrs *dl = nullptr;
  if ((rc = alloc_n(m, (size_t)c.layers, &dl))) return rc;
  std::vector<LayerPtrs> hl(c.layers);
  for (int i = 0; i < c.layers; i++) {
    const Layer &L = m->layers[i];
    hl[i] = LayerPtrs{L.qkv.w, L.o.w, L.up.w, L.down.w, L.qkv.scale, L.o.scale, L.up.scale,
                      L.down.scale, L.norm1_g, L.norm2_g, L.q_norm, L.k_norm, L.kcache, L.vcache};
  }
  SH_HIP_TRY(hipMemcpyAsync(dl, hl.data(), hl.size() * sizeof(LayerPtrs), hipMemcpyHostToDevice,
                            stream_of(m->ctx)));
  SH_HIP_TRY(hipStreamSynchronize(stream_of(m->ctx)));
  a.layers = dl;
  a.epoch = m->epoch;
  // the final norm and LM head run inside the kernel on steps with logits
  // (STRICT_HIP_LLM_HEAD=0: separate kernels, as the per-op path)
  const char *he = getenv("STRICT_HIP_LLM_HEAD");
  m->head_in_layers = !(he && he[0] == '0');
  // ordinary launches by default (back to back with the embed kernel on one
  // queue); STRICT_HIP_LLM_COOP=1: cooperative launches
  const char *co = getenv("STRICT_HIP_LLM_COOP");
  m->coop_layers = co && co[0] == '1';
  a.head_w = m->head.w;
  a.head_scale = m->head.scale;
  a.final_g = m->final_g;
  a.head_tiles = m->head.N / 16;
  a.n_valid = c.vocab;
  a.logits = m->logits;
  a.logits_ld = m->vocab_pad;
  m->layers_grid = cus;
  m->layers_kernel = true;
  return SH_OK;
}

// Sets up the persistent GPT-2 layers kernel (batch 1) when the model's
// shape and the device allow it; otherwise the per-op kernels stay in use.
int setup_gpt2_kernel(sh_llm *m) {
  const sh_llm_config &c = m->cfg;
  const char *env = getenv("STRICT_HIP_LLM_LAYERS");
  if (env && env[0] == '0') return SH_OK;
  const int dev = device_of(m->ctx);
  int cus = 0, clock_khz = 0;
  SH_HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  SH_HIP_TRY(hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeWallClockRate, dev));
  if (m->qwen || cus <= 0 || clock_khz <= 0 ||
      !gpt2_layers_supported(c.layers, c.hidden, c.heads, c.head_dim, c.intermediate,
                             c.max_positions, cus) ||
      c.kv_heads != c.heads)
    return SH_OK;
  Gpt2Args &a = m->ga;
  a.n_layers = c.layers;
  a.H = c.hidden;
  a.heads = c.heads;
  a.inter = c.intermediate;
  a.qkv_n = m->qkv_n;
  a.max_pos = c.max_positions;
  a.chunk = gpt2_layers_chunk(c.max_positions);
  a.eps = c.norm_eps;
  a.scale = 1.0f / std::sqrt((float)c.head_dim);
  a.lens = m->lens;
  a.pos = m->pos;
  a.hist = m->hist;
  a.hist_len = c.max_positions;
  a.vocab = c.vocab;
  a.wpe = m->wpe;
  a.spin_ticks = (unsigned long long)clock_khz * 50;  // 50 ms per wait
  int per_cu = 0;
  SH_HIP_TRY(gpt2_layers_occupancy(a, &per_cu));
  if (per_cu < 1) return SH_OK;
  int rc;
  if ((rc = alloc_n(m, (size_t)c.hidden, &a.x0c)) || (rc = alloc_n(m, (size_t)c.hidden, &a.x1c)) ||
      (rc = alloc_n(m, (size_t)m->qkv_n, &a.qkvc)) ||
      (rc = alloc_n(m, gpt2_layers_partial_cells(c.heads), &a.partc)) ||
      (rc = alloc_n(m, (size_t)c.intermediate / 2, &a.actc)) || (rc = alloc_n(m, 64, &a.err)) ||
      (!m->epoch && (rc = alloc_n(m, 64, &m->epoch))))
    return rc;
  a.x_in = m->x;
  a.epoch = m->epoch;
  Gpt2LayerPtrs *dl = nullptr;
  if ((rc = alloc_n(m, (size_t)c.layers, &dl))) return rc;
  std::vector<Gpt2LayerPtrs> hl(c.layers);
  for (int i = 0; i < c.layers; i++) {
    const Layer &L = m->layers[i];
    hl[i] = Gpt2LayerPtrs{reinterpret_cast<const uint16_t *>(L.qkv.w),
                          reinterpret_cast<const uint16_t *>(L.o.w),
                          reinterpret_cast<const uint16_t *>(L.up.w),
                          reinterpret_cast<const uint16_t *>(L.down.w),
                          L.qkv.bias, L.o.bias, L.up.bias, L.down.bias,
                          L.norm1_g, L.norm1_b, L.norm2_g, L.norm2_b, L.kcache, L.vcache};
  }
  SH_HIP_TRY(hipMemcpyAsync(dl, hl.data(), hl.size() * sizeof(Gpt2LayerPtrs),
                            hipMemcpyHostToDevice, stream_of(m->ctx)));
  SH_HIP_TRY(hipStreamSynchronize(stream_of(m->ctx)));
  a.layers = dl;
  a.head_w = reinterpret_cast<const uint16_t *>(m->head.w);
  a.final_g = m->final_g;
  a.final_b = m->final_b;
  a.head_tiles = m->head.N / 16;
  a.n_valid = c.vocab;
  a.logits = m->logits;
  a.keys = m->keys;  // both sets: the kernel picks them by the step number
  m->gpt2_grid = cus;
  m->gpt2_kernel = true;
  return SH_OK;
}

void drop_graphs(sh_llm *m) {
  for (int i = 0; i < 2; i++) {
    if (m->graph[i]) (void)hipGraphExecDestroy(m->graph[i]);
    m->graph[i] = nullptr;
    m->graph_batch[i] = -1;
  }
}

}  // namespace

extern "C" {

SH_API int sh_quantize_e4m3(sh_ctx *ctx, const float *W, int N, int K, uint8_t *q,
                            float *scales) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if (N < 0 || K <= 0 || K % 64 != 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "quantize: need N >= 0 and K a positive multiple of 64 (N=%d K=%d)", N, K);
  if (N == 0) return SH_OK;
  if ((rc = check_range(ctx, W, (size_t)N * K * 4, "W")) != SH_OK) return rc;
  if ((rc = check_range(ctx, q, (size_t)N * K, "q")) != SH_OK) return rc;
  if ((rc = check_range(ctx, scales, (size_t)N * 4, "scales")) != SH_OK) return rc;
  hipError_t e = launch_quantize_e4m3_tiled(stream_of(ctx), W, N, K, 0, q, scales, false);
  return e == hipSuccess ? SH_OK : hip_fail(e, "quantize_e4m3");
}

SH_API int sh_pack_e4m3_tiles(sh_ctx *ctx, const uint8_t *q, int N, int K, uint8_t *tiled) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if (N < 0 || N % 16 != 0 || K <= 0 || K % 64 != 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "pack: N must be a multiple of 16 and K of 64 (N=%d K=%d)", N, K);
  if (N == 0) return SH_OK;
  if ((rc = check_range(ctx, q, (size_t)N * K, "q")) != SH_OK) return rc;
  if ((rc = check_range(ctx, tiled, (size_t)N * K, "tiled")) != SH_OK) return rc;
  const hipError_t e = launch_pack_e4m3_tiles(stream_of(ctx), q, N, K, tiled);
  return e == hipSuccess ? SH_OK : hip_fail(e, "pack_e4m3_tiles");
}

SH_API int sh_gemv_w8a16(sh_ctx *ctx, const uint16_t *x, const uint8_t *w_tiled,
                         const float *scales, float *y, int batch, int K, int N) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if (batch < 1 || batch > kMaxBatch)
    return fail(SH_ERR_INVALID_ARGUMENT, "gemv batch %d outside 1..%d", batch, kMaxBatch);
  if (K <= 0 || K % 256 != 0 || N < 0 || N % 16 != 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "gemv: K must be a multiple of 256 and N of 16 (K=%d N=%d)", K, N);
  if (N == 0) return SH_OK;
  if ((rc = check_range(ctx, x, (size_t)batch * K * 2, "x")) != SH_OK) return rc;
  if ((rc = check_range(ctx, w_tiled, (size_t)N * K, "w_tiled")) != SH_OK) return rc;
  if ((rc = check_range(ctx, scales, (size_t)N * 4, "scales")) != SH_OK) return rc;
  if ((rc = check_range(ctx, y, (size_t)batch * N * 4, "y")) != SH_OK) return rc;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_tiled)) & 15)
    return fail(SH_ERR_INVALID_ARGUMENT, "x and w_tiled must be 16-byte aligned");
  static bool prepared = false;  // dynamic-LDS attributes (process-wide, first device)
  if (!prepared) {
    SH_HIP_TRY(prepare_gemv_kernels());
    prepared = true;
  }
  GemvArgs g;
  g.w = w_tiled;
  g.scale = scales;
  g.act = x;
  g.act_ld = K;
  g.B = batch;
  g.K = K;
  g.N = N;
  g.out = y;
  g.out_ld = N;
  const hipError_t e = launch_gemv(stream_of(ctx), g, kWeightFp8, kProNone, kEpiStore, 2048);
  return e == hipSuccess ? SH_OK : hip_fail(e, "gemv_w8a16");
}

SH_API int sh_llm_create(sh_ctx *ctx, const sh_llm_config *config, sh_llm **out) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  if (!config || !out) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = nullptr;
  const sh_llm_config c = *config;
  const bool qwen = c.arch == SH_LLM_QWEN3;
  if (c.arch != SH_LLM_QWEN3 && c.arch != SH_LLM_GPT2)
    return fail(SH_ERR_INVALID_ARGUMENT, "unknown architecture %d", c.arch);
  if (c.layers <= 0 || c.hidden <= 0 || c.heads <= 0 || c.kv_heads <= 0 || c.vocab <= 0 ||
      c.intermediate <= 0 || c.max_positions <= 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "model sizes must be positive");
  if (c.max_batch < 1 || c.max_batch > kMaxBatch)
    return fail(SH_ERR_INVALID_ARGUMENT, "max_batch must be 1..%d", kMaxBatch);
  if (c.heads % c.kv_heads != 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "heads %d not a multiple of kv_heads %d", c.heads, c.kv_heads);
  const int group = c.heads / c.kv_heads;
  const bool attn_ok = qwen ? (c.head_dim == 128 && (group == 1 || group == 2))
                            : ((c.head_dim == 64 || c.head_dim == 128) && group == 1);
  if (!attn_ok)
    return fail(SH_ERR_UNSUPPORTED, "attention kernel not built for head_dim %d, group %d (%s)",
                c.head_dim, group, qwen ? "qwen3" : "gpt2");
  // K of every GEMV must split into 4 waves of whole 16-byte tile loads
  const int kalign = qwen ? 256 : 128;
  const int ks[3] = {c.hidden, c.heads * c.head_dim, c.intermediate};
  for (int k : ks)
    if (k % kalign != 0)
      return fail(SH_ERR_UNSUPPORTED, "GEMV input width %d is not a multiple of %d", k, kalign);
  if (c.intermediate % 16 != 0 || c.hidden % 16 != 0)
    return fail(SH_ERR_UNSUPPORTED, "hidden and intermediate must be multiples of 16");
  if (c.max_positions > 65536) return fail(SH_ERR_INVALID_ARGUMENT, "max_positions > 65536");
  if (!qwen && c.hidden % 8 != 0) return fail(SH_ERR_UNSUPPORTED, "hidden must be a multiple of 8");

  auto *m = new sh_llm();
  m->ctx = ctx;
  m->cfg = c;
  m->qwen = qwen;
  m->wtype = qwen ? kWeightFp8 : kWeightFp16;
  m->qkv_n = (c.heads + 2 * c.kv_heads) * c.head_dim;
  {
    const char *g = getenv("STRICT_HIP_LLM_GRAPHS");
    m->use_graphs = !(g && g[0] == '0');
  }
  m->vocab_pad = (c.vocab + 15) / 16 * 16;
  const int B = c.max_batch, H = c.hidden, d = c.head_dim;
  // positions rounded up to 16: the decode-layers kernel keeps V transposed
  // with rows of that many positions
  m->kv_layer_elems = (size_t)B * c.kv_heads * ((c.max_positions + 15) / 16 * 16) * d;
  const int max_splits = attention_splits(1, c.kv_heads, c.max_positions);

  auto cleanup = [&](int status) {
    (void)hipStreamSynchronize(stream_of(ctx));
    for (void *p : m->allocs) {
      (void)sh_unregister_external(ctx, p);
      (void)hipFree(p);
    }
    delete m;
    return status;
  };
  m->layers.resize(c.layers);
  for (Layer &L : m->layers) {
    if ((rc = alloc_n(m, H, &L.norm1_g)) || (rc = alloc_n(m, H, &L.norm2_g))) return cleanup(rc);
    if (!qwen && ((rc = alloc_n(m, H, &L.norm1_b)) || (rc = alloc_n(m, H, &L.norm2_b))))
      return cleanup(rc);
    if (qwen && ((rc = alloc_n(m, d, &L.q_norm)) || (rc = alloc_n(m, d, &L.k_norm))))
      return cleanup(rc);
    const bool bias = !qwen;
    if ((rc = alloc_linear(m, L.qkv, m->qkv_n, H, 0, bias)) ||
        (rc = alloc_linear(m, L.o, H, c.heads * d, 0, bias)) ||
        (rc = alloc_linear(m, L.up, qwen ? 2 * c.intermediate : c.intermediate, H,
                           qwen ? c.intermediate : 0, bias)) ||
        (rc = alloc_linear(m, L.down, H, c.intermediate, 0, bias)))
      return cleanup(rc);
    if ((rc = alloc_n(m, m->kv_layer_elems, &L.kcache)) ||
        (rc = alloc_n(m, m->kv_layer_elems, &L.vcache)))
      return cleanup(rc);
  }
  if ((rc = alloc_linear(m, m->head, m->vocab_pad, H, 0, false))) return cleanup(rc);
  if ((rc = alloc_n(m, H, &m->final_g))) return cleanup(rc);
  if (!qwen && ((rc = alloc_n(m, H, &m->final_b)) ||
                (rc = alloc_n(m, (size_t)c.max_positions * H, &m->wpe))))
    return cleanup(rc);
  if (qwen) {
    if ((rc = alloc_n(m, d / 2, &m->inv_freq))) return cleanup(rc);
    if ((rc = alloc_n(m, (size_t)B * d, &m->rope))) return cleanup(rc);
    std::vector<float> f(d / 2);
    for (int i = 0; i < d / 2; i++)
      f[i] = (float)std::pow((double)c.rope_theta, -2.0 * i / (double)d);
    hipError_t e = hipMemcpyAsync(m->inv_freq, f.data(), f.size() * 4, hipMemcpyHostToDevice,
                                  stream_of(ctx));
    if (e == hipSuccess) e = hipStreamSynchronize(stream_of(ctx));
    if (e != hipSuccess) return cleanup(hip_fail(e, "uploading RoPE frequencies"));
  }
  if (c.hidden > 4096) return cleanup(fail(SH_ERR_UNSUPPORTED, "hidden %d > 4096", c.hidden));
  if ((rc = alloc_n(m, (size_t)B * H, &m->hnorm))) return cleanup(rc);
  if ((rc = alloc_n(m, (size_t)B * H, &m->x)) || (rc = alloc_n(m, (size_t)B * m->qkv_n, &m->qkv)) ||
      (rc = alloc_n(m, (size_t)B * c.heads * d, &m->attn)) ||
      (rc = alloc_n(m, (size_t)B * c.intermediate, &m->act)) ||
      (rc = alloc_n(m, (size_t)B * m->vocab_pad, &m->logits)) ||
      (rc = alloc_n(m, (size_t)B * c.heads * max_splits * (d + 2), &m->part)) ||
      (rc = alloc_n(m, (size_t)B * c.kv_heads, &m->counters)) ||
      (rc = alloc_n(m, (size_t)B, &m->lens)) || (rc = alloc_n(m, (size_t)B, &m->pos)) ||
      (rc = alloc_n(m, (size_t)B * c.max_positions, &m->hist)) ||
      (rc = alloc_n(m, (size_t)2 * kKeySet, &m->keys)))
    return cleanup(rc);
  // norm gains start at 1 (biases and weights at 0)
  for (Layer &L : m->layers) {
    if ((rc = fill(m, L.norm1_g, H, 1.0f)) || (rc = fill(m, L.norm2_g, H, 1.0f)) ||
        (rc = fill(m, L.q_norm, d, 1.0f)) || (rc = fill(m, L.k_norm, d, 1.0f)))
      return cleanup(rc);
  }
  if ((rc = fill(m, m->final_g, H, 1.0f))) return cleanup(rc);
  hipError_t e = prepare_gemv_kernels();
  if (e == hipSuccess) e = hipStreamSynchronize(stream_of(ctx));
  if (e != hipSuccess) return cleanup(hip_fail(e, "preparing the model"));
  if ((rc = setup_layers_kernel(m)) != SH_OK) return cleanup(rc);
  if ((rc = setup_gpt2_kernel(m)) != SH_OK) return cleanup(rc);
  *out = m;
  return SH_OK;
}

#ifdef SH_GPT2_TRACE
// Diagnostic builds only (-DSH_GPT2_TRACE): the GPT-2 layers kernel's marks
// of the last step, [256][16][12] wall-clock ticks.
SH_API int sh_debug_gpt2_trace(void *dst, size_t bytes) {
  SH_HIP_TRY(gpt2_layers_trace(dst, bytes));
  return SH_OK;
}
#endif

#ifdef SH_DECODE_TRACE
// Diagnostic builds only (-DSH_DECODE_TRACE): the decode-layers kernel's
// per-workgroup phase timeline of the last step, [2][256][32][24] wall-clock ticks.
SH_API int sh_debug_decode_trace(void *dst, size_t bytes) {
  SH_HIP_TRY(decode_layers_trace(dst, bytes));
  return SH_OK;
}
#endif

SH_API int sh_llm_destroy(sh_llm *m) {
  if (!m) return SH_OK;
  (void)hipSetDevice(device_of(m->ctx));
  (void)hipStreamSynchronize(stream_of(m->ctx));
  drop_graphs(m);
  for (void *p : m->allocs) {
    (void)sh_unregister_external(m->ctx, p);
    (void)hipFree(p);
  }
  delete m;
  return SH_OK;
}

SH_API int sh_llm_init_random(sh_llm *m, uint64_t seed, float stddev) {
  if (!m) return fail(SH_ERR_INVALID_ARGUMENT, "model is NULL");
  int rc = enter(m->ctx);
  if (rc != SH_OK) return rc;
  hipStream_t s = stream_of(m->ctx);
  size_t max_elems = (size_t)m->head.N * m->head.K;
  for (Layer &L : m->layers)
    for (Linear *l : {&L.qkv, &L.o, &L.up, &L.down})
      if ((size_t)l->N * l->K > max_elems) max_elems = (size_t)l->N * l->K;
  float *tmp = nullptr;
  SH_HIP_TRY(hipMalloc(&tmp, max_elems * sizeof(float)));
  uint64_t stream_id = seed * 1000003ull;
  auto gen = [&](Linear &l) -> int {
    hipError_t e = launch_fill_normal(s, tmp, (size_t)l.N * l.K, stream_id++, 0.0f, stddev);
    if (e != hipSuccess) return hip_fail(e, "fill_normal");
    return store_linear(m, l, tmp);
  };
  for (Layer &L : m->layers)
    for (Linear *l : {&L.qkv, &L.o, &L.up, &L.down})
      if ((rc = gen(*l)) != SH_OK) break;
  if (rc == SH_OK) {
    // head: only the real vocabulary rows are random, padding rows stay zero
    Linear real = m->head;
    real.N = m->cfg.vocab / 16 * 16;
    if ((rc = gen(real)) == SH_OK && real.N < m->head.N) {
      // the last partial tile: generate full rows, zero the padding rows
      const int n0 = real.N, rows = m->head.N - n0;
      hipError_t e = launch_fill_normal(s, tmp, (size_t)rows * m->head.K, stream_id++, 0.0f, stddev);
      if (e == hipSuccess)
        e = hipMemsetAsync(tmp + (size_t)(m->cfg.vocab - n0) * m->head.K, 0,
                           (size_t)(m->head.N - m->cfg.vocab) * m->head.K * 4, s);
      Linear last = m->head;
      last.N = 16;
      last.w = m->head.w + (size_t)n0 * m->head.K * (m->wtype == kWeightFp8 ? 1 : 2);
      last.scale = m->head.scale ? m->head.scale + n0 : nullptr;
      if (e != hipSuccess) rc = hip_fail(e, "head padding");
      else rc = store_linear(m, last, tmp);
    }
  }
  if (rc == SH_OK && m->wpe) {
    hipError_t e = launch_fill_normal(s, tmp, (size_t)m->cfg.max_positions * m->cfg.hidden,
                                      stream_id++, 0.0f, stddev);
    if (e == hipSuccess)
      e = launch_f32_to_f16(s, tmp, m->wpe, (size_t)m->cfg.max_positions * m->cfg.hidden);
    if (e != hipSuccess) rc = hip_fail(e, "wpe");
  }
  hipError_t e = hipStreamSynchronize(s);
  (void)hipFree(tmp);
  if (rc == SH_OK && e != hipSuccess) rc = hip_fail(e, "init_random");
  return rc;
}

SH_API int sh_llm_load_linear(sh_llm *m, const char *name, int layer, const float *W) {
  if (!m || !name) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  int rc = enter(m->ctx);
  if (rc != SH_OK) return rc;
  Linear *l = find_linear(m, name, layer);
  if (!l) return fail(SH_ERR_NOT_FOUND, "no linear '%s' in layer %d", name, layer);
  if ((rc = check_range(m->ctx, W, (size_t)l->N * l->K * 4, "W")) != SH_OK) return rc;
  return store_linear(m, *l, W);
}

SH_API int sh_llm_tensor(sh_llm *m, const char *name, int layer, void **ptr, size_t *bytes) {
  if (!m || !name || !ptr || !bytes) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  const sh_llm_config &c = m->cfg;
  std::string n(name);
  *ptr = nullptr;
  *bytes = 0;
  auto set = [&](void *p, size_t b) {
    *ptr = p;
    *bytes = p ? b : 0;
    return p ? SH_OK : fail(SH_ERR_NOT_FOUND, "tensor '%s' does not exist in this model", name);
  };
  const size_t dot = n.find('.');
  if (dot != std::string::npos) {
    const std::string base = n.substr(0, dot), field = n.substr(dot + 1);
    Linear *l = find_linear(m, base, layer);
    if (l) {
      if (field == "w") return set(l->w, l->w_bytes);
      if (field == "scale") return set(l->scale, (size_t)l->N * 4);
      if (field == "bias") return set(l->bias, (size_t)l->N * 4);
    }
  }
  if (n == "logits") return set(m->logits, (size_t)c.max_batch * m->vocab_pad * 4);
  if (n == "hist") return set(m->hist, (size_t)c.max_batch * c.max_positions * 4);
  if (n == "lens") return set(m->lens, (size_t)c.max_batch * 4);
  if (n == "final.g") return set(m->final_g, (size_t)c.hidden * 4);
  if (n == "final.b") return set(m->final_b, (size_t)c.hidden * 4);
  if (n == "wpe") return set(m->wpe, (size_t)c.max_positions * c.hidden * 2);
  if (n == "inv_freq") return set(m->inv_freq, (size_t)c.head_dim / 2 * 4);
  // present only when the decode-layers kernel runs the layers
  if (n == "layers.err")
    return set(m->layers_kernel ? m->la.err : m->gpt2_kernel ? m->ga.err : nullptr, 4);
  if (layer < 0 || layer >= c.layers)
    return fail(SH_ERR_NOT_FOUND, "tensor '%s' layer %d not found", name, layer);
  Layer &L = m->layers[layer];
  if (n == "norm1.g") return set(L.norm1_g, (size_t)c.hidden * 4);
  if (n == "norm1.b") return set(L.norm1_b, (size_t)c.hidden * 4);
  if (n == "norm2.g") return set(L.norm2_g, (size_t)c.hidden * 4);
  if (n == "norm2.b") return set(L.norm2_b, (size_t)c.hidden * 4);
  if (n == "q_norm") return set(L.q_norm, (size_t)c.head_dim * 4);
  if (n == "k_norm") return set(L.k_norm, (size_t)c.head_dim * 4);
  if (n == "kcache") return set(L.kcache, m->kv_layer_elems * 2);
  if (n == "vcache") return set(L.vcache, m->kv_layer_elems * 2);
  return fail(SH_ERR_NOT_FOUND, "tensor '%s' not found", name);
}

SH_API int sh_llm_reset(sh_llm *m, int batch) {
  if (!m) return fail(SH_ERR_INVALID_ARGUMENT, "model is NULL");
  int rc = enter(m->ctx);
  if (rc != SH_OK) return rc;
  if (batch < 1 || batch > m->cfg.max_batch)
    return fail(SH_ERR_INVALID_ARGUMENT, "batch %d outside 1..%d", batch, m->cfg.max_batch);
  hipStream_t s = stream_of(m->ctx);
  SH_HIP_TRY(hipMemsetAsync(m->lens, 0, (size_t)m->cfg.max_batch * 4, s));
  SH_HIP_TRY(hipMemsetAsync(m->keys, 0, (size_t)2 * kKeySet * 8, s));
  if (m->epoch) {
    // the device's step number to the mirror's: a layers kernel whose wait
    // timed out may have ended before storing it (tags only ever grow)
    SH_HIP_TRY(hipMemcpyAsync(m->epoch, &m->epoch_host, 4, hipMemcpyHostToDevice, s));
    SH_HIP_TRY(hipStreamSynchronize(s));
  }
  SH_HIP_TRY(hipMemsetAsync(m->counters, 0, (size_t)m->cfg.max_batch * m->cfg.kv_heads * 4, s));
  m->batch = batch;
  m->splits = attention_splits(batch, m->cfg.kv_heads, m->cfg.max_positions);
  m->chunk = ((m->cfg.max_positions + m->splits - 1) / m->splits + 15) / 16 * 16;
  m->steps_done = 0;
  if (m->layers_kernel) {
    // splits per (row, KV head): as many as give every workgroup one item at
    // batch 1, no split longer than kMaxSplitChunk, at most the kernel's
    // merge limit (setup checked that both hold together); independent of
    // the batch, so a row's arithmetic does not depend on its batch
    LayersArgs &a = m->la;
    const sh_llm_config &c = m->cfg;
    int sp = (m->layers_grid + c.kv_heads - 1) / c.kv_heads;
    const int min_sp = (c.max_positions + kMaxSplitChunk - 1) / kMaxSplitChunk;
    const int max_sp = decode_layers_max_splits(c.hidden, c.heads, c.kv_heads, c.intermediate);
    if (sp < min_sp) sp = min_sp;
    if (sp > max_sp) sp = max_sp;
    a.B = batch;
    a.splits = sp;
    a.chunk = ((c.max_positions + sp - 1) / sp + 15) / 16 * 16;
    // XCD-local placement at batch 1 (STRICT_HIP_LLM_XCD=0: off; also off
    // for the model's life once a step found a workgroup off its XCD)
    const char *xe = getenv("STRICT_HIP_LLM_XCD");
    a.xcd = !(xe && xe[0] == '0') && !m->xcd_off && decode_layers_xcd_ok(a, m->layers_grid) ? 1 : 0;
    m->layers_lds = decode_layers_lds(batch, c.hidden, c.heads, c.intermediate, &a.lds_misc);
    SH_HIP_TRY(hipMemsetAsync(a.err, 0, 4, s));
  }
  if (m->gpt2_kernel) {
    const char *xe = getenv("STRICT_HIP_LLM_XCD");
    m->ga.xcd = !(xe && xe[0] == '0') && !m->xcd_off && gpt2_layers_xcd_ok(m->ga, m->gpt2_grid) ? 1 : 0;
    SH_HIP_TRY(hipMemsetAsync(m->ga.err, 0, 4, s));
  }
  return SH_OK;
}

SH_API int sh_llm_step(sh_llm *m, const int32_t *tokens, int want_logits) {
  if (!m) return fail(SH_ERR_INVALID_ARGUMENT, "model is NULL");
  int rc = enter(m->ctx);
  if (rc != SH_OK) return rc;
  if (m->batch == 0) return fail(SH_ERR_INVALID_ARGUMENT, "sh_llm_reset was not called");
  if (m->steps_done >= m->cfg.max_positions)
    return fail(SH_ERR_INVALID_ARGUMENT, "KV cache full (%d positions)", m->cfg.max_positions);
  hipStream_t s = stream_of(m->ctx);
  if (tokens) {
    // the token in slot 0, every other slot cleared (a previous head's keys)
    unsigned long long keys[kKeySlots * kKeyStride] = {};
    for (int b = 0; b < m->batch; b++) {
      if (tokens[b] < 0 || tokens[b] >= m->cfg.vocab)
        return fail(SH_ERR_INVALID_ARGUMENT, "token %d of row %d outside the vocabulary", tokens[b], b);
      keys[b] = (unsigned long long)(0xffffffffu - (uint32_t)tokens[b]);
    }
    SH_HIP_TRY(hipMemcpyAsync(key_set(m), keys, sizeof(keys), hipMemcpyHostToDevice, s));
    SH_HIP_TRY(hipStreamSynchronize(s));  // `keys` is a stack array
  }
  const int g = want_logits ? 1 : 0;
  if (!m->use_graphs || m->layers_kernel || (m->gpt2_kernel && m->batch == 1)) {
    if ((rc = enqueue_step(m, want_logits != 0)) != SH_OK) return rc;
  } else if (m->graph_batch[g] != m->batch || m->graph_keys[g] != key_set(m)) {
    // (a layers kernel's steps at another batch may have moved the step
    // number to the other key set since the capture)
    if (m->graph[g]) (void)hipGraphExecDestroy(m->graph[g]);
    m->graph[g] = nullptr;
    m->graph_batch[g] = -1;
    // first step of this batch size runs eagerly, and is captured for replay
    if ((rc = enqueue_step(m, want_logits != 0)) != SH_OK) return rc;
    hipGraph_t graph = nullptr;
    SH_HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    rc = enqueue_step(m, want_logits != 0);
    hipError_t e = hipStreamEndCapture(s, &graph);
    if (rc != SH_OK) {
      if (graph) (void)hipGraphDestroy(graph);
      return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "capturing the decode step");
    e = hipGraphInstantiate(&m->graph[g], graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(e, "instantiating the decode graph");
    m->graph_batch[g] = m->batch;
    m->graph_keys[g] = key_set(m);
  } else {
    SH_HIP_TRY(hipGraphLaunch(m->graph[g], s));
  }
  m->steps_done++;
  return SH_OK;
}

SH_API int sh_llm_next_tokens(sh_llm *m, int32_t *tokens) {
  if (!m || !tokens) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  int rc = enter(m->ctx);
  if (rc != SH_OK) return rc;
  unsigned long long keys[kKeySlots * kKeyStride];
  hipStream_t s = stream_of(m->ctx);
  SH_HIP_TRY(hipMemcpyAsync(keys, key_set(m), sizeof(keys), hipMemcpyDeviceToHost, s));
  unsigned err = 0;
  if (m->layers_kernel)
    SH_HIP_TRY(hipMemcpyAsync(&err, m->la.err, 4, hipMemcpyDeviceToHost, s));
  else if (m->gpt2_kernel && m->batch == 1)
    SH_HIP_TRY(hipMemcpyAsync(&err, m->ga.err, 4, hipMemcpyDeviceToHost, s));
  SH_HIP_TRY(hipStreamSynchronize(s));
  // a failed step in XCD-local placement turns it off from the next reset
  // on: a grid whose workgroups were not spread over the XCDs round robin
  // would leave roles unrun, and their consumers' waits would time out
  if (err && ((m->layers_kernel && m->la.xcd) || (m->gpt2_kernel && m->batch == 1 && m->ga.xcd)))
    m->xcd_off = true;
  if (err & 2u)
    return fail(SH_ERR_HIP, "layers kernel: a workgroup read an XCD id outside 0..7 in XCD-local "
                            "placement (step state lost; reset the model, which turns that placement off)");
  if (err)
    return fail(SH_ERR_HIP, "decode-layers kernel: a wait between workgroups timed out (step state lost; reset the model)");
  for (int b = 0; b < m->batch; b++) {
    unsigned long long key = 0;
    for (int sl = 0; sl < kKeySlots; sl++) key = std::max(key, keys[sl * kKeyStride + b]);
    if (key == 0) return fail(SH_ERR_INVALID_ARGUMENT, "no greedy token yet (step without logits?)");
    tokens[b] = (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffu));
  }
  return SH_OK;
}

SH_API int sh_llm_generate(sh_llm *m, const int32_t *prompt, int prompt_len, int steps,
                           int32_t *out) {
  if (!m || !prompt || !out) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (m->batch == 0) return fail(SH_ERR_INVALID_ARGUMENT, "sh_llm_reset was not called");
  if (prompt_len < 1 || steps < 1)
    return fail(SH_ERR_INVALID_ARGUMENT, "prompt_len and steps must be >= 1");
  if (m->steps_done + prompt_len + steps - 1 > m->cfg.max_positions)
    return fail(SH_ERR_INVALID_ARGUMENT, "prompt + steps exceed max_positions %d", m->cfg.max_positions);
  const int B = m->batch;
  int rc;
  std::vector<int32_t> col(B);
  const int start = m->steps_done;
  for (int i = 0; i < prompt_len; i++) {
    for (int b = 0; b < B; b++) col[b] = prompt[(size_t)b * prompt_len + i];
    if ((rc = sh_llm_step(m, col.data(), i == prompt_len - 1)) != SH_OK) return rc;
  }
  for (int j = 1; j < steps; j++)
    if ((rc = sh_llm_step(m, nullptr, 1)) != SH_OK) return rc;
  if ((rc = sh_llm_next_tokens(m, col.data())) != SH_OK) return rc;
  // generated tokens 0 .. steps-2 were embedded (history), the last is the key
  std::vector<int32_t> hist((size_t)B * m->cfg.max_positions);
  hipStream_t s = stream_of(m->ctx);
  SH_HIP_TRY(hipMemcpyAsync(hist.data(), m->hist, hist.size() * 4, hipMemcpyDeviceToHost, s));
  SH_HIP_TRY(hipStreamSynchronize(s));
  for (int b = 0; b < B; b++) {
    for (int j = 0; j + 1 < steps; j++)
      out[(size_t)b * steps + j] = hist[(size_t)b * m->cfg.max_positions + start + prompt_len + j];
    out[(size_t)b * steps + steps - 1] = col[b];
  }
  return SH_OK;
}

}  // extern "C"
