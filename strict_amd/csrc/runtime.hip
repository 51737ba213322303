// libstrict_hip runtime: errors, contexts, buffers, hipRTC programs, modules,
// raw launches and the argument checks of the typed ops. Kernels live in the
// other translation units; this file only validates and dispatches.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "common.h"

struct sh_function {
  hipFunction_t fn;
  sh_module *module;
};

struct sh_module {
  hipModule_t mod;
  sh_ctx *ctx;
  std::map<std::string, sh_function *> functions;
};

struct sh_program {
  std::vector<char> code;
  std::string log;
};

struct sh_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t timer_begin = nullptr, timer_end = nullptr;
  bool timer_running = false;
  std::mutex mu;
  std::map<uintptr_t, size_t> owned;     // sh_alloc'd ranges
  std::map<uintptr_t, size_t> external;  // sh_register_external ranges
  std::set<sh_module *> modules;
  void *scratch = nullptr;  // work buffer of typed ops (context_scratch)
  size_t scratch_bytes = 0;
};

namespace sh {

static thread_local std::string t_last_error;

int fail(int status, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  t_last_error = buf;
  return status;
}

int hip_fail(hipError_t err, const char *what) {
  int status = (err == hipErrorOutOfMemory || err == hipErrorMemoryAllocation)
                   ? SH_ERR_OUT_OF_MEMORY
                   : SH_ERR_HIP;
  return fail(status, "%s failed: %s (%d)", what, hipGetErrorString(err), (int)err);
}

void clear_error() { t_last_error.clear(); }

static bool in_map(const std::map<uintptr_t, size_t> &m, uintptr_t p, size_t bytes) {
  auto it = m.upper_bound(p);
  if (it == m.begin()) return false;
  --it;
  uintptr_t base = it->first;
  size_t size = it->second;
  return p >= base && bytes <= size && p - base <= size - bytes;
}

int check_range(sh_ctx *ctx, const void *ptr, size_t bytes, const char *name) {
  if (ptr == nullptr) return fail(SH_ERR_INVALID_ARGUMENT, "%s is NULL", name);
  uintptr_t p = reinterpret_cast<uintptr_t>(ptr);
  std::lock_guard<std::mutex> lock(ctx->mu);
  if (in_map(ctx->owned, p, bytes) || in_map(ctx->external, p, bytes)) return SH_OK;
  return fail(SH_ERR_INVALID_ARGUMENT,
              "%s (%p, %zu bytes) is not inside an allocation of this context", name, ptr,
              bytes);
}

hipStream_t stream_of(sh_ctx *ctx) { return ctx->stream; }

int context_scratch(sh_ctx *ctx, size_t bytes, void **ptr) {
  std::lock_guard<std::mutex> lock(ctx->mu);
  if (ctx->scratch_bytes < bytes) {
    // the old buffer may still be read by work queued on the stream
    SH_HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
    const size_t grown = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    SH_HIP_TRY(hipMalloc(&ctx->scratch, grown));
    ctx->scratch_bytes = grown;
  }
  *ptr = ctx->scratch;
  return SH_OK;
}
int device_of(sh_ctx *ctx) { return ctx->device; }

int enter(sh_ctx *ctx) {
  if (ctx == nullptr) return fail(SH_ERR_INVALID_ARGUMENT, "context is NULL");
  SH_HIP_TRY(hipSetDevice(ctx->device));
  return SH_OK;
}

}  // namespace sh

using namespace sh;

#define SH_CHECK(expr)           \
  do {                           \
    int sh_rc_ = (expr);         \
    if (sh_rc_ != SH_OK) return sh_rc_; \
  } while (0)

extern "C" {

SH_API const char *sh_last_error(void) { return t_last_error.c_str(); }

SH_API int sh_version(void) { return 1 * 10000 + 0 * 100 + 0; }

SH_API int sh_device_count(int *count) {
  if (!count) return fail(SH_ERR_INVALID_ARGUMENT, "count is NULL");
  *count = 0;
  int n = 0;
  hipError_t err = hipGetDeviceCount(&n);
  if (err == hipErrorNoDevice || err == hipErrorInsufficientDriver) {
    (void)hipGetLastError();
    return SH_OK;
  }
  if (err != hipSuccess) return hip_fail(err, "hipGetDeviceCount");
  *count = n;
  return SH_OK;
}

// ---- context ---------------------------------------------------------------

SH_API int sh_create(int device, sh_ctx **out) {
  if (!out) return fail(SH_ERR_INVALID_ARGUMENT, "ctx out-pointer is NULL");
  *out = nullptr;
  int n = 0;
  SH_CHECK(sh_device_count(&n));
  if (n == 0) return fail(SH_ERR_NO_DEVICE, "no HIP device is visible");
  if (device < 0 || device >= n)
    return fail(SH_ERR_NO_DEVICE, "device %d out of range (%d visible)", device, n);
  SH_HIP_TRY(hipSetDevice(device));
  auto *ctx = new sh_ctx();
  ctx->device = device;
  hipError_t err = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (err == hipSuccess) err = hipEventCreate(&ctx->timer_begin);
  if (err == hipSuccess) err = hipEventCreate(&ctx->timer_end);
  if (err != hipSuccess) {
    if (ctx->timer_begin) (void)hipEventDestroy(ctx->timer_begin);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return hip_fail(err, "creating the context stream/events");
  }
  *out = ctx;
  clear_error();
  return SH_OK;
}

SH_API int sh_module_unload(sh_module *module);

SH_API int sh_destroy(sh_ctx *ctx) {
  if (!ctx) return SH_OK;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  std::vector<sh_module *> mods(ctx->modules.begin(), ctx->modules.end());
  for (auto *m : mods) sh_module_unload(m);
  for (auto &kv : ctx->owned) (void)hipFree(reinterpret_cast<void *>(kv.first));
  ctx->owned.clear();
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  (void)hipEventDestroy(ctx->timer_begin);
  (void)hipEventDestroy(ctx->timer_end);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return SH_OK;
}

SH_API int sh_device_info(sh_ctx *ctx, sh_device_info_t *info) {
  SH_CHECK(enter(ctx));
  if (!info) return fail(SH_ERR_INVALID_ARGUMENT, "info is NULL");
  hipDeviceProp_t p;
  SH_HIP_TRY(hipGetDeviceProperties(&p, ctx->device));
  std::memset(info, 0, sizeof *info);
  info->device = ctx->device;
  info->compute_units = p.multiProcessorCount;
  info->wavefront_size = p.warpSize;
  info->clock_khz = p.clockRate;
  info->memory_clock_khz = p.memoryClockRate;
  info->memory_bus_width_bits = p.memoryBusWidth;
  info->total_memory_bytes = p.totalGlobalMem;
  info->lds_bytes_per_block = p.sharedMemPerBlock;
  std::snprintf(info->name, sizeof info->name, "%s", p.name);
  std::snprintf(info->arch, sizeof info->arch, "%s", p.gcnArchName);
  return SH_OK;
}

SH_API int sh_sync(sh_ctx *ctx) {
  SH_CHECK(enter(ctx));
  SH_HIP_TRY(hipStreamSynchronize(ctx->stream));
  return SH_OK;
}

SH_API int sh_stream(sh_ctx *ctx, void **stream) {
  if (!ctx || !stream) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  *stream = ctx->stream;
  return SH_OK;
}

// ---- buffers ---------------------------------------------------------------

SH_API int sh_alloc(sh_ctx *ctx, size_t bytes, void **device_ptr) {
  SH_CHECK(enter(ctx));
  if (!device_ptr) return fail(SH_ERR_INVALID_ARGUMENT, "device_ptr out-pointer is NULL");
  *device_ptr = nullptr;
  if (bytes == 0) return fail(SH_ERR_INVALID_ARGUMENT, "zero-byte allocation");
  void *p = nullptr;
  SH_HIP_TRY(hipMalloc(&p, bytes));
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ctx->owned[reinterpret_cast<uintptr_t>(p)] = bytes;
  }
  *device_ptr = p;
  return SH_OK;
}

SH_API int sh_free(sh_ctx *ctx, void *device_ptr) {
  SH_CHECK(enter(ctx));
  if (!device_ptr) return SH_OK;
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    auto it = ctx->owned.find(reinterpret_cast<uintptr_t>(device_ptr));
    if (it == ctx->owned.end())
      return fail(SH_ERR_INVALID_ARGUMENT, "%p is not an allocation of this context (double free?)",
                  device_ptr);
    ctx->owned.erase(it);
  }
  // The stream may still use the buffer: finish its work first.
  SH_HIP_TRY(hipStreamSynchronize(ctx->stream));
  SH_HIP_TRY(hipFree(device_ptr));
  return SH_OK;
}

SH_API int sh_upload(sh_ctx *ctx, void *dst, const void *src, size_t bytes) {
  SH_CHECK(enter(ctx));
  if (bytes == 0) return SH_OK;
  if (!src) return fail(SH_ERR_INVALID_ARGUMENT, "host source is NULL");
  SH_CHECK(check_range(ctx, dst, bytes, "device destination"));
  SH_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  SH_HIP_TRY(hipStreamSynchronize(ctx->stream));
  return SH_OK;
}

SH_API int sh_download(sh_ctx *ctx, void *dst, const void *src, size_t bytes) {
  SH_CHECK(enter(ctx));
  if (bytes == 0) return SH_OK;
  if (!dst) return fail(SH_ERR_INVALID_ARGUMENT, "host destination is NULL");
  SH_CHECK(check_range(ctx, src, bytes, "device source"));
  SH_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  SH_HIP_TRY(hipStreamSynchronize(ctx->stream));
  return SH_OK;
}

SH_API int sh_copy(sh_ctx *ctx, void *dst, const void *src, size_t bytes) {
  SH_CHECK(enter(ctx));
  if (bytes == 0) return SH_OK;
  SH_CHECK(check_range(ctx, dst, bytes, "device destination"));
  SH_CHECK(check_range(ctx, src, bytes, "device source"));
  uintptr_t d = reinterpret_cast<uintptr_t>(dst), r = reinterpret_cast<uintptr_t>(src);
  if (d != r && d < r + bytes && r < d + bytes)
    return fail(SH_ERR_INVALID_ARGUMENT, "source and destination overlap");
  if (d == r) return SH_OK;
  SH_HIP_TRY(launch_copy_bytes(ctx->stream, dst, src, bytes));
  return SH_OK;
}

SH_API int sh_memset(sh_ctx *ctx, void *ptr, int value, size_t bytes) {
  SH_CHECK(enter(ctx));
  if (bytes == 0) return SH_OK;
  SH_CHECK(check_range(ctx, ptr, bytes, "device buffer"));
  SH_HIP_TRY(hipMemsetAsync(ptr, value, bytes, ctx->stream));
  return SH_OK;
}

SH_API int sh_register_external(sh_ctx *ctx, void *ptr, size_t bytes) {
  if (!ctx) return fail(SH_ERR_INVALID_ARGUMENT, "context is NULL");
  if (!ptr || bytes == 0) return fail(SH_ERR_INVALID_ARGUMENT, "empty external range");
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->external[reinterpret_cast<uintptr_t>(ptr)] = bytes;
  return SH_OK;
}

SH_API int sh_unregister_external(sh_ctx *ctx, void *ptr) {
  if (!ctx) return fail(SH_ERR_INVALID_ARGUMENT, "context is NULL");
  std::lock_guard<std::mutex> lock(ctx->mu);
  if (ctx->external.erase(reinterpret_cast<uintptr_t>(ptr)) == 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "%p was not registered", ptr);
  return SH_OK;
}

// ---- timing ----------------------------------------------------------------

SH_API int sh_timer_start(sh_ctx *ctx) {
  SH_CHECK(enter(ctx));
  SH_HIP_TRY(hipEventRecord(ctx->timer_begin, ctx->stream));
  ctx->timer_running = true;
  return SH_OK;
}

SH_API int sh_timer_stop(sh_ctx *ctx, float *ms) {
  SH_CHECK(enter(ctx));
  if (!ms) return fail(SH_ERR_INVALID_ARGUMENT, "elapsed_ms is NULL");
  if (!ctx->timer_running) return fail(SH_ERR_INVALID_ARGUMENT, "sh_timer_start was not called");
  SH_HIP_TRY(hipEventRecord(ctx->timer_end, ctx->stream));
  SH_HIP_TRY(hipEventSynchronize(ctx->timer_end));
  SH_HIP_TRY(hipEventElapsedTime(ms, ctx->timer_begin, ctx->timer_end));
  ctx->timer_running = false;
  return SH_OK;
}

struct sh_event {
  hipEvent_t ev;
  sh_ctx *ctx;
};

SH_API int sh_event_create(sh_ctx *ctx, sh_event **event) {
  SH_CHECK(enter(ctx));
  if (!event) return fail(SH_ERR_INVALID_ARGUMENT, "event out-pointer is NULL");
  *event = nullptr;
  hipEvent_t ev;
  SH_HIP_TRY(hipEventCreate(&ev));
  *event = new sh_event{ev, ctx};
  return SH_OK;
}

SH_API int sh_event_record(sh_event *event) {
  if (!event) return fail(SH_ERR_INVALID_ARGUMENT, "event is NULL");
  SH_CHECK(enter(event->ctx));
  SH_HIP_TRY(hipEventRecord(event->ev, event->ctx->stream));
  return SH_OK;
}

SH_API int sh_event_elapsed(sh_event *start, sh_event *stop, float *ms) {
  if (!start || !stop || !ms) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (start->ctx != stop->ctx)
    return fail(SH_ERR_INVALID_ARGUMENT, "events belong to different contexts");
  SH_CHECK(enter(stop->ctx));
  SH_HIP_TRY(hipEventSynchronize(stop->ev));
  SH_HIP_TRY(hipEventElapsedTime(ms, start->ev, stop->ev));
  return SH_OK;
}

SH_API int sh_event_destroy(sh_event *event) {
  if (!event) return SH_OK;
  (void)hipSetDevice(event->ctx->device);
  (void)hipEventDestroy(event->ev);
  delete event;
  return SH_OK;
}

// ---- hipRTC programs -----------------------------------------------------

SH_API int sh_compile(const char *source, const char *name, const char *const *options,
                      int num_options, sh_program **program) {
  if (!program) return fail(SH_ERR_INVALID_ARGUMENT, "program out-pointer is NULL");
  *program = nullptr;
  if (!source || !*source) return fail(SH_ERR_INVALID_ARGUMENT, "empty source");
  if (num_options < 0 || (num_options > 0 && !options))
    return fail(SH_ERR_INVALID_ARGUMENT, "bad options array");
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, name ? name : "kernel", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS)
    return fail(SH_ERR_COMPILE, "hiprtcCreateProgram: %s", hiprtcGetErrorString(r));
  std::vector<const char *> opts;
  bool has_arch = false;
  for (int i = 0; i < num_options; i++) {
    if (!options[i]) continue;
    if (std::strstr(options[i], "offload-arch") || std::strstr(options[i], "gpu-architecture"))
      has_arch = true;
    opts.push_back(options[i]);
  }
  if (!has_arch) opts.push_back("--offload-arch=gfx950");
  opts.push_back("-O3");
  r = hiprtcCompileProgram(prog, (int)opts.size(), opts.data());
  auto *p = new sh_program();
  size_t log_size = 0;
  if (hiprtcGetProgramLogSize(prog, &log_size) == HIPRTC_SUCCESS && log_size > 1) {
    p->log.resize(log_size);
    hiprtcGetProgramLog(prog, &p->log[0]);
    while (!p->log.empty() && p->log.back() == '\0') p->log.pop_back();
  }
  *program = p;
  if (r != HIPRTC_SUCCESS) {
    hiprtcDestroyProgram(&prog);
    return fail(SH_ERR_COMPILE, "hipRTC compile of '%s' failed: %s\n%s", name ? name : "kernel",
                hiprtcGetErrorString(r), p->log.c_str());
  }
  size_t code_size = 0;
  r = hiprtcGetCodeSize(prog, &code_size);
  if (r == HIPRTC_SUCCESS) {
    p->code.resize(code_size);
    r = hiprtcGetCode(prog, p->code.data());
  }
  hiprtcDestroyProgram(&prog);
  if (r != HIPRTC_SUCCESS)
    return fail(SH_ERR_COMPILE, "reading the code object: %s", hiprtcGetErrorString(r));
  return SH_OK;
}

SH_API int sh_program_code(sh_program *program, const void **code, size_t *bytes) {
  if (!program || !code || !bytes) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (program->code.empty()) return fail(SH_ERR_COMPILE, "program has no code object");
  *code = program->code.data();
  *bytes = program->code.size();
  return SH_OK;
}

SH_API const char *sh_program_log(sh_program *program) {
  return program ? program->log.c_str() : "";
}

SH_API int sh_program_destroy(sh_program *program) {
  delete program;
  return SH_OK;
}

// ---- modules and raw launches ----------------------------------------------

SH_API int sh_module_load(sh_ctx *ctx, const void *code, size_t bytes, sh_module **module) {
  SH_CHECK(enter(ctx));
  if (!module) return fail(SH_ERR_INVALID_ARGUMENT, "module out-pointer is NULL");
  *module = nullptr;
  if (!code || bytes == 0) return fail(SH_ERR_INVALID_ARGUMENT, "empty code object");
  hipModule_t mod;
  SH_HIP_TRY(hipModuleLoadData(&mod, code));
  auto *m = new sh_module();
  m->mod = mod;
  m->ctx = ctx;
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ctx->modules.insert(m);
  }
  *module = m;
  return SH_OK;
}

SH_API int sh_module_function(sh_module *module, const char *name, sh_function **function) {
  if (!module || !name || !function) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  *function = nullptr;
  SH_CHECK(enter(module->ctx));
  auto it = module->functions.find(name);
  if (it != module->functions.end()) {
    *function = it->second;
    return SH_OK;
  }
  hipFunction_t fn;
  hipError_t err = hipModuleGetFunction(&fn, module->mod, name);
  if (err != hipSuccess) {
    (void)hipGetLastError();
    return fail(SH_ERR_NOT_FOUND, "kernel '%s' not found in module (%s)", name,
                hipGetErrorString(err));
  }
  auto *f = new sh_function{fn, module};
  module->functions[name] = f;
  *function = f;
  return SH_OK;
}

SH_API int sh_module_unload(sh_module *module) {
  if (!module) return SH_OK;
  sh_ctx *ctx = module->ctx;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  for (auto &kv : module->functions) delete kv.second;
  (void)hipModuleUnload(module->mod);
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ctx->modules.erase(module);
  }
  delete module;
  return SH_OK;
}

SH_API int sh_launch(sh_function *function, const unsigned grid[3], const unsigned block[3],
                     unsigned shared_bytes, void **args, float *elapsed_ms) {
  if (!function || !grid || !block) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  sh_ctx *ctx = function->module->ctx;
  SH_CHECK(enter(ctx));
  for (int d = 0; d < 3; d++)
    if (grid[d] == 0 || block[d] == 0)
      return fail(SH_ERR_INVALID_ARGUMENT, "grid and block dimensions must be >= 1");
  unsigned long long threads = (unsigned long long)block[0] * block[1] * block[2];
  if (threads > 1024)
    return fail(SH_ERR_INVALID_ARGUMENT, "block of %llu threads exceeds 1024", threads);
  if (shared_bytes > 160 * 1024)
    return fail(SH_ERR_INVALID_ARGUMENT, "%u bytes of LDS exceed 160 KiB", shared_bytes);
  SH_HIP_TRY(hipEventRecord(ctx->timer_begin, ctx->stream));
  SH_HIP_TRY(hipModuleLaunchKernel(function->fn, grid[0], grid[1], grid[2], block[0], block[1],
                                   block[2], shared_bytes, ctx->stream, args, nullptr));
  SH_HIP_TRY(hipEventRecord(ctx->timer_end, ctx->stream));
  SH_HIP_TRY(hipEventSynchronize(ctx->timer_end));
  float ms = 0.f;
  SH_HIP_TRY(hipEventElapsedTime(&ms, ctx->timer_begin, ctx->timer_end));
  if (elapsed_ms) *elapsed_ms = ms;
  return SH_OK;
}

// ---- typed ops: elementwise --------------------------------------------------

static int launched(hipError_t err, const char *what) {
  return err == hipSuccess ? SH_OK : hip_fail(err, what);
}

SH_API int sh_binary_f32(sh_ctx *ctx, int op, const float *first, const float *second,
                         float *output, size_t count) {
  SH_CHECK(enter(ctx));
  if (op < SH_ADD || op > SH_DIVIDE)
    return fail(SH_ERR_INVALID_ARGUMENT, "unknown binary op %d", op);
  if (count == 0) return SH_OK;
  size_t bytes = count * sizeof(float);
  SH_CHECK(check_range(ctx, first, bytes, "first"));
  SH_CHECK(check_range(ctx, second, bytes, "second"));
  SH_CHECK(check_range(ctx, output, bytes, "output"));
  return launched(launch_binary_f32(ctx->stream, op, first, second, output, count), "binary_f32");
}

SH_API int sh_fill_f32(sh_ctx *ctx, float value, float *output, size_t count) {
  SH_CHECK(enter(ctx));
  if (count == 0) return SH_OK;
  SH_CHECK(check_range(ctx, output, count * sizeof(float), "output"));
  return launched(launch_fill_f32(ctx->stream, value, output, count), "fill_f32");
}

SH_API int sh_saxpy_f32(sh_ctx *ctx, float a, const float *x, const float *y, float *out,
                        size_t n) {
  SH_CHECK(enter(ctx));
  if (n == 0) return SH_OK;
  size_t bytes = n * sizeof(float);
  SH_CHECK(check_range(ctx, x, bytes, "x"));
  SH_CHECK(check_range(ctx, y, bytes, "y"));
  SH_CHECK(check_range(ctx, out, bytes, "out"));
  return launched(launch_saxpy_f32(ctx->stream, a, x, y, out, n), "saxpy_f32");
}

SH_API int sh_sigmoid_f32(sh_ctx *ctx, const float *x, float *y, size_t n) {
  SH_CHECK(enter(ctx));
  if (n == 0) return SH_OK;
  size_t bytes = n * sizeof(float);
  SH_CHECK(check_range(ctx, x, bytes, "x"));
  SH_CHECK(check_range(ctx, y, bytes, "y"));
  return launched(launch_sigmoid_f32(ctx->stream, x, y, n), "sigmoid_f32");
}

// ---- typed ops: image --------------------------------------------------------

static int check_image(int width, int height, int channels, size_t *bytes) {
  if (width < 0 || height < 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "negative image size %dx%d", width, height);
  if (channels < 1 || channels > 4)
    return fail(SH_ERR_INVALID_ARGUMENT, "channels must be 1..4, got %d", channels);
  if ((long long)width * height > (1LL << 31) / 4)
    return fail(SH_ERR_INVALID_ARGUMENT, "image %dx%d too large", width, height);
  *bytes = (size_t)width * (size_t)height * (size_t)channels;
  return SH_OK;
}

static bool overlaps(const void *a, const void *b, size_t bytes) {
  uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + bytes && y < x + bytes;
}

SH_API int sh_adjust_brightness_u8(sh_ctx *ctx, const uint8_t *in, uint8_t *out, int width,
                                   int height, int channels, int delta, int flags) {
  SH_CHECK(enter(ctx));
  size_t bytes = 0;
  SH_CHECK(check_image(width, height, channels, &bytes));
  if (delta < -255 || delta > 255)
    return fail(SH_ERR_INVALID_ARGUMENT, "delta %d outside [-255, 255]", delta);
  if (flags & ~SH_BRIGHTNESS_ALL_CHANNELS)
    return fail(SH_ERR_INVALID_ARGUMENT, "unknown brightness flags 0x%x", flags);
  if (bytes == 0) return SH_OK;
  SH_CHECK(check_range(ctx, in, bytes, "in"));
  SH_CHECK(check_range(ctx, out, bytes, "out"));
  if (in != out && overlaps(in, out, bytes))
    return fail(SH_ERR_INVALID_ARGUMENT, "in and out partially overlap");
  return launched(launch_brightness_u8(ctx->stream, in, out, bytes, channels, delta,
                                       (flags & SH_BRIGHTNESS_ALL_CHANNELS) != 0),
                  "adjust_brightness_u8");
}

// Image layout adapters. Sizes are checked in size_t before any launch; a
// stride must cover its row.
static int check_adapter_size(int width, int height) {
  if (width < 0 || height < 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "negative image size %dx%d", width, height);
  if (height > 65535) return fail(SH_ERR_INVALID_ARGUMENT, "height %d above 65535", height);
  return SH_OK;
}

SH_API int sh_bgr_to_rgba_u8(sh_ctx *ctx, const uint8_t *src, int bytes_per_pixel,
                             size_t src_stride, uint8_t *dst, int width, int height) {
  SH_CHECK(enter(ctx));
  SH_CHECK(check_adapter_size(width, height));
  if (bytes_per_pixel != 3 && bytes_per_pixel != 4)
    return fail(SH_ERR_INVALID_ARGUMENT, "bytes_per_pixel %d is not 3 or 4", bytes_per_pixel);
  if (width == 0 || height == 0) return SH_OK;
  if (src_stride < (size_t)width * bytes_per_pixel)
    return fail(SH_ERR_INVALID_ARGUMENT, "src_stride %zu below %d x %d", src_stride, width,
                bytes_per_pixel);
  if (reinterpret_cast<uintptr_t>(dst) % 4)
    return fail(SH_ERR_INVALID_ARGUMENT, "dst is not 4-byte aligned");
  const size_t in_bytes = (size_t)(height - 1) * src_stride + (size_t)width * bytes_per_pixel;
  const size_t out_bytes = (size_t)width * height * 4;
  SH_CHECK(check_range(ctx, src, in_bytes, "src"));
  SH_CHECK(check_range(ctx, dst, out_bytes, "dst"));
  if (reinterpret_cast<uintptr_t>(src) < reinterpret_cast<uintptr_t>(dst) + out_bytes &&
      reinterpret_cast<uintptr_t>(dst) < reinterpret_cast<uintptr_t>(src) + in_bytes)
    return fail(SH_ERR_INVALID_ARGUMENT, "src and dst overlap");
  return launched(launch_bgr_to_rgba_u8(ctx->stream, src, bytes_per_pixel, src_stride,
                                        reinterpret_cast<uint32_t *>(dst), width, height),
                  "bgr_to_rgba_u8");
}

SH_API int sh_rgb_to_bgr_u8(sh_ctx *ctx, const uint8_t *src, uint8_t *dst, int width, int height,
                            size_t dst_stride) {
  SH_CHECK(enter(ctx));
  SH_CHECK(check_adapter_size(width, height));
  if (width == 0 || height == 0) return SH_OK;
  if (dst_stride < (size_t)width * 3)
    return fail(SH_ERR_INVALID_ARGUMENT, "dst_stride %zu below 3 x %d", dst_stride, width);
  const size_t in_bytes = (size_t)width * height * 3;
  const size_t out_bytes = (size_t)(height - 1) * dst_stride + (size_t)width * 3;
  SH_CHECK(check_range(ctx, src, in_bytes, "src"));
  SH_CHECK(check_range(ctx, dst, out_bytes, "dst"));
  if (reinterpret_cast<uintptr_t>(src) < reinterpret_cast<uintptr_t>(dst) + out_bytes &&
      reinterpret_cast<uintptr_t>(dst) < reinterpret_cast<uintptr_t>(src) + in_bytes)
    return fail(SH_ERR_INVALID_ARGUMENT, "src and dst overlap");
  return launched(launch_rgb_to_bgr_u8(ctx->stream, src, dst, width, height, dst_stride),
                  "rgb_to_bgr_u8");
}

static int blur_common(sh_ctx *ctx, const uint8_t *in, uint8_t *out, int width, int height,
                       int channels, int mode, bool fuse, int delta, int flags) {
  SH_CHECK(enter(ctx));
  size_t bytes = 0;
  SH_CHECK(check_image(width, height, channels, &bytes));
  if (mode != SH_BLUR_CONFIG && mode != SH_BLUR_REFERENCE)
    return fail(SH_ERR_INVALID_ARGUMENT, "unknown blur mode %d", mode);
  if (fuse) {
    if (delta < -255 || delta > 255)
      return fail(SH_ERR_INVALID_ARGUMENT, "delta %d outside [-255, 255]", delta);
    if (flags & ~SH_BRIGHTNESS_ALL_CHANNELS)
      return fail(SH_ERR_INVALID_ARGUMENT, "unknown brightness flags 0x%x", flags);
  }
  if (bytes == 0) return SH_OK;
  SH_CHECK(check_range(ctx, in, bytes, "in"));
  SH_CHECK(check_range(ctx, out, bytes, "out"));
  if (overlaps(in, out, bytes))
    return fail(SH_ERR_INVALID_ARGUMENT, "blur needs distinct in and out buffers");
  return launched(launch_blur5_u8(ctx->stream, in, out, width, height, channels, mode, fuse,
                                  delta, (flags & SH_BRIGHTNESS_ALL_CHANNELS) != 0),
                  "box_blur5_u8");
}

SH_API int sh_box_blur5_u8(sh_ctx *ctx, const uint8_t *in, uint8_t *out, int width, int height,
                           int channels, int mode) {
  return blur_common(ctx, in, out, width, height, channels, mode, false, 0, 0);
}

SH_API int sh_brightness_blur5_u8(sh_ctx *ctx, const uint8_t *in, uint8_t *out, int width,
                                  int height, int channels, int delta, int flags, int mode) {
  return blur_common(ctx, in, out, width, height, channels, mode, true, delta, flags);
}

// ---- typed ops: dense GEMM ----------------------------------------------------

// Elements a row-major [rows x cols] operand with leading dimension ld spans.
static size_t span_elems(int rows, int cols, int ld) {
  return rows == 0 || cols == 0 ? 0 : (size_t)(rows - 1) * (size_t)ld + (size_t)cols;
}

static int check_gemm_dims(int M, int N, int K, int lda, int ldb, int ldc) {
  if (M < 0 || N < 0 || K < 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "negative GEMM size M=%d N=%d K=%d", M, N, K);
  if (lda < K || ldb < N || ldc < N)
    return fail(SH_ERR_INVALID_ARGUMENT,
                "leading dimensions too small: lda=%d (K=%d) ldb=%d (N=%d) ldc=%d (N=%d)", lda, K,
                ldb, N, ldc, N);
  return SH_OK;
}

SH_API int sh_gemm_bf16(sh_ctx *ctx, const uint16_t *A, const uint16_t *B, uint16_t *C, int M,
                        int N, int K, int lda, int ldb, int ldc) {
  SH_CHECK(enter(ctx));
  SH_CHECK(check_gemm_dims(M, N, K, lda, ldb, ldc));
  if (M == 0 || N == 0) return SH_OK;
  SH_CHECK(check_range(ctx, C, span_elems(M, N, ldc) * 2, "C"));
  if (K == 0) {  // empty sum: C = 0
    for (int m = 0; m < M; m++) SH_HIP_TRY(hipMemsetAsync(C + (size_t)m * ldc, 0, (size_t)N * 2, ctx->stream));
    return SH_OK;
  }
  SH_CHECK(check_range(ctx, A, span_elems(M, K, lda) * 2, "A"));
  SH_CHECK(check_range(ctx, B, span_elems(K, N, ldb) * 2, "B"));
  return launched(launch_gemm_bf16(ctx->stream, A, B, C, M, N, K, lda, ldb, ldc), "gemm_bf16");
}

SH_API int sh_gemm_fp8(sh_ctx *ctx, const uint8_t *A, const float *sa, const uint8_t *Bt,
                       const float *sb, uint16_t *C, int M, int N, int K, int lda, int ldb,
                       int ldc) {
  SH_CHECK(enter(ctx));
  if (M < 0 || N < 0 || K < 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "negative GEMM size M=%d N=%d K=%d", M, N, K);
  if (lda < K || ldb < K || ldc < N)
    return fail(SH_ERR_INVALID_ARGUMENT,
                "leading dimensions too small: lda=%d (K=%d) ldb=%d (K=%d) ldc=%d (N=%d)", lda, K,
                ldb, K, ldc, N);
  if (M == 0 || N == 0) return SH_OK;
  SH_CHECK(check_range(ctx, C, span_elems(M, N, ldc) * 2, "C"));
  if (K == 0) {  // empty sum: C = 0
    for (int m = 0; m < M; m++) SH_HIP_TRY(hipMemsetAsync(C + (size_t)m * ldc, 0, (size_t)N * 2, ctx->stream));
    return SH_OK;
  }
  SH_CHECK(check_range(ctx, A, span_elems(M, K, lda), "A"));
  SH_CHECK(check_range(ctx, Bt, span_elems(N, K, ldb), "Bt"));
  SH_CHECK(check_range(ctx, sa, (size_t)M * 4, "sa"));
  SH_CHECK(check_range(ctx, sb, (size_t)N * 4, "sb"));
  return launched(launch_gemm_fp8(ctx->stream, A, sa, Bt, sb, C, M, N, K, lda, ldb, ldc),
                  "gemm_fp8");
}

}  // extern "C"
