/*
 * libstrict_hip -- C ABI of the MI355X (gfx950) kernel path behind Strict's
 * `Strict.Compiler.Cuda` surface.
 *
 * The reference reaches the GPU through ManagedCuda objects (Kernel.cs,
 * CSharpToCudaTranspilerTests.cs, Cuda.Tests/BlurPerformanceTests.cs). This
 * header is the flat replacement a C# host binds with P/Invoke: opaque
 * handles, plain pointers and sizes, an int status per call (0 = SH_OK) and a
 * thread-local message from sh_last_error() in place of the exceptions
 * ManagedCuda throws.
 *
 * Conventions
 *  - Device pointers are the addresses sh_alloc returns (the counterpart of
 *    CudaDeviceVariable<T>.DevicePointer). Typed ops check that every pointer
 *    plus its extent lies inside one allocation of the context (or a range
 *    registered with sh_register_external) before anything is launched.
 *  - Ops are ordered on the context's stream and return before the GPU is
 *    done; sh_sync() waits. sh_upload/sh_download/sh_launch are synchronous,
 *    as the ManagedCuda calls they replace.
 *  - Zero-sized work is a successful no-op.
 */
#ifndef STRICT_HIP_H
#define STRICT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SH_API __attribute__((visibility("default")))

typedef enum sh_status {
  SH_OK = 0,
  SH_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size, pointer outside its allocation */
  SH_ERR_NO_DEVICE = 2,        /* no HIP device / device index out of range */
  SH_ERR_HIP = 3,              /* a HIP runtime call failed (message has the HIP error) */
  SH_ERR_OUT_OF_MEMORY = 4,
  SH_ERR_COMPILE = 5,          /* hipRTC compile failed; the program holds the log */
  SH_ERR_NOT_FOUND = 6,        /* unknown kernel name in a module */
  SH_ERR_UNSUPPORTED = 7,      /* valid request this build does not implement */
  SH_ERR_INVALID_FILE = 8,     /* malformed .strictbinary: the message starts with the
                                  reference's exception (InvalidFile, InvalidBytecodeEntry,
                                  InvalidVersion) */
} sh_status;

typedef struct sh_ctx sh_ctx;
typedef struct sh_program sh_program;
typedef struct sh_module sh_module;
typedef struct sh_function sh_function;

typedef struct sh_device_info_t {
  int device;
  int compute_units;
  int wavefront_size;
  int clock_khz;
  int memory_clock_khz;
  int memory_bus_width_bits;
  size_t total_memory_bytes;
  size_t lds_bytes_per_block;
  char name[256];
  char arch[64]; /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
} sh_device_info_t;

/* ---- errors and library ------------------------------------------------- */

/* Message of the last failing call on this thread ("" if none). Replaces the
 * exception text of CudaException / NVRTCException. */
SH_API const char *sh_last_error(void);
SH_API int sh_version(void); /* major * 10000 + minor * 100 + patch */
SH_API int sh_device_count(int *count);

/* ---- context: replaces `new CudaContext(0)` (Kernel.cs:9) and
 *      Kernel.Dispose (Kernel.cs:13-17) -------------------------------------- */

SH_API int sh_create(int device, sh_ctx **ctx);
SH_API int sh_destroy(sh_ctx *ctx); /* frees every allocation and module of ctx */
SH_API int sh_device_info(sh_ctx *ctx, sh_device_info_t *info);
SH_API int sh_sync(sh_ctx *ctx);
/* Raw hipStream_t the context orders its work on (for interop). */
SH_API int sh_stream(sh_ctx *ctx, void **stream);

/* ---- buffers: replace CudaDeviceVariable<T> and its implicit T[] <-> device
 *      conversions (CSharpToCudaTranspilerTests.cs:64, :75-76;
 *      Cuda.Tests/BlurPerformanceTests.cs:151-153, :178) ------------------- */

SH_API int sh_alloc(sh_ctx *ctx, size_t bytes, void **device_ptr);
SH_API int sh_free(sh_ctx *ctx, void *device_ptr);
SH_API int sh_upload(sh_ctx *ctx, void *device_dst, const void *host_src, size_t bytes);
SH_API int sh_download(sh_ctx *ctx, void *host_dst, const void *device_src, size_t bytes);
/* Stream-ordered device-to-device copy by a plain 16-byte-vector kernel;
 * the ranges must not overlap (dst == src is a no-op). */
SH_API int sh_copy(sh_ctx *ctx, void *device_dst, const void *device_src, size_t bytes);
SH_API int sh_memset(sh_ctx *ctx, void *device_ptr, int byte_value, size_t bytes);
/* Lets typed ops accept device memory the context did not allocate. */
SH_API int sh_register_external(sh_ctx *ctx, void *device_ptr, size_t bytes);
SH_API int sh_unregister_external(sh_ctx *ctx, void *device_ptr);

/* ---- timing on the context stream (HIP events) ---------------------------- */

SH_API int sh_timer_start(sh_ctx *ctx);
SH_API int sh_timer_stop(sh_ctx *ctx, float *elapsed_ms); /* waits for the stop event */

/* Free-standing events for per-launch timing (CudaEvent counterpart). */
typedef struct sh_event sh_event;
SH_API int sh_event_create(sh_ctx *ctx, sh_event **event);
SH_API int sh_event_record(sh_event *event); /* on the context stream */
/* ms between two recorded events of one context; waits for `stop`. */
SH_API int sh_event_elapsed(sh_event *start, sh_event *stop, float *elapsed_ms);
SH_API int sh_event_destroy(sh_event *event);

/* ---- runtime compilation and modules: replace CudaRuntimeCompiler (NVRTC,
 *      Kernel.cs:29-30, :43), GetPTX / GetLogAsString
 *      (Cuda.Tests/BlurPerformanceTests.cs:133, :148) and
 *      CudaContext.LoadKernelPTX (CSharpToCudaTranspilerTests.cs:65) --------- */

/* Compiles HIP C++ `source` with hipRTC for the device's architecture (gfx950
 * unless an --offload-arch option is given). On SH_ERR_COMPILE *program is
 * still set so the log can be read; always release it with
 * sh_program_destroy. */
SH_API int sh_compile(const char *source, const char *name, const char *const *options,
                      int num_options, sh_program **program);
SH_API int sh_program_code(sh_program *program, const void **code, size_t *bytes);
SH_API const char *sh_program_log(sh_program *program);
SH_API int sh_program_destroy(sh_program *program);

SH_API int sh_module_load(sh_ctx *ctx, const void *code_object, size_t bytes, sh_module **module);
SH_API int sh_module_function(sh_module *module, const char *name, sh_function **function);
SH_API int sh_module_unload(sh_module *module);

/* Replaces CudaKernel.Run (CSharpToCudaTranspilerTests.cs:77, :86): launches
 * with kernelParams-style `args` (one pointer per argument value), waits for
 * completion and returns the kernel time in ms (may be NULL). */
SH_API int sh_launch(sh_function *function, const unsigned grid[3], const unsigned block[3],
                     unsigned shared_bytes, void **args, float *elapsed_ms);

/* ---- kernel source generation: replaces InstructionsToCuda.BuildCudaKernel
 *      (Strict.Compiler.Cuda/InstructionsToCuda.cs:19-74) ------------------- */

/* Instruction types, numbered as Strict.Bytecode's InstructionType
 * (Strict.Bytecode/InstructionType.cs:9-47); only those the generator reads
 * are named. Register ids are Strict.Bytecode's Register values (R0 = 0 ...,
 * Register.cs:8-26). */
enum {
  SH_BC_LOAD_CONSTANT = 0, /* LoadConstantInstruction: registers[0] = number */
  SH_BC_LOAD_VARIABLE = 1, /* LoadVariableToRegister: registers[0] = identifier */
  SH_BC_ADD = 11,          /* BinaryInstruction: registers[2] = [0] op [1] */
  SH_BC_SUBTRACT = 12,
  SH_BC_MULTIPLY = 13,
  SH_BC_DIVIDE = 14,
  SH_BC_MODULO = 15,       /* no kernel operator: rejected as the reference does */
  SH_BC_EQUAL = 21,        /* 21..24: conditional binaries, skipped */
  SH_BC_GREATER_THAN = 24,
  SH_BC_RETURN = 32        /* ReturnInstruction: the output is registers[0] */
};

/* One bytecode instruction, flattened from the C# Instruction objects. */
typedef struct sh_bc_instruction {
  int type;               /* SH_BC_* / InstructionType value; others are ignored */
  int register_count;     /* registers in use: 1 for loads and return, 3 for binaries */
  int registers[3];
  const char *identifier; /* SH_BC_LOAD_VARIABLE */
  double number;          /* SH_BC_LOAD_CONSTANT */
} sh_bc_instruction;

/* Writes the HIP source of an elementwise kernel named `method_name` that
 * evaluates the instructions per element, as BuildCudaKernel does:
 * `parameters` are the method's parameter names, all Strict Numbers (width and
 * height become int scalars, initialDepth a float scalar, every other name a
 * float array indexed per element); `float *output` follows, then
 * `const int count` when add_count_parameter is non-zero. The bounds check is
 * `idx >= count`, or `x >= width || y >= height` when both are parameters and
 * no count is added. Two deliberate differences from the reference, which
 * produce the same values wherever the reference's text is correct:
 *  - the element index is the true row-major one (y * gridDim.x * blockDim.x
 *    + x, or y * width + x), where the reference's `y * blockDim.x + x` aliases
 *    rows once gridDim.x > 1;
 *  - an operand that is itself a binary expression is parenthesised where C's
 *    precedence would regroup it, where the reference concatenates without
 *    parentheses ((a + b) * c would otherwise print as a + b * c).
 * Constants print as .NET's invariant-culture double.ToString() does.
 * `*length` always receives the source length (excluding the NUL); the text
 * is written only when `capacity` > length, else SH_ERR_INVALID_ARGUMENT.
 * A Modulo (or other non-arithmetic) binary gives SH_ERR_UNSUPPORTED, the
 * reference's NotSupportedException (InstructionsToCuda.cs:101-109). */
SH_API int sh_instructions_to_hip(const char *method_name, const char *const *parameters,
                                  int parameter_count, int add_count_parameter,
                                  const sh_bc_instruction *instructions, int instruction_count,
                                  char *source, size_t capacity, size_t *length);

/* ---- .strictbinary loading: replaces BinaryExecutable's loader
 *      (Strict.Bytecode/BinaryExecutable.cs:40-61) and Serialize (:144-156) -- */

/* A loaded .strictbinary: a ZIP archive whose "<type full name>.bytecode"
 * entries each hold one type's members and method groups
 * (Serialization/BinaryType.cs:11-28). Types keep the archive's entry order
 * (MethodsPerType's order); a type's methods are the overloads of its method
 * groups, groups in file order, overloads in group order. Errors are
 * SH_ERR_INVALID_FILE with the reference's exception and message, e.g.
 * "InvalidBytecodeEntry: Entry does not start with compact 'S' magic byte"
 * (BinaryType.cs:43-62), "InvalidVersion: File version: 0, ...",
 * "InvalidFile: Unknown instruction type: 105" (BinaryExecutable.cs:167-203),
 * "InvalidFile: Unknown ValueKind: ..." (:278-292), "InvalidFile: End of
 * Central Directory record could not be found." for a file that is no ZIP.
 * Strings returned by the accessors live until sh_strictbinary_free. A handle
 * is not safe to use from two threads at once. */
typedef struct sh_strictbinary sh_strictbinary;

/* One value-carrying instruction (LoadConstantToRegister, StoreConstantToVariable,
 * Set) of a method, or a member's initial value (method_index -1). */
typedef struct sh_strictbinary_constant {
  int instruction;        /* index in the method (member index for members) */
  int instruction_type;   /* InstructionType: 0 LoadConstant, 2 StoreConstant, 4 Set */
  int kind;               /* ValueKind as stored: 0 None, 1 SmallNumber, 2 IntegerNumber,
                             3 Number, 4 Text, 5 Boolean, 6 List, 9 Dictionary */
  int register_id;        /* LoadConstant / Set: the register; otherwise -1 */
  const char *identifier; /* StoreConstant: the variable; member: its name; else NULL */
  size_t count;           /* Numbers held: 1 for a Number, the items of a List of Numbers,
                             0 otherwise */
} sh_strictbinary_constant;

/* Parses a whole .strictbinary image held in memory (the bytes of the file). */
SH_API int sh_strictbinary_load(const void *data, size_t bytes, sh_strictbinary **binary);
SH_API int sh_strictbinary_free(sh_strictbinary *binary);
SH_API int sh_strictbinary_type_count(const sh_strictbinary *binary, int *count);
SH_API int sh_strictbinary_type(const sh_strictbinary *binary, int type_index,
                                const char **full_name, int *member_count, int *method_count);
/* A member of the type (method_index -1) or a parameter of a method. */
SH_API int sh_strictbinary_member(const sh_strictbinary *binary, int type_index, int method_index,
                                  int member_index, const char **name, const char **full_type_name,
                                  int *has_initial_value);
SH_API int sh_strictbinary_method(const sh_strictbinary *binary, int type_index, int method_index,
                                  const char **name, int *parameter_count,
                                  const char **return_type, int *instruction_count);
/* EntryPoint: the first overload of the first Run group, types in order
 * (BinaryExecutable.cs:113-120); SH_ERR_NOT_FOUND without one. */
SH_API int sh_strictbinary_entry_point(const sh_strictbinary *binary, int *type_index,
                                       int *method_index);
/* FindInstructions (BinaryExecutable.cs:125-138): the first overload of
 * `method_name` in type `type_full_name` with `parameter_count` parameters
 * whose return type matches (NULL or "" matches any; "Number" matches
 * "Strict/Number" either way round); SH_ERR_NOT_FOUND otherwise. */
SH_API int sh_strictbinary_find(const sh_strictbinary *binary, const char *type_full_name,
                                const char *method_name, int parameter_count,
                                const char *return_type, int *type_index, int *method_index);
/* The method's instructions as sh_instructions_to_hip takes them: type,
 * register operands in payload order (the first three), identifier (variable,
 * list or table name; Print's text; Invoke's method name) and number (a Number
 * constant's value, NaN for other constants; the count of Jump, JumpToId and
 * LoopEnd). `*count` always receives the instruction count; with
 * instructions == NULL nothing else is written. */
SH_API int sh_strictbinary_instructions(const sh_strictbinary *binary, int type_index,
                                        int method_index, sh_bc_instruction *instructions,
                                        int capacity, int *count);
/* The value-carrying instructions of a method (method_index -1: the members'
 * initial values), in order; `*count` always receives their number. */
SH_API int sh_strictbinary_constants(sh_strictbinary *binary, int type_index, int method_index,
                                     sh_strictbinary_constant *constants, int capacity, int *count);
/* The Numbers of a constant (count > 0, or an empty List) as doubles. */
SH_API int sh_strictbinary_constant_values(sh_strictbinary *binary, int type_index,
                                           int method_index, int constant_index, double *values,
                                           size_t capacity);
/* Kernel input: the constant's Numbers rounded to fp32 (nearest even) into
 * device_dst, which holds `capacity` floats; synchronous, as sh_upload. */
SH_API int sh_strictbinary_upload_f32(sh_ctx *ctx, sh_strictbinary *binary, int type_index,
                                      int method_index, int constant_index, float *device_dst,
                                      size_t capacity);
/* Serialize: the binary as a .strictbinary image (deflated entries, types in
 * order, each entry as BinaryType.Write lays it out with a name table rebuilt
 * as the reference builds one). `*bytes` always receives the size; the image
 * is written only when capacity >= size, else SH_ERR_INVALID_ARGUMENT. */
SH_API int sh_strictbinary_serialize(sh_strictbinary *binary, void *data, size_t capacity,
                                     size_t *bytes);

/* ---- range-loop dispatch ---------------------------------------------------- */

/* Where a range loop of the VM runs (VirtualMachine.Loops.cs:111+), by the
 * rule of the reference's MLIR backend (InstructionsToMlir.cs:397-418):
 * complexity = iterations x max(body_instructions, 1), body_instructions
 * being the instructions between the loop's begin and end
 * (CountLoopBodyInstructions, :420-432); above SH_GPU_COMPLEXITY_THRESHOLD
 * the body runs as a generated GPU kernel (gpu.launch there), above
 * SH_PARALLEL_COMPLEXITY_THRESHOLD as a CPU-parallel loop (scf.parallel),
 * otherwise as a serial loop (scf.for). Negative arguments count as 0. */
#define SH_GPU_COMPLEXITY_THRESHOLD 10000000LL    /* GpuComplexityThreshold, :418 */
#define SH_PARALLEL_COMPLEXITY_THRESHOLD 100000LL /* ComplexityThreshold, :414 */
typedef enum sh_loop_target {
  SH_LOOP_SERIAL = 0,
  SH_LOOP_PARALLEL = 1,
  SH_LOOP_GPU = 2,
} sh_loop_target;
SH_API int sh_range_loop_target(long long iterations, int body_instructions);

/* ---- typed ops: elementwise ------------------------------------------------ */

typedef enum sh_binary_op {
  SH_ADD = 0,      /* InstructionsToCuda.cs:104 "+" */
  SH_SUBTRACT = 1, /* :105 "-" */
  SH_MULTIPLY = 2, /* :106 "*" */
  SH_DIVIDE = 3,   /* :107 "/" */
} sh_binary_op;

/* output[i] = first[i] OP second[i] for i < count: the kernel
 * InstructionsToCuda.BuildCudaKernel emits (InstructionsToCuda.cs:58-73),
 * with a linear index (the generator's `y * blockDim.x + x` aliases rows once
 * gridDim.x > 1). */
SH_API int sh_binary_f32(sh_ctx *ctx, int op, const float *first, const float *second,
                         float *output, size_t count);
/* output[i] = value: the generated `Process` kernel of InitializeDepths
 * (InstructionsToCuda.cs:79-96, Output/InitializeDepths.cu:5-11). */
SH_API int sh_fill_f32(sh_ctx *ctx, float value, float *output, size_t count);
/* out[i] = a * x[i] + y[i], product and sum rounded separately: the saxpy
 * Kernel.CompileKernelAndSaveAsPtxFile builds (Kernel.cs:22-28). */
SH_API int sh_saxpy_f32(sh_ctx *ctx, float a, const float *x, const float *y, float *out,
                        size_t n);
/* y[i] = 1 / (1 + exp(-x[i])): SigmoidPerformanceTests.cs:27 over an array
 * (the reference's GPU leg, RunGpu at :32, is an empty stub). <= 2 ulp. */
SH_API int sh_sigmoid_f32(sh_ctx *ctx, const float *x, float *y, size_t n);

/* ---- typed ops: image (interleaved 8-bit channels, row-major, no padding) -- */

#define SH_BRIGHTNESS_ALL_CHANNELS 1 /* also adjust the 4th (alpha) byte */

typedef enum sh_blur_mode {
  /* clamp-to-edge taps, (sum + 12) / 25 on every channel */
  SH_BLUR_CONFIG = 0,
  /* Assembly.Tests/BlurPerformanceTests.cs:85-141: in-bounds taps only,
   * sum / count truncating (interior count = 25) */
  SH_BLUR_REFERENCE = 1,
} sh_blur_mode;

/* p' = clamp(p + delta, 0, 255) on channels 0..2 of each pixel
 * (Assembly.Tests/BlurPerformanceTests.cs:287-294); channel 3 passes through
 * unless flags has SH_BRIGHTNESS_ALL_CHANNELS. in == out is allowed.
 * channels: 1..4 bytes per pixel; delta in [-255, 255]. */
SH_API int sh_adjust_brightness_u8(sh_ctx *ctx, const uint8_t *in, uint8_t *out, int width,
                                   int height, int channels, int delta, int flags);
/* 5x5 box blur of every channel; in and out must not overlap. */
SH_API int sh_box_blur5_u8(sh_ctx *ctx, const uint8_t *in, uint8_t *out, int width, int height,
                           int channels, int mode);
/* Brightness then blur in one pass (same bytes as the two calls in a row). */
SH_API int sh_brightness_blur5_u8(sh_ctx *ctx, const uint8_t *in, uint8_t *out, int width,
                                  int height, int channels, int delta, int flags, int mode);

/* ---- image layout adapters ----------------------------------------------------
 * The steps either side of the image kernels in the reference's blur test. */

/* Bitmap pixels to the test's RGBA byte image (CreateColorImageFromBitmapData,
 * Cuda.Tests/BlurPerformanceTests.cs:87-101): for each pixel, dst R, G, B =
 * src bytes 2, 1, 0 (BGR order), alpha 0 (the reference writes into a new,
 * zeroed array). bytes_per_pixel: 3 (24 bpp) or 4 (32 bpp, the fourth byte
 * ignored); rows src_stride bytes apart (the reference's pointer walks the
 * pixels without row padding: src_stride = width * bytes_per_pixel). dst holds
 * width * height * 4 bytes, 4-byte aligned; src and dst must not overlap;
 * height <= 65535 (for both adapters). */
SH_API int sh_bgr_to_rgba_u8(sh_ctx *ctx, const uint8_t *src, int bytes_per_pixel,
                             size_t src_stride, uint8_t *dst, int width, int height);
/* Packed RGB bytes to 24-bpp bitmap rows (SwitchRgbToBgr,
 * Cuda.Tests/BlurPerformanceTests.cs:191-213): dst[y * dst_stride + 3 x + c] =
 * src[3 (y * width + x) + 2 - c]; the row padding past 3 * width is left as it
 * was. dst_stride >= 3 * width; src and dst must not overlap. */
SH_API int sh_rgb_to_bgr_u8(sh_ctx *ctx, const uint8_t *src, uint8_t *dst, int width, int height,
                            size_t dst_stride);

/* ---- typed ops: dense GEMM --------------------------------------------------
 * The reference's only GEMM hook is the cuBLAS handle of Kernel.Handle
 * (Kernel.cs:10-11, :16), never used; BASELINE configs[2] fixes the op. */

/* C[M,N] = A[M,K] * B[K,N]: bf16 operands (raw 16-bit patterns), fp32
 * accumulation, bf16 result (round to nearest even), row-major with leading
 * dimensions lda >= K, ldb >= N, ldc >= N (elements). K == 0 writes zeros.
 * The MFMA path needs M, N multiples of 256, K of 64, lda/ldb multiples of 8
 * and 16-byte aligned A/B; other shapes run a slower exact-fp32 kernel. */
SH_API int sh_gemm_bf16(sh_ctx *ctx, const uint16_t *A, const uint16_t *B, uint16_t *C, int M,
                        int N, int K, int lda, int ldb, int ldc);

/* C[m,n] = bf16(sa[m] * sb[n] * sum_k e4m3(A[m,k]) * e4m3(Bt[n,k])): OCP E4M3
 * bytes, fp32 accumulation, bf16 result (round to nearest even). A is
 * row-major [M][K] (lda >= K bytes), B arrives transposed as Bt [N][K]
 * (ldb >= K bytes; a weight matrix W[N][K]), C row-major (ldc >= N
 * elements); sa (M floats) and sb (N floats) are the per-row / per-column
 * scales sh_quantize_e4m3 produces. K == 0 writes zeros. The MFMA path needs
 * M, N multiples of 256, K of 128, lda / ldb multiples of 16, 16-byte aligned
 * A, Bt and sb; other shapes run a slower exact-fp32 kernel. No counterpart in
 * the reference (BASELINE's FP8 GEMM measurement). */
SH_API int sh_gemm_fp8(sh_ctx *ctx, const uint8_t *A, const float *sa, const uint8_t *Bt,
                       const float *sb, uint16_t *C, int M, int N, int K, int lda, int ldb,
                       int ldc);

/* ---- weight quantization ------------------------------------------------------
 * No reference counterpart: BASELINE configs[4] fixes the format. */

/* Per-row OCP E4M3 quantization of a device fp32 matrix W[N][K]:
 * scale[n] = max_k |W[n][k]| / 448 (1 for an all-zero row), q = e4m3(W / scale)
 * rounded to nearest even and saturated to +-448, written row-major
 * (q[n * K + k]); K must be a multiple of 64. */
SH_API int sh_quantize_e4m3(sh_ctx *ctx, const float *W, int N, int K, uint8_t *q, float *scales);

/* Row-major E4M3 q[N][K] -> the tiled layout sh_gemv_w8a16 reads (16-row x
 * 64-column 1 KiB tiles in MFMA operand order; N % 16 == 0, K % 64 == 0). */
SH_API int sh_pack_e4m3_tiles(sh_ctx *ctx, const uint8_t *q, int N, int K, uint8_t *tiled);

/* W8A16 GEMV / skinny GEMM: y[b][n] = scale[n] * sum_k x[b][k] * e4m3(q[n][k])
 * for b < batch (1..16); x fp16 [batch][K], y fp32 [batch][N], fp32
 * accumulation of exact products. K % 256 == 0, N % 16 == 0, x and w_tiled
 * 16-byte aligned. */
SH_API int sh_gemv_w8a16(sh_ctx *ctx, const uint16_t *x, const uint8_t *w_tiled,
                         const float *scales, float *y, int batch, int K, int N);

/* ---- typed ops: decoder building blocks ---------------------------------------
 * No reference counterpart (Strict has no LLM path): the operations of the
 * GPT-2 and Qwen3 decoders, which the model runners below fuse into their
 * kernels, as ops on the caller's device buffers. fp32 in and out; the norms
 * take their statistics in fp64 and RoPE its cos / sin in fp64, every other
 * product and sum is rounded in fp32 on its own. */

/* y[r][i] = (x[r][i] * inv_r) * gain[i], inv_r = fp32(1 / sqrt(mean_i x[r][i]^2 + eps))
 * (RMSNorm), rows of n values. in-place (y == x) is allowed. */
SH_API int sh_rmsnorm_f32(sh_ctx *ctx, const float *x, const float *gain, float *y, int rows,
                          int n, float eps);
/* y[r][i] = ((x[r][i] - mean_r) * inv_r) * gain[i] + bias[i], inv_r = fp32(1 /
 * sqrt(var_r + eps)) (LayerNorm, population variance). y == x is allowed. */
SH_API int sh_layernorm_f32(sh_ctx *ctx, const float *x, const float *gain, const float *bias,
                            float *y, int rows, int n, float eps);
/* In place on x[rows][heads][head_dim]: rotate-half RoPE at positions[r]
 * (device int32 per row): for i < head_dim / 2, angle = fp32(pos) *
 * fp32(theta^(-2i / head_dim)), (x_i, x_{i+d/2}) <- (x_i c - x_{i+d/2} s,
 * x_{i+d/2} c + x_i s). head_dim even, <= 512. */
SH_API int sh_rope_f32(sh_ctx *ctx, float *x, const int32_t *positions, int rows, int heads,
                       int head_dim, float theta);
/* out[i] = silu(gate[i]) * up[i], silu(g) = g / (1 + exp(-g)) (SwiGLU). */
SH_API int sh_swiglu_f32(sh_ctx *ctx, const float *gate, const float *up, float *out, size_t n);
/* y[i] = 0.5 x (1 + tanh(sqrt(2 / pi) (x + 0.044715 x^3))) (GELU, tanh form). */
SH_API int sh_gelu_f32(sh_ctx *ctx, const float *x, float *y, size_t n);
/* index[r] = the first i of the largest x[r][i] (NaN counts as the largest,
 * as numpy.argmax), rows of n >= 1 values (greedy decoding). */
SH_API int sh_argmax_f32(sh_ctx *ctx, const float *x, int rows, int n, int32_t *index);
/* Decode attention, grouped-query: for row b and query head h (KV head
 * h / (heads / kv_heads)), with L = min(lengths[b], max_positions),
 *   out[b][h] = sum_p softmax_p(fp32(q[b][h] * scale) . k[b][kvh][p]) v[b][kvh][p],  p < L
 * (zeros for L <= 0). q, out fp32 [batch][heads][head_dim]; k, v fp16 [batch]
 * [kv_heads][max_positions][head_dim] (the runners' cache layout), 16-byte
 * aligned; lengths a device int32 [batch]. head_dim 64 or 128, heads /
 * kv_heads <= 16. Split-K over positions: the split partials go to the
 * context's work buffer (allocated on first use, grown on demand). */
SH_API int sh_attn_decode_f16(sh_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v,
                              const int32_t *lengths, float *out, int batch, int heads,
                              int kv_heads, int head_dim, int max_positions, float scale);

/* sh_attn_decode_f16 without any allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, kernels and results as sh_attn_decode_f16, but the split partials
 * go to a fixed device array of SH_ATTN_NOALLOC_MAX_BYTES per GPU, held from
 * the library's load until the process ends; calls whose partials
 * (batch * heads * splits * (head_dim + 2) * 4 bytes) exceed it fail with
 * SH_ERR_INVALID_ARGUMENT. Calls no hipMalloc / hipFree. Every call on one
 * GPU shares that GPU's array (nothing in it needs clearing between calls:
 * each call writes every partial it reads): calls that overlap on one GPU,
 * from different streams or contexts, race. */
#define SH_ATTN_NOALLOC_MAX_BYTES ((size_t)16 << 20)
SH_API int sh_attn_decode_f16_noalloc(sh_ctx *ctx, const float *q, const uint16_t *k,
                                      const uint16_t *v, const int32_t *lengths, float *out,
                                      int batch, int heads, int kv_heads, int head_dim,
                                      int max_positions, float scale);

/* ---- LLM decode (model runners) ------------------------------------------------
 * No reference counterpart: BASELINE configs[3] (GPT-2 small, fp16 weights)
 * and configs[4] (Qwen3-0.6B shape, FP8-E4M3 weights with per-output-channel
 * fp32 scales) define the models. One sh_llm owns its weights, KV cache and
 * work buffers on the context's device; steps are ordered on the context's
 * stream and replayed from a HIP graph after the first step of a batch. */

typedef enum sh_llm_arch {
  SH_LLM_QWEN3 = 0, /* RMSNorm, q/k head RMSNorm, RoPE (rotate-half), GQA, SwiGLU,
                       FP8 linears, FP8 LM head tied to the embedding */
  SH_LLM_GPT2 = 1,  /* LayerNorm, learned positions, MHA, GELU (tanh), biases,
                       fp16 linears, LM head tied to the token embedding */
} sh_llm_arch;

typedef struct sh_llm_config {
  int arch;
  int layers, hidden, heads, kv_heads, head_dim, intermediate, vocab;
  int max_positions; /* KV cache length per sequence (GPT-2: also the position table) */
  int max_batch;     /* 1..16 */
  float rope_theta;  /* Qwen3 */
  float norm_eps;
} sh_llm_config;

typedef struct sh_llm sh_llm;

SH_API int sh_llm_create(sh_ctx *ctx, const sh_llm_config *config, sh_llm **model);
SH_API int sh_llm_destroy(sh_llm *model);
/* Every linear (and the head / GPT-2 position table) ~ N(0, stddev) from a
 * counter-based generator seeded by `seed`, then quantized (Qwen3) or rounded
 * to fp16 (GPT-2); norm gains 1, biases 0. */
SH_API int sh_llm_init_random(sh_llm *model, uint64_t seed, float stddev);
/* Replaces one linear from a device fp32 matrix W[N][K] in logical row order.
 * name: "qkv" (rows q | k | v), "o", "gate_up" (Qwen3, rows gate | up), "fc"
 * (GPT-2), "down" (Qwen3) / "proj" (GPT-2), "head" (layer ignored; vocab
 * rounded up to a multiple of 16 rows, the padding rows zero). */
SH_API int sh_llm_load_linear(sh_llm *model, const char *name, int layer, const float *W);
/* Device address and size of a named tensor, for uploads and read-back:
 * "<linear>.w" (tiled layout), "<linear>.scale", "<linear>.bias", "norm1.g",
 * "norm1.b", "norm2.g", "norm2.b", "q_norm", "k_norm", "final.g", "final.b",
 * "wpe", "inv_freq", "kcache", "vcache" (per layer), "logits", "hist", "lens";
 * "layers.err" exists only when a persistent layers kernel runs the layers:
 * the Qwen3 decode-layers kernel (shapes it is built for, cooperative launch
 * available) or the GPT-2 layers kernel (batch 1), with STRICT_HIP_LLM_LAYERS
 * not "0" when the model is created. */
SH_API int sh_llm_tensor(sh_llm *model, const char *name, int layer, void **device_ptr,
                         size_t *bytes);
/* Starts `batch` empty sequences (clears the KV lengths, the greedy keys and
 * a failed step's error word). */
SH_API int sh_llm_reset(sh_llm *model, int batch);
/* One decode step for every sequence: embeds tokens[b] (host array) or, when
 * tokens is NULL, the greedy token the previous step produced; runs the layers;
 * with want_logits, the LM head writes logits and the greedy (argmax) token. */
SH_API int sh_llm_step(sh_llm *model, const int32_t *tokens, int want_logits);
/* Waits for the stream and copies the greedy tokens of the last step (host).
 * SH_ERR_HIP when a persistent layers kernel's wait between workgroups gave up
 * in a step since the last reset: the steps' state is lost and the model needs
 * sh_llm_reset (which also turns an XCD-local placement off for the rest of
 * the model's life if the failed step used it). */
SH_API int sh_llm_next_tokens(sh_llm *model, int32_t *tokens);
/* prompt[b * prompt_len + i] (host): prompt_len steps, then greedy decoding
 * until `steps` tokens per sequence are produced into out[b * steps + j]. */
SH_API int sh_llm_generate(sh_llm *model, const int32_t *prompt, int prompt_len, int steps,
                           int32_t *out);

#ifdef __cplusplus
}
#endif
#endif /* STRICT_HIP_H */
