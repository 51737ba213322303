"""GPU tests of the runtime half of the C ABI: contexts, buffers, hipRTC
modules and raw launches -- the ManagedCuda calls the reference's tests make
(CSharpToCudaTranspilerTests.cs:59-98, KernelTests.cs:8-12)."""
import ctypes

import numpy as np
import pytest

import oracle
import strict_amd

pytestmark = pytest.mark.gpu

ADD_KERNEL = r'''extern "C" __global__ void Add(const float *first, const float *second, float *output, const int count)
{
  int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= count) return;
  output[idx] = first[idx] + second[idx];
}'''

PROCESS_KERNEL = r'''extern "C" __global__ void Process(const float *input, const int width, const int height, const float initialDepth, float *output)
{
  int x = blockIdx.x * blockDim.x + threadIdx.x;
  int y = blockIdx.y * blockDim.y + threadIdx.y;
  if (x >= width || y >= height) return;
  output[y * width + x] = initialDepth;
}'''


def test_device_info(ctx):
    info = ctx.info()
    assert info["arch"].startswith("gfx950")
    assert info["compute_units"] >= 200 and info["wavefront_size"] == 64


def test_upload_download_roundtrip(ctx):
    a = np.arange(1 << 20, dtype=np.uint32)
    d = ctx.upload(a)
    assert np.array_equal(d.to_host(), a)
    c = ctx.empty(a.shape, np.uint32)
    ctx.copy(c, d)
    ctx.sync()
    assert np.array_equal(c.to_host(), a)
    ctx.memset(c, 0)
    ctx.sync()
    assert not c.to_host().any()
    d.free()
    c.free()


def test_double_free_and_foreign_pointer_are_errors(ctx):
    d = ctx.empty(256, np.uint8)
    p = d.ptr
    d.free()
    status = ctx._l.sh_free(ctx.handle, ctypes.c_void_p(p))
    assert status == strict_amd._lib.SH_ERR_INVALID_ARGUMENT
    assert b"double free" in ctx._l.sh_last_error()
    host = np.zeros(4, np.float32)
    status = ctx._l.sh_sigmoid_f32(ctx.handle, host.ctypes.data_as(ctypes.c_void_p),
                                   host.ctypes.data_as(ctypes.c_void_p), 4)
    assert status == strict_amd._lib.SH_ERR_INVALID_ARGUMENT  # host memory never reaches a kernel


def test_external_registration(ctx):
    d = ctx.empty(1024, np.float32)
    other = strict_amd.Context(0)
    try:
        with pytest.raises(strict_amd.StrictHipError):
            other.fill(1.0, d.ptr, 1024)  # not an allocation of `other`
        other.register_external(d.ptr, d.nbytes)
        other.fill(1.0, d.ptr, 1024)
        other.sync()
        assert np.all(d.to_host() == 1.0)
        other.unregister_external(d.ptr)
    finally:
        other.dispose()
        d.free()


@pytest.mark.parametrize("count", [1, 10, 1000])
def test_generated_add_kernel_through_modules(ctx, count):
    # ParseGenerateCudaAndExecute(AddNumbers, 3): compile, load, Run(first, second, output, count)
    with strict_amd.RuntimeCompiler(ADD_KERNEL, "AddNumbers") as rtc:
        rtc.compile()
        kernel = ctx.load_kernel(rtc.get_code(), "Add")
    first = ctx.upload(np.ones(count, np.float32))
    second = ctx.upload(np.full(count, 2.0, np.float32))
    output = ctx.empty(count, np.float32)
    kernel.block_dimensions = 256
    kernel.grid_dimensions = (count + 255) // 256
    ms = kernel.run(first, second, output, count)
    assert ms >= 0.0
    assert np.all(output.to_host() == 3.0)
    kernel.module.unload()


def test_generated_process_kernel_scalar_broadcast(ctx):
    # InitializeDepths -> Process(input, width=1, height=1, initialDepth=5) -> 5
    with strict_amd.RuntimeCompiler(PROCESS_KERNEL, "InitializeDepths") as rtc:
        rtc.compile()
        kernel = ctx.load_kernel(rtc.get_code(), "Process")
    inp = ctx.upload(np.ones(1, np.float32))
    out = ctx.empty(1, np.float32)
    kernel.run(inp, 1, 1, 5.0, out)  # default grid/block of 1, as ManagedCuda
    assert out.to_host()[0] == 5.0


def test_kernel_compile_saxpy_save_load_and_run(ctx, tmp_path):
    # KernelTests.CompileCudaCode + running the saved code object
    path = tmp_path / "VectorAdd.hsaco"
    with strict_amd.Kernel() as k:
        assert k.compile_kernel_and_save_code_object(str(path)) == 0
    code = path.read_bytes()
    fn = ctx.load_kernel(code, "saxpy")
    n = 100_000
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, n).astype(np.float32)
    y = rng.normal(0, 1, n).astype(np.float32)
    dx, dy, do = ctx.upload(x), ctx.upload(y), ctx.empty(n, np.float32)
    fn.block_dimensions = 256
    fn.grid_dimensions = (n + 255) // 256
    fn.run(2.5, dx, dy, do, ctypes.c_size_t(n))
    out = do.to_host()
    # the generic source may contract a*x+y into an FMA: compare within 1 ulp
    ref = oracle.saxpy_f32(2.5, x, y)
    assert np.max(np.abs(out - ref) / np.maximum(np.abs(ref), 1e-30)) < 1e-6 or \
        np.allclose(out, ref, rtol=1e-6, atol=1e-6)


def test_missing_kernel_name_is_not_found(ctx):
    with strict_amd.RuntimeCompiler(ADD_KERNEL, "AddNumbers") as rtc:
        rtc.compile()
        mod = ctx.load_module(rtc.get_code())
    with pytest.raises(strict_amd.StrictHipError) as e:
        mod.function("Subtract")
    assert e.value.status == strict_amd._lib.SH_ERR_NOT_FOUND
    mod.unload()


def test_launch_rejects_oversized_block(ctx):
    with strict_amd.RuntimeCompiler(ADD_KERNEL, "AddNumbers") as rtc:
        rtc.compile()
        fn = ctx.load_kernel(rtc.get_code(), "Add")
    fn.block_dimensions = (1024, 2, 1)
    d = ctx.empty(4, np.float32)
    with pytest.raises(strict_amd.StrictHipError) as e:
        fn.run(d, d, d, 1)
    assert e.value.status == strict_amd._lib.SH_ERR_INVALID_ARGUMENT
