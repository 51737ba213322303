"""GPU parity of the FP8 GEMM (sh_gemm_fp8) against the oracle.

C[m,n] = sa[m] * sb[n] * sum_k e4m3(A[m,k]) * e4m3(Bt[n,k]), fp32 accumulation,
bf16 output; A and Bt quantized per row (oracle.quantize_e4m3_rows, the same
rule as sh_quantize_e4m3). The reference has no GEMM; BASELINE's FP8 GEMM
measurement fixes 4096^3 with per-row / per-column scales. Reference product:
the dequantized operands multiplied with double accumulation (oracle.gemm_f32).
Tolerance, as for the bf16 GEMM:
  max |C_gpu - C_ref| <= 1e-2 * max |C_ref|  and  ||C_gpu - C_ref|| <= 1e-2 ||C_ref||.
"""
import numpy as np
import pytest

import oracle
import strict_amd

pytestmark = pytest.mark.gpu


def _operands(m, n, k, seed):
    rng = np.random.default_rng(seed)
    qa, sa = oracle.quantize_e4m3_rows(rng.normal(0, 0.02, (m, k)).astype(np.float32))
    qb, sb = oracle.quantize_e4m3_rows(rng.normal(0, 0.02, (n, k)).astype(np.float32))
    return qa, sa, qb, sb


def _reference(qa, sa, qb, sb):
    a = oracle.e4m3_to_f32(qa) * sa[:, None]
    bt = oracle.e4m3_to_f32(qb) * sb[:, None]
    return oracle.gemm_f32(a, np.ascontiguousarray(bt.T))


def _run(ctx, qa, sa, qb, sb, m, n, k, lda=None, ldb=None, ldc=None):
    dev = [ctx.upload(x) for x in (qa, sa, qb, sb)]
    ldc_ = n if ldc is None else ldc
    dc = ctx.empty((max(m, 1), ldc_), np.uint16)
    ctx.gemm_fp8(dev[0], dev[1], dev[2], dev[3], dc, m, n, k, lda, ldb, ldc_)
    ctx.sync()
    c = dc.to_host()
    for v in dev + [dc]:
        v.free()
    return c


def _check(c_bits, ref):
    c = oracle.bf16_to_f32(c_bits)
    err = np.abs(c - ref)
    scale = np.abs(ref).max()
    assert err.max() <= 1e-2 * scale, (err.max(), scale)
    assert np.linalg.norm(c - ref) <= 1e-2 * np.linalg.norm(ref)
    return float(err.max() / scale)


def test_gemm_fp8_4096_config(ctx):
    m = n = k = 4096
    qa, sa, qb, sb = _operands(m, n, k, seed=42)
    c = _run(ctx, qa, sa, qb, sb, m, n, k)
    rows = np.random.default_rng(1).choice(m, 48, replace=False)
    ref_rows = _reference(qa[rows], sa[rows], qb, sb)
    rel = _check(c[rows], ref_rows)
    print(f"gemm_fp8 4096^3 max err / max |C| = {rel:.3e}")


@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (512, 768, 384), (768, 512, 4096),
                                   (1024, 2048, 256)])
def test_gemm_fp8_mfma_shapes(ctx, m, n, k):
    qa, sa, qb, sb = _operands(m, n, k, seed=m + n + k)
    _check(_run(ctx, qa, sa, qb, sb, m, n, k), _reference(qa, sa, qb, sb))


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (100, 37, 50), (3, 300, 7), (257, 255, 129),
                                   (256, 256, 64)])
def test_gemm_fp8_generic_shapes(ctx, m, n, k):
    qa, sa, qb, sb = _operands(m, n, k, seed=m * 7 + n)
    _check(_run(ctx, qa, sa, qb, sb, m, n, k), _reference(qa, sa, qb, sb))


def test_gemm_fp8_leading_dimensions(ctx):
    m, n, k, lda, ldb, ldc = 256, 256, 256, 272, 288, 264
    rng = np.random.default_rng(3)
    qa, sa, qb, sb = _operands(m, n, k, seed=5)
    pa = np.zeros((m, lda), np.uint8)
    pa[:, :k] = qa
    pa[:, k:] = rng.integers(0, 256, (m, lda - k))  # padding never read
    pb = np.zeros((n, ldb), np.uint8)
    pb[:, :k] = qb
    pb[:, k:] = rng.integers(0, 256, (n, ldb - k))
    c = _run(ctx, pa, sa, pb, sb, m, n, k, lda, ldb, ldc)
    _check(c[:, :n], _reference(qa, sa, qb, sb))


def test_gemm_fp8_device_quantized_pipeline(ctx):
    # sh_quantize_e4m3 on both operands, then the GEMM: the oracle quantizes
    # the same fp32 matrices (bit-exact rule) and multiplies in double
    m, n, k = 512, 256, 512
    rng = np.random.default_rng(9)
    a = rng.normal(0, 0.05, (m, k)).astype(np.float32)
    bt = rng.normal(0, 0.05, (n, k)).astype(np.float32)
    da, dbt = ctx.upload(a), ctx.upload(bt)
    qa, sa = ctx.empty((m, k), np.uint8), ctx.empty(m, np.float32)
    qb, sb = ctx.empty((n, k), np.uint8), ctx.empty(n, np.float32)
    ctx.quantize_e4m3(da, qa, sa, m, k)
    ctx.quantize_e4m3(dbt, qb, sb, n, k)
    c = ctx.empty((m, n), np.uint16)
    ctx.gemm_fp8(qa, sa, qb, sb, c, m, n, k)
    ctx.sync()
    oqa, osa = oracle.quantize_e4m3_rows(a)
    oqb, osb = oracle.quantize_e4m3_rows(bt)
    assert np.array_equal(qa.to_host(), oqa) and np.array_equal(qb.to_host(), oqb)
    _check(c.to_host(), _reference(oqa, osa, oqb, osb))


def test_gemm_fp8_k0_and_bad_arguments(ctx):
    m, n = 256, 256
    c = ctx.upload(np.full((m, n), 0x3F80, np.uint16))
    a = ctx.empty(16, np.uint8)
    s = ctx.upload(np.ones(max(m, n), np.float32))
    ctx.gemm_fp8(a, s, a, s, c, m, n, 0, 1, 1, n)
    ctx.sync()
    assert not c.to_host().any()  # empty sum
    with pytest.raises(strict_amd.StrictHipError) as e:
        ctx.gemm_fp8(a, s, a, s, c, m, n, 64, 32, 64, n)  # lda < K
    assert e.value.status == strict_amd._lib.SH_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 4096), (512, 768, 384)])
def test_gemm_fp8_hipblaslt_yardstick(ctx, m, n, k):
    # the bench's vendor yardstick (a library of its own, not in libstrict_hip), same bar
    from strict_amd import yardstick

    qa, sa, qb, sb = _operands(m, n, k, seed=13)
    dev = [ctx.upload(x) for x in (qa, sa, qb, sb)]
    dc = ctx.empty((m, n), np.uint16)
    yardstick.gemm_fp8(ctx, dev[0], dev[1], dev[2], dev[3], dc, m, n, k)
    ctx.sync()
    c = dc.to_host()
    for v in dev + [dc]:
        v.free()
    rows = np.random.default_rng(2).choice(m, 48, replace=False)
    _check(c[rows], _reference(qa[rows], sa[rows], qb, sb))
