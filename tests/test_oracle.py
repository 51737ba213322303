"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each oracle function is checked against the reference's own known answers
where they exist, and otherwise against an independent implementation
(numpy / scipy / torch CPU conversions) or against invariants chosen so that a
plausible slip (wrong rounding, dropped channel, swapped edge rule, sign)
fails. No test restates the oracle's formula.
"""
import math

import numpy as np
import pytest

import oracle


# --- generated elementwise kernels: CSharpToCudaTranspilerTests.cs:46-49 ----

@pytest.mark.parametrize("op,expected", [(oracle.ADD, 3.0), (oracle.SUBTRACT, -1.0),
                                         (oracle.MULTIPLY, 2.0)])
def test_binary_known_answers(op, expected):
    # ParseGenerateCudaAndExecute runs first = {1}, second = {2}, count = 1
    out = oracle.binary_f32(op, [1.0], [2.0])
    assert out[0] == expected


def test_binary_output_fixtures_n10():
    # Output/AddNumbers.cu:16-20,46 (N = 10, 1 + 2 == 3); MultiplyNumbers.cu (2)
    ones, twos = np.ones(10, np.float32), np.full(10, 2, np.float32)
    assert np.all(oracle.binary_f32(oracle.ADD, ones, twos) == 3.0)
    assert np.all(oracle.binary_f32(oracle.MULTIPLY, ones, twos) == 2.0)
    # SubtractNumbers.cu computes 2 - 1 == 1
    assert np.all(oracle.binary_f32(oracle.SUBTRACT, twos, ones) == 1.0)
    assert np.all(oracle.binary_f32(oracle.DIVIDE, ones, twos) == 0.5)


def test_fill_known_answer():
    # InitializeDepths -> Process(...) with initialDepth = 5 (CSharpToCudaTranspilerTests.cs:49, :85)
    assert np.all(oracle.fill_f32(5.0, 10) == 5.0)


def test_saxpy_rounds_product_first():
    # a*x + y with the product rounded (no FMA): pick values where FMA differs.
    a = np.float32(1.0 + 2.0 ** -12)
    x = np.array([1.0 + 2.0 ** -12], np.float32)
    y = np.array([-(1.0 + 2.0 ** -11)], np.float32)
    out = oracle.saxpy_f32(float(a), x, y)
    exact = float(a) * float(x[0]) + float(y[0])          # = 2^-24, what an FMA returns
    rounded_product = float(np.float32(float(a) * float(x[0])))
    assert exact == 2.0 ** -24
    assert out[0] == np.float32(rounded_product + float(y[0]))
    assert out[0] == 0.0


# --- sigmoid: SigmoidPerformanceTests.cs:27 --------------------------------

def test_sigmoid_special_values():
    x = np.array([0.0, 0.265, 8.0, -8.0, 20.0, -20.0, -100.0], np.float32)
    y = oracle.sigmoid_f32(x)
    assert y[0] == 0.5
    # the reference's own input, Input = 0.265f (:31)
    assert abs(float(y[1]) - 1.0 / (1.0 + math.exp(-0.265))) < 1e-7
    assert y[4] == 1.0 and y[5] > 0 and y[6] >= 0


def test_sigmoid_against_scipy_expit():
    from scipy.special import expit

    rng = np.random.default_rng(1)
    x = rng.uniform(-8, 8, 200_000).astype(np.float32)
    y = oracle.sigmoid_f32(x)
    ref = expit(x.astype(np.float64))
    # The reference rounds three times (exp -> float, the add, the divide); each
    # contributes at most 2^-24 relative error (the exp term is damped by
    # e / (1 + e) < 1), so the formula sits within 3 * 2^-24 of the exact value.
    rel = np.abs(y.astype(np.float64) - ref) / ref
    assert np.max(rel) <= 3 * 2.0 ** -24 * (1 + 1e-9)
    # and most results are the correctly rounded value
    assert np.mean(y == ref.astype(np.float32)) > 0.5


def test_sigmoid_symmetry_and_monotone():
    x = np.linspace(-8, 8, 100_001, dtype=np.float32)
    y = oracle.sigmoid_f32(x)
    assert np.all(np.diff(y) >= 0)
    ys = oracle.sigmoid_f32(-x)
    assert np.max(np.abs((y + ys) - 1.0)) < 2e-7


def test_sigmoid_parallel_equals_serial():
    x = np.random.default_rng(2).uniform(-8, 8, 100_003).astype(np.float32)
    assert np.array_equal(oracle.sigmoid_f32(x, 1), oracle.sigmoid_f32(x, 7))


# --- brightness: BlurPerformanceTests.cs:287-294, README.md:436-443 ------------

def test_brightness_readme_known_answers():
    # Color(0, 1, 2) + 5 -> (5, 6, 7); (0, 0, 0) - 5 -> (0, 0, 0); + 0 identity
    px = np.array([0, 1, 2], np.uint8)
    assert list(oracle.adjust_brightness(px, 5, channels=3)) == [5, 6, 7]
    assert list(oracle.adjust_brightness(px, 0, channels=3)) == [0, 1, 2]
    assert list(oracle.adjust_brightness(np.zeros(3, np.uint8), 5, channels=3)) == [5, 5, 5]
    assert list(oracle.adjust_brightness(np.zeros(3, np.uint8), -5, channels=3)) == [0, 0, 0]


def test_brightness_saturation_points_and_alpha():
    v = np.arange(256, dtype=np.uint8)
    img = np.stack([v, v, v, v], axis=1).reshape(-1)
    up = oracle.adjust_brightness(img, 40, channels=4).reshape(256, 4)
    down = oracle.adjust_brightness(img, -40, channels=4).reshape(256, 4)
    assert np.all(up[:, 3] == v) and np.all(down[:, 3] == v)          # alpha passes through
    assert up[215, 0] == 255 and up[214, 0] == 254 and up[255, 0] == 255
    assert down[40, 0] == 0 and down[41, 0] == 1 and down[0, 0] == 0
    assert np.all(np.diff(up[:, :3].astype(int), axis=0) >= 0)       # monotone
    both = oracle.adjust_brightness(img, 40, channels=4, all_channels=True).reshape(256, 4)
    assert np.array_equal(both[:, 3], up[:, 0])


# --- blur: independent sums from scipy.ndimage ---------------------------------

def _scipy_box_sums(img, w, h, c, mode):
    from scipy import ndimage

    a = img.reshape(h, w, c).astype(np.int64)
    k = np.ones((5, 5, 1), np.int64)
    if mode == "config":
        return ndimage.correlate(a, k, mode="nearest"), None
    sums = ndimage.correlate(a, k, mode="constant", cval=0)
    counts = ndimage.correlate(np.ones((h, w, 1), np.int64), k, mode="constant", cval=0)
    return sums, counts


@pytest.mark.parametrize("w,h,c", [(1, 1, 4), (2, 3, 3), (5, 5, 4), (10, 10, 3), (20, 20, 3),
                                   (17, 9, 4), (33, 6, 1)])
def test_blur_config_matches_scipy_nearest(w, h, c):
    img = np.random.default_rng(w * 100 + h).integers(0, 256, w * h * c, dtype=np.uint8)
    sums, _ = _scipy_box_sums(img, w, h, c, "config")
    expected = ((sums + 12) // 25).astype(np.uint8).reshape(-1)
    assert np.array_equal(oracle.blur5_config(img, w, h, c), expected)


@pytest.mark.parametrize("w,h,c", [(1, 1, 3), (2, 3, 3), (5, 5, 4), (10, 10, 3), (20, 20, 3),
                                   (17, 9, 4)])
def test_blur_reference_matches_scipy_inbounds_average(w, h, c):
    img = np.random.default_rng(w * 7 + h).integers(0, 256, w * h * c, dtype=np.uint8)
    sums, counts = _scipy_box_sums(img, w, h, c, "reference")
    expected = (sums // counts).astype(np.uint8).reshape(-1)
    assert np.array_equal(oracle.blur5_reference(img, w, h, c), expected)


@pytest.mark.parametrize("size", [10, 20])
def test_blur_parallel_equals_serial(size):
    # BlurProducesCorrectResults (Assembly BlurPerformanceTests.cs:193-206), 3-byte RGB
    img = np.random.default_rng(42).integers(0, 256, size * size * 3, dtype=np.uint8)
    assert np.array_equal(oracle.blur5_reference(img, size, size, 3, nthreads=1),
                          oracle.blur5_reference(img, size, size, 3, nthreads=4))


def test_blur_invariants():
    const = np.full(12 * 9 * 4, 77, np.uint8)
    assert np.all(oracle.blur5_config(const, 12, 9) == 77)
    assert np.all(oracle.blur5_reference(const, 12, 9) == 77)
    imp = np.zeros((9, 9, 4), np.uint8)
    imp[4, 4, 1] = 255
    out = oracle.blur5_config(imp.reshape(-1), 9, 9).reshape(9, 9, 4)
    assert np.all(out[2:7, 2:7, 1] == (255 + 12) // 25) and out[1, 4, 1] == 0
    assert np.all(out[..., 0] == 0)
    ref = oracle.blur5_reference(imp.reshape(-1), 9, 9).reshape(9, 9, 4)
    assert np.all(ref[2:7, 2:7, 1] == 255 // 25)


def test_brightness_blur_fused_is_two_passes():
    w, h = 13, 11
    img = np.random.default_rng(5).integers(0, 256, w * h * 4, dtype=np.uint8)
    two = oracle.blur5_config(oracle.adjust_brightness(img, -40), w, h)
    assert np.array_equal(oracle.brightness_blur5_config(img, w, h, -40), two)


# --- number formats vs independent converters -----------------------------------

def _interesting_floats(n=200_000, seed=3):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    extra = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 6.1035156e-05,
                      5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-10, 3.0e38], np.float32)
    return np.concatenate([f, extra, rng.normal(0, 1, 50_000).astype(np.float32)])


def test_f16_matches_numpy():
    f = _interesting_floats()
    ours = oracle.f32_to_f16(f)
    ref = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)
    allh = np.arange(65536, dtype=np.uint16)
    back = oracle.f16_to_f32(allh)
    ref_back = allh.view(np.float16).astype(np.float32)
    same = (back.view(np.uint32) == ref_back.view(np.uint32)) | (np.isnan(back) & np.isnan(ref_back))
    assert np.all(same)


def test_bf16_matches_torch():
    import torch

    f = _interesting_floats()
    ours = oracle.f32_to_bf16(f)
    ref = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    back = oracle.bf16_to_f32(ours)
    assert np.array_equal(back, torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16)
                          .float().numpy())


def test_e4m3_decode_matches_torch_and_spec():
    import torch

    codes = np.arange(256, dtype=np.uint8)
    ours = oracle.e4m3_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    finite = ~np.isnan(ref)
    assert np.array_equal(ours[finite], ref[finite])
    assert np.isnan(ours[0x7F]) and np.isnan(ours[0xFF]) and finite.sum() == 254
    # OCP E4M3 landmarks: max normal 448, min normal 2^-6, min subnormal 2^-9
    assert ours[0x7E] == 448.0 and ours[0x08] == 2.0 ** -6 and ours[0x01] == 2.0 ** -9


def test_e4m3_encode_matches_torch_in_range():
    import torch

    rng = np.random.default_rng(4)
    f = np.concatenate([rng.uniform(-448, 448, 20_000), rng.normal(0, 1, 20_000),
                        rng.normal(0, 0.01, 5_000)]).astype(np.float32)
    # exact midpoints between neighbouring codes test ties-to-even
    vals = oracle.e4m3_to_f32(np.arange(0, 0x7E, dtype=np.uint8))
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    f = np.concatenate([f, mids, -mids])
    ours = np.array([oracle.f32_to_e4m3_scalar(float(x)) for x in f], np.uint8)
    ref = torch.from_numpy(f).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    assert oracle.f32_to_e4m3_scalar(1000.0) == 0x7E and oracle.f32_to_e4m3_scalar(-1e9) == 0xFE


def test_quantize_rows_roundtrip():
    w = np.random.default_rng(6).normal(0, 0.02, (64, 333)).astype(np.float32)
    w[3] = 0
    q, s = oracle.quantize_e4m3_rows(w)
    assert s[3] == 1.0 and np.all(q[3] == 0)
    deq = oracle.e4m3_to_f32(q) * s[:, None]
    nz = np.abs(w) > 1e-3
    assert np.max(np.abs(deq - w)[nz] / np.abs(w)[nz]) <= 2.0 ** -4 + 1e-6
    rows = [i for i in range(64) if i != 3]
    assert np.all(np.max(q[rows] & 0x7F, axis=1) == 0x7E)  # the row max maps to 448


def test_gemm_matches_numpy():
    rng = np.random.default_rng(7)
    a = rng.normal(0, 1, (37, 53)).astype(np.float32)
    b = rng.normal(0, 1, (53, 29)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert np.max(np.abs(oracle.gemm_f32(a, b) - ref)) < 1e-5
    eye = np.eye(53, dtype=np.float32)
    assert np.array_equal(oracle.gemm_f32(a, eye), a)


# ---- TestPerformance's CPU modes and the CUDA harness's cross blur ------------------

def _chunked_prefix(n, mode, chunk=oracle.CHUNK_SIZE):
    """Indices a mode computes: all of them, or whole chunks only (Iterations /
    ChunkSize chunks, TestPerformance.cs:41, :48)."""
    return n if mode in (0, 2) else n // chunk * chunk


@pytest.mark.parametrize("mode", range(4))
def test_perf_modes_sigmoid_equal_the_array_oracle(mode):
    # every mode computes SigmoidPerformanceTests.cs:27 per element: the same
    # bits as or_sigmoid_f32 on the indices it covers (parallel == serial)
    x = np.random.default_rng(1).uniform(-8, 8, 100_037).astype(np.float32)
    y = np.full_like(x, np.nan)
    oracle.perf_sigmoid(mode, x, y, nthreads=4)
    n = _chunked_prefix(x.size, mode)
    ref = oracle.sigmoid_f32(x)
    assert np.array_equal(y[:n].view(np.uint32), ref[:n].view(np.uint32))
    assert np.all(np.isnan(y[n:]))


@pytest.mark.parametrize("mode", range(4))
def test_perf_modes_brightness_and_blurs_equal_the_image_oracles(mode):
    w, h = 61, 23
    img = np.random.default_rng(2).integers(0, 256, w * h * 4, dtype=np.uint8)
    n = _chunked_prefix(w * h, mode)
    out = np.zeros_like(img)
    oracle.perf_brightness(mode, img, out, 4, -40, nthreads=3)
    assert np.array_equal(out[:n * 4], oracle.adjust_brightness(img, -40, 4)[:n * 4])
    cases = [(oracle.BLUR_REFERENCE, 0, oracle.blur5_reference(img, w, h, 4)),
             (oracle.BLUR_CONFIG, 0, oracle.blur5_config(img, w, h, 4)),
             (oracle.BLUR_FUSED, 40, oracle.brightness_blur5_config(img, w, h, 40, 4))]
    for kind, delta, ref in cases:
        out = np.zeros_like(img)
        oracle.perf_blur5(mode, kind, img, out, w, h, 4, nthreads=3, delta=delta)
        assert np.array_equal(out[:n * 4], ref[:n * 4]), kind
        assert not out[n * 4:].any()


@pytest.mark.parametrize("mode", range(4))
def test_perf_blur5_from_covers_the_tail_rows(mode):
    # the CPU share of CudaGpuAndCpu: output pixels [first, first + pixels)
    # of the whole image, its clamp-to-edge / in-bounds taps reaching above
    # `first`; pixels outside the range untouched
    w, h = 37, 29
    img = np.random.default_rng(3).integers(0, 256, w * h * 4, dtype=np.uint8)
    first = 25 * w + 3
    n = _chunked_prefix(w * h - first, mode)
    for kind, delta, ref in [(oracle.BLUR_REFERENCE, 0, oracle.blur5_reference(img, w, h, 4)),
                             (oracle.BLUR_CONFIG, 0, oracle.blur5_config(img, w, h, 4)),
                             (oracle.BLUR_FUSED, -40,
                              oracle.brightness_blur5_config(img, w, h, -40, 4))]:
        out = np.zeros_like(img)
        oracle.perf_blur5_from(mode, kind, img, out, w, h, 4, nthreads=3, first=first,
                               pixels=w * h - first, delta=delta)
        lo, hi = first * 4, (first + n) * 4
        assert np.array_equal(out[lo:hi], ref[lo:hi]), kind
        assert not out[:lo].any() and not out[hi:].any()


def test_cross_blur_hand_worked_single_thread():
    # Cuda.Tests/BlurPerformanceTests.cs:160-169 worked by hand on a 2x1 RGBA
    # image (size 8, width * 4 = 8): indices 0..7 are skipped (:162), and for
    # n >= 8 the five taps are n % 8 three times and (n + 4) % 8 twice, so
    # b[n % 8] = (3 b[n % 8] + 2 b[(n + 4) % 8]) / 5, in place:
    #   n=8: b0 = (30 + 100) / 5 = 26   n=12: b4 = (150 + 2*26) / 5 = 40
    #   n=9: b1 = (60 + 120) / 5 = 36   n=13: b5 = (180 + 2*36) / 5 = 50
    #  n=10: b2 = (90 + 140) / 5 = 46   n=14: b6 = (210 + 2*46) / 5 = 60
    #  n=11: b3 = (120 + 160) / 5 = 56  n=15: b7 = (240 + 2*56) / 5 = 70
    img = np.array([10, 20, 30, 40, 50, 60, 70, 80], np.uint8)
    oracle.perf_cross_blur(oracle.PERF_MODES.index("SingleThread"), img, 2, 1, 16, nthreads=1)
    assert img.tolist() == [26, 36, 46, 56, 40, 50, 60, 70]


def test_cross_blur_hand_worked_chunks_skip_whole_chunks():
    # SingleThreadChunks with ChunkSize 5 and 20 iterations: chunks start at
    # 0, 5, 10, 15; the chunks at 0 and 5 start below width * 4 = 8 and are
    # skipped whole (so n = 8, 9 never run), then n = 10..19 in order:
    #  n=10: b2 = (90 + 2*70) / 5 = 46   n=15: b7 = (240 + 2*56) / 5 = 70
    #  n=11: b3 = (120 + 2*80) / 5 = 56  n=16: b0 = (30 + 2*34) / 5 = 19
    #  n=12: b4 = (150 + 2*10) / 5 = 34  n=17: b1 = (60 + 2*44) / 5 = 29
    #  n=13: b5 = (180 + 2*20) / 5 = 44  n=18: b2 = (138 + 2*60) / 5 = 51
    #  n=14: b6 = (210 + 2*46) / 5 = 60  n=19: b3 = (168 + 2*70) / 5 = 61
    img = np.array([10, 20, 30, 40, 50, 60, 70, 80], np.uint8)
    oracle.perf_cross_blur(oracle.PERF_MODES.index("SingleThreadChunks"), img, 2, 1, 20,
                           nthreads=1, chunk=5)
    assert img.tolist() == [19, 29, 51, 61, 34, 44, 60, 70]


@pytest.mark.parametrize("mode", range(4))
def test_cross_blur_keeps_a_constant_image(mode):
    # five equal taps average to the same value, in every mode (even racing)
    img = np.full(64 * 32 * 4, 173, np.uint8)
    oracle.perf_cross_blur(mode, img, 64, 32, 64 * 32 * 4 * 3, nthreads=4)
    assert np.all(img == 173)
