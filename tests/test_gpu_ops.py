"""GPU parity of the standalone decoder ops (sh_rmsnorm_f32, sh_layernorm_f32,
sh_rope_f32, sh_swiglu_f32, sh_gelu_f32, sh_argmax_f32, sh_attn_decode_f16)
against the oracle (oracle/llm.py), each op on its own buffers.

The reference has no implementation of any of them; the GPT-2 and Qwen3
decoders define them. Bars, stated per test:
  - RMSNorm, LayerNorm, RoPE: the GPU takes the oracle's rounding points
    (fp64 statistics, fp64 cos / sin, each fp32 product and sum rounded), so
    at most 1 ulp apart (an fp64 sum in another order can flip the last bit
    of the fp32 scale);
  - SwiGLU: at most 8 ulp of the result (the device's expf and numpy's
    float32 exp each err by up to a few ulp, and the divide and the product
    by up to half an ulp each);
  - GELU: |gpu - oracle| <= 4 ulp(1) * |x| (1 + tanh cancels near the
    negative tail, so the error is bounded relative to x, not the result);
  - argmax: identical indices (first maximum, NaN largest);
  - attention: max |gpu - oracle| <= 1e-2 * max |oracle| (the attention bar),
    the measured error printed.
"""
import numpy as np
import pytest

import oracle.llm as ollm
import strict_amd

pytestmark = pytest.mark.gpu


def _ulps(a, b):
    ai = a.astype(np.float32).view(np.int32).astype(np.int64)
    bi = b.astype(np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


def _run(ctx, fn, *host_in, out_shapes):
    dev_in = [ctx.upload(np.ascontiguousarray(h)) for h in host_in]
    dev_out = [ctx.empty(shape, dtype) for shape, dtype in out_shapes]
    fn(*dev_in, *dev_out)
    ctx.sync()
    res = [o.to_host() for o in dev_out]
    for v in dev_in + dev_out:
        v.free()
    return res


@pytest.mark.parametrize("rows,n", [(7, 1024), (3, 3000), (1, 1), (2, 768)])
def test_rmsnorm_vs_oracle(ctx, rows, n):
    rng = np.random.default_rng(rows * n)
    x = rng.normal(0, 3, (rows, n)).astype(np.float32)
    g = (1 + rng.normal(0, 0.2, n)).astype(np.float32)
    eps = float(np.float32(1e-6))
    (y,) = _run(ctx, lambda dx, dg, dy: ctx.rmsnorm(dx, dg, dy, rows, n, eps), x, g,
                out_shapes=[((rows, n), np.float32)])
    ref = ollm.rms_norm(x, g, eps)
    u = _ulps(y, ref)
    print(f"rmsnorm {rows}x{n}: max {u.max()} ulp, {np.mean(u == 0):.4f} bit-exact")
    assert u.max() <= 1


def test_rmsnorm_in_place(ctx):
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (4, 512)).astype(np.float32)
    g = np.ones(512, np.float32)
    dx, dg = ctx.upload(x), ctx.upload(g)
    ctx.rmsnorm(dx, dg, dx, 4, 512, 1e-6)
    ctx.sync()
    assert _ulps(dx.to_host(), ollm.rms_norm(x, g, float(np.float32(1e-6)))).max() <= 1
    dx.free()
    dg.free()


@pytest.mark.parametrize("rows,n", [(5, 768), (2, 1000)])
def test_layernorm_vs_oracle(ctx, rows, n):
    rng = np.random.default_rng(rows + n)
    x = (rng.normal(0, 2, (rows, n)) + 3).astype(np.float32)
    g = (1 + rng.normal(0, 0.2, n)).astype(np.float32)
    b = rng.normal(0, 0.3, n).astype(np.float32)
    eps = float(np.float32(1e-5))
    (y,) = _run(ctx, lambda dx, dg, db, dy: ctx.layernorm(dx, dg, db, dy, rows, n, eps), x, g, b,
                out_shapes=[((rows, n), np.float32)])
    u = _ulps(y, ollm.layer_norm(x, g, b, eps))
    print(f"layernorm {rows}x{n}: max {u.max()} ulp, {np.mean(u == 0):.4f} bit-exact")
    assert u.max() <= 1


@pytest.mark.parametrize("heads,d,theta", [(16, 128, 1e6), (12, 64, 1e4)])
def test_rope_vs_oracle(ctx, heads, d, theta):
    rng = np.random.default_rng(heads)
    positions = np.array([0, 1, 7, 4095, 4351, 65535, 1_000_003], np.int32)
    rows = positions.size
    x = rng.normal(0, 1, (rows, heads, d)).astype(np.float32)
    dx, dp = ctx.upload(x), ctx.upload(positions)
    ctx.rope(dx, dp, rows, heads, d, theta)
    ctx.sync()
    y = dx.to_host()
    dx.free()
    dp.free()
    cos, sin = ollm.rope_tables(ollm.inv_freq(theta, d), positions)
    u = _ulps(y, ollm.rope(x, cos, sin))
    print(f"rope heads={heads} d={d}: max {u.max()} ulp, {np.mean(u == 0):.4f} bit-exact")
    assert u.max() <= 1


def test_swiglu_and_gelu_vs_oracle(ctx):
    rng = np.random.default_rng(2)
    n = 1 << 20
    gate = rng.normal(0, 4, n).astype(np.float32)
    gate[:6] = [0.0, -0.0, 30.0, -30.0, 88.0, -88.0]
    up = rng.normal(0, 2, n).astype(np.float32)
    (y,) = _run(ctx, lambda dg, du, dy: ctx.swiglu(dg, du, dy, n), gate, up,
                out_shapes=[((n,), np.float32)])
    ref = ollm.silu(gate) * up
    u = _ulps(y, ref)
    print(f"swiglu: max {u.max()} ulp, {np.mean(u == 0):.4f} bit-exact, {np.sum(u > 2)} above 2 ulp "
          f"(worst at gate={gate[np.argmax(u)]!r})")
    assert u.max() <= 8
    x = np.concatenate([np.linspace(-10, 10, 200_001), rng.normal(0, 3, n)]).astype(np.float32)
    (y,) = _run(ctx, lambda dx, dy: ctx.gelu(dx, dy, x.size), x,
                out_shapes=[((x.size,), np.float32)])
    err = np.abs(y.astype(np.float64) - ollm.gelu_tanh(x).astype(np.float64))
    bound = 4 * 2.0 ** -23 * np.abs(x.astype(np.float64)) + 1e-30
    print(f"gelu: max |err| / (ulp(1) |x|) = {np.max(err / (2.0 ** -23 * np.abs(x) + 1e-30)):.2f}")
    assert np.all(err <= bound)


def test_argmax_vs_numpy(ctx):
    rng = np.random.default_rng(3)
    rows, n = 8, 151936
    x = rng.normal(0, 1, (rows, n)).astype(np.float32)
    x[1, [5, 900, 151000]] = 9.0           # ties: the first wins
    x[2, :] = -np.inf                      # all -inf: index 0
    x[3, 77] = np.nan                      # NaN counts as the largest
    x[3, 500] = np.inf
    x[4, n - 1] = 50.0                     # the last column
    x[5, :] = 0.0
    x[5, 3] = -0.0                         # zeros: the first
    (idx,) = _run(ctx, lambda dx, di: ctx.argmax(dx, rows, n, di), x,
                  out_shapes=[((rows,), np.int32)])
    assert np.array_equal(idx, np.argmax(x, axis=1).astype(np.int32))


@pytest.mark.parametrize("batch,heads,kv_heads,d,max_pos,lengths", [
    (1, 16, 8, 128, 4096, [4096]),                 # configs[4] shape, full cache
    (3, 16, 8, 128, 4133, [1, 4133, 2000]),        # ragged, a partial last tile
    (4, 12, 12, 64, 384, [384, 0, 129, 64]),       # GPT-2 MHA, an empty row
    (2, 16, 1, 128, 300, [300, 65]),               # 16 query heads on one KV head
    (16, 16, 8, 128, 1024, list(range(60, 1024, 60))[:16]),
])
def test_attn_decode_vs_oracle(ctx, batch, heads, kv_heads, d, max_pos, lengths):
    rng = np.random.default_rng(batch * 1000 + heads + max_pos)
    q = rng.normal(0, 1, (batch, heads, d)).astype(np.float32)
    k = rng.normal(0, 1, (batch, kv_heads, max_pos, d)).astype(np.float16)
    v = rng.normal(0, 1, (batch, kv_heads, max_pos, d)).astype(np.float16)
    lens = np.array(lengths, np.int32)
    scale = float(1 / np.sqrt(d))
    (out,) = _run(ctx, lambda dq, dk, dv, dl, do: ctx.attn_decode(
        dq, dk, dv, dl, do, batch, heads, kv_heads, d, max_pos, scale),
        q, k.view(np.uint16), v.view(np.uint16), lens,
        out_shapes=[((batch, heads, d), np.float32)])
    ref = ollm.attn_decode(q, k.astype(np.float32), v.astype(np.float32), lens, scale)
    rel = float(np.max(np.abs(out - ref)) / np.max(np.abs(ref)))
    print(f"attn b={batch} h={heads}/{kv_heads} d={d} P={max_pos}: max err / max |ref| = {rel:.2e}")
    assert rel <= 1e-2
    for b, L in enumerate(lengths):
        if L <= 0:
            assert not out[b].any()


def test_ops_reject_bad_arguments(ctx):
    buf = ctx.empty(1 << 16, np.float32)
    with pytest.raises(strict_amd.StrictHipError):
        ctx.rmsnorm(buf, buf, buf, 1 << 10, 1 << 10, 1e-6)  # x does not fit its buffer
    with pytest.raises(strict_amd.StrictHipError):
        ctx.rope(buf, buf, 1, 1, 3, 1e4)  # odd head_dim
    with pytest.raises(strict_amd.StrictHipError):
        ctx.argmax(buf, 1, 0, buf)  # empty rows
    with pytest.raises(strict_amd.StrictHipError) as e:
        ctx.attn_decode(buf, buf, buf, buf, buf, 1, 4, 4, 96, 8, 1.0)  # head_dim 96
    assert e.value.status == strict_amd._lib.SH_ERR_UNSUPPORTED
    with pytest.raises(strict_amd.StrictHipError):
        ctx.attn_decode(buf, buf, buf, buf, buf, 1, 6, 4, 64, 8, 1.0)  # heads % kv_heads
    buf.free()
