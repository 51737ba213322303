"""sh_attn_decode_f16_noalloc (the allocation-free decode attention) against
sh_attn_decode_f16, through the C ABI: the same kernels and split layout, so
the outputs must be bit-identical, on two calls in a row, the second with a
smaller input (the fixed work array keeps the first call's partials); each
output is also checked against the oracle at the attention bar
(max |gpu - oracle| <= 1e-2 * max |oracle|). A call whose partials exceed
the array is refused before anything is launched."""
import numpy as np
import pytest

import oracle.llm as ollm
import strict_amd

pytestmark = pytest.mark.gpu


def _inputs(seed, batch, heads, kv_heads, d, max_pos, lengths):
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 1, (batch, heads, d)).astype(np.float32)
    k = rng.normal(0, 1, (batch, kv_heads, max_pos, d)).astype(np.float16)
    v = rng.normal(0, 1, (batch, kv_heads, max_pos, d)).astype(np.float16)
    return q, k, v, np.array(lengths, np.int32)


def _both(ctx, q, k, v, lens, heads, kv_heads, d, max_pos):
    batch = q.shape[0]
    scale = float(1 / np.sqrt(d))
    dq, dk, dv, dl = (ctx.upload(a) for a in (q, k.view(np.uint16), v.view(np.uint16), lens))
    outs = []
    for fn in (ctx.attn_decode, ctx.attn_decode_noalloc):
        do = ctx.empty((batch, heads, d), np.float32)
        fn(dq, dk, dv, dl, do, batch, heads, kv_heads, d, max_pos, scale)
        ctx.sync()
        outs.append(do.to_host())
        do.free()
    for a in (dq, dk, dv, dl):
        a.free()
    ref = ollm.attn_decode(q, k.astype(np.float32), v.astype(np.float32), lens, scale)
    return outs[0], outs[1], ref


def test_noalloc_matches_allocating_entry_point_twice(ctx):
    cases = [
        # first call: 4 rows at the Qwen3 shape, many splits
        (11, 4, 16, 8, 128, 2048, [2048, 1, 1500, 777]),
        # second call, smaller: one GPT-2-shaped row over fewer positions
        (12, 1, 12, 12, 64, 200, [150]),
    ]
    for seed, batch, heads, kvh, d, max_pos, lengths in cases:
        q, k, v, lens = _inputs(seed, batch, heads, kvh, d, max_pos, lengths)
        alloc, noalloc, ref = _both(ctx, q, k, v, lens, heads, kvh, d, max_pos)
        assert np.array_equal(alloc.view(np.uint32), noalloc.view(np.uint32)), (batch, heads)
        rel = float(np.max(np.abs(noalloc - ref)) / np.max(np.abs(ref)))
        print(f"noalloc b={batch} h={heads}/{kvh} d={d} P={max_pos}: bit-identical to the "
              f"allocating call, max err / max |ref| = {rel:.2e}")
        assert rel <= 1e-2


def test_noalloc_refuses_partials_beyond_its_array(ctx):
    # 2048 rows x 16 heads x 1 split x (128 + 2) x 4 bytes = 17 MB > 16 MiB
    batch, heads, kvh, d, max_pos = 2048, 16, 1, 128, 1
    q = ctx.empty((batch, heads, d), np.float32)
    kv = ctx.empty((batch, kvh, max_pos, d), np.uint16)
    lens = ctx.upload(np.ones(batch, np.int32))
    out = ctx.empty((batch, heads, d), np.float32)
    with pytest.raises(strict_amd.StrictHipError) as e:
        ctx.attn_decode_noalloc(q, kv, kv, lens, out, batch, heads, kvh, d, max_pos, 1.0)
    assert e.value.status == strict_amd._lib.SH_ERR_INVALID_ARGUMENT
    assert "allocation-free" in str(e.value)
    for a in (q, kv, lens, out):
        a.free()
