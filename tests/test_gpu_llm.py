"""GPU parity of the LLM decode path (FP8 quantizer, W8A16 GEMV, GPT-2 and
Qwen3-shaped greedy decoding) against the numpy oracle (oracle/llm.py).

The reference has no implementation of any of these
(GPT-2 small, fp16, 128-token prompt, 256 greedy steps) and configs[4]
(Qwen3-0.6B shape, FP8 weights, fp16 activations) define them. North-star
bar: identical greedy top-1 tokens, with the logit max-abs-diff stated.

Greedy comparison is teacher-forced: the oracle is fed the GPU's tokens and
its own argmax is compared at every step. Tolerances (stated here):
  - logits: max |logit_gpu - logit_oracle| <= LOGIT_REL_TOL * max |logit_oracle|
    with LOGIT_REL_TOL = 5e-3 (fp16 activations: one fp16 ulp is 1e-3
    relative, and rounding flips compound over the layers);
  - tokens: identical at every step, except that a step whose oracle top-2
    margin is below twice the observed logit max-abs-diff (a tie at the
    precision both sides share) may pick either of the tied tokens; such
    steps are counted and printed;
  - configs[3] (GPT-2, 256 steps): in addition, identical at every step,
    near-ties included, to the oracle with its linears summed in fp64.
"""
import numpy as np
import pytest

import oracle
import oracle.llm as ollm
import strict_amd
from strict_amd import llm

pytestmark = pytest.mark.gpu

LOGIT_REL_TOL = 5e-3


# ---- FP8 quantization and the E4M3 code table --------------------------------

def test_quantize_e4m3_bit_exact(ctx):
    rng = np.random.default_rng(0)
    n, k = 64, 1024
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    w[1] = 0.0                                   # all-zero row: scale 1
    w[2] = rng.normal(0, 1e-6, k)                # tiny values
    w[3, :] = 1e-4
    w[3, 5] = 3.0                                # one outlier: most values subnormal in E4M3
    w[4] = np.linspace(-5, 5, k)                 # a ramp through every binade
    w[5, ::2] = 448.0
    w[5, 1::2] = -448.0 * 0.9999
    dw = ctx.upload(w)
    dq = ctx.empty((n, k), np.uint8)
    ds = ctx.empty((n,), np.float32)
    ctx.quantize_e4m3(dw, dq, ds, n, k)
    ctx.sync()
    q_ref, s_ref = oracle.quantize_e4m3_rows(w)
    assert np.array_equal(ds.to_host().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(dq.to_host(), q_ref)
    for v in (dw, dq, ds):
        v.free()


def _gemv(ctx, x16, q, s, batch, k, n):
    dx = ctx.upload(x16)
    dq = ctx.upload(q)
    dt = ctx.empty((n * k,), np.uint8)
    ds = ctx.upload(s)
    dy = ctx.empty((batch, n), np.float32)
    ctx.pack_e4m3_tiles(dq, dt, n, k)
    ctx.gemv_w8a16(dx, dt, ds, dy, batch, k, n)
    ctx.sync()
    y = dy.to_host()
    for v in (dx, dq, dt, ds, dy):
        v.free()
    return y


def test_e4m3_decode_table_matches_ocp(ctx):
    # row n holds code n in column 0; x = e_0; scale 1 -> y[n] = e4m3(code n).
    # Pins the hardware conversion (OCP E4M3, not the FNUZ variant).
    n, k = 256, 256
    q = np.zeros((n, k), np.uint8)
    q[:, 0] = np.arange(256, dtype=np.uint8)
    x = np.zeros((1, k), np.float16)
    x[0, 0] = 1.0
    y = _gemv(ctx, x.view(np.uint16), q, np.ones(n, np.float32), 1, k, n)[0]
    ref = oracle.e4m3_to_f32(np.arange(256, dtype=np.uint8))
    finite = np.isfinite(ref)
    assert np.array_equal(y[finite], ref[finite])
    assert np.all(np.isnan(y[~finite]))  # 0x7f and 0xff are NaN
    assert ref[0x7e] == 448.0 and ref[0x01] == 2.0 ** -9


@pytest.mark.parametrize("n,k,batch", [(151936, 1024, 1), (4096, 1024, 4), (1024, 3072, 16),
                                       (2048, 1024, 3), (32, 256, 1)])
def test_gemv_w8a16_vs_oracle(ctx, n, k, batch):
    rng = np.random.default_rng(n + k + batch)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    q, s = oracle.quantize_e4m3_rows(w)
    x16 = rng.normal(0, 1, (batch, k)).astype(np.float16)
    y = _gemv(ctx, x16.view(np.uint16), q, s, batch, k, n)
    wq = oracle.e4m3_to_f32(q)
    xf = x16.astype(np.float32)
    ref = (xf.astype(np.float64) @ wq.T.astype(np.float64)) * s
    bound = (np.abs(xf) @ np.abs(wq).T) * s  # sum of |products|: fp32 sum error scale
    assert np.all(np.abs(y - ref) <= 1e-5 * bound + 1e-30)


def test_gemv_rejects_bad_shapes(ctx):
    buf = ctx.empty(1 << 20, np.uint8)
    with pytest.raises(strict_amd.StrictHipError):
        ctx.gemv_w8a16(buf, buf, buf, buf, 1, 100, 16)  # K not a multiple of 256
    with pytest.raises(strict_amd.StrictHipError):
        ctx.gemv_w8a16(buf, buf, buf, buf, 17, 256, 16)  # batch > 16
    buf.free()


# ---- model runners --------------------------------------------------------------

QWEN_SMALL = llm.Config(llm.QWEN3, layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128,
                        intermediate=768, vocab=1000, max_positions=512, max_batch=4)
GPT2_SMALL_TEST = llm.Config(llm.GPT2, layers=2, hidden=256, heads=4, kv_heads=4, head_dim=64,
                             intermediate=512, vocab=997, max_positions=512, max_batch=4,
                             norm_eps=1e-5)


def _randomize_small_params(model, seed):
    """Random norm gains / biases, so those code paths are exercised."""
    rng = np.random.default_rng(seed)
    c = model.cfg
    for li in range(c.layers):
        for name in ("norm1.g", "norm2.g"):
            model.write(name, li, (1 + rng.normal(0, 0.1, c.hidden)).astype(np.float32))
        if c.arch == llm.QWEN3:
            for name in ("q_norm", "k_norm"):
                model.write(name, li, (1 + rng.normal(0, 0.1, c.head_dim)).astype(np.float32))
        else:
            for name in ("norm1.b", "norm2.b"):
                model.write(name, li, rng.normal(0, 0.05, c.hidden).astype(np.float32))
            for name in ("qkv", "o", "fc", "proj"):
                rows = llm.linear_shapes(c)[name][0]
                model.write(f"{name}.bias", li, rng.normal(0, 0.02, rows).astype(np.float32))
    model.write("final.g", 0, (1 + rng.normal(0, 0.1, c.hidden)).astype(np.float32))
    if c.arch == llm.GPT2:
        model.write("final.b", 0, rng.normal(0, 0.05, c.hidden).astype(np.float32))


def _greedy_check(model, prompt, steps, label, exact64=False):
    """GPU generate vs teacher-forced oracle; returns (max logit diff, near-ties).

    exact64: also require every GPU token to equal the one the oracle picks
    with its linears summed in fp64 (the exactly rounded sum of the exact
    products), near-ties included."""
    model.reset(1)
    weights = ollm.load_from_model(model)
    dec = ollm.Decoder(weights)
    # step by step on the GPU, keeping the logits of every step
    gpu_tokens, gpu_logits = [], []
    for i, t in enumerate(prompt):
        model.step([int(t)], logits=(i == len(prompt) - 1))
    for j in range(steps):
        gpu_logits.append(model.logits()[0].copy())
        tok = int(model.next_tokens()[0])
        gpu_tokens.append(tok)
        if j + 1 < steps:
            model.step(None, logits=True)
    ours, margins, ref_logits = ollm.greedy_compare(gpu_tokens, dec, np.asarray(prompt), steps)
    max_diff = max(float(np.max(np.abs(g - r))) for g, r in zip(gpu_logits, ref_logits))
    scale = max(float(np.max(np.abs(r))) for r in ref_logits)
    gpu_tokens = np.array(gpu_tokens)
    mismatch = gpu_tokens != ours
    ties = int(np.sum(mismatch & (margins < 2 * max_diff)))
    print(f"[{label}] {steps} steps: logit max-abs-diff {max_diff:.3e} (max |logit| {scale:.3f}), "
          f"token mismatches {int(mismatch.sum())} (near-ties {ties}), "
          f"min top-2 margin {margins.min():.3e}")
    if mismatch.any() or exact64:
        # second opinion at the near-ties: the oracle again with every linear
        # summed in fp64 (another valid summation order); how far the two
        # oracles drift apart is the precision floor of fp16 activations
        ours64, _, ref64 = ollm.greedy_compare(gpu_tokens, ollm.Decoder(weights, np.float64),
                                               np.asarray(prompt), steps)
        floor = max(float(np.max(np.abs(a - b))) for a, b in zip(ref_logits, ref64))
        sides = int(np.sum(mismatch & (ours64 == gpu_tokens)))
        diff64 = max(float(np.max(np.abs(g - r))) for g, r in zip(gpu_logits, ref64))
        print(f"[{label}] fp32-summed vs fp64-summed oracle: logit max-abs-diff {floor:.3e}; "
              f"at the {int(mismatch.sum())} mismatched step(s) the fp64-summed oracle picks "
              f"the GPU's token {sides} time(s); GPU vs fp64-summed oracle over all {steps} "
              f"steps: token mismatches {int(np.sum(ours64 != gpu_tokens))}, "
              f"logit max-abs-diff {diff64:.3e}")
        if exact64:
            assert np.array_equal(ours64, gpu_tokens), np.nonzero(ours64 != gpu_tokens)[0]
    assert max_diff <= LOGIT_REL_TOL * scale, (max_diff, scale)
    assert not np.any(mismatch & (margins >= 2 * max_diff)), np.nonzero(mismatch)[0]
    return max_diff, ties


def test_qwen3_small_greedy_256(ctx):
    with llm.Model(ctx, QWEN_SMALL) as m:
        assert m.uses_layers_kernel  # a shape the persistent kernel is built for
        m.init_random(seed=7, stddev=0.02)
        _randomize_small_params(m, 1)
        prompt = np.random.default_rng(3).integers(0, QWEN_SMALL.vocab, 16)
        _greedy_check(m, prompt, 256, "qwen3-small")


def test_qwen3_small_per_op_kernels_greedy(ctx, monkeypatch):
    # the per-op path (one kernel per GEMV / attention / merge), which shapes
    # the persistent kernel is not built for take
    monkeypatch.setenv("STRICT_HIP_LLM_LAYERS", "0")
    with llm.Model(ctx, QWEN_SMALL) as m:
        assert not m.uses_layers_kernel
        m.init_random(seed=7, stddev=0.02)
        _randomize_small_params(m, 1)
        prompt = np.random.default_rng(3).integers(0, QWEN_SMALL.vocab, 16)
        _greedy_check(m, prompt, 96, "qwen3-small-per-op")


def test_qwen3_small_head_as_separate_kernels(ctx, monkeypatch):
    # STRICT_HIP_LLM_HEAD=0: the decode-layers kernel ends with the last layer
    # and the final norm and LM head run as their own kernels
    monkeypatch.setenv("STRICT_HIP_LLM_HEAD", "0")
    with llm.Model(ctx, QWEN_SMALL) as m:
        assert m.uses_layers_kernel
        m.init_random(seed=7, stddev=0.02)
        _randomize_small_params(m, 1)
        prompt = np.random.default_rng(3).integers(0, QWEN_SMALL.vocab, 16)
        _greedy_check(m, prompt, 64, "qwen3-small-head-separate")


def test_qwen3_small_cooperative_launch(ctx, monkeypatch):
    # STRICT_HIP_LLM_COOP=1: the decode-layers kernel goes through HIP's
    # cooperative launch (residency guaranteed)
    monkeypatch.setenv("STRICT_HIP_LLM_COOP", "1")
    with llm.Model(ctx, QWEN_SMALL) as m:
        assert m.uses_layers_kernel
        m.init_random(seed=7, stddev=0.02)
        _randomize_small_params(m, 1)
        prompt = np.random.default_rng(3).integers(0, QWEN_SMALL.vocab, 16)
        _greedy_check(m, prompt, 64, "qwen3-small-coop")


@pytest.mark.parametrize("cfg", [QWEN_SMALL, GPT2_SMALL_TEST], ids=["qwen3", "gpt2"])
def test_per_op_path_without_graphs(ctx, monkeypatch, cfg):
    # STRICT_HIP_LLM_GRAPHS=0: the per-op path enqueues every kernel of a
    # step eagerly instead of replaying its captured graph; tokens and
    # logits equal the graph-replayed run's
    monkeypatch.setenv("STRICT_HIP_LLM_LAYERS", "0")
    prompt = np.random.default_rng(21).integers(0, cfg.vocab, 10)
    runs = []
    for graphs in ("1", "0"):
        monkeypatch.setenv("STRICT_HIP_LLM_GRAPHS", graphs)
        with llm.Model(ctx, cfg) as m:
            m.init_random(seed=9, stddev=0.02)
            m.reset(1)
            toks = m.generate(prompt[None, :], 24)[0]
            runs.append((toks, m.logits()[0].copy()))
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1], runs[1][1])


@pytest.mark.parametrize("cfg,err,text", [(QWEN_SMALL, 1, "timed out"), (GPT2_SMALL_TEST, 1, "timed out"),
                                          (QWEN_SMALL, 2, "outside 0..7"), (GPT2_SMALL_TEST, 2, "outside 0..7")],
                         ids=["qwen3", "gpt2", "qwen3-placement-bit", "gpt2-placement-bit"])
def test_decode_layers_wait_failure_reported_and_reset_recovers(ctx, cfg, err, text):
    # The bounded waits of the persistent layers kernels (Qwen3's decode-layers
    # kernel, GPT-2's layers kernel): the host sets the sticky error word
    # before a step, so every wait between workgroups gives up after a few
    # polls and the kernel ends normally; sh_llm_next_tokens reports the
    # failed step (bit 1: a workgroup read an XCD id outside 0..7 in the
    # XCD-local placement; a failed step in that placement turns it off), and
    # sh_llm_reset clears the error.
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 12)
    with llm.Model(ctx, cfg) as m:
        assert m.uses_layers_kernel
        m.init_random(seed=7, stddev=0.02)
        m.reset(1)
        expected = m.generate(prompt[None, :], 6)[0]
        m.reset(1)
        for i, t in enumerate(prompt):
            m.step([int(t)], logits=(i == len(prompt) - 1))
        m.write("layers.err", 0, np.array([err], np.uint32))
        m.step(None, logits=True)
        with pytest.raises(strict_amd.StrictHipError) as e:
            m.next_tokens()
        assert text in str(e.value)
        assert m.read("layers.err", 0, np.uint32)[0] != 0
        m.reset(1)
        assert m.read("layers.err", 0, np.uint32)[0] == 0
        again = m.generate(prompt[None, :], 6)[0]
        assert np.array_equal(again, expected)


def test_gpt2_small_shape_greedy_256(ctx):
    with llm.Model(ctx, GPT2_SMALL_TEST) as m:
        assert m.uses_layers_kernel  # the persistent GPT-2 layers kernel at batch 1
        m.init_random(seed=8, stddev=0.02)
        _randomize_small_params(m, 2)
        prompt = np.random.default_rng(4).integers(0, GPT2_SMALL_TEST.vocab, 16)
        _greedy_check(m, prompt, 256, "gpt2-small-shape")


def test_gpt2_full_width_three_and_four_splits(ctx):
    # GPT-2 small's widths with max_positions 160: 48-position attention
    # splits, so a 140-token prompt and 16 steps (contexts 141..156) run the
    # O items' staging over 3 and then 4 active splits per head at hidden
    # 768 (two dim pairs per lane), which configs[3] (256-position splits)
    # reaches only past 512 positions
    cfg = llm.GPT2_SMALL.with_(max_positions=160)
    with llm.Model(ctx, cfg) as m:
        assert m.uses_layers_kernel
        m.init_random(seed=11, stddev=0.02)
        _randomize_small_params(m, 3)
        prompt = np.random.default_rng(5).integers(0, cfg.vocab, 140)
        _greedy_check(m, prompt, 16, "gpt2-full-width-splits")


def test_gpt2_config3_greedy_256(ctx):
    # GPT-2 small, random N(0, 0.02) fp16 weights, batch 1,
    # 128-token prompt of seeded uniform ids, 256 greedy steps with KV cache
    cfg = llm.GPT2_SMALL
    with llm.Model(ctx, cfg) as m:
        assert m.uses_layers_kernel
        m.init_random(seed=42, stddev=0.02)
        prompt = np.random.default_rng(42).integers(0, cfg.vocab, 128)
        # one step of the 256 is a near-tie (top-2 margin 2.5e-4) where the
        # fp32-summed oracle's token differs; the fp64-summed one picks the
        # GPU's token there, and matches the GPU at every step
        _greedy_check(m, prompt, 256, "gpt2-config3", exact64=True)


# ---- configs[4] at its own shape: one model, max_batch 16, KV room for 4096+ --------

QWEN_CONFIG4 = llm.QWEN3_0_6B.with_(max_positions=4096 + 64, max_batch=16)


@pytest.fixture(scope="module")
def config4(ctx):
    """The configs[4] model (28 layers, hidden 1024, 16 Q / 8 KV heads, head_dim
    128, SwiGLU 3072, vocab 151936, FP8 weights) and its dequantized weights
    for the oracle, shared by the configs[4] tests."""
    m = llm.Model(ctx, QWEN_CONFIG4)
    m.init_random(seed=42, stddev=0.02)
    assert m.uses_layers_kernel
    weights = ollm.load_from_model(m)
    yield m, weights
    m.close()


def _batch_greedy_check(model, weights, prompts, steps, label):
    """Every row of a batched GPU run against its own teacher-forced oracle
    decoder: logits within LOGIT_REL_TOL, greedy tokens identical except at
    oracle near-ties. Returns (max logit diff, mismatches, near-ties, decoders)."""
    B = prompts.shape[0]
    model.reset(B)
    for i in range(prompts.shape[1]):
        model.step(prompts[:, i], logits=(i == prompts.shape[1] - 1))
    gpu_tokens, gpu_logits = [], []
    for j in range(steps):
        gpu_logits.append(model.logits().copy())
        gpu_tokens.append(model.next_tokens().copy())
        if j + 1 < steps:
            model.step(None, logits=True)
    gpu_tokens = np.array(gpu_tokens)  # [steps, B]
    max_diff, scale, mism, ties, decs = 0.0, 0.0, 0, 0, []
    for b in range(B):
        dec = ollm.Decoder(weights)
        ours, margins, ref = ollm.greedy_compare(gpu_tokens[:, b], dec, prompts[b], steps)
        d = max(float(np.max(np.abs(g[b] - r))) for g, r in zip(gpu_logits, ref))
        sc = max(float(np.max(np.abs(r))) for r in ref)
        bad = gpu_tokens[:, b] != ours
        assert d <= LOGIT_REL_TOL * sc, (b, d, sc)
        assert not np.any(bad & (margins >= 2 * d)), (b, np.nonzero(bad)[0])
        max_diff, scale = max(max_diff, d), max(scale, sc)
        mism += int(bad.sum())
        ties += int(np.sum(bad & (margins < 2 * d)))
        decs.append(dec)
    print(f"[{label}] B={B}, {steps} steps: logit max-abs-diff {max_diff:.3e} (max |logit| "
          f"{scale:.3f}), token mismatches {mism} (near-ties {ties})")
    return max_diff, mism, ties, decs


def _check_kv_cache(model, decs, label):
    """The K and V^T caches the decode-layers kernel appended (q/k RMSNorm,
    RoPE, cache layout) against the oracle decoders' caches, every layer and
    row: max |gpu - oracle| <= 1e-2 * max |oracle| (attention's bar)."""
    c = model.cfg
    vt = (c.max_positions + 15) // 16 * 16
    worst = 0.0
    for li in range(c.layers):
        k = oracle.f16_to_f32(model.read("kcache", li, np.uint16)).reshape(
            c.max_batch, c.kv_heads, -1, c.head_dim)
        v = oracle.f16_to_f32(model.read("vcache", li, np.uint16)).reshape(
            c.max_batch, c.kv_heads, c.head_dim, vt)
        for b, dec in enumerate(decs):
            P = dec.k[li].shape[0]  # prompt + steps - 1 positions on both sides
            kr = dec.k[li][:P].transpose(1, 0, 2)       # [kvh, P, d]
            vr = dec.v[li][:P].transpose(1, 2, 0)       # [kvh, d, P]
            for got, ref in ((k[b, :, :P], kr), (v[b, :, :, :P], vr)):
                rel = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
                assert rel <= 1e-2, (li, b, rel)
                worst = max(worst, rel)
    print(f"[{label}] K / V caches: max |gpu - oracle| / max |oracle| = {worst:.3e}")


def test_qwen3_config4_greedy_256(ctx, config4):
    # BASELINE configs[4] at batch 1: 32-token prompt, 256 greedy steps
    m, w = config4
    prompt = np.random.default_rng(42).integers(0, QWEN_CONFIG4.vocab, (1, 32))
    _batch_greedy_check(m, w, prompt, 256, "qwen3-config4-b1")


def test_qwen3_config4_xcd_local_placement_bit_identical(ctx, config4, monkeypatch):
    # Batch 1 at configs[4]'s shape runs XCD-local: KV head h's QKV tiles,
    # attention splits and merge items on XCD h, their cells stored into
    # that XCD's L2. The items and their arithmetic are the same as with the
    # default placement (STRICT_HIP_LLM_XCD=0), so logits and tokens of 24
    # greedy steps after a 600-token prompt (19 active splits) are equal bit
    # for bit.
    m, _ = config4
    prompt = np.random.default_rng(77).integers(0, QWEN_CONFIG4.vocab, 600)
    runs = []
    for xcd in ("1", "0"):
        monkeypatch.setenv("STRICT_HIP_LLM_XCD", xcd)
        m.reset(1)
        for i, t in enumerate(prompt):
            m.step([int(t)], logits=(i == len(prompt) - 1))
        toks, logits = [], []
        for j in range(24):
            logits.append(m.logits()[0].copy())
            toks.append(int(m.next_tokens()[0]))
            if j + 1 < 24:
                m.step(None, logits=True)
        runs.append((np.array(toks), np.array(logits)))
        print(f"STRICT_HIP_LLM_XCD={xcd}: tokens {toks[:8]}", flush=True)
    monkeypatch.delenv("STRICT_HIP_LLM_XCD")
    m.reset(1)
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1], runs[1][1])


@pytest.mark.parametrize("batch", [4, 6, 8, 16])
def test_qwen3_config4_batch_vs_oracle(ctx, config4, batch):
    # configs[4] at batch 4 to 16 after 12-token prompts: every row its own
    # prompt, each checked against its own oracle decoder, and every row's K
    # and V^T cache entries against the oracle's. At this length each (row,
    # KV head) has one active attention split, so every workgroup runs at
    # most one attention item that does anything; the multi-item runs are
    # the long-context tests below.
    m, w = config4
    prompts = np.random.default_rng(100 + batch).integers(0, QWEN_CONFIG4.vocab, (batch, 12))
    _, _, _, decs = _batch_greedy_check(m, w, prompts, 8, f"qwen3-config4-b{batch}")
    _check_kv_cache(m, decs, f"qwen3-config4-b{batch}")


def _batch_long_check(model, weights, prompts, steps, single_rows, oracle_rows, label):
    """A batched run after long prompts against batch-1 runs of the same
    prompts (logits bit-identical and tokens identical at every step: a
    split's arithmetic does not depend on the batch or on which workgroup
    runs it) and against teacher-forced oracle decoders for oracle_rows
    (logits within LOGIT_REL_TOL, tokens identical except at near-ties)."""
    B, T = prompts.shape
    model.reset(B)
    for i in range(T):
        model.step(prompts[:, i], logits=(i == T - 1))
    toks, logits = [], []
    for j in range(steps):
        logits.append(model.logits().copy())
        toks.append(model.next_tokens().copy())
        if j + 1 < steps:
            model.step(None, logits=True)
    toks = np.array(toks)  # [steps, B]
    for b in single_rows:
        model.reset(1)
        for i in range(T):
            model.step(prompts[b:b + 1, i], logits=(i == T - 1))
        for j in range(steps):
            single = model.logits()[0]
            assert np.array_equal(single, logits[j][b]), (
                b, j, float(np.max(np.abs(single - logits[j][b]))))
            assert int(model.next_tokens()[0]) == int(toks[j][b]), (b, j)
            if j + 1 < steps:
                model.step(None, logits=True)
    worst, ties = 0.0, 0
    for b in oracle_rows:
        ours, margins, ref = ollm.greedy_compare(toks[:, b], ollm.Decoder(weights), prompts[b], steps)
        d = max(float(np.max(np.abs(g[b] - r))) for g, r in zip(logits, ref))
        sc = max(float(np.max(np.abs(r))) for r in ref)
        bad = toks[:, b] != ours
        assert d <= LOGIT_REL_TOL * sc, (b, d, sc)
        assert not np.any(bad & (margins >= 2 * d)), (b, np.nonzero(bad)[0])
        worst, ties = max(worst, d), ties + int(bad.sum())
    print(f"[{label}] B={B} after {T}-token prompts, {steps} steps: rows {list(single_rows)} "
          f"bit-identical to batch 1; rows {list(oracle_rows)} vs oracle: logit max-abs-diff "
          f"{worst:.3e}, token mismatches {ties} (all near-ties)")


# Attention items at configs[4]'s split size (144 positions, 32 splits per
# (row, KV head)): a context of ~2,200 positions has 16 active splits per
# (row, KV head), one of ~4,100 has 29. The 256 workgroups' runs then are:
#   b = 4  (small-batch kernel, the active items partitioned by a cursor):
#          2 items each at 2,200, 3-4 at 4,100 -- later items reuse the run's
#          q / k / v from LDS, and runs cross into the next KV head and row;
#   b = 6  (large-batch kernel, all 1,536 items partitioned): 6 items each,
#          runs crossing (row, KV head) pairs, inactive splits among them;
#   b = 8  (large-batch, 4 workgroups per pair split its active splits):
#          4 items each at 2,200;
#   b = 12 (all 3,072 items partitioned): runs of 12, so each item stages its
#          successor's first K / V^T block in LDS, across pair boundaries;
#   b = 16 (2 workgroups per pair): runs of 14-15 with LDS staging at 4,100.
# Rows always hold the same number of positions: sh_llm_step advances every
# row of the batch by one, so no row has zero active splits while another
# has some.

@pytest.mark.parametrize("batch,rows", [(4, (0, 1, 2, 3)), (6, (0, 1, 2, 3, 4, 5)),
                                        (8, (0, 1, 2, 3, 4, 5, 6, 7)), (12, (0, 5, 11))])
def test_qwen3_config4_batch_long_prompt_rows(ctx, config4, batch, rows):
    m, w = config4
    prompts = np.random.default_rng(300 + batch).integers(0, QWEN_CONFIG4.vocab, (batch, 2200))
    _batch_long_check(m, w, prompts, 4, rows, (batch - 1,), f"qwen3-config4-b{batch}-kv2200")


def test_qwen3_config4_batch4_kv4096(ctx, config4):
    # BASELINE configs[4] at batch 4 against a 4096-token KV cache: every row
    # against batch 1, row 0 against the oracle
    m, w = config4
    prompts = np.random.default_rng(11).integers(0, QWEN_CONFIG4.vocab, (4, 4096))
    _batch_long_check(m, w, prompts, 4, (0, 1, 2, 3), (0,), "qwen3-config4-b4-kv4096")


def test_qwen3_config4_batch16_kv4096(ctx, config4):
    # BASELINE configs[4] at batch 16 against a 4096-token KV cache: rows from
    # both staging passes of the GEMV items (0-7, 8-15) against batch 1, row
    # 15 against the oracle
    m, w = config4
    prompts = np.random.default_rng(7).integers(0, QWEN_CONFIG4.vocab, (16, 4096))
    _batch_long_check(m, w, prompts, 4, (0, 5, 10, 15), (15,), "qwen3-config4-b16-kv4096")


def test_qwen3_long_context_step(ctx, config4):
    # BASELINE configs[4] KV length: a 4096-token prompt fills the cache, then
    # greedy steps attend over 4096+ positions (split-K attention with many
    # splits and the cross-workgroup merge)
    m, w = config4
    prompt = np.random.default_rng(6).integers(0, QWEN_CONFIG4.vocab, (1, 4096))
    _batch_greedy_check(m, w, prompt, 4, "qwen3-config4-kv4096")


def test_inv_freq_table(ctx):
    with llm.Model(ctx, QWEN_SMALL) as m:
        got = m.read("inv_freq", 0, np.float32)
        assert np.array_equal(got, ollm.inv_freq(QWEN_SMALL.rope_theta, QWEN_SMALL.head_dim))


def test_load_linear_roundtrip(ctx):
    rng = np.random.default_rng(5)
    with llm.Model(ctx, QWEN_SMALL) as m:
        rows, cols = llm.linear_shapes(QWEN_SMALL)["gate_up"]
        w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
        m.load_linear("gate_up", 1, w)
        q_ref, s_ref = oracle.quantize_e4m3_rows(w)
        q = llm.interleaved_to_logical(llm.untile_fp8(m.read("gate_up.w", 1), rows, cols),
                                       QWEN_SMALL.intermediate)
        s = llm.interleaved_to_logical(m.read("gate_up.scale", 1, np.float32)[:, None],
                                       QWEN_SMALL.intermediate)[:, 0]
        assert np.array_equal(q, q_ref) and np.array_equal(s, s_ref)
    with llm.Model(ctx, GPT2_SMALL_TEST) as m:
        rows, cols = llm.linear_shapes(GPT2_SMALL_TEST)["fc"]
        w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
        m.load_linear("fc", 0, w)
        h = llm.untile_f16(m.read("fc.w", 0).view(np.uint16), rows, cols)
        assert np.array_equal(h, oracle.f32_to_f16(w))


def test_init_random_statistics(ctx):
    with llm.Model(ctx, QWEN_SMALL) as m:
        m.init_random(seed=11, stddev=0.02)
        rows, cols = llm.linear_shapes(QWEN_SMALL)["qkv"]
        w = oracle.e4m3_to_f32(llm.untile_fp8(m.read("qkv.w", 0), rows, cols))
        w = w * m.read("qkv.scale", 0, np.float32)[:, None]
        assert abs(float(w.mean())) < 5e-4
        assert abs(float(w.std()) / 0.02 - 1) < 0.03


def test_batch_rows_match_single_rows(ctx):
    rng = np.random.default_rng(9)
    prompts = rng.integers(0, QWEN_SMALL.vocab, (4, 12))
    with llm.Model(ctx, QWEN_SMALL) as m:
        m.init_random(seed=7, stddev=0.02)
        _randomize_small_params(m, 1)
        m.reset(4)
        batched = m.generate(prompts, 40)
        for b in range(4):
            m.reset(1)
            single = m.generate(prompts[b:b + 1], 40)
            assert np.array_equal(batched[b], single[0]), b


def test_generate_matches_stepwise(ctx):
    prompt = np.random.default_rng(12).integers(0, GPT2_SMALL_TEST.vocab, 10)
    with llm.Model(ctx, GPT2_SMALL_TEST) as m:
        m.init_random(seed=3, stddev=0.02)
        m.reset(1)
        gen = m.generate(prompt[None, :], 20)[0]
        m.reset(1)
        for i, t in enumerate(prompt):
            m.step([int(t)], logits=(i == len(prompt) - 1))
        steps = []
        for j in range(20):
            steps.append(int(m.next_tokens()[0]))
            if j + 1 < 20:
                m.step(None, logits=True)
        assert np.array_equal(gen, np.array(steps))
        hist = m.read("hist", 0, np.int32)[: len(prompt)]
        assert np.array_equal(hist, prompt)


@pytest.mark.parametrize("cfg", [GPT2_SMALL_TEST, llm.GPT2_SMALL], ids=["small-shape", "gpt2-small"])
def test_gpt2_xcd_local_placement_bit_identical(ctx, monkeypatch, cfg):
    # The GPT-2 layers kernel with head h's QKV tiles and attention splits on
    # XCD h % 8 (q / k / v cells stored into that XCD's L2) against the
    # default placement (STRICT_HIP_LLM_XCD=0): same items, same arithmetic,
    # so tokens and logits of 20 greedy steps after a 40-token prompt are
    # equal bit for bit.
    prompt = np.random.default_rng(8).integers(0, cfg.vocab, 40)
    runs = []
    with llm.Model(ctx, cfg) as m:
        m.init_random(seed=5, stddev=0.02)
        for xcd in ("1", "0"):
            monkeypatch.setenv("STRICT_HIP_LLM_XCD", xcd)
            m.reset(1)
            for i, t in enumerate(prompt):
                m.step([int(t)], logits=(i == len(prompt) - 1))
            toks, logits = [], []
            for j in range(20):
                logits.append(m.logits()[0].copy())
                toks.append(int(m.next_tokens()[0]))
                if j + 1 < 20:
                    m.step(None, logits=True)
            runs.append((np.array(toks), np.array(logits)))
            print(f"STRICT_HIP_LLM_XCD={xcd}: tokens {toks[:8]}", flush=True)
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1], runs[1][1])


def test_gpt2_key_sets_across_batch_sizes(ctx):
    # GPT-2 runs its layers kernel at batch 1 (one launch per step, which
    # embeds the token itself and advances the step number, alternating the
    # two argmax key sets) and the per-op path, graph-replayed, at batch 2.
    # Between the two rounds' batch-2 runs, 15 + 16 = 31 layers-kernel steps
    # move the current key set; each run must repeat the first round's tokens
    # (a graph replayed on the other key set would not), and the history
    # must hold the prompt and the generated tokens.
    prompts = np.random.default_rng(31).integers(0, GPT2_SMALL_TEST.vocab, (2, 10))
    plan = ((1, 7), (2, 6), (1, 6))
    with llm.Model(ctx, GPT2_SMALL_TEST) as m:
        m.init_random(seed=3, stddev=0.02)
        first = {}
        for rnd in range(2):
            for b, steps in plan:
                m.reset(b)
                toks = m.generate(prompts[:b], steps)
                print(f"round {rnd} batch {b} steps {steps}: {toks[0][:6]}", flush=True)
                if rnd == 0:
                    first[(b, steps)] = toks
                else:
                    assert np.array_equal(toks, first[(b, steps)]), (b, steps)
                hist = m.read("hist", 0, np.int32)[:10 + steps - 1]
                assert np.array_equal(hist[:10], prompts[0])
                assert np.array_equal(hist[10:], toks[0][:steps - 1])


def test_llm_rejects_bad_arguments(ctx):
    with pytest.raises(strict_amd.StrictHipError):
        llm.Model(ctx, QWEN_SMALL.with_(head_dim=96))
    with pytest.raises(strict_amd.StrictHipError):
        llm.Model(ctx, QWEN_SMALL.with_(max_batch=17))
    with llm.Model(ctx, QWEN_SMALL.with_(max_positions=8)) as m:
        with pytest.raises(strict_amd.StrictHipError):
            m.step([1])  # reset was not called
        m.reset(1)
        with pytest.raises(strict_amd.StrictHipError):
            m.step([QWEN_SMALL.vocab])  # token outside the vocabulary
        for _ in range(8):
            m.step([1], logits=False)
        with pytest.raises(strict_amd.StrictHipError):
            m.step([1])  # KV cache full
