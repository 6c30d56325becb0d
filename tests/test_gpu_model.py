"""Whole decode steps through the C ABI against the oracle's CpuSession on the same seeded model: logits, hidden
state, routing (ids and weights) and the KV cache are compared bit for bit, and greedy sequences token for token.
Workloads: the reference's synthetic test shapes (tests/model.rs:253-281), the 1B model with a 128-token prompt
and 256 generated tokens, and the 3B model at 4096 cached positions with 256 decode steps, each through the one
launch per layer the bench times, the three fused launches per layer, and the unfused kernels."""
import os

import numpy as np
import pytest

import moert
import oracle

pytestmark = pytest.mark.gpu
THREADS = min(16, os.cpu_count() or 1)


def say(msg):
    print(f"[case] {msg}", flush=True)


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("wdtype,edtype", [(moert.Q8_0, moert.Q8_0), (moert.Q4_0, moert.F32), (moert.F32, moert.F32)])
def test_tiny_model_steps_are_bit_identical_over_more_than_one_attention_tile(gpu, wdtype, edtype):
    """tests/model.rs:253-270: 70 positions (two 64-position tiles), logits, routes, hidden state and KV."""
    cfg = moert.Config(**{**moert.TINY, "embedding_multiplier": 2.0, "residual_multiplier": 0.5,
                          "attention_multiplier": 0.125, "logits_scaling": 4.0})
    m = moert.SynthModel(cfg, seed=5, wdtype=wdtype, embed_dtype=edtype, std=0.1)
    g = moert.GpuModel(m, 128, attn_splits=8)
    s = oracle.CpuSession(m, 128, attn_splits=8, threads=4)
    toks = np.random.default_rng(77).integers(0, cfg.vocab, 70)
    for t, tok in enumerate(toks):
        say(f"tiny dtype={wdtype} pos={t}")
        lg, ids, w, am = g.step(int(tok))
        olg, oids, ow, oh = s.step(int(tok))
        assert bits_equal(lg, olg), t
        assert np.array_equal(ids, oids), t
        assert bits_equal(w, ow), t
        assert bits_equal(g.hidden(), oh), t
        assert am == oracle.argmax(olg)
    for l in range(cfg.layers):
        gk, gv = g.read_kv(l, 70)
        ok, ov = s.read_kv(l, 70)
        assert np.array_equal(gk, ok) and np.array_equal(gv, ov)
    # back to position 0: the same tokens give the same logits (old KV masked by the length)
    g.reset()
    s.set_position(0)
    for tok in toks[:3]:
        assert bits_equal(g.step(int(tok))[0], s.step(int(tok))[0])
    g.close()


def test_decode_step_refuses_bad_tokens_and_a_full_cache(gpu):
    m = moert.SynthModel(moert.Config(**moert.TINY), seed=3)
    g = moert.GpuModel(m, 64, attn_splits=2)
    with pytest.raises(moert.MoertError) as e:
        g.step(m.cfg.vocab)
    assert e.value.code == -5
    g.set_position(63)
    g.step(1)
    with pytest.raises(moert.MoertError) as e:
        g.step(1)
    assert e.value.code == -4
    g.close()


def test_generate_on_the_device_equals_step_by_step_decoding(gpu):
    cfg = moert.Config(**moert.TINY)
    m = moert.SynthModel(cfg, seed=8, std=0.3)
    g = moert.GpuModel(m, 256, attn_splits=4)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 20)
    say("generate vs step")
    out, gaps = g.generate(prompt, 40, gaps=True)
    g.reset()
    lg = None
    for t in prompt:
        lg = g.step(int(t))[0]
    seq = []
    for i in range(40):
        nxt = oracle.argmax(lg)
        seq.append(nxt)
        if i + 1 < 40:
            lg = g.step(nxt)[0]
    assert out.tolist() == seq
    assert (gaps >= 0).all()
    g.close()


def _kv_rows_equal(g, s, cfg, lo, hi):
    """KV rows [lo, hi) of every layer, bit for bit."""
    for l in range(cfg.layers):
        gk, gv = g.read_kv(l, hi)
        ok, ov = s.read_kv(l, hi)
        assert np.array_equal(gk[:, lo:hi], ok[:, lo:hi]) and np.array_equal(gv[:, lo:hi], ov[:, lo:hi]), l


def _greedy_identity(g, s, prompt, n_new, label, min_distinct=1):
    """Greedy generation on the device against the oracle: identical tokens, the last step's logits and hidden
    state bit for bit. Prints the number of distinct tokens and the smallest top1 - top2 logit gap (the reference
    logs the gap against TIE_GAP, bin/m1b-gulosa.rs:20) and asserts at least min_distinct distinct tokens."""
    say(f"{label} gpu generate")
    out = g.generate(prompt, n_new)
    say(f"{label} oracle greedy")
    want, gaps = s.generate(prompt, n_new)
    distinct = len(set(want.tolist()))
    say(f"{label}: {distinct} distinct tokens of {n_new}, smallest top1-top2 gap {float(gaps.min()):.3g}")
    assert out.tolist() == want.tolist()
    assert bits_equal(g.read_logits(), s.last_logits)
    assert bits_equal(g.hidden(), s.last_hidden)
    assert distinct >= min_distinct, distinct
    return want


def _forced_identity(g, s, toks, label, every=1):
    """A forced token stream (the model is never at a fixed point): logits, routes and weights of every step bit
    for bit (tests/model.rs:253-281 compares the GPU model with CpuSession at every position)."""
    for t, tok in enumerate(toks):
        if t % 32 == 0:
            say(f"{label} forced step {t}")
        want_logits = t % every == 0 or t == len(toks) - 1
        lg, ids, w, am = g.step(int(tok), want_logits=want_logits)
        olg, oids, ow, oh = s.step(int(tok), want_logits=want_logits)
        assert np.array_equal(ids, oids) and bits_equal(w, ow), t
        if want_logits:
            assert bits_equal(lg, olg), t
            assert am == oracle.argmax(olg), t
    assert bits_equal(g.hidden(), oh)


# The decode step has three kernel paths, each run below with its launch counts asserted:
#   layer   each layer one launch (attention, output projection and MoE exchanging through the XCDs' L2s and
#           device-wide), where the cache shape gives 2..3 tiles per split and at most 32 splits: the bench's path;
#   fused   the same shapes with three launches per layer (the attention block, the output projection, the MoE
#           kernel over the XCDs; MOERT_LAYER=0);
#   unfused q/k/v, split attention, combine, output projection, router + gate/up, down.
PATHS_1B = {"layer": (4416, 32), "fused": (4416, 32), "unfused": (448, 64)}  # 4416/32: 23 splits of 3 tiles
PATHS_3B = {"layer": (4416, 32), "fused": (4416, 32), "unfused": (4352, 64)}  # 4352/64: 34 splits (over 32)
ALL_PATHS = ["layer", "fused", "unfused"]


def make_model(m, path, max_len, splits):
    if path != "fused":
        return moert.GpuModel(m, max_len, attn_splits=splits)
    os.environ["MOERT_LAYER"] = "0"
    try:
        return moert.GpuModel(m, max_len, attn_splits=splits)
    finally:
        del os.environ["MOERT_LAYER"]


def assert_kernel_path(g, cfg, path):
    """The step's kernels: the model's own report, then the launches of one step (run last: it moves the position
    to the cache's end)."""
    assert g.kernel_path() == path
    kinds = (moert.K_LAYER, moert.K_LAYER_COMBINE, moert.K_ATTN_BLOCK, moert.K_MOE_XCD, moert.K_QKV,
             moert.K_ROUTE_UP, moert.K_EXPERT_DOWN, moert.K_MOE_COMBINE, moert.K_OPROJ)
    n = {}
    for k in kinds:
        g.set_position(g.max_len - 1)
        n[k] = g.time_kernel(k, 1)[1]
    L = cfg.layers
    want = dict.fromkeys(kinds, 0)
    if path == "layer":
        want.update({moert.K_LAYER: L, moert.K_LAYER_COMBINE: 1})
    elif path == "fused":
        want.update({moert.K_ATTN_BLOCK: L, moert.K_MOE_XCD: L, moert.K_MOE_COMBINE: 1, moert.K_OPROJ: L})
    else:
        want.update({moert.K_QKV: L, moert.K_ROUTE_UP: L, moert.K_EXPERT_DOWN: L, moert.K_OPROJ: L})
    assert n == want, n


@pytest.fixture(scope="module")
def granite_1b():
    cfg = moert.Config(**moert.GRANITE_1B)
    say("1B build")
    return cfg, moert.SynthModel(cfg, seed=2024, wdtype=moert.Q8_0, embed_dtype=moert.F32)


def _pair_1b(m, path):
    max_len, splits = PATHS_1B[path]
    return (make_model(m, path, max_len, splits),
            oracle.CpuSession(m, max_len, attn_splits=splits, threads=THREADS))


@pytest.mark.parametrize("path", ALL_PATHS)
def test_granite_1b_greedy_128_prompt_256_tokens_identical(gpu, granite_1b, path):
    """Granite-1B-A400M shape, Q8_0 weights, fp32 embedding/head; 128-token uniform prompt, 256 greedy tokens:
    identical tokens, last logits and hidden state bit for bit, every KV row the run appended. (With N(0, 0.02)
    weights and a tied head the greedy run settles on one token; the forced and wider-init tests below cover
    trajectories that move.)"""
    cfg, m = granite_1b
    prompt = np.random.default_rng(2024).integers(0, cfg.vocab, 128)
    g, s = _pair_1b(m, path)
    _greedy_identity(g, s, prompt, 256, f"1B {path}")
    _kv_rows_equal(g, s, cfg, 0, 128 + 255)
    assert_kernel_path(g, cfg, path)
    g.close()


@pytest.mark.parametrize("path", ALL_PATHS)
def test_granite_1b_forced_tokens_every_step_bit_identical(gpu, granite_1b, path):
    """The 1B workload with a forced random token stream over its 384 positions (128 prompt + 256): logits, routes
    and weights of every step, the final hidden state and every KV row, bit for bit."""
    cfg, m = granite_1b
    toks = np.random.default_rng(99).integers(0, cfg.vocab, 384)
    g, s = _pair_1b(m, path)
    _forced_identity(g, s, toks, f"1B {path}")
    _kv_rows_equal(g, s, cfg, 0, 384)
    assert_kernel_path(g, cfg, path)
    g.close()


@pytest.mark.parametrize("path", ALL_PATHS)
def test_granite_1b_wider_init_greedy_moves_and_stays_identical(gpu, path):
    """The 1B shape with N(0, 0.1) weights, whose greedy trajectory does not settle: 128-token prompt, 256 greedy
    tokens identical to the oracle (at least 100 distinct), last logits and hidden state bit for bit."""
    cfg = moert.Config(**moert.GRANITE_1B)
    say("1B wide build")
    m = moert.SynthModel(cfg, seed=2024, wdtype=moert.Q8_0, embed_dtype=moert.F32, std=0.1)
    prompt = np.random.default_rng(2025).integers(0, cfg.vocab, 128)
    g, s = _pair_1b(m, path)
    _greedy_identity(g, s, prompt, 256, f"1B wide {path}", min_distinct=100)
    assert_kernel_path(g, cfg, path)
    g.close()


def _granite_3b(std):
    cfg = moert.Config(**moert.GRANITE_3B)
    say(f"3B build std={std}")
    m = moert.SynthModel(cfg, seed=3003, wdtype=moert.Q8_0, embed_dtype=moert.Q8_0, std=std)
    return cfg, m, [moert.kv_prefill_data(cfg, 3003, l, 4096) for l in range(cfg.layers)]


def _prefilled_pair(cfg, m, kv, path, ctx=4096):
    max_len, splits = PATHS_3B[path]
    g = make_model(m, path, max_len, splits)
    s = oracle.CpuSession(m, max_len, attn_splits=splits, threads=THREADS)
    for l, (k, v) in enumerate(kv):
        g.kv_prefill(l, k, v)
        s.kv_prefill(l, k, v)
    g.set_position(ctx)
    s.set_position(ctx)
    return g, s


@pytest.fixture(scope="module")
def granite_3b():
    return _granite_3b(0.02)


@pytest.mark.parametrize("path", ALL_PATHS)
def test_granite_3b_long_context_256_steps_identical(gpu, granite_3b, path):
    """Granite-3B-A800M shape, Q8_0 weights and head; KV cache pre-filled to 4096 positions with fp16 N(0,1);
    256 decode steps: the first step's logits and routes, the greedy tokens, the last step's logits and hidden state,
    and the 256 KV rows of every layer, bit for bit."""
    cfg, m, kv = granite_3b
    g, s = _prefilled_pair(cfg, m, kv, path)
    tok = int(np.random.default_rng(3003).integers(0, cfg.vocab))
    say(f"3B {path} first step")
    lg, ids, w, am = g.step(tok)
    olg, oids, ow, _ = s.step(tok)
    assert bits_equal(lg, olg) and np.array_equal(ids, oids) and bits_equal(w, ow)
    assert am == oracle.argmax(olg)
    _greedy_identity(g, s, [am], 255, f"3B {path}")
    _kv_rows_equal(g, s, cfg, 4096, 4352)
    assert_kernel_path(g, cfg, path)
    g.close()


@pytest.mark.parametrize("path", ALL_PATHS)
def test_granite_3b_forced_tokens_at_4096_every_step_bit_identical(gpu, granite_3b, path):
    """The 3B workload with a forced random token stream: 256 steps after the 4096 cached positions, logits, routes
    and weights of every step, the final hidden state and the appended KV rows, bit for bit."""
    cfg, m, kv = granite_3b
    g, s = _prefilled_pair(cfg, m, kv, path)
    toks = np.random.default_rng(31).integers(0, cfg.vocab, 256)
    _forced_identity(g, s, toks, f"3B {path}")
    _kv_rows_equal(g, s, cfg, 4096, 4352)
    assert_kernel_path(g, cfg, path)
    g.close()


@pytest.fixture(scope="module")
def granite_3b_wide():
    return _granite_3b(0.1)


@pytest.mark.parametrize("path", ALL_PATHS)
def test_granite_3b_wider_init_greedy_moves_and_stays_identical(gpu, granite_3b_wide, path):
    """The 3B long-context workload with N(0, 0.1) weights, whose greedy trajectory does not settle: 256 greedy steps
    after 4096 cached positions, identical tokens (at least 100 distinct), last logits and hidden state bit for
    bit."""
    cfg, m, kv = granite_3b_wide
    g, s = _prefilled_pair(cfg, m, kv, path)
    tok = int(np.random.default_rng(7).integers(0, cfg.vocab))
    _greedy_identity(g, s, [tok], 256, f"3B wide {path}", min_distinct=100)
    assert_kernel_path(g, cfg, path)
    g.close()


def test_model_loaded_from_a_bf16_checkpoint_decodes_like_the_oracle(gpu, tmp_path):
    """A synthetic Granite-MoE checkpoint in BF16 (two safetensors files) loaded with quantize-on-load to Q8_0, then
    decoded on the device: 24 steps bit for bit against the oracle's session over the same loaded weights."""
    from test_checkpoint import granite_checkpoint
    cfg = moert.Config(**moert.TINY)
    granite_checkpoint(str(tmp_path), cfg)
    ck = moert.Checkpoint(tmp_path)
    m = moert.LoadedModel(ck, cfg, moert.Q8_0, moert.Q8_0)
    g = moert.GpuModel(m, 64, attn_splits=4)
    s = oracle.CpuSession(m, 64, attn_splits=4, threads=2)
    for t, tok in enumerate(np.random.default_rng(24).integers(0, cfg.vocab, 24)):
        say(f"loaded checkpoint pos={t}")
        lg, ids, w, am = g.step(int(tok))
        olg, oids, ow, _ = s.step(int(tok))
        assert bits_equal(lg, olg) and np.array_equal(ids, oids) and bits_equal(w, ow), t
    g.close()
    del s
    m.close()
    ck.close()
