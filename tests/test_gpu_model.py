"""Whole decode steps through the C ABI against the oracle's CpuSession on the same seeded model: logits, hidden
state, routing (ids and weights) and the KV cache are compared bit for bit, and greedy sequences token for token.
Workloads: the reference's synthetic test shapes (tests/model.rs:253-281), the 1B model with a 128-token prompt
and 256 generated tokens, and the 3B model at 4096 cached positions with 256 decode steps."""
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


def test_granite_1b_greedy_128_prompt_256_tokens_identical(gpu):
    """Granite-1B-A400M shape, Q8_0 weights, fp32 embedding/head; 128-token uniform prompt, 256 greedy tokens."""
    cfg = moert.Config(**moert.GRANITE_1B)
    say("1B build")
    m = moert.SynthModel(cfg, seed=2024, wdtype=moert.Q8_0, embed_dtype=moert.F32)
    prompt = np.random.default_rng(2024).integers(0, cfg.vocab, 128)
    g = moert.GpuModel(m, 448, attn_splits=64)
    say("1B gpu generate")
    out = g.generate(prompt, 256)
    say("1B oracle generate")
    s = oracle.CpuSession(m, 448, attn_splits=64, threads=THREADS)
    want, gaps = s.generate(prompt, 256)
    assert out.tolist() == want.tolist()
    assert bits_equal(g.hidden(), s.last_hidden)  # residual stream after the last step
    g.close()


def test_granite_3b_long_context_256_steps_identical(gpu):
    """Granite-3B-A800M shape, Q8_0 weights and head; KV cache pre-filled to 4096 positions with fp16 N(0,1);
    256 decode steps. Logits of the first and last steps bit-identical, greedy tokens identical."""
    cfg = moert.Config(**moert.GRANITE_3B)
    say("3B build")
    m = moert.SynthModel(cfg, seed=3003, wdtype=moert.Q8_0, embed_dtype=moert.Q8_0)
    ctx, steps, max_len = 4096, 256, 4352
    g = moert.GpuModel(m, max_len, attn_splits=64)
    s = oracle.CpuSession(m, max_len, attn_splits=64, threads=THREADS)
    for l in range(cfg.layers):
        k, v = moert.kv_prefill_data(cfg, 3003, l, ctx)
        g.kv_prefill(l, k, v)
        s.kv_prefill(l, k, v)
    g.set_position(ctx)
    s.set_position(ctx)
    tok = int(np.random.default_rng(3003).integers(0, cfg.vocab))
    say("3B first step")
    lg, ids, w, am = g.step(tok)
    olg, oids, ow, _ = s.step(tok)
    assert bits_equal(lg, olg) and np.array_equal(ids, oids) and bits_equal(w, ow)
    say("3B gpu generate")
    out = g.generate([am], steps - 1)
    say("3B oracle greedy")
    want, _ = s.generate([oracle.argmax(olg)], steps - 1)
    assert out.tolist() == want.tolist()
    g.close()
