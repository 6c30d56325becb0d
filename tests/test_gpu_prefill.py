"""Multi-position steps of the whole model (moert_step_batched, moert_prefill) through the C ABI: a block of up to 32
positions must leave exactly what the same tokens leave when decoded one at a time (the model-mode block step,
cuda_backend.rs:499-516, 751-917, whose per-position loops make it equal to single steps): the KV rows of every
position, the hidden state and logits of the last one, bit for bit, and the same greedy continuation. The
single-position decode is itself pinned bit for bit against the oracle (test_gpu_model.py); the tiny case also
checks the oracle directly."""
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


def decode_reference(g, toks, pos0, layers):
    """Decodes toks one at a time from pos0: (last logits, last argmax, hidden, KV rows [pos0, pos0 + n) per layer)."""
    g.set_position(pos0)
    for t in toks:
        lg, _, _, am = g.step(int(t))
    n = pos0 + len(toks)
    kv = [tuple(a[:, pos0:n] for a in g.read_kv(l, n)) for l in range(layers)]
    return lg, am, g.hidden(), kv


def check_block(g, toks, pos0, layers, ref, label):
    lg, am, hid, kv = ref
    g.set_position(pos0)
    blg, bam = g.step_batched(toks) if len(toks) <= 32 else g.prefill(toks)
    n = pos0 + len(toks)
    assert g.position() == n, label
    assert bits_equal(blg, lg), label
    assert bam == am, label
    assert bits_equal(g.hidden(), hid), label
    for l in range(layers):
        bk, bv = g.read_kv(l, n)
        assert np.array_equal(bk[:, pos0:n], kv[l][0]) and np.array_equal(bv[:, pos0:n], kv[l][1]), (label, l)


@pytest.mark.parametrize("wdtype,edtype", [(moert.Q8_0, moert.Q8_0), (moert.Q4_0, moert.F32), (moert.F32, moert.F32)])
def test_tiny_batched_steps_equal_single_steps_and_the_oracle(gpu, wdtype, edtype):
    cfg = moert.Config(**{**moert.TINY, "embedding_multiplier": 2.0, "residual_multiplier": 0.5,
                          "attention_multiplier": 0.125, "logits_scaling": 4.0})
    m = moert.SynthModel(cfg, seed=11, wdtype=wdtype, embed_dtype=edtype, std=0.1)
    g = moert.GpuModel(m, 192, attn_splits=8)
    toks = np.random.default_rng(12).integers(0, cfg.vocab, 150)
    # blocks of 1, 5, 32, 17 and 32 positions, then the rest through prefill (blocks of 32 and a remainder)
    pos = 0
    for size in (1, 5, 32, 17, 32, 63):
        block = toks[pos:pos + size]
        say(f"tiny dtype={wdtype} block at {pos} of {size}")
        ref = decode_reference(g, block, pos, cfg.layers)
        check_block(g, block, pos, cfg.layers, ref, (wdtype, pos, size))
        pos += size
    # the oracle session over the same 150 tokens ends with the same logits and hidden state
    s = oracle.CpuSession(m, 192, attn_splits=8, threads=4)
    for t in toks:
        olg, _, _, oh = s.step(int(t))
    g.set_position(0)
    blg, bam = g.prefill(toks)
    assert bits_equal(blg, olg) and bits_equal(g.hidden(), oh) and bam == oracle.argmax(olg)
    # the greedy continuation after a batched step equals the one after single steps
    out_b = g.generate([bam], 8)
    g.set_position(0)
    for t in toks:
        lg, _, _, am = g.step(int(t))
    out_s = g.generate([am], 8)
    assert np.array_equal(out_b, out_s)
    g.close()


def test_granite_1b_prefill_of_70_tokens_equals_decoding_them(gpu):
    cfg = moert.Config(**moert.GRANITE_1B)
    m = moert.SynthModel(cfg, seed=21)
    g = moert.GpuModel(m, 256, attn_splits=32)
    toks = np.random.default_rng(22).integers(0, cfg.vocab, 70)
    say("1b decode 70 tokens")
    ref = decode_reference(g, toks, 0, cfg.layers)
    say("1b prefill 70 tokens (blocks 32, 32, 6)")
    check_block(g, toks, 0, cfg.layers, ref, "1b prefill")
    g.close()


def test_granite_3b_batched_step_of_32_at_4096_cached_positions(gpu):
    """The bench workload: 32 positions appended after 4096 cached ones (2-tile attention splits, G = 3)."""
    cfg = moert.Config(**moert.GRANITE_3B)
    m = moert.SynthModel(cfg, seed=31)
    ctx = 4096
    max_len = (ctx + 32 + 63) // 64 * 64
    g = moert.GpuModel(m, max_len, attn_splits=32)
    for l in range(cfg.layers):
        k, v = moert.kv_prefill_data(cfg, 31, l, ctx)
        g.kv_prefill(l, k, v)
    toks = np.random.default_rng(32).integers(0, cfg.vocab, 32)
    say("3b decode 32 tokens at 4096")
    ref = decode_reference(g, toks, ctx, cfg.layers)
    say("3b batched step of 32 at 4096")
    check_block(g, toks, ctx, cfg.layers, ref, "3b block")
    g.close()


def test_batched_step_refuses_bad_blocks(gpu):
    cfg = moert.Config(**moert.TINY)
    m = moert.SynthModel(cfg, seed=3)
    g = moert.GpuModel(m, 64, attn_splits=2)
    for toks in ([], list(range(33))):
        with pytest.raises(moert.MoertError):
            g.step_batched(np.array(toks, np.int32) % cfg.vocab)
    with pytest.raises(moert.MoertError) as e:
        g.step_batched([1, cfg.vocab])
    assert e.value.code == moert.E_RANGE
    g.set_position(40)
    with pytest.raises(moert.MoertError) as e:
        g.prefill(np.zeros(25, np.int32))
    assert e.value.code == moert.E_FULL
    assert g.position() == 40  # nothing ran
    with pytest.raises(moert.MoertError) as e:
        g.prefill([0, cfg.vocab + 3])  # the vocabulary check comes first, as in valida
    assert e.value.code == moert.E_RANGE
    g.step_batched(np.arange(24) % cfg.vocab)  # exactly up to the end of the cache
    assert g.position() == 64
    g.close()
    c = moert.GpuModel(m, 64, attn_splits=2, cache_slots=4)
    with pytest.raises(moert.MoertError) as e:
        c.step_batched([1, 2])
    assert e.value.code == moert.E_CONFIG
    c.close()


@pytest.mark.parametrize("shape,seed", [("1b", 41), ("3b", 43)])
def test_grouped_mode_prefill_within_1e2_of_the_fma_path(gpu, shape, seed):
    """moert_batched_mode(1): the block prefill's experts through the grouped int8 MFMA kernels (15-bit activation
    codes, exact int32 block products, experts summed in first-appearance order). A 70-token prompt (blocks 32, 32,
    6), then 8 forced decode steps: the last prompt position's logits and every decode step's logits within 1e-2 of
    the default per-row FMA path (which equals decode steps and the oracle bit for bit), and the argmax equal wherever
    that path's top1 - top2 gap exceeds 2e-2. Switching back to mode 0 gives the FMA path's logits bit for bit."""
    cfg = moert.Config(**(moert.GRANITE_1B if shape == "1b" else moert.GRANITE_3B))
    m = moert.SynthModel(cfg, seed=seed, zipf_s=1.1)
    rng = np.random.default_rng(seed + 1)
    toks = rng.integers(0, cfg.vocab, 70)
    forced = rng.integers(0, cfg.vocab, 8)
    fma = moert.GpuModel(m, 128, attn_splits=32)
    grp = moert.GpuModel(m, 128, attn_splits=32)
    say(f"{shape} grouped mode on")
    grp.batched_mode(1)

    def close(a, b, label):
        d = float(np.abs(a - b).max())
        s = np.sort(a)
        if s[-1] - s[-2] > 2e-2:
            assert int(np.argmax(a)) == int(np.argmax(b)), label
        assert d <= 1e-2, (label, d)
        return d

    say(f"{shape} prefill 70 tokens, fma and grouped")
    lf, af = fma.prefill(toks)
    lg, ag = grp.prefill(toks)
    diffs = [close(lf, lg, "prefill")]
    for i, tok in enumerate(forced):
        a = fma.step(int(tok))[0]
        b = grp.step(int(tok))[0]
        diffs.append(close(a, b, f"decode {i}"))
    say(f"{shape} grouped mode: max logit difference {max(diffs):.2e}")
    assert max(diffs) > 0.0  # the modes really differ (codes, sum order)
    grp.batched_mode(0)
    grp.reset()
    fma.reset()
    a = fma.prefill(toks)[0]
    b = grp.prefill(toks)[0]
    assert bits_equal(a, b)
    fma.close()
    grp.close()


@pytest.mark.parametrize("shape,seed,ctx", [("1b", 41, 0), ("3b", 43, 4096)])
def test_grouped_mode_blocks_equal_the_oracle_grouped_step(gpu, shape, seed, ctx):
    """moert_batched_mode(1) against the oracle's restatement of the grouped step (orc_session_step_grouped: 15-bit
    codes, exact integer block products in four quarters per q/k/v and output row, the engine's norm orders, experts
    grouped in first-appearance order), bit for bit: blocks of 32, 5 and 17 positions (the 3B model after 4096
    positions pre-filled with fp16 N(0, 1)), each block's last logits, argmax and hidden state, then every KV row the
    blocks appended, then 4 decode steps after them (the decode path, against the oracle's decode)."""
    cfg = moert.Config(**(moert.GRANITE_1B if shape == "1b" else moert.GRANITE_3B))
    say(f"{shape} build")
    m = moert.SynthModel(cfg, seed=seed, zipf_s=1.1)
    max_len = 4416 if ctx else 128
    g = moert.GpuModel(m, max_len, attn_splits=32)
    s = oracle.CpuSession(m, max_len, attn_splits=32, threads=THREADS)
    if ctx:
        for l in range(cfg.layers):
            k, v = moert.kv_prefill_data(cfg, seed, l, ctx)
            g.kv_prefill(l, k, v)
            s.kv_prefill(l, k, v)
        g.set_position(ctx)
        s.set_position(ctx)
    g.batched_mode(1)
    rng = np.random.default_rng(seed + 7)
    pos = ctx
    for n in (32, 5, 17):
        toks = rng.integers(0, cfg.vocab, n)
        say(f"{shape} grouped block of {n} at {pos}")
        blg, bam = g.step_batched(toks)
        olg, _, _, ohid = s.step_grouped(toks)
        assert bits_equal(blg, olg), (n, float(np.abs(blg - olg).max()))
        assert bam == oracle.argmax(olg)
        assert bits_equal(g.hidden(), ohid), n
        pos += n
    for l in range(cfg.layers):
        gk, gv = g.read_kv(l, pos)
        ok, ov = s.read_kv(l, pos)
        assert np.array_equal(gk[:, ctx:pos], ok[:, ctx:pos]) and np.array_equal(gv[:, ctx:pos], ov[:, ctx:pos]), l
    for t, tok in enumerate(rng.integers(0, cfg.vocab, 4)):
        lg, ids, w, _ = g.step(int(tok))
        olg, oids, ow, _ = s.step(int(tok))
        assert bits_equal(lg, olg) and np.array_equal(ids, oids) and bits_equal(w, ow), t
    g.close()


def test_grouped_mode_refusals(gpu):
    """Mode 1 needs a resident model with Q8_0 experts at a row length the grouped kernels are built for."""
    tiny = moert.SynthModel(moert.Config(**moert.TINY), seed=3)
    g = moert.GpuModel(tiny, 64, attn_splits=2)
    with pytest.raises(moert.MoertError, match="hidden"):
        g.batched_mode(1)
    with pytest.raises(moert.MoertError):
        g.batched_mode(2)
    g.batched_mode(0)
    g.close()
    cfg = moert.Config(**moert.GRANITE_1B)
    m4 = moert.SynthModel(cfg, seed=5, wdtype=moert.Q4_0)
    g4 = moert.GpuModel(m4, 64, attn_splits=2)
    with pytest.raises(moert.MoertError, match="Q8_0"):
        g4.batched_mode(1)
    g4.close()
