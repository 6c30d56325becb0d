"""Expert cache (experts in pinned host memory, an HBM pool of slots, LRU on the device) through the C ABI: every
output equals the resident model's bit for bit, and the hit / copy counters equal the LRU oracle replayed over the
routes the model took (the reference's check against reference_lru, tests/model.rs:414-434)."""
import numpy as np
import pytest

import moert
import oracle

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


TINY8 = dict(hidden=256, inter=128, layers=3, heads=4, kv_heads=2, head_dim=64, vocab=97, experts=8, top_k=2)


@pytest.mark.parametrize("wdtype", [moert.Q4_0, moert.Q8_0])
@pytest.mark.parametrize("slots", [2, 3, 5, 6, 24])
def test_cached_model_equals_the_resident_model_and_counts_like_the_lru_oracle(gpu, wdtype, slots):
    """tests/model.rs:414-434 with cache sizes 2..24 (24 = every expert of every layer fits)."""
    cfg = moert.Config(**TINY8)
    m = moert.SynthModel(cfg, seed=13, wdtype=wdtype, embed_dtype=moert.F32, std=0.1, zipf_s=1.1)
    res = moert.GpuModel(m, 64, attn_splits=4)
    cac = moert.GpuModel(m, 64, attn_splits=4, cache_slots=slots)
    toks = np.random.default_rng(123).integers(0, cfg.vocab, 48)
    routes = []
    for t, tok in enumerate(toks):
        say(f"cache dtype={wdtype} slots={slots} pos={t}")
        lg, ids, w, am = res.step(int(tok))
        clg, cids, cw, cam = cac.step(int(tok))
        assert bits_equal(lg, clg) and np.array_equal(ids, cids) and bits_equal(w, cw) and am == cam, t
        routes.append(ids)
    hits, copies, cpu = oracle.lru_replay(np.array(routes), cfg.experts, slots)
    assert cpu == 0
    assert cac.cache_stats() == (hits, copies)
    res.close()
    cac.close()


WIDE = dict(hidden=256, inter=128, layers=4, heads=4, kv_heads=2, head_dim=64, vocab=97, experts=64, top_k=8)


@pytest.mark.parametrize("slots", [8, 100, 200])
def test_pool_of_more_slots_than_a_wave_has_lanes(gpu, slots):
    """64 experts x 4 layers = 256 keys: the slot tables span several passes of a wave (slots > 64)."""
    cfg = moert.Config(**WIDE)
    m = moert.SynthModel(cfg, seed=21, wdtype=moert.Q4_0, embed_dtype=moert.F32, std=0.1, zipf_s=1.1)
    res = moert.GpuModel(m, 64, attn_splits=4)
    cac = moert.GpuModel(m, 64, attn_splits=4, cache_slots=slots)
    toks = np.random.default_rng(77).integers(0, cfg.vocab, 40)
    routes = []
    for t, tok in enumerate(toks):
        say(f"wide cache slots={slots} pos={t}")
        lg, ids, w, am = res.step(int(tok))
        clg, cids, cw, cam = cac.step(int(tok))
        assert bits_equal(lg, clg) and np.array_equal(ids, cids) and bits_equal(w, cw) and am == cam, t
        routes.append(ids)
    hits, copies, cpu = oracle.lru_replay(np.array(routes), cfg.experts, slots)
    assert cpu == 0
    assert cac.cache_stats() == (hits, copies)
    res.close()
    cac.close()


def test_cache_clear_restarts_from_an_empty_pool(gpu):
    cfg = moert.Config(**TINY8)
    m = moert.SynthModel(cfg, seed=14, wdtype=moert.Q4_0, embed_dtype=moert.F32, std=0.1)
    g = moert.GpuModel(m, 64, attn_splits=4, cache_slots=4)
    toks = [3, 17, 5, 60, 2, 9]
    say("cache clear")
    first = [g.step(t) for t in toks]
    s1 = g.cache_stats()
    g.cache_clear()
    assert g.cache_stats() == (0, 0)
    g.reset()
    again = [g.step(t) for t in toks]
    assert g.cache_stats() == s1
    for a, b in zip(first, again):
        assert bits_equal(a[0], b[0])
    g.close()


def test_cached_model_refuses_fewer_slots_than_top_k(gpu):
    m = moert.SynthModel(moert.Config(**TINY8), seed=15, wdtype=moert.Q4_0)
    with pytest.raises(moert.MoertError):
        moert.GpuModel(m, 64, attn_splits=4, cache_slots=1)


def _forced_pair(res, cac, toks, label, every=1):
    """Steps the resident and the cached model through the same forced tokens: logits (every `every` steps), ids,
    weights and argmax bit for bit. Returns the routes [steps, layers, k]."""
    routes = []
    for t, tok in enumerate(toks):
        if t % 64 == 0:
            say(f"{label} step {t}")
        want = t % every == 0
        lg, ids, w, am = res.step(int(tok), want_logits=want)
        clg, cids, cw, cam = cac.step(int(tok), want_logits=want)
        assert np.array_equal(ids, cids) and bits_equal(w, cw) and am == cam, t
        if want:
            assert bits_equal(lg, clg), t
        routes.append(ids)
    return np.array(routes)


def test_granite_3b_q4_0_quarter_pool_forced_512_steps_equals_the_resident_model(gpu, granite_3b_q4):
    """The expert-cache workload: 3B shape, Q4_0, Zipf(1.1) router bias, a pool of 25% of the 1280 experts (320
    slots), 512 steps from an empty pool with a forced random token stream (so the pool keeps evicting): every
    step's logits, ids, weights and argmax equal the resident model's bit for bit, and the hit / copy counters
    equal the LRU oracle replayed over the routes."""
    cfg, m = granite_3b_q4
    toks = np.random.default_rng(512).integers(0, cfg.vocab, 512)
    res = moert.GpuModel(m, 576, attn_splits=64)
    cac = moert.GpuModel(m, 576, attn_splits=64, cache_slots=320)
    routes = _forced_pair(res, cac, toks, "3b q4_0 forced")
    hits, copies, cpu = oracle.lru_replay(routes, cfg.experts, 320)
    say(f"3b q4_0 forced: {hits} hits, {copies} copies")
    assert cpu == 0 and copies > 20000
    assert cac.cache_stats() == (hits, copies)
    res.close()
    cac.close()


def test_granite_3b_q4_0_filled_pool_copies_nothing_for_the_filled_layers(gpu, granite_3b_q4):
    """A 320-slot pool filled from the host right after create holds keys 0..319 (layers 0-7): the first step then
    copies only the experts of layers 8-31 (24 x 8), its outputs equal the resident model's, and 64 forced steps
    keep equal outputs and counters equal to the LRU oracle started from the same fill (checks the strided fill
    copies at the 3B Q4_0 record size)."""
    cfg, m = granite_3b_q4
    toks = np.random.default_rng(64).integers(0, cfg.vocab, 64)
    res = moert.GpuModel(m, 128, attn_splits=64)
    cac = moert.GpuModel(m, 128, attn_splits=64, cache_slots=320)
    assert cac.cache_fill() == 320
    routes = _forced_pair(res, cac, toks[:1], "3b q4_0 filled")
    assert cac.cache_stats() == (8 * 8, 24 * 8)
    routes = np.concatenate([routes, _forced_pair(res, cac, toks[1:], "3b q4_0 filled")])
    lru = oracle.Lru(cfg.layers, cfg.experts, 320)
    assert lru.fill() == 320
    for r in routes:
        lru.step(r)
    hits, copies, _ = lru.stats()
    assert cac.cache_stats() == (hits, copies)
    res.close()
    cac.close()


def _replay_with_predictions(cfg, slots, routes, preds):
    """The LRU state machine over a prefetched run: per step and layer, the prefetch tick over the recorded
    prediction, then the layer's counted step. Returns (stats, per-step-layer prefetched copies)."""
    lru = oracle.Lru(cfg.layers, cfg.experts, slots)
    pf = np.zeros(routes.shape[:2], np.int64)
    for t in range(routes.shape[0]):
        for l in range(cfg.layers):
            assert (preds[t, l] >= 0).all(), (t, l)
            pf[t, l] = lru.prefetch(l, preds[t, l])
            lib = oracle.lib()
            a = np.ascontiguousarray(routes[t, l], np.int32)
            lib.orc_lru_step_layer(lru.h, l, a.ctypes.data_as(oracle.ctypes.c_void_p), a.size)
    return lru.stats(), pf


@pytest.mark.parametrize("slots", [3, 6, 12])
def test_prefetch_branch_keeps_outputs_and_its_evictions_replay_on_the_lru_oracle(gpu, slots):
    """The cached step with the prefetch branch (each layer's experts predicted from its input and copied on a side
    stream during attention): outputs equal the resident model's bit for bit; the recorded predictions replayed on
    the LRU state machine (prefetch tick, then the counted step, per layer) give the device's counters, per position
    and layer and in total."""
    cfg = moert.Config(**TINY8)
    m = moert.SynthModel(cfg, seed=13, wdtype=moert.Q4_0, embed_dtype=moert.F32, std=0.1, zipf_s=1.1)
    res = moert.GpuModel(m, 64, attn_splits=4)
    cac = moert.GpuModel(m, 64, attn_splits=4, cache_slots=slots)
    cac.cache_prefetch_mode(True)
    toks = np.random.default_rng(321).integers(0, cfg.vocab, 40)
    say(f"prefetch branch slots={slots}")
    routes = _forced_pair(res, cac, toks, "prefetch branch")
    preds = cac.cache_predictions(0, len(toks))
    (hits, copies, cpu), pf = _replay_with_predictions(cfg, slots, routes, preds)
    counts = cac.cache_token_counts(0, len(toks))
    c = cac.cache_counters()
    assert (c["hits"], c["copies"], c["prefetched"]) == (hits, copies, int(pf.sum()))
    assert np.array_equal(counts[:, :, 2], pf)
    assert counts[:, :, 0].sum() == hits and counts[:, :, 1].sum() == copies
    assert cpu == 0 and c["needed"] == hits + copies
    res.close()
    cac.close()


@pytest.mark.parametrize("max_len,splits,path", [(576, 64, "unfused"), (4416, 32, "block")])
def test_granite_3b_q4_0_prefetch_forced_512_steps(gpu, granite_3b_q4, max_len, splits, path):
    """The expert-cache workload with the prefetch: 512 forced steps from an empty 320-slot pool, outputs equal to
    the resident model's bit for bit, counters equal to the replay with the recorded predictions, and most predicted
    experts used (the prediction from the layer's input routes like the layer). At 576 positions (one tile per split)
    the prefetch is the side-stream branch beside the three-kernel attention; at the decode bench's 4416 / 32 splits
    it runs inside the attention block's launch."""
    cfg, m = granite_3b_q4
    toks = np.random.default_rng(512).integers(0, cfg.vocab, 512)
    res = moert.GpuModel(m, max_len, attn_splits=splits)
    cac = moert.GpuModel(m, max_len, attn_splits=splits, cache_slots=320)
    cac.cache_prefetch_mode(True)
    assert cac.kernel_path() == path
    routes = _forced_pair(res, cac, toks, f"3b q4_0 prefetch ({path})")
    preds = cac.cache_predictions(0, len(toks))
    (hits, copies, _), pf = _replay_with_predictions(cfg, 320, routes, preds)
    c = cac.cache_counters()
    say(f"3b prefetch: {hits} hits, {copies} copies in steps, {int(pf.sum())} prefetched")
    assert (c["hits"], c["copies"], c["prefetched"]) == (hits, copies, int(pf.sum()))
    agree = np.mean([len(set(preds[t, l]) & set(routes[t, l])) / cfg.top_k
                     for t in range(len(toks)) for l in range(cfg.layers)])
    say(f"3b prefetch: predicted experts routed {agree:.3f}")
    assert agree > 0.5
    res.close()
    cac.close()


def test_fill_after_decode_steps_stamps_the_current_clock(gpu):
    """ExpertCache::fill on a partly filled pool after decode steps (no clear): the filled experts take the current
    clock as their last use (copy_on_compute, cache/core.rs:366-377), so later steps evict them as recently used.
    Counters equal the LRU oracle over the same trace (steps, fill, steps); the trace is one where stamping the fill
    with 0 would give other counters."""
    cfg = moert.Config(**TINY8)
    m = moert.SynthModel(cfg, seed=13, wdtype=moert.Q4_0, embed_dtype=moert.F32, std=0.1, zipf_s=1.1)
    res = moert.GpuModel(m, 64, attn_splits=4)
    cac = moert.GpuModel(m, 64, attn_splits=4, cache_slots=22)
    toks = np.random.default_rng(321).integers(0, cfg.vocab, 40)
    say("fill after decode")
    first = _forced_pair(res, cac, toks[:4], "fill after decode")
    filled = cac.cache_fill()
    second = _forced_pair(res, cac, toks[4:], "fill after decode")
    ops = [("step", l, r[l].tolist()) for r in first for l in range(cfg.layers)] + [("fill", cfg.layers * cfg.experts)]
    ops += [("step", l, r[l].tolist()) for r in second for l in range(cfg.layers)]
    want = oracle.lru_reference_ops(ops, cfg.experts, 22)
    assert want != oracle.lru_reference_ops(ops, cfg.experts, 22, fill_stamp_clock=False)
    lru = oracle.Lru(cfg.layers, cfg.experts, 22)
    for r in first:
        lru.step(r)
    assert lru.fill() == filled
    for r in second:
        lru.step(r)
    assert lru.stats() == want
    assert cac.cache_stats() == want[:2]
    res.close()
    cac.close()


def test_prefetch_ticks_evict_like_the_lru_oracle(gpu):
    """Per-layer prefetches (one uncounted tick of the LRU rule each) interleaved with decode steps on a 5-slot pool:
    the outputs stay the resident model's, and the step counters equal the oracle's state machine over the same
    trace, so each prefetch evicted the slots the rule chooses."""
    cfg = moert.Config(**TINY8)
    m = moert.SynthModel(cfg, seed=17, wdtype=moert.Q8_0, embed_dtype=moert.F32, std=0.1, zipf_s=1.1)
    res = moert.GpuModel(m, 64, attn_splits=4)
    cac = moert.GpuModel(m, 64, attn_splits=4, cache_slots=5)
    lru = oracle.Lru(cfg.layers, cfg.experts, 5)
    rng = np.random.default_rng(8)
    toks = rng.integers(0, cfg.vocab, 24)
    for t, tok in enumerate(toks):
        say(f"prefetch trace step {t}")
        if t % 3 == 1:
            layer = int(rng.integers(0, cfg.layers))
            ex = rng.choice(cfg.experts, size=int(rng.integers(1, 4)), replace=False)
            assert cac.cache_prefetch(layer, ex) == lru.prefetch(layer, ex)
        r = _forced_pair(res, cac, [tok], "prefetch trace")
        lru.step(r[0])
        assert cac.cache_stats() == lru.stats()[:2], t
    res.close()
    cac.close()


@pytest.mark.parametrize("wdtype,slots", [(moert.Q4_0, 6), (moert.Q8_0, 8)])
def test_prefetch_of_a_steps_routes_makes_that_step_all_hits(gpu, wdtype, slots):
    """Before each step, every layer's routed experts (taken from the resident model) are prefetched: the step then
    copies nothing and hits k per layer, and its outputs stay those of the resident model. A prefetch counts no
    requests, so the counters grow by the steps' hits only."""
    cfg = moert.Config(**TINY8)
    m = moert.SynthModel(cfg, seed=16, wdtype=wdtype, embed_dtype=moert.F32, std=0.1, zipf_s=1.1)
    res = moert.GpuModel(m, 64, attn_splits=4)
    cac = moert.GpuModel(m, 64, attn_splits=4, cache_slots=slots)
    toks = np.random.default_rng(31).integers(0, cfg.vocab, 20)
    copied_total = 0
    for t, tok in enumerate(toks):
        say(f"prefetch dtype={wdtype} slots={slots} pos={t}")
        lg, ids, w, am = res.step(int(tok))
        for l in range(cfg.layers):
            copied_total += cac.cache_prefetch(l, ids[l])
        before = cac.cache_stats()
        clg, cids, cw, cam = cac.step(int(tok))
        after = cac.cache_stats()
        assert after[1] == before[1], t
        assert after[0] - before[0] == cfg.layers * cfg.top_k, t
        assert bits_equal(lg, clg) and np.array_equal(ids, cids) and bits_equal(w, cw) and am == cam, t
    assert copied_total > 0
    hits, copies = cac.cache_stats()
    assert (hits, copies) == (len(toks) * cfg.layers * cfg.top_k, 0)
    # refusals: a repeated expert, more experts than slots, a layer out of range, a model without a cache
    with pytest.raises(moert.MoertError):
        cac.cache_prefetch(0, [1, 1])
    with pytest.raises(moert.MoertError):
        cac.cache_prefetch(0, list(range(slots + 1)))
    with pytest.raises(moert.MoertError):
        cac.cache_prefetch(cfg.layers, [0])
    with pytest.raises(moert.MoertError):
        res.cache_prefetch(0, [0])
    res.close()
    cac.close()


@pytest.mark.parametrize("slots", [24, 5])
def test_fill_puts_missing_experts_into_free_slots_in_key_order(gpu, slots):
    """ExpertCache::fill (cache.rs:212-227): with room for every key (24 = 3 layers x 8 experts) the fill copies all
    of them and later steps copy nothing; with 5 slots it copies keys 0..4 and stops. A second fill copies nothing.
    Outputs stay the resident model's either way."""
    cfg = moert.Config(**TINY8)
    m = moert.SynthModel(cfg, seed=17, wdtype=moert.Q4_0, embed_dtype=moert.F32, std=0.1, zipf_s=1.1)
    res = moert.GpuModel(m, 64, attn_splits=4)
    cac = moert.GpuModel(m, 64, attn_splits=4, cache_slots=slots)
    say(f"fill slots={slots}")
    assert cac.cache_fill() == min(slots, cfg.layers * cfg.experts)
    assert cac.cache_fill() == 0
    assert cac.cache_stats() == (0, 0)
    toks = np.random.default_rng(32).integers(0, cfg.vocab, 16)
    for t, tok in enumerate(toks):
        lg, ids, w, am = res.step(int(tok))
        clg, cids, cw, cam = cac.step(int(tok))
        assert bits_equal(lg, clg) and np.array_equal(ids, cids) and bits_equal(w, cw) and am == cam, t
    hits, copies = cac.cache_stats()
    assert hits + copies == len(toks) * cfg.layers * cfg.top_k
    if slots == 24:
        assert copies == 0
    cac.cache_clear()
    assert cac.cache_fill() == min(slots, cfg.layers * cfg.experts)
    with pytest.raises(moert.MoertError):
        res.cache_fill()
    res.close()
    cac.close()
