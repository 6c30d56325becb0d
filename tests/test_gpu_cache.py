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


def test_granite_3b_q4_0_quarter_pool_greedy_decode_equals_the_resident_model(gpu):
    """The expert-cache workload at a reduced length: 3B shape, Q4_0, Zipf(1.1) router bias, a pool of 25% of the
    1280 experts (320 slots); 96 greedy tokens identical to the resident model, counters equal to the oracle."""
    cfg = moert.Config(**moert.GRANITE_3B)
    m = moert.SynthModel(cfg, seed=4242, wdtype=moert.Q4_0, embed_dtype=moert.Q4_0, zipf_s=1.1)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 8)
    say("3b q4_0 resident")
    res = moert.GpuModel(m, 128, attn_splits=64)
    want = res.generate(prompt, 96)
    res.close()
    say("3b q4_0 cached")
    cac = moert.GpuModel(m, 128, attn_splits=64, cache_slots=320)
    routes = []
    toks = list(prompt) + list(want[:-1])
    got = []
    for t, tok in enumerate(toks):
        lg, ids, w, am = cac.step(int(tok))
        routes.append(ids)
        if t >= len(prompt) - 1:
            got.append(am)
    assert got == list(want)
    hits, copies, cpu = oracle.lru_replay(np.array(routes), cfg.experts, 320)
    assert cac.cache_stats() == (hits, copies)
    assert hits > 0 and copies > 0
    cac.close()
