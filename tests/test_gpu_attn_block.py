"""The attention block kernel (q/k/v + RoPE + KV append, split-KV attention and merge in one launch, exchanging
through the L2 of each KV head's XCD) against the oracle's session and against the three-kernel path
(MOERT_ATTN_BLOCK=0), bit for bit: logits, routes and weights of every step, hidden state and KV rows. Shapes: the
3B model at the bench's 32 requested splits (23 splits of 3 tiles) across a tile and a split boundary, the 1B model
from position 0 (one used split), a Q4_0 expert-cache model, and the launch counts of both paths."""
import os

import numpy as np
import pytest

import moert
import oracle

pytestmark = pytest.mark.gpu
THREADS = min(16, os.cpu_count() or 1)
MAX_LEN, SPLITS = 4416, 32  # the bench's cache: 23 splits of 3 tiles


def say(msg):
    print(f"[case] {msg}", flush=True)


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def env_model(m, max_len, splits, var, val, **kw):
    os.environ[var] = val
    try:
        return moert.GpuModel(m, max_len, attn_splits=splits, **kw)
    finally:
        del os.environ[var]


def three_kernel_model(m, max_len, splits, var="MOERT_ATTN_BLOCK", **kw):
    """A model created with `var`=0 (MOERT_ATTN_BLOCK: q/k/v, split attention and combine as three kernels, and the
    MoE half as k_route_up + k_expert_down; MOERT_MOE_XCD: only the MoE half as those two kernels)."""
    return env_model(m, max_len, splits, var, "0", **kw)


def fused_model(m, max_len, splits, **kw):
    """The attention block, the output projection and the MoE kernel over the XCDs as separate launches
    (MOERT_LAYER=0), not one launch per layer."""
    return env_model(m, max_len, splits, "MOERT_LAYER", "0", **kw)


def path_model(m, max_len, splits, path, **kw):
    """path "layer": one launch per layer (the default where the shape allows it); "fused": MOERT_LAYER=0."""
    if path == "fused":
        return fused_model(m, max_len, splits, **kw)
    return moert.GpuModel(m, max_len, attn_splits=splits, **kw)


def launches(g, kind):
    """Launches of a kernel class in one step (run at the cache's last position, after the parity checks)."""
    g.set_position(g.max_len - 1)
    return g.time_kernel(kind, 1)[1]


@pytest.fixture(scope="module")
def granite_3b():
    cfg = moert.Config(**moert.GRANITE_3B)
    say("3B build")
    m = moert.SynthModel(cfg, seed=3003, wdtype=moert.Q8_0, embed_dtype=moert.Q8_0)
    return cfg, m, [moert.kv_prefill_data(cfg, 3003, l, 4096) for l in range(cfg.layers)]


@pytest.mark.parametrize("path", ["layer", "fused"])
def test_attn_block_3b_forced_tokens_across_tile_and_split_boundaries(gpu, granite_3b, path):
    """3B, KV pre-filled to 4096: forced tokens at positions 4088..4103 (the tile boundary at 4096, inside split 21)
    and 4218..4229 (the split boundary at 4224): every step's logits, routes and weights equal the oracle's, then
    the hidden state and every KV row written."""
    cfg, m, kv = granite_3b
    g = path_model(m, MAX_LEN, SPLITS, path)
    assert g.kernel_path() == path
    s = oracle.CpuSession(m, MAX_LEN, attn_splits=SPLITS, threads=THREADS)
    for l, (k, v) in enumerate(kv):
        g.kv_prefill(l, k, v)
        s.kv_prefill(l, k, v)
    rng = np.random.default_rng(41)
    for start, n in ((4088, 16), (4218, 12)):
        g.set_position(start)
        s.set_position(start)
        for t, tok in enumerate(rng.integers(0, cfg.vocab, n)):
            say(f"3B attention block pos={start + t}")
            lg, ids, w, am = g.step(int(tok))
            olg, oids, ow, oh = s.step(int(tok))
            assert np.array_equal(ids, oids) and bits_equal(w, ow), start + t
            assert bits_equal(lg, olg) and am == oracle.argmax(olg), start + t
        assert bits_equal(g.hidden(), oh)
    for l in range(cfg.layers):
        gk, gv = g.read_kv(l, 4230)
        ok, ov = s.read_kv(l, 4230)
        assert np.array_equal(gk, ok) and np.array_equal(gv, ov), l
    if path == "fused":
        assert launches(g, moert.K_ATTN_BLOCK) == cfg.layers and launches(g, moert.K_MOE_XCD) == cfg.layers
        assert launches(g, moert.K_MOE_COMBINE) == 1 and launches(g, moert.K_LAYER) == 0
    else:
        assert launches(g, moert.K_LAYER) == cfg.layers and launches(g, moert.K_LAYER_COMBINE) == 1
        assert launches(g, moert.K_ATTN_BLOCK) == 0 and launches(g, moert.K_OPROJ) == 0
    assert launches(g, moert.K_ROUTE_UP) == 0 and launches(g, moert.K_QKV) == 0
    assert launches(g, moert.K_ATTN_COMBINE) == 0
    g.close()


@pytest.mark.parametrize("path", ["layer", "fused"])
def test_attn_block_1b_from_position_zero_greedy_identical(gpu, path):
    """1B shape (2 query heads per KV head) with the bench's cache shape: a 128-token prompt and 64 greedy tokens
    from position 0 (only the first split is used, the new row moves through its three tiles): identical tokens,
    last logits and hidden state, every KV row."""
    cfg = moert.Config(**moert.GRANITE_1B)
    say("1B build")
    m = moert.SynthModel(cfg, seed=2024, wdtype=moert.Q8_0, embed_dtype=moert.F32, std=0.1)
    g = path_model(m, MAX_LEN, SPLITS, path)
    assert g.kernel_path() == path
    s = oracle.CpuSession(m, MAX_LEN, attn_splits=SPLITS, threads=THREADS)
    prompt = np.random.default_rng(2025).integers(0, cfg.vocab, 128)
    say("1B attention block generate")
    out = g.generate(prompt, 64)
    want, _ = s.generate(prompt, 64)
    assert out.tolist() == want.tolist()
    assert bits_equal(g.read_logits(), s.last_logits)
    assert bits_equal(g.hidden(), s.last_hidden)
    for l in range(cfg.layers):
        gk, gv = g.read_kv(l, 192)
        ok, ov = s.read_kv(l, 192)
        assert np.array_equal(gk, ok) and np.array_equal(gv, ov), l
    assert launches(g, moert.K_ATTN_BLOCK if path == "fused" else moert.K_LAYER) == cfg.layers
    g.close()


def test_attn_block_equals_the_three_kernel_path(gpu, granite_3b):
    """The same 3B model with and without the attention block: 64 forced steps after 4096 cached positions, logits
    and hidden state bit for bit; the three-kernel model launches q/k/v, split and combine and no block."""
    cfg, m, kv = granite_3b
    a = fused_model(m, MAX_LEN, SPLITS)
    b = three_kernel_model(m, MAX_LEN, SPLITS)
    assert a.kernel_path() == "fused" and b.kernel_path() == "unfused"
    for l, (k, v) in enumerate(kv):
        a.kv_prefill(l, k, v)
        b.kv_prefill(l, k, v)
    a.set_position(4096)
    b.set_position(4096)
    for t, tok in enumerate(np.random.default_rng(43).integers(0, cfg.vocab, 64)):
        if t % 16 == 0:
            say(f"3B block vs three kernels step {t}")
        la, ia, wa, ma = a.step(int(tok))
        lb, ib, wb, mb = b.step(int(tok))
        assert bits_equal(la, lb) and np.array_equal(ia, ib) and bits_equal(wa, wb) and ma == mb, t
    assert bits_equal(a.hidden(), b.hidden())
    assert launches(b, moert.K_ATTN_BLOCK) == 0 and launches(b, moert.K_QKV) == cfg.layers
    a.close()
    b.close()


def test_attn_block_in_the_expert_cache_model(gpu):
    """1B shape with its experts in a 192-slot pool (25% of 768) and the Zipf router bias: 48 forced steps with
    the attention block equal the resident three-kernel model's logits bit for bit."""
    cfg = moert.Config(**moert.GRANITE_1B)
    say("1B cached build")
    m = moert.SynthModel(cfg, seed=77, wdtype=moert.Q8_0, embed_dtype=moert.Q8_0, zipf_s=1.1)
    res = three_kernel_model(m, MAX_LEN, SPLITS)
    cac = moert.GpuModel(m, MAX_LEN, attn_splits=SPLITS, cache_slots=192)
    for t, tok in enumerate(np.random.default_rng(45).integers(0, cfg.vocab, 48)):
        lr, ir, wr, _ = res.step(int(tok))
        lc, ic, wc, _ = cac.step(int(tok))
        assert bits_equal(lr, lc) and np.array_equal(ir, ic) and bits_equal(wr, wc), t
    assert launches(cac, moert.K_ATTN_BLOCK) == cfg.layers
    res.close()
    cac.close()


def test_attn_block_q4_0_rows_equal_the_three_kernel_path(gpu):
    """Q4_0 q/k/v rows of the 3B shape (the expert-cache workload's dtype), four layers: 40 forced steps after 4096
    cached positions with and without the attention block, logits bit for bit."""
    cfg = moert.Config(**{**moert.GRANITE_3B, "layers": 4})
    say("3B-shaped Q4_0 build")
    m = moert.SynthModel(cfg, seed=5, wdtype=moert.Q4_0, embed_dtype=moert.Q8_0, zipf_s=1.1)
    a = fused_model(m, MAX_LEN, SPLITS)
    b = three_kernel_model(m, MAX_LEN, SPLITS)
    c = path_model(m, MAX_LEN, SPLITS, "layer")
    assert a.kernel_path() == "fused" and c.kernel_path() == "layer"
    for l in range(cfg.layers):
        k, v = moert.kv_prefill_data(cfg, 5, l, 4096)
        for g in (a, b, c):
            g.kv_prefill(l, k, v)
    for g in (a, b, c):
        g.set_position(4096)
    for t, tok in enumerate(np.random.default_rng(47).integers(0, cfg.vocab, 40)):
        la, ia, wa, _ = a.step(int(tok))
        lb, ib, wb, _ = b.step(int(tok))
        lc, ic, wc, _ = c.step(int(tok))
        assert bits_equal(la, lb) and np.array_equal(ia, ib) and bits_equal(wa, wb), t
        assert bits_equal(lc, lb) and np.array_equal(ic, ib) and bits_equal(wc, wb), t
    assert launches(a, moert.K_ATTN_BLOCK) == cfg.layers and launches(c, moert.K_LAYER) == cfg.layers
    for g in (a, b, c):
        g.close()


def test_moe_spread_over_the_xcds_equals_route_up_and_down(gpu, granite_3b):
    """The MoE half with the routed experts spread over the XCDs (k_moe_xcd, combined by the next attention block)
    against k_route_up + k_expert_down, both with the attention block: 48 forced steps after 4096 cached positions,
    logits, routes, weights and hidden state bit for bit; the launch counts of both."""
    cfg, m, kv = granite_3b
    a = fused_model(m, MAX_LEN, SPLITS)
    b = three_kernel_model(m, MAX_LEN, SPLITS, var="MOERT_MOE_XCD")
    assert a.kernel_path() == "fused" and b.kernel_path() == "block"
    for l, (k, v) in enumerate(kv):
        a.kv_prefill(l, k, v)
        b.kv_prefill(l, k, v)
    a.set_position(4096)
    b.set_position(4096)
    for t, tok in enumerate(np.random.default_rng(49).integers(0, cfg.vocab, 48)):
        if t % 16 == 0:
            say(f"3B experts over the XCDs vs route_up + down step {t}")
        la, ia, wa, ma = a.step(int(tok))
        lb, ib, wb, mb = b.step(int(tok))
        assert bits_equal(la, lb) and np.array_equal(ia, ib) and bits_equal(wa, wb) and ma == mb, t
    assert bits_equal(a.hidden(), b.hidden())
    assert launches(b, moert.K_MOE_XCD) == 0 and launches(b, moert.K_ROUTE_UP) == cfg.layers
    assert launches(b, moert.K_ATTN_BLOCK) == cfg.layers
    assert launches(a, moert.K_MOE_XCD) == cfg.layers and launches(a, moert.K_EXPERT_DOWN) == 0
    a.close()
    b.close()


@pytest.fixture(scope="module")
def granite_1b_wide():
    cfg = moert.Config(**moert.GRANITE_1B)
    say("1B wide build")
    return cfg, moert.SynthModel(cfg, seed=2024, wdtype=moert.Q8_0, embed_dtype=moert.F32, std=0.1)


WAIT_NAMES = {2: "the wait for queries / the new K/V row", 4: "the wait for split partials",
              8: "the wait for an expert's act vector"}


@pytest.mark.parametrize("path", ["layer", "fused"])
@pytest.mark.parametrize("bit", [2, 4, 8])
def test_a_wait_that_gives_up_is_reported_and_poisons_the_handle(gpu, granite_1b_wide, bit, path):
    """The failure path of the fused kernels, forced from the host (moert_fault_inject: the named wait looks for an
    epoch no launch writes, every wait of those launches is bounded to a few hundred polls, and every kernel still
    ends): a 64-step generate reports MOERT_E_DEVICE naming that wait, the launches queued after the failure wait
    for nothing (the whole call ends within seconds), the handle is poisoned, and a fresh model in the same process
    decodes bit for bit like the oracle."""
    import time
    cfg, m = granite_1b_wide
    g = path_model(m, MAX_LEN, SPLITS, path)
    assert g.kernel_path() == path
    g.step(5)
    say(f"fault inject bit {bit}")
    g.fault_inject(bit)
    t0 = time.time()
    with pytest.raises(moert.MoertError) as e:
        g.generate([7], 64)
    dt = time.time() - t0
    assert e.value.code == moert.E_DEVICE, str(e.value)
    msg = str(e.value)
    assert WAIT_NAMES[bit] in msg and f"error bits {bit:#x}" in msg, msg
    for other, name in WAIT_NAMES.items():
        assert other == bit or name not in msg, msg
    assert dt < 20, dt
    with pytest.raises(moert.MoertError) as e:
        g.step(5)
    assert e.value.code == moert.E_POISONED
    g.close()
    say("fresh model after the failure")
    f = moert.GpuModel(m, MAX_LEN, attn_splits=SPLITS)
    s = oracle.CpuSession(m, MAX_LEN, attn_splits=SPLITS, threads=THREADS)
    for t, tok in enumerate(np.random.default_rng(51).integers(0, cfg.vocab, 12)):
        lg, ids, w, am = f.step(int(tok))
        olg, oids, ow, _ = s.step(int(tok))
        assert bits_equal(lg, olg) and np.array_equal(ids, oids) and bits_equal(w, ow), t
    f.close()


def test_fault_inject_refusals(gpu, granite_1b_wide):
    cfg, m = granite_1b_wide
    g = three_kernel_model(m, MAX_LEN, SPLITS)
    assert g.kernel_path() == "unfused"
    with pytest.raises(moert.MoertError) as e:
        g.fault_inject(2)
    assert e.value.code == moert.E_CONFIG
    g.close()
    g = moert.GpuModel(m, MAX_LEN, attn_splits=SPLITS)
    with pytest.raises(moert.MoertError) as e:
        g.fault_inject(1)
    assert e.value.code == moert.E_CONFIG
    g.fault_inject(0)  # an empty mask is a no-op
    g.step(3)
    g.close()


def test_prefetch_runs_inside_the_attention_block_and_decides_like_the_branch(gpu):
    """The cache's prefetch at the bench's cache shape runs inside the attention launch (one decide and 64 copy
    workgroups after the attention workgroups, cache_pf.h): with it on, the cached model still launches the attention
    block, its logits, ids and weights equal the resident three-kernel model's bit for bit, and its predictions and
    counters (hits, copies, prefetched) equal those of the same model with the side-stream branch (MOERT_PF_BLOCK=0,
    which uses the three-kernel attention) over the same forced tokens."""
    cfg = moert.Config(**moert.GRANITE_1B)
    say("1B cached build (prefetch inside the block)")
    m = moert.SynthModel(cfg, seed=78, wdtype=moert.Q8_0, embed_dtype=moert.Q8_0, zipf_s=1.1)
    res = three_kernel_model(m, MAX_LEN, SPLITS)
    blk = moert.GpuModel(m, MAX_LEN, attn_splits=SPLITS, cache_slots=192)
    brn = moert.GpuModel(m, MAX_LEN, attn_splits=SPLITS, cache_slots=192)
    assert blk.kernel_path() == "block"
    blk.cache_prefetch_mode(True)
    assert blk.kernel_path() == "block"
    os.environ["MOERT_PF_BLOCK"] = "0"
    try:
        brn.cache_prefetch_mode(True)
    finally:
        del os.environ["MOERT_PF_BLOCK"]
    assert brn.kernel_path() == "unfused"
    toks = np.random.default_rng(46).integers(0, cfg.vocab, 40)
    for t, tok in enumerate(toks):
        lr, ir, wr, _ = res.step(int(tok))
        for g in (blk, brn):
            lc, ic, wc, _ = g.step(int(tok))
            assert bits_equal(lr, lc) and np.array_equal(ir, ic) and bits_equal(wr, wc), t
    assert np.array_equal(blk.cache_predictions(0, len(toks)), brn.cache_predictions(0, len(toks)))
    cb, cr = blk.cache_counters(), brn.cache_counters()
    say(f"prefetch inside the block: {cb['hits']} hits, {cb['copies']} copies, {cb['prefetched']} prefetched")
    assert cb["prefetched"] > 0
    assert all(cb[k] == cr[k] for k in ("hits", "copies", "prefetched", "needed")), (cb, cr)
    # prefetch off again: the same block without the extra workgroups, same logits
    blk.cache_prefetch_mode(False)
    assert blk.kernel_path() == "block"
    for tok in toks[:4]:
        lr, _, _, _ = res.step(int(tok))
        lc, _, _, _ = blk.step(int(tok))
        assert bits_equal(lr, lc)
    blk.cache_prefetch_mode(True)
    assert launches(blk, moert.K_ATTN_BLOCK) == cfg.layers and launches(blk, moert.K_QKV) == 0
    assert launches(brn, moert.K_ATTN_BLOCK) == 0 and launches(brn, moert.K_QKV) == cfg.layers
    for g in (res, blk, brn):
        g.close()


def test_hybrid_with_the_attention_block_equals_the_three_kernel_hybrid(gpu):
    """The host-CPU hybrid at the bench's cache shape uses the attention block: 32 forced steps with a 96-slot pool
    and backlog 4 give the same logits bit for bit as the same hybrid built with the three-kernel attention (the
    placement decides alike, the host part is computed alike), and the same placement counters."""
    cfg = moert.Config(**moert.GRANITE_1B)
    say("1B hybrid build")
    m = moert.SynthModel(cfg, seed=79, wdtype=moert.Q8_0, embed_dtype=moert.Q8_0, zipf_s=1.1)
    a = moert.GpuModel(m, MAX_LEN, attn_splits=SPLITS, hybrid=(96, 4, 4))
    b = three_kernel_model(m, MAX_LEN, SPLITS, hybrid=(96, 4, 4))
    assert a.kernel_path() == "block" and b.kernel_path() == "unfused"
    for t, tok in enumerate(np.random.default_rng(48).integers(0, cfg.vocab, 32)):
        la, ia, wa, _ = a.step(int(tok))
        lb, ib, wb, _ = b.step(int(tok))
        assert bits_equal(la, lb) and np.array_equal(ia, ib) and bits_equal(wa, wb), t
    assert a.cache_counters() == b.cache_counters()
    a.close()
    b.close()


@pytest.mark.parametrize("path", ["layer", "fused"])
def test_prefill_then_fused_decode_equals_the_oracle(gpu, granite_1b_wide, path):
    """A 70-token block prefill (multi-position kernels) into the bench's cache shape, then 24 forced decode steps
    through the fused kernels: the prefill's last logits and every decode step's logits, routes and weights equal
    the oracle's session, and every KV row."""
    cfg, m = granite_1b_wide
    g = path_model(m, MAX_LEN, SPLITS, path)
    s = oracle.CpuSession(m, MAX_LEN, attn_splits=SPLITS, threads=THREADS)
    rng = np.random.default_rng(52)
    prompt = rng.integers(0, cfg.vocab, 70)
    say("prefill 70 into 4416/32")
    plg, pam = g.prefill(prompt)
    for tok in prompt:
        olg = s.step(int(tok))[0]
    assert bits_equal(plg, olg) and pam == oracle.argmax(olg)
    for t, tok in enumerate(rng.integers(0, cfg.vocab, 24)):
        lg, ids, w, am = g.step(int(tok))
        olg, oids, ow, _ = s.step(int(tok))
        assert bits_equal(lg, olg) and np.array_equal(ids, oids) and bits_equal(w, ow), t
    for l in range(cfg.layers):
        gk, gv = g.read_kv(l, 94)
        ok, ov = s.read_kv(l, 94)
        assert np.array_equal(gk, ok) and np.array_equal(gv, ov), l
    assert g.kernel_path() == path
    if path == "layer":
        assert launches(g, moert.K_LAYER) == cfg.layers and launches(g, moert.K_LAYER_COMBINE) == 1
    else:
        assert launches(g, moert.K_ATTN_BLOCK) == cfg.layers and launches(g, moert.K_MOE_XCD) == cfg.layers
    g.close()


def test_prefetch_copy_wait_failure_is_reported_and_poisons(gpu):
    """The failure path of the prefetch inside the attention launch, forced from the host (moert_fault_inject bit
    16: the copy workgroups wait for an epoch the decide does not write, a few hundred polls): the step returns
    MOERT_E_DEVICE naming the prefetch's wait, every kernel ends, the handle is poisoned afterwards, and a fresh
    cached model with the prefetch in the same process still decodes bit-identically to the resident model. The bit
    is refused without the in-launch prefetch and together with other bits."""
    cfg = moert.Config(**moert.GRANITE_1B)
    say("1B cached build (prefetch failure path)")
    m = moert.SynthModel(cfg, seed=81, wdtype=moert.Q8_0, embed_dtype=moert.Q8_0, zipf_s=1.1)
    res = three_kernel_model(m, MAX_LEN, SPLITS)
    cac = moert.GpuModel(m, MAX_LEN, attn_splits=SPLITS, cache_slots=192)
    with pytest.raises(moert.MoertError) as e:
        cac.fault_inject(16)  # prefetch off
    assert e.value.code == moert.E_CONFIG
    cac.cache_prefetch_mode(True)
    with pytest.raises(moert.MoertError) as e:
        cac.fault_inject(16 | 2)
    assert e.value.code == moert.E_CONFIG
    toks = np.random.default_rng(52).integers(0, cfg.vocab, 12)
    for tok in toks[:4]:
        lr, _, _, _ = res.step(int(tok))
        lc, _, _, _ = cac.step(int(tok))
        assert bits_equal(lr, lc)
    cac.fault_inject(16)
    with pytest.raises(moert.MoertError) as e:
        cac.step(int(toks[4]))
    assert e.value.code == moert.E_DEVICE and "prefetch" in str(e.value), str(e.value)
    with pytest.raises(moert.MoertError) as e:
        cac.step(int(toks[5]))
    assert e.value.code == moert.E_POISONED
    cac.close()
    res.close()
    say("fresh cached model after the failure")
    res = three_kernel_model(m, MAX_LEN, SPLITS)
    fresh = moert.GpuModel(m, MAX_LEN, attn_splits=SPLITS, cache_slots=192)
    fresh.cache_prefetch_mode(True)
    assert fresh.kernel_path() == "block"
    for tok in toks:
        lr, ir, wr, _ = res.step(int(tok))
        lc, ic, wc, _ = fresh.step(int(tok))
        assert bits_equal(lr, lc) and np.array_equal(ir, ic) and bits_equal(wr, wc)
    fresh.close()
    res.close()
