"""The CPU port of the reference's CPU decode path (oracle/cpu_port.cpp), the CPU baseline bench.py times: its dot
(dot_avx2's four 8-lane accumulators, rust/moe-rt/src/cpu.rs:30-52) is pinned against float64, and whole decode
steps agree with the oracle's session within float rounding (the two differ only in their summation orders)."""
import numpy as np
import pytest

import moert
import oracle


@pytest.mark.parametrize("dtype", [moert.F32, moert.Q8_0, moert.Q4_0])
def test_port_dot_matches_float64_of_the_dequantised_row(dtype):
    """Every row length the models use, plus f32 rows whose length leaves a tail after the 32-element steps
    (dot_scalar's groups of four and remainder)."""
    shapes = [(5, 128), (9, 512), (6, 1024), (4, 1536)] + ([(3, 100), (3, 37), (2, 3)] if dtype == moert.F32 else [])
    for rows, cols in shapes:
        w = moert.synth_quantized(21, rows, rows * cols, 0.02, dtype)
        x = moert.synth_normal(22, cols, cols)
        wf = oracle.dequant(w, dtype, rows * cols).reshape(rows, cols).astype(np.float64)
        for r in range(rows):
            got = oracle.port_dot(w, dtype, cols, r, x)
            want = float(wf[r] @ x.astype(np.float64))
            tol = 1e-5 * (1.0 + float(np.abs(wf[r]) @ np.abs(x.astype(np.float64))))
            assert abs(got - want) <= tol, (rows, cols, r, got, want)


def test_port_dot_accumulates_in_four_lanes_of_eight():
    """The accumulation order itself: with weights 1 and x = [2^24, 1, 1, ..., -2^24, ...] placed so that each
    accumulator lane sees its own large value, the small terms survive only if lanes are kept apart as in
    dot_avx2 (lane j of accumulator a holds elements 32t + 8a + j) and summed after the loop."""
    cols = 64
    w = np.ones(cols, np.float32)
    x = np.ones(cols, np.float32)
    x[0] = 2.0 ** 24   # lane 0 of accumulator 0, first step
    x[32] = -2.0 ** 24  # the same lane, second step: cancels exactly in that lane
    got = oracle.port_dot(w, moert.F32, cols, 0, x)
    # lane (0, 0) ends at 0 exactly (2^24 + (-2^24)); the other 62 elements add up to 62
    assert got == 62.0
    # a plain sequential sum would lose the ones added to 2^24 (2^24 + 1 == 2^24 in f32)
    seq = np.float32(0)
    for v in x:
        seq = np.float32(seq + v)
    assert seq != got


def _pair(cfg, seed, std, max_len, wdtype=moert.Q8_0, edtype=moert.Q8_0):
    m = moert.SynthModel(cfg, seed=seed, wdtype=wdtype, embed_dtype=edtype, std=std)
    return m, oracle.CpuSession(m, max_len, attn_splits=4, threads=3), oracle.PortSession(m, max_len, threads=3)


@pytest.mark.parametrize("wdtype,edtype", [(moert.Q8_0, moert.Q8_0), (moert.Q4_0, moert.F32), (moert.F32, moert.F32)])
def test_port_session_agrees_with_the_oracle_within_rounding(wdtype, edtype):
    """70 forced steps of the tiny model (two attention tiles): the same routed experts, and routing weights and
    logits within float rounding of the oracle's session (bounds two orders of magnitude under the 1e-2 bar)."""
    cfg = moert.Config(**moert.TINY)
    m, s, p = _pair(cfg, 17, 0.1, 128, wdtype, edtype)
    for t, tok in enumerate(np.random.default_rng(3).integers(0, cfg.vocab, 70)):
        olg, oids, ow, _ = s.step(int(tok))
        plg, pids, pw = p.step(int(tok))
        assert np.array_equal(oids, pids), t
        assert float(np.abs(ow - pw).max()) <= 1e-3, t  # measured: below 1.5e-4
        scale = float(np.abs(olg).max())
        assert float(np.abs(plg - olg).max()) <= 2e-4 * scale, t  # measured: below 3e-5 of the largest logit


def test_port_session_after_a_prefilled_cache():
    """A 3B-shaped model cut to two layers, the KV cache pre-filled to 600 positions with fp16 N(0,1) (converted to
    the port's f32 rows), then 6 steps: logits within float rounding of the oracle's session."""
    cfg = moert.Config(**{**moert.GRANITE_3B, "layers": 2, "vocab": 512})
    m, s, p = _pair(cfg, 23, 0.02, 640)
    for l in range(cfg.layers):
        k, v = moert.kv_prefill_data(cfg, 23, l, 600)
        s.kv_prefill(l, k, v)
        p.kv_prefill(l, k, v)
    s.set_position(600)
    p.set_position(600)
    for t, tok in enumerate(np.random.default_rng(5).integers(0, cfg.vocab, 6)):
        olg, oids, _, _ = s.step(int(tok))
        plg, pids, _ = p.step(int(tok))
        assert np.array_equal(oids, pids), t
        scale = float(np.abs(olg).max())
        assert float(np.abs(plg - olg).max()) <= 2e-4 * scale + 1e-6, t
