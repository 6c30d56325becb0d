"""Pins the oracle (CPU restatement of the reference path) against the reference's own known answers and golden
cases, against transformers' GraniteMoeForCausalLM, and against closed forms and float64 mathematics. No GPU.

Each test names the reference test or formula it follows (paths relative to the reference root).
"""
import math
import os

import numpy as np
import pytest

import moert
import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---- exp ----------------------------------------------------------------------------------------------------------
def test_exp_is_within_two_ulp_of_float64_exp_over_the_softmax_range():
    x = np.concatenate([np.linspace(-86.5, 88.5, 2_000_001, dtype=np.float32),
                        np.float32(np.random.default_rng(1).standard_normal(200_000) * 10)])
    y = oracle.exp(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    err = np.abs(y - want) / ulp
    assert err.max() <= 2.0, f"max error {err.max():.2f} ulp at x={x[err.argmax()]}"


def test_exp_special_values():
    x = np.array([0.0, -0.0, -np.inf, np.inf, np.nan, -87.0, -1000.0, 89.5, 1000.0, 1.0], np.float32)
    y = oracle.exp(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[2] == 0.0 and y[5] == 0.0 and y[6] == 0.0
    assert np.isinf(y[3]) and np.isinf(y[7]) and np.isinf(y[8])
    assert np.isnan(y[4])
    assert abs(float(y[9]) - math.e) <= 2 * np.spacing(np.float32(math.e))


# ---- fp16 ---------------------------------------------------------------------------------------------------------
def test_fp16_decoding_matches_numpy_for_all_codes():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.h2f(h)
    want = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_fp16_rounding_matches_numpy_round_to_nearest_even():
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.standard_normal(300_000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 300_000),
        np.array([65504, 65519.99, 65520, 65536, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-9, 0.0, -0.0, np.inf, -np.inf],
                 np.float32),
        # exact ties of the 10-bit mantissa
        (np.arange(1, 2049, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
    ]).astype(np.float32)
    got = oracle.f2h(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---- quantised blocks ---------------------------------------------------------------------------------------------
def _q8_blocks(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    nb = scales.size
    out = np.zeros((nb, 34), np.uint8)
    out[:, 0:2] = scales.astype(np.float16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = codes.astype(np.int8).view(np.uint8).reshape(nb, 32)
    return out.reshape(-1)


def test_q8_0_dequant_is_code_times_fp16_scale_exactly_for_every_code():
    rng = np.random.default_rng(4)
    codes = np.tile(np.arange(-128, 128), 8).reshape(-1, 32)  # every int8 code
    scales = (rng.standard_normal(codes.shape[0]) * 0.01).astype(np.float16)
    blob = _q8_blocks(codes, scales)
    got = oracle.dequant(blob, moert.Q8_0, codes.size)
    want = (codes.astype(np.float64) * scales.astype(np.float64)[:, None]).reshape(-1)
    assert np.array_equal(got.astype(np.float64), want)  # q * d is exact in f32


def test_q4_0_dequant_is_nibble_minus_8_times_scale_exactly_for_every_code():
    rng = np.random.default_rng(5)
    nb = 64
    lo = rng.integers(0, 16, (nb, 16))
    hi = rng.integers(0, 16, (nb, 16))
    lo[0], hi[0] = np.arange(16), np.arange(16)[::-1]
    scales = (rng.standard_normal(nb) * 0.01).astype(np.float16)
    blob = np.zeros((nb, 18), np.uint8)
    blob[:, 0:2] = scales.view(np.uint8).reshape(nb, 2)
    blob[:, 2:] = (lo | (hi << 4)).astype(np.uint8)
    got = oracle.dequant(blob.reshape(-1), moert.Q4_0, nb * 32).reshape(nb, 32)
    d = scales.astype(np.float64)[:, None]
    assert np.array_equal(got[:, :16].astype(np.float64), (lo - 8) * d)
    assert np.array_equal(got[:, 16:].astype(np.float64), (hi - 8) * d)


# ---- dot / gemv ---------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [moert.F32, moert.Q8_0, moert.Q4_0])
def test_gemv_matches_float64_of_the_dequantised_weights(dtype):
    """tests/block.rs:26-48 (GEMV/dot against f64), on every row length the engine compiles."""
    for rows, cols in [(7, 128), (33, 256), (64, 512), (24, 1024), (40, 1536)]:
        w = moert.synth_quantized(11, rows, rows * cols, 0.02, dtype)
        x = moert.synth_normal(12, cols, cols)
        y = oracle.gemv(w, dtype, rows, cols, x, threads=3)
        wf = oracle.dequant(w, dtype, rows * cols).reshape(rows, cols).astype(np.float64)
        want = wf @ x.astype(np.float64)
        tol = 1e-5 * (1.0 + np.abs(wf) @ np.abs(x.astype(np.float64)))
        assert (np.abs(y - want) <= tol).all(), (rows, cols)


def test_gemv_result_does_not_depend_on_the_thread_count():
    w = moert.synth_quantized(13, 0, 300 * 1536, 0.02, moert.Q8_0)
    x = moert.synth_normal(14, 0, 1536)
    a = oracle.gemv(w, moert.Q8_0, 300, 1536, x, threads=1)
    b = oracle.gemv(w, moert.Q8_0, 300, 1536, x, threads=7)
    assert np.array_equal(a, b)


# ---- rmsnorm / rope / swiglu -----------------------------------------------------------------------------------------
def test_rmsnorm_known_answer():
    """tests/model.rs:50-54: rmsnorm([3, 4], [1, 2], 0) = [3/r, 8/r], r = sqrt(12.5)."""
    y = oracle.rmsnorm([3.0, 4.0], [1.0, 2.0], 0.0)
    r = math.sqrt(12.5)
    assert abs(y[0] - 3.0 / r) < 1e-6 and abs(y[1] - 8.0 / r) < 1e-6


def test_rmsnorm_matches_float64():
    x = moert.synth_normal(20, 0, 1536, 3.0)
    w = moert.synth_normal(20, 1, 1536, 0.02, 1.0)
    y = oracle.rmsnorm(x, w, 1e-6).astype(np.float64)
    x64 = x.astype(np.float64)
    want = w * x64 / np.sqrt((x64 * x64).mean() + 1e-6)
    assert np.abs(y - want).max() <= 1e-6 * np.abs(want).max()


def test_rope_position_zero_is_identity_and_matches_the_closed_form():
    """tests/model.rs:27-47."""
    d, theta = 64, 10000.0
    x = moert.synth_normal(21, 0, 2 * d)
    assert np.array_equal(oracle.rope(x, d, oracle.rope_cos_sin(theta, d, 0)), x)
    pos = 7
    y = oracle.rope(x, d, oracle.rope_cos_sin(theta, d, pos)).astype(np.float64)
    half = d // 2
    for head in range(2):
        for j in range(half):
            a = pos * (1.0 / theta ** (2 * j / d))
            x1, x2 = float(x[head * d + j]), float(x[head * d + j + half])
            assert abs(y[head * d + j] - (x1 * math.cos(a) - x2 * math.sin(a))) < 1e-5
            assert abs(y[head * d + j + half] - (x2 * math.cos(a) + x1 * math.sin(a))) < 1e-5


def test_swiglu_is_silu_of_the_first_half_times_the_second():
    """tests/block.rs:122-129."""
    a = oracle.swiglu([0.0, 1.0, -2.0, 3.0, 4.0, 5.0])
    silu = lambda g: g / (1.0 + math.exp(-g))
    for got, want in zip(a, [silu(0.0) * 3.0, silu(1.0) * 4.0, silu(-2.0) * 5.0]):
        assert abs(got - want) < 1e-6


# ---- router -------------------------------------------------------------------------------------------------------
def test_router_known_answer():
    """tests/block.rs:14-23: [0.5, 2, -1, 2, 1], k=3 -> [1, 3, 4], softmax over [2, 2, 1]."""
    ids, w = oracle.route([0.5, 2.0, -1.0, 2.0, 1.0], 3)
    assert ids.tolist() == [1, 3, 4]
    ex = np.exp([2.0, 2.0, 1.0])
    assert np.abs(w - ex / ex.sum()).max() < 1e-6
    assert abs(w.sum() - 1.0) < 1e-6


def lcg_cases(per_family=50):
    """The logit families of rust/moe-rt/src/route.rs:121-238 (seed 7, same LCG, same draw order including the
    1536 x values each case draws), at E=32 and E=40. Yields (family, E, logits)."""
    s = 7
    A, C, M = 6364136223846793005, 1442695040888963407, (1 << 64) - 1

    def lcg():
        nonlocal s
        s = (s * A + C) & M
        return np.float32(np.int32(np.uint32(s >> 32))) / np.float32(2 ** 31) * np.float32(8.0)

    fams = ["distinct", "ties", "negative", "spread", ("equal", -1.0e30), ("equal", -2.0e30), "two_max", "tie_at_cut"]
    for fam in fams:
        for e in (32, 40):
            for _ in range(per_family):
                v = np.array([lcg() for _ in range(e)], np.float32)
                if fam == "ties":
                    v = np.floor(v * np.float32(2.0)) / np.float32(2.0)
                elif fam == "negative":
                    v = v - np.float32(10.0)
                elif fam == "spread":
                    v = v * np.float32(12.0)
                elif isinstance(fam, tuple):
                    v[:] = np.float32(fam[1])
                elif fam == "two_max":
                    v = v - np.float32(20.0)
                    v[e - 1] = 5.0
                    v[3] = 5.0
                elif fam == "tie_at_cut":
                    v = v - np.float32(20.0)
                    for r, i in enumerate([0, 1, 2, 3, 4, 6, 7]):
                        v[i] = 10.0 - r
                    for i in (5, 9, 20):
                        v[i] = 1.0
                for _ in range(1536):
                    lcg()
                yield (fam if isinstance(fam, str) else f"equal{fam[1]:g}"), e, v.astype(np.float32)


TIE_FAMILIES = {"ties", "equal-1e+30", "equal-2e+30", "two_max", "tie_at_cut"}


def test_router_topk_matches_a_sort_on_the_reference_golden_families():
    """route.rs:240-246: ids equal to a descending sort with ties to the lower index; weights within 1e-6."""
    k = 8
    for fam, e, v in lcg_cases():
        ids, w = oracle.route(v, k)
        want = sorted(range(e), key=lambda i: (-float(v[i]), i))[:k]
        assert ids.tolist() == want, (fam, e)
        top = v[want].astype(np.float64)
        ex = np.exp(top - top[0])
        ww = ex / ex.sum()
        assert np.all(np.abs(w - ww) <= 1e-6 * np.maximum(np.abs(ww), 1e-3)), (fam, e)


def test_control_reversed_tie_break_differs_exactly_on_the_tie_families():
    """route.rs:248-258: the case set sees the tie-break; a higher-index-first sort differs only on tie families."""
    k, bad = 8, {}
    for fam, e, v in lcg_cases():
        ids, _ = oracle.route(v, k)
        rev = sorted(range(e), key=lambda i: (-float(v[i]), -i))[:k]
        bad[fam] = bad.get(fam, 0) + (ids.tolist() != rev)
    for fam, n in bad.items():
        assert (n > 0) == (fam in TIE_FAMILIES), (fam, n, bad)


def test_router_bias_is_added_before_the_top_k():
    logits = np.array([1.0, 0.5, 0.2, 0.1], np.float32)
    bias = np.array([-5.0, 0.0, 0.0, 1.0], np.float32)
    ids, w = oracle.route(logits, 2, bias)
    assert ids.tolist() == [3, 1]
    ex = np.exp([1.1 - 1.1, 0.5 - 1.1])
    assert np.abs(w - ex / ex.sum()).max() < 1e-6


def test_argmax_keeps_the_last_of_equal_maxima():
    """bin/m1b-gulosa.rs:22-24: max_by(total_cmp) returns the last maximum."""
    assert oracle.argmax([1.0, 3.0, 2.0, 3.0, -1.0]) == 3
    assert oracle.argmax([0.0, -0.0]) == 0  # total order: +0 > -0
    assert oracle.argmax([-np.inf, -1.0, -1.0]) == 2


# ---- attention ----------------------------------------------------------------------------------------------------
def _attn_f64(q, kc, vc, heads, kvh, max_len, length, scale):
    d = 64
    G = heads // kvh
    K = oracle.h2f(kc).reshape(kvh, max_len, d).astype(np.float64)
    V = oracle.h2f(vc).reshape(kvh, max_len, d).astype(np.float64)
    out = np.zeros(heads * d)
    for h in range(heads):
        g = h // G
        sc = K[g, :length] @ q[h * d:(h + 1) * d].astype(np.float64) * scale
        p = np.exp(sc - sc.max())
        out[h * d:(h + 1) * d] = (p @ V[g, :length]) / p.sum()
    return out


def test_split_kv_attention_matches_float64_at_every_slice_and_block_boundary():
    """tests/model.rs:183-250: lengths at tile and split boundaries (splits of 4 tiles over a 32-tile cache, of 2
    tiles over 128, of 1 and 3 tiles), with amplified scores (q x4, a middle tile x4); positions past len hold finite
    garbage that must stay masked."""
    heads, kvh, b, scale = 4, 2, 64, 0.125
    configs = [(4, 32 * b, [1, 2, b - 1, b, b + 1, 8 * b, 8 * b + 1, 9 * b - 1, 3 * b + 7, 17 * b + 5, 32 * b - 1, 32 * b]),
               (2, 128 * b, [1, b + 1, 64 * b, 64 * b + 1, 67 * b + 9, 128 * b]),
               (1, 16 * b, [1, b, b + 1, 16 * b]),
               (3, 24 * b, [1, 3 * b, 3 * b + 1, 10 * b + 7, 24 * b])]
    for ns, max_len, lens in configs:
        for amp in (False, True):
            q = moert.synth_normal(31, ns, heads * 64)
            kf = moert.synth_normal(32, ns, kvh * max_len * 64)
            vf = moert.synth_normal(33, ns, kvh * max_len * 64)
            if amp:
                q = q * np.float32(4.0)
                mid = (max_len // 3 // b) * b
                kf = kf.reshape(kvh, max_len, 64)
                kf[:, mid:mid + b] *= np.float32(4.0)
                kf = kf.reshape(-1)
            kc, vc = oracle.f2h(kf), oracle.f2h(vf)
            for length in lens:
                got = oracle.attention(q, kc, vc, heads, kvh, max_len, length, scale, ns)
                want = _attn_f64(q, kc, vc, heads, kvh, max_len, length, scale)
                err = np.abs(got - want).max()
                assert err < 1e-5, (ns, max_len, amp, length, err)


# ---- MoE block ----------------------------------------------------------------------------------------------------
def _block_f64(hidden, inter, experts, k, router, gate_up, down, dtype, x):
    f = lambda a, r, c: oracle.dequant(a, dtype, r * c).reshape(r, c).astype(np.float64)
    rl = f(router, experts, hidden) @ x.astype(np.float64)
    ids, w = oracle.route(rl.astype(np.float32), k)
    gu = f(gate_up, experts * 2 * inter, hidden).reshape(experts, 2 * inter, hidden)
    dn = f(down, experts * hidden, inter).reshape(experts, hidden, inter)
    y = np.zeros(hidden)
    for e, we in zip(ids, w):
        hh = gu[e] @ x
        g, u = hh[:inter], hh[inter:]
        y += float(we) * (dn[e] @ (g / (1.0 + np.exp(-g)) * u))
    return y, ids


@pytest.mark.parametrize("dtype", [moert.F32, moert.Q8_0, moert.Q4_0])
def test_moe_block_matches_a_naive_float64_block(dtype):
    """tests/block.rs:204-239 (rel-L2 < 1e-5, same experts), at the 1B block shape and a small one."""
    for hidden, inter, experts, k in [(256, 128, 6, 2), (1024, 512, 32, 8)]:
        router = moert.synth_quantized(41, hidden, experts * hidden, 0.02, dtype)
        gate_up = moert.synth_quantized(42, hidden, experts * 2 * inter * hidden, 0.02, dtype)
        down = moert.synth_quantized(43, hidden, experts * hidden * inter, 0.02, dtype)
        for t in range(3):
            x = moert.synth_normal(44, t, hidden)
            y, ids, w = oracle.moe_block(hidden, inter, experts, k, router, gate_up, down, dtype, x, threads=3)
            want, wids = _block_f64(hidden, inter, experts, k, router, gate_up, down, dtype, x)
            assert ids.tolist() == wids.tolist()
            rel = np.linalg.norm(y - want) / np.linalg.norm(want)
            assert rel < 1e-5, (hidden, t, rel)


def test_batched_experts_step_matches_the_per_position_path():
    """cpu.rs:314-363: experts_step over m positions equals per-position experts within 1e-5 of the max norm."""
    hidden, inter, experts, k = 256, 128, 8, 2
    gate_up = moert.synth_quantized(51, 0, experts * 2 * inter * hidden, 0.02, moert.Q8_0)
    down = moert.synth_quantized(52, 0, experts * hidden * inter, 0.02, moert.Q8_0)
    router = moert.synth_quantized(53, 0, experts * hidden, 0.02, moert.Q8_0)
    for m in (1, 2, 4, 8):
        x = moert.synth_normal(54, m, m * hidden).reshape(m, hidden)
        ids = np.zeros((m, k), np.int32)
        ws = np.zeros((m, k), np.float32)
        per = np.zeros((m, hidden), np.float32)
        for p in range(m):
            per[p], ids[p], ws[p] = oracle.moe_block(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, x[p])
        got = oracle.experts_step(hidden, inter, m, k, gate_up, down, moert.Q8_0, x, ids, ws)
        assert np.abs(got - per).max() <= 1e-5 * np.abs(per).max(), m


# ---- grouped (multi-position) integer path ---------------------------------------------------------------------------
def test_hilo_codes_reconstruct_every_block_within_half_a_step():
    """v = 256*hi + lo with lo in [-128, 127], |x - v*d| <= d/2 (plus the f32 rounding of x/d, below 32639 * 2^-24)
    and the block maximum at +-32639; zero blocks give d = 0 and zero codes."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(32 * 400) * np.exp(rng.uniform(-20, 8, 32 * 400))).astype(np.float32)
    x[:32] = 0.0
    x[64:96] = np.float32(-3.5)
    hi, lo, d = oracle.quant_hilo(x)
    v = 256 * hi.astype(np.int64) + lo.astype(np.int64)
    assert lo.min() >= -128 and lo.max() <= 127 and np.abs(hi).max() <= 127
    blk = x.reshape(-1, 32).astype(np.float64)
    assert d[0] == 0.0 and not v[:32].any()
    rec = v.reshape(-1, 32) * d[:, None].astype(np.float64)
    assert np.all(np.abs(rec - blk) <= (0.5 + 2.0 ** -8) * d[:, None])
    amax_idx = np.abs(blk).argmax(axis=1)
    nz = d > 0
    assert np.all(np.abs(v.reshape(-1, 32)[np.arange(len(d)), amax_idx][nz]) == 32639)
    assert np.all(v[64:96] == -32639)


@pytest.mark.parametrize("dtype", [moert.Q8_0, moert.Q4_0])
def test_integer_block_dot_equals_the_float64_dot_of_the_codes(dtype):
    """The hi/lo block product is exact: the result equals float64 sum_b dw_b*dx_b*(q . v)_b up to the f32
    accumulation, and differs from the dot with the unrounded x by at most sum |w| * d / 2."""
    cols = 1536
    w = moert.synth_quantized(71, dtype, 6 * cols, 0.02, dtype)
    deq = oracle.dequant(w, dtype, 6 * cols).reshape(6, cols).astype(np.float64)
    for t in range(4):
        x = moert.synth_normal(72, t, cols, 1.0 + 10 * t)
        hi, lo, d = oracle.quant_hilo(x)
        xq = ((256 * hi.astype(np.float64) + lo) .reshape(-1, 32) * d[:, None]).reshape(-1)
        for r in range(6):
            got = oracle.dot_hilo(w, dtype, cols, r, hi, lo, d)
            exact = float(deq[r] @ xq)
            scale = float(np.abs(deq[r]) @ np.abs(xq))
            assert abs(got - exact) <= 48 * 2 ** -23 * scale, (t, r, got, exact)
            bound = float(np.abs(deq[r]).reshape(-1, 32).sum(axis=1) @ d) / 2
            assert abs(got - float(deq[r] @ x.astype(np.float64))) <= bound + 48 * 2 ** -23 * scale


def test_grouped_experts_step_agrees_with_the_f32_path():
    """orc_experts_grouped (integer block products of 15-bit activation codes) against Cpu::experts_step in f32
    (cpu.rs:239-296): the 3B expert shape, 16 positions with Zipf-skewed routing; rel-L2 per position < 2e-4."""
    hidden, inter, experts, k, m = 1536, 512, 40, 8, 16
    router = moert.synth_quantized(81, 0, experts * hidden, 0.02, moert.Q8_0)
    gate_up = moert.synth_quantized(82, 0, experts * 2 * inter * hidden, 0.02, moert.Q8_0)
    down = moert.synth_quantized(83, 0, experts * hidden * inter, 0.02, moert.Q8_0)
    bias = moert.zipf_bias(experts, 5)
    x = moert.synth_normal(84, 0, m * hidden).reshape(m, hidden)
    y, ids, w = oracle.moe_block_batched(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, x, bias=bias)
    ref = oracle.experts_step(hidden, inter, m, k, gate_up, down, moert.Q8_0, x, ids, w)
    rel = np.linalg.norm(y - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert rel.max() < 2e-4, rel
    assert len(np.unique(ids)) < experts  # the skew leaves some experts unused


def test_batched_block_routes_every_position_like_the_single_position_block():
    """Per-position router + top-k of the batched block equals HostLayer::forward_cpu's (block.rs:56-62), bit for
    bit, with and without the router bias."""
    hidden, inter, experts, k, m = 1024, 128, 32, 8, 9
    router = moert.synth_quantized(91, 0, experts * hidden, 0.02, moert.Q8_0)
    gate_up = moert.synth_quantized(92, 0, experts * 2 * inter * hidden, 0.02, moert.Q8_0)
    down = moert.synth_quantized(93, 0, experts * hidden * inter, 0.02, moert.Q8_0)
    x = moert.synth_normal(94, 0, m * hidden).reshape(m, hidden)
    for bias in (None, moert.zipf_bias(experts, 3)):
        _, ids, w = oracle.moe_block_batched(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, x, bias=bias)
        for p in range(m):
            _, i1, w1 = oracle.moe_block(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, x[p], bias=bias)
            assert ids[p].tolist() == i1.tolist()
            assert np.array_equal(w[p].view(np.uint32), w1.view(np.uint32))


# ---- MoE-half norm + router from 8-row partials ----------------------------------------------------------------------
def test_moe_norm_route_known_answer():
    """h = [3, 4, 0, ...] (H = 16), norm weights 1, eps 0: ss = 25, r = 1/sqrt(25/16) = 0.8, xn = [2.4, 3.2, 0...];
    router rows all ones and alternating +1/-1 give z = [7, -1] and logits [5.6, -0.8]; a bias is added after."""
    h = np.zeros(16, np.float32)
    h[:2] = [3, 4]
    w = np.ones((2, 16), np.float32)
    w[1, 1::2] = -1
    xn, lg = oracle.moe_norm_route(h, np.ones(16, np.float32), w.ravel(), moert.F32, 2, 0.0)
    assert np.allclose(xn[:2], [2.4, 3.2], rtol=1e-6) and not xn[2:].any()
    assert np.allclose(lg, [5.6, -0.8], rtol=1e-6)
    _, lb = oracle.moe_norm_route(h, np.ones(16, np.float32), w.ravel(), moert.F32, 2, 0.0, bias=np.array([1, 2], np.float32))
    assert np.allclose(lb, [6.6, 1.2], rtol=1e-6)


@pytest.mark.parametrize("dtype", [moert.Q8_0, moert.Q4_0, moert.F32])
@pytest.mark.parametrize("H,E", [(1536, 40), (1024, 32), (256, 4), (512, 64)])
def test_moe_norm_route_matches_float64_and_its_own_block_order(dtype, H, E):
    """Against float64 rmsnorm + router over the dequantised weights (xn within 1e-6, logits within 1e-5 of the
    largest); against a direct numpy restatement of the block order (per 8-row block fma chains, blocks summed per
    lane b % 64, pairwise lane tree) bit for bit; and not the unblocked order (canonical rmsnorm, then dot): the two
    must differ on some logit, so the block order is what is pinned."""
    rng = np.random.default_rng(H + E + dtype)
    h = rng.normal(size=H).astype(np.float32) * 3
    lnw = (1 + 0.1 * rng.normal(size=H)).astype(np.float32)
    w = moert.quantize(rng.normal(size=E * H).astype(np.float32) * 0.02, dtype) if dtype != moert.F32 else \
        (rng.normal(size=E * H).astype(np.float32) * 0.02)
    bias = rng.normal(size=E).astype(np.float32)
    xn, lg = oracle.moe_norm_route(h, lnw, w, dtype, E, 1e-6, bias=bias)
    wd = oracle.dequant(w, dtype, E * H).reshape(E, H).astype(np.float64)
    h64 = h.astype(np.float64)
    xn64 = lnw * h64 / np.sqrt((h64 * h64).mean() + 1e-6)
    assert np.abs(xn - xn64).max() <= 1e-6 * np.abs(xn64).max()
    lg64 = wd @ xn64 + bias
    assert np.abs(lg - lg64).max() <= 1e-5 * np.abs(lg64).max()
    # numpy restatement with float32 rounding at every step (np.float32 arithmetic; fma emulated in float64, exact
    # for one product + one addend then rounded once)
    def fma(a, b, c):
        return np.float32(np.float64(a) * np.float64(b) + np.float64(c))
    def reduce(parts):
        acc = [np.float32(0)] * 64
        for b, v in enumerate(parts):
            acc[b % 64] = np.float32(acc[b % 64] + v)
        s = 1
        while s < 64:
            for l in range(0, 64, 2 * s):
                acc[l] = np.float32(acc[l] + acc[l + s])
            s *= 2
        return acc[0]
    nb = H // 8
    ssp = []
    for b in range(nb):
        a = np.float32(0)
        for t in range(8):
            a = fma(h[8 * b + t], h[8 * b + t], a)
        ssp.append(a)
    r = np.float32(1) / np.sqrt(np.float32(reduce(ssp) / np.float32(H) + np.float32(1e-6)), dtype=np.float32)
    wf = wd.astype(np.float32)
    for e in range(0, E, max(1, E // 4)):
        zp = []
        for b in range(nb):
            a = np.float32(0)
            for t in range(8):
                a = fma(wf[e, 8 * b + t], np.float32(lnw[8 * b + t] * h[8 * b + t]), a)
            zp.append(a)
        want = np.float32(np.float32(reduce(zp) * r) + bias[e])
        assert np.float32(lg[e]).view(np.uint32) == want.view(np.uint32), e
    old = oracle.gemv(w, dtype, E, H, oracle.rmsnorm(h, lnw, 1e-6)) + bias
    assert not np.array_equal(old.view(np.uint32), lg.view(np.uint32))


# ---- expert cache (LRU) -----------------------------------------------------------------------------------------------
def test_lru_known_answers():
    """Hand-worked traces of the LruSync rule (tests/model.rs:380-412): a 2-slot cache over 4 tokens; the pin rule
    (a hit that comes after a miss in top-k order is still protected: without it the answer would be 0 hits,
    4 copies); and a cache smaller than k, whose extra miss goes to the CPU."""
    trace = [[[0, 1]], [[2, 0]], [[1, 2]], [[0, 3]]]
    assert oracle.lru_replay(np.array(trace), 4, 2) == (2, 6, 0)
    pin = [[[0, 1]], [[2, 0]]]
    assert oracle.lru_replay(np.array(pin), 3, 2) == (1, 3, 0)
    small = [[[0, 1, 2]]]
    assert oracle.lru_replay(np.array(small), 4, 2) == (0, 2, 1)
    for t in (trace, pin, small):
        assert oracle.lru_reference(t, 4, 2) == oracle.lru_replay(np.array(t), 4, 2)


def test_lru_table_replay_equals_the_list_statement_and_keeps_its_invariants():
    """The C replay (slot tables) against the list-scan statement on random and skewed traces, plus invariants:
    every request is a hit, a copy or a CPU miss; a cache holding every key copies each key exactly once."""
    rng = np.random.default_rng(21)
    for trial in range(40):
        layers, experts = int(rng.integers(1, 5)), int(rng.integers(3, 12))
        k = int(rng.integers(1, min(experts, 4) + 1))
        steps = int(rng.integers(1, 30))
        p = rng.zipf(1.3, size=experts).astype(np.float64) if trial % 2 else np.ones(experts)
        p = p / p.sum()
        routes = np.stack([np.stack([rng.choice(experts, size=k, replace=False, p=p) for _ in range(layers)])
                           for _ in range(steps)]).astype(np.int32)
        for cap in sorted({1, k, k + 1, layers * experts // 2 + 1, layers * experts}):
            got = oracle.lru_replay(routes, experts, cap)
            assert got == oracle.lru_reference(routes.tolist(), experts, cap), (trial, cap)
            assert sum(got) == steps * layers * k
            if cap >= layers * experts:
                distinct = len({(l, int(e)) for st in routes for l, ch in enumerate(st) for e in ch})
                assert got[1] == distinct and got[2] == 0
            if cap >= k:
                assert got[2] == 0


def _random_ops(rng, layers, experts, k, n):
    ops = []
    for _ in range(n):
        r = rng.random()
        if r < 0.08:
            ops.append(("fill", layers * experts))
        elif r < 0.25:
            l = int(rng.integers(0, layers))
            ops.append(("prefetch", l, rng.choice(experts, size=int(rng.integers(1, k + 1)), replace=False).tolist()))
        else:
            for l in range(layers):
                ops.append(("step", l, rng.choice(experts, size=k, replace=False).tolist()))
    return ops


def _run_lru(ops, layers, experts, cap):
    c = oracle.Lru(layers, experts, cap)
    copied = []
    for op in ops:
        if op[0] == "fill":
            copied.append(c.fill())
        elif op[0] == "prefetch":
            copied.append(c.prefetch(op[1], op[2]))
        else:
            lib = oracle.lib()
            a = np.ascontiguousarray(op[2], np.int32)
            lib.orc_lru_step_layer(c.h, op[1], a.ctypes.data_as(oracle.ctypes.c_void_p), a.size)
    return c.stats(), copied, c.slot_keys()


def test_lru_state_machine_with_fills_and_prefetches_equals_the_list_statement():
    """The slot-table state machine (decode steps, prefetch ticks, fills) against the list-scan statement on random
    traces: equal counters after every trace, prefetch and fill copies uncounted. A fill stamps the current clock
    (copy_on_compute, cache/core.rs:366-377): the mutant that stamps 0 must give different counters on some of them,
    so the traces do tell the two rules apart."""
    rng = np.random.default_rng(33)
    differs = 0
    for trial in range(60):
        layers, experts = int(rng.integers(1, 4)), int(rng.integers(3, 10))
        k = int(rng.integers(1, min(experts, 4) + 1))
        ops = _random_ops(rng, layers, experts, k, int(rng.integers(3, 25)))
        for cap in sorted({k, k + 1, layers * experts // 2 + 1, layers * experts}):
            got, _, _ = _run_lru(ops, layers, experts, cap)
            assert got == oracle.lru_reference_ops(ops, experts, cap), (trial, cap)
            differs += got != oracle.lru_reference_ops(ops, experts, cap, fill_stamp_clock=False)
            assert got[2] == 0
    assert differs > 0


def test_lru_fill_known_answer_and_replay_equivalence():
    """A fill after one step of a 3-key pool over 2 layers x 2 experts: step [0] at layer 0 and [1] at layer 1 fill
    slots 0, 1; the fill puts key 1 (layer 0, expert 1) into slot 2 with the current clock (2). The next step asks
    for layer 0 expert 0 (hit, tick 3) and layer 1 expert 0 (miss, tick 4): slots 1 and 2 were both last used at 2,
    so the victim is the lower index, slot 1. (Stamping the fill with 0 would evict the filled slot 2 instead.) The
    replay of steps alone equals the state machine."""
    c = oracle.Lru(2, 2, 3)
    c.step([[0], [1]])
    assert c.fill() == 1
    assert c.slot_keys().tolist() == [0, 3, 1]
    c.step([[0], [0]])
    assert c.stats() == (1, 3, 0)
    assert c.slot_keys().tolist() == [0, 2, 1]
    ops = [("step", 0, [0]), ("step", 1, [1]), ("fill", 4), ("step", 0, [0]), ("step", 1, [0]), ("step", 0, [1])]
    assert oracle.lru_reference_ops(ops, 2, 3) == (2, 3, 0)
    assert oracle.lru_reference_ops(ops, 2, 3, fill_stamp_clock=False) == (1, 4, 0)
    rng = np.random.default_rng(4)
    routes = rng.integers(0, 6, size=(20, 3, 1)).astype(np.int32)
    d = oracle.Lru(3, 6, 5)
    for st in routes:
        d.step(st)
    assert d.stats() == oracle.lru_replay(routes, 6, 5)


# ---- whole model ----------------------------------------------------------------------------------------------------
def _granite_golden():
    import make_granite_golden as g
    z = np.load(os.path.join(GOLDEN, "granite_tiny.npz"))
    cfg = moert.Config(**g.CFG)
    m = moert.SynthModel(cfg, seed=int(z["seed"]), wdtype=moert.F32, embed_dtype=moert.F32, std=float(z["std"]))
    return z, cfg, m


def test_decode_step_matches_transformers_granitemoe():
    """The oracle's CpuSession against transformers' GraniteMoeForCausalLM (float32, teacher forcing, the reference's
    synthetic test shapes): logits within 3e-3 of the max logit against the plain float32 model (the oracle keeps K and V
    in fp16, as the engine's cache stores them, and transformers' float32 CPU path itself sits ~1e-4 from float64);
    within 3e-4 against the variant of the golden run with K and V rounded to fp16; and the same top-k experts wherever
    transformers' k-th and (k+1)-th router logits are not within 1e-4."""
    z, cfg, m = _granite_golden()
    s = oracle.CpuSession(m, 128, attn_splits=8, threads=3)
    for t, tok in enumerate(z["tokens"]):
        lg, ids, w, _ = s.step(int(tok))
        for key, tol in (("logits", 3e-3), ("logits_fp16kv", 3e-4)):
            ref = z[key][t]
            assert np.abs(lg - ref).max() <= tol * np.abs(ref).max(), (key, t)
        for l in range(cfg.layers):
            rl = z["router_logits_fp16kv"][l, t]
            srt = np.sort(rl)[::-1]
            if srt[cfg.top_k - 1] - srt[cfg.top_k] > 1e-4:
                want = np.argsort(-rl, kind="stable")[:cfg.top_k]
                assert ids[l].tolist() == want.tolist(), (t, l)


def test_session_reset_reuses_the_cache_without_leaking_old_positions():
    """tests/model.rs:272-281: after going back to position 0 the same tokens give the same logits."""
    _, cfg, m = _granite_golden()
    s = oracle.CpuSession(m, 128, attn_splits=8, threads=2)
    first = [s.step(t)[0] for t in (3, 5, 7, 11)]
    s.set_position(0)
    again = [s.step(t)[0] for t in (3, 5, 7)]
    for a, b in zip(first, again):
        assert np.array_equal(a, b)


def test_session_refuses_a_full_cache_and_an_out_of_vocabulary_token():
    _, cfg, m = _granite_golden()
    s = oracle.CpuSession(m, 64, attn_splits=1, threads=1)
    with pytest.raises(RuntimeError):
        s.step(cfg.vocab)
    s.set_position(64)
    with pytest.raises(RuntimeError):
        s.step(1)
