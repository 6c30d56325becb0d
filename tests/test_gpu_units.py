"""Each kernel of the decode step, through the C ABI, against the oracle on the same inputs. The kernels follow the
oracle's evaluation order, so integer results and float results are compared bit for bit."""
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


def test_exp_is_bit_identical(gpu):
    say("exp")
    x = np.concatenate([np.linspace(-90, 90, 1_000_003, dtype=np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan], np.float32)])
    got = moert.exp_device(x)
    want = oracle.exp(x)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


@pytest.mark.parametrize("dtype", [moert.Q8_0, moert.Q4_0, moert.F32])
def test_dequantised_weights_are_bit_identical(gpu, dtype):
    say(f"dequant dtype={dtype}")
    rows, cols = 97, 1536
    w = moert.synth_quantized(61, dtype, rows * cols, 0.02, dtype)
    got = moert.dequant(w, dtype, rows, cols)
    want = oracle.dequant(w, dtype, rows * cols)
    assert bits_equal(got, want)


@pytest.mark.parametrize("dtype", [moert.Q8_0, moert.Q4_0, moert.F32])
@pytest.mark.parametrize("rows,cols", [(5, 128), (33, 256), (64, 512), (1000, 1024), (2563, 1536)])
def test_gemv_is_bit_identical(gpu, dtype, rows, cols):
    say(f"gemv dtype={dtype} {rows}x{cols}")
    w = moert.synth_quantized(62, rows, rows * cols, 0.02, dtype)
    x = moert.synth_normal(63, cols, cols)
    assert bits_equal(moert.gemv(w, dtype, rows, cols, x), oracle.gemv(w, dtype, rows, cols, x))


@pytest.mark.parametrize("n", [16, 256, 1024, 1536])
def test_rmsnorm_is_bit_identical(gpu, n):
    say(f"rmsnorm n={n}")
    x = moert.synth_normal(64, n, n, 2.0)
    w = moert.synth_normal(65, n, n, 0.02, 1.0)
    assert bits_equal(moert.rmsnorm(x, w, 1e-6), oracle.rmsnorm(x, w, 1e-6))


@pytest.mark.parametrize("pos", [0, 1, 7, 4095, 4351])
def test_rope_is_bit_identical(gpu, pos):
    say(f"rope pos={pos}")
    x = moert.synth_normal(66, pos, 24 * 64)
    got = moert.rope(x, 64, 10000.0, pos)
    want = oracle.rope(x, 64, oracle.rope_cos_sin(10000.0, 64, pos))
    assert bits_equal(got, want)


def test_router_topk_is_bit_identical_on_the_reference_golden_families(gpu):
    """route.rs:240-246 (ids and weights), here bit for bit against the oracle."""
    from test_oracle import lcg_cases
    say("router top-k families")
    for fam, e, v in lcg_cases(per_family=20):
        ids, w = moert.router_topk(v, 8)
        oi, ow = oracle.route(v, 8)
        assert ids.tolist() == oi.tolist(), (fam, e)
        assert bits_equal(w, ow), (fam, e)


def test_router_never_picks_a_padding_lane(gpu):
    """route.rs:260-269: with 40 experts in a 64-lane wave, all-negative logits must not pick lanes 40..63."""
    say("router padding")
    for c in (-1.0, -1.0e30, -3.0e38):
        v = np.full(40, c, np.float32)
        v[7] = c * 2 if c > -1e38 else c
        ids, w = moert.router_topk(v, 8)
        assert ids.max() < 40
        oi, ow = oracle.route(v, 8)
        assert ids.tolist() == oi.tolist() and bits_equal(w, ow)


def test_argmax_is_greedy_with_the_last_index_on_ties(gpu):
    say("argmax")
    rng = np.random.default_rng(7)
    for n in (1, 33, 49155, 1 << 20):
        v = rng.standard_normal(n).astype(np.float32)
        if n > 40:
            v[[5, n // 2, n - 3]] = v.max() + 1.0
        assert moert.argmax(v) == oracle.argmax(v), n
    assert moert.argmax(np.array([0.0, -0.0], np.float32)) == 0


def test_split_kv_attention_is_bit_identical_at_every_slice_and_block_boundary(gpu):
    """tests/model.rs:183-250 cases (splits of 4 tiles over 32, of 2 over 68, of 1 over 16; amplified scores),
    G=2 and G=3; plus splits whose tile count does not divide the cache (30 tiles by 4), and splits of 3 and 8 tiles,
    which take the sequential-tile kernel instead of the tile-parallel one."""
    b = 64
    configs = [(4, 2, 4, 32 * b, [1, 2, b - 1, b, b + 1, 8 * b, 8 * b + 1, 9 * b - 1, 3 * b + 7, 17 * b + 5, 32 * b - 1, 32 * b]),
               (24, 8, 2, 68 * b, [1, b + 1, 64 * b, 64 * b + 1, 67 * b + 9, 68 * b]),
               (4, 1, 1, 16 * b, [1, b, b + 1, 16 * b]),
               (8, 2, 4, 30 * b, [1, 5 * b + 3, 28 * b, 28 * b + 1, 29 * b + 7, 30 * b]),
               (6, 2, 3, 20 * b, [1, b + 1, 7 * b, 19 * b + 5, 20 * b]),
               (4, 4, 8, 40 * b, [1, 9 * b, 33 * b + 2, 40 * b])]
    for heads, kvh, ns, max_len, lens in configs:
        for amp in (False, True):
            q = moert.synth_normal(71, ns, heads * 64)
            kf = moert.synth_normal(72, ns, kvh * max_len * 64).reshape(kvh, max_len, 64)
            vf = moert.synth_normal(73, ns, kvh * max_len * 64)
            if amp:
                q = q * np.float32(4.0)
                mid = (max_len // 3 // b) * b
                kf[:, mid:mid + b] *= np.float32(4.0)
            kc, vc = oracle.f2h(kf.reshape(-1)), oracle.f2h(vf)
            for length in lens:
                say(f"attn heads={heads} kv={kvh} tiles/split={ns} len={length} amp={amp}")
                got = moert.attn_decode(q, kc, vc, heads, kvh, max_len, length, 0.125, ns)
                want = oracle.attention(q, kc, vc, heads, kvh, max_len, length, 0.125, ns)
                assert bits_equal(got, want), (heads, ns, length, amp)


def test_split_kv_attention_ignores_cache_rows_past_the_length(gpu):
    """Cache rows at and after the length hold fp16 NaN and infinity: no output may depend on them."""
    b = 64
    for heads, kvh, ns, max_len, length in [(24, 8, 2, 8 * b, 3 * b + 5), (4, 2, 4, 8 * b, 5 * b + 1),
                                            (8, 2, 4, 8 * b, 2 * b), (6, 2, 3, 8 * b, b + 9)]:
        q = moert.synth_normal(74, 1, heads * 64)
        kc = oracle.f2h(moert.synth_normal(75, 1, kvh * max_len * 64)).reshape(kvh, max_len, 64)
        vc = oracle.f2h(moert.synth_normal(76, 1, kvh * max_len * 64)).reshape(kvh, max_len, 64)
        kc[:, length:, ::2] = 0x7E00   # NaN
        kc[:, length:, 1::2] = 0x7C00  # +inf
        vc[:, length:, ::2] = 0xFC00   # -inf
        vc[:, length:, 1::2] = 0x7E00
        kc, vc = kc.reshape(-1), vc.reshape(-1)
        say(f"attn past-length poison heads={heads} kv={kvh} tiles/split={ns} len={length}")
        got = moert.attn_decode(q, kc, vc, heads, kvh, max_len, length, 0.125, ns)
        want = oracle.attention(q, kc, vc, heads, kvh, max_len, length, 0.125, ns)
        assert np.isfinite(got).all()
        assert bits_equal(got, want), (heads, ns, length)


@pytest.mark.parametrize("dtype", [moert.Q8_0, moert.Q4_0, moert.F32])
def test_moe_block_is_bit_identical(gpu, dtype):
    """The 1B MoE block (router 1024->32, top-8, experts 1024->512->1024) and a small one."""
    for hidden, inter, experts, k in [(256, 128, 6, 2), (1024, 512, 32, 8), (1536, 512, 40, 8)]:
        router = moert.synth_quantized(81, hidden, experts * hidden, 0.02, dtype)
        gate_up = moert.synth_quantized(82, hidden, experts * 2 * inter * hidden, 0.02, dtype)
        down = moert.synth_quantized(83, hidden, experts * hidden * inter, 0.02, dtype)
        blk = moert.GpuBlock(hidden, inter, experts, k, router, gate_up, down, dtype)
        for t in range(4):
            say(f"moe block dtype={dtype} hidden={hidden} t={t}")
            x = moert.synth_normal(84, t, hidden)
            y, ids, w = blk.forward(x)
            oy, oi, ow = oracle.moe_block(hidden, inter, experts, k, router, gate_up, down, dtype, x)
            assert ids.tolist() == oi.tolist()
            assert bits_equal(w, ow)
            assert bits_equal(y, oy)
        blk.close()
