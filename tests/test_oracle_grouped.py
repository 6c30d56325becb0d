"""Pins of the oracle's grouped-mode step (orc_session_step_grouped: the engine's moert_batched_mode(1), every weight
GEMM over 15-bit activation codes), on the CPU:
  - the four-quarter integer block dot equals the float64 dot of the codes up to its f32 accumulation;
  - the norms in the engine's 256- and 1024-thread orders equal the float64 rmsnorm up to f32 rounding;
  - whole steps stay within 2e-4 rel-L2 of the f32 session (the decode order) on the same positions: logits, hidden
    state and the KV rows they append, with the same routed experts; a planted mistake in that comparison's reference
    (RoPE's sine sign flipped, or the output projection's residual dropped) moves the difference far past the bound.
"""
import numpy as np
import pytest

import moert
import oracle


@pytest.mark.parametrize("dtype", [moert.Q8_0, moert.Q4_0])
@pytest.mark.parametrize("cols", [1024, 1536])
def test_quarter_block_dot_equals_the_float64_dot_of_the_codes(dtype, cols):
    """Each quarter is an f32 fmaf chain over its blocks and the quarters are added in order, so the result is within
    (blocks + 3) f32 roundings of sum_b dw_b * dx_b * S_b in float64; it can differ from the one-chain dot (the expert
    kernels' order) in the last bits only."""
    w = moert.synth_quantized(171, dtype, 6 * cols, 0.02, dtype)
    deq = oracle.dequant(w, dtype, 6 * cols).reshape(6, cols).astype(np.float64)
    differs = 0
    for t in range(4):
        x = moert.synth_normal(172, t, cols, 1.0 + 10 * t)
        hi, lo, d = oracle.quant_hilo(x)
        xq = ((256 * hi.astype(np.float64) + lo).reshape(-1, 32) * d[:, None]).reshape(-1)
        for r in range(6):
            got = oracle.dot_hilo_quarters(w, dtype, cols, r, hi, lo, d)
            exact = float(deq[r] @ xq)
            scale = float(np.abs(deq[r]) @ np.abs(xq))
            assert abs(got - exact) <= (cols // 32 + 3) * 2 ** -23 * scale, (t, r, got, exact)
            one = oracle.dot_hilo(w, dtype, cols, r, hi, lo, d)
            assert abs(got - one) <= (cols // 32 + 3) * 2 ** -23 * scale
            differs += got != one
    assert differs > 0  # the quarter order is a different order


def test_quarter_dot_uses_every_block_once():
    """A row of zeros but one block (in each quarter in turn) gives exactly that block's product: no block is
    dropped or counted twice, whichever quarter holds it."""
    cols = 1536
    x = moert.synth_normal(174, 0, cols)
    hi, lo, d = oracle.quant_hilo(x)
    base = moert.quantize(np.zeros(cols, np.float32), moert.Q8_0)
    for b in (0, 11, 12, 23, 24, 35, 36, 47):
        row = np.zeros(cols, np.float32)
        row[32 * b: 32 * b + 32] = np.linspace(-1, 1, 32, dtype=np.float32)
        w = moert.quantize(row, moert.Q8_0)
        deq = oracle.dequant(w, moert.Q8_0, cols).astype(np.float64)
        xq = ((256 * hi.astype(np.float64) + lo).reshape(-1, 32) * d[:, None]).reshape(-1)
        got = oracle.dot_hilo_quarters(w, moert.Q8_0, cols, 0, hi, lo, d)
        want = float(deq @ xq)
        assert abs(got - want) <= 2 ** -22 * abs(want), b
    assert oracle.dot_hilo_quarters(base, moert.Q8_0, cols, 0, hi, lo, d) == 0.0


@pytest.mark.parametrize("threads", [256, 1024])
@pytest.mark.parametrize("H", [1024, 1536])
def test_thread_order_norms_equal_the_float64_rmsnorm(threads, H):
    rng = np.random.default_rng(H + threads)
    for scale in (1e-3, 1.0, 300.0):
        h = (rng.standard_normal(H) * scale).astype(np.float32)
        lnw = (1 + 0.02 * rng.standard_normal(H)).astype(np.float32)
        got = oracle.rmsnorm_threads(h, lnw, 1e-6, threads)
        h64 = h.astype(np.float64)
        want = lnw * (h64 / np.sqrt(np.mean(h64 * h64) + 1e-6))
        assert np.allclose(got, want, rtol=4e-6, atol=1e-30)
    # the known answer of tests/model.rs:50-54 padded with zeros: [3, 4, 0, ...], w = [1, 2, 1, ...], eps 0
    h = np.zeros(H, np.float32)
    h[:2] = [3.0, 4.0]
    lnw = np.ones(H, np.float32)
    lnw[1] = 2.0
    got = oracle.rmsnorm_threads(h, lnw, 0.0, threads)
    r = np.sqrt(25.0 / H)
    assert abs(got[0] - 3.0 / r) < 1e-5 and abs(got[1] - 8.0 / r) < 1e-5 and not got[2:].any()


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(np.asarray(b, np.float64)))


def _pair(cfg, seed, std, max_len):
    m = moert.SynthModel(cfg, seed=seed, wdtype=moert.Q8_0, embed_dtype=moert.Q8_0, std=std, zipf_s=1.1)
    return m, oracle.CpuSession(m, max_len, attn_splits=8, threads=4), oracle.CpuSession(m, max_len, attn_splits=8,
                                                                                         threads=4)


@pytest.mark.parametrize("shape", ["1b", "3b"])
def test_grouped_step_agrees_with_the_f32_session(shape):
    """Granite shapes cut to 3 layers and a 512-token vocabulary: blocks of 32, 5 and 17 positions through the
    grouped step against the same positions decoded one at a time by the f32 session: the last logits and hidden
    state within 2e-4 rel-L2, every appended KV row within fp16 rounding of the codes' difference, and the same
    routed experts with the same weights at every position and layer (two of near-equal weight may trade ranks)."""
    base = moert.GRANITE_1B if shape == "1b" else moert.GRANITE_3B
    cfg = moert.Config(**{**base, "layers": 3, "vocab": 512})
    m, g, f = _pair(cfg, 61, 0.05, 128)
    rng = np.random.default_rng(62)
    pos, swaps, entries = 0, 0, 0
    for n in (32, 5, 17):
        toks = rng.integers(0, cfg.vocab, n)
        lg, ids, w, hid = g.step_grouped(toks)
        for j, t in enumerate(toks):
            flg, fids, fw, fhid = f.step(int(t))
            for l in range(cfg.layers):
                entries += 1
                # two experts of near-equal weight may trade ranks under the different rounding; the routed set and
                # every expert's weight stay the same
                if not np.array_equal(ids[j, l], fids[l]):
                    swaps += 1
                assert sorted(ids[j, l]) == sorted(fids[l]), (n, j, l)
                got = dict(zip(ids[j, l].tolist(), w[j, l].tolist()))
                want = dict(zip(fids[l].tolist(), fw[l].tolist()))
                assert max(abs(got[e] - want[e]) for e in want) < 1e-3, (n, j, l)
        assert _rel(lg, flg) < 2e-4 and _rel(hid, fhid) < 2e-4, (n, _rel(lg, flg), _rel(hid, fhid))
        pos += n
    assert swaps <= 0.05 * entries, (swaps, entries)
    for l in range(cfg.layers):
        gk, gv = g.read_kv(l, pos)
        fk, fv = f.read_kv(l, pos)
        for a, b in ((gk, fk), (gv, fv)):
            a = a.view(np.float16).astype(np.float64)
            b = b.view(np.float16).astype(np.float64)
            assert _rel(a, b) < 1e-3, l


def test_grouped_step_bound_catches_planted_mistakes():
    """The 2e-4 bound above is tight enough to notice the mistakes a restatement could make: the grouped step of a
    3-layer 1B-shaped model against an f32 reference computed with RoPE's sine sign flipped, or with the attention
    half's residual dropped, differs by far more than 2e-4 rel-L2 (the mistakes are planted in a float64 numpy
    reference of the first layer's attention half, on the CPU)."""
    cfg = moert.Config(**{**moert.GRANITE_1B, "layers": 1, "vocab": 512})
    m = moert.SynthModel(cfg, seed=63, wdtype=moert.Q8_0, embed_dtype=moert.Q8_0, std=0.05)
    g = oracle.CpuSession(m, 64, attn_splits=8, threads=4)
    toks = np.array([5, 9, 200, 31], np.int32)
    _, _, _, hid = g.step_grouped(toks)
    want = _np_layer0_hidden(m, toks, sign=1.0, residual=True)
    assert _rel(hid, want) < 2e-4
    assert _rel(hid, _np_layer0_hidden(m, toks, sign=-1.0, residual=True)) > 1e-2
    assert _rel(hid, _np_layer0_hidden(m, toks, sign=1.0, residual=False)) > 1e-2


def _np_layer0_hidden(m, toks, sign, residual):
    """float64 numpy restatement of a one-layer model's last hidden state (model.rs:181-243), with the planted
    mistakes as options: `sign` multiplies RoPE's sine terms, `residual` False drops h from the attention half's
    residual."""
    c = m.cfg
    H, d, nh, nkv, I, E = c.hidden, c.head_dim, c.heads, c.kv_heads, c.inter, c.experts
    a = m.arrays

    def mat(name, rows, cols):
        return oracle.dequant(a[name], m.wdtype, rows * cols).reshape(rows, cols).astype(np.float64)

    W = {"ln_attn": a["0.ln_attn"].astype(np.float64), "ln_moe": a["0.ln_moe"].astype(np.float64),
         "q": mat("0.q", nh * d, H), "k": mat("0.k", nkv * d, H), "v": mat("0.v", nkv * d, H),
         "o": mat("0.o", H, nh * d), "router": mat("0.router", E, H),
         "gate_up": mat("0.gate_up", E * 2 * I, H).reshape(E, 2 * I, H),
         "down": mat("0.down", E * H, I).reshape(E, H, I)}
    emb = oracle.dequant(a["embed"], m.embed_dtype, c.vocab * H).reshape(c.vocab, H).astype(np.float64)

    def norm(x, w):
        return w * (x / np.sqrt(np.mean(x * x) + c.eps))

    def rope(v, pos):
        inv = (1.0 / (c.rope_theta ** (np.arange(0, d, 2, dtype=np.float64) / d)))
        cs, sn = np.cos(pos * inv), sign * np.sin(pos * inv)
        v = v.reshape(-1, d).copy()
        x1, x2 = v[:, : d // 2].copy(), v[:, d // 2:].copy()
        v[:, : d // 2] = x1 * cs - x2 * sn
        v[:, d // 2:] = x2 * cs + x1 * sn
        return v.reshape(-1)

    ks, vs, h = [], [], None
    for pos, t in enumerate(toks):
        h = emb[t] * c.embedding_multiplier
        xn = norm(h, W["ln_attn"])
        q, k, v = rope(W["q"] @ xn, pos), rope(W["k"] @ xn, pos), W["v"] @ xn
        ks.append(k.reshape(nkv, d))
        vs.append(v.reshape(nkv, d))
        att = np.zeros(nh * d)
        for hq in range(nh):
            g = hq // (nh // nkv)
            K = np.array([kk[g] for kk in ks])
            V = np.array([vv[g] for vv in vs])
            s = K @ q[hq * d:(hq + 1) * d] * c.attention_multiplier
            p = np.exp(s - s.max())
            att[hq * d:(hq + 1) * d] = (p / p.sum()) @ V
        h = (h if residual else 0.0) + c.residual_multiplier * (W["o"] @ att)
        xn = norm(h, W["ln_moe"])
        lg = W["router"] @ xn
        top = np.argsort(-lg, kind="stable")[: c.top_k]
        wt = np.exp(lg[top] - lg[top[0]])
        wt /= wt.sum()
        y = np.zeros(H)
        for e, we in zip(top, wt):
            gu = W["gate_up"][e] @ xn
            gt, up = gu[: c.inter], gu[c.inter:]
            y += we * (W["down"][e] @ (gt / (1 + np.exp(-gt)) * up))
        h = h + c.residual_multiplier * y
    return h
