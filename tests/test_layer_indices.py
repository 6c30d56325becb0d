"""CPU transcription of the index arithmetic of the one-launch layer (lastro-rust_amd/csrc/layers.hip, k_layer): for
every launch shape px_shape admits, the 32 workgroups of an XCD cover the layer input, the q/k/v row pairs of their
KV head group, the output rows, the MoE-norm items, the gate/up pairs and the down rows of their expert exactly once;
every row index stays inside its matrix, every tile read and KV row write inside the head's cache, every exchange
entry inside its area (8-byte entries), and every read-ahead line inside the next layer's matrices and cache."""
import pytest

NT, NW, WAVE = 1024, 16, 64        # kPxThreads, waves, lanes
NU = NW // 2                       # gate/up waves; the rest down rows
ENTRY = 8
MAX_SPLITS = 64                    # AbGroup::part
CE = {"q8_0": 16, "q4_0": 32}      # elements of one 16-byte payload chunk
ROW_BYTES = {"q8_0": lambda k: k, "q4_0": lambda k: k // 2}


def lanes_per_row(nch):
    for lim, lpr in ((32, 64), (16, 32), (8, 16), (4, 8), (2, 4), (1, 2)):
        if nch > lim:
            return lpr
    return 1


def geo(dt, k):
    lpr = lanes_per_row(k // CE[dt])
    return lpr, WAVE // lpr


def attn_splits_for(max_len, tps):
    return ((max_len + 63) // 64 + tps - 1) // tps


def px_shape(dt, hidden, heads, max_len, tps, experts, cus=256):
    """Restatement of px_shape(): (G, T, splits, pp) or None when the layer does not run as one launch."""
    if not ((dt == "q8_0" and hidden in (1024, 1536)) or (dt == "q4_0" and hidden == 1536)):
        return None
    if heads % 8 or heads * 64 != hidden or experts > 63 or max_len % 64 or cus < 256:
        return None
    G, T = heads // 8, tps
    if not ((G == 2 and hidden == 1024) or (G == 3 and hidden == 1536)) or not 2 <= T <= 4:
        return None
    splits = attn_splits_for(max_len, T)
    if splits < G or splits > 32:
        return None
    return G, T, splits, G + 2


def shapes():
    out = set()
    for dt, hidden, heads in (("q8_0", 1024, 16), ("q8_0", 1536, 24), ("q4_0", 1536, 24), ("q4_0", 1024, 16)):
        for max_len in range(64, 8192 + 1, 64):
            for tps in range(1, 6):
                sh = px_shape(dt, hidden, heads, max_len, tps, 40)
                if sh:
                    out.add((dt, hidden, heads, max_len, sh))
    return sorted(out)


SHAPES = shapes()


def test_the_bench_shape_runs_as_one_launch():
    assert px_shape("q8_0", 1536, 24, 4416, 3, 40) == (3, 3, 23, 5)
    assert px_shape("q8_0", 1024, 16, 4416, 3, 40) == (2, 3, 23, 4)
    assert px_shape("q4_0", 1024, 16, 4416, 3, 40) is None  # Q4_0 rows of 1024 take two rows per wave
    assert px_shape("q8_0", 1536, 24, 4352, 2, 40) is None  # 34 splits
    assert px_shape("q8_0", 1536, 24, 4416, 3, 64) is None  # 64 experts: the 65 router items do not fit
    assert len(SHAPES) > 50


@pytest.mark.parametrize("dt,K,heads,max_len,sh", SHAPES[:: max(1, len(SHAPES) // 48)])
def test_layer_indices_in_bounds_and_once(dt, K, heads, max_len, sh):
    G, T, splits, pp = sh
    E, I = 40, 512
    npair = (G + 2) * 32
    qkv_rows = (heads + 16) * 64
    ntiles = max_len // 64
    HR, NOW, PW = K // 32, K // 64, I // 32
    lpr, rpw = geo(dt, K)
    dlpr, drpw = geo(dt, I)
    assert rpw == 1  # one row of length K per wave and pass
    ND = NW - NU
    NPU = (PW + NU - 1) // NU
    DP = (HR + ND * drpw - 1) // (ND * drpw)
    assert G * T <= NW and G + 2 <= G * T and 32 * pp >= npair and HR <= 64
    # A. the input: the last K / 256 waves, one quad per thread, every quad once
    IW = K // 256
    quads = [tx - (NW - IW) * 64 for tx in range((NW - IW) * 64, NT)]
    assert sorted(quads) == list(range(K // 4))
    # the norm: 16-element chunks j = lane + 64 jj of the last wave
    chunks = [lane + 64 * jj for jj in range((K // 16 + 63) // 64) for lane in range(64) if lane + 64 * jj < K // 16]
    assert sorted(chunks) == list(range(K // 16))
    o_rows, hp_pub = [], []
    for x in range(8):
        g = x
        pairs, items, up_pairs, down_rows, att_gather = [], [], [], [], []
        for w in range(32):
            s = w
            t0 = s * T
            for wid in range(NW):
                # B. the wave's row pair
                pl = w * pp + wid
                pok = wid < pp and pl < npair
                plc = pl if pok else 0
                lh, jp = plc // 32, plc % 32
                gh = g * G + lh if lh < G else 8 * G + g if lh == G else 8 * G + 8 + g
                assert 0 <= gh * 64 + jp < qkv_rows and gh * 64 + jp + 32 < qkv_rows
                if pok:
                    pairs.append(pl)
                    if lh < G:
                        assert (lh * 64 + jp + 32 + 1) * ENTRY <= 4 * 64 * ENTRY       # q[lh][jp + 32]
                    else:
                        assert ((lh - G) * 64 + jp + 32 + 1) * ENTRY <= 2 * 64 * ENTRY  # kv[.][jp + 32]
                # tiles: wave wid < G T holds tile t0 + wid / G (clamped to the cache)
                if wid < G * T:
                    tc = min(t0 + wid // G, ntiles - 1)
                    assert 0 <= tc < ntiles
                    assert s < MAX_SPLITS
                # C. output rows (waves 0..7 of workgroups w < NOW)
                if w < NOW and wid < 8:
                    orw = x * (K // 8) + 8 * w + wid
                    assert 0 <= orw < K
                    o_rows.append(orw)
                # D. the router items w and w + 32 of waves 0 and 1
                if wid < 2:
                    item = w + 32 * wid
                    if item <= E:
                        items.append(item)
                        assert item < 64  # PxXcd::item
                # E. gate/up pairs and down rows of the XCD's expert
                for lane in range(WAVE):
                    if wid < NU:
                        for a in range(NPU):
                            li = wid * NPU + a
                            pi = w * PW + li
                            r0 = 7 * 1024 + (pi if li < PW else 0)  # expert 7's rows as an example
                            assert r0 + 512 < E * 1024
                            if li < PW and lane == 0:
                                up_pairs.append(pi)
                    else:
                        dsub, drw = lane % dlpr, lane // dlpr
                        for p in range(DP):
                            li = ((wid - NU) * DP + p) * drpw + drw
                            if li < HR and dsub == 0:
                                dr = w * HR + li
                                down_rows.append(dr)
                                assert x * K + dr < 8 * K  # ys[x][dr]
            # C. the gather of the merged heads by waves 8.. (from the XCD's relayed copy)
            if w < NOW:
                FTC = NT - 512
                for tx in range(512, NT):
                    for m in range((K + FTC - 1) // FTC):
                        i = tx - 512 + m * FTC
                        if i < K:
                            att_gather.append((w, i))
            # the workgroup's 8 rows of h' published with one 8-lane store
            if w < NOW:
                hp_pub.extend(x * (K // 8) + 8 * w + lane for lane in range(8))
        assert sorted(pairs) == list(range(npair)), "every row pair of the group once"
        assert sorted(items) == list(range(E + 1)), "every router item (and the sum of squares) once"
        assert sorted(up_pairs) == list(range(I)), "every gate/up pair of the expert once"
        assert sorted(down_rows) == list(range(K)), "every down row once"
        assert len(att_gather) == NOW * K and max(i for _, i in att_gather) == K - 1
        # the relays: wave 8 (merged heads) and the last wave (h') of workgroup w < 8 copy XCD w's G heads
        relayed = sorted(w * G * 64 + m * 64 + lane for w in range(8) for m in range(G) for lane in range(64))
        assert relayed == list(range(K)) and K <= 2048  # PxDev / PxXcd areas of 2048 entries
        # the merges: workgroup s < G merges head g G + s, its partial reads stay in the area
        for s in range(G):
            assert (g * G + s) * 64 + 63 < K
            for s2 in range(32):
                off = (min(s2, splits - 1) * 4 * 66 + s * 66 + 2 + 63) * ENTRY
                assert off + ENTRY <= MAX_SPLITS * 4 * 66 * ENTRY
    assert sorted(o_rows) == list(range(K)), "every output row once"
    assert sorted(hp_pub) == list(range(K)), "every h' row published once"


@pytest.mark.parametrize("dt,K,heads,max_len,sh", SHAPES[:: max(1, len(SHAPES) // 24)])
def test_read_ahead_lines_stay_inside_the_next_layer(dt, K, heads, max_len, sh):
    """Slot A: payload lines of the wave's two pair rows and its output row, then their scale rows' first dwords;
    slot B: the split's K then V tiles, one line per lane over waves 0..7; a lane without a line reads head g's
    first line."""
    G, T, splits, pp = sh
    npair = (G + 2) * 32
    qkv_rows, o_rows = (heads + 16) * 64, K
    rb = ROW_BYTES[dt](K)
    RL = rb // 128
    assert RL * 128 == rb and 3 * RL + 3 <= 64
    NOW = K // 64
    cache_bytes = 8 * max_len * 64 * 2  # one layer's K (or V) cache, fp16
    for x in range(8):
        g = x
        for w in range(32):
            s, t0 = w, w * T
            for wid in range(8):
                pa = w * pp + wid
                pc = min(pa, npair - 1)
                ah, aj = pc // 32, pc % 32
                agh = g * G + ah if ah < G else 8 * G + g if ah == G else 8 * G + 8 + g
                arow0, orow0 = agh * 64 + aj, x * (K // 8) + 8 * w + wid
                apair = wid < pp and pa < npair
                for lane in range(64):
                    ar = lane // RL if lane < 3 * RL else lane - 3 * RL
                    apay = lane < 3 * RL
                    aval = apair if ar <= 1 else (ar == 2 and w < NOW)
                    rsel = arow0 if ar == 0 else arow0 + 32 if ar == 1 else orow0
                    rows = o_rows if ar == 2 else qkv_rows
                    if aval:
                        assert 0 <= rsel < rows
                        if apay:
                            assert rsel * rb + (lane % RL) * 128 + 4 <= rows * rb
                        else:
                            assert (rsel * (K // 32) + 2) * 2 <= rows * (K // 32) * 2
                    ntl = min(T, max_len // 64 - t0) if s < splits else 0
                    u = wid * 64 + lane
                    bk = u < ntl * 64
                    bv = not bk and u < 2 * ntl * 64
                    if bk or bv:
                        off = ((g * max_len + t0 * 64) * 64) * 2 + (u if bk else u - ntl * 64) * 128
                        assert (g * max_len * 64 * 2) <= off and off + 4 <= ((g + 1) * max_len * 64) * 2
                        assert off + 4 <= cache_bytes
