"""CPU transcription of the index arithmetic of the one-launch batched step (lastro-rust_amd/csrc/grouped.hip,
k_grp_fused) against the sizes its buffers are allocated with (engine.hip, moert_block::ensure_fused; the GroupBufs
of ensure_grouped): every global read and write of every workgroup stays inside its buffer, every LDS access inside
its array, and the router dots, gate/up items, act records, down tiles, output slots and combined rows are each
covered once."""
import numpy as np
import pytest

NT, NW, P, EMAX, I, AW = 512, 8, 16, 48, 512, 17   # kFbThreads, waves, kFbPos, kFbExperts, kFbInter, kFbActW
NBI = I // 32
ENTRY = 8
RE = (EMAX + 15) // 16


def alloc_bytes(H, E):
    """Bytes of each buffer as ensure_fused / ensure_grouped allocate them (element count x element size)."""
    return {
        "err": 1 * 4,
        "lg": 8 * P * 64 * 2 * 4,
        "xflag": 8 * P * 2 * 4,
        "xh": 8 * P * H * 1,
        "xl": 8 * P * H * 1,
        "xd": 8 * P * (H // 32) * 4,
        "act": EMAX * NBI * AW * P * 2 * 4,
        "o": P * 8 * H * 2 * 4,
        "rk": 8 * P * 16 * 2 * 4,
        "gu_q": E * 2 * I * H,             # tiled gate_up payload (Q8_0: one byte per weight)
        "gu_d": E * 2 * I * H // 32 * 2,
        "dn_q": E * H * I,
        "dn_d": E * H * I // 32 * 2,
        "router_rows": E,
        "x": 32 * H * 4,                   # gx and gy: kGrpMaxPos rows
        "y": 32 * H * 4,
        "ids": 32 * 8 * 4,
    }


def lds_bytes(H):
    NB, STR, SA = H // 32, H + 16, I + 16
    return {"big": max(2 * P * STR, 2 * 2 * P * SA), "xd": P * NB * 4, "ad": 2 * P * NBI * 4, "lgs": 64 * 4,
            "sdt": NW * NB * 16 * 2, "gout": 2 * 2 * 32 * (P + 1) * 4, "ids": P * 8 * 4, "w": P * 8 * 4}


def make_plan(ids):
    """List in first-appearance order (position-major, top-k order), member masks and first member slots."""
    lst, bits = [], {}
    for row in ids:
        for p_e in row:
            if p_e not in bits:
                lst.append(p_e)
                bits[p_e] = 0
    for p, row in enumerate(ids):
        for e in row:
            bits[e] |= 1 << p
    offe, off = {}, 0
    for e in lst:
        offe[e] = off
        off += bin(bits[e]).count("1")
    return lst, bits, offe


def check_step(H, E, m, k, pool):
    NB, STR, SA = H // 32, H + 16, I + 16
    NTILE, R, LGN = H // 16, H // 256, P * 64
    sz, lds = alloc_bytes(H, E), lds_bytes(H)
    rng = np.random.default_rng(H + 7 * E + 13 * m + pool)
    experts = rng.permutation(E)[:pool]
    ids = [list(rng.choice(experts, size=k, replace=False)) for _ in range(m)]
    lst, bits, offe = make_plan(ids)
    nu = len(lst)
    assert nu <= E <= EMAX and m <= P and k <= 8
    # R: each XCD codes the m inputs once (workgroup w = bid / 8 codes input w)
    coded = set()
    for bid in range(256):
        xc, w = bid % 8, bid // 8
        if w < m:
            for t in range(NB * 8):
                b, part = t // 8, t % 8
                assert (w * H + 32 * b + 4 * part + 3 + 1) * 4 <= m * H * 4
                row = xc * P + w
                assert row * H + 4 * (8 * b + part) + 4 <= sz["xh"] == sz["xl"]
                assert (row * NB + b + 1) * 4 <= sz["xd"]
                coded.add((xc, w, b, part))
            assert (xc * P + w + 1) * ENTRY <= sz["xflag"]
    assert coded == {(xc, w, b, part) for xc in range(8) for w in range(m) for b in range(NB) for part in range(8)}
    # router dots: wave slot s of an XCD takes position s % 16 and experts s / 16 + 16 i
    dots = {}
    for bid in range(256):
        xc, w = bid % 8, bid // 8
        for wid in range(NW):
            s = 8 * w + wid
            p, e0 = s % 16, s // 16
            if p < m:
                assert (p * H + H) * 4 <= sz["x"]
                for i in range(RE):
                    e = e0 + 16 * i
                    if e < E:
                        assert e < sz["router_rows"]
                        idx = xc * LGN + p * E + e
                        assert (idx + 1) * ENTRY <= sz["lg"]
                        dots[(xc, p, e)] = dots.get((xc, p, e), 0) + 1
    assert dots == {(xc, p, e): 1 for xc in range(8) for p in range(m) for e in range(E)}
    # the top-k of position w by wave 0 of workgroup w < m of each XCD: its E logits, then 8 ids and 8 weights
    ranked = {}
    for bid in range(256):
        xc, w = bid % 8, bid // 8
        if w < m:
            for lane in range(64):
                idx = w * E + (lane if lane < E else 0)
                assert idx < LGN and (xc * LGN + idx + 1) * ENTRY <= sz["lg"] and lane < 64
                if lane < k:
                    for off in (lane, 8 + lane):
                        e = (xc * P + w) * 16 + off
                        assert (e + 1) * ENTRY <= sz["rk"]
                        ranked[e] = ranked.get(e, 0) + 1
    assert ranked == {(xc * P + w) * 16 + o: 1 for xc in range(8) for w in range(m) for o in
                      list(range(k)) + list(range(8, 8 + k))}
    # every workgroup gathers the m positions' entries it uses, each once, into ids_s / w_s
    got = set()
    for t in range(NT):
        p, j = t // 16, t % 16
        if t < m * 16 and (j & 7) < k:
            assert (t + 1) * ENTRY <= P * 16 * ENTRY
            tgt = ("id", p * k + j) if j < 8 else ("w", p * k + j - 8)
            assert tgt[1] < m * k <= P * 8 and tgt not in got
            got.add(tgt)
    assert got == {(kind, i) for kind in ("id", "w") for i in range(m * k)}
    XC, XD = (P * (H // 16) + NT - 1) // NT, (P * NB + NT - 1) // NT
    loaded = []
    for t in range(NT):
        for j in range(XC):
            i = t + j * NT
            if i < m * (H // 16):
                row, c = i // (H // 16), i % (H // 16)
                assert 16 * i + 16 <= P * H
                assert row * STR + 16 * c + 16 <= P * STR
                loaded.append(i)
        for j in range(XD):
            i = t + j * NT
            if i < m * NB:
                assert (i + 1) * 4 <= min(lds["xd"], P * NB * 4)
    assert sorted(loaded) == list(range(m * (H // 16)))
    # U: item q = 2 bid + slot + 512 r (act rows [32 blk, +32) of list expert q / 16)
    items, records = set(), {}
    for bid in range(256):
        for r in range((nu * 16 + 511) // 512):
            for sl in range(2):
                q = 2 * bid + sl + 512 * r
                has = q < nu * 16
                u, blk = (q // 16 if has else 0), q % 16
                e = lst[u]
                for role in range(4):
                    t16 = (e * 2 * I + (role >> 1) * I + 32 * blk + 16 * (role & 1)) // 16
                    assert (t16 * (NB // 2) * 64 + (NB // 2 - 1) * 64 + 63 + 1) * 16 <= sz["gu_q"]
                    assert ((t16 * NB) * 16 + 4 * 63 + 4) * 2 <= sz["gu_d"]
                    for lane in range(64):
                        grp = lane >> 4
                        for i in range(4):
                            assert 16 * (role & 1) + 4 * grp + i < 32 and (lane & 15) < P + 1
                if has:
                    items.add(q)
            # the act codes of the two items' members: 8 lanes per (item, position)
            for t in range(2 * P * 8):
                ss, p, part = t // (P * 8), (t // 8) % P, t & 7
                qq = 2 * bid + ss + 512 * r
                hq = qq < nu * 16
                uu, bb = (qq // 16 if hq else 0), qq % 16
                if hq and p < m and (bits[lst[uu]] >> p) & 1:
                    base = (uu * NBI + bb) * AW * P + p
                    for wd in [part, 8 + part] + ([16] if part == 0 else []):
                        idx = base + wd * P
                        assert (idx + 1) * ENTRY <= sz["act"]
                        records[idx] = records.get(idx, 0) + 1
    assert items == set(range(nu * 16))
    want = {(u * NBI + bb) * AW * P + p + wd * P: 1 for u in range(nu) for bb in range(NBI) for p in range(m)
            if (bits[lst[u]] >> p) & 1 for wd in range(AW)}
    assert records == want, "every act entry of every member written once"
    # D: workgroup b takes tiles [T b, +T) (wave w: tiles w, w + 8, ...) and gathers the act records of their
    # (at most two) experts
    tiles, outs = set(), {}
    total = nu * NTILE
    T = (total + 255) // 256
    TMAX = (EMAX * NTILE + 255) // 256
    JD = (TMAX + NW - 1) // NW
    assert T <= NTILE and T <= TMAX
    for bid in range(256):
        t0 = min(bid * T, total)
        t1 = min(t0 + T, total)
        u0 = min(t0, total - 1) // NTILE
        u1 = (t1 - 1) // NTILE if t1 > t0 else u0
        assert u0 < nu and u1 < nu and u1 - u0 <= 1
        gathered = set()
        for t in range(NT):
            s2, bb, p = t // (NBI * P), t // P % NBI, t % P
            uu = u0 if s2 == 0 else u1
            use = t0 < t1 and (s2 == 0 or u1 != u0) and p < m and (bits[lst[uu]] >> p) & 1
            for wd in range(AW):
                idx = (uu * NBI + bb) * AW * P + p + P * wd
                assert (idx + 1) * ENTRY <= sz["act"]          # loaded whether used or not
                if use:
                    assert idx in want
            if use:
                assert (s2 * P + p) * SA + 32 * bb + 32 <= 2 * P * SA
                assert ((s2 * P + p) * NBI + bb + 1) * 4 <= lds["ad"]
                gathered.add((uu, bb, p))
        for wid in range(NW):
            for j in range(JD):
                dq = t0 + wid + NW * j
                if dq >= t1:
                    continue
                u, t = dq // NTILE, dq % NTILE
                assert u in (u0, u1)
                s2 = 0 if u == u0 else 1
                e = lst[u]
                # the B operand of the tile: the members of u, gathered into slot s2
                for p in range(m):
                    if (bits[e] >> p) & 1:
                        assert all((u, bb, p) in gathered for bb in range(NBI))
                assert (u, t) not in tiles
                tiles.add((u, t))
                t16 = (e * H + 16 * t) // 16
                assert (t16 * (NBI // 2) * 64 + (NBI // 2 - 1) * 64 + 64) * 16 <= sz["dn_q"]
                assert ((t16 * NBI) * 16 + 4 * 63 + 4) * 2 <= sz["dn_d"]
                assert (s2 * P + P - 1) * SA + 32 * (NBI - 1) + 32 <= 2 * P * SA
                for p in range(m):
                    if (bits[e] >> p) & 1:
                        slot = offe[e] + bin(bits[e] & ((1 << p) - 1)).count("1")
                        assert slot < m * k
                        for grp in range(4):
                            for i in range(4):
                                idx = slot * H + 16 * t + 4 * grp + i
                                assert (idx + 1) * ENTRY <= sz["o"]
                                outs[idx] = outs.get(idx, 0) + 1
    assert tiles == {(u, t) for u in range(nu) for t in range(NTILE)}, "every down tile of every expert once"
    assert outs == {i: 1 for i in range(m * k * H)}, "every output row of every member slot once"
    # C: workgroup b combines rows [R b, +R) of every position
    rows = []
    for bid in range(256):
        for t in range(m * R):
            p, row = t // R, R * bid + t % R
            rows.append((p, row))
            assert (p * H + row + 1) * 4 <= sz["y"]
            for e in ids[p]:
                slot = offe[e] + bin(bits[e] & ((1 << p) - 1)).count("1")
                assert (slot * H + row + 1) * ENTRY <= sz["o"]
    assert sorted(rows) == [(p, r) for p in range(m) for r in range(H)]
    assert m * k * 4 <= sz["ids"]


CASES = [(H, E, m, k, pool) for H in (1024, 1536) for E in (8, 32, 40, 48) for m in (1, 5, 16) for k in (1, 8)
         for pool in sorted({k, min(E, 12), E}) if k <= pool <= E]


@pytest.mark.parametrize("H,E,m,k,pool", CASES[:: max(1, len(CASES) // 24)])
def test_fused_block_accesses_stay_inside_their_buffers(H, E, m, k, pool):
    check_step(H, E, m, k, pool)


def test_the_largest_step_is_covered():
    check_step(1536, 48, 16, 8, 48)


def test_lds_fits_one_workgroup_per_compute_unit():
    for H in (1024, 1536):
        assert sum(lds_bytes(H).values()) + 8 * 1024 < 160 * 1024


def test_the_act_records_are_word_sized():
    """act holds 48 experts x 16 blocks x 17 words x 16 positions entries of 8 bytes, allocated as twice that many
    4-byte words (a count of entries would cover half and put the records of experts 24.. past the end)."""
    sz = alloc_bytes(1536, 40)
    last = ((EMAX - 1) * NBI + NBI - 1) * AW * P + P - 1 + (AW - 1) * P
    assert (last + 1) * ENTRY == sz["act"]
