"""CPU transcription of the index arithmetic of the MoE kernel spread over the XCDs (lastro-rust_amd/csrc/
moe_block.hip, k_moe_xcd): for every compiled shape, the 32 workgroups of an XCD compute each gate/up pair and each
down row of their expert exactly once, every row index stays inside the layer's matrices, and every exchange and
output index stays inside its buffer (the act vector: one epoch-tagged entry per value, polled by the down threads)."""
import pytest

WGS, WAVES, WAVE = 32, 16, 64      # kMxWgs, kMxWaves, lanes
NU = 8                             # kMxUpWaves: waves 0..7 gate/up pairs, waves 8..15 down rows
CE = {"q8_0": 16, "q4_0": 32}      # elements of one 16-byte payload chunk


def lanes_per_row(nch):
    for lim, lpr in ((32, 64), (16, 32), (8, 16), (4, 8), (2, 4), (1, 2)):
        if nch > lim:
            return lpr
    return 1


def geo(dt, k):
    nch = k // CE[dt]
    lpr = lanes_per_row(nch)
    return lpr, WAVE // lpr


@pytest.mark.parametrize("dt", ["q8_0", "q4_0"])
@pytest.mark.parametrize("K", [1024, 1536])
@pytest.mark.parametrize("E", [32, 40, 64])
def test_pairs_and_down_rows_once_and_in_bounds(dt, K, E):
    I = 512
    lpr, rpw = geo(dt, K)
    dlpr, drpw = geo(dt, I)
    ND = WAVES - NU
    NP = (I // WGS + NU * rpw - 1) // (NU * rpw)
    DP = (K // WGS + ND * drpw - 1) // (ND * drpw)
    PW, RB = I // WGS, K // WGS
    assert NU * NP * rpw >= PW and ND * DP * drpw >= RB
    for ej in (0, E - 1):
        for x in range(8):
            pairs, rows = [], []
            for w in range(WGS):
                for wave in range(WAVES):
                    up = wave < NU
                    for lane in range(WAVE):
                        sub, rw = lane % lpr, lane // lpr
                        for a in range(NP if up else 0):
                            li = (wave * NP + a) * rpw + rw
                            pi = w * PW + li
                            v = li < PW
                            r0 = ej * 2 * I + (pi if v else 0)
                            assert 0 <= r0 < E * 2 * I and 0 <= r0 + I < E * 2 * I
                            if v and sub == 0:
                                pairs.append(pi)
                                assert pi < I  # act[pi] of the XCD's area
                        dsub, drw = lane % dlpr, lane // dlpr
                        for p in range(DP):
                            li = ((wave - NU) * DP + p) * drpw + drw
                            dr = w * RB + li
                            ok = not up and li < RB
                            drow = ej * K + (dr if ok else 0)
                            assert 0 <= drow < E * K
                            if ok and dsub == 0:
                                rows.append(dr)
                                assert x * K + dr < 8 * K  # ys[x][dr]
                for t in range(NU * 64, WAVES * 64):  # down thread t polls act[t - NU * 64]
                    assert 0 <= t - NU * 64 < I
            assert sorted(pairs) == list(range(I)), "every gate/up pair of the expert once"
            assert sorted(rows) == list(range(K)), "every down row of the expert once"
