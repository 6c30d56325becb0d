"""CPU transcription of the attention block kernel's index arithmetic (lastro-rust_amd/csrc/attn_block.hip): for
every launch shape the eligibility rule admits, the q/k/v row pairs of each KV head group are computed exactly
once and every row index stays inside the [q; k; v] matrix, every tile read stays inside the cache, exactly one
workgroup of the group takes the new K/V row for every position, each query head is merged by exactly one
workgroup, and every query, K/V row and partial entry offset stays inside the group's exchange area (8-byte
entries: value bits and epoch)."""
import itertools

import pytest

MAX_SPLITS = 64          # kAbMaxSplits
ENTRY = 8                # bytes of an exchange entry
Q_BYTES = 4 * 64 * ENTRY
KV_BYTES = 2 * 64 * ENTRY
PART_REC = 66 * ENTRY    # bytes of one (split, head) partial record: m, l, acc[64]
PART_SPLIT = 4 * PART_REC
PART_BYTES = MAX_SPLITS * PART_SPLIT


def tiles_per_split(max_len, splits):
    return (max_len // 64 + splits - 1) // splits


def attn_splits_for(max_len, tps):
    return ((max_len + 63) // 64 + tps - 1) // tps


def ab_shape(heads, kv_heads, hidden, max_len, tps, cus=256, dtype="q8_0"):
    """Restatement of ab_shape(): the launch shape, or None when the three-kernel path is used."""
    rows_ok = (dtype == "q8_0" and hidden in (1024, 1536)) or (dtype == "q4_0" and hidden == 1536)
    if kv_heads != 8 or heads % 8 or not rows_ok:
        return None
    G, T = heads // 8, tps
    if not ((G == 2 and hidden == 1024) or (G == 3 and hidden == 1536)) or not 2 <= T <= 4 or max_len % 64:
        return None
    splits = attn_splits_for(max_len, T)
    if splits < G or splits > MAX_SPLITS or splits > 32 or 8 * splits > cus:
        return None
    npair = (G + 2) * 32
    pp = (npair + splits - 1) // splits
    np_ = (pp + G * T - 1) // (G * T)
    if np_ > 2:
        return None
    return G, T, splits, pp, np_


def shapes():
    out = []
    for heads, hidden in ((16, 1024), (24, 1536), (16, 1536), (24, 1024)):
        for max_len in range(64, 8192 + 1, 64):
            for req in range(1, 65):
                tps = tiles_per_split(max_len, req)
                sh = ab_shape(heads, 8, hidden, max_len, tps)
                if sh:
                    out.append((heads, hidden, max_len, sh))
    # one entry per distinct (heads, hidden, max_len, shape)
    return sorted(set(out))


SHAPES = shapes()


def test_the_bench_and_test_shapes_are_eligible():
    assert ab_shape(24, 8, 1536, 4416, tiles_per_split(4416, 32)) == (3, 3, 23, 7, 1)
    assert ab_shape(16, 8, 1024, 4416, tiles_per_split(4416, 32)) == (2, 3, 23, 6, 1)
    assert ab_shape(24, 8, 1536, 4352, tiles_per_split(4352, 64)) is None  # 34 splits: three kernels
    assert ab_shape(16, 8, 1024, 448, tiles_per_split(448, 64)) is None    # one tile per split
    assert ab_shape(24, 8, 1536, 4416, tiles_per_split(4416, 32), dtype="q4_0") == (3, 3, 23, 7, 1)
    assert ab_shape(16, 8, 1024, 4416, tiles_per_split(4416, 32), dtype="q4_0") is None  # two rows per wave
    assert len(SHAPES) > 100


@pytest.mark.parametrize("heads,hidden,max_len,sh", SHAPES[:: max(1, len(SHAPES) // 400)])
def test_indices_stay_in_bounds_and_cover_the_work_once(heads, hidden, max_len, sh):
    G, T, splits, pp, NP = sh
    NW = G * T
    npair = (G + 2) * 32
    rows = (heads + 16) * 64
    TR = 64 if 8 % G == 0 else 72
    assert T * TR * 64 >= hidden  # the normalised input fits the V tiles' LDS
    ntiles = max_len // 64
    for g in range(8):
        seen = []
        for s in range(splits):
            assert s < MAX_SPLITS  # part[s]
            for wid, a in itertools.product(range(NW), range(NP)):
                li = wid + NW * a
                l = s * pp + li
                v = li < pp and l < npair
                lc = l if v else 0
                lh, jp = lc // 32, lc % 32
                gh = g * G + lh if lh < G else heads + g if lh == G else heads + 8 + g
                r0, r1 = gh * 64 + jp, gh * 64 + jp + 32
                assert 0 <= r0 < rows and 0 <= r1 < rows  # rows are loaded even when unused
                assert lh < G + 2 and jp < 32  # q[lh][jp + 32] for lh < G; kv[lh - G][jp + 32] otherwise
                if lh < G:
                    assert (lh * 64 + jp + 32) * ENTRY + ENTRY <= Q_BYTES
                else:
                    assert ((lh - G) * 64 + jp + 32) * ENTRY + ENTRY <= KV_BYTES
                if v:
                    seen.append(l)
                    # the right head: q of this group, then the group's K, then its V
                    assert (lh < G and gh // G == g) or gh in (heads + g, heads + 8 + g)
            for wid in range(NW):
                t = s * T + wid // G
                tc = min(t, ntiles - 1)  # past the cache's end: the last tile
                assert 0 <= tc < ntiles
                wh = wid % G
                for lane in range(64):  # the query poll of head wh, the K/V row poll, the partial store
                    assert (wh * 64 + lane) * ENTRY + ENTRY <= Q_BYTES
                    assert (64 + lane) * ENTRY + ENTRY <= KV_BYTES
                    assert s * PART_SPLIT + wh * PART_REC + (2 + lane) * ENTRY + ENTRY <= PART_BYTES
        assert sorted(seen) == list(range(npair)), "every pair of the group exactly once"
    # per position: the patched tile, the used splits, the merge reads
    for pos in sorted({0, 1, 63, 64, 65, max_len // 2, max_len - 65, max_len - 64, max_len - 2, max_len - 1}):
        if not 0 <= pos < max_len:
            continue
        nb = (pos + 1 + 63) // 64
        nsplit = (nb + T - 1) // T
        assert 1 <= nsplit <= splits
        patch = [s for s in range(splits) if 0 <= pos // 64 - s * T < T]
        assert len(patch) == 1 and patch[0] < nsplit
        tp = pos // 64 - patch[0] * T
        assert (pos & 63) < min(64, pos + 1 - (patch[0] * T + tp) * 64)  # the patched row is a valid row
        for hh in range(G):  # workgroup s = hh merges query head g*G + hh
            assert hh < splits
            for s2 in range(32):
                off = min(s2, splits - 1) * PART_SPLIT + hh * PART_REC + ENTRY * (2 + 63)
                assert off + ENTRY <= PART_BYTES
            for lane in range(64):
                sl = min(lane, splits - 1)
                assert sl * PART_SPLIT + hh * PART_REC + 2 * ENTRY <= PART_BYTES
        # every used split holds at least one valid tile; the unused ones write no partial
        for s in range(splits):
            used = min(T, nb - s * T)
            assert (used > 0) == (s < nsplit)


def vt_col(row, dm):
    """VShare::vt_col: column of position `row` in dim row `dm` of the transposed fp16 V tile."""
    return 8 * ((row >> 3) ^ ((dm ^ (dm >> 3)) & 7)) + (row & 7)


def test_transposed_v_tile_layout_is_a_permutation_read_in_order_without_bank_conflicts():
    for dm in range(64):
        assert sorted(vt_col(r, dm) for r in range(64)) == list(range(64))
        sd = (dm ^ (dm >> 3)) & 7
        for cj in range(8):  # p.v reads positions 8cj..8cj+7 of dim dm from 16-byte slot cj ^ sd, in order
            assert [vt_col(8 * cj + t, dm) for t in range(8)] == [8 * (cj ^ sd) + t for t in range(8)]
    # 16-byte reads of one chunk by 8 consecutive dims: 8 different 4-bank groups (row stride 128 B, 32 banks)
    for g in range(8):
        for cj in range(8):
            starts = {(dm * 32 + 4 * (cj ^ ((dm ^ (dm >> 3)) & 7))) % 32 for dm in range(8 * g, 8 * g + 8)}
            assert len(starts) == 8
    # 2-byte writes of element k of a piece (rows 8e..8e+7, lane l: row 8e + l // 8, dims 8 (l % 8) + k): the 64
    # lanes write 32 different dwords in 32 different banks (two lanes share each dword, one half each)
    for e in range(8):
        for k in range(8):
            words = {}
            for lane in range(64):
                row, dm = 8 * e + lane // 8, 8 * (lane % 8) + k
                w = (dm * 64 + vt_col(row, dm)) // 2
                words.setdefault(w, []).append(lane)
            assert len(words) == 32 and len({w % 32 for w in words}) == 32
