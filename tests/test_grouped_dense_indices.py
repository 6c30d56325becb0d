"""CPU transcription of the index arithmetic of the grouped mode's dense kernels (lastro-rust_amd/csrc/
grouped_dense.hip, mfma_q8.h): the rows and K quarter of each wave of k_gd_dense, its reads of the tiled weights
(payload and scales), of the member codes and their LDS staging, the MFMA tile's LDS reads, the quarter-sum buffer,
and the epilogues' q / K / V / RoPE / residual indices; the element, block and code indices of k_gd_norm_codes and
k_gd_combine. For the 1B and 3B shapes and every position count 1..32, every index is checked against the buffer it
addresses (sizes as the engine allocates them), and the row / element coverage against being complete and
disjoint, so that a launch writes each output once."""
import numpy as np
import pytest

M = 32          # positions per step
THREADS = 512   # k_gd_dense
SHAPES = {"1b": dict(hidden=1024, heads=16, kvh=8), "3b": dict(hidden=1536, heads=24, kvh=8)}


def dense_waves(K, NM, rows, qkv):
    """Per (workgroup, wave): row0, t16 and the first block of the wave's K quarter."""
    NB = K // 32
    NBW = NB // 4
    grid = rows // 64 * 2 if qkv else rows // 32
    out = []
    for bx in range(grid):
        for wave in range(THREADS // 64):
            p, kq = wave & 1, wave >> 1
            row0 = (bx >> 1) * 64 + 16 * (bx & 1) + 32 * p if qkv else 32 * bx + 16 * p
            out.append((bx, wave, p, kq, row0, row0 // 16, kq * NBW))
    return grid, out


@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("which", ["qkv", "oproj"])
def test_dense_weight_reads_cover_each_row_and_block_once(shape, which):
    c = SHAPES[shape]
    H, qd = c["hidden"], c["heads"] * 64
    rows, K = ((c["heads"] + 2 * c["kvh"]) * 64, H) if which == "qkv" else (H, qd)
    NB, NBW = K // 32, K // 32 // 4
    assert NB % 8 == 0 and rows % 64 == 0
    seen = np.zeros((rows, NB), int)
    n_payload = rows // 16 * (NB // 2) * 64  # 16-byte pieces of the tiled payload
    n_scales = rows * NB                     # fp16 scales
    for _, _, _, _, row0, t16, b0 in dense_waves(K, 32, rows, which == "qkv")[1]:
        assert row0 % 16 == 0 and b0 % 2 == 0
        lane = np.arange(64)
        # fetch_tile_q8: ((t16 * NB/2 + b0/2) * 64 + lane) + q * 64, q < NBW/2
        for q in range(NBW // 2):
            idx = (t16 * (NB // 2) + b0 // 2) * 64 + lane + q * 64
            assert idx.max() < n_payload
        # fetch_scales: uint2 pieces lane + 64 q < 4 NBW of (t16 * NB + b0) * 16 halves
        pieces = np.arange(4 * NBW)
        halves = (t16 * NB + b0) * 16 + 4 * pieces + 3
        assert halves.max() < n_scales
        seen[row0:row0 + 16, b0:b0 + NBW] += 1
    assert (seen == 1).all()


@pytest.mark.parametrize("K", [1024, 1536])
@pytest.mark.parametrize("NM", [16, 32])
def test_member_staging_and_mfma_lds_reads_stay_in_bounds(K, NM):
    NB, NBW, STR = K // 32, K // 32 // 4, K + 16
    C16 = K // 16
    PER = -(-NM * C16 // THREADS)
    PERD = -(-NM * NB // THREADS)
    X = 1536  # code row length the engine allocates (max of hidden and heads * 64)
    for m in ([1, 7, 16] if NM == 16 else [17, 31, 32]):
        written = np.zeros(NM * STR, int)
        for t in range(THREADS):
            for q in range(PER):
                i = t + q * THREADS
                c, j = i // C16, i % C16
                if i < NM * C16:
                    if c < m:
                        assert (c * K + 16 * j + 16) <= M * X  # global read r * K + 16 j, r = c (positions 0..m-1)
                    lo = c * STR + 16 * j
                    assert lo + 16 <= NM * STR
                    written[lo:lo + 16] += 1
            for q in range(PERD):
                i = t + q * THREADS
                if i < NM * NB:
                    assert i < NM * NB
        used = np.zeros(NM * STR, bool)
        for c in range(NM):
            used[c * STR:c * STR + K] = True
        assert (written[used] == 1).all() and (written[~used] == 0).all()
        # mfma_tile: bh + 32 kq NBW + c * STR + 32 b + 8 grp, 8 bytes
        for kq in range(4):
            for b in range(NBW):
                top = 32 * kq * NBW + (NM - 1) * STR + 32 * b + 8 * 3 + 8
                assert top <= NM * STR
                assert 32 * kq * NBW + 32 * b + 8 * 3 + 8 <= K  # inside the member's row
                assert (NM - 1) * NB + kq * NBW + b < NM * NB   # dx
                assert b * 16 + 4 * 3 + 4 <= NBW * 16            # sdt of the wave


@pytest.mark.parametrize("shape", list(SHAPES))
def test_qkv_epilogue_writes_each_output_once(shape):
    c = SHAPES[shape]
    heads, kvh = c["heads"], c["kvh"]
    rows = (heads + 2 * kvh) * 64
    max_len = 128
    for m in (1, 5, 16, 17, 32):
        NM = 32 if m > 16 else 16
        pos0 = max_len - m
        q = np.zeros(m * heads * 64, int)
        kc = np.zeros(kvh * max_len * 64, int)
        vc = np.zeros(kvh * max_len * 64, int)
        grid = rows // 64 * 2
        for bx in range(grid):
            for t in range(THREADS):
                jj, cpos = t & 15, t >> 4
                if cpos >= NM or cpos >= m:
                    continue
                assert 16 + jj < 32 and cpos < NM  # red rows / columns
                head, jp = bx >> 1, 16 * (bx & 1) + jj
                pos = pos0 + cpos
                assert pos * 64 + 32 + jp < max_len * 64  # rope
                if head < heads:
                    base = cpos * heads * 64 + head * 64
                    q[base + jp] += 1
                    q[base + jp + 32] += 1
                elif head < heads + kvh:
                    base = ((head - heads) * max_len + pos) * 64
                    kc[base + jp] += 1
                    kc[base + jp + 32] += 1
                else:
                    base = ((head - heads - kvh) * max_len + pos) * 64
                    vc[base + jp] += 1
                    vc[base + jp + 32] += 1
        assert (q == 1).all()
        for cache in (kc, vc):
            cc = cache.reshape(kvh, max_len, 64)
            assert (cc[:, pos0:pos0 + m] == 1).all() and cc[:, :pos0].sum() == 0


@pytest.mark.parametrize("shape", list(SHAPES))
def test_residual_epilogue_writes_each_element_once(shape):
    H = SHAPES[shape]["hidden"]
    for m in (1, 16, 17, 32):
        NM = 32 if m > 16 else 16
        h = np.zeros(m * H, int)
        for bx in range(H // 32):
            for t in range(THREADS):
                for it in range(t, 32 * NM, THREADS):
                    r, cpos = it & 31, it >> 5
                    if cpos < m:
                        h[cpos * H + 32 * bx + r] += 1
        assert (h == 1).all()


@pytest.mark.parametrize("H", [1024, 1536])
def test_norm_and_combine_elements_and_codes(H):
    """k_gd_norm_codes / k_gd_combine: pass j of thread t holds elements 1024 j + 4 t .. +3 (valid below H); the codes
    of block b = e0 / 32, part t % 8 land at uint32 8 b + part of the row, the scale at b (part 0)."""
    NP = -(-H // 1024)
    seen = np.zeros(H, int)
    codes = np.zeros(H // 4, int)
    scales = np.zeros(H // 32, int)
    for t in range(256):
        for j in range(NP):
            e0 = 1024 * j + 4 * t
            if e0 < H:
                seen[e0:e0 + 4] += 1
                b, part = e0 // 32, t & 7
                assert 32 * b + 4 * part == e0
                codes[8 * b + part] += 1
                if part == 0:
                    scales[b] += 1
    assert (seen == 1).all() and (codes == 1).all() and (scales == 1).all()
    # the eight lanes of a block (group_max over 8) are lanes 8 (t // 8) .. +7 of one wave, all valid or all not
    for t0 in range(0, 256, 8):
        for j in range(NP):
            v = [1024 * j + 4 * t < H for t in range(t0, t0 + 8)]
            assert all(v) or not any(v)


def _nth_set_bit(bits, c):
    for _ in range(c):
        bits &= bits - 1
    return (bits & -bits).bit_length() - 1


@pytest.mark.parametrize("m,k,E", [(1, 8, 40), (16, 8, 40), (17, 8, 40), (32, 8, 40), (32, 2, 6), (24, 4, 64)])
def test_expert_member_groups_cover_every_member_once(m, k, E):
    """k_grp_up / k_grp_down take an expert's members in groups of 16 (grid z = ceil(m / 16)): workgroup z handles
    members [16 z, 16 z + 16) and ends at once when the expert has no more. Each (expert, member) is computed once,
    its position is the member index's set bit of the expert's mask (the group's mask has its first 16 z bits
    cleared), and its slot off + 16 z + j stays below m * k."""
    rng = np.random.default_rng(m * 100 + k * 10 + E)
    ids = [list(rng.choice(E, size=k, replace=False)) for _ in range(m)]
    # a skewed step: the first expert routed by every position
    ids = [[0] + [e for e in row if e != 0][:k - 1] for row in ids]
    order, bits = [], {}
    for row in ids:
        for e in row:
            if e not in bits:
                order.append(e)
                bits[e] = 0
    for p, row in enumerate(ids):
        for e in row:
            bits[e] |= 1 << p
    offe, off = {}, 0
    for e in order:
        offe[e] = off
        off += bin(bits[e]).count("1")
    CH = (m + 15) // 16
    done = {}
    for u, e in enumerate(order):
        ne_all = bin(bits[e]).count("1")
        for z in range(CH):
            c0 = 16 * z
            if ne_all <= c0:
                continue  # the workgroup ends at once
            b = bits[e]
            for _ in range(c0):
                b &= b - 1
            ne = bin(b).count("1")
            assert ne == ne_all - c0
            for j in range(min(16, ne)):
                pos = _nth_set_bit(b, j)
                assert pos == _nth_set_bit(bits[e], c0 + j)
                slot = offe[e] + c0 + j
                assert slot < m * k
                done[(e, c0 + j)] = done.get((e, c0 + j), 0) + 1
    assert done == {(e, c): 1 for e in order for c in range(bin(bits[e]).count("1"))}
    assert max(bin(bits[e]).count("1") for e in order) == m  # expert 0: every position, so z reaches m - 1
