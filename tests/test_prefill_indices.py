"""CPU transcription of the index arithmetic of the multi-position step's row kernels (lastro-rust_amd/csrc/
prefill.hip): the xor-swizzled LDS layout of staged activations (xslot), the staging of a group of positions
(stage_group, and the member staging of k_moe_up_b / k_moe_down_b), the per-position norms (wave_rms, rsv), the RoPE
table rows (csv), the output projection's row buffer (hn) and the bounds of a partial last group, for every block
size 1..32 and every row length and dtype the kernels are built for. Every LDS and global index is checked against
the array it addresses, and the swizzle against being a permutation inside each weight chunk (so each staged
element is written once and read back where the unswizzled layout has it)."""
import numpy as np
import pytest

PF_WAVES, PF_NT, PF_GROUP, PF_MAX_POS = 8, 512, 8, 32
CHUNK = {"f32": 4, "q8_0": 16, "q4_0": 32}  # elements per 16-byte payload chunk (Fmt<DT>::kElems)
ROW_LENGTHS = [128, 256, 512, 1024, 1536, 2048]


def xslot(dt, s):
    """xslot<DT>(s) of prefill.hip (vectorised)."""
    nq = CHUNK[dt] // 4
    s = np.asarray(s)
    if nq == 1:
        return s
    j, q = s // nq, s % nq
    sw = (((j >> 1) ^ (j >> 3)) & 3) if nq == 4 else ((j ^ (j >> 3)) & 7)
    return nq * j + (q ^ sw)


@pytest.mark.parametrize("dt", list(CHUNK))
@pytest.mark.parametrize("K", ROW_LENGTHS)
def test_swizzle_is_a_permutation_inside_each_chunk(dt, K):
    k4 = K // 4
    if K % CHUNK[dt]:
        pytest.skip("row length not a whole number of chunks")
    s = np.arange(k4)
    x = xslot(dt, s)
    assert x.min() == 0 and x.max() == k4 - 1 and len(np.unique(x)) == k4
    nq = CHUNK[dt] // 4
    assert np.array_equal(x // nq, s // nq)  # a slot stays in its chunk


def _threads(total):
    """The (thread, index) pairs of `for (i = threadIdx.x; i < total; i += kPfNT)` over one workgroup."""
    return np.arange(total)


@pytest.mark.parametrize("dt", list(CHUNK))
@pytest.mark.parametrize("K", ROW_LENGTHS)
def test_group_staging_norms_and_reads_stay_in_bounds(dt, K):
    """stage_group + wave_rms + load_xs over groups v0 = 0, 8, ... of nv positions (the last one partial)."""
    if K % CHUNK[dt]:
        pytest.skip("row length not a whole number of chunks")
    k4, nq = K // 4, CHUNK[dt] // 4
    nch = K // CHUNK[dt]
    for nv in range(1, PF_MAX_POS + 1):
        covered = np.zeros((nv, K), bool)
        for v0 in range(0, nv, PF_GROUP):
            n = min(PF_GROUP, nv - v0)
            assert 1 <= n <= PF_GROUP
            i = _threads(n * k4)
            row, slot = i // k4, xslot(dt, i % k4)
            assert row.max() < PF_GROUP and slot.max() < k4  # xs[i / K4][xslot(i % K4)]
            src = v0 * k4 + i  # float4 index of x + v0 * K
            assert src.max() < nv * k4  # inside the nv staged rows of the buffer
            # each staged float4 lands in a distinct LDS slot of its row
            assert len(np.unique(row * k4 + slot)) == len(i)
            # wave_rms: wave w < n reads x4[xslot(4 j + e)] of row w for chunks j < K/16
            j = np.arange(K // 16)[:, None] * 4 + np.arange(4)[None, :]
            assert xslot(dt, j).max() < k4
            assert min(PF_WAVES, n) == n  # rsv[wave] for wave < n: every position of the group has a wave
            # load_xs: lane sub reads chunk j = sub + LPR * jj < NCH, slots xslot(NQ j + e)
            cj = np.arange(nch)[:, None] * nq + np.arange(nq)[None, :]
            assert xslot(dt, cj).max() < k4
            # the swizzled read of chunk j, slot e returns element 4 (NQ j + e) .. of the unswizzled row
            staged = np.empty(k4, int)
            staged[xslot(dt, np.arange(k4))] = np.arange(k4)
            assert np.array_equal(staged[xslot(dt, cj)], cj)
            covered[v0:v0 + n] = True
        assert covered.all()


@pytest.mark.parametrize("heads,kvh", [(4, 2), (16, 8), (24, 8), (32, 8)])
def test_rope_rows_and_head_rows(heads, kvh):
    """k_qkv_b: csv[i / 64][i % 64] = rope[(pos0 + v0 + i / 64) * 64 + i % 64] for i < n * 64, then csv[v][jp] and
    csv[v][32 + jp] for v < n, jp < 32; q rows of position v0 + v at qb + (v0 + v) * heads * 64."""
    max_len = 256
    for nv in range(1, PF_MAX_POS + 1):
        for pos0 in (0, max_len - nv):
            for v0 in range(0, nv, PF_GROUP):
                n = min(PF_GROUP, nv - v0)
                i = _threads(n * 64)
                assert (i // 64).max() < PF_GROUP
                assert ((pos0 + v0 + i // 64) * 64 + i % 64).max() < max_len * 64
                q_top = (v0 + n - 1) * heads * 64 + (heads - 1) * 64 + 63
                assert q_top < PF_MAX_POS * heads * 64


@pytest.mark.parametrize("dt", list(CHUNK))
@pytest.mark.parametrize("H", [256, 1024, 1536])
def test_output_projection_row_buffer(dt, H):
    """k_oproj_b: hn[v][row - r0] with row = (blockIdx.x * 8 + wave) * (P * RPW) + p * RPW + rw, r0 = blockIdx.x * RB,
    RB = 8 * P * RPW; every index < RB for the rows of every workgroup (including the last, partial one)."""
    for rpw in (1, 2, 4, 8):  # rows per wave of the Geo variants (64 / LPR lanes per row)
        for P in (1, 2, 4):
            rb = PF_WAVES * P * rpw
            nblk = -(-H // rb)
            for b in range(nblk):
                wave = np.arange(PF_WAVES)[:, None, None]
                p = np.arange(P)[None, :, None]
                rw = np.arange(rpw)[None, None, :]
                row = (b * PF_WAVES + wave) * (P * rpw) + p * rpw + rw
                off = row - b * rb
                assert off.min() >= 0 and off.max() < rb


@pytest.mark.parametrize("k", [1, 2, 8])
def test_expert_member_staging(k):
    """k_moe_up_b / k_moe_down_b: members of an expert are the set bits of a 32-bit mask over positions; staging
    c0 .. c0 + n - 1 (up: groups of 8 into xs[8][K]; down: all ne into xs[32][K]) reads member c through
    nth_bit64(members, c), always a position < nv; act / o rows (vpos * k + rank) * len stay below nv * k * len."""
    rng = np.random.default_rng(7)

    def nth_bit(b, u):
        for _ in range(u):
            b &= b - 1
        return (b & -b).bit_length() - 1 if b else -1

    for nv in range(1, PF_MAX_POS + 1):
        for _ in range(4):
            members = int(rng.integers(1, 1 << nv))
            ne = bin(members).count("1")
            assert ne <= PF_MAX_POS
            for c0 in range(0, ne, PF_GROUP):
                n = min(PF_GROUP, ne - c0)
                for c in range(n):
                    vpos = nth_bit(members, c0 + c)
                    assert 0 <= vpos < nv
                    for rank in range(k):
                        assert (vpos * k + rank) < nv * k
            assert all(0 <= nth_bit(members, c) < nv for c in range(ne))
            assert nth_bit(members, ne) == -1
