"""Host-side checks of the tiled GEMM kernel's LDS layout and load schedule (CPU).

The kernel (teamredbench_amd/csrc/gemm_tiled.hip) keeps A two K stages at a
time in rows of 128 bytes and B one stage at a time, fed by LDS-DMA loads
whose issue order fixes the vmcnt waits. These tests restate the index
arithmetic and check it against the properties the kernel relies on:
  - the A-row swizzle keeps every operand read free of LDS bank conflicts
    for 8-lane (32 banks) and 16-lane (64 banks) phases, and so do the B-row
    swizzles of the transposing reads;
  - every A load instruction covers whole 128-byte lines (one L2 request per
    line, the reason for the pair layout) and its offsets split into two
    vector offsets plus a uniform one, as the kernel computes them;
  - an event-level simulation of the ring (loads complete in issue order,
    slots hold the latest completed load) shows that with the waits the
    kernel derives, every stage's A pair and B stage are in their slots when
    read, no pending load targets them, and this holds for every K length
    (tail loads clamp to the last stage / pair).
"""
from __future__ import annotations

import pytest

STAGE = 64  # bytes of K per row per stage


def swz_a2(r: int) -> int:
    return ((r >> 1) & 7) ^ ((r & 1) << 2)


def swz_b16(k: int) -> int:
    return ((k << 2) ^ (k << 1)) & 15


def swz_b8(k: int) -> int:
    return (2 * k) ^ (k >> 2)


def worst_lanes_per_bank(addrs: list[int], width: int, phase: int, banks: int) -> int:
    """Largest number of lanes of one phase touching one 4-byte bank (1 = conflict-free)."""
    worst = 0
    for p in range(0, len(addrs), phase):
        seen: dict[int, int] = {}
        for a in addrs[p:p + phase]:
            for d in range(width // 4):
                b = (a // 4 + d) % banks
                seen[b] = seen.get(b, 0) + 1
        worst = max(worst, max(seen.values()))
    return worst


def a_read_addrs(row0: int, pair_half: int, sub: int, fp8: bool) -> list[int]:
    out = []
    for lane in range(64):
        half = lane >> 5
        row = row0 + (lane & 31)
        chunk = 4 * pair_half + (2 * half + sub if fp8 else 2 * sub + half)
        out.append(row * 2 * STAGE + ((chunk ^ swz_a2(row)) << 4))
    return out


@pytest.mark.parametrize("bm", [128, 256])
def test_a_pair_reads_are_conflict_free(bm):
    for row0 in range(0, bm, 32):
        for pair_half in range(2):
            for sub in range(2):
                for fp8 in (False, True):
                    addrs = a_read_addrs(row0, pair_half, sub, fp8)
                    assert worst_lanes_per_bank(addrs, 16, 8, 32) == 1
                    assert worst_lanes_per_bank(addrs, 16, 16, 64) == 1


def test_a_swizzle_is_a_permutation_per_row():
    for r in range(256):
        assert sorted(c ^ swz_a2(r) for c in range(8)) == list(range(8))


def b_tr16_addrs(row_bytes: int, nb: int, s: int, t: int) -> list[int]:
    out = []
    for lane in range(64):
        g, i = lane >> 4, lane & 15
        k = 16 * s + 8 * (g >> 1) + 4 * t + (i >> 2)
        n = nb + 16 * (g & 1) + 4 * (i & 3)
        out.append(k * row_bytes + (((n >> 3) ^ swz_b16(k & 3)) << 4) + 8 * (i & 1))
    return out


def b_tr8_addrs(nb: int, t: int, row_bytes: int = 256) -> list[int]:
    out = []
    for lane in range(64):
        g, i = lane >> 4, lane & 15
        k = 32 * (g >> 1) + 8 * t + (i >> 1)
        n = nb + 16 * (g & 1) + 8 * (i & 1)
        f = swz_b8(k & 7) if row_bytes == 256 else k & 7  # 128-byte rows (128 columns): f = k
        out.append(k * row_bytes + (((n >> 4) ^ f) << 4) + 8 * (i & 1))
    return out


def test_b_transposing_reads_are_conflict_free():
    for row_bytes, bn in ((512, 256), (256, 128)):
        for nb in range(0, bn, 32):
            for s in range(2):
                for t in range(2):
                    addrs = b_tr16_addrs(row_bytes, nb, s, t)
                    assert worst_lanes_per_bank(addrs, 8, 16, 32) == 1
                    assert worst_lanes_per_bank(addrs, 8, 32, 64) == 1
    for row_bytes in (256, 128):
        for nb in range(0, row_bytes, 32):
            for t in range(4):
                addrs = b_tr8_addrs(nb, t, row_bytes)
                assert worst_lanes_per_bank(addrs, 8, 16, 32) == 1
                assert worst_lanes_per_bank(addrs, 8, 32, 64) == 1


@pytest.mark.parametrize("bm, waves", [(256, 4), (128, 4)])
@pytest.mark.parametrize("lda", [128, 8192, 16384 + 128])  # A row bytes, multiples of 128
def test_a_loads_cover_whole_lines_and_split_offsets(bm, waves, lda):
    pair_bytes = 2 * bm * STAGE
    a_instr = pair_bytes // 1024 // waves
    assert a_instr % 2 == 0
    for wave in range(waves):
        def voff(q: int, lane: int) -> int:
            lin = (wave * a_instr + q) * 1024 + lane * 16
            row, pchunk = lin // (2 * STAGE), (lin % (2 * STAGE)) >> 4
            return row * lda + ((pchunk ^ swz_a2(row)) << 4)

        covered = set()
        for q in range(a_instr):
            offs = [voff(q, lane) for lane in range(64)]
            lines = {o // 128 for o in offs}
            pieces = set(offs)
            # 8 rows x 128 bytes: each row's 8 pieces are one whole 128-byte run of K
            rows = {o // lda for o in offs}
            assert len(rows) == 8 and len(pieces) == 64
            for r in rows:
                assert sorted(o - r * lda for o in offs if o // lda == r) == list(range(0, 128, 16))
            assert len(lines) == 8
            # the kernel's decomposition: vector offset of q's parity + 16 * (q / 2) rows
            for lane in range(64):
                assert voff(q, lane) == voff(q & 1, lane) + 16 * (q >> 1) * lda
            covered |= rows
        assert covered == set(range(wave * a_instr * 8, (wave + 1) * a_instr * 8))


def load_schedule(na: int, nb: int, ai: int, bi: int) -> tuple[int, int, int]:
    """The waits the kernel derives (gemm_tiled.hip load_schedule): prologue, odd steps, even steps."""
    steps = 64
    end_a: dict[int, int] = {}
    end_b: dict[int, int] = {}
    before: dict[int, int] = {}
    total = 0
    v0 = max(2 * na - 1, nb)
    for v in range(-v0, steps):
        if v >= 0:
            before[v] = total
        if v & 1:
            pair = (v - 1) // 2 + na
            if pair >= 0:
                total += ai
                end_a[pair] = total
        if v + nb >= 0:
            total += bi
            end_b[v + nb] = total
    prologue = before[0] - max(end_a[0], end_b[0])
    waits = {0: 1 << 20, 1: 1 << 20}
    for j in range(steps - 1):
        w = before[j] - max(end_a[(j + 1) // 2], end_b[j + 1])
        waits[j & 1] = min(waits[j & 1], w)
    return prologue, waits[1], waits[0]


def simulate_ring(na: int, nb: int, ai: int, bi: int, ksteps: int,
                  waits: tuple[int, int, int] | None = None) -> None:
    prologue, odd, even = waits or load_schedule(na, nb, ai, bi)
    assert 0 <= prologue < 64 and 0 <= odd < 64 and 0 <= even < 64
    last, last_pair = ksteps - 1, (ksteps - 1) // 2
    issued: list[tuple[str, int, int]] = []

    def issue(kind: str, idx: int, slot: int, n: int) -> None:
        issued.extend([(kind, idx, slot)] * n)

    def check(wait: int, stage: int) -> None:
        done, pending = issued[:len(issued) - wait], issued[len(issued) - wait:]
        content: dict[tuple[str, int], int] = {}
        for kind, idx, slot in done:
            content[(kind, slot)] = idx
        pair = stage // 2
        assert content.get(("A", pair % na)) == pair, (ksteps, stage)
        assert content.get(("B", stage % nb)) == stage, (ksteps, stage)
        assert ("A", pair % na) not in {(k, s) for k, _, s in pending if k == "A"}
        assert ("B", stage % nb) not in {(k, s) for k, _, s in pending if k == "B"}

    for v in range(-max(2 * na - 1, nb), 0):
        if v & 1 and (v - 1) // 2 + na >= 0:
            pair = (v - 1) // 2 + na
            issue("A", min(pair, last_pair), pair % na, ai)
        if v + nb >= 0:
            issue("B", min(v + nb, last), (v + nb) % nb, bi)
    check(prologue, 0)
    for kt in range(ksteps):
        if kt + 1 < ksteps:
            check(odd if kt & 1 else even, kt + 1)
        if kt & 1:
            pair = (kt - 1) // 2 + na
            issue("A", min(pair, last_pair), pair % na, ai)
        issue("B", min(kt + nb, last), (kt + nb) % nb, bi)


# (A pair slots, B stage slots, A loads per wave per pair, B loads per wave per stage) of the
# three tiled configurations: 256x256 (16-bit and fp8), 128x256, 128x128 (16-bit).
CONFIGS = [(3, 4, 8, 4), (3, 6, 4, 4), (3, 6, 4, 2)]


@pytest.mark.parametrize("cfg", CONFIGS)
def test_ring_schedule_is_safe_for_every_k_length(cfg):
    for ksteps in list(range(1, 41)) + [63, 64, 65, 128, 129, 256]:
        simulate_ring(*cfg, ksteps)


def test_ring_waits_of_the_configurations():
    # The steady state waits only for the B stage issued NB - 1 steps earlier.
    assert load_schedule(3, 4, 8, 4) == (28, 16, 16)
    assert load_schedule(3, 6, 4, 4) == (28, 20, 24)
    assert load_schedule(3, 6, 4, 2) == (18, 12, 16)


@pytest.mark.parametrize("loosen", [(1, 0, 0), (0, 1, 0), (0, 0, 1)])
def test_simulation_catches_a_wait_one_load_too_loose(loosen):
    # Allowing one more pending load than the schedule derives leaves a needed stage in flight.
    prologue, odd, even = load_schedule(3, 4, 8, 4)
    waits = (prologue + loosen[0], odd + loosen[1], even + loosen[2])
    with pytest.raises(AssertionError):
        simulate_ring(3, 4, 8, 4, 16, waits)
