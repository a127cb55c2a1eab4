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


def swz_b16_128(k: int) -> int:
    """16-bit B rows of 128 bytes (64 columns)."""
    return 2 * k


def swz_b8_64(k: int) -> int:
    """fp8 B rows of 64 bytes (64 columns)."""
    return (k >> 1) & 3


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
    swz = swz_b16_128 if row_bytes == 128 else swz_b16
    out = []
    for lane in range(64):
        g, i = lane >> 4, lane & 15
        k = 16 * s + 8 * (g >> 1) + 4 * t + (i >> 2)
        n = nb + 16 * (g & 1) + 4 * (i & 3)
        out.append(k * row_bytes + (((n >> 3) ^ swz(k & 3)) << 4) + 8 * (i & 1))
    return out


def b_tr8_addrs(nb: int, t: int, row_bytes: int = 256) -> list[int]:
    out = []
    for lane in range(64):
        g, i = lane >> 4, lane & 15
        k = 32 * (g >> 1) + 8 * t + (i >> 1)
        n = nb + 16 * (g & 1) + 8 * (i & 1)
        # 128-byte rows (128 columns): f = k; 64-byte rows (64 columns): swz_b8_64
        f = swz_b8(k & 7) if row_bytes == 256 else (k & 7) if row_bytes == 128 else swz_b8_64(k & 7)
        out.append(k * row_bytes + (((n >> 4) ^ f) << 4) + 8 * (i & 1))
    return out


def test_b_transposing_reads_are_conflict_free():
    for row_bytes, bn in ((512, 256), (256, 128), (128, 64)):
        for nb in range(0, bn, 32):
            for s in range(2):
                for t in range(2):
                    addrs = b_tr16_addrs(row_bytes, nb, s, t)
                    assert worst_lanes_per_bank(addrs, 8, 16, 32) == 1
                    assert worst_lanes_per_bank(addrs, 8, 32, 64) == 1
    for row_bytes in (256, 128, 64):
        for nb in range(0, row_bytes, 32):
            for t in range(4):
                addrs = b_tr8_addrs(nb, t, row_bytes)
                assert worst_lanes_per_bank(addrs, 8, 16, 32) == 1
                assert worst_lanes_per_bank(addrs, 8, 32, 64) == 1


@pytest.mark.parametrize("bm, waves", [(256, 4), (128, 4), (64, 4)])   # 64 rows: the 64 x 128 and 64 x 64 tiles
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
# five tiled configurations: 256x256 (16-bit and fp8), 128x256, 128x128, 64x128 and 64x64 (16-bit).
CONFIGS = [(3, 4, 8, 4), (3, 6, 4, 4), (3, 6, 4, 2), (3, 6, 2, 2), (3, 6, 2, 1)]


@pytest.mark.parametrize("cfg", CONFIGS)
def test_ring_schedule_is_safe_for_every_k_length(cfg):
    for ksteps in list(range(1, 41)) + [63, 64, 65, 128, 129, 256]:
        simulate_ring(*cfg, ksteps)


def test_ring_waits_of_the_configurations():
    # The steady state waits only for the B stage issued NB - 1 steps earlier.
    assert load_schedule(3, 4, 8, 4) == (28, 16, 16)
    assert load_schedule(3, 6, 4, 4) == (28, 20, 24)
    assert load_schedule(3, 6, 4, 2) == (18, 12, 16)
    assert load_schedule(3, 6, 2, 2) == (14, 10, 12)
    assert load_schedule(3, 6, 2, 1) == (9, 6, 8)


@pytest.mark.parametrize("loosen", [(1, 0, 0), (0, 1, 0), (0, 0, 1)])
def test_simulation_catches_a_wait_one_load_too_loose(loosen):
    # Allowing one more pending load than the schedule derives leaves a needed stage in flight.
    prologue, odd, even = load_schedule(3, 4, 8, 4)
    waits = (prologue + loosen[0], odd + loosen[1], even + loosen[2])
    with pytest.raises(AssertionError):
        simulate_ring(3, 4, 8, 4, 16, waits)


# ---------------------------------------------------------------------------
# fp8 kernel on v_mfma_scale_f32_16x16x128_f8f6f4 (gemm_fp8_mi16_kernel). Lane
# l, g = l // 16, holds K 16g..16g+15 (first stage of a pair) and 64+16g..
# (second stage); B rows are swizzled by swz_b8(k & 7) (256-byte rows) or
# k & 7 (128-byte rows), XORed with bit 4 of k.

def swz_b8_mi16(k: int, row_bytes: int) -> int:
    return (swz_b8(k & 7) if row_bytes == 256 else k & 7) ^ ((k >> 4) & 1)


def mi16_b_read_addrs(row_bytes: int, b_col: int, j: int, t: int) -> list[int]:
    out = []
    for lane in range(64):
        g, i = lane >> 4, lane & 15
        k = 16 * g + 8 * t + (i >> 1)
        n = b_col + 16 * j + 8 * (i & 1)
        out.append(k * row_bytes + (((n >> 4) ^ swz_b8_mi16(k, row_bytes)) << 4) + 8 * (i & 1))
    return out


def mi16_a_read_addrs(wm_rows: int, i: int, hi: int) -> list[int]:
    out = []
    for lane in range(64):
        g, l16 = lane >> 4, lane & 15
        row = wm_rows + l16 + 16 * i
        chunk = 4 * hi + g
        out.append(row * 2 * STAGE + ((chunk ^ swz_a2(row)) << 4))
    return out


@pytest.mark.parametrize("row_bytes, wtn", [(256, 128), (128, 64)])
def test_mi16_b_reads_conflict_free_and_offsets_split(row_bytes, wtn):
    for wn in range(row_bytes // wtn):
        b_col = wn * wtn
        for j in range(wtn // 16):
            for t in range(2):
                addrs = mi16_b_read_addrs(row_bytes, b_col, j, t)
                assert worst_lanes_per_bank(addrs, 8, 16, 32) == 1
                assert worst_lanes_per_bank(addrs, 8, 32, 64) == 1
                # the kernel's decomposition: one offset per j, part t as an immediate
                for lane in range(64):
                    g, l16 = lane >> 4, lane & 15
                    kb = 16 * g + (l16 >> 1)
                    off = kb * row_bytes + ((((b_col >> 4) + j) ^ swz_b8_mi16(kb, row_bytes)) << 4) + 8 * (l16 & 1)
                    assert addrs[lane] == off + t * 8 * row_bytes


@pytest.mark.parametrize("wtm", [128, 64])
def test_mi16_a_reads_conflict_free_and_offsets_split(wtm):
    for wm in range(2):
        for i in range(wtm // 16):
            for hi in range(2):
                addrs = mi16_a_read_addrs(wm * wtm, i, hi)
                assert worst_lanes_per_bank(addrs, 16, 8, 32) == 1
                assert worst_lanes_per_bank(addrs, 16, 16, 64) == 1
                for lane in range(64):
                    g, l16 = lane >> 4, lane & 15
                    a_row, sa = wm * wtm + l16, swz_a2(l16)
                    off = a_row * 2 * STAGE + ((((4 * hi) + g) ^ sa) << 4)
                    assert addrs[lane] == off + i * 16 * 2 * STAGE


def tr8_read(lds: bytearray, addrs: list[int]) -> list[bytes]:
    """ds_read_b64_tr_b8 as the kernels use it: in each 16-lane group, lanes 2r and 2r + 1 address
    row r (columns 0-7 and 8-15) of an 8 x 16 byte block; lane i receives column i, rows 0-7."""
    out = []
    for lane in range(64):
        base, i = lane & ~15, lane & 15
        out.append(bytes(lds[addrs[base + 2 * r + (i >> 3)] + (i & 7)] for r in range(8)))
    return out


@pytest.mark.parametrize("row_bytes", [256, 128])
def test_mi16_b_dma_layout_feeds_each_lane_its_k_and_column(row_bytes):
    # Global B stage: 64 K rows x row_bytes columns, byte value encodes (k, n). The DMA lanes of
    # instruction q of a wave place 16-byte chunks as the kernel computes them (two vector offsets
    # plus a uniform 2 * RPI * (q // 2) rows); then the transposing reads must hand lane l of
    # fragment j, part t exactly K rows 16g + 8t + r (r = 0..7) of column b_col + 16j + l % 16.
    rpi, waves = 1024 // row_bytes, 4
    b_instr = 64 * row_bytes // 1024 // waves
    assert b_instr % 2 == 0 and b_instr * rpi * waves == 64
    key = {}
    lds = bytearray(64 * row_bytes)
    for wave in range(waves):
        voff = []
        for q in range(2):
            lin = (wave * b_instr + q) * 1024
            row = lin // row_bytes
            voff.append([(row + (lane * 16) // row_bytes, ((lin % row_bytes + lane * 16) % row_bytes) >> 4)
                         for lane in range(64)])
        for q in range(b_instr):
            for lane in range(64):
                lin = (wave * b_instr + q) * 1024 + lane * 16
                row, pchunk = lin // row_bytes, (lin % row_bytes) >> 4
                # kernel: vector offset of parity q & 1 plus 2 * RPI * (q >> 1) rows
                r0, c0 = voff[q & 1][lane]
                grow = r0 + 2 * rpi * (q >> 1)
                gchunk = c0 ^ swz_b8_mi16(r0, row_bytes)
                assert grow == row and gchunk == pchunk ^ swz_b8_mi16(row, row_bytes)
                for b in range(16):
                    n = gchunk * 16 + b
                    key[lin + b] = (grow, n)
    assert len(key) == 64 * row_bytes and len(set(key.values())) == 64 * row_bytes
    # encode (k, n) as an index into a table instead of bytes
    ids = {kn: idx for idx, kn in enumerate(sorted(key.values()))}
    cells = [0] * (64 * row_bytes)
    for addr, kn in key.items():
        cells[addr] = ids[kn]
    inv = {v: k for k, v in ids.items()}
    wtn = 128 if row_bytes == 256 else 64
    for wn in range(row_bytes // wtn):
        for j in range(wtn // 16):
            for t in range(2):
                addrs = mi16_b_read_addrs(row_bytes, wn * wtn, j, t)
                for lane in range(64):
                    base, i = lane & ~15, lane & 15
                    got = [inv[cells[addrs[base + 2 * r + (i >> 3)] + (i & 7)]] for r in range(8)]
                    g = lane >> 4
                    assert got == [(16 * g + 8 * t + r, wn * wtn + 16 * j + i) for r in range(8)]


def load_schedule_mi16(na: int, nb: int, ai: int, bi: int, split_a: bool = False) -> tuple[int, int, int]:
    """The waits gemm_fp8_mi16_kernel derives (load_schedule_mi16): prologue, odd steps, even steps.
    A loads of step v: all ai of pair v // 2 + na - 1 on even v, or (split_a) ai // 2 of pair
    v // 2 + na - 1 on every step."""
    steps = 64
    end_a: dict[int, int] = {}
    end_b: dict[int, int] = {}
    before: dict[int, int] = {}
    total = 0

    def a_step(v: int) -> None:
        nonlocal total
        pair = v // 2 + na - 1
        if pair < 0 or (not split_a and v % 2):
            return
        total += ai // 2 if split_a else ai
        end_a[pair] = total

    for v in range(-max(nb + 1, 2 * na - 2), 0):
        a_step(v)
        if 0 <= v + 1 + nb < nb:
            total += bi
            end_b[v + 1 + nb] = total
    prologue = total - max(end_a[0], end_b[0], end_b[1])
    total += bi
    end_b[nb] = total
    for k in range(steps):
        before[k] = total
        a_step(k)
        total += bi
        end_b[k + 1 + nb] = total
    waits = {0: 1 << 20, 1: 1 << 20}
    for j in range(steps - 2):
        w = before[j] - max(end_a[(j + 1) // 2], end_b[j + 2])
        waits[j & 1] = min(waits[j & 1], w)
    return prologue, waits[1], waits[0]


def simulate_ring_mi16(na: int, nb: int, ai: int, bi: int, ksteps: int,
                       waits: tuple[int, int, int] | None = None, split_a: bool = False) -> None:
    """Event-level model of the fp8 16x16x128 ring: loads land in issue order; B stage S is read
    during step S - 2 (stages 0, 1 in the prologue), A pair P during steps 2P - 1 .. 2P + 1 (pair 0
    from the prologue on). Checks every read sees its stage / pair, with no load pending or issued
    into a slot while it is read, and that every load targets a slot whose reads are over."""
    assert ksteps % 2 == 0
    prologue, odd, even = waits or load_schedule_mi16(na, nb, ai, bi, split_a)
    assert 0 <= prologue < 64 and 0 <= odd < 64 and 0 <= even < 64
    last, last_pair = ksteps - 1, ksteps // 2 - 1
    a_per_step = ai // 2 if split_a else ai
    issued: list[tuple[str, int, int]] = []
    b_last_read = lambda s: max(s - 2, -1)          # step index; -1 = prologue
    a_last_read = lambda p: 2 * p + 1
    b_in_slot: dict[int, int] = {}
    a_in_slot: dict[int, int] = {}

    def issue(kind: str, idx: int, slot: int, n: int, now: int) -> None:
        # the slot's previous occupant must be read completely before step `now` (its barrier)
        prev = (b_in_slot if kind == "B" else a_in_slot).get(slot)
        if prev is not None:
            done = b_last_read(prev) if kind == "B" else a_last_read(prev)
            assert done < now, (kind, idx, slot, prev, now)
        (b_in_slot if kind == "B" else a_in_slot)[slot] = idx
        issued.extend([(kind, idx, slot)] * n)

    def check(wait: int, b_stages: list[int], a_pairs: list[int], ctx) -> None:
        done, pending = issued[:len(issued) - wait], issued[len(issued) - wait:]
        content: dict[tuple[str, int], int] = {}
        for kind, idx, slot in done:
            content[(kind, slot)] = idx
        pend = {(k, s) for k, _, s in pending}
        for s in b_stages:
            if s <= last:
                assert content.get(("B", s % nb)) == s, (ctx, "B", s)
                assert ("B", s % nb) not in pend, (ctx, "B pending", s)
        for p in a_pairs:
            if p <= last_pair:
                assert content.get(("A", p % na)) == p, (ctx, "A", p)
                assert ("A", p % na) not in pend, (ctx, "A pending", p)

    def issue_a_step(v: int, now: int) -> None:
        p = v // 2 + na - 1
        if p >= 0 and (split_a or v % 2 == 0):
            if split_a and v % 2:      # second half: the slot already holds this pair
                issued.extend([("A", min(p, last_pair), p % na)] * a_per_step)
            else:
                issue("A", min(p, last_pair), p % na, a_per_step, now)

    V = max(nb + 1, 2 * na - 2)
    for v in range(-V, 0):
        issue_a_step(v, -2)
        if 0 <= v + 1 + nb < nb:
            s = v + 1 + nb
            issue("B", min(s, last), s % nb, bi, -2)
    check(prologue, [0, 1], [0], "prologue")
    issue("B", min(nb, last), 0, bi, 0)                 # after the prologue's barrier
    for k in range(ksteps):
        reads_a = [k // 2] + ([k // 2 + 1] if k % 2 else [])
        check(odd if k % 2 else even, [k + 2], reads_a, ("step", k))
        n_before = len(issued)
        issue_a_step(k, k)
        s = k + 1 + nb
        issue("B", min(s, last), s % nb, bi, k)
        for kind, idx, slot in issued[n_before:]:        # nothing lands in a slot read this step
            if kind == "B":
                assert slot != (k + 2) % nb or k + 2 > last
            else:
                assert all(slot != p % na for p in reads_a if p <= last_pair)


# (A pair slots, B stage slots, A loads per wave per pair, B loads per wave per stage): 256x256,
# 128x256, 128x128 and 64x128 tiles; steady-state waits allow the loads of the two previous steps pending.
MI16_CONFIGS = [(3, 4, 8, 4), (3, 6, 4, 4), (3, 6, 4, 2), (3, 6, 2, 2)]
MI16_WAITS = [(16, 16, 16), (16, 16, 20), (10, 10, 12), (8, 8, 10)]
MI16_WAITS_SPLIT_A = [(16, 12, 16), (12, 10, 16), (8, 6, 10), (6, 5, 8)]


@pytest.mark.parametrize("split_a", [False, True])
@pytest.mark.parametrize("cfg", MI16_CONFIGS)
def test_mi16_ring_schedule_is_safe_for_every_k_length(cfg, split_a):
    for ksteps in list(range(2, 42, 2)) + [64, 128, 256]:
        simulate_ring_mi16(*cfg, ksteps, split_a=split_a)


def test_mi16_ring_waits_of_the_configurations():
    assert [load_schedule_mi16(*c) for c in MI16_CONFIGS] == MI16_WAITS
    assert [load_schedule_mi16(*c, split_a=True) for c in MI16_CONFIGS] == MI16_WAITS_SPLIT_A


@pytest.mark.parametrize("split_a", [False, True])
@pytest.mark.parametrize("loosen", [(1, 0, 0), (0, 1, 0), (0, 0, 1)])
def test_mi16_simulation_catches_a_wait_one_load_too_loose(loosen, split_a):
    prologue, odd, even = load_schedule_mi16(3, 4, 8, 4, split_a)
    waits = (prologue + loosen[0], odd + loosen[1], even + loosen[2])
    with pytest.raises(AssertionError):
        simulate_ring_mi16(3, 4, 8, 4, 16, waits, split_a=split_a)


def test_b_swizzles_of_narrow_rows_permute_within_the_row():
    # chunk c of B row k sits at chunk c ^ f(k): f must keep every chunk inside its row
    for k in range(4):
        assert sorted(c ^ swz_b16_128(k) for c in range(8)) == list(range(8))      # 128-byte 16-bit rows
    for k in range(8):
        assert sorted(c ^ swz_b8_64(k) for c in range(4)) == list(range(4))        # 64-byte fp8 rows
