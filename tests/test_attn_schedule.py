"""Host model of the attention kernels' barrier and LDS-ring schedule.

``sage_attn_kernel`` (csrc/sage_attn.hip) and ``w8a8_attn_kernel``
(csrc/w8a8_attn.hip, 4 loads per tile instead of 6) run 8 waves in two groups that
share one workgroup barrier per key tile.  Group 0 issues a tile's loads
between its MFMA and softmax clusters.  The model also covers issuing them
after the softmax, an order the W8A8 kernel once used.  Every wave executes, per tile t,
an MFMA cluster M_t = {QK(t + 1), PV(t)} and a softmax cluster V_t; group 0
orders an interval as [M_t, V_{t+1}], group 1 as [V_t, M_t], so the two
groups' MFMA clusters overlap on each SIMD.  Group 0 alone streams the K and
V^T tiles into a ring of kStages LDS stages, kAhead tiles ahead, and waits on
its own load counter before a barrier.

This model replays, wave by wave, the same loops, bounds and counts as the
kernel (non-causal and causal, ragged tails, waves past the causal diagonal)
and checks what the GPU cannot be allowed to get wrong:
  * every wave executes the same number of barriers (a mismatch hangs);
  * every LDS stage a cluster reads holds the tile it expects, resident
    (its loads waited for before the barrier that opens the interval);
  * no stage is reloaded while any wave may still read it (no load into a
    stage in the interval of, or between the issue and, a read of another
    tile from it);
  * each softmax consumes the scores of the QK it follows and each PV the
    P of the softmax of the same tile, in order.
"""
from __future__ import annotations

import itertools

import pytest

K_STAGES = 4
K_AHEAD = K_STAGES - 1
# per kernel: 1 KiB blocks a group-0 wave loads per tile (Sage head_dim 128:
# 2 K + 4 V^T, Sage head_dim 64: 1 K + 2 V^T, W8A8 2 K + 2 V^T), and whether
# it issues them after the softmax
KERNELS = {"sage": (6, False), "sage64": (3, False), "w8a8": (4, False), "w8a8_after": (4, True)}
KBKEY = 64
KBQ = 256
KWAVEQ = 32


class Wave:
    def __init__(self, wave: int):
        self.wave = wave
        self.grp = wave >> 2
        self.events = []  # (kind, payload) in program order
        self.tile_base = 0  # global index of local tile 0 (key splits)

    def barrier(self):
        self.events.append(("barrier", None))

    def issue(self, stage, tile):
        self.events.append(("issue", (stage, tile)))

    def wait(self, n):
        self.events.append(("wait", n))

    def qk(self, stage, tile):
        self.events.append(("read", (stage, tile, "K")))
        self.events.append(("qk", tile))

    def pv(self, stage, tile):
        self.events.append(("read", (stage, tile, "V")))
        self.events.append(("pv", tile))

    def softmax(self, tile, masked):
        self.events.append(("softmax", (tile, masked)))


def split_plan(lk: int, kv_splits: int):
    """tu_sage_attn_fwd_split's ranges: split_tiles = ceil(tiles / kv_splits)
    and the number of ranges that covers the key tiles."""
    tiles = (lk + KBKEY - 1) // KBKEY
    split_tiles = (tiles + kv_splits - 1) // kv_splits
    return split_tiles, (tiles + split_tiles - 1) // split_tiles


def kernel_program(wave: int, lq: int, lk: int, causal: bool, qblock: int, kernel: str = "sage",
                   split_z: int | None = None, split_tiles: int = 0) -> Wave:
    """The kernel's control flow for one wave, statement for statement.
    split_z / split_tiles model the kSplit instantiation (blockIdx.z and its
    key range); tiles are then numbered from the range's first tile, and the
    loads carry global tile indices."""
    LOADS_PER_TILE, issue_late = KERNELS[kernel]
    w = Wave(wave)
    grp, w4 = wave >> 2, wave & 3
    qblock0 = qblock * KBQ
    q0 = qblock0 + grp * (KBQ // 2) + w4 * KWAVEQ
    key_end = min(lk, qblock0 + KBQ) if causal else lk
    tile_base = split_z * split_tiles if split_z is not None else 0
    tiles = (key_end + KBKEY - 1) // KBKEY
    if split_z is not None:
        assert not causal
        tiles = min(split_tiles, tiles - tile_base)
    my_tiles = tiles
    if causal:
        my_tiles = min(tiles, max(1, (min(q0 + KWAVEQ, lq) + KBKEY - 1) // KBKEY))
    mask_from = lk // KBKEY - tile_base
    if causal:
        mask_from = min(mask_from, q0 // KBKEY)
    first_masked = min(tiles, mask_from)
    tile_key0 = lambda it: tile_base + min(it, tiles - 1)  # noqa: E731  (global tile index the load reads)

    def softmax(it, mask_tag):
        if not mask_tag:
            assert it < first_masked, "unmasked softmax on a tile that needs a mask"
        w.softmax(it, mask_tag and it >= first_masked)

    w.tile_base = tile_base
    if grp == 0:
        for j in range(K_AHEAD):
            w.issue(j, tile_key0(j))
        w.wait((K_AHEAD - 1) * LOADS_PER_TILE)
    w.barrier()
    # interval 0: QK(0) (and, group 0, softmax(0)); group 1 runs softmax(0)
    # right after the barrier
    w.qk(0, 0)
    main_steps = max(0, min(my_tiles, first_masked) - 1)
    if grp == 0:
        softmax(0, True)
        w.wait((K_AHEAD - 2) * LOADS_PER_TILE)
    w.barrier()
    if grp == 1:
        softmax(0, True)
    # intervals 1 .. main_steps: unmasked steady state; the same sequence for
    # both groups, group 1's barrier before the softmax, group 0's after
    for it in range(main_steps):
        w.qk((it + 1) % K_STAGES, it + 1)
        w.pv(it % K_STAGES, it)
        if grp == 0 and not issue_late:
            w.issue((it + K_AHEAD) % K_STAGES, tile_key0(it + K_AHEAD))
        if grp == 1:
            w.barrier()
        softmax(it + 1, False)
        if grp == 0:
            if issue_late:
                w.issue((it + K_AHEAD) % K_STAGES, tile_key0(it + K_AHEAD))
            w.wait((K_AHEAD - 2) * LOADS_PER_TILE)
            w.barrier()
    # remaining intervals: masked tiles, the last tile, causal tiles past the
    # wave's diagonal (barriers only)
    for it in range(main_steps, tiles):
        if grp == 0 and not issue_late:
            w.issue((it + K_AHEAD) % K_STAGES, tile_key0(it + K_AHEAD))
        if it + 1 < my_tiles:
            w.qk((it + 1) % K_STAGES, it + 1)
        if it < my_tiles:
            w.pv(it % K_STAGES, it)
        if grp == 1:
            w.barrier()
        if it + 1 < my_tiles:
            softmax(it + 1, True)
        if grp == 0:
            if issue_late:
                w.issue((it + K_AHEAD) % K_STAGES, tile_key0(it + K_AHEAD))
            w.wait((K_AHEAD - 2) * LOADS_PER_TILE)
            w.barrier()
    return w, dict(tiles=tiles, my_tiles=my_tiles)


def check_schedule(lq: int, lk: int, causal: bool, qblock: int, kernel: str = "sage",
                   split_z: int | None = None, split_tiles: int = 0):
    LOADS_PER_TILE = KERNELS[kernel][0]
    waves = [kernel_program(i, lq, lk, causal, qblock, kernel, split_z, split_tiles) for i in range(8)]
    progs = [w for w, _ in waves]
    # 1. equal barrier counts
    counts = [sum(1 for k, _ in p.events if k == "barrier") for p in progs]
    assert len(set(counts)) == 1, f"barrier counts differ: {counts}"
    n_intervals = counts[0] + 1  # interval i precedes barrier i
    # split each wave's events into intervals
    intervals = []
    for p in progs:
        cur, out = [], []
        for ev in p.events:
            if ev[0] == "barrier":
                out.append(cur)
                cur = []
            else:
                cur.append(ev)
        out.append(cur)
        assert len(out) == n_intervals
        intervals.append(out)
    # 2. loads: group 0 waves issue identical loads; model the loader's
    # outstanding queue (loads complete in issue order for the wait counter)
    loaders = [i for i in range(8) if progs[i].grp == 0]
    for i in loaders[1:]:
        assert [e for e in progs[i].events if e[0] in ("issue", "wait")] == \
               [e for e in progs[loaders[0]].events if e[0] in ("issue", "wait")]
    stage_content = {}  # stage -> (tile, resident_from_interval)
    outstanding = []  # [(stage, tile, ops_left)] in issue order
    resident_at = {}  # (stage, tile) -> first interval in which it may be read
    issued_in = {}  # (stage, tile) -> interval of issue
    reads = []  # (interval, wave, stage, tile)
    for k in range(n_intervals):
        for ev in intervals[loaders[0]][k]:
            kind, pay = ev
            if kind == "issue":
                stage, tile = pay
                outstanding.append([stage, tile])
                issued_in[(stage, tile, len(outstanding))] = k
                stage_content.setdefault(stage, [])
                stage_content[stage].append((tile, k))
            elif kind == "wait":
                # all but the most recent pay // LOADS_PER_TILE tiles complete
                keep = pay // LOADS_PER_TILE
                assert pay % LOADS_PER_TILE == 0
                while len(outstanding) > keep:
                    stage, tile = outstanding.pop(0)
                    resident_at.setdefault((stage, tile), k + 1)
        for wi in range(8):
            for kind, pay in intervals[wi][k]:
                if kind == "read":
                    stage, tile, _ = pay
                    reads.append((k, wi, stage, progs[wi].tile_base + tile))
    # 3. every read finds its tile resident and not overwritten
    for k, wi, stage, tile in reads:
        hist = stage_content.get(stage, [])
        # the most recent load into the stage issued before interval k
        before = [(t, ki) for t, ki in hist if ki < k]
        assert before, f"interval {k} wave {wi}: stage {stage} never loaded"
        t_last, k_last = before[-1]
        assert t_last == tile, f"interval {k} wave {wi}: stage {stage} holds tile {t_last}, expected {tile}"
        assert resident_at.get((stage, tile), 10 ** 9) <= k, \
            f"interval {k} wave {wi}: tile {tile} in stage {stage} not waited for"
        # no load into this stage during interval k (a concurrent overwrite)
        assert not any(ki == k and t != tile for t, ki in hist), \
            f"interval {k}: stage {stage} reloaded while wave {wi} reads tile {tile}"
    # 4. per-wave data flow: QK(t) -> softmax(t) -> PV(t), each once, in order
    for (p, info), wi in zip(waves, range(8)):
        seq = [(k, pay) for k, pay in p.events if k in ("qk", "softmax", "pv")]
        last_qk, last_sm, last_pv = -1, -1, -1
        for kind, pay in seq:
            if kind == "qk":
                assert pay == last_qk + 1 and last_sm == pay - 1
                last_qk = pay
            elif kind == "softmax":
                t = pay[0]
                assert t == last_sm + 1 and last_qk == t, (wi, kind, pay, last_qk)
                last_sm = t
            else:
                assert pay == last_pv + 1 and last_sm == pay
                last_pv = pay
        assert last_pv == info["my_tiles"] - 1 and last_sm == info["my_tiles"] - 1, (wi, info, last_pv)


@pytest.mark.parametrize("kernel", sorted(KERNELS))
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lk", [1, 2, 63, 64, 65, 127, 128, 129, 191, 256, 257, 300, 333, 511, 700, 1000, 32760])
def test_schedule_every_block(causal, lk, kernel):
    lq = lk if causal else max(lk, 300)
    nblk = (lq + KBQ - 1) // KBQ
    # non-causal: the schedule does not depend on the query block
    blocks = range(nblk) if causal else sorted({0, nblk - 1})
    for qblock in blocks:
        check_schedule(lq, lk, causal, qblock, kernel)


@pytest.mark.parametrize("kernel", sorted(KERNELS))
@pytest.mark.parametrize("lq,lk", list(itertools.product([1, 40, 129, 256, 257, 700], [1, 2, 64, 65, 151, 333])))
def test_schedule_ragged_pairs(lq, lk, kernel):
    for causal in (False, True):
        for qblock in range((lq + KBQ - 1) // KBQ):
            check_schedule(lq, lk, causal, qblock, kernel)


@pytest.mark.parametrize("kernel", ["sage", "sage64"])
@pytest.mark.parametrize("lk", [1024, 1025, 1087, 1100, 2048, 4095, 8190, 32760])
@pytest.mark.parametrize("kv_splits", [2, 3, 4, 5, 8])
def test_schedule_key_splits(lk, kv_splits, kernel):
    """The kSplit instantiation: every key range tu_sage_attn_fwd_split forms
    (tile offsets, a truncated last range, mask_from shifted by the range's
    first tile) keeps equal barrier counts and ring residency."""
    tiles = (lk + KBKEY - 1) // KBKEY
    if kv_splits > tiles:
        pytest.skip("more ranges than key tiles")
    split_tiles, splits = split_plan(lk, kv_splits)
    covered = []
    for z in range(splits):
        lq = 300
        for qblock in range((lq + KBQ - 1) // KBQ):
            check_schedule(lq, lk, False, qblock, kernel, z, split_tiles)
        w, info = kernel_program(0, 300, lk, False, 0, kernel, z, split_tiles)
        covered += [z * split_tiles + t for t in range(info["my_tiles"])]
    assert covered == list(range(tiles)), "key ranges must cover every tile exactly once"


# --- K tile loads: the byte range each lane's buffer load touches ----------
# The loads are raw buffer loads over [kp, kp + lk * k_sl) with the tile's key
# offset in the per-lane offset (the part the range check covers) and a zero
# scalar offset; a lane whose offset is at or past the range end reads zeros.


def kperm_sage(p: int) -> int:
    i, kt = p & 15, (p >> 4) & 1
    return (p & ~31) + 8 * (i >> 2) + 4 * kt + (i & 3)


def kperm_w8a8(p: int) -> int:
    i, kt = p & 15, p >> 4
    return 16 * (i >> 2) + 4 * kt + (i & 3)


def k_load_offsets(kernel: str, k_sl: int):
    """(row, per-lane offset relative to key0's row) of every group-0 lane's K
    loads: lane_geom / lane_geom8's k_src."""
    out = []
    for w4 in range(4):
        for lane in range(64):
            if kernel == "sage64":
                row = w4 * 16 + (lane >> 2)
                out.append((kperm_sage(row), kperm_sage(row) * k_sl + ((lane & 3) ^ ((row >> 2) & 3)) * 16))
                continue
            for i in range(2):
                row = (2 * w4 + i) * 8 + (lane >> 3)
                perm = kperm_sage(row) if kernel == "sage" else kperm_w8a8(row)
                out.append((perm, perm * k_sl + ((lane & 7) ^ ((row >> 1) & 7)) * 16))
    return out


@pytest.mark.parametrize("kernel", sorted(KERNELS))
@pytest.mark.parametrize("lk", [1, 2, 63, 64, 65, 100, 127, 129, 333, 1000, 8190])
@pytest.mark.parametrize("layout", ["HND", "NHD3"])
@pytest.mark.parametrize("kv_splits", [1, 3])
def test_k_loads_stay_in_bounds(kernel, lk, layout, kv_splits):
    """Every K byte a lane reads lies in a visible key row of its own head
    (row < lk, bytes within head_dim), or the lane's offset is at or past the
    buffer range end, so it reads zeros.  NHD3: three kv heads interleaved, the
    last head's rows end at the allocation's end."""
    d = 64 if kernel == "sage64" else 128
    nh = 3 if layout == "NHD3" else 1
    k_sl = nh * d
    head_off = (nh - 1) * d  # the last head: its rows end at the allocation end
    alloc_end = lk * k_sl  # bytes of the K tensor
    rng = lk * k_sl  # buffer range from the head's base
    splits = [(None, 0)]
    if kv_splits > 1 and not kernel.startswith("w8a8") and (lk + KBKEY - 1) // KBKEY >= kv_splits:
        st, n = split_plan(lk, kv_splits)
        splits = [(z, st) for z in range(n)]
    offs = k_load_offsets(kernel, k_sl)
    for z, st in splits:
        prog, info = kernel_program(0, 300, lk, False, 0, kernel, z, st)
        for kind, pay in prog.events:
            if kind != "issue":
                continue
            key0 = pay[1] * KBKEY
            for perm, off in offs:
                voff = off + key0 * k_sl
                assert voff < 2 ** 32
                if voff >= rng:
                    continue  # out of range: zero-filled
                key = key0 + perm
                assert key < lk, f"key {key} past lk {lk} read from memory"
                chunk = voff - key * k_sl
                assert 0 <= chunk and chunk + 16 <= d
                assert head_off + voff + 16 <= alloc_end


def test_k_bound_model_catches_a_scalar_offset():
    """Planted mistake: with the key offset in the scalar offset (not range
    checked) a ragged last tile reads rows past lk."""
    lk, k_sl = 100, 128
    bad = False
    for perm, off in k_load_offsets("sage", k_sl):
        key0 = 64
        if off < lk * k_sl and key0 + perm >= lk:  # the check sees only `off`
            bad = True
    assert bad


@pytest.mark.parametrize("kernel", sorted(KERNELS))
def test_model_catches_a_missing_wait(kernel):
    """Planted mistake: loading one stage further ahead than the ring holds
    overwrites a stage that is still to be read."""
    global K_AHEAD
    saved = K_AHEAD
    try:
        K_AHEAD = 5
        with pytest.raises(AssertionError):
            check_schedule(1000, 1000, False, 0, kernel)
    finally:
        K_AHEAD = saved


# LDS layout of the W8A8 kernel's V^T blocks (lane_geom8 in csrc/w8a8_attn.hip):
# a loader lane writes its 16 bytes to position `lane` of a 1 KiB block (16
# channels x 64 keys), fetching channel 2 ((lane & 7) ^ g) + ((lane >> 3) & 1)
# and keys 16 g .. 16 g + 15 with g = lane >> 4; the PV reader (g, lc) wants
# channel lc, keys 16 g .., and reads position 16 g + 8 (lc & 1) + (g ^ (lc >> 1)).
def w8a8_v_dma_chunk(lane: int):
    g = lane >> 4
    return 2 * ((lane & 7) ^ g) + ((lane >> 3) & 1), g


def w8a8_v_read_pos(lane: int) -> int:
    g, lc = lane >> 4, lane & 15
    return 16 * g + 8 * (lc & 1) + (g ^ ((lc >> 1) & 7))


def sage_k_read_pos(lane: int, i: int) -> int:
    """16-byte position of the K read of chunk column 4 i + g (128-byte rows)."""
    g, lc = lane >> 4, lane & 15
    return 8 * lc + ((4 * i + g) ^ ((lc >> 1) & 7))


def test_w8a8_v_layout_is_consistent():
    """Every reader finds at its position the chunk a loader lane wrote
    there, and the 64 positions are a permutation of the block."""
    reads = [w8a8_v_read_pos(lane) for lane in range(64)]
    assert sorted(reads) == list(range(64))
    for lane in range(64):
        g, lc = lane >> 4, lane & 15
        assert w8a8_v_dma_chunk(reads[lane]) == (lc, g)


def test_w8a8_v_reads_spread_like_k_reads():
    """Each lane's V^T read falls on the same 16-byte slot modulo 256 bytes
    (the same banks) as its K read, a pattern the bank-conflict counter
    reads as zero; the plain 64-byte-row layout does not."""
    for lane in range(64):
        assert w8a8_v_read_pos(lane) % 16 == sage_k_read_pos(lane, 0) % 16

    def plain(lane):
        g, lc = lane >> 4, lane & 15
        return 4 * lc + (g ^ ((lc >> 2) & 3))

    assert any(plain(lane) % 16 != sage_k_read_pos(lane, 0) % 16 for lane in range(64))
