"""The pair layout of the compiled forward and dQ kernels at head dims <= 64
(ra_kernels.hip: DirectLoader<..., Pair = true>, the kPair fragment indexing
of fwd_kernel and dq_kernel), restated on the host: a 128-row tile in one
64-row XOR tile, key row R at physical row R % 64, chunks 8 (R / 64) + 0..7.

Checks that the copy slots fill every (row, data chunk) of the 128 rows
exactly once, and that the row-fragment reads (k-step ks + 4 for rows
64-127) and the transposed reads (d block db + 2) find the data the MFMAs
expect, for every key block, step and lane; and that both read patterns
still hit 16 distinct 4-byte bank groups per 16 lanes.  A planted mistake
(the second half at k-step offset 2 instead of 4) fails the check."""


def swz(r):
    return ((r & 3) << 2) | ((r >> 2) & 3)


def copy_map():
    """(key row, data chunk) -> (physical row, physical chunk position) from
    the copy slots: slot s of a tile lands at row s // 16, position s % 16,
    and holds logical chunk (s % 16) ^ swz(row)."""
    pos = {}
    for s in range(64 * 16):
        r, c = s >> 4, (s & 15) ^ swz(s >> 4)
        key = (r + 64 * (c >> 3), c & 7)
        assert key not in pos
        pos[key] = (r, s & 15)
    return pos


def row_reads(ks_half=4):
    """Row fragments of the S phase: key block kb (32 keys), k-step ks, lane:
    physical (row, position) read and the (key, data chunk) it must hold."""
    for kb in range(4):
        for ks in range(4):
            for lane in range(64):
                l32, g = lane & 31, lane >> 5
                ksp = ks + ks_half * (kb >> 1)
                yield (kb & 1) * 32 + l32, (2 * ksp) ^ (g ^ swz(l32)), kb * 32 + l32, 2 * ks + g, lane


def tr_reads(db_half=2):
    """Transposed fragments of the O (dQ) phase: 16-key step ks2, d block db,
    lane, half hh."""
    for ks2 in range(8):
        for db in range(2):
            for hh in range(2):
                for lane in range(64):
                    g, j, s, m = lane >> 5, lane >> 4, (lane >> 2) & 3, lane & 3
                    cl = 2 * (j & 1) + (m >> 1)
                    row = 8 * hh + 4 * g + s
                    dbp = db + db_half * (ks2 // 4)
                    yield (ks2 % 4) * 16 + row, (4 * dbp + cl) ^ swz(row), 16 * ks2 + row, 4 * db + cl, lane


def _consistent(ks_half=4, db_half=2):
    pos = copy_map()
    for prow, ppos, key, chunk, _ in row_reads(ks_half):
        if pos.get((key, chunk)) != (prow, ppos):
            return False
    for prow, ppos, key, chunk, _ in tr_reads(db_half):
        if pos.get((key, chunk)) != (prow, ppos):
            return False
    return True


def test_copy_slots_cover_the_128_rows_once():
    assert len(copy_map()) == 128 * 8


def test_reads_find_the_copied_data():
    assert _consistent()


def test_planted_offset_fails():
    assert not _consistent(ks_half=2)
    assert not _consistent(db_half=1)


def test_reads_stay_conflict_free():
    # an LDS row of the tile is 256 bytes, one pass over the 64 four-byte
    # banks, so a 16-byte position p holds banks 4p .. 4p + 3 in every row.
    # ds_read_b128 serves 16 lanes (256 bytes) per cycle: their positions
    # must be distinct.
    by_instr = {}
    for prow, ppos, key, chunk, lane in row_reads():
        by_instr.setdefault((key // 32, chunk >> 1, lane >> 4), []).append(ppos)
    assert len(by_instr) == 4 * 4 * 4
    for pos in by_instr.values():
        assert sorted(pos) == list(range(16))
    # ds_read_b64_tr_b16 serves 32 lanes (8 bytes each) per cycle: their
    # (position, 8-byte half) units must be distinct
    by_tr = {}
    for ks2 in range(8):
        for db in range(2):
            for hh in range(2):
                for lane in range(64):
                    g, j, s_, m = lane >> 5, lane >> 4, (lane >> 2) & 3, lane & 3
                    cl = 2 * (j & 1) + (m >> 1)
                    row = 8 * hh + 4 * g + s_
                    ppos = (4 * (db + 2 * (ks2 // 4)) + cl) ^ swz(row)
                    by_tr.setdefault((ks2, db, hh, g), []).append((ppos, m & 1))
    for units in by_tr.values():
        assert len(set(units)) == 32
