"""Host emulation of the persistent W8A8 GEMV's launch and index mapping (no GPU).

Restates ``launch_gemv_stream`` and ``w8a8_gemv_nk_stream_kernel``
(qxt_w8a8.hip) and checks, for the shapes the library sends there:

* the launch: two (fused rows) or three (int8 rows) 512-thread workgroups per
  CU, fewer when the rows' LDS would not fit 160 KB, at most one workgroup per
  eight columns; one row fused takes this form from two columns per wave, and
  no problem of more than 64 columns per wave does;
* every column is owned by exactly one wave (wave gw takes gw, gw + W, ...)
  and each workgroup holds the same number of columns to within eight;
* the ring: the load issued for step t (column t // chunks of the wave,
  kilobyte t % chunks) is the one step t reduces, D steps later, so the
  incrementally advanced issue pointer never drifts from the consumer;
* lane l of kilobyte i reads 16-byte chunk l + 64 i: every chunk of K once,
  LDS reads inside [MR][K / 16], weight offsets inside the descriptor range;
* the final stores: lane j < ncols stores column gw + j * W, every column once.
"""

from __future__ import annotations

import numpy as np
import pytest

NT = 512
WAVES_PER_WG = NT // 64
LDS_PER_CU = 160 * 1024


def launch(m: int, n: int, k: int, cus: int, fused: bool):
    """(workgroups, ring depth) of the persistent form, or None when the one-column kernels run."""
    mr = m if m <= 2 else 4
    depth, per_cu_req = (4, 2) if fused else (3, 3)
    lds = mr * k
    per_cu = max(1, min(per_cu_req, LDS_PER_CU // (lds + 1024)))
    wgs = min(per_cu * cus, -(-n // WAVES_PER_WG))
    waves = wgs * WAVES_PER_WG
    min_cols = (2 if fused else 0) if mr == 1 else 0
    if n < min_cols * waves or n > 64 * waves:
        return None
    return wgs, depth


def emulate(m: int, n: int, k: int, ldw: int, cus: int, fused: bool) -> dict:
    shape = launch(m, n, k, cus, fused)
    assert shape is not None
    wgs, depth = shape
    waves = wgs * WAVES_PER_WG
    k16 = k // 16
    chunks = -(-k16 // 64)
    w_bytes = (n - 1) * ldw + k
    owner = np.full(n, -1, np.int64)
    stored = np.zeros(n, np.int64)
    per_wg = np.zeros(wgs, np.int64)
    max_cols = 0
    for wave in range(WAVES_PER_WG):
        for block in range(wgs):
            gw = wave * wgs + block
            ncols = -(-(n - gw) // waves) if gw < n else 0
            max_cols = max(max_cols, ncols)
            total = ncols * chunks
            # Issue pointer, advanced once per issued load, D loads ahead.
            icol, ichunk = gw, 0
            issued = {}
            def issue(t):
                nonlocal icol, ichunk
                issued[t] = (icol, ichunk) if t < total else None
                ichunk += 1
                if ichunk == chunks:
                    ichunk = 0
                    icol += waves
            for d in range(depth):
                issue(d)
            col, chunk = gw, 0
            for t0 in range(0, total, depth):
                for d in range(depth):
                    t = t0 + d
                    if t < total:
                        assert issued[t] == (col, chunk), (gw, t)
                        chunk += 1
                        if chunk == chunks:
                            chunk = 0
                            col += waves
                    issue(t0 + d + depth)
            for j in range(ncols):
                c = gw + j * waves
                assert c < n
                assert owner[c] == -1
                owner[c] = gw
                stored[c] += 1
                # largest in-range weight offset of the column: its last 16-byte chunk
                assert c * ldw + (k16 - 1) * 16 + 16 <= w_bytes
            per_wg[block] += ncols
    return {"owner": owner, "stored": stored, "per_wg": per_wg, "max_cols": max_cols, "chunks": chunks}


def lane_chunks(k: int) -> np.ndarray:
    """How often lanes 0..63 over kilobytes 0..chunks-1 reduce each 16-byte chunk of K."""
    k16 = k // 16
    chunks = -(-k16 // 64)
    hits = np.zeros(k16, np.int64)
    for i in range(chunks):
        for lane in range(64):
            c = lane + 64 * i
            if c < k16:
                hits[c] += 1
    return hits


SHAPES = [
    # m, n, k, fused
    (1, 14336, 4096, True),    # cfg4 gate_up at M = 1
    (1, 11008, 4096, True),
    (1, 16384, 2048, True),
    (1, 8192, 16, True),
    (1, 8195, 4112, True),
    (1, 20000, 16384, True),
    (2, 100, 4096, True),
    (2, 4096, 14336, True),
    (2, 3000, 4112, True),
    (2, 520, 16384, True),
    (1, 14336, 4096, False),
    (1, 7, 16, False),
    (3, 5000, 4096, False),
    (4, 4096, 14336, False),
    (2, 12288, 8208, False),
    (4, 14336, 4096, False),
]


@pytest.mark.parametrize("cus", [256, 80])
@pytest.mark.parametrize("m,n,k,fused", SHAPES)
def test_persistent_gemv_covers_every_column_and_chunk_once(m: int, n: int, k: int, fused: bool, cus: int) -> None:
    if launch(m, n, k, cus, fused) is None:
        pytest.skip("the one-column kernels take this shape on this many CUs")
    r = emulate(m, n, k, ldw=k + 16 * (n % 3), cus=cus, fused=fused)
    assert (r["owner"] >= 0).all() and (r["stored"] == 1).all()
    assert r["max_cols"] <= 64
    assert r["per_wg"].max() - r["per_wg"].min() <= WAVES_PER_WG
    hits = lane_chunks(k)
    assert (hits == 1).all()
    mr = m if m <= 2 else 4
    # LDS reads: row r < MR, chunk c < K / 16 inside [MR][K / 16].
    assert (mr - 1) * (k // 16) + (k // 16 - 1) < mr * (k // 16)


@pytest.mark.parametrize("cus", [256, 80])
def test_persistent_gemv_launch_boundaries(cus: int) -> None:
    waves = 2 * cus * WAVES_PER_WG
    # One fused row: from two columns per wave.
    assert launch(1, 2 * waves - 1, 4096, cus, True) is None
    assert launch(1, 2 * waves, 4096, cus, True) is not None
    # More than 64 columns per wave: the one-column kernels.
    assert launch(1, 64 * waves, 16, cus, True) is not None
    assert launch(1, 64 * waves + 1, 16, cus, True) is None
    unfused = 3 * cus * WAVES_PER_WG
    assert launch(4, 64 * unfused, 16, cus, False) is not None
    assert launch(4, 64 * unfused + 1, 16, cus, False) is None
    # Four rows of 14336 bytes: two workgroups per CU fit 160 KB of LDS, not three.
    assert launch(4, 4096, 14336, cus, False)[0] == min(2 * cus, 4096 // 8)
