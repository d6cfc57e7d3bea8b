"""Host emulation of the W8A8 GEMV kernels' index mapping (no GPU).

Restates, for every launch shape the library picks, how
``w8a8_gemv_nk_kernel`` and ``w8a8_gemv_k4n_kernel`` (qxt_w8a8.hip) address
the fp32 row, the LDS activation rows and the weight, and checks that

* the fused row load (``load_row``: thread t, register chunk u reads 16-byte
  chunk t + u * NT) and the in-workgroup quantisation write every 4-byte word
  of every activation row exactly once;
* the [N, K] kernel's four-slot ring (slot d of lane l holds chunk
  c0 + 64 d, c0 = l, l + 256, ...; reloaded with chunk c + 256 after use)
  reduces every 16-byte chunk of K exactly once per column, each from the
  slot that was loaded with it, and reads LDS only inside [MR][K / 16];
* the K4N kernel's four waves split the K / 4 words without gap or overlap;
* every in-range buffer offset stays inside the descriptor range the
  launcher sets, so the out-of-range sentinel is the only way past it.

The shapes mirror ``launch_gemv`` / ``qxt_w8a8_linear``: fused rows for
M <= 4 when MR * K <= 60 KiB and K <= 16384; [N, K] weights on 512-thread
workgroups with RC = 4 (K <= 8192) or 8; K4N weights on 256 threads with RC
= 4, 8 or 16 (K <= 4096, 8192, 16384).
"""

from __future__ import annotations

import numpy as np
import pytest

LDS_LIMIT = 60 * 1024
FUSED_MAX_K = 16384


def fused_shape(m: int, k: int, layout: str) -> tuple[int, int, int] | None:
    """(MR, RC, NT) of the fused GEMV launch, or None when the two-kernel path runs."""
    mr = m if m <= 2 else 4
    if m > 4 or mr * k > LDS_LIMIT or k > FUSED_MAX_K:
        return None
    if layout == "nk":
        return mr, (4 if k <= 4 * 4 * 512 else 8), 512
    return mr, (4 if k <= 4 * 4 * 256 else 8 if k <= 8 * 4 * 256 else 16), 256


def row_words_written(k: int, rc: int, nt: int) -> np.ndarray:
    """How many times the fused quantiser writes each 4-byte word of one row."""
    k4 = k // 4
    hits = np.zeros(k4, np.int64)
    for t in range(nt):
        for u in range(rc):
            c = t + u * nt
            if c >= k4:
                break
            hits[c] += 1
    return hits


def nk_chunks_reduced(k: int) -> tuple[np.ndarray, int]:
    """Per lane, emulate the ring: how often each 16-byte chunk is reduced, and the largest LDS chunk read."""
    k16 = k // 16
    depth = 4
    hits = np.zeros(k16, np.int64)
    max_lds = -1
    for lane in range(64):
        ring = [lane + 64 * d for d in range(depth)]  # the chunk each slot was loaded with (>= k16: zeros)
        c0 = lane
        while c0 < k16:
            for d in range(depth):
                c = c0 + 64 * d
                if c < k16:
                    assert ring[d] == c, (k, lane, c0, d)
                    hits[c] += 1
                    max_lds = max(max_lds, c)
                ring[d] = c + 64 * depth
            c0 += 64 * depth
    return hits, max_lds


KS = sorted({16, 32, 48, 1024, 2048, 2064, 4096, 4112, 5632, 8192, 8208, 12288, 14336, 15360, 16368, 16384}
            | set(range(16, 16385, 16 * 37)))


@pytest.mark.parametrize("layout", ["nk", "k4n"])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_fused_rows_cover_every_word_once(layout: str, m: int) -> None:
    for k in KS:
        shape = fused_shape(m, k, layout)
        if shape is None:
            continue
        mr, rc, nt = shape
        hits = row_words_written(k, rc, nt)
        assert np.all(hits == 1), (layout, m, k, rc, nt)
        # The register chunks hold the whole row: RC * NT * 4 words >= K / 4.
        assert rc * nt * 4 >= k


def test_fused_path_limits() -> None:
    # The widest fused rows sit exactly on the register capacity of each shape.
    assert fused_shape(1, 16384, "nk") == (1, 8, 512) and 8 * 512 * 4 == 16384
    assert fused_shape(1, 16384, "k4n") == (1, 16, 256) and 16 * 256 * 4 == 16384
    assert fused_shape(4, 15360, "nk") == (4, 8, 512)
    assert fused_shape(4, 15376, "nk") is None  # 4 rows of K > 15360 exceed 60 KiB of LDS
    assert fused_shape(1, 16400, "nk") is None
    assert fused_shape(5, 64, "nk") is None


def test_nk_ring_reduces_every_chunk_once_from_its_own_slot() -> None:
    for k in KS:
        hits, max_lds = nk_chunks_reduced(k)
        assert np.all(hits == 1), k  # each chunk once, by one lane, for every column of the wave
        assert max_lds == k // 16 - 1


@pytest.mark.parametrize("m", [1, 2, 4])
def test_nk_offsets_stay_inside_the_descriptors(m: int) -> None:
    # Weight [N, K] with row stride ldw >= K: the last in-range load of the
    # last column ends exactly at w_bytes = (N - 1) ldw + K.  Activation rows
    # (fp32, stride ldx >= 4 K): x_bytes = (M - 1) ldx + 4 K.  LDS rows:
    # index r * K / 16 + c < MR * K / 16 chunks = the dynamic MR * K bytes.
    for k in (16, 2048, 8208, 14336, 16384):
        for n, extra in ((16, 0), (4096, 16), (4100, 48)):
            ldw = k + extra
            w_bytes = (n - 1) * ldw + k
            last = (n - 1) * ldw + (k // 16 - 1) * 16 + 16
            assert last == w_bytes
            ldx = 4 * k + 64
            x_bytes = (m - 1) * ldx + 4 * k
            # Row r of the fused load reads 16-byte chunks c < K / 4 at r * ldx + 16 c:
            # the last one ends at r * ldx + 4 K.
            assert (m - 1) * ldx + 16 * (k // 4 - 1) + 16 == x_bytes
            mr = m if m <= 2 else 4
            assert (mr - 1) * (k // 16) + (k // 16 - 1) < mr * k // 16


def test_k4n_waves_split_k_without_gap_or_overlap() -> None:
    for k in KS:
        k4 = k // 4
        per = (k4 + 3) // 4
        hits = np.zeros(k4, np.int64)
        for wave in range(4):
            q0, q1 = wave * per, min(k4, wave * per + per)
            for q in range(q0, q1):
                hits[q] += 1
        assert np.all(hits == 1), k


def gemv_cols_nk(nt: int) -> int:
    """Output columns per [N, K] GEMV workgroup: 8 (one per wave) at 512 threads, else 16."""
    return 8 if nt == 512 else 16


@pytest.mark.parametrize("nt", [256, 512])
def test_nk_columns_cover_every_output_once(nt: int) -> None:
    # Workgroup b, wave w, slot j owns column b * cols + w * CPW + j; the grid
    # has ceil(N / cols) workgroups and columns >= N read and write nothing.
    cols = gemv_cols_nk(nt)
    cpw = cols // (nt // 64)
    assert cpw * (nt // 64) == cols and cpw >= 1
    for n in (1, 7, 8, 16, 17, 256, 4096, 4100, 14336):
        hits = np.zeros(n, np.int64)
        for b in range(-(-n // cols)):
            for w in range(nt // 64):
                for j in range(cpw):
                    c = b * cols + w * cpw + j
                    if c < n:
                        hits[c] += 1
        assert np.all(hits == 1), (nt, n)
