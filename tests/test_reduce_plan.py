"""The reductions' split plan as the partials-size query reports it
(tp_amd_reduce_partial_bytes, pure host arithmetic, no GPU): exact figures
for known splits, and the bound that keeps the allocation-free entry's
1 MiB static array sufficient on a 256-CU MI355X.

Why the bound holds: a row split writes outer * nseg partials with nseg
about 2 CUs / outer (at most 2 CUs + outer < 16 CUs floats); a column split
runs nchunk = round(CUs / (column ranges x outer)) chunks of every column,
so outer * nchunk * inner is at most 1.5 x CUs x the columns of one range
(256 for float32 packets): 98,304 floats, 393 KB, for 256 CUs.  The
refusal path of the allocation-free entry (partials above 1 MiB) is
therefore reachable only on a GPU with several times more CUs; the sweep
below shows both sides."""

import itertools

import pytest

F32, F16, BF16 = 0, 1, 2


@pytest.fixture(scope="module")
def lib(amd):
    return amd.load()


def test_exact_figures(lib):
    q = lib.tp_amd_reduce_partial_bytes
    # whole 2^24-element float32 tensor: 512 segments of 32768 (two blocks a CU)
    assert q(256, F32, 1, 1 << 24, 1) == 512 * 4
    # whole 4096^2 bf16 tensor: 256 segments of 65536 (one block a CU)
    assert q(256, BF16, 1, 4096 * 4096, 1) == 256 * 4
    # [32768, 4096] float32 over dim 0: 16 column ranges of 256 -> 16 chunks of 2048 rows
    assert q(256, F32, 1, 32768, 4096) == 16 * 4096 * 4
    # [4096, 32000] bf16 over dim 0: 250 ranges of 128 columns -> one chunk, no partials
    assert q(256, BF16, 1, 4096, 32000) == 0
    # rows that fill the chip, or short rows: one segment a row, no partials
    assert q(256, F32, 32768, 4096, 1) == 0
    assert q(256, F32, 3, 4000, 1) == 0
    assert q(256, F32, 0, 10, 10) == 0
    assert q(256, 3, 1, 10, 10) == -1          # float64 has no device reduction
    assert q(0, F32, 1, 10, 10) == -1
    assert q(256, F32, -1, 10, 10) == -1


def test_static_scratch_suffices_on_256_cus(lib):
    q, cap = lib.tp_amd_reduce_partial_bytes, lib.tp_amd_reduce_noalloc_scratch_bytes()
    assert cap == 1 << 20
    worst = 0
    shapes = itertools.product((F32, F16, BF16), (1, 2, 3, 7, 64, 255, 4095, 100000),
                               (1, 63, 64, 100, 8192, 32768, 1 << 20, (1 << 24) + 3),
                               (1, 3, 63, 64, 100, 255, 256, 257, 1000, 4096, 32000, 65536, 98304, 1 << 20))
    for dt, outer, r, inner in shapes:
        b = q(256, dt, outer, r, inner)
        assert 0 <= b <= 98304 * 4, (dt, outer, r, inner, b)
        worst = max(worst, b)
    assert worst <= cap // 2
    # a GPU with 2048 CUs would split further, past the static array
    assert q(2048, F32, 1, 32768, 98304) > cap
