"""The caching allocator's policy (tensorplay_mlu/csrc/MLUAllocator.cpp:37-236)
on a host-memory backend with an injected capacity: size rounding, best-fit
reuse within a quarter, statistics and peaks, the release-and-retry-once
response to out-of-memory, and empty_cache waiting for the device before
returning blocks.  The same allocator_core.h backs the device allocator."""

import ctypes as C
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MiB = 1 << 20


@pytest.fixture(scope="module")
def shim(tmp_path_factory):
    out = tmp_path_factory.mktemp("alloc") / "libshim.so"
    subprocess.run(["g++", "-O1", "-std=c++17", "-shared", "-fPIC", "-o", str(out),
                    os.path.join(ROOT, "tests", "native", "alloc_shim.cpp")], check=True)
    lib = C.CDLL(str(out))
    lib.shim_reset.argtypes = [C.c_size_t]
    lib.shim_round.argtypes = [C.c_size_t]
    lib.shim_round.restype = C.c_size_t
    lib.shim_take.argtypes = [C.c_int, C.c_size_t]
    lib.shim_take.restype = C.c_void_p
    lib.shim_block_size.argtypes = [C.c_void_p]
    lib.shim_block_size.restype = C.c_size_t
    lib.shim_block_ptr.argtypes = [C.c_void_p]
    lib.shim_block_ptr.restype = C.c_void_p
    lib.shim_give.argtypes = [C.c_void_p]
    lib.shim_stats.argtypes = [C.c_int, C.POINTER(C.c_longlong)]
    lib.shim_cached.argtypes = [C.c_int]
    lib.shim_cached.restype = C.c_size_t
    lib.shim_counts.argtypes = [C.POINTER(C.c_long)]
    lib.shim_reset_peak.argtypes = [C.c_int]
    lib.shim_capture_holding.argtypes = [C.c_int]
    lib.shim_capture_stats.argtypes = [C.POINTER(C.c_longlong)]
    return lib


def stats(lib, dev=0):
    out = (C.c_longlong * 4)()
    lib.shim_stats(dev, out)
    return list(out)


def counts(lib):
    out = (C.c_long * 4)()
    lib.shim_counts(out)
    return list(out)


@pytest.mark.parametrize("n,want", [(1, 512), (512, 512), (513, 1024), (MiB - 1, MiB),
                                    (MiB, MiB), (MiB + 1, 2 * MiB), (3 * MiB, 4 * MiB),
                                    (4 * MiB, 4 * MiB), (0, 0)])
def test_round_size(shim, n, want):
    assert shim.shim_round(n) == want


def test_reuse_within_a_quarter(shim):
    shim.shim_reset(1 << 30)
    b = shim.shim_take(0, 8 * MiB)
    ptr = shim.shim_block_ptr(b)
    shim.shim_give(b)
    # 7 MiB rounds to 8 MiB: exact reuse
    b2 = shim.shim_take(0, 7 * MiB)
    assert shim.shim_block_ptr(b2) == ptr
    shim.shim_give(b2)
    # 6 MiB: 8 <= 6 + 6/4 = 7.5 is false -> a new block
    b3 = shim.shim_take(0, 6 * MiB)
    assert shim.shim_block_ptr(b3) != ptr and shim.shim_block_size(b3) == 6 * MiB
    # 6.5 MiB rounds to 8 MiB -> the cached 8 MiB block
    b4 = shim.shim_take(0, 6 * MiB + MiB // 2)
    assert shim.shim_block_ptr(b4) == ptr
    assert counts(shim)[0] == 2


def test_best_fit_picks_the_smallest_adequate_block(shim):
    shim.shim_reset(1 << 30)
    big, mid = shim.shim_take(0, 10 * MiB), shim.shim_take(0, 8 * MiB)
    pbig, pmid = shim.shim_block_ptr(big), shim.shim_block_ptr(mid)
    shim.shim_give(big)
    shim.shim_give(mid)
    b = shim.shim_take(0, 8 * MiB)
    assert shim.shim_block_ptr(b) == pmid
    b2 = shim.shim_take(0, 9 * MiB)  # rounds to 10 MiB
    assert shim.shim_block_ptr(b2) == pbig


def test_statistics_and_peaks(shim):
    shim.shim_reset(1 << 30)
    a = shim.shim_take(0, 1000)        # 1024
    b = shim.shim_take(0, 3 * MiB)     # 4 MiB
    assert stats(shim) == [1024 + 4 * MiB, 1024 + 4 * MiB, 1024 + 4 * MiB, 1024 + 4 * MiB]
    shim.shim_give(b)
    assert stats(shim) == [1024, 1024 + 4 * MiB, 1024 + 4 * MiB, 1024 + 4 * MiB]
    shim.shim_reset_peak(0)
    assert stats(shim) == [1024, 1024 + 4 * MiB, 1024, 1024 + 4 * MiB]
    assert stats(shim, 1) == [0, 0, 0, 0]  # per device
    shim.shim_give(a)
    shim.shim_empty()
    s = stats(shim)
    assert s[0] == 0 and s[1] == 0
    allocs, frees, waits, used = counts(shim)
    assert frees == 2 and waits == 1 and used == 0


def test_out_of_memory_releases_the_cache_and_retries_once(shim):
    shim.shim_reset(20 * MiB)
    a = shim.shim_take(0, 8 * MiB)
    b = shim.shim_take(0, 8 * MiB)
    shim.shim_give(a)                      # cached, still reserved
    assert shim.shim_cached(0) == 1
    # 12 MiB does not fit beside 16 reserved -> release the cache, retry
    c = shim.shim_take(0, 12 * MiB)
    assert c is not None
    assert shim.shim_cached(0) == 0
    allocs, frees, waits, used = counts(shim)
    assert frees == 1 and waits == 1 and used == 20 * MiB
    # nothing cached and still no room: an error, and the statistics stay
    assert shim.shim_take(0, 8 * MiB) is None
    assert stats(shim)[0] == 20 * MiB
    shim.shim_give(b)
    shim.shim_give(c)


def capture_stats(shim):
    out = (C.c_longlong * 2)()
    shim.shim_capture_stats(out)
    return out[0], out[1]


def test_recording_sets_blocks_aside(shim):
    """Blocks handed out while a sequence is recorded are reused during the
    recording, set aside once it ends, and returned when it is dropped
    (the reference's MLUAllocator.cpp:130-201)."""
    shim.shim_reset(1 << 30)
    plain = shim.shim_take(0, 1 * MiB)           # before the recording
    shim.shim_capture_holding(1)
    a = shim.shim_take(0, 4 * MiB)
    a_ptr = shim.shim_block_ptr(a)
    shim.shim_give(a)                            # freed inside the recording ...
    b = shim.shim_take(0, 4 * MiB)               # ... may be reused inside it
    assert shim.shim_block_ptr(b) == a_ptr
    c = shim.shim_take(0, 8 * MiB)
    shim.shim_give(c)                            # free at the end of the recording
    shim.shim_capture_holding(0)
    shim.shim_freeze()
    assert capture_stats(shim) == (3, 1)         # three hand-outs; c set aside
    assert shim.shim_cached(0) == 0
    shim.shim_give(b)                            # a recorded block freed afterwards
    assert capture_stats(shim)[1] == 2
    d = shim.shim_take(0, 4 * MiB)               # is not handed out again
    assert shim.shim_block_ptr(d) != a_ptr
    shim.shim_give(d)
    shim.shim_give(plain)
    assert shim.shim_cached(0) == 2              # unrecorded blocks stay cached
    reserved_before = stats(shim, 0)[1]
    waits_before = counts(shim)[2]
    shim.shim_drop()
    assert capture_stats(shim)[1] == 0
    assert stats(shim, 0)[1] == reserved_before - 12 * MiB
    assert counts(shim)[2] > waits_before        # the device was drained first
    # a block of the dropped recording freed afterwards returns to the pool
    shim.shim_capture_holding(1)
    e = shim.shim_take(0, 2 * MiB)
    shim.shim_capture_holding(0)
    shim.shim_freeze()
    shim.shim_drop()
    cached = shim.shim_cached(0)
    shim.shim_give(e)
    assert capture_stats(shim)[1] == 0 and shim.shim_cached(0) == cached + 1
