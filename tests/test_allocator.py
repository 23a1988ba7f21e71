"""The block cache's policy (the reference's MLUAllocator.cpp:42-45, 98-128,
208-219) on a host-memory backend with an injected capacity: size
quantization, best-fit reuse within a quarter, statistics and peaks, the
return-idle-and-retry-once response to out-of-memory, trimming that waits
for the device before returning blocks, and recording epochs.  The same
block_cache.h backs the device allocator."""

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
def test_quantize(shim, n, want):
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


def test_best_fit_matches_a_brute_force_model(shim):
    """A random sequence of hand-outs and returns against a plain model of
    the policy: a request is served by the most recently returned of the
    smallest idle blocks in [quantized size, quantized size * 5 / 4], else
    by a new block.  Sizes cluster around the 64-class words of the fine
    classes' bitmap (32 KiB multiples) and around the 1 MiB edge between
    fine and 2 MiB classes."""
    import random

    rng = random.Random(7)
    shim.shim_reset(1 << 40)

    def quantize(n):
        step = 512 if n <= MiB else 2 * MiB
        return (n + step - 1) // step * step

    centres = [32 * 1024 * k for k in (1, 2, 3, 31, 32)] + [MiB, 2 * MiB, 6 * MiB, 40 * MiB]
    live = []          # (block, ptr, size)
    idle = []          # model: (size, ptr) in return order
    for step in range(4000):
        if live and (rng.random() < 0.45 or len(live) > 60):
            blk, ptr, size = live.pop(rng.randrange(len(live)))
            shim.shim_give(blk)
            idle.append((size, ptr))
            continue
        want = max(1, rng.choice(centres) + rng.randint(-3000, 3000))
        q = quantize(want)
        fits = [(s, i) for i, (s, p) in enumerate(idle) if q <= s <= q + q // 4]
        blk = shim.shim_take(0, want)
        ptr, size = shim.shim_block_ptr(blk), shim.shim_block_size(blk)
        if fits:
            best = min(s for s, _ in fits)
            i = max(i for s, i in fits if s == best)     # most recently returned
            assert (size, ptr) == idle[i], (step, want, size, idle[i])
            idle.pop(i)
        else:
            assert size == q and all(p != ptr for _, p in idle), (step, want, size)
        live.append((blk, ptr, size))
    assert shim.shim_cached(0) == len(idle)
    for blk, _, _ in live:
        shim.shim_give(blk)
