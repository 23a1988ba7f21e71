"""Copies, casts, fills and factories on the GPU (the reference's cases,
tests/test_mlu.py:64-132): every result bit-exact against the host data or
the CPU oracle's conversion."""

import importlib

import numpy as np
import pytest

from _check import BF16, F16, F32, assert_bitexact

pytestmark = pytest.mark.gpu

F64, I8, I16, I32, I64, U8, BOOL = 3, 4, 5, 6, 7, 8, 9
ALL = [F32, F16, BF16, F64, I8, I16, I32, I64, U8, BOOL]
NP = {F32: np.float32, F16: np.float16, BF16: np.uint16, F64: np.float64, I8: np.int8,
      I16: np.int16, I32: np.int32, I64: np.int64, U8: np.uint8, BOOL: np.bool_}


def values(orc, shape, dtype, seed=0):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * 10
    if dtype in (F32, F16, BF16):
        return orc.from_float(x, dtype)
    return orc.cast(F32, dtype, x)


@pytest.mark.parametrize("dtype", ALL)
def test_round_trip(dev, orc, dtype):
    x = values(orc, (5, 7), dtype)
    d = dev.from_numpy(x, dtype=dtype)
    assert d.dtype == dtype and d.shape == (5, 7)
    assert_bitexact(d.numpy(), x, "round trip")


def test_strided_copies_both_ways(dev, ops, orc):
    x = values(orc, (6, 8), F32)
    # host strided source -> device
    d = dev.empty((8, 6), F32)
    ops.copy_(d, x.T)
    assert_bitexact(d.numpy(), np.ascontiguousarray(x.T), "host .T -> device")
    d = dev.from_numpy(x)
    assert_bitexact(d.t().numpy(), np.ascontiguousarray(x.T), "device .t() -> host")
    assert_bitexact(d[:, 1::3].numpy(), np.ascontiguousarray(x[:, 1::3]), "device slice -> host")
    out = ops.zeros_like(d.t())
    ops.copy_(out, d.t())
    assert_bitexact(out.numpy(), np.ascontiguousarray(x.T), "device .t() -> device")
    # a large transpose (LDS-tiled kernel) and a strided destination
    big = values(orc, (1000, 777), F32, 1)
    db = dev.from_numpy(big)
    assert_bitexact(ops.contiguous(db.t()).numpy(), np.ascontiguousarray(big.T), "transpose")
    dst = dev.from_numpy(np.zeros((777, 1000), np.float32))
    ops.copy_(dst.t(), db)
    assert_bitexact(dst.numpy(), np.ascontiguousarray(big.T), "into transposed view")


@pytest.mark.parametrize("dtype", [U8, BF16, F32, I64], ids=["1B", "2B", "4B", "8B"])
def test_strided_copies_in_packets(dev, ops, orc, dtype):
    """Rows whose bytes, strides and base addresses are whole 16-byte packets
    copy a packet a lane (two dimensions: one kernel walking the rows; more:
    the general kernel on 16-byte elements); a slice starting off a packet
    boundary, or rows of a partial packet, keeps the element kernel.  Both
    directions (a strided source, a strided destination), bit-exact."""
    es = {U8: 1, BF16: 2, F32: 4, I64: 8}[dtype]
    per = 16 // es                       # elements in a packet
    x = values(orc, (96, 8 * per + 40), dtype, 3)
    d = dev.from_numpy(x, dtype=dtype)
    cases = [(d[:, 0:4 * per], x[:, 0:4 * per], "row slice"),
             (d[:, per:5 * per], x[:, per:5 * per], "row slice one packet in"),
             (d[5:77, 2 * per:8 * per], x[5:77, 2 * per:8 * per], "block"),
             (d[:, 1:4 * per + 1], x[:, 1:4 * per + 1], "off a packet boundary"),
             (d[:, 0:4 * per + 1], x[:, 0:4 * per + 1], "partial packet rows")]
    if es < 16:
        cases.append((d[:, 3:3 + per], x[:, 3:3 + per], "misaligned packet"))
    y = values(orc, (4, 30, 6 * per), dtype, 4)
    dy = dev.from_numpy(y, dtype=dtype)
    cases.append((dy[:, 3:23, per:5 * per], y[:, 3:23, per:5 * per], "3-D"))
    for view, want, what in cases:
        assert_bitexact(ops.contiguous(view).numpy(), np.ascontiguousarray(want), what)
    # a strided destination: write a block into a row slice of a larger tensor
    out = dev.from_numpy(np.zeros_like(x), dtype=dtype)
    ops.copy_(out[:, per:5 * per], dev.from_numpy(np.ascontiguousarray(x[:, 0:4 * per]), dtype=dtype))
    want = np.zeros_like(x)
    want[:, per:5 * per] = x[:, 0:4 * per]
    assert_bitexact(out.numpy(), want, "into a row slice")


def test_broadcasting_copy_on_device(dev, ops, orc):
    row = values(orc, (1, 5), F32)
    out = dev.empty((4, 5), F32)
    ops.copy_(out, dev.from_numpy(row))
    assert_bitexact(out.numpy(), np.broadcast_to(row, (4, 5)).copy(), "broadcast copy")


@pytest.mark.parametrize("src,dst", [(F32, F16), (F16, F32), (F32, BF16), (BF16, F32),
                                     (F16, BF16), (F32, I32), (I64, F32), (F64, F32),
                                     (F32, F64), (F64, BF16), (I32, I8), (BOOL, F32),
                                     (F32, BOOL), (U8, I64), (BF16, I64)])
def test_casts_on_device(dev, ops, orc, src, dst):
    x = values(orc, (3, 9), src)
    got = ops.to(dev.from_numpy(x, dtype=src), dst).numpy()
    want = orc.cast(src, dst, x) if not (src == F16 and dst == BF16) else \
        orc.cast(F32, BF16, orc.cast(F16, F32, x))
    assert_bitexact(got, want, f"cast {src}->{dst}")


@pytest.mark.parametrize("src,dst", [(F32, BF16), (F32, F16), (BF16, F32), (F16, F32), (BF16, F16),
                                     (I32, F32), (F32, I32)])
def test_casts_packed_and_scalar_paths(dev, ops, orc, src, dst):
    """Aligned buffers of 2- and 4-byte types convert 8 elements a thread as
    16-byte packets, the last n % 8 elements and unaligned buffers element by
    element: the same bits either way.  1003 elements from the start of the
    buffer (packets and a 3-element tail), and from one element in (a view
    whose data is 16-byte aligned for neither 2- nor 4-byte elements)."""
    x = values(orc, (1004,), src)
    d = dev.from_numpy(x, dtype=src)
    whole = ops.to(d[0:1003], dst).numpy()
    shifted = ops.to(d[1:1004], dst).numpy()
    assert_bitexact(whole, orc.cast(src, dst, x[:1003]), f"cast {src}->{dst}, aligned")
    assert_bitexact(shifted, orc.cast(src, dst, x[1:]), f"cast {src}->{dst}, unaligned")


def test_cast_every_bf16_and_f16_pattern(dev, ops, orc):
    bits = np.arange(1 << 16, dtype=np.uint16)
    for dtype in (BF16, F16):
        d = dev.from_numpy(bits, dtype=dtype)
        got = ops.to(d, F32).numpy()
        want = orc.cast(dtype, F32, bits)
        nan = np.isnan(want)
        assert_bitexact(got[~nan], want[~nan], f"{dtype} -> f32")
        assert np.isnan(got[nan]).all()
    # 16-bit to 16-bit goes through float32, as the reference's cast table
    # routes it (CopyKernels.cpp:152-158)
    for src, dst in ((BF16, F16), (F16, BF16)):
        got = ops.to(dev.from_numpy(bits, dtype=src), dst).numpy()
        want = orc.cast(F32, dst, orc.cast(src, F32, bits))
        nan = np.isnan(orc.to_float(want, dst))
        assert np.array_equal(np.isnan(orc.to_float(got, dst)), nan), f"{src} -> {dst}: NaN"
        assert np.array_equal(got.view(np.uint16)[~nan], want.view(np.uint16)[~nan]), f"{src} -> {dst}"
    f = np.random.default_rng(0).standard_normal(1 << 20).astype(np.float32) * 1e3
    f[:6] = [np.inf, -np.inf, 0.0, -0.0, 3.4e38, 1e-40]
    for dtype in (BF16, F16):
        got = ops.to(dev.from_numpy(f), dtype).numpy()
        assert_bitexact(got, orc.cast(F32, dtype, f), f"f32 -> {dtype}")


def test_cast_every_float32_pattern(dev, ops, orc):
    """float32 -> float16 and float32 -> bfloat16 at every one of the 2^32
    float32 bit patterns (16 chunks of 2^28), bit-exact against the oracle's
    round-to-nearest-even; a NaN stays NaN (its payload is not compared)."""
    chunk = 1 << 28
    for c in range((1 << 32) // chunk):
        bits = (np.arange(chunk, dtype=np.uint64) + np.uint64(c * chunk)).astype(np.uint32)
        f = bits.view(np.float32)
        d = dev.from_numpy(f)
        for dt in (F16, BF16):
            got, want = ops.to(d, dt).numpy(), orc.cast(F32, dt, f)
            g, w = got.view(np.uint16), want.view(np.uint16)
            differ = g != w
            if differ.any():
                both_nan = np.isnan(orc.to_float(got, dt)) & np.isnan(orc.to_float(want, dt))
                bad = np.flatnonzero(differ & ~both_nan)
                assert bad.size == 0, (f"f32 -> {dt}: {bad.size} patterns differ, first "
                                       f"{hex(int(bits[bad[0]]))}: got {hex(int(g[bad[0]]))} want {hex(int(w[bad[0]]))}")
        del d


@pytest.mark.parametrize("dtype", ALL)
def test_fill_and_factories(dev, ops, dtype):
    d = dev.empty((3, 4), dtype)
    value = 2.5 if dtype in (F32, F16, BF16, F64) else 3
    ops.fill_(d, value)
    want_val = {BF16: np.uint16(0x4020)}.get(dtype, value)
    assert_bitexact(d.numpy(), np.full((3, 4), want_val, dtype=NP[dtype]), "fill_")
    ops.zero_(d)
    assert_bitexact(d.numpy(), np.zeros((3, 4), NP[dtype]), "zero_")
    one = {BF16: np.uint16(0x3f80)}.get(dtype, 1)
    assert_bitexact(ops.ones_like(d).numpy(), np.full((3, 4), one, NP[dtype]), "ones_like")
    assert_bitexact(ops.zeros_like(d).numpy(), np.zeros((3, 4), NP[dtype]), "zeros_like")
    assert ops.ones_like(d, dtype=F32).dtype == F32
    seven = {BF16: np.uint16(0x40e0)}.get(dtype, 7)
    assert_bitexact(ops.full_like(d, 7).numpy(), np.full((3, 4), seven, NP[dtype]), "full_like")
    big = dev.empty((1000, 333), dtype)
    ops.fill_(big, value)
    assert_bitexact(big.numpy(), np.full((1000, 333), want_val, dtype=NP[dtype]), "large fill")


@pytest.mark.parametrize("dtype", [F32, F16, BF16, F64])
def test_fill_special_values(dev, ops, orc, dtype):
    """fill_ with -0.0, +-inf, NaN, a float32 subnormal and values that round
    in the narrow dtypes (0.1, 65519, 1e30): the host encodes the scalar as
    the reference does (float -> dtype, CopyKernels.cpp:231-291) and every
    element holds that encoding -- the sign of zero and the NaN included."""
    d = dev.empty((7, 130), dtype)
    for value in (-0.0, np.inf, -np.inf, np.nan, 1e-40, 0.1, 65519.0, 1e30):
        ops.fill_(d, value)
        got = d.numpy()
        with np.errstate(over="ignore"):
            want = np.full(got.shape, orc.from_float(np.float32([value]), dtype)[0]) if dtype != F64 \
                else np.full(got.shape, np.float64(value))
        assert np.array_equal(got.view(np.uint8), want.astype(got.dtype).view(np.uint8)), (dtype, value)


def test_views_share_device_memory(dev, ops, orc):
    x = values(orc, (4, 6), F32)
    d = dev.from_numpy(x)
    v = d.view(6, 4)
    ops.mul__scalar(v, 2.0)
    assert_bitexact(d.numpy(), x * np.float32(2), "view mul_")
    assert_bitexact(ops.contiguous(d.permute(1, 0)).numpy().reshape(-1),
                    (x * np.float32(2)).T.reshape(-1), "permute")
    assert_bitexact(d[1:3].numpy(), (x * np.float32(2))[1:3], "narrow")


def test_item_clone_and_empty(dev, ops, orc):
    x = values(orc, (1,), F32)
    assert ops.item(dev.from_numpy(x)) == float(x[0])
    assert ops.item(dev.from_numpy(np.array([7], np.int64))) == 7
    c = ops.clone(dev.from_numpy(x))
    assert_bitexact(c.numpy(), x, "clone")
    e = ops.empty((0, 3))
    assert e.shape == (0, 3) and e.numel() == 0
    tensor = importlib.import_module("tensorplay-mlu_amd.tensor")
    with pytest.raises(tensor.DeviceError):
        ops.item(dev.from_numpy(values(orc, (2,), F32)))


def test_memory_statistics(dev, ops):
    runtime = importlib.import_module("tensorplay-mlu_amd.runtime")
    runtime.synchronize()
    runtime.empty_cache()
    before = runtime.memory_allocated()
    x = ops.empty((1 << 20,))
    assert runtime.memory_allocated() >= before + (4 << 20)
    assert runtime.max_memory_allocated() >= runtime.memory_allocated()
    del x
    assert runtime.memory_allocated() == before
    assert runtime.memory_reserved() >= before
    free, total = runtime.mem_get_info()
    assert 0 < free <= total
    assert runtime.device_count() >= 1 and runtime.current_device() == 0
