"""tp_amd_copy_bytes, the PrivateUse1HooksInterface::copy_bytes counterpart
(the reference's MLUHooks.cpp:23-44, MLURuntime.cpp:112-129), on the GPU:
host to device, device to device on one device, and device to host, each
bit-exact on random bytes; odd sizes and unaligned offsets on both sides;
64 MiB, the size of the reference README's h2d / d2h rows; sizes either side
of 8 MiB, from which host copies go through four pinned 4 MiB chunks, and
one of 18 chunks (each chunk buffer reused four or five times in each
direction); two sizes whose last chunk (262,148 and 4,177,924 bytes) does
not split into eight equal 64-byte multiples over the host copy threads; a
zero-byte copy is a no-op."""

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HOST = -1
U8 = 8


def _host_ptr(buf: np.ndarray, offset: int = 0) -> C.c_void_p:
    return C.c_void_p(buf.ctypes.data + offset)


@pytest.mark.parametrize("nbytes", [1, 3, 4097, (1 << 20) + 7, (8 << 20) - 1, 8 << 20, (8 << 20) + 1,
                                    64 << 20, (68 << 20) + 5, (8 << 20) + 262148, 2047 * 2047 * 4],
                         ids=["1B", "3B", "4097B", "1MiB+7", "8MiB-1", "8MiB", "8MiB+1", "64MiB", "68MiB+5",
                              "8MiB+256KiB+4", "2047^2-fp32"])
@pytest.mark.parametrize("offset", [0, 3], ids=["aligned", "offset3"])
def test_round_trip_is_bit_exact(amd, dev, ops, nbytes, offset):
    lib = amd.load()
    rng = np.random.default_rng(nbytes + offset)
    src = rng.integers(0, 256, size=nbytes + offset + 8, dtype=np.uint8)
    # two device buffers with slack on both sides, to see that nothing
    # outside [offset, offset + nbytes) is written
    a = ops.empty((nbytes + offset + 64,), U8)
    b = ops.empty((nbytes + offset + 64,), U8)
    fill = np.full(nbytes + offset + 64, 0xA5, np.uint8)
    assert lib.tp_amd_copy_bytes(C.c_void_p(b.data_ptr), 0, _host_ptr(fill), HOST, fill.size) == 0
    assert lib.tp_amd_copy_bytes(C.c_void_p(a.data_ptr + offset), 0, _host_ptr(src, offset), HOST,
                                 nbytes) == 0                                    # host -> device
    assert lib.tp_amd_copy_bytes(C.c_void_p(b.data_ptr + offset), 0, C.c_void_p(a.data_ptr + offset), 0,
                                 nbytes) == 0                                    # device -> device
    back = np.full(nbytes + offset + 8, 0x5A, np.uint8)
    assert lib.tp_amd_copy_bytes(_host_ptr(back, offset), HOST, C.c_void_p(b.data_ptr + offset), 0,
                                 nbytes) == 0                                    # device -> host
    assert np.array_equal(back[offset:offset + nbytes], src[offset:offset + nbytes])
    assert np.all(back[:offset] == 0x5A) and np.all(back[offset + nbytes:] == 0x5A)
    whole = b.numpy()
    assert np.array_equal(whole[offset:offset + nbytes], src[offset:offset + nbytes])
    assert np.all(whole[:offset] == 0xA5) and np.all(whole[offset + nbytes:] == 0xA5)


def test_zero_bytes_and_errors(amd, dev, ops):
    lib = amd.load()
    a = ops.empty((16,), U8)
    host = np.arange(16, dtype=np.uint8)
    assert lib.tp_amd_copy_bytes(C.c_void_p(a.data_ptr), 0, _host_ptr(host), HOST, 0) == 0
    assert lib.tp_amd_copy_bytes(C.c_void_p(a.data_ptr), 0, _host_ptr(host), HOST, 16) == 0
    assert np.array_equal(a.numpy(), host)
    # a device index that does not exist is an error with a message
    assert lib.tp_amd_copy_bytes(C.c_void_p(a.data_ptr), 999, _host_ptr(host), HOST, 16) != 0
    assert lib.tp_mlu_last_error()
