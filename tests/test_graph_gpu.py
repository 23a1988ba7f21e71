"""Recording and replaying device work (tp_mlu_capture_*, the reference's
GraphCapture.cpp:38-130 and graph.py:38-92) on the GPU: a recorded step
replays to the same results as the eager step on refilled inputs, several
times with eager work and synchronisations in between; a step that reads a
value back cannot be recorded; the allocator sets aside the recording's
blocks until it is dropped."""

import importlib

import numpy as np
import pytest

from _check import assert_normwise, F32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def graph_mod(amd):
    return importlib.import_module("tensorplay-mlu_amd.graph")


@pytest.fixture(scope="module")
def runtime(amd):
    return importlib.import_module("tensorplay-mlu_amd.runtime")


def step(ops, x, w, b):
    """mm -> bias add -> relu -> softmax -> sum over rows: one kernel each."""
    y = ops.relu(ops.add(ops.mm(x, w), b))
    z = ops.softmax(y, -1)
    return z, ops.sum_dim(z, [0])


def test_replay_matches_eager(dev, ops, graph_mod, runtime):
    rng = np.random.default_rng(3)
    w = dev.from_numpy(rng.standard_normal((256, 192)).astype(np.float32) / 16)
    b = dev.from_numpy(rng.standard_normal(192).astype(np.float32))
    x = dev.from_numpy(rng.standard_normal((128, 256)).astype(np.float32))
    g = graph_mod.Graph()
    try:
        z, s = g.capture(lambda: step(ops, x, w, b))
        assert g.ready
        for i in range(4):
            host = rng.standard_normal((128, 256)).astype(np.float32) * (1 + i)
            ops.copy_(x, host)                      # refill the recorded input
            g.replay()
            runtime.synchronize()
            want_z, want_s = step(ops, dev.from_numpy(host), w, b)   # eager, same kernels
            assert_normwise(z.numpy(), want_z.numpy(), F32, 1, f"replay {i}: softmax")
            assert_normwise(s.numpy(), want_s.numpy(), F32, 1, f"replay {i}: column sums")
            ops.mul_(x, 0.5)                        # unrelated eager work between replays
            runtime.synchronize()
        allocations, held = g.stats()
        assert allocations >= 5                     # one block per recorded result
        del want_z, want_s
    finally:
        g.reset()
    assert not g.ready
    assert g.stats()[1] == 0


def test_host_read_back_cannot_be_recorded(dev, ops, graph_mod):
    x = dev.from_numpy(np.ones((4, 4), np.float32))
    g = graph_mod.Graph()
    with pytest.raises(RuntimeError):
        g.capture(lambda: ops.item(ops.sum(x)))     # a read-back inside the recording
    assert not g.ready
    # the library recovers: a device-only step records and replays afterwards
    out = g.capture(lambda: ops.mul_scalar(x, 3.0))
    g.replay()
    assert np.array_equal(out.numpy(), np.full((4, 4), 3.0, np.float32))
    g.reset()


def test_blocks_set_aside_until_reset(dev, ops, graph_mod, runtime):
    x = dev.from_numpy(np.ones((1024, 1024), np.float32))
    g = graph_mod.Graph()
    out = g.capture(lambda: ops.exp(ops.mul_scalar(x, 0.5)))   # the temporary is freed inside
    g.replay()
    runtime.synchronize()
    assert np.allclose(out.numpy(), np.exp(0.5), rtol=1e-6)
    assert g.stats()[1] >= 1                     # the temporary's block is set aside
    del out                                      # the graph still keeps its result
    y = ops.mul_scalar(x, 2.0)                   # eager work cannot take either block
    g.replay()
    runtime.synchronize()
    assert np.allclose(g._outputs.numpy(), np.exp(0.5), rtol=1e-6)
    assert np.array_equal(y.numpy(), np.full((1024, 1024), 2.0, np.float32))
    g.reset()                                    # result released, blocks returned
    assert g.stats()[1] == 0
