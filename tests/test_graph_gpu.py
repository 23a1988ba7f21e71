"""Recording and replaying device work (tp_mlu_capture_*, the reference's
GraphCapture.cpp:38-130 and graph.py:38-92) on the GPU: on every refilled
input a recorded step replays to the CPU oracle's results (and to the same
bits as the eager step, which runs the same kernels), several times with
eager work and synchronisations in between; a step that reads a value back
cannot be recorded; the allocator pins the recording's blocks until it is
discarded."""

import importlib

import numpy as np
import pytest

from _check import assert_bitexact, assert_normwise, assert_sum, F32

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


def oracle_step(orc, x, w, b):
    """The same step on the CPU oracle, one operator at a time (float64
    inside each, rounded to float32 between them, as the device does)."""
    y = orc.unary(8, F32, orc.binary(0, F32, orc.gemm(F32, x, w), b))
    z = orc.softmax(False, F32, y, y.shape[0], y.shape[1], 1)
    return z, orc.reduce(0, F32, z, 1, z.shape[0], z.shape[1])


def test_replay_matches_oracle(dev, ops, orc, graph_mod, runtime):
    rng = np.random.default_rng(3)
    wh = rng.standard_normal((256, 192)).astype(np.float32) / 16
    bh = rng.standard_normal(192).astype(np.float32)
    w, b = dev.from_numpy(wh), dev.from_numpy(bh)
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
            oz, os_ = oracle_step(orc, host, wh, bh)
            assert_normwise(z.numpy(), oz, F32, 1, f"replay {i}: softmax against the oracle")
            assert_sum(s.numpy(), os_, F32, f"replay {i}: column sums against the oracle")
            want_z, want_s = step(ops, dev.from_numpy(host), w, b)   # eager, same kernels
            assert_bitexact(z.numpy(), want_z.numpy(), f"replay {i}: softmax against eager")
            assert_bitexact(s.numpy(), want_s.numpy(), f"replay {i}: column sums against eager")
            ops.mul_(x, 0.5)                        # unrelated eager work between replays
            runtime.synchronize()
        allocations, held = g.stats()
        assert allocations >= 5                     # one block per recorded result
        del want_z, want_s
    finally:
        g.reset()
    assert not g.ready
    assert g.stats()[1] == 0


@pytest.mark.parametrize("adds", [1, 16, 17, 40])
def test_short_and_long_recordings(dev, ops, graph_mod, runtime, adds):
    """A chain of up to 16 kernels is replayed kernel by kernel from the
    recorded launches, a longer one as the HIP graph: both give the eager
    result on every refilled input, replayed several times in a row."""
    rng = np.random.default_rng(adds)
    x = dev.from_numpy(rng.standard_normal((64, 96)).astype(np.float32))
    y = dev.from_numpy(rng.standard_normal((64, 96)).astype(np.float32))

    def chain(a, b):
        for _ in range(adds):
            a = ops.add(a, b, alpha=0.5)
        return a

    g = graph_mod.Graph()
    try:
        out = g.capture(lambda: chain(x, y))
        assert graph_mod.Graph.direct_kernels() == (adds if adds <= 16 else 0)
        for i in range(3):
            host = rng.standard_normal((64, 96)).astype(np.float32)
            ops.copy_(x, host)
            g.replay()
            g.replay()                              # the same inputs again: the same result
            runtime.synchronize()
            want = chain(dev.from_numpy(host), y)
            assert_bitexact(out.numpy(), want.numpy(), f"{adds} adds, replay {i}")
    finally:
        g.reset()
    assert graph_mod.Graph.direct_kernels() == 0


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
    assert np.allclose(g.results.numpy(), np.exp(0.5), rtol=1e-6)
    assert np.array_equal(y.numpy(), np.full((1024, 1024), 2.0, np.float32))
    g.reset()                                    # result released, blocks returned
    assert g.stats()[1] == 0


def nn_step(ops, t):
    """NN layers whose kernels keep state on the device or take workspaces:
    layer norm forward and backward (block partials, then a folding
    launch), the embedding gradient (the row-range plan's device-wide
    cursors, reset by the plan's last block), nll_loss forward (the last
    block folds the partials) and backward, and a whole-tensor sum (one
    launch, the last block folds)."""
    D = t["x"].shape[1]
    y, mean, rstd = ops.native_layer_norm(t["x"], (D,), t["w"], t["b"])
    dx, dw, db = ops.native_layer_norm_backward(t["dy"], t["x"], (D,), mean, rstd, t["w"], t["b"])
    de = ops.embedding_dense_backward(t["g"], t["idx"], 3000, 5, False)
    loss, tw = ops.nll_loss(t["logits"], t["tgt"], None, 1)
    dl = ops.nll_loss_backward(t["one"], t["logits"], t["tgt"], None, 1, -100, tw)
    s = ops.sum(t["big"])
    return y, dx, dw, db, de, loss, dl, s


def nn_inputs(rng, i):
    return {"x": rng.standard_normal((64, 512)).astype(np.float32) * (1 + i),
            "dy": rng.standard_normal((64, 512)).astype(np.float32),
            "g": rng.standard_normal((1000, 64)).astype(np.float32),
            "idx": rng.integers(0, 3000, size=1000).astype(np.int64),
            "logits": rng.standard_normal((1000, 37)).astype(np.float32),
            "tgt": rng.integers(0, 37, size=1000).astype(np.int64),
            "big": rng.standard_normal((1000, 3000)).astype(np.float32)}


def test_replay_nn_layers(dev, ops, orc, graph_mod, runtime):
    """The recorded NN step replays to the eager step's bits on every refilled
    input, with the same operators run eagerly in between (they use the same
    device counters and cursors), and its embedding gradient to the float32
    sum of each row's samples in sample order."""
    rng = np.random.default_rng(8)
    wh = rng.standard_normal(512).astype(np.float32)
    bh = rng.standard_normal(512).astype(np.float32)
    fixed = {"w": dev.from_numpy(wh), "b": dev.from_numpy(bh),
             "one": dev.from_numpy(np.array(1.0, np.float32))}
    t = dict(fixed)
    t.update({k: dev.from_numpy(v) for k, v in nn_inputs(rng, 0).items()})
    g = graph_mod.Graph()
    names = ["y", "dx", "dw", "db", "de", "loss", "dl", "s"]
    try:
        outs = g.capture(lambda: nn_step(ops, t))
        for i in range(3):
            host = nn_inputs(rng, i + 1)
            for k, v in host.items():
                ops.copy_(t[k], v)                  # refill the recorded inputs
            g.replay()
            runtime.synchronize()
            fresh = dict(fixed)
            fresh.update({k: dev.from_numpy(v) for k, v in host.items()})
            want = nn_step(ops, fresh)              # eager, same kernels
            for name, got, w in zip(names, outs, want):
                assert_bitexact(got.numpy(), w.numpy(), f"replay {i}: {name} against eager")
            keep = (host["idx"] != 5)
            acc = np.zeros((3000, 64), np.float32)
            np.add.at(acc, host["idx"][keep], host["g"][keep])
            assert_bitexact(outs[4].numpy(), acc, f"replay {i}: embedding gradient in sample order")
            assert_sum(outs[7].numpy(), np.float32(host["big"].astype(np.float64).sum()), F32,
                       f"replay {i}: whole-tensor sum against float64")
            yo, _, _ = orc.layer_norm(F32, host["x"], 512, wh, bh)
            assert_normwise(outs[0].numpy(), yo, F32, 1, f"replay {i}: layer norm against the oracle")
            del want, fresh
            ops.mul_(t["big"], 0.5)                 # unrelated eager work between replays
            runtime.synchronize()
    finally:
        g.reset()
    assert g.stats()[1] == 0


def thin_step(ops, t):
    """Products whose kernels fold partials across blocks: a thin product
    with W K-major (tiles split over blocks, arrival counters), one with W
    N-major and an odd K, and a 16-bit split-K product (float32 partials
    and a finish kernel)."""
    return (ops.linear(t["x"], t["w"]), ops.mm(t["dy"], t["w2"]), ops.mm(t["a"], t["b"]))


def test_replay_thin_and_split_products(dev, ops, graph_mod, runtime):
    """The recorded thin and split-K products replay to the eager bits on
    every refilled input, with the same products run eagerly in between
    (they share the arrival counters and the workspace pool)."""
    rng = np.random.default_rng(9)
    bf = lambda a: ops.to(dev.from_numpy(a.astype(np.float32)), 2)  # noqa: E731

    def inputs():
        return {"x": rng.standard_normal((1, 4096)), "dy": rng.standard_normal((1, 3001)),
                "a": rng.standard_normal((200, 4096)) / 16}

    fixed = {"w": bf(rng.standard_normal((2048, 4096)) / 64), "w2": bf(rng.standard_normal((3001, 1024)) / 64),
             "b": bf(rng.standard_normal((4096, 384)) / 64)}
    t = dict(fixed)
    t.update({k: bf(v) for k, v in inputs().items()})
    g = graph_mod.Graph()
    try:
        outs = g.capture(lambda: thin_step(ops, t))
        for i in range(3):
            host = {k: bf(v) for k, v in inputs().items()}
            for k, v in host.items():
                ops.copy_(t[k], v)                  # refill the recorded inputs
            g.replay()
            runtime.synchronize()
            fresh = dict(fixed)
            fresh.update(host)
            want = thin_step(ops, fresh)            # eager, same kernels
            for name, got, w in zip(("thin K-major", "thin N-major", "split-K"), outs, want):
                assert_bitexact(got.numpy(), w.numpy(), f"replay {i}: {name} against eager")
            del want, fresh
            thin_step(ops, t)                       # eager products between replays
            runtime.synchronize()
    finally:
        g.reset()
    assert g.stats()[1] == 0
