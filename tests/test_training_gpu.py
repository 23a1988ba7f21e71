"""End-to-end workloads on the GPU: the operator sequences TensorPlay's
autograd dispatches for the quickstart (config 1) and the MLP training step
(config 5), against a float64 numpy restatement of the same mathematics.

Bar: the reference's ``close`` rule (tests/test_mlu.py:25-34) with the
float32 tolerance 1e-5 -- max |got - want| <= 1e-4 * max(max |want|, 1) -- and
its training-step bar of 1e-4 absolute on loss and gradients
(tests/test_mlu.py:363-378).  Config 5 runs here at a reduced size (batch
256, width 256, 100 classes) with the same operator sequence; at full size
(batch 8192, width 4096, 1000 classes) it is checked through properties that
do not need a float64 replay of 3.2 TFLOP: sampled gradient entries
recomputed from the device's own operands, log_softmax-backward rows
summing to zero, bias gradients equal to column sums, and the SGD update.
"""

import importlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-5


def close(got, want, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = float(np.max(np.abs(got - want))) if got.size else 0.0
    bar = TOL * max(float(np.max(np.abs(want))) if want.size else 0.0, 1.0) * 10
    assert err <= bar, f"{what}: max error {err:.3g} > {bar:.3g}"


@pytest.fixture(scope="module")
def wl(amd):
    return importlib.import_module("tensorplay-mlu_amd.workloads")


def randn(shape, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


# ---- config 1: quickstart ----------------------------------------------------------


def quickstart_ref(x, w, weight=None):
    x = x.astype(np.float64)
    w = w.astype(np.float64)
    y = x @ w
    r = np.maximum(y, 0.0)
    e = np.exp(r - r.max(-1, keepdims=True))
    z = e / e.sum(-1, keepdims=True)
    c = np.ones_like(z) if weight is None else weight.astype(np.float64)
    loss = float((z * c).sum())
    g_r = z * (c - (c * z).sum(-1, keepdims=True))
    g_y = np.where(r > 0, g_r, 0.0)
    return z, loss, g_y @ w.T, x.T @ g_y


@pytest.mark.parametrize("weighted", [False, True])
def test_quickstart_step(dev, ops, wl, weighted):
    x = randn((256, 256), 0)
    w = randn((256, 256), 1)
    c = randn((256, 256), 2) if weighted else None
    z, loss, gx, gw = wl.quickstart_step(ops, dev.from_numpy(x), dev.from_numpy(w),
                                         dev.from_numpy(c) if weighted else None)
    z_ref, loss_ref, gx_ref, gw_ref = quickstart_ref(x, w, c)
    close(z.numpy(), z_ref, "z")
    assert abs(float(loss.numpy()) - loss_ref) < 1e-4 * max(abs(loss_ref), 1.0) * 10
    close(gx.numpy(), gx_ref, "x.grad")
    close(gw.numpy(), gw_ref, "w.grad")


# ---- config 5: MLP training step -------------------------------------------------


def mlp_ref(ws, bs, x, labels, lr):
    """float64 forward, backward and SGD of the same network."""
    ws = [w.astype(np.float64) for w in ws]
    bs = [b.astype(np.float64) for b in bs]
    n = len(ws)
    acts = [x.astype(np.float64)]
    h = acts[0]
    for i in range(n):
        out = h @ ws[i].T + bs[i]
        h = np.maximum(out, 0.0) if i < n - 1 else out
        acts.append(h)
    m = h.max(-1, keepdims=True)
    logp = h - m - np.log(np.exp(h - m).sum(-1, keepdims=True))
    batch = x.shape[0]
    onehot = np.zeros_like(logp)
    onehot[np.arange(batch), labels] = 1.0
    loss = -(logp * onehot).sum() / batch
    g_logp = -onehot / batch
    g = g_logp - np.exp(logp) * g_logp.sum(-1, keepdims=True)
    grads = [None] * n
    for i in reversed(range(n)):
        if i < n - 1:
            g = np.where(acts[i + 1] > 0, g, 0.0)
        grads[i] = (g.T @ acts[i], g.sum(0))
        if i > 0:
            g = g @ ws[i]
    new_ws = [ws[i] - lr * grads[i][0] for i in range(n)]
    new_bs = [bs[i] - lr * grads[i][1] for i in range(n)]
    return loss, grads, new_ws, new_bs


def test_mlp_step_reduced(dev, ops, wl):
    batch, width, layers, classes, lr = 256, 256, 4, 100, 0.1
    ws, bs = wl.MLP.host_init(width, layers, width, classes, seed=0)
    x = randn((batch, width), 100)
    labels = np.random.default_rng(101).integers(0, classes, batch)
    onehot = np.zeros((batch, classes), np.float32)
    onehot[np.arange(batch), labels] = 1.0
    model = wl.MLP.to_device(ws, bs)
    loss, grads = wl.mlp_step(ops, model, dev.from_numpy(x), dev.from_numpy(onehot), lr)
    loss_ref, grads_ref, new_ws, new_bs = mlp_ref(ws, bs, x, labels, lr)
    assert abs(float(loss.numpy()) - loss_ref) < 1e-4
    for i, ((dW, db), (dW_ref, db_ref)) in enumerate(zip(grads, grads_ref)):
        assert np.max(np.abs(dW.numpy() - dW_ref)) < 1e-4, f"layer {i} weight grad"
        assert np.max(np.abs(db.numpy() - db_ref)) < 1e-4, f"layer {i} bias grad"
        close(dW.numpy(), dW_ref, f"layer {i} weight grad")
        close(model.weights[i].numpy(), new_ws[i], f"layer {i} weight after SGD")
        close(model.biases[i].numpy(), new_bs[i], f"layer {i} bias after SGD")


def test_mlp_step_full_size_properties(dev, ops, wl):
    """Config 5 at its real shape: batch 8192, four 4096-wide layers, 1000
    classes, float32.  Every GEMM of the step is checked on sampled entries
    recomputed in float64 from the device's own operands (bar 2e-3 of the
    product's largest magnitude), the reductions in full."""
    batch, width, layers, classes, lr = 8192, 4096, 4, 1000, 0.01
    ws, bs = wl.MLP.host_init(width, layers, width, classes, seed=0)
    x = randn((batch, width), 100)
    labels = np.random.default_rng(101).integers(0, classes, batch)
    onehot = np.zeros((batch, classes), np.float32)
    onehot[np.arange(batch), labels] = 1.0
    model = wl.MLP.to_device(ws, bs)
    trace = {}
    loss, grads = wl.mlp_step(ops, model, dev.from_numpy(x), dev.from_numpy(onehot), lr, trace)
    acts = [a.numpy() for a in trace["acts"]]
    gout = [g.numpy() for g in trace["grad_out"]]
    logp = trace["logp"].numpy().astype(np.float64)
    rng = np.random.default_rng(7)

    def sampled(got, a, b, what):
        """got[r, c] against float64 a[r, :] . b[:, c] on 512 sampled entries."""
        r = rng.integers(0, got.shape[0], 512)
        c = rng.integers(0, got.shape[1], 512)
        want = np.einsum("ik,ki->i", a[r, :].astype(np.float64), b[:, c].astype(np.float64))
        scale = max(float(np.max(np.abs(got))), 1e-30)
        err = float(np.max(np.abs(got[r, c].astype(np.float64) - want))) / scale
        assert err <= 2e-3, f"{what}: sampled relative error {err:.3g}"

    for i in range(layers + 1):
        # forward: acts[i+1] = act(acts[i] @ W^T + b)
        pre = acts[i + 1] if i == layers else None
        if pre is not None:
            sampled(pre, acts[i], ws[i].T, f"layer {i} forward")
        else:
            r = rng.integers(0, batch, 256)
            c = rng.integers(0, ws[i].shape[0], 256)
            want = np.maximum(np.einsum("ik,ik->i", acts[i][r].astype(np.float64),
                                        ws[i][c].astype(np.float64)) + bs[i][c], 0.0)
            scale = max(float(np.max(np.abs(acts[i + 1]))), 1e-30)
            assert np.max(np.abs(acts[i + 1][r, c] - want)) / scale <= 2e-3, f"layer {i} forward"
        dW, db = grads[i][0].numpy(), grads[i][1].numpy()
        sampled(dW, gout[i].T, acts[i], f"layer {i} weight grad")
        np.testing.assert_allclose(db, gout[i].astype(np.float64).sum(0), rtol=0,
                                   atol=1e-5 * max(float(np.abs(db).max()), 1.0) * 10)
        if i > 0:
            # the input gradient of layer i, masked by layer i-1's ReLU
            below = np.where(acts[i] > 0, 1.0, 0.0)
            r = rng.integers(0, batch, 256)
            c = rng.integers(0, width, 256)
            want = below[r, c] * np.einsum("ik,ki->i", gout[i][r].astype(np.float64),
                                           ws[i][:, c].astype(np.float64))
            scale = max(float(np.max(np.abs(gout[i - 1]))), 1e-30)
            assert np.max(np.abs(gout[i - 1][r, c] - want)) / scale <= 2e-3, f"layer {i} input grad"

    # log_softmax rows: exp sums to 1; its backward rows sum to 0
    assert np.max(np.abs(np.exp(logp).sum(-1) - 1.0)) < 1e-4
    assert np.max(np.abs(gout[-1].astype(np.float64).sum(-1))) < 1e-6
    loss_want = -logp[np.arange(batch), labels].mean()
    assert abs(float(loss.numpy()) - loss_want) < 1e-4 * max(abs(loss_want), 1.0) * 10
    # SGD: W_new = W + (-lr) * dW, one float32 rounding of each product and sum
    for i in range(layers + 1):
        dW = grads[i][0].numpy()
        want = (ws[i] + np.float32(-lr) * dW).astype(np.float32)
        got = model.weights[i].numpy()
        assert np.max(np.abs(got - want)) <= 1e-6 * max(float(np.abs(want).max()), 1.0)
