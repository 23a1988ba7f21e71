"""The benchmark's two end-to-end workloads, written as the operator
sequences TensorPlay's autograd dispatches to the PrivateUse1 backend: the
forward registrations, then the calls the backward formulas make.  Every
step is one operator of ``ops`` (one C-ABI entry of libtp_amd.so), so a
workload exercises exactly the kernels a TensorPlay training step would.

* ``quickstart_step`` -- the reference README's quickstart on the device
  (config 1): ``y = x @ w``, ``z = relu(y).softmax(-1)``, ``loss = z.sum()``,
  ``loss.backward()``.
* ``mlp_step`` -- the fp32 MLP training step of config 5: four
  ``Linear + ReLU`` layers, a final ``Linear``, ``log_softmax``, the NLL loss
  built from ``mul`` + ``sum`` with a one-hot, backward, then SGD through
  ``add_`` (reference test_mlu.py:363-378 checks the same kind of step).

Backward formulas used (the registrations they reach):
  sum:          grad.expand(self.shape)                       (a stride-0 view)
  mul / mul.Scalar: grad * other                              (mul.Tensor, mul.Scalar)
  _softmax:     _softmax_backward_data(grad, result, dim, dtype)
  _log_softmax: _log_softmax_backward_data(grad, result, dim, dtype)
  relu:         threshold_backward(grad, result, 0)
  mm:           grad @ mat2.t(), self.t() @ grad              (transposes read in place)
  linear:       grad @ weight, grad.t() @ input, grad.sum(0)  (mm, mm, sum.dim_IntList)
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .tensor import DeviceTensor

# FLOP of one config-5 step at its full size (forward + backward GEMMs):
# forward 4 * 2*B*H*H + 2*B*H*C, backward 2 per layer except the first
# layer's input gradient.
def mlp_step_flops(batch: int, width: int, hidden_layers: int, classes: int) -> int:
    fwd = hidden_layers * 2 * batch * width * width + 2 * batch * width * classes
    bwd = (2 * hidden_layers - 1) * 2 * batch * width * width + 2 * 2 * batch * width * classes
    return fwd + bwd


def quickstart_step(ops, x: DeviceTensor, w: DeviceTensor, weight: DeviceTensor | None = None):
    """Forward and backward of ``loss = (softmax(relu(x @ w), -1) [* weight]).sum()``.

    ``weight`` (optional, same shape as the product) turns the loss into a
    weighted sum so the gradients are not identically zero; the reference's
    quickstart has none (its gradients are zero up to rounding, since every
    softmax row sums to 1).  Returns (z, loss, x_grad, w_grad)."""
    y = ops.mm(x, w)
    r = ops.relu(y)
    z = ops._softmax(r, -1)
    loss = ops.sum(z if weight is None else ops.mul(z, weight))
    # backward
    g = ops.ones_like(loss)
    g_z = g.expand(*z.shape)
    if weight is not None:
        g_z = ops.mul(g_z, weight)
    g_r = ops._softmax_backward_data(g_z, z, -1, "float32")
    g_y = ops.threshold_backward(g_r, r, 0)
    x_grad = ops.mm(g_y, w.t())
    w_grad = ops.mm(x.t(), g_y)
    return z, loss, x_grad, w_grad


@dataclass
class MLP:
    """Parameters of the config-5 MLP: ``weights[i]`` is ``[out, in]`` (the
    Linear layout, read transposed in place by ``linear``), ``biases[i]`` is
    ``[out]``."""

    weights: list = field(default_factory=list)
    biases: list = field(default_factory=list)

    @staticmethod
    def host_init(width: int, hidden_layers: int, in_features: int, classes: int,
                  seed: int = 0):
        """float32 host parameters: W ~ N(0, 1/sqrt(in)), b = 0 (one seeded
        stream per tensor)."""
        dims = [in_features] + [width] * hidden_layers + [classes]
        ws, bs = [], []
        for i in range(len(dims) - 1):
            rng = np.random.default_rng(seed + 1 + i)
            ws.append((rng.standard_normal((dims[i + 1], dims[i]), dtype=np.float32)
                       / np.float32(np.sqrt(dims[i]))).astype(np.float32))
            bs.append(np.zeros(dims[i + 1], np.float32))
        return ws, bs

    @staticmethod
    def to_device(ws, bs) -> "MLP":
        return MLP([DeviceTensor.from_numpy(w) for w in ws],
                   [DeviceTensor.from_numpy(b) for b in bs])


def mlp_step(ops, model: MLP, x: DeviceTensor, onehot: DeviceTensor, lr: float,
             trace: dict | None = None):
    """One SGD step in place on ``model``; returns the loss (a 0-d device
    tensor) and the gradients [(dW, db), ...] in layer order.  A ``trace``
    dict receives the intermediates: ``acts`` (each layer's input, then the
    logits), ``logp``, and ``grad_out`` (the gradient at each layer's
    pre-activation output)."""
    batch = x.shape[0]
    n = len(model.weights)
    # forward: Linear + ReLU for every hidden layer, Linear for the last
    acts = [x]  # inputs of each layer
    h = x
    for i in range(n):
        out = ops.linear(h, model.weights[i], model.biases[i])
        h = ops.relu(out) if i < n - 1 else out
        acts.append(h)
    logp = ops._log_softmax(h, -1)
    picked = ops.mul(logp, onehot)
    total = ops.sum(picked)
    loss = ops.mul_scalar(total, -1.0 / batch)
    # backward
    g = ops.ones_like(loss)
    g_total = ops.mul_scalar(g, -1.0 / batch)
    g_picked = g_total.expand(*picked.shape)
    g_logp = ops.mul(g_picked, onehot)
    g = ops._log_softmax_backward_data(g_logp, logp, -1, "float32")
    grads = [None] * n
    grad_out = [None] * n
    for i in reversed(range(n)):
        if i < n - 1:  # through the ReLU of layer i (its output acts[i + 1])
            g = ops.threshold_backward(g, acts[i + 1], 0)
        grad_out[i] = g
        dW = ops.mm(g.t(), acts[i])
        db = ops.sum_dim(g, [0])
        grads[i] = (dW, db)
        if i > 0:
            g = ops.mm(g, model.weights[i])
    if trace is not None:
        trace.update(acts=acts, logp=logp, grad_out=grad_out)
    # SGD: p.add_(grad, alpha=-lr)
    for i in range(n):
        ops.add_(model.weights[i], grads[i][0], alpha=-lr)
        ops.add_(model.biases[i], grads[i][1], alpha=-lr)
    return loss, grads
