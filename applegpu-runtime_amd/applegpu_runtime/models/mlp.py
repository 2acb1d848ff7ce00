"""MLP training step on the eager C ABI.

The reference trains `nn.Sequential(Linear, ReLU, ..., Linear)` with MSE and
SGD through its PrivateUse1 shim (benchmarks/bench_mlp_cpp.py:29-52,
python/tests/bench_comparison.py:11-38); autograd turns each step into these
aten calls: addmm (Linear), relu, mse_loss, mse_loss_backward, mm for the
weight and input gradients, threshold_backward (relu'), sum over the batch
(bias grads) and add_(alpha=-lr) per parameter (backend_cpp/applegpu_backend.cpp:
533-566, 584-620, 678-686, 801-895).  This module issues the same sequence
through the eager C ABI, with the fusions the MI355X backend offers:

  forward   h = relu(x W^T + b)        one GEMM, bias + relu in the epilogue
  loss      mse and dL/dout             one launch
  backward  dh = (g W) * (h > 0)        one GEMM, relu' mask in the epilogue
  + SGD     W += -lr * g^T h            one GEMM, the update in its epilogue
            b += -lr * sum(g, 0)        folded into the packing of g
(the first two layers' weight updates share one pack launch and one GEMM
launch; the output layer's 4096 -> 1 products run on the unit-extent GEMM
kernels).
A two-layer net is one op, mlp2_sgd_step_: at small sizes (config C1,
64 -> 128 -> 10 at batch 32) the whole step runs in one workgroup, one launch.
Every gradient is formed from the step's starting parameters, as autograd
does: layer i's input gradient (which reads W_i) is computed before W_i is
updated in place.

Parameters follow torch.nn.Linear's layout (W [out, in], b [out]).
"""
from __future__ import annotations

import numpy as np

from .. import eager as E


def torch_default_init(sizes, seed=42):
    """Kaiming-uniform weights/biases as torch.nn.Linear initialises them, made
    with torch's own generator so the CPU reference starts from the same bits."""
    import torch
    torch.manual_seed(seed)
    params = []
    for fin, fout in zip(sizes[:-1], sizes[1:]):
        lin = torch.nn.Linear(fin, fout)
        params.append((lin.weight.detach().numpy().copy(), lin.bias.detach().numpy().copy()))
    return params


class EagerMLP:
    """Linear -> ReLU -> ... -> Linear trained with MSE + SGD on the device."""

    def __init__(self, params_np):
        E.init()
        self.params = [(E.from_numpy(np.asarray(w, np.float32)), E.from_numpy(np.asarray(b, np.float32)))
                       for w, b in params_np]
        self._one = E.from_numpy(np.ones((1,), np.float32))

    def forward(self, x):
        acts = [x]
        h = x
        n = len(self.params)
        for i, (w, b) in enumerate(self.params):
            h = E.linear(h, w, b, act=1 if i < n - 1 else 0)
            acts.append(h)
        return h, acts

    def train_step(self, x, y, lr=0.01):
        """One forward + MSE + backward + SGD step; returns the loss tensor (on device)."""
        n = len(self.params)
        if n == 2:
            # Linear -> ReLU -> Linear: one op (one launch at small sizes)
            (w1, b1), (w2, b2) = self.params
            return E.mlp2_sgd_step_(x, y, w1, b1, w2, b2, -lr)
        if n == 1:
            w, b = self.params[0]
            return E.linear_mse_backward_sgd_(x, w, b, y, -lr, grad_in=False)[0]
        acts = [x]
        h = x
        for w, b in self.params[:-2]:
            h = E.linear(h, w, b, act=1)
            acts.append(h)
        # the last hidden layer and the output layer (no activation) with the
        # loss, its gradient and the output layer's SGD step (the hidden
        # GEMM's split-K sums are reduced by the output layer's forward)
        (wh, bh), (w, b) = self.params[-2], self.params[-1]
        loss, g, h = E.linear_relu_mse_backward_sgd_(h, wh, bh, w, b, y, -lr, grad_in=True)
        acts.append(h)
        for i in range(n - 2, 1, -1):
            w, b = self.params[i]
            # dL/d(input of layer i) masked by relu' of the previous layer's
            # output (from W_i before its update), then W_i -= lr * g^T a_i
            # and b_i -= lr * sum(g, 0)
            g = E.linear_backward_sgd_(w, b, g, acts[i], acts[i], -lr)
        if n > 2:
            # the first two layers together: both weight updates in one
            # launch pair
            (w0, b0), (w1, b1) = self.params[0], self.params[1]
            E.linear_backward_sgd_pair_(w1, b1, g, acts[1], w0, b0, x, -lr)
        return loss

    def train_step_unfused(self, x, y, lr=0.01):
        """The same step with every gradient materialised and one axpy per
        parameter (the reference's aten sequence); kept for comparison."""
        out, acts = self.forward(x)
        loss = E.mse_loss(out, y)
        g = E.mse_loss_backward(self._one, out, y)
        grads = [None] * len(self.params)
        for i in range(len(self.params) - 1, -1, -1):
            w, _ = self.params[i]
            a_in = acts[i]
            dw = E.matmul_ex(g, a_in, True, False)
            db = E.sum_dim(g, 0, False)
            grads[i] = (dw, db)
            if i > 0:
                g = E.matmul_masked(g, w, False, False, acts[i])
        for (w, b), (dw, db) in zip(self.params, grads):
            E.add_(w, dw, -lr)
            E.add_(b, db, -lr)
        return loss

    def numpy_params(self):
        return [(w.numpy(), b.numpy()) for w, b in self.params]
