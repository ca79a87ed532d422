"""The recorded model workloads against a second, library oracle: torch on the
CPU in float64, with autograd for the gradients.

Each fixture is replayed through the oracle (oracle/oracle.c, itself pinned
bit for bit to the engine's CPU backend by tests/test_oracle.py), and every
buffer the workload read back (READ records: losses, gradients, updated
parameters) is compared with the textbook model computed by torch from the
same generated inputs:

  MLP        x [64,784] -> linear 128 -> relu -> linear 10, softmax
             cross-entropy (src/nn/loss.c:8-44: logsumexp - onehot . logits,
             mean over the batch); loss, dW1, dW2.
  LeNet-5    conv5x5 pad 2 -> relu -> maxpool 2 -> conv5x5 -> relu -> maxpool 2
             -> fc 400-120-84-10 (relu between), cross-entropy; loss, and each
             parameter's SGD update (lr 0.01).
  conv block conv3x3 pad 1 -> batchnorm in train mode (biased variance in the
             normalisation, eps 1e-5, running statistics with momentum 0.1 and
             the unbiased variance, src/nn/batchnorm.c:35-87) -> relu ->
             maxpool 2 -> sum; loss, dW, dX, running mean and variance.

This pins that the kernels the engine lowers for these workloads compute the
models they are named after (the engine's own gradient rules are not used:
the workloads compose their backward passes explicitly). Tolerances are
normwise (max |x - y| / max |y|): 1e-5 for the losses, forward statistics and
gradients, 1e-4 for the SGD updates (differences of float32 parameters that
move by about 1 %); the errors measured are 5e-8 to 1.5e-6.
"""
import ctypes as C

import numpy as np
import pytest

from tests import tracetools as tt
from tinyhvm_amd import trace

torch = pytest.importorskip("torch")
F = torch.nn.functional


def _normwise(x, y):
    x, y = np.asarray(x, np.float64).ravel(), np.asarray(y, np.float64).ravel()
    return float(np.max(np.abs(x - y))) / max(float(np.max(np.abs(y))), 1e-30)


def _run(name, extra_ids=()):
    """Replays a fixture through the oracle; returns the generated / written
    inputs by trace id, the buffers read back (READ records, by trace id, in
    order) and the final contents of `extra_ids`."""
    path = tt.fixtures(name)[0]
    recs = trace.read_trace(path)
    ora = tt.oracle()
    be = ora.oracle_backend_ptr()
    be.contents.init()
    rp = tt.Replay(path, be)
    inputs, reads = {}, []
    try:
        for i, r in enumerate(recs):
            if r.tag == trace.WRITE:
                f = r.f
                data = (trace.gen_data(f["dist"], f["dtype"], f["seed"], f["p0"], f["p1"], f["bytes"])
                        if f["enc"] == trace.ENC_GEN else f["data"])
                inputs.setdefault(f["id"], np.frombuffer(data, np.float32).copy())
            rp.run(i, i + 1)
            if r.tag == trace.READ:
                p = ora.oracle_buf_ptr(rp.live(r.f["id"]))
                reads.append((r.f["id"], np.frombuffer(C.string_at(p, r.f["bytes"]), np.float32).copy()))
        final = {}
        for t in extra_ids:
            p = ora.oracle_buf_ptr(rp.live(t))
            final[t] = np.frombuffer(C.string_at(p, ora.oracle_buf_size(rp.live(t))), np.float32).copy()
    finally:
        rp.close()
        be.contents.shutdown()
    return inputs, reads, final


def _t(a, *shape):
    return torch.tensor(np.asarray(a, np.float64).reshape(shape), dtype=torch.float64)


def _ce(logits, onehot):
    return (torch.logsumexp(logits, dim=1) - (onehot * logits).sum(dim=1)).mean()


def test_mlp_matches_torch_autograd():
    inp, reads, _ = _run("mlp_64x784x128x10.trc")
    x = _t(inp[1], 64, 784)
    W1, b1 = _t(inp[2], 784, 128).requires_grad_(), _t(inp[3], 128)
    W2, b2 = _t(inp[4], 128, 10).requires_grad_(), _t(inp[5], 10)
    onehot = _t(inp[6], 64, 10)
    loss = _ce(F.relu(x @ W1 + b1) @ W2 + b2, onehot)
    loss.backward()
    (_, l), (_, dW1), (_, dW2) = reads
    assert _normwise(l, loss.item()) <= 1e-5
    assert _normwise(dW1, W1.grad.numpy()) <= 1e-5
    assert _normwise(dW2, W2.grad.numpy()) <= 1e-5


def test_lenet_step_matches_torch_autograd():
    inp, reads, _ = _run("lenet_b2.trc")
    B = 2
    x = _t(inp[1], B, 1, 28, 28)
    shapes = {2: (6, 1, 5, 5), 3: (6,), 4: (16, 6, 5, 5), 5: (16,), 6: (400, 120), 7: (120,),
              8: (120, 84), 9: (84,), 10: (84, 10), 11: (10,)}
    P = {k: _t(inp[k], *s).requires_grad_() for k, s in shapes.items()}
    onehot = _t(inp[12], B, 10)
    a1 = F.relu(F.conv2d(x, P[2], P[3], padding=2))
    a2 = F.relu(F.conv2d(F.max_pool2d(a1, 2), P[4], P[5]))
    f = F.max_pool2d(a2, 2).reshape(B, 400)
    h3 = F.relu(f @ P[6] + P[7])
    h4 = F.relu(h3 @ P[8] + P[9])
    loss = _ce(h4 @ P[10] + P[11], onehot)
    loss.backward()
    assert reads[0][0] == 89
    assert _normwise(reads[0][1], loss.item()) <= 1e-5
    updated = dict(reads[1:])
    assert sorted(updated) == sorted(shapes)
    for k in shapes:
        got = updated[k].astype(np.float64) - inp[k].astype(np.float64)
        want = -0.01 * P[k].grad.numpy().ravel()
        assert _normwise(got, want) <= 1e-4, "parameter %d: %.2e" % (k, _normwise(got, want))


def test_convblock_matches_torch_autograd():
    inp, reads, final = _run("convblock_2x4x8.trc", extra_ids=(5, 6))
    B, Cc, H = 2, 4, 8
    x = _t(inp[1], B, Cc, H, H).requires_grad_()
    W = _t(inp[2], Cc, Cc, 3, 3).requires_grad_()
    gamma, beta = _t(inp[3], Cc), _t(inp[4], Cc)
    c = F.conv2d(x, W, padding=1)
    mean = c.mean(dim=(0, 2, 3))
    var = c.var(dim=(0, 2, 3), unbiased=False)
    xhat = (c - mean.view(1, -1, 1, 1)) / torch.sqrt(var.view(1, -1, 1, 1) + 1e-5)
    y = xhat * gamma.view(1, -1, 1, 1) + beta.view(1, -1, 1, 1)
    loss = F.max_pool2d(F.relu(y), 2).sum()
    loss.backward()
    (_, l), (_, dW), (_, dx) = reads
    assert _normwise(l, loss.item()) <= 1e-5
    assert _normwise(dW, W.grad.numpy()) <= 1e-5
    assert _normwise(dx, x.grad.numpy()) <= 1e-5
    n = B * H * H
    unbiased = var.detach().numpy() * n / (n - 1)
    assert _normwise(final[5], 0.1 * mean.detach().numpy()) <= 1e-5
    assert _normwise(final[6], 0.9 + 0.1 * unbiased) <= 1e-5


def test_planted_mistake_fails_the_comparison():
    """The same comparison against a model that differs in one place (the MLP
    without its relu) must fail."""
    inp, reads, _ = _run("mlp_64x784x128x10.trc")
    x = _t(inp[1], 64, 784)
    W1, b1 = _t(inp[2], 784, 128).requires_grad_(), _t(inp[3], 128)
    W2, b2 = _t(inp[4], 128, 10).requires_grad_(), _t(inp[5], 10)
    loss = _ce((x @ W1 + b1) @ W2 + b2, _t(inp[6], 64, 10))
    loss.backward()
    assert _normwise(reads[1][1], W1.grad.numpy()) > 1e-2
