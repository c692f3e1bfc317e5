"""Pins of the oracle's Conv2D input gradient and Dropout backward against
float64 torch autograd (CPU only).

- Conv2D backward (conv2d.go:997-1174, oracle/refcpu.c conv_backward): the
  input gradient of a conv alone (accumulate_grad's per-sample input
  gradients) and of a conv below another conv, where the lower conv's weight
  gradient flows through the upper conv's input gradient.  Strides 1 and 2,
  paddings 0..2, kernels 3 and 5.  The 3x3 / stride 1 / padding 1 forward
  leaves interior-row edge columns at the bias (Q7, conv2d.go:265-357) while
  the backward is the generic loop over every position; the torch model
  carries that as a zero-valued term (pre + (bias - pre).detach() at those
  positions), so the value is the reference's and the gradient the full
  convolution's.
- Dropout backward (dropout.go:241-293): g * 1/(1-p) where the mask keeps,
  the mask being the closed-form first draws of RNG(42) (Q9), which is a
  constant factor in the torch model.

A test that swaps the kernel taps (a transposed operand), drops the stride in
the input index, or drops the dropout scale fails here: each test also checks
that such a variant differs from the oracle by far more than the tolerance.
"""
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")
F = torch.nn.functional

TOL = 1e-5  # max|a - r| / max|r|, float32 oracle vs float64 autograd


def rel(a, r):
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.abs(a - r).max() / np.abs(r).max())


def q7_mask(oh, ow, k, s, p):
    """Positions the 3x3 fast path never accumulates (Q7)."""
    m = np.zeros((oh, ow), bool)
    if k == 3 and s == 1 and p == 1:
        m[1:oh - 1, 0] = True
        m[1:oh - 1, ow - 1] = True
    return m


def torch_conv(x, w, b, s, p, act):
    """Reference forward of one Conv2D over a batch, with Q7's values."""
    z = F.conv2d(x, w, b, stride=s, padding=p)
    m = torch.tensor(q7_mask(z.shape[2], z.shape[3], w.shape[2], s, p))
    if m.any():
        bias_map = b.view(1, -1, 1, 1).expand_as(z)
        z = z + torch.where(m, bias_map - z, torch.zeros_like(z)).detach()
    return torch.relu(z) if act == "relu" else z


def lcg_floats(seed, n):
    out = []
    s = seed
    for _ in range(n):
        s = (s * 6364136223846793005 + 1) % (1 << 64)
        out.append(np.float32(s >> 33) / np.float32(2 ** 31))
    return np.array(out, np.float32)


CONV_SHAPES = [(3, 1, 0), (3, 1, 1), (3, 2, 0), (3, 2, 1), (5, 1, 0), (5, 1, 2), (5, 2, 1), (5, 2, 2)]


@pytest.mark.parametrize("k,s,p", CONV_SHAPES)
@pytest.mark.parametrize("act", ["linear", "relu"])
def test_conv_input_gradient_vs_autograd(oracle, k, s, p, act):
    C, O, H, B = 3, 4, 9, 3
    oh = (H + 2 * p - k) // s + 1
    rng = np.random.default_rng(100 + 10 * k + 3 * s + p)
    net = oracle.Net([oracle.spec(oracle.LAYER_CONV2D, in_size=C * H * H, in_channels=C, out_channels=O,
                                  kernel=k, stride=s, padding=p,
                                  act=oracle.ACT_RELU if act == "relu" else oracle.ACT_LINEAR)],
                     oracle.LOSS_MSE)
    x = rng.normal(size=(B, C, H, H)).astype(np.float32)
    g = rng.normal(size=(B, O * oh * oh)).astype(np.float32)
    p0 = net.params.copy().astype(np.float64)
    out, gin = net.accumulate_grad(x.reshape(B, -1), g, B, C * H * H, O * oh * oh)

    nw = O * C * k * k
    P = torch.tensor(p0, requires_grad=True)
    xt = torch.tensor(x.astype(np.float64), requires_grad=True)
    y = torch_conv(xt, P[:nw].view(O, C, k, k), P[nw:], s, p, act)
    assert rel(out, y.detach().numpy().reshape(B, -1)) < TOL
    # parameter gradients are averaged over the batch (net.go:767-770)
    y.backward(torch.tensor(g.astype(np.float64)).view_as(y) / B)
    gin_ref = xt.grad.numpy().reshape(B, -1) * B
    assert rel(gin, gin_ref) < TOL
    assert rel(net.grads[:nw], P.grad[:nw].numpy()) < TOL
    assert rel(net.grads[nw:], P.grad[nw:].numpy()) < TOL

    # plausible mistakes are far outside the tolerance: taps flipped (the
    # forward's correlation read as a convolution), stride ignored in the
    # input index
    wf = torch.tensor(p0[:nw]).view(O, C, k, k).flip(2, 3)
    xt2 = torch.tensor(x.astype(np.float64), requires_grad=True)
    y2 = torch_conv(xt2, wf, torch.tensor(p0[nw:]), s, p, act)
    y2.backward(torch.tensor(g.astype(np.float64)).view_as(y2))
    assert rel(gin, xt2.grad.numpy().reshape(B, -1)) > 1e-2
    if s > 1:
        w = torch.tensor(p0[:nw]).view(O, C, k, k)
        gz = torch.tensor(g.astype(np.float64)).view(B, O, oh, oh)
        if act == "relu":
            gz = gz * (y.detach() > 0)
        wrong = F.conv_transpose2d(gz, w, stride=1, padding=p)  # no stride
        hw = min(wrong.shape[2], H)
        assert rel(gin.reshape(B, C, H, H)[:, :, :hw, :hw], wrong[:, :, :hw, :hw].numpy()) > 1e-2


@pytest.mark.parametrize("lower,upper", [((3, 2, 1), (3, 1, 1)), ((3, 1, 1), (3, 1, 1)),
                                         ((5, 1, 2), (3, 2, 0)), ((3, 1, 0), (5, 1, 1))])
def test_conv_below_conv_grads_vs_autograd(oracle, lower, upper):
    """conv -> conv -> Flatten -> Dense(Softmax) with cross-entropy: the lower
    conv's dW and db come through the upper conv's input gradient."""
    (k1, s1, p1), (k2, s2, p2) = lower, upper
    C, O1, O2, H, B, NC = 2, 3, 4, 10, 4, 5
    h1 = (H + 2 * p1 - k1) // s1 + 1
    h2 = (h1 + 2 * p2 - k2) // s2 + 1
    rng = np.random.default_rng(7 + k1 + 10 * k2 + s1 + 3 * s2)
    specs = [oracle.spec(oracle.LAYER_CONV2D, in_size=C * H * H, in_channels=C, out_channels=O1,
                         kernel=k1, stride=s1, padding=p1, act=oracle.ACT_RELU),
             oracle.spec(oracle.LAYER_CONV2D, in_size=O1 * h1 * h1, in_channels=O1, out_channels=O2,
                         kernel=k2, stride=s2, padding=p2, act=oracle.ACT_RELU),
             oracle.spec(oracle.LAYER_FLATTEN),
             oracle.spec(oracle.LAYER_DENSE, in_size=O2 * h2 * h2, out_size=NC, act=oracle.ACT_SOFTMAX,
                         act_is_ptr=1)]
    net = oracle.Net(specs, oracle.LOSS_CE)
    # both convs start from RNG(42): give the upper one other weights so a
    # swapped operand between the two layers cannot cancel out
    p0 = net.params.copy()
    sl1, sl2 = net.layer_slice(0), net.layer_slice(1)
    p0[sl2] = rng.normal(scale=0.3, size=sl2.stop - sl2.start).astype(np.float32)
    net.params[:] = p0
    x = rng.normal(size=(B, C, H, H)).astype(np.float32)
    y = np.eye(NC, dtype=np.float32)[rng.integers(0, NC, B)]
    net.accumulate_batch(x.reshape(B, -1), y, B)

    P = torch.tensor(p0.astype(np.float64), requires_grad=True)
    n1 = O1 * C * k1 * k1
    n2 = O2 * O1 * k2 * k2
    o2 = sl2.start
    o3 = net.layer_slice(3).start
    a1 = torch_conv(torch.tensor(x.astype(np.float64)), P[:n1].view(O1, C, k1, k1), P[n1:n1 + O1],
                    s1, p1, "relu")
    a2 = torch_conv(a1, P[o2:o2 + n2].view(O2, O1, k2, k2), P[o2 + n2:o2 + n2 + O2], s2, p2, "relu")
    nin = O2 * h2 * h2
    W = P[o3:o3 + nin * NC].view(NC, nin)
    b = P[o3 + nin * NC:o3 + nin * NC + NC]
    prob = torch.softmax(a2.reshape(B, -1) @ W.T + b, dim=1)
    # CrossEntropy.BackwardInPlace gives p - y; Dense applies the softmax
    # Jacobian to it (Q4), which is autograd of p fed with (p - y)
    prob.backward((prob - torch.tensor(y.astype(np.float64))).detach() / B)
    ref = P.grad.numpy()
    for name, sl in (("conv1.W", slice(0, n1)), ("conv1.b", slice(n1, n1 + O1)),
                     ("conv2.W", slice(o2, o2 + n2)), ("conv2.b", slice(o2 + n2, o2 + n2 + O2)),
                     ("dense", slice(o3, o3 + nin * NC + NC))):
        assert rel(net.grads[sl], ref[sl]) < TOL, name


def dropout_mask(n, p):
    """Q9: Reset reseeds RNG(42) before every sample (dropout.go:399-401),
    so the mask is the first n draws compared with p (dropout.go:85-153)."""
    u = lcg_floats(42, n)
    return (~(u < np.float32(p))).astype(np.float64)


def test_dropout_backward_alone_vs_autograd(oracle):
    n, p, B = 96, 0.3, 5
    rng = np.random.default_rng(11)
    net = oracle.Net([oracle.spec(oracle.LAYER_DROPOUT, in_size=n, p=p)], oracle.LOSS_MSE)
    x = rng.normal(size=(B, n)).astype(np.float32)
    g = rng.normal(size=(B, n)).astype(np.float32)
    out, gin = net.accumulate_grad(x, g, B, n, n)
    scale = float(np.float32(1) / (np.float32(1) - np.float32(p)))
    keep = dropout_mask(n, p)
    xt = torch.tensor(x.astype(np.float64), requires_grad=True)
    yt = xt * torch.tensor(keep * scale)
    yt.backward(torch.tensor(g.astype(np.float64)))
    assert rel(out, yt.detach().numpy()) < TOL
    assert rel(gin, xt.grad.numpy()) < TOL
    # the scale is part of the gradient: dropping it is far off
    assert rel(gin, g * keep) > 0.1
    assert 0 < keep.sum() < n


@pytest.mark.parametrize("act", ["relu", "sigmoid", "tanh"])
@pytest.mark.parametrize("workers", [1, 3])
def test_dense_dropout_dense_grads_vs_autograd(oracle, act, workers):
    """Dense -> Dropout -> Dense(Softmax) + CE, the C1 arrangement: every
    gradient of the lower Dense passes through the Dropout's backward."""
    I, Hd, NC, B, p = 20, 24, 6, 9, 0.2
    codes = {"relu": oracle.ACT_RELU, "sigmoid": oracle.ACT_SIGMOID, "tanh": oracle.ACT_TANH}
    specs = [oracle.spec(oracle.LAYER_DENSE, in_size=I, out_size=Hd, act=codes[act]),
             oracle.spec(oracle.LAYER_DROPOUT, in_size=Hd, p=p),
             oracle.spec(oracle.LAYER_DENSE, in_size=Hd, out_size=NC, act=oracle.ACT_SOFTMAX, act_is_ptr=1)]
    net = oracle.Net(specs, oracle.LOSS_CE, workers=workers)
    rng = np.random.default_rng(12)
    x = rng.uniform(size=(B, I)).astype(np.float32)
    y = np.eye(NC, dtype=np.float32)[rng.integers(0, NC, B)]
    p0 = net.params.copy().astype(np.float64)
    net.accumulate_batch(x, y, B)

    P = torch.tensor(p0, requires_grad=True)
    W1 = P[:I * Hd].view(Hd, I)
    b1 = P[I * Hd:I * Hd + Hd]
    o = I * Hd + Hd
    W2 = P[o:o + Hd * NC].view(NC, Hd)
    b2 = P[o + Hd * NC:o + Hd * NC + NC]
    z = torch.tensor(x.astype(np.float64)) @ W1.T + b1
    h = {"relu": torch.relu, "sigmoid": torch.sigmoid, "tanh": torch.tanh}[act](z)
    scale = float(np.float32(1) / (np.float32(1) - np.float32(p)))
    keep = torch.tensor(dropout_mask(Hd, p))
    d = h * keep * scale
    prob = torch.softmax(d @ W2.T + b2, dim=1)
    prob.backward((prob - torch.tensor(y.astype(np.float64))).detach() / B)
    ref = P.grad.numpy()
    assert rel(net.grads[:o], ref[:o]) < TOL
    assert rel(net.grads[o:], ref[o:]) < TOL
    # without the dropout scale in the backward the lower layer is off by 1/(1-p)
    assert rel(net.grads[:o], ref[:o] / scale) > 0.1
