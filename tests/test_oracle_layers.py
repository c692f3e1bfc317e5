"""Pins the oracle's stand-alone MultiHeadAttention and LayerNorm layers (used
as the per-layer references of the GPU operators) against float64 torch.

MultiHeadAttention (transformer.go:277-690): wQ, wK, wV, wOut are Linear Dense
layers called once per token, so each one's backward sees the last token's
input (Q10: dW = (sum_t dz_t) x_last^T, db = sum_t dz_t); the attention and
softmax gradients are autograd's; RoPE rotates Q and K (transformer.go:212-236)
and the backward applies the conjugate rotation, which is autograd's gradient
of a rotation.  LayerNorm (layernorm.go:193-441): Q18, the backward's last term
uses N std^2 where the exact gradient has N std^3.  The batch pass is
gno_net_accumulate_grad (output gradients given, parameter gradients averaged
over the batch)."""
import numpy as np
import pytest

from cfgutil import max_rel

torch = pytest.importorskip("torch")


class _PTDense(torch.autograd.Function):  # Q10: dW from the last token's input
    @staticmethod
    def forward(ctx, xx, W, b):
        ctx.save_for_backward(xx, W)
        return xx @ W.T + b

    @staticmethod
    def backward(ctx, g):
        xx, W = ctx.saved_tensors
        s = g.sum(0)
        return g @ W, s[:, None] * xx[-1][None, :], s


def _rope(q, T, NH, hd):
    half = hd // 2
    out = q.clone()
    for t in range(T):
        for k in range(half):
            theta = np.float32(10000.0 ** (-(2.0 * k) / hd))
            m = np.float32(t) * theta
            c, s = float(np.float32(np.cos(np.float64(m)))), float(np.float32(np.sin(np.float64(m))))
            for h in range(NH):
                i1, i2 = h * hd + k, h * hd + k + half
                out[t, i1] = q[t, i1] * c - q[t, i2] * s
                out[t, i2] = q[t, i1] * s + q[t, i2] * c
    return out


def _mha_torch(p, x, g, T, D, NH, causal, rope):
    """Per sample: returns (out, dx, dparams) of MultiHeadAttention."""
    hd = D // NH
    P = torch.tensor(p.astype(np.float64), requires_grad=True)
    X = torch.tensor(x.astype(np.float64).reshape(T, D), requires_grad=True)
    nd = D * D + D
    Wq, Wk, Wv, Wo = (P[i * nd:i * nd + D * D].view(D, D) for i in range(4))
    bq, bk, bv, bo = (P[i * nd + D * D:(i + 1) * nd] for i in range(4))
    Q, K, Vv = _PTDense.apply(X, Wq, bq), _PTDense.apply(X, Wk, bk), _PTDense.apply(X, Wv, bv)
    if rope:
        Q, K = _rope(Q, T, NH, hd), _rope(K, T, NH, hd)
    outs = []
    for h in range(NH):
        sl = slice(h * hd, (h + 1) * hd)
        sc = Q[:, sl] @ K[:, sl].T / float(np.float32(np.sqrt(hd)))
        if causal:
            sc = sc.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), -1e9)
        outs.append(torch.softmax(sc, 1) @ Vv[:, sl])
    O = torch.cat(outs, 1)
    Y = _PTDense.apply(O, Wo, bo)
    Y.backward(torch.tensor(g.astype(np.float64).reshape(T, D)))
    return Y.detach().numpy().ravel(), X.grad.numpy().ravel(), P.grad.numpy()


@pytest.mark.parametrize("T,D,NH,causal,rope,B", [(6, 8, 2, True, False, 3), (5, 12, 3, False, False, 2),
                                                  (7, 8, 2, True, True, 2), (4, 16, 1, False, True, 1)])
def test_mha_layer_vs_autograd(oracle, T, D, NH, causal, rope, B):
    rng = np.random.default_rng(T * 10 + D)
    net = oracle.Net([oracle.spec(oracle.LAYER_MHA, dim=D, num_heads=NH, seq_len=T, causal=int(causal),
                                  use_rope=int(rope))], oracle.LOSS_MSE)
    assert net.n == 4 * (D * D + D) and not net.params.any()  # Build rebinds to zeros
    p = (rng.normal(size=net.n) * 0.3).astype(np.float32)
    net.params[:] = p
    x = rng.normal(size=(B, T * D)).astype(np.float32)
    g = rng.normal(size=(B, T * D)).astype(np.float32)
    out, gin = net.accumulate_grad(x, g, B, T * D, T * D)
    grads = net.grads.copy()
    gp_ref = np.zeros(net.n)
    for b in range(B):
        o, dx, dp = _mha_torch(p, x[b], g[b], T, D, NH, causal, rope)
        assert max_rel(out[b], o) <= 1e-5
        assert max_rel(gin[b], dx) <= 1e-4
        gp_ref += dp
    gp_ref /= B
    nd = D * D + D
    for i, name in enumerate(("wQ", "wK", "wV", "wOut")):
        for part, sl in (("W", slice(i * nd, i * nd + D * D)), ("b", slice(i * nd + D * D, (i + 1) * nd))):
            ref = gp_ref[sl]
            if np.abs(ref).max() <= 1e-9 * np.abs(gp_ref).max():   # wK without RoPE: sums to 0
                assert np.abs(grads[sl]).max() <= 1e-5 * np.abs(gp_ref).max(), (name, part)
                continue
            assert max_rel(grads[sl], ref) <= 1e-4, (name, part, max_rel(grads[sl], ref))


@pytest.mark.parametrize("rows,N,B,eps", [(1, 16, 4, 1e-5), (6, 10, 3, 1e-3), (3, 64, 2, 0.0)])
def test_layernorm_layer_vs_formula(oracle, rows, N, B, eps):
    rng = np.random.default_rng(rows * 100 + N)
    net = oracle.Net([oracle.spec(oracle.LAYER_LAYERNORM, dim=N, in_size=rows * N, eps=eps)],
                     oracle.LOSS_MSE)
    np.testing.assert_array_equal(net.params[:N], 1.0)
    assert not net.params[N:].any()
    p = np.concatenate([1 + 0.3 * rng.normal(size=N), 0.3 * rng.normal(size=N)]).astype(np.float32)
    net.params[:] = p
    x = (rng.normal(size=(B, rows * N)) * 2 + 0.5).astype(np.float32)
    g = rng.normal(size=(B, rows * N)).astype(np.float32)
    out, gin = net.accumulate_grad(x, g, B, rows * N, rows * N)
    e = eps if eps > 0 else 1e-5
    X = x.astype(np.float64).reshape(B * rows, N)
    G = g.astype(np.float64).reshape(B * rows, N)
    gam, bet = p[:N].astype(np.float64), p[N:].astype(np.float64)
    mu = X.mean(1, keepdims=True)
    std = np.sqrt(((X - mu) ** 2).mean(1, keepdims=True) + e)
    xh = (X - mu) / std
    assert max_rel(out.reshape(-1, N), gam * xh + bet) <= 1e-5
    gp = G * gam
    dx = (gp - gp.sum(1, keepdims=True) / N) / std - (X - mu) * (gp * (X - mu)).sum(1, keepdims=True) / (N * std * std)
    assert max_rel(gin.reshape(-1, N), dx) <= 1e-4
    assert max_rel(net.grads[:N], (G * xh).sum(0) / B) <= 1e-4
    assert max_rel(net.grads[N:], G.sum(0) / B) <= 1e-4


def test_global_average_pooling_1d_closed_form(oracle):
    """GlobalAveragePooling1D (transformer.go:1541-1600): the float32 sum over
    the rows in order, divided by float32(seqLen); the backward spreads
    grad / seqLen over every row."""
    T, D, B = 7, 5, 3
    rng = np.random.default_rng(77)
    net = oracle.Net([oracle.spec(oracle.LAYER_GAP1D, seq_len=T, dim=D)], oracle.LOSS_MSE)
    x = rng.normal(size=(B, T * D)).astype(np.float32)
    g = rng.normal(size=(B, D)).astype(np.float32)
    out, gin = net.accumulate_grad(x, g, B, T * D, D)
    for b in range(B):
        acc = np.zeros(D, np.float32)
        for s in range(T):
            acc = (acc + x[b, s * D:(s + 1) * D]).astype(np.float32)
        np.testing.assert_array_equal(out[b], (acc / np.float32(T)).astype(np.float32))
        np.testing.assert_array_equal(gin[b], np.tile((g[b] / np.float32(T)).astype(np.float32), T))
    np.testing.assert_allclose(out, x.reshape(B, T, D).mean(axis=1), rtol=1e-6, atol=1e-6)
