"""GPU tests of the per-layer operators (the batched Layer.Forward / Backward
entry points of the C ABI) against the oracle's single-layer networks.

Each case builds a one-layer oracle network, runs its batch pass with given
output gradients (gno_net_accumulate_grad: per-sample Forward and Backward,
parameter gradients averaged over the batch, the worker chunks of
trainBatchParallel when workers > 1), and runs the operator pair on the same
inputs and parameters through ctypes.  Outputs, input gradients and every
parameter tensor are compared per tensor at 1e-4 of the reference's largest
magnitude (float32 summation order differs; integer results - argmax, ids,
masks - bit-exact)."""
import ctypes as C

import numpy as np
import pytest

from cfgutil import max_rel
from gpuutil import DBuf, TOL, log

pytestmark = pytest.mark.gpu

F = C.c_float


def _zeros(dev, shape, dtype=np.float32):
    return DBuf(dev, np.zeros(shape, dtype))


def _lib():
    from goneuron_amd._lib import check, lib
    return lib(), check


def _close(name, got, want, tol=TOL):
    e = max_rel(got, want)
    assert e <= tol, (name, e)


# ---------------------------------------------------------------- Conv2D
@pytest.mark.parametrize("B,inC,HW,outC,k,s,p,act", [
    (8, 3, 32, 16, 3, 1, 1, 1),     # the CNN config's first layer
    (5, 4, 11, 6, 5, 2, 2, 3),      # 5x5 stride 2, tanh
    (3, 2, 9, 5, 3, 2, 0, 2),       # no padding, sigmoid
    (4, 16, 16, 32, 3, 1, 1, 6)])   # linear
def test_conv2d_ops(dev, oracle, B, inC, HW, outC, k, s, p, act):
    L, check = _lib()
    log(f"conv2d B={B} inC={inC} HW={HW} outC={outC} k={k} s={s} p={p} act={act}")
    n_in = inC * HW * HW
    net = oracle.Net([oracle.spec(oracle.LAYER_CONV2D, in_size=n_in, in_channels=inC, out_channels=outC,
                                  kernel=k, stride=s, padding=p, act=act)], oracle.LOSS_MSE)
    oH = (HW + 2 * p - k) // s + 1
    n_out = outC * oH * oH
    rng = np.random.default_rng(B * 7 + HW)
    x = rng.normal(size=(B, n_in)).astype(np.float32)
    g = rng.normal(size=(B, n_out)).astype(np.float32)
    params = net.params.copy()
    out_r, gin_r = net.accumulate_grad(x, g, B, n_in, n_out)
    grads_r = net.grads.copy()
    dx, dp, dg = DBuf(dev, x), DBuf(dev, params), DBuf(dev, g)
    dout, dgr, dgin = _zeros(dev, (B, n_out)), _zeros(dev, params.shape), _zeros(dev, (B, n_in))
    check(dev.h, L.gn_conv2d_forward(dev.h, dx.p, dp.p, dout.p, B, inC, HW, HW, outC, k, s, p, act))
    check(dev.h, L.gn_conv2d_backward(dev.h, dx.p, dp.p, dout.p, dg.p, dgr.p, dgin.p, B, inC, HW, HW,
                                      outC, k, s, p, act, F(np.float32(1) / np.float32(B))))
    nw = outC * inC * k * k
    _close("out", dout.get(), out_r)
    _close("gin", dgin.get(), gin_r)
    gr = dgr.get()
    _close("dW", gr[:nw], grads_r[:nw])
    _close("db", gr[nw:], grads_r[nw:])


def test_conv2d_ops_reject_bad_geometry(dev):
    L, _ = _lib()
    rc = L.gn_conv2d_forward(dev.h, None, None, None, 1, 1, 2, 2, 1, 5, 1, 0, 1)
    assert rc != 0
    x, w, o = _zeros(dev, 4), _zeros(dev, 26), _zeros(dev, 4)
    assert L.gn_conv2d_forward(dev.h, x.p, w.p, o.p, 1, 1, 2, 2, 1, 5, 1, 0, 1) == -5  # GN_ERR_SHAPE


# ---------------------------------------------------------------- MaxPool2D
@pytest.mark.parametrize("B,C_,HW,k,s,p", [(8, 16, 32, 2, 2, 0), (3, 4, 9, 3, 2, 1), (2, 3, 7, 3, 1, 1)])
def test_maxpool2d_ops(dev, oracle, B, C_, HW, k, s, p):
    L, check = _lib()
    log(f"maxpool2d B={B} C={C_} HW={HW} k={k} s={s} p={p}")
    n_in = C_ * HW * HW
    net = oracle.Net([oracle.spec(oracle.LAYER_MAXPOOL2D, in_size=n_in, in_channels=C_, kernel=k,
                                  stride=s, padding=p)], oracle.LOSS_MSE)
    oH = (HW + 2 * p - k) // s + 1
    n_out = C_ * oH * oH
    rng = np.random.default_rng(HW * 3 + k)
    # ties in a few windows: the first maximum wins
    x = rng.integers(-3, 4, size=(B, n_in)).astype(np.float32)
    g = rng.normal(size=(B, n_out)).astype(np.float32)
    out_r, gin_r = net.accumulate_grad(x, g, B, n_in, n_out)
    am_last = net.argmax(0)
    dx, dg = DBuf(dev, x), DBuf(dev, g)
    dout, dam, dgin = _zeros(dev, (B, n_out)), _zeros(dev, (B, n_out), np.int32), _zeros(dev, (B, n_in))
    check(dev.h, L.gn_maxpool2d_forward(dev.h, dx.p, dout.p, dam.p, B, C_, HW, HW, k, s, p))
    check(dev.h, L.gn_maxpool2d_backward(dev.h, dg.p, dam.p, dgin.p, B, C_, HW, HW, k, s, p))
    np.testing.assert_array_equal(dout.get(), out_r)
    np.testing.assert_array_equal(dam.get()[-1], am_last[:n_out])
    _close("gin", dgin.get(), gin_r, 1e-6)


# ---------------------------------------------------------------- Dropout
@pytest.mark.parametrize("B,n,p", [(16, 128, 0.2), (5, 1000, 0.5), (3, 77, 0.0)])
@pytest.mark.parametrize("training", [1, 0])
def test_dropout_ops(dev, oracle, B, n, p, training):
    L, check = _lib()
    net = oracle.Net([oracle.spec(oracle.LAYER_DROPOUT, in_size=n, p=p)], oracle.LOSS_MSE)
    net.set_training(training)
    rng = np.random.default_rng(n)
    x = rng.normal(size=(B, n)).astype(np.float32)
    g = rng.normal(size=(B, n)).astype(np.float32)
    out_r, gin_r = net.accumulate_grad(x, g, B, n, n)
    dx, dg = DBuf(dev, x), DBuf(dev, g)
    dout, dmask, dgin = _zeros(dev, (B, n)), _zeros(dev, n), _zeros(dev, (B, n))
    check(dev.h, L.gn_dropout_forward(dev.h, dx.p, dout.p, dmask.p, B, n, F(p), training))
    check(dev.h, L.gn_dropout_backward(dev.h, dg.p, dmask.p, dgin.p, B, n, F(p), training))
    np.testing.assert_array_equal(dout.get(), out_r)
    np.testing.assert_array_equal(dgin.get(), gin_r)
    if training:
        m = dmask.get()
        assert set(np.unique(m)) <= {0.0, 1.0}
        np.testing.assert_array_equal(m == 0, out_r[0] == 0)  # x has no exact zeros


# ---------------------------------------------------------------- output layer + loss
@pytest.mark.parametrize("B,I,Cn,act,ptr,loss", [
    (64, 32, 10, 4, 1, 2),   # pointer Softmax + CrossEntropy (the MLP head)
    (17, 20, 7, 5, 1, 2),    # pointer LogSoftmax + CrossEntropy
    (9, 12, 5, 6, 0, 1),     # Linear + MSE
    (12, 16, 6, 2, 0, 1),    # Sigmoid + MSE
    (8, 10, 4, 4, 0, 2)])    # value Softmax (identity forward, NaN derivative) + CE
def test_softmax_ce_backward(dev, oracle, B, I, Cn, act, ptr, loss):
    """The oracle's Dense(I, Cn) head with the loss: its averaged weight
    gradient is scale * dz^T x, so dz from the operator (on the same
    pre-activations) reproduces it; the mean of loss_rows is the batch loss."""
    L, check = _lib()
    net = oracle.Net([oracle.spec(oracle.LAYER_DENSE, in_size=I, out_size=Cn, act=act, act_is_ptr=ptr)],
                     loss)
    rng = np.random.default_rng(B * Cn)
    x = rng.normal(size=(B, I)).astype(np.float32)
    if loss == 2:
        y = np.zeros((B, Cn), np.float32)
        y[np.arange(B), rng.integers(0, Cn, size=B)] = 1
    else:
        y = rng.normal(size=(B, Cn)).astype(np.float32)
    lo = net.accumulate_batch(x, y, B)
    gr = net.grads.copy()
    W, b = net.params[:Cn * I].reshape(Cn, I), net.params[Cn * I:]
    dx, dW, db, dy = DBuf(dev, x), DBuf(dev, W.copy()), DBuf(dev, b.copy()), DBuf(dev, y)
    dzo, ddz, dl = _zeros(dev, (B, Cn)), _zeros(dev, (B, Cn)), _zeros(dev, B)
    check(dev.h, L.gn_dense_forward(dev.h, dx.p, dW.p, db.p, dzo.p, B, I, Cn, 6, 0))  # pre-activations
    check(dev.h, L.gn_softmax_ce_backward(dev.h, dzo.p, dy.p, ddz.p, dl.p, B, Cn, act, ptr, loss))
    dz = ddz.get().astype(np.float64)
    rows = dl.get()
    if act == 4 and not ptr:  # NaN derivative: every gradient NaN on both sides
        assert np.isnan(dz).all() and np.isnan(gr).all()
        assert abs(rows.mean() - lo) <= TOL * abs(lo)
        return
    assert abs(rows.astype(np.float64).mean() - lo) <= TOL * abs(lo), (rows.mean(), lo)
    _close("dW", (dz.T @ x.astype(np.float64) / B).ravel(), gr[:Cn * I])
    _close("db", dz.sum(0) / B, gr[Cn * I:])


# ---------------------------------------------------------------- LayerNorm
@pytest.mark.parametrize("B,rows,N,eps", [(8, 16, 64, 1e-5), (3, 5, 10, 1e-3), (4, 1, 300, 0.0)])
def test_layernorm_ops(dev, oracle, B, rows, N, eps):
    L, check = _lib()
    net = oracle.Net([oracle.spec(oracle.LAYER_LAYERNORM, dim=N, in_size=rows * N, eps=eps)],
                     oracle.LOSS_MSE)
    rng = np.random.default_rng(rows * N)
    p = np.concatenate([1 + 0.3 * rng.normal(size=N), 0.3 * rng.normal(size=N)]).astype(np.float32)
    net.params[:] = p
    x = (rng.normal(size=(B, rows * N)) * 2 + 0.5).astype(np.float32)
    g = rng.normal(size=(B, rows * N)).astype(np.float32)
    out_r, gin_r = net.accumulate_grad(x, g, B, rows * N, rows * N)
    gr = net.grads.copy()
    R = B * rows
    dx, dgam, dbet, dg = DBuf(dev, x), DBuf(dev, p[:N]), DBuf(dev, p[N:]), DBuf(dev, g)
    dy, dst, ddx = _zeros(dev, (B, rows * N)), _zeros(dev, 2 * R), _zeros(dev, (B, rows * N))
    dgg, dgb, dwk = _zeros(dev, N), _zeros(dev, N), _zeros(dev, (R, N))
    check(dev.h, L.gn_layernorm_forward(dev.h, dx.p, dgam.p, dbet.p, dy.p, dst.p, R, N, F(eps)))
    check(dev.h, L.gn_layernorm_backward(dev.h, dg.p, dx.p, dgam.p, dst.p, ddx.p, dgg.p, dgb.p, dwk.p,
                                         R, N, F(np.float32(1) / np.float32(B))))
    _close("out", dy.get(), out_r)
    _close("gin", ddx.get(), gin_r)
    _close("dgamma", dgg.get(), gr[:N])
    _close("dbeta", dgb.get(), gr[N:])


# ---------------------------------------------------------------- MultiHeadAttention
@pytest.mark.parametrize("B,T,D,NH,causal,rope", [
    (4, 16, 64, 4, 1, 0), (3, 32, 64, 2, 0, 0), (2, 12, 48, 3, 1, 1), (5, 8, 32, 1, 0, 1),
    # beyond the fused kernels (T > 128 or heads wider than 32): the batched-GEMM path
    (2, 136, 80, 2, 1, 0), (3, 40, 128, 2, 0, 1), (1, 200, 96, 3, 1, 1)])
def test_mha_ops(dev, oracle, B, T, D, NH, causal, rope):
    L, check = _lib()
    log(f"mha B={B} T={T} D={D} heads={NH} causal={causal} rope={rope}")
    net = oracle.Net([oracle.spec(oracle.LAYER_MHA, dim=D, num_heads=NH, seq_len=T, causal=causal,
                                  use_rope=rope)], oracle.LOSS_MSE)
    rng = np.random.default_rng(T * D + NH)
    p = (rng.normal(size=net.n) * (0.5 / np.sqrt(D))).astype(np.float32)
    net.params[:] = p
    x = rng.normal(size=(B, T * D)).astype(np.float32)
    g = rng.normal(size=(B, T * D)).astype(np.float32)
    out_r, gin_r = net.accumulate_grad(x, g, B, T * D, T * D)
    gr = net.grads.copy()
    ws = C.c_int64()
    check(None, L.gn_mha_workspace(B, T, D, NH, rope, C.byref(ws)))
    dx, dp, dg = DBuf(dev, x), DBuf(dev, p), DBuf(dev, g)
    dout, dgr, dgin, dwk = (_zeros(dev, (B, T * D)), _zeros(dev, p.shape), _zeros(dev, (B, T * D)),
                            _zeros(dev, ws.value))
    check(dev.h, L.gn_mha_forward(dev.h, dx.p, dp.p, dout.p, dwk.p, B, T, D, NH, causal, rope))
    check(dev.h, L.gn_mha_backward(dev.h, dx.p, dp.p, dg.p, dgr.p, dgin.p, dwk.p, B, T, D, NH, causal,
                                   rope, F(np.float32(1) / np.float32(B))))
    _close("out", dout.get(), out_r)
    _close("gin", dgin.get(), gin_r)
    got = dgr.get()
    nd = D * D + D
    scale = np.abs(gr).max()
    for i, name in enumerate(("wQ", "wK", "wV", "wOut")):
        for part, sl in (("W", slice(i * nd, i * nd + D * D)), ("b", slice(i * nd + D * D, (i + 1) * nd))):
            ref = gr[sl]
            if np.abs(ref).max() <= 1e-6 * scale:  # wK without RoPE: the softmax rows sum it to zero
                assert np.abs(got[sl]).max() <= 1e-5 * scale, (name, part)
                continue
            _close(name + "." + part, got[sl], ref)


@pytest.mark.parametrize("D,NH,T", [(128, 2, 2), (64, 2, 4)])
def test_mha_ops_beyond_grid_limit(dev, oracle, D, NH, T):
    """More (sample, head) pairs than a grid dimension holds (33,000 samples x
    2 heads): the batched-GEMM path (heads 64 wide) runs the pairs in chunks,
    the fused path (heads 32 wide) takes them on the grid's x dimension.  The
    batch repeats 10 distinct samples 3,300 times, so every output row equals
    its distinct sample's and the batch-averaged gradients equal the 10-sample
    batch's, which the oracle computes."""
    L, check = _lib()
    nd, reps = 10, 3300
    B = nd * reps
    log(f"mha B={B} T={T} D={D} heads={NH}: {B * NH} (sample, head) pairs")
    net = oracle.Net([oracle.spec(oracle.LAYER_MHA, dim=D, num_heads=NH, seq_len=T, causal=1, use_rope=0)],
                     oracle.LOSS_MSE)
    rng = np.random.default_rng(D + T)
    p = (rng.normal(size=net.n) * (0.5 / np.sqrt(D))).astype(np.float32)
    net.params[:] = p
    x0 = rng.normal(size=(nd, T * D)).astype(np.float32)
    g0 = rng.normal(size=(nd, T * D)).astype(np.float32)
    out_r, gin_r = net.accumulate_grad(x0, g0, nd, T * D, T * D)
    gr = net.grads.copy()
    x, g = np.tile(x0, (reps, 1)), np.tile(g0, (reps, 1))
    ws = C.c_int64()
    check(None, L.gn_mha_workspace(B, T, D, NH, 0, C.byref(ws)))
    dx, dp, dg = DBuf(dev, x), DBuf(dev, p), DBuf(dev, g)
    dout, dgr, dgin, dwk = (_zeros(dev, (B, T * D)), _zeros(dev, p.shape), _zeros(dev, (B, T * D)),
                            _zeros(dev, ws.value))
    check(dev.h, L.gn_mha_forward(dev.h, dx.p, dp.p, dout.p, dwk.p, B, T, D, NH, 1, 0))
    check(dev.h, L.gn_mha_backward(dev.h, dx.p, dp.p, dg.p, dgr.p, dgin.p, dwk.p, B, T, D, NH, 1, 0,
                                   F(np.float32(1) / np.float32(B))))
    out, gin = dout.get().reshape(reps, nd, T * D), dgin.get().reshape(reps, nd, T * D)
    for r in (0, reps // 2, reps - 1):  # first, middle and last copies (the last chunk of pairs)
        _close(f"out[{r}]", out[r], out_r)
        _close(f"gin[{r}]", gin[r], gin_r)
    # the parameter gradients sum B = 33,000 per-sample terms in float32, in
    # sample order as the reference's batch loop does: that sum's own
    # rounding reaches about B * 2^-24 of its value (the 10-sample oracle sum
    # has almost none), so that is the tolerance here
    gtol = max(TOL, B * 2.0 ** -24)
    got = dgr.get()
    nd4 = D * D + D
    for i, name in enumerate(("wQ", "wK", "wV", "wOut")):
        for part, sl in (("W", slice(i * nd4, i * nd4 + D * D)), ("b", slice(i * nd4 + D * D, (i + 1) * nd4))):
            ref = gr[sl]
            if np.abs(ref).max() <= 1e-6 * np.abs(gr).max():
                continue
            _close(name + "." + part, got[sl], ref, gtol)


# ---------------------------------------------------------------- SequenceUnroller(LSTM)
@pytest.mark.parametrize("B,T,I,H,workers,gscale,seq", [
    (6, 10, 8, 16, 1, 1e-3, 0),   # clip inactive
    (6, 10, 8, 16, 1, 3.0, 0),    # clip active on one chain
    (8, 7, 5, 12, 4, 3.0, 0),     # four worker chains, clip active
    (5, 12, 6, 32, 2, 0.3, 0),
    (6, 9, 8, 16, 1, 0.5, 1),     # returnSequences: every step's h out, a gradient per step in
    (7, 6, 5, 24, 3, 2.0, 1)])
def test_lstm_seq_ops(dev, oracle, B, T, I, H, workers, gscale, seq):
    L, check = _lib()
    log(f"lstm B={B} T={T} I={I} H={H} workers={workers} gscale={gscale} seq={seq}")
    net = oracle.Net([oracle.spec(oracle.LAYER_LSTM_UNROLLER, in_size=I, out_size=H, seq_len=T,
                                  return_sequences=seq)], oracle.LOSS_MSE, workers=workers)
    rng = np.random.default_rng(T * H + workers)
    p = (rng.normal(size=net.n) * 0.3).astype(np.float32)  # every gate live
    net.params[:] = p
    x = rng.normal(size=(B, T * I)).astype(np.float32)
    OL = T * H if seq else H
    g = (rng.normal(size=(B, OL)) * gscale).astype(np.float32)
    out_r, gin_r = net.accumulate_grad(x, g, B, T * I, OL)
    gr = net.grads.copy()
    ws = C.c_int64()
    check(None, L.gn_lstm_workspace(B, T, I, H, workers, C.byref(ws)))
    dx, dp, dg = DBuf(dev, x), DBuf(dev, p), DBuf(dev, g)
    dout, dgr, dgin, dwk = (_zeros(dev, (B, OL)), _zeros(dev, p.shape), _zeros(dev, (B, T * I)),
                            _zeros(dev, ws.value))
    check(dev.h, L.gn_lstm_seq_forward(dev.h, dx.p, dp.p, dout.p, dwk.p, B, T, I, H, seq))
    check(dev.h, L.gn_lstm_seq_backward(dev.h, dx.p, dp.p, dg.p, dgr.p, dgin.p, dwk.p, B, T, I, H, workers,
                                        F(np.float32(1) / np.float32(B)), seq))
    _close("out", dout.get(), out_r)
    _close("gin", dgin.get(), gin_r)
    got = dgr.get()
    nwx, nwh = 4 * H * I, 4 * H * H
    for gi, gname in enumerate("ifgo"):
        for part, sl in (("Wx", slice(gi * H * I, (gi + 1) * H * I)),
                         ("Wh", slice(nwx + gi * H * H, nwx + (gi + 1) * H * H)),
                         ("b", slice(nwx + nwh + gi * H, nwx + nwh + (gi + 1) * H))):
            _close(part + "_" + gname, got[sl], gr[sl])


# ---------------------------------------------------------------- Embedding
@pytest.mark.parametrize("B,T,V,D,workers,bad", [
    (8, 16, 100, 32, 1, False), (10, 6, 50, 16, 4, False), (9, 5, 40, 8, 3, True), (7, 4, 30, 8, 1, True),
    # more than 2048 contributing rows (64 worker chunks x 40 tokens): the global row lists
    (64, 40, 700, 24, 64, False), (128, 40, 300, 20, 64, True)])
def test_embedding_ops(dev, oracle, B, T, V, D, workers, bad):
    """Forward rows bit-exact; the table gradient is the last sample of each
    worker chunk (Backward zeroes it first).  With an out-of-range id in some
    samples, `bad` flags them; the sequential loop skips them (continue) and
    a worker stops at its first one."""
    L, check = _lib()
    net = oracle.Net([oracle.spec(oracle.LAYER_EMBEDDING, in_size=T, vocab=V, dim=D)], oracle.LOSS_MSE,
                     workers=workers)
    rng = np.random.default_rng(B * T + V)
    ids = rng.integers(0, V, size=(B, T))
    if bad:
        ids[1, 2] = V + 3
        ids[B - 1, 0] = -1
    x = ids.astype(np.float32)
    g = rng.normal(size=(B, T * D)).astype(np.float32)
    E = net.params.copy()
    out_r, _ = net.accumulate_grad(x, g, B, T, T * D)
    gr = net.grads.copy()
    dxb, dE, dg = DBuf(dev, x), DBuf(dev, E), DBuf(dev, g)
    dout, dids, dbad, dgE = (_zeros(dev, (B, T * D)), _zeros(dev, (B, T), np.int32), _zeros(dev, B, np.int32),
                             _zeros(dev, E.shape))
    check(dev.h, L.gn_embedding_forward(dev.h, dxb.p, dE.p, dout.p, dids.p, dbad.p, B, T, V, D))
    check(dev.h, L.gn_embedding_backward(dev.h, dg.p, dids.p, dbad.p, dgE.p, B, T, V, D, workers,
                                         F(np.float32(1) / np.float32(B))))
    flags = dbad.get()
    want_bad = ((ids < 0) | (ids >= V)).any(1).astype(np.int32)
    np.testing.assert_array_equal(flags, want_bad)
    # samples the reference's loop runs: all good ones when sequential; in a
    # worker chunk, those before its first bad sample
    ok = want_bad == 0
    if workers > 1:
        chunk = -(-B // min(workers, B))
        for c0 in range(0, B, chunk):
            hit = np.nonzero(want_bad[c0:c0 + chunk])[0]
            if hit.size:
                ok[c0 + hit[0]:c0 + chunk] = False
    np.testing.assert_array_equal(dout.get()[ok], out_r[ok])
    np.testing.assert_array_equal(dids.get()[ok], ids[ok])
    _close("gradE", dgE.get(), gr, 1e-6)


# ---------------------------------------------------------------- AvgPool2D
@pytest.mark.parametrize("B,C,HW,k,s,p", [(4, 3, 8, 2, 2, 0), (3, 2, 9, 3, 2, 1), (5, 4, 7, 3, 1, 1)])
def test_avgpool2d_ops(dev, oracle, B, C, HW, k, s, p):
    L, check = _lib()
    net = oracle.Net([oracle.spec(oracle.LAYER_AVGPOOL2D, in_channels=C, kernel=k, stride=s, padding=p,
                                  in_size=C * HW * HW)], oracle.LOSS_MSE)
    o = (HW + 2 * p - k) // s + 1
    rng = np.random.default_rng(B * C + HW)
    x = rng.normal(size=(B, C * HW * HW)).astype(np.float32)
    g = rng.normal(size=(B, C * o * o)).astype(np.float32)
    out_r, gin_r = net.accumulate_grad(x, g, B, C * HW * HW, C * o * o)
    dx, dg = DBuf(dev, x), DBuf(dev, g)
    dout, dgin = _zeros(dev, (B, C * o * o)), _zeros(dev, (B, C * HW * HW))
    check(dev.h, L.gn_avgpool2d_forward(dev.h, dx.p, dout.p, B, C, HW, HW, k, s, p))
    check(dev.h, L.gn_avgpool2d_backward(dev.h, dg.p, dgin.p, B, C, HW, HW, k, s, p))
    _close("out", dout.get(), out_r, 1e-6)
    _close("gin", dgin.get(), gin_r, 1e-6)


# ---------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("B,rows,N", [(4, 3, 16), (6, 1, 100), (2, 5, 33)])
def test_rmsnorm_ops(dev, oracle, B, rows, N):
    L, check = _lib()
    net = oracle.Net([oracle.spec(oracle.LAYER_RMSNORM, dim=N, in_size=rows * N)], oracle.LOSS_MSE)
    rng = np.random.default_rng(rows * N + B)
    p = (1 + 0.3 * rng.normal(size=N)).astype(np.float32)  # gamma away from 1 (Q19 differs there)
    net.params[:] = p
    x = (rng.normal(size=(B, rows * N)) + 0.2).astype(np.float32)
    g = rng.normal(size=(B, rows * N)).astype(np.float32)
    out_r, gin_r = net.accumulate_grad(x, g, B, rows * N, rows * N)
    gr = net.grads.copy()
    R = B * rows
    dx, dgam, dg = DBuf(dev, x), DBuf(dev, p), DBuf(dev, g)
    dy, drms, ddx, dgg, dwk = (_zeros(dev, (B, rows * N)), _zeros(dev, R), _zeros(dev, (B, rows * N)),
                               _zeros(dev, N), _zeros(dev, (R, N)))
    check(dev.h, L.gn_rmsnorm_forward(dev.h, dx.p, dgam.p, dy.p, drms.p, R, N, F(1e-5)))
    check(dev.h, L.gn_rmsnorm_backward(dev.h, dg.p, dx.p, dgam.p, drms.p, ddx.p, dgg.p, dwk.p, R, N,
                                       F(np.float32(1) / np.float32(B))))
    _close("out", dy.get(), out_r)
    _close("gin", ddx.get(), gin_r)
    _close("dgamma", dgg.get(), gr)


# ---------------------------------------------------------------- SwiGLU
@pytest.mark.parametrize("B,I,O", [(8, 16, 12), (5, 33, 7), (64, 128, 96)])
def test_swiglu_ops(dev, oracle, B, I, O):
    L, check = _lib()
    net = oracle.Net([oracle.spec(oracle.LAYER_SWIGLU, in_size=I, out_size=O)], oracle.LOSS_MSE)
    rng = np.random.default_rng(I * O + B)
    p = net.params.copy()  # the reference's init
    x = rng.normal(size=(B, I)).astype(np.float32)
    g = rng.normal(size=(B, O)).astype(np.float32)
    out_r, gin_r = net.accumulate_grad(x, g, B, I, O)
    gr = net.grads.copy()
    ws = C.c_int64()
    check(None, L.gn_swiglu_workspace(B, O, C.byref(ws)))
    dx, dp, dg = DBuf(dev, x), DBuf(dev, p), DBuf(dev, g)
    dout, dgr, dgin, dwk = _zeros(dev, (B, O)), _zeros(dev, p.shape), _zeros(dev, (B, I)), _zeros(dev, ws.value)
    check(dev.h, L.gn_swiglu_forward(dev.h, dx.p, dp.p, dout.p, dwk.p, B, I, O))
    check(dev.h, L.gn_swiglu_backward(dev.h, dx.p, dp.p, dg.p, dgr.p, dgin.p, dwk.p, B, I, O,
                                      F(np.float32(1) / np.float32(B))))
    _close("out", dout.get(), out_r)
    _close("gin", dgin.get(), gin_r)
    got = dgr.get()
    _close("dW", got[:I * O], gr[:I * O])
    _close("dV", got[I * O:], gr[I * O:])


# ---------------------------------------------------------------- BatchNorm2D
@pytest.mark.parametrize("B,Cc,HW,affine,training", [(4, 3, 25, True, True), (6, 8, 16, False, True),
                                                      (3, 5, 36, True, False)])
def test_batchnorm2d_ops(dev, oracle, B, Cc, HW, affine, training):
    """Training: per-sample statistics (Q22) and the running statistics
    advanced per sample in sample order; inference: the running statistics,
    dx only."""
    L, check = _lib()
    net = oracle.Net([oracle.spec(oracle.LAYER_BATCHNORM2D, in_channels=Cc, momentum=0.1, in_size=Cc * HW,
                                  no_affine=int(not affine))], oracle.LOSS_MSE)
    rng = np.random.default_rng(B * Cc + HW)
    if affine:
        p = np.concatenate([1 + 0.2 * rng.normal(size=Cc), 0.2 * rng.normal(size=Cc)]).astype(np.float32)
        net.params[:] = p
    x = (rng.normal(size=(B, Cc * HW)) * 1.5 + 0.3).astype(np.float32)
    g = rng.normal(size=(B, Cc * HW)).astype(np.float32)
    rm0, rv0 = np.zeros(Cc, np.float32), np.ones(Cc, np.float32)
    if not training:
        # running statistics from a training pass first, on both sides
        net.accumulate_grad(x[::-1].copy(), g, B, Cc * HW, Cc * HW)
        rm0, rv0 = net.running_stats(0)
        net.set_training(False)
    out_r, gin_r = net.accumulate_grad(x, g, B, Cc * HW, Cc * HW)
    gr = net.grads.copy()
    rm_r, rv_r = net.running_stats(0)
    dx, dg = DBuf(dev, x), DBuf(dev, g)
    dp = DBuf(dev, p) if affine else None
    drm, drv = DBuf(dev, rm0), DBuf(dev, rv0)
    dout, dst, dgin, dwk = (_zeros(dev, (B, Cc * HW)), _zeros(dev, 3 * B * Cc), _zeros(dev, (B, Cc * HW)),
                            _zeros(dev, 2 * B * Cc))
    dgr = _zeros(dev, 2 * Cc) if affine else None
    pp = dp.p if affine else None
    check(dev.h, L.gn_batchnorm2d_forward(dev.h, dx.p, pp, dout.p, dst.p, drm.p, drv.p, B, Cc, HW, F(1e-5),
                                          F(0.1), int(training)))
    check(dev.h, L.gn_batchnorm2d_backward(dev.h, dg.p, dx.p, pp, dst.p, drv.p, dgr.p if affine else None,
                                           dgin.p, dwk.p, B, Cc, HW, F(1e-5), int(training),
                                           F(np.float32(1) / np.float32(B))))
    _close("out", dout.get(), out_r)
    _close("gin", dgin.get(), gin_r)
    _close("running_mean", drm.get(), rm_r, 1e-5)
    _close("running_var", drv.get(), rv_r, 1e-5)
    if affine:
        got = dgr.get()
        if training:
            _close("dgamma", got[:Cc], gr[:Cc])
            _close("dbeta", got[Cc:], gr[Cc:])
        else:
            assert not got.any()


# ---------------------------------------------------------------- SequenceUnroller(GRU)
@pytest.mark.parametrize("B,T,I,H,seq", [(6, 8, 5, 12, 0), (4, 5, 7, 32, 1), (9, 12, 16, 64, 0)])
def test_gru_seq_ops(dev, oracle, B, T, I, H, seq):
    L, check = _lib()
    net = oracle.Net([oracle.spec(oracle.LAYER_GRU_UNROLLER, in_size=I, out_size=H, seq_len=T,
                                  return_sequences=seq)], oracle.LOSS_MSE)
    rng = np.random.default_rng(T * H + I)
    p = (rng.normal(size=net.n) * 0.2).astype(np.float32)
    net.params[:] = p
    x = rng.normal(size=(B, T * I)).astype(np.float32)
    OL = T * H if seq else H
    g = rng.normal(size=(B, OL)).astype(np.float32)
    out_r, gin_r = net.accumulate_grad(x, g, B, T * I, OL)
    gr = net.grads.copy()
    ws = C.c_int64()
    check(None, L.gn_gru_workspace(B, T, I, H, C.byref(ws)))
    dx, dp, dg = DBuf(dev, x), DBuf(dev, p), DBuf(dev, g)
    dout, dgr, dgin, dwk = (_zeros(dev, (B, OL)), _zeros(dev, p.shape), _zeros(dev, (B, T * I)),
                            _zeros(dev, ws.value))
    check(dev.h, L.gn_gru_seq_forward(dev.h, dx.p, dp.p, dout.p, dwk.p, B, T, I, H, seq))
    check(dev.h, L.gn_gru_seq_backward(dev.h, dx.p, dp.p, dg.p, dgr.p, dgin.p, dwk.p, B, T, I, H,
                                       F(np.float32(1) / np.float32(B)), seq))
    _close("out", dout.get(), out_r)
    _close("gin", dgin.get(), gin_r)
    got = dgr.get()
    nwx, nwh = 3 * H * I, 2 * H * H
    for gi, gname in enumerate("urc"):
        sl = slice(gi * H * I, (gi + 1) * H * I)
        if gname == "r":  # Q24: the reset gate's input weights get no gradient
            assert not got[sl].any() and not gr[sl].any()
            continue
        _close("Wx_" + gname, got[sl], gr[sl])
    for gi, gname in enumerate("ur"):
        sl = slice(nwx + gi * H * H, nwx + (gi + 1) * H * H)
        _close("Wh_" + gname, got[sl], gr[sl])
    _close("b", got[nwx + nwh:], gr[nwx + nwh:])


# ---------------------------------------------------------------- MoE
@pytest.mark.parametrize("B,I,O,E,K,training", [(8, 10, 6, 4, 2, True), (12, 16, 8, 8, 3, False),
                                                 (5, 7, 5, 3, 1, True)])
def test_moe_ops(dev, oracle, B, I, O, E, K, training):
    """Routes bit-exact (gate noise from the layer's RNG(42) stream in
    training, the stream advanced by E draws per sample)."""
    L, check = _lib()
    net = oracle.Net([oracle.spec(oracle.LAYER_MOE, in_size=I, out_size=O, num_experts=E, top_k=K)],
                     oracle.LOSS_MSE)
    net.set_training(training)
    rng = np.random.default_rng(B * E + K)
    p = (rng.normal(size=net.n) * 0.4).astype(np.float32)  # the reference starts at 0: live experts
    net.params[:] = p
    x = rng.normal(size=(B, I)).astype(np.float32)
    g = rng.normal(size=(B, O)).astype(np.float32)
    net.routes(0)
    out_r, gin_r = net.accumulate_grad(x, g, B, I, O)
    gr = net.grads.copy()
    routes_r = net.routes(0).reshape(B, K)
    ws = C.c_int64()
    check(None, L.gn_moe_workspace(B, I, O, E, K, C.byref(ws)))
    dx, dp, dg = DBuf(dev, x), DBuf(dev, p), DBuf(dev, g)
    dout, dgr, dgin, dwk = _zeros(dev, (B, O)), _zeros(dev, p.shape), _zeros(dev, (B, I)), _zeros(dev, ws.value)
    noise = C.c_uint64(42)
    check(dev.h, L.gn_moe_forward(dev.h, dx.p, dp.p, dout.p, dwk.p, B, I, O, E, K, int(training),
                                  C.byref(noise)))
    check(dev.h, L.gn_moe_backward(dev.h, dx.p, dp.p, dg.p, dgr.p, dgin.p, dwk.p, B, I, O, E, K, int(training),
                                   F(np.float32(1) / np.float32(B))))
    s = 42
    if training:
        for _ in range(B * E):
            s = (s * 6364136223846793005 + 1) % (1 << 64)
    assert noise.value == s
    # the routes sit at the end of the workspace, after the float regions
    wk = dwk.get()
    off = sum(-(-n // 64) * 64 for n in (B * E, B * E, B * E, E * B * O, E * B * O))
    np.testing.assert_array_equal(wk[off:off + B * K].view(np.int32).reshape(B, K), routes_r)
    _close("out", dout.get(), out_r)
    _close("gin", dgin.get(), gin_r)
    _close("grads", dgr.get(), gr)
