"""Pins the oracle's BPTT recursions (SequenceUnroller over LSTM and GRU, with a
Dense head and MSE) against float64 torch autograd.

Each torch model computes the reference's forward values and, through
zero-valued terms of the form ``v - v.detach()`` (value 0, gradient that of
``v``) or detached factors, exactly the gradient the reference's hand-written
backward produces.  Only the quirks are written by hand; every per-step
derivative (sigmoid', tanh', the cell chain, Wh^T dG, the Dense head, MSE) is
autograd's.  Each test also shows that the textbook recurrence gives different
gradients, so a dropped quirk fails it.

LSTM (internal/layer/lstm.go, unroller.go):
  Q13  only the input gate adds Wx x + Wh h to its bias (lstmComputeInputGates
       loops over the first outSize rows, lstm.go:1065-1101); f, g, o keep the
       bias as value, but the backward gives them the full LSTM's gradient
       (lstm.go:560-606) -> pre = b + (z - z.detach()) on those gates;
  Q10  the input-weight gradient uses inputBuf, the last step's input
       (lstm.go:612-640) -> Wx x_t in value, Wx x_{T-1} in gradient;
  Q15  LSTM.Backward adds dhPrev into the caller's gradient (lstm.go:727-730)
       and the unroller carries that buffer to the previous step
       (unroller.go:189-206): dh_{t-1} = dh_t + Wh^T dG -> h_t + (h_{t-1} -
       h_{t-1}.detach());
  Q14  clipGradients scales the layer's cumulative gradient to norm 1 after
       every step (lstm.go:732-761): checked with the clip active by taking
       autograd's per-step pre-activation gradients dG_t, forming each step's
       contribution [dG x_last | dG h_{t-1} | dG] and clipping the running sum
       (worker chain order: samples in order, steps T-1 .. 0).
GRU (internal/layer/gru.go, unroller.go):
  Q23  the candidate's delta weights dh by (1 - u) and the direct path by u
       (gru.go:397-411, 519-520) while the forward is h + u (c - h);
  Q24  the reset delta is never computed (gru.go:437-447): no gradient into the
       reset gate; input weights use the last step's input (gru.go:433-454);
       the candidate's use of the reset block reaches dh_prev as
       Wh_r[j][i] dC[j] r[j] (row index j, gru.go:515-517);
  carry dh_{t-1} = dh_t + dhPrev (gru.go:524-527, unroller.go:189-206).
"""
import math

import numpy as np
import pytest

from cfgutil import max_rel

torch = pytest.importorskip("torch")
from recurrent_ref import (_clip_chain, _gru_params, _gru_torch, _lstm_params,  # noqa: E402
                           _lstm_torch)


def _lstm_net(oracle, I, H, T, workers=1):
    return oracle.Net([oracle.spec(oracle.LAYER_LSTM_UNROLLER, in_size=I, out_size=H, seq_len=T),
                       oracle.spec(oracle.LAYER_DENSE, in_size=H, out_size=1, act=oracle.ACT_LINEAR)],
                      oracle.LOSS_MSE, workers=workers)


def _lstm_parts(I, H):
    nwx, nwh = 4 * H * I, 4 * H * H
    parts = {}
    for gi, gname in enumerate("ifgo"):
        parts["Wx_" + gname] = np.s_[gi * H * I:(gi + 1) * H * I]
        parts["Wh_" + gname] = np.s_[nwx + gi * H * H:nwx + (gi + 1) * H * H]
        parts["b_" + gname] = np.s_[nwx + nwh + gi * H:nwx + nwh + (gi + 1) * H]
    parts["dense_W"] = np.s_[nwx + nwh + 4 * H:nwx + nwh + 5 * H]
    parts["dense_b"] = np.s_[nwx + nwh + 5 * H:nwx + nwh + 5 * H + 1]
    return parts


def _check_parts(got, ref, parts, tol=1e-4):
    errs = {k: max_rel(got[s], ref[s]) for k, s in parts.items()}
    bad = {k: e for k, e in errs.items() if e > tol}
    assert not bad, bad
    return errs


@pytest.mark.parametrize("T,I,H,B", [(6, 5, 7, 3), (9, 4, 6, 2), (12, 3, 5, 1)])
def test_lstm_bptt_vs_autograd_clip_inactive(oracle, T, I, H, B):
    """Random parameters (every gate live, non-zero cell-gate bias), targets a
    small step from the predictions so the cumulative gradient stays far
    below the clip norm; every gate block of Wx, Wh, b and the Dense head to
    1e-4 of float64 autograd."""
    rng = np.random.default_rng(100 + T)
    p = _lstm_params(rng, I, H)
    x = rng.normal(size=(B, T * I)).astype(np.float32)
    net = _lstm_net(oracle, I, H, T)
    net.params[:] = p
    # predictions first, then targets 1e-3 away
    preds = np.array([net.forward(x[b])[0] for b in range(B)], np.float32)
    y = (preds + 1e-3 * rng.choice([-1.0, 1.0], size=B)).astype(np.float32)
    loss = net.accumulate_batch(x, y.reshape(B, 1), B)
    g = net.grads.copy()
    nl = 4 * H * (I + H) + 4 * H
    assert np.linalg.norm(g[:nl]) * B < 0.05  # the clip never acts
    l_ref, g_ref, _, _ = _lstm_torch(p, x, y, I, H, T)
    assert abs(loss - l_ref) <= 1e-4 * abs(l_ref)
    _check_parts(g, g_ref, _lstm_parts(I, H))
    # the textbook LSTM (all gates from Wx x + Wh h, own-step inputs, no
    # carried dh) gives other gradients: the quirks are what is pinned
    _, g_std, _, _ = _lstm_torch(p, x, y, I, H, T, reference=False)
    assert max_rel(g[:nl], g_std[:nl]) > 1e-2


@pytest.mark.parametrize("workers", [1, 2, 3])
def test_lstm_bptt_with_clip_active(oracle, workers):
    """Large targets: the per-step clip acts.  The recursion's deltas come from
    autograd (the clip never feeds back into it); each step contributes
    [dG (x) x_{T-1} | dG (x) h_{t-1} | dG]; each worker chain clips its running
    sum after every step; the chains are summed and averaged over B."""
    T, I, H, B = 7, 4, 6, 6
    rng = np.random.default_rng(77)
    p = _lstm_params(rng, I, H, scale=0.5)
    x = rng.normal(size=(B, T * I)).astype(np.float32)
    y = (rng.normal(size=B) * 30).astype(np.float32)
    net = _lstm_net(oracle, I, H, T, workers=workers)
    net.params[:] = p
    net.accumulate_batch(x, y.reshape(B, 1), B)
    g = net.grads.copy()
    _, g_ref, dpre, hs = _lstm_torch(p, x, y, I, H, T, keep_pre=True)
    X = x.astype(np.float64).reshape(B, T, I)
    W = min(workers, B)
    chunk = (B + W - 1) // W
    nl = 4 * H * (I + H) + 4 * H
    total = np.zeros(nl)
    active = 0
    for c0 in range(0, B, chunk):
        deltas = []
        for bb in range(c0, min(B, c0 + chunk)):
            for t in range(T - 1, -1, -1):
                dg = dpre[t][bb]
                deltas.append(np.concatenate([np.outer(dg, X[bb, T - 1]).ravel(),
                                              np.outer(dg, hs[t][bb]).ravel(), dg]))
        total += _clip_chain(deltas)
        run = np.cumsum(np.stack(deltas), axis=0)
        active += int((np.linalg.norm(run, axis=1) > 1).sum())
    assert active > 0  # the clip acted somewhere in every configuration
    ref = g_ref.copy()
    ref[:nl] = total / B
    _check_parts(g, ref, _lstm_parts(I, H))


@pytest.mark.parametrize("T,I,H,B,workers", [(6, 5, 7, 3, 1), (8, 4, 6, 4, 2)])
def test_lstm_input_gradient_vs_autograd(oracle, T, I, H, B, workers):
    """The unroller's input gradient (lstm.go:642-663, unroller.go:189-206):
    dx_t = Wx^T dG_t over all four gates with autograd's per-step
    pre-activation gradients dG_t, the clip (which scales parameter
    gradients only) acting or not.  The output gradient given to the oracle
    is the per-sample MSE gradient 2 (pred - y) of the torch model's loss."""
    rng = np.random.default_rng(300 + T)
    p = _lstm_params(rng, I, H)
    x = rng.normal(size=(B, T * I)).astype(np.float32)
    y = (rng.normal(size=B) * 5).astype(np.float32)
    net = _lstm_net(oracle, I, H, T, workers=workers)
    net.params[:] = p
    preds = np.array([net.forward(x[b])[0] for b in range(B)], np.float32)
    gout = (2 * (preds - y)).astype(np.float32).reshape(B, 1)
    _, gin = net.accumulate_grad(x, gout, B, T * I, 1)
    _, _, dpre, _ = _lstm_torch(p, x, y, I, H, T, keep_pre=True)
    Wx = p[:4 * H * I].astype(np.float64).reshape(4 * H, I)
    ref = np.stack([np.stack([dpre[t][b] @ Wx for t in range(T)]) for b in range(B)]).reshape(B, T * I)
    assert max_rel(gin, ref) <= 1e-4, max_rel(gin, ref)
    # the input gate alone (a dropped gate sum) or the own-step weights differ
    only_i = np.stack([np.stack([dpre[t][b][:H] @ Wx[:H] for t in range(T)]) for b in range(B)])
    assert max_rel(gin, only_i.reshape(B, T * I)) > 1e-2


def _gru_parts(I, H):
    nwx, nwh = 3 * H * I, 2 * H * H
    parts = {}
    for gi, gname in enumerate("urc"):
        parts["Wx_" + gname] = np.s_[gi * H * I:(gi + 1) * H * I]
        parts["b_" + gname] = np.s_[nwx + nwh + gi * H:nwx + nwh + (gi + 1) * H]
    parts["Wh_u"] = np.s_[nwx:nwx + H * H]
    parts["Wh_r"] = np.s_[nwx + H * H:nwx + nwh]
    parts["dense_W"] = np.s_[nwx + nwh + 3 * H:nwx + nwh + 4 * H]
    parts["dense_b"] = np.s_[nwx + nwh + 4 * H:nwx + nwh + 4 * H + 1]
    return parts


@pytest.mark.parametrize("T,I,H,B,workers", [(7, 4, 5, 3, 1), (11, 3, 8, 4, 2), (5, 6, 4, 1, 1)])
def test_gru_bptt_vs_autograd(oracle, T, I, H, B, workers):
    """T > 1 from random parameters: the Wh gradients (update block, and the
    reset block through the candidate), the carried dh and the quirks against
    float64 autograd, every block to 1e-4; the textbook GRU differs."""
    rng = np.random.default_rng(200 + T)
    p = _gru_params(rng, I, H)
    x = rng.normal(size=(B, T * I)).astype(np.float32)
    y = rng.normal(size=B).astype(np.float32)
    net = oracle.Net([oracle.spec(oracle.LAYER_GRU_UNROLLER, in_size=I, out_size=H, seq_len=T),
                      oracle.spec(oracle.LAYER_DENSE, in_size=H, out_size=1, act=oracle.ACT_LINEAR)],
                     oracle.LOSS_MSE, workers=workers)
    net.params[:] = p
    loss = net.accumulate_batch(x, y.reshape(B, 1), B)
    g = net.grads.copy()
    l_ref, g_ref = _gru_torch(p, x, y, I, H, T)
    assert abs(loss - l_ref) <= 1e-4 * abs(l_ref)
    parts = _gru_parts(I, H)
    # the reset gate's input weights and bias get nothing (both sides exactly 0)
    for k in ("Wx_r", "b_r"):
        assert not g[parts[k]].any() and not g_ref[parts[k]].any()
        del parts[k]
    _check_parts(g, g_ref, parts)
    _, g_std = _gru_torch(p, x, y, I, H, T, reference=False)
    nl = 3 * H * I + 2 * H * H + 3 * H
    assert max_rel(g[:nl], g_std[:nl]) > 1e-2


def _seq_params(rng, n_rec, T, H, scale=0.4):
    return (rng.normal(size=n_rec + T * H + 1) * scale).astype(np.float32)


@pytest.mark.parametrize("workers,big", [(1, False), (2, True)])
def test_lstm_return_sequences_vs_autograd(oracle, workers, big):
    """SequenceUnroller(LSTM, returnSequences = true) -> Dense(T H, 1): the
    output is every step's state (unroller.go:115-119) and the backward adds
    each step's own gradient to the carried one (unroller.go:192-198).  The
    torch model's loss reads all T states, so autograd gives that injection;
    with large targets (big) the per-step clip acts and is applied to
    autograd's per-step deltas in the worker chains."""
    T, I, H, B = 6, 3, 5, 4
    rng = np.random.default_rng(400 + workers)
    nrec = 4 * H * I + 4 * H * H + 4 * H
    p = _seq_params(rng, nrec, T, H)
    x = rng.normal(size=(B, T * I)).astype(np.float32)
    net = oracle.Net([oracle.spec(oracle.LAYER_LSTM_UNROLLER, in_size=I, out_size=H, seq_len=T,
                                  return_sequences=1),
                      oracle.spec(oracle.LAYER_DENSE, in_size=T * H, out_size=1, act=oracle.ACT_LINEAR)],
                     oracle.LOSS_MSE, workers=workers)
    assert net.n == p.size
    net.params[:] = p
    preds = np.array([net.forward(x[b])[0] for b in range(B)], np.float32)
    y = (preds + (rng.normal(size=B) * 30 if big else 1e-2 * rng.choice([-1.0, 1.0], size=B))).astype(np.float32)
    loss = net.accumulate_batch(x, y.reshape(B, 1), B)
    g = net.grads.copy()
    l_ref, g_ref, dpre, hs = _lstm_torch(p, x, y, I, H, T, keep_pre=True, seq=True)
    # (targets 1e-3 from float32 predictions: the loss itself is ~1e-6)
    assert abs(loss - l_ref) <= 1e-4 * abs(l_ref) + 1e-9
    if big:
        X = x.astype(np.float64).reshape(B, T, I)
        W = min(workers, B)
        chunk = (B + W - 1) // W
        total = np.zeros(nrec)
        active = 0
        for c0 in range(0, B, chunk):
            deltas = []
            for bb in range(c0, min(B, c0 + chunk)):
                for t in range(T - 1, -1, -1):
                    dg = dpre[t][bb]
                    deltas.append(np.concatenate([np.outer(dg, X[bb, T - 1]).ravel(),
                                                  np.outer(dg, hs[t][bb]).ravel(), dg]))
            total += _clip_chain(deltas)
            run = np.cumsum(np.stack(deltas), axis=0)
            active += int((np.linalg.norm(run, axis=1) > 1).sum())
        assert active > 0
        g_ref = g_ref.copy()
        g_ref[:nrec] = total / B
    else:
        assert np.linalg.norm(g[:nrec]) * B < 0.5  # the clip never acts (running norms stay below 1)
    parts = {k: v for k, v in _lstm_parts(I, H).items() if not k.startswith("dense")}
    parts["dense_W"] = np.s_[nrec:nrec + T * H]
    parts["dense_b"] = np.s_[nrec + T * H:]
    _check_parts(g, g_ref, parts)
    # only the last state read (returnSequences = false) gives other gradients
    _, g_last, _, _ = _lstm_torch(np.concatenate([p[:nrec], p[nrec + (T - 1) * H:]]), x, y, I, H, T)
    assert max_rel(g[:nrec], g_last[:nrec]) > 1e-2


def test_gru_return_sequences_vs_autograd(oracle):
    T, I, H, B = 5, 4, 6, 3
    rng = np.random.default_rng(500)
    nrec = 3 * H * I + 2 * H * H + 3 * H
    p = _seq_params(rng, nrec, T, H)
    x = rng.normal(size=(B, T * I)).astype(np.float32)
    y = rng.normal(size=B).astype(np.float32)
    net = oracle.Net([oracle.spec(oracle.LAYER_GRU_UNROLLER, in_size=I, out_size=H, seq_len=T,
                                  return_sequences=1),
                      oracle.spec(oracle.LAYER_DENSE, in_size=T * H, out_size=1, act=oracle.ACT_LINEAR)],
                     oracle.LOSS_MSE)
    net.params[:] = p
    loss = net.accumulate_batch(x, y.reshape(B, 1), B)
    g = net.grads.copy()
    l_ref, g_ref = _gru_torch(p, x, y, I, H, T, seq=True)
    assert abs(loss - l_ref) <= 1e-4 * abs(l_ref)
    parts = {k: v for k, v in _gru_parts(I, H).items() if not k.startswith("dense")}
    for k in ("Wx_r", "b_r"):
        assert not g[parts[k]].any() and not g_ref[parts[k]].any()
        del parts[k]
    parts["dense_W"] = np.s_[nrec:nrec + T * H]
    parts["dense_b"] = np.s_[nrec + T * H:]
    _check_parts(g, g_ref, parts)
