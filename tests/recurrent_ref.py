"""float64 torch restatements of SequenceUnroller(LSTM) and (GRU) with a Dense
head and MSE, whose autograd gradients are the reference's hand-written BPTT
(quirks as zero-valued ``v - v.detach()`` terms or detached factors; see
test_oracle_recurrent.py for the list), and the float64 evaluation of the
LSTM's per-step clip (lstm.go:732-761) used as the exact answer at full size.
Test infrastructure only."""
import math

import numpy as np
import torch


def _det(v):
    return v - v.detach()


def _lstm_params(rng, I, H, scale=0.4):
    n = 4 * H * I + 4 * H * H + 4 * H + H + 1
    return (rng.normal(size=n) * scale).astype(np.float32)


def _lstm_torch(p, x, y, I, H, T, reference=True, keep_pre=False, seq=False):
    """Mean MSE over the batch of SequenceUnroller(LSTM(I, H), T, last) ->
    Dense(H, 1, Linear) (seq: returnSequences, the Dense reads all T states);
    returns (loss, flat gradient, pre-activation gradients [T][B, 4H], hidden
    states [T + 1][B, H])."""
    B = x.shape[0]
    P = torch.tensor(p.astype(np.float64), requires_grad=True)
    nwx, nwh = 4 * H * I, 4 * H * H
    Wx = P[:nwx].view(4 * H, I)
    Wh = P[nwx:nwx + nwh].view(4 * H, H)
    b = P[nwx + nwh:nwx + nwh + 4 * H]
    nd = (T if seq else 1) * H
    Wd = P[nwx + nwh + 4 * H:nwx + nwh + 4 * H + nd].view(1, nd)
    bd = P[nwx + nwh + 4 * H + nd:]
    X = torch.tensor(x.astype(np.float64)).view(B, T, I)
    xl = X[:, T - 1, :]
    h = torch.zeros(B, H, dtype=torch.float64)
    c = torch.zeros(B, H, dtype=torch.float64)
    pres, hs, states = [], [h.detach().numpy().copy()], []
    for t in range(T):
        xt = X[:, t, :]
        if reference:
            zx = xt @ Wx.detach().T + _det(xl @ Wx.T)          # Q10
            z = zx + h @ Wh.T
            z = torch.cat([z[:, :H], _det(z[:, H:])], dim=1)     # Q13
        else:
            z = xt @ Wx.T + h @ Wh.T
        pre = b + z
        if keep_pre:
            pre.retain_grad()
            pres.append(pre)
        i = torch.sigmoid(pre[:, :H])
        f = torch.sigmoid(pre[:, H:2 * H])
        g = torch.tanh(pre[:, 2 * H:3 * H])
        o = torch.sigmoid(pre[:, 3 * H:])
        c = f * c + i * g
        hn = o * torch.tanh(c)
        if reference:
            hn = hn + _det(h)                                    # Q15
        h = hn
        states.append(h)
        hs.append(h.detach().numpy().copy())
    out = ((torch.cat(states, 1) if seq else h) @ Wd.T + bd)[:, 0]
    Y = torch.tensor(y.astype(np.float64)).view(B)
    loss = ((out - Y) ** 2).sum() / B
    loss.backward()
    dpre = [q.grad.numpy() * B for q in pres]  # per-sample gradients (the loss is a batch mean)
    return float(loss.detach()), P.grad.numpy(), dpre, hs


def _clip_chain(deltas):
    """G <- clip(G + D_t) over a chain, in float64 (Q14): the running sum of the
    contributions scaled to norm 1 whenever its norm exceeds 1."""
    G = np.zeros_like(deltas[0])
    for d in deltas:
        G = G + d
        n = math.sqrt(float(G @ G))
        if n > 1:
            G = G * (1.0 / n)
    return G


def _gru_params(rng, I, H, scale=0.4):
    n = 3 * H * I + 2 * H * H + 3 * H + H + 1
    return (rng.normal(size=n) * scale).astype(np.float32)


def _gru_torch(p, x, y, I, H, T, reference=True, seq=False):
    """Mean MSE over the batch of SequenceUnroller(GRU(I, H), T, last) ->
    Dense(H, 1, Linear) (seq: returnSequences, the Dense reads all T states)."""
    B = x.shape[0]
    P = torch.tensor(p.astype(np.float64), requires_grad=True)
    nwx, nwh = 3 * H * I, 2 * H * H
    Wx = P[:nwx].view(3 * H, I)
    Wh = P[nwx:nwx + nwh].view(2 * H, H)
    b = P[nwx + nwh:nwx + nwh + 3 * H]
    nd = (T if seq else 1) * H
    Wd = P[nwx + nwh + 3 * H:nwx + nwh + 3 * H + nd].view(1, nd)
    bd = P[nwx + nwh + 3 * H + nd:]
    Whu, Whr = Wh[:H], Wh[H:]
    states = []
    X = torch.tensor(x.astype(np.float64)).view(B, T, I)
    xl = X[:, T - 1, :]
    h = torch.zeros(B, H, dtype=torch.float64)
    for t in range(T):
        xt = X[:, t, :]
        if reference:
            zx = xt @ Wx.detach().T + _det(xl @ Wx.T)                      # last step's input
            r = torch.sigmoid(b[H:2 * H] + zx[:, H:2 * H] + h @ Whr.T).detach()  # no reset delta
            u = torch.sigmoid(b[:H] + zx[:, :H] + h @ Whu.T)
            hd = h.detach()
            pre_c = (b[2 * H:] + zx[:, 2 * H:] + (r * hd) @ Whr.T
                     + r * _det(h @ Whr.detach().T))                           # r[j] on row j
            c = torch.tanh(pre_c)
            ud, cd = u.detach(), c.detach()
            h = ((h + u * (c - h)).detach() + (1 - ud) * _det(c) + _det(u) * (cd - hd)
                 + ud * _det(h) + _det(h))                                    # (1-u), u, carry
        else:
            zx = xt @ Wx.T
            r = torch.sigmoid(b[H:2 * H] + zx[:, H:2 * H] + h @ Whr.T)
            u = torch.sigmoid(b[:H] + zx[:, :H] + h @ Whu.T)
            c = torch.tanh(b[2 * H:] + zx[:, 2 * H:] + (r * h) @ Whr.T)
            h = h + u * (c - h)
        states.append(h)
    out = ((torch.cat(states, 1) if seq else h) @ Wd.T + bd)[:, 0]
    Y = torch.tensor(y.astype(np.float64)).view(B)
    loss = ((out - Y) ** 2).sum() / B
    loss.backward()
    return float(loss.detach()), P.grad.numpy()



def lstm_clip_truth(p, x, y, I, H, T, workers):
    """The averaged gradient of SequenceUnroller(LSTM) + Dense + MSE with the
    per-step clip evaluated exactly: autograd's per-step pre-activation
    gradients dG_t (the clip never feeds back into the recursion), each step's
    contribution [dG x_{T-1} | dG h_{t-1} | dG], and for every worker chain the
    running sum clipped to norm 1 after every step, through the chain's Gram
    matrix <D_u, D_v> = (dG_u . dG_v)(x_u . x_v + h_u . h_v + 1) in float64."""
    B = x.shape[0]
    _, g_ref, dpre, hs = _lstm_torch(p, x, y, I, H, T, keep_pre=True)
    X = x.astype(np.float64).reshape(B, T, I)
    W = min(max(workers, 1), B)
    chunk = (B + W - 1) // W
    nwx, nwh = 4 * H * I, 4 * H * H
    gWx = np.zeros((4 * H, I))
    gWh = np.zeros((4 * H, H))
    gb = np.zeros(4 * H)
    for c0 in range(0, B, chunk):
        idx = [(b, t) for b in range(c0, min(B, c0 + chunk)) for t in range(T - 1, -1, -1)]
        DG = np.stack([dpre[t][b] for b, t in idx])
        XL = np.stack([X[b, T - 1] for b, t in idx])
        HP = np.stack([hs[t][b] for b, t in idx])
        Gm = (DG @ DG.T) * (XL @ XL.T + HP @ HP.T + 1.0)
        n = len(idx)
        w = np.zeros(n)
        nrm2 = 0.0
        for t in range(n):
            N2 = nrm2 + 2 * (w[:t] @ Gm[:t, t]) + Gm[t, t]
            c = 1.0 / math.sqrt(N2) if N2 > 1 else 1.0
            w[:t] *= c
            w[t] = c
            nrm2 = c * c * N2
        gWx += (DG * w[:, None]).T @ XL
        gWh += (DG * w[:, None]).T @ HP
        gb += (DG * w[:, None]).sum(0)
    out = g_ref.copy()
    out[:nwx] = gWx.ravel() / B
    out[nwx:nwx + nwh] = gWh.ravel() / B
    out[nwx + nwh:nwx + nwh + 4 * H] = gb / B
    return out
