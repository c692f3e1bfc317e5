"""Test helpers: build the CPU oracle network for a neutral config description
(goneuron_amd.configs) and compare tensors by the BASELINE tolerances."""
import numpy as np

ACT = {"relu": 1, "sigmoid": 2, "tanh": 3, "softmax": 4, "logsoftmax": 5, "linear": 6, "gelu": 7}


def oracle_specs(refcpu, cfg):
    specs = []
    for i, d in enumerate(cfg["layers"]):
        k = d["kind"]
        if k == "dense":
            specs.append(refcpu.spec(refcpu.LAYER_DENSE, in_size=d["in"], out_size=d["out"],
                                     act=ACT[d["act"]], act_is_ptr=int(d["ptr"])))
        elif k == "dropout":
            specs.append(refcpu.spec(refcpu.LAYER_DROPOUT, in_size=d["n"], p=d["p"]))
        elif k == "avgpool2d":
            specs.append(refcpu.spec(refcpu.LAYER_AVGPOOL2D, in_channels=d["inC"], kernel=d["k"],
                                     stride=d["s"], padding=d["p"]))
        elif k == "flatten":
            specs.append(refcpu.spec(refcpu.LAYER_FLATTEN, in_size=d["n"]))
        elif k == "moe":
            specs.append(refcpu.spec(refcpu.LAYER_MOE, in_size=d["in"], out_size=d["out"],
                                     num_experts=d["E"], top_k=d["k"]))
        elif k == "batchnorm2d":
            specs.append(refcpu.spec(refcpu.LAYER_BATCHNORM2D, in_channels=d["C"], momentum=0.1,
                                     in_size=cfg["in_len"] if i == 0 else 0))
        elif k == "swiglu":
            specs.append(refcpu.spec(refcpu.LAYER_SWIGLU, in_size=d["in"], out_size=d["out"]))
        elif k == "rmsnorm":
            specs.append(refcpu.spec(refcpu.LAYER_RMSNORM, dim=d["n"],
                                     in_size=cfg["in_len"] if i == 0 else 0))
        elif k == "layernorm":  # "len": the per-sample input length (rows of n)
            specs.append(refcpu.spec(refcpu.LAYER_LAYERNORM, dim=d["n"], in_size=d["len"]))
        elif k == "mha":
            specs.append(refcpu.spec(refcpu.LAYER_MHA, dim=d["dim"], num_heads=d["heads"], seq_len=d["T"],
                                     causal=int(d["causal"]), use_rope=0))
        elif k == "gap1d":
            specs.append(refcpu.spec(refcpu.LAYER_GAP1D, seq_len=d["T"], dim=d["dim"]))
        elif k == "conv2d":
            specs.append(refcpu.spec(refcpu.LAYER_CONV2D, in_size=cfg["in_len"], in_channels=d["inC"],
                                     out_channels=d["outC"], kernel=d["k"], stride=d["s"],
                                     padding=d["p"], act=ACT[d["act"]]))
        elif k == "maxpool2d":
            specs.append(refcpu.spec(refcpu.LAYER_MAXPOOL2D, in_channels=d["inC"], kernel=d["k"],
                                     stride=d["s"], padding=d["p"]))
        elif k == "embedding":
            specs.append(refcpu.spec(refcpu.LAYER_EMBEDDING, in_size=d.get("T", cfg["in_len"]),
                                     vocab=d["vocab"], dim=d["dim"]))
        elif k == "posenc":
            specs.append(refcpu.spec(refcpu.LAYER_POSENC, seq_len=d["T"], dim=d["dim"]))
        elif k == "transformer":
            specs.append(refcpu.spec(refcpu.LAYER_TRANSFORMER, dim=d["dim"], num_heads=d["heads"],
                                     seq_len=d["T"], ff_dim=d["ff"], causal=int(d["causal"]),
                                     block_act={"relu": 0, "swiglu": 1, "gelu": 2}[d.get("act", "relu")],
                                     block_norm={"ln": 0, "rms": 1}[d.get("norm", "ln")],
                                     use_rope=int(bool(d.get("rope", False)))))
        elif k == "clspool":
            specs.append(refcpu.spec(refcpu.LAYER_CLSPOOL, seq_len=d["T"], dim=d["dim"]))
        elif k == "gru":
            specs.append(refcpu.spec(refcpu.LAYER_GRU_UNROLLER, in_size=d["in"], out_size=d["hidden"],
                                     seq_len=d["T"], return_sequences=int(d.get("seq", False))))
        elif k == "lstm":
            specs.append(refcpu.spec(refcpu.LAYER_LSTM_UNROLLER, in_size=d["in"], out_size=d["hidden"],
                                     seq_len=d["T"], return_sequences=int(d.get("seq", False))))
        else:
            raise NotImplementedError(k)
    return specs


def oracle_net(refcpu, cfg, workers=1):
    return refcpu.Net(oracle_specs(refcpu, cfg), refcpu.LOSS_CE if cfg["loss"] == "ce" else refcpu.LOSS_MSE,
                      lr=cfg["lr"], workers=workers)


def max_rel(a, r):
    """max|a - r| / max|r| (BASELINE per-tensor gradient tolerance)."""
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    den = np.abs(r).max()
    if den == 0:
        return float(np.abs(a).max())
    return float(np.abs(a - r).max() / den)


def norm_rel(a, r):
    """||a - r||_2 / ||r||_2 (BASELINE updated-weight tolerance)."""
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    den = np.linalg.norm(r)
    return float(np.linalg.norm(a - r) / den) if den else float(np.linalg.norm(a))


def tensor_parts(cfg, net):
    """(name, slice) of every parameter tensor of the flat arena, layer by
    layer in the reference's Params() order, so tolerances apply per tensor
    (gate blocks of recurrent weights, each block weight and bias, each
    expert) rather than per layer."""
    parts = []
    for i, d in enumerate(cfg["layers"]):
        sl = net.layer_slice(i)
        o = sl.start

        def add(name, n):
            nonlocal o
            parts.append((f"{i}:{d['kind']}.{name}", slice(o, o + n)))
            o += n
        k = d["kind"]
        if k == "dense":
            add("W", d["in"] * d["out"])
            add("b", d["out"])
        elif k == "conv2d":
            add("W", d["outC"] * d["inC"] * d["k"] * d["k"])
            add("b", d["outC"])
        elif k == "lstm":
            I, H = d["in"], d["hidden"]
            for g in "ifgo":
                add("Wx_" + g, H * I)
            for g in "ifgo":
                add("Wh_" + g, H * H)
            for g in "ifgo":
                add("b_" + g, H)
        elif k == "gru":
            I, H = d["in"], d["hidden"]
            for g in "urc":
                add("Wx_" + g, H * I)
            for g in "ur":
                add("Wh_" + g, H * H)
            for g in "urc":
                add("b_" + g, H)
        elif k == "embedding":
            add("E", d["vocab"] * d["dim"])
        elif k == "posenc":
            add("P", d["T"] * d["dim"])
        elif k == "transformer":
            D, FF = d["dim"], d["ff"]
            for name in ("wq", "wk", "wv", "wo"):
                add(name + ".W", D * D)
                add(name + ".b", D)
            for name in ("norm1", "norm2"):
                add(name + ".gamma", D)
                if d.get("norm", "ln") != "rms":
                    add(name + ".beta", D)
            if d.get("act", "relu") == "swiglu":
                add("ff1.W", FF * D)
                add("ff1.V", FF * D)
            else:
                add("ff1.W", FF * D)
                add("ff1.b", FF)
            add("ff2.W", D * FF)
            add("ff2.b", D)
        elif k == "rmsnorm":
            add("gamma", d["n"])
        elif k == "layernorm":
            add("gamma", d["n"])
            add("beta", d["n"])
        elif k == "mha":
            for name in ("wq", "wk", "wv", "wo"):
                add(name + ".W", d["dim"] * d["dim"])
                add(name + ".b", d["dim"])
        elif k == "batchnorm2d":
            add("gamma", d["C"])
            add("beta", d["C"])
        elif k == "swiglu":
            add("W", d["in"] * d["out"])
            add("V", d["in"] * d["out"])
        elif k == "moe":
            add("gate.W", d["E"] * d["in"])
            add("gate.b", d["E"])
            for e in range(d["E"]):
                add(f"expert{e}.W", d["out"] * d["in"])
                add(f"expert{e}.b", d["out"])
        assert o == sl.stop, (i, k, o, sl)
    return parts


def adam_flips(p_new, p_old, r_new, m_ref, rel=1e-4):
    """Adam updates whose direction differs between two runs.  A flip is
    expected only where the reference's new first moment m is at noise level
    (|m| <= rel * max|m| of the tensor: the sign of m, hence of the update, is
    then within rounding; at the first step m = (1 - beta1) g, so this is the
    sub-noise-gradient count BASELINE asks for).  Returns (mask of those
    allowed flips, their count, count of flips elsewhere)."""
    p_old = np.asarray(p_old, np.float64)
    du = np.asarray(p_new, np.float64) - p_old
    dr = np.asarray(r_new, np.float64) - p_old
    if not dr.size:
        return np.zeros(0, bool), 0, 0
    flips = np.sign(du) != np.sign(dr)
    m_ref = np.asarray(m_ref, np.float64)
    small = np.abs(m_ref) <= rel * np.abs(m_ref).max()
    allowed = flips & small
    return allowed, int(allowed.sum()), int((flips & ~small).sum())


def adam_update_bound(g, m_old, v_old, tau, timestep, lr=1e-3, b1=0.9, b2=0.999, eps=1e-8):
    """Largest change of each Adam update (opt.go:207-258, Q1: t = timestep+1)
    that a gradient change of at most tau per element can cause, from the
    moments m_old, v_old before the step.  Per element the update is
        effLR * u(g),  u(g) = (b1 m + (1-b1) g) / (sqrt(b2 v + (1-b2) g^2) + eps),
    one function of g, whose extremes on [g - tau, g + tau] lie at the ends
    or where u'(g) = 0, i.e. g* = (1-b1) b2 v / (b1 m (1-b2)) (eps left out
    there; it shifts the extreme by a relative 1e-8 of the update).
    Elements whose gradient is small next to tau get a large bound: Adam
    normalises each element, so their updates move by up to a full step
    under rounding-level gradient changes."""
    g = np.asarray(g, np.float64)
    m = np.asarray(m_old, np.float64)
    v = np.asarray(v_old, np.float64)
    ts = timestep + 1
    efflr = lr * np.sqrt(1.0 - b2 ** ts) / (1.0 - b1 ** ts)

    def u(x):
        return (b1 * m + (1.0 - b1) * x) / (np.sqrt(b2 * v + (1.0 - b2) * x * x) + eps)

    u0 = u(g)
    dev = np.maximum(np.abs(u(g - tau) - u0), np.abs(u(g + tau) - u0))
    with np.errstate(divide="ignore", invalid="ignore"):
        gs = (1.0 - b1) * b2 * v / (b1 * m * (1.0 - b2))
    inside = np.isfinite(gs) & (np.abs(gs - g) <= tau)
    if inside.any():
        dev = np.where(inside, np.maximum(dev, np.abs(u(np.where(inside, gs, g)) - u0)), dev)
    return efflr * dev * (1.0 + 1e-6)
