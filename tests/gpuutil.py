"""Shared helpers of the GPU parity tests: device buffers, the step-by-step
comparison of a model against the oracle, non-zero starting weights."""
import ctypes as C
import sys

import numpy as np

from cfgutil import max_rel, norm_rel, oracle_net, sign_flips, tensor_parts

TOL = 1e-4


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class DBuf:
    """A device buffer holding a numpy array (float32 or int32)."""

    def __init__(self, dev, arr):
        from goneuron_amd._lib import lib, check
        self.lib, self.check, self.dev = lib(), check, dev
        self.arr = np.ascontiguousarray(arr)
        self.p = C.c_void_p()
        check(dev.h, self.lib.gn_malloc(dev.h, max(self.arr.nbytes, 4), C.byref(self.p)))
        if self.arr.nbytes:
            check(dev.h, self.lib.gn_memcpy_h2d(dev.h, self.p, self.arr.ctypes.data, self.arr.nbytes))

    def get(self):
        out = np.empty_like(self.arr)
        self.check(self.dev.h, self.lib.gn_memcpy_d2h(self.dev.h, out.ctypes.data, self.p, out.nbytes))
        return out

    def __del__(self):
        try:
            self.lib.gn_free(self.dev.h, self.p)
        except Exception:
            pass


def compare_step(gn, oracle, cfg, steps=1, workers=1, perturb=None, setup=None, xy=None):
    """perturb(params) -> params: optional replacement of the initial weights,
    loaded into both implementations (e.g. non-zero TransformerBlock weights).
    setup(model, net): called before the first step on both sides.
    Every parameter tensor is checked on its own: gradient max|a-r|/max|r| and
    updated weights ||a-r||/||r|| to 1e-4; Adam updates whose direction
    differs are counted (allowed only where the reference gradient is below
    1e-4 of its tensor's maximum)."""
    from goneuron_amd import configs
    log(f"model parity {cfg['name']} B={cfg['B']} steps={steps} W={workers}")
    x, y = configs.inputs(cfg) if xy is None else xy
    B = cfg["B"]
    model = configs.build(cfg, workers=workers)
    net = oracle_net(oracle, cfg, workers=workers)
    np.testing.assert_array_equal(model.Params(), net.params)  # LCG init is exact
    parts = tensor_parts(cfg, net)
    if perturb is not None:
        p = perturb(net.params.copy())
        net.params[:] = p
        model.SetParams(p)
    if setup is not None:
        setup(model, net)
    for s in range(steps):
        p_old = net.params.copy()
        lg = model.TrainBatch(x, y)
        lo = net.accumulate_batch(x, y, B)
        g_gpu = model.Gradients()
        g_ref = net.grads.copy()
        assert abs(lg - lo) <= TOL * max(abs(lo), 1e-30), (s, lg, lo)
        bad = {name: e for name, sl in parts if (e := max_rel(g_gpu[sl], g_ref[sl])) > TOL}
        assert not bad, (s, bad)
        net.step()
        p_gpu = model.Params()
        bad = {name: e for name, sl in parts if (e := norm_rel(p_gpu[sl], net.params[sl])) > TOL}
        assert not bad, (s, bad)
        small = big = 0
        for name, sl in parts:
            a, b_ = sign_flips(p_gpu[sl], p_old[sl], net.params[sl], g_ref[sl])
            small += a
            big += b_
        log(f"  step {s}: {len(parts)} tensors within 1e-4; Adam direction flips "
            f"{small} on sub-1e-4 gradients, {big} on updates above 1e-2 of the largest")
        assert big == 0, (s, big)
        # keep the two runs on identical weights so each step is checked alone
        net.params[:] = p_gpu
    m_gpu, v_gpu, t = model.AdamState()
    assert t == net.timestep
    assert norm_rel(m_gpu, net.adam_m) <= TOL
    assert norm_rel(v_gpu, net.adam_v) <= TOL
    return model, net


def random_block(cfg, scale=0.2, seed=21):
    """Non-zero TransformerBlock weights (the reference starts it at 0, Q11),
    so attention, LayerNorm and the FF path carry gradient."""
    d = cfg["layers"][2]
    D, FF, T, V = d["dim"], d["ff"], d["T"], cfg["classes"]
    start = V * D + T * D
    nn = D if d.get("norm", "ln") == "rms" else 2 * D
    n1 = 2 * FF * D if d.get("act", "relu") == "swiglu" else FF * D + FF
    n = 4 * (D * D + D) + 2 * nn + n1 + (D * FF + D)

    def f(p):
        rng = np.random.default_rng(seed)
        p[start:start + n] = (rng.normal(size=n) * scale).astype(np.float32)
        g1 = start + 4 * (D * D + D)
        p[g1:g1 + D] += 1.0          # norm gammas around 1
        p[g1 + nn:g1 + nn + D] += 1.0
        return p
    return f


