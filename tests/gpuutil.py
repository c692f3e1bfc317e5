"""Shared helpers of the GPU parity tests: device buffers, the step-by-step
comparison of a model against the oracle, non-zero starting weights."""
import ctypes as C
import sys

import numpy as np

from cfgutil import adam_flips, max_rel, norm_rel, oracle_net, tensor_parts

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


def compare_step(gn, oracle, cfg, steps=1, workers=1, perturb=None, setup=None, xy=None,
                 arbiter=None):
    """One model on the GPU and the oracle, step by step from the same weights.

    perturb(params) -> params: replacement of the initial weights, loaded into
    both (e.g. a non-zero TransformerBlock).  setup(model, net): called before
    the first step.  xy: inputs other than the config's synthetic ones.

    Every parameter tensor is checked on its own:
      - gradient max|a - r| / max|r| <= 1e-4.  A tensor whose reference
        gradient is numerically zero (max|r| <= 1e-6 of its layer's largest
        gradient; e.g. the attention K projection without RoPE, whose token
        sum of gK vanishes because softmax Jacobian rows sum to zero) must be
        below that floor on the GPU too;
      - with arbiter(params) -> float64 gradient (the exact answer), a tensor
        that misses 1e-4 against the oracle passes if the GPU is within 1e-4
        of the exact answer and no further from it than the oracle, i.e. the
        difference is the oracle's (the reference's) own float32 rounding;
      - updated weights ||a - r|| / ||r|| <= 1e-4 outside the Adam updates
        whose direction legitimately differs (first moment at noise level);
        those are counted, and flips anywhere else fail.  The updates of
        numerically zero tensors are Adam-normalised rounding noise on both
        sides and are not compared."""
    from goneuron_amd import configs
    log(f"model parity {cfg['name']} B={cfg['B']} steps={steps} W={workers}")
    x, y = configs.inputs(cfg) if xy is None else xy
    B = cfg["B"]
    model = configs.build(cfg, workers=workers)
    net = oracle_net(oracle, cfg, workers=workers)
    np.testing.assert_array_equal(model.Params(), net.params)  # LCG init is exact
    parts = tensor_parts(cfg, net)
    layer_of = {name: int(name.split(":")[0]) for name, _ in parts}
    if perturb is not None:
        p = perturb(net.params.copy())
        net.params[:] = p
        model.SetParams(p)
    if setup is not None:
        setup(model, net)
    for s in range(steps):
        p_old = net.params.copy()
        truth = arbiter(p_old) if arbiter is not None else None
        lg = model.TrainBatch(x, y)
        lo = net.accumulate_batch(x, y, B)
        g_gpu = model.Gradients()
        g_ref = net.grads.copy()
        assert abs(lg - lo) <= TOL * max(abs(lo), 1e-30), (s, lg, lo)
        lmax = {i: float(np.abs(g_ref[net.layer_slice(i)]).max()) if net.layer_slice(i).stop >
                net.layer_slice(i).start else 0.0 for i in set(layer_of.values())}
        bad, zero, arb = {}, [], {}
        for name, sl in parts:
            floor = 1e-6 * lmax[layer_of[name]]
            if float(np.abs(g_ref[sl]).max()) <= floor:
                zero.append(name)
                if float(np.abs(g_gpu[sl]).max()) > floor:
                    bad[name] = ("numerically zero in the reference", float(np.abs(g_gpu[sl]).max()), floor)
                continue
            e = max_rel(g_gpu[sl], g_ref[sl])
            if e <= TOL:
                continue
            if truth is not None:
                e_gt, e_ot = max_rel(g_gpu[sl], truth[sl]), max_rel(g_ref[sl], truth[sl])
                arb[name] = (e, e_gt, e_ot)
                if e_gt <= TOL and e_gt <= e_ot:
                    continue
            bad[name] = e
        if zero:
            log(f"  step {s}: numerically zero in both: {zero}")
        for name, (e, e_gt, e_ot) in arb.items():
            log(f"  step {s}: {name}: gpu-oracle {e:.2e}, gpu-exact {e_gt:.2e}, oracle-exact {e_ot:.2e}")
        assert not bad, (s, bad)
        net.step()
        p_gpu = model.Params()
        m_ref = net.adam_m
        nflip, bad = 0, {}
        for name, sl in parts:
            if name in zero:
                # Adam normalises the rounding noise of a numerically zero
                # gradient to full-size steps of either sign: not comparable
                continue
            allowed, n_ok, n_bad = adam_flips(p_gpu[sl], p_old[sl], net.params[sl], m_ref[sl])
            nflip += n_ok
            if n_bad:
                bad[name] = ("direction flips", n_bad)
                continue
            keep = ~allowed
            if norm_rel(p_gpu[sl][keep], net.params[sl][keep]) > TOL:
                bad[name] = norm_rel(p_gpu[sl][keep], net.params[sl][keep])
        assert not bad, (s, bad)
        log(f"  step {s}: {len(parts)} tensors checked; {nflip} Adam updates flipped where the "
            f"first moment is at noise level")
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


