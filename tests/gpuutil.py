"""Shared helpers of the GPU parity tests: device buffers, the step-by-step
comparison of a model against the oracle, non-zero starting weights."""
import ctypes as C
import sys

import numpy as np

from cfgutil import adam_flips, adam_update_bound, max_rel, norm_rel, oracle_net, tensor_parts

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
                 arbiter=None, record=None):
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
        difference is the oracle's (the reference's) own float32 rounding.
        Every tensor the arbiter is asked about is appended to `record` (a
        list) as a dict: step, tensor, the three errors and whether it passed
        only through the arbiter;
      - updated weights ||a - r|| / ||r|| <= 1e-4 outside the Adam updates
        whose direction legitimately differs (first moment at noise level);
        those are counted, and flips anywhere else fail.  The updates of
        numerically zero tensors are Adam-normalised rounding noise on both
        sides and are not compared.  A tensor that misses 1e-4 in norm is
        checked again without its ill-conditioned updates: elements where a
        gradient change within the gradient tolerance (1e-4 of the tensor's
        largest gradient) can move the update by more than 1e-4 of the weight
        (adam_update_bound); each of those must lie within twice that bound,
        the rest within 1e-4 in norm, and their number is logged;
      - Adam moments m, v: from equal moments before the step, each element
        within what the gradient tolerance allows ((1-b1) tau for m,
        (1-b2)(2|g| tau + tau^2) for v, tau = 1e-4 of the tensor's largest
        gradient); the oracle then takes the GPU's parameters and moments,
        so every step is checked alone (a moment difference from an earlier
        step would otherwise be counted again in every later update)."""
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
        m_old, v_old = net.adam_m.copy(), net.adam_v.copy()
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
                ok = e_gt <= TOL and e_gt <= e_ot
                if record is not None:
                    record.append({"step": s, "tensor": name, "gpu_oracle": e, "gpu_exact": e_gt,
                                   "oracle_exact": e_ot, "passed_by_arbiter": ok})
                if ok:
                    continue
            bad[name] = e
        if zero:
            log(f"  step {s}: numerically zero in both: {zero}")
        for name, (e, e_gt, e_ot) in arb.items():
            log(f"  step {s}: {name}: gpu-oracle {e:.2e}, gpu-exact {e_gt:.2e}, oracle-exact {e_ot:.2e}")
        assert not bad, (s, bad)
        net.step()
        p_gpu = model.Params()
        m_gpu, v_gpu, t = model.AdamState()
        assert t == net.timestep
        m_ref, v_ref = net.adam_m, net.adam_v
        nflip, nill, bad = 0, 0, {}
        for name, sl in parts:
            if name in zero:
                # Adam normalises the rounding noise of a numerically zero
                # gradient to full-size steps of either sign: not comparable
                continue
            # moments: from the same m, v before the step they differ only
            # through the gradient (m by (1-b1) dg, v by (1-b2)(2|g| dg + dg^2))
            tau = TOL * float(np.abs(g_ref[sl]).max())
            ga = np.abs(np.asarray(g_ref[sl], np.float64))
            for what, a, r, lim in (("m", m_gpu, m_ref, 0.1 * tau),
                                    ("v", v_gpu, v_ref, 0.001 * (2.0 * ga * tau + tau * tau))):
                r64 = np.asarray(r[sl], np.float64)
                over = np.abs(np.asarray(a[sl], np.float64) - r64) > lim + 2e-7 * np.abs(r64)
                if over.any():
                    bad[name + "." + what] = ("moment beyond the gradient tolerance", int(over.sum()))
            allowed, n_ok, n_bad = adam_flips(p_gpu[sl], p_old[sl], net.params[sl], m_ref[sl])
            nflip += n_ok
            if n_bad:
                bad[name] = ("direction flips", n_bad)
                continue
            keep = ~allowed
            if norm_rel(p_gpu[sl][keep], net.params[sl][keep]) <= TOL:
                continue
            bnd = adam_update_bound(g_ref[sl], m_old[sl], v_old[sl], tau, net.timestep, lr=cfg["lr"])
            ref = np.asarray(net.params[sl], np.float64)
            diff = np.abs(np.asarray(p_gpu[sl], np.float64) - ref)
            ill = keep & (bnd > TOL * np.abs(ref))
            if (diff[ill] > 2.0 * bnd[ill]).any():
                bad[name] = ("update outside its propagated bound", int((diff[ill] > 2.0 * bnd[ill]).sum()))
                continue
            rest = keep & ~ill
            if rest.any() and norm_rel(p_gpu[sl][rest], net.params[sl][rest]) > TOL:
                bad[name] = norm_rel(p_gpu[sl][rest], net.params[sl][rest])
                continue
            nill += int(ill.sum())
            log(f"  step {s}: {name}: {int(ill.sum())} of {ill.size} updates ill-conditioned at the "
                f"gradient tolerance, each within its bound; the rest within 1e-4")
        assert not bad, (s, bad)
        log(f"  step {s}: {len(parts)} tensors checked; {nflip} Adam updates flipped where the "
            f"first moment is at noise level; {nill} ill-conditioned updates within their bound")
        # keep the two runs on identical weights and moments so each step is
        # checked alone
        net.params[:] = p_gpu
        net.adam_m[:] = m_gpu
        net.adam_v[:] = v_gpu
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


