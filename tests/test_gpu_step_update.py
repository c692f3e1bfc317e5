"""GPU: Network.Step's update carried by the backward's last launch.

A train step of a small model (under 8 Mi parameters) whose backward ends in
the weight-gradient reduction of a first Conv2D, or in the gradient launch of
a first Embedding, runs the Adam update (Adam.NewStep + StepInPlace,
opt.go:237-258) in that launch instead of a launch of its own: each gradient
the launch writes is updated by the thread that writes it (an Embedding's
zeroed rows with g = 0, a PositionalEncoding's gradient summed by the same
launch too), and extra blocks of the launch update every other layer (their
gradients are final and no later kernel of the step reads their parameters).
Other models keep the update as its own launch.

Each case trains two copies of a model from the same weights for four steps
(the first eager, the second captured into a graph, the others replayed),
one as above and one with gn_debug_step_update(0) (the update always as its
own launch), and requires parameters, gradients and Adam moments to be equal
bit for bit after every step; the per-launch timing records show which path
ran.  The oracle parity of these steps is covered by the model tests (C2, C4
and the two-conv CNN go through the same train step).
"""
import numpy as np
import pytest

from gpuutil import log
from test_gpu_tail import _kernel_names

pytestmark = pytest.mark.gpu


def _dense(i, o, act, ptr=False):
    return {"kind": "dense", "in": i, "out": o, "act": act, "ptr": ptr}


def cases():
    """name -> (config, workers, the launch expected to carry the update or None)"""
    from goneuron_amd import configs
    out = {}
    out["cnn_w4"] = (configs.cnn(), 4, "wgrad_reduce_adam")
    out["cnn_w1"] = (configs.cnn(B=24), 1, "wgrad_reduce_adam")
    # a conv below a conv: the first conv's reduction updates the second's
    # parameters (read by its input-gradient launch before it)
    out["cnn2"] = (configs.cnn2(B=16), 2, "wgrad_reduce_adam")
    # Conv2D (stride 2) -> Flatten -> Dense: no pooling between
    out["conv_dense"] = (dict(num=49, name="conv_dense", B=12, loss="mse", lr=1e-3, x="normal", in_len=2 * 8 * 8,
                              targets="normal",
                              layers=[{"kind": "conv2d", "inC": 2, "outC": 4, "k": 3, "s": 2, "p": 1,
                                       "act": "tanh"},
                                      {"kind": "flatten", "n": 64}, _dense(64, 1, "linear")]), 1,
                         "wgrad_reduce_adam")
    # a first Embedding (+ PositionalEncoding) under a transformer block: the
    # Embedding's gradient launch carries the update (C4's shape, small)
    out["gpt_small"] = (configs.gpt(B=4, T=32, vocab=37, dim=32, heads=2, ff=48), 1, "embed_grad_adam")
    out["gpt_w2"] = (configs.gpt(B=6, T=16, vocab=29, dim=64, heads=4, ff=40), 2, "embed_grad_adam")
    # models whose backward ends elsewhere: the update keeps its own launch
    out["mlp_w4"] = (configs.mlp(), 4, None)
    out["three_dense"] = (dict(num=47, name="three_dense", B=70, loss="ce", lr=1e-3, x="normal", in_len=10,
                               classes=3,
                               layers=[_dense(10, 16, "relu"), _dense(16, 24, "tanh"),
                                       _dense(24, 3, "softmax", True)]), 2, None)
    return out


@pytest.mark.parametrize("name", sorted(cases()))
def test_update_in_last_launch(gn, dev, name):
    from goneuron_amd import configs
    from goneuron_amd._lib import lib
    cfg, workers, carrier = cases()[name]
    x, y = configs.inputs(cfg)
    on = configs.build(cfg, workers=workers)
    off = configs.build(cfg, workers=workers)
    assert lib().gn_debug_step_update(off.h, 0) == 0
    np.testing.assert_array_equal(on.Params(), off.Params())
    try:
        for s in range(4):
            la, lb = on.TrainBatch(x, y), off.TrainBatch(x, y)
            assert la == lb, (s, la, lb)
            np.testing.assert_array_equal(on.Gradients(), off.Gradients(), err_msg=f"grads, step {s}")
            np.testing.assert_array_equal(on.Params(), off.Params(), err_msg=f"params, step {s}")
            (ma, va, ta), (mb, vb, tb) = on.AdamState(), off.AdamState()
            assert ta == tb == s + 1
            np.testing.assert_array_equal(ma, mb, err_msg=f"m, step {s}")
            np.testing.assert_array_equal(va, vb, err_msg=f"v, step {s}")
        k_on, k_off = _kernel_names(dev, on, x, y), _kernel_names(dev, off, x, y)
        log(f"{name}: update in the last launch {sorted(k_on)}; alone {sorted(k_off)}")
        assert "adam" in k_off
        if carrier is None:
            assert "adam" in k_on
        else:
            assert carrier in k_on and "adam" not in k_on, sorted(k_on)
        # the timed steps (eager) and the graph replays keep agreeing
        for s in range(2):
            on.TrainBatch(x, y)
            off.TrainBatch(x, y)
        np.testing.assert_array_equal(on.Params(), off.Params())
        np.testing.assert_array_equal(on.AdamState()[1], off.AdamState()[1])
    finally:
        on.Close()
        off.Close()
