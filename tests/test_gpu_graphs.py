"""GPU tests of the graph-replayed training step (gn_model_set_graphs).

A model whose forward + loss + backward launches replay from a HIP graph must
give bit-identical results to the same model run eagerly: the replay runs the
same kernels on the same buffers.  Each test builds two identical models, one
with graphs (the default) and one without, and runs several steps on each,
with the program's own eager work and synchronisations between the replays
(other models' steps, parameter downloads, a Predict), two input buffers
alternating (two graph keys), and a change of training flags (a new key).
Every step's loss and the parameters, gradients and Adam moments after it
are compared bit for bit."""
import ctypes as C

import numpy as np
import pytest

from gpuutil import DBuf, log

pytestmark = pytest.mark.gpu


def _cfgs():
    from goneuron_amd import configs
    return {
        "mlp": configs.mlp(),
        "cnn": configs.cnn(B=32),
        "gpt": configs.gpt(B=8, T=32, vocab=500, dim=64, heads=2, ff=128),
        "gpt_swiglu_rms_rope": configs.gpt(B=4, T=16, vocab=300, dim=32, heads=2, ff=64, act="swiglu",
                                           norm="rms", rope=True),
    }


def _state(model):
    m, v, t = model.AdamState()
    return model.Params(), model.Gradients(), m, v, t


@pytest.mark.parametrize("name", sorted(_cfgs()))
def test_graph_replay_matches_eager(gn, dev, name):
    from goneuron_amd import configs
    from goneuron_amd._lib import check, lib
    L = lib()
    cfg = _cfgs()[name]
    B = cfg["B"]
    x1, y1 = configs.inputs(cfg)
    cfg2 = dict(cfg, num=cfg["num"] + 40)   # other seeds, same shapes
    x2, y2 = configs.inputs(cfg2)
    bufs = [(DBuf(dev, x1), DBuf(dev, y1)), (DBuf(dev, x2), DBuf(dev, y2))]
    g = configs.build(cfg, device=dev)
    e = configs.build(cfg, device=dev)
    other = configs.build(configs.mlp(), device=dev)  # eager work between the replays
    ox, oy = configs.inputs(configs.mlp())
    check(dev.h, L.gn_model_set_graphs(e.h, 0))
    n = C.c_int32()
    seq = [0, 0, 1, 0, 1, 1, 0, 0]
    for step, k in enumerate(seq):
        if step == 5:  # Network.SetTraining(false): new flags, a new key on the graph side
            g.SetTraining(False)
            e.SetTraining(False)
        dx, dy = bufs[k]
        losses = []
        for m in (g, e):
            check(dev.h, L.gn_model_train_step_device(m.h, dx.p, dy.p, B))
            lo = C.c_float()
            check(dev.h, L.gn_model_read_loss(m.h, C.byref(lo)))
            losses.append(lo.value)
        other.TrainBatch(ox, oy)
        assert losses[0] == losses[1] or (np.isnan(losses[0]) and np.isnan(losses[1])), (step, losses)
        sg, se = _state(g), _state(e)
        for part, a, b in zip(("params", "grads", "m", "v"), sg[:4], se[:4]):
            np.testing.assert_array_equal(a, b, err_msg=f"{name} step {step} {part}")
        assert sg[4] == se[4]
        if step == 2:
            check(dev.h, L.gn_model_graph_count(g.h, C.byref(n)))
            assert n.value == 1, n.value  # key 0 captured at its second step; key 1 seen once
        if step == 4:
            g.Predict(x1[0])   # an inference pass in between (flags go off and stay off)
            e.Predict(x1[0])
    check(dev.h, L.gn_model_graph_count(g.h, C.byref(n)))
    log(f"  {name}: {n.value} graphs after {len(seq)} steps")
    assert n.value >= 2
    check(dev.h, L.gn_model_graph_count(e.h, C.byref(n)))
    assert n.value == 0
    for m in (g, e, other):
        m.Close()


def test_graph_host_step_and_reserve(gn, dev):
    """The host-pointer step (staged through the model's own input buffers)
    replays too; gn_model_reserve frees the graphs (they hold the old batch
    buffers) and the next steps capture anew."""
    from goneuron_amd import configs
    from goneuron_amd._lib import check, lib
    L = lib()
    cfg = configs.mlp()
    x, y = configs.inputs(cfg)
    g = configs.build(cfg, device=dev)
    e = configs.build(cfg, device=dev)
    check(dev.h, L.gn_model_set_graphs(e.h, 0))
    n = C.c_int32()
    for step in range(6):
        if step == 3:
            g._reserve(2 * cfg["B"])
            e._reserve(2 * cfg["B"])
            check(dev.h, L.gn_model_graph_count(g.h, C.byref(n)))
            assert n.value == 0
        lg, le = g.TrainBatch(x, y), e.TrainBatch(x, y)
        assert lg == le, (step, lg, le)
        np.testing.assert_array_equal(g.Params(), e.Params())
    check(dev.h, L.gn_model_graph_count(g.h, C.byref(n)))
    assert n.value == 1
    g.Close()
    e.Close()


def test_no_graph_for_lstm_and_moe(gn, dev):
    from goneuron_amd import configs
    from goneuron_amd._lib import check, lib
    L = lib()
    cfg = configs.lstm(B=4, T=5, inp=3, hidden=8)
    x, y = configs.inputs(cfg)
    m = configs.build(cfg, device=dev)
    for _ in range(3):
        m.TrainBatch(x, y)
    n = C.c_int32()
    check(dev.h, L.gn_model_graph_count(m.h, C.byref(n)))
    assert n.value == 0
    m.Close()


def test_graph_adam_timestep_moved(gn, dev):
    """A timestep moved from the host between replays (a checkpoint restore,
    gn_model_set_adam, far ahead and back): the update after each replayed
    pass takes its bias corrections from the model's timestep, so every step
    equals the eager model's bit for bit."""
    from goneuron_amd import configs
    from goneuron_amd._lib import check, lib
    L = lib()
    cfg = configs.mlp()
    x, y = configs.inputs(cfg)
    g = configs.build(cfg, device=dev)
    e = configs.build(cfg, device=dev)
    check(dev.h, L.gn_model_set_graphs(e.h, 0))
    for step in range(12):
        if step in (4, 8):
            t = 5000 if step == 4 else 7
            for m in (g, e):
                check(dev.h, L.gn_model_set_adam(m.h, None, None, 0, 0, t))
        lg, le = g.TrainBatch(x, y), e.TrainBatch(x, y)
        assert lg == le, (step, lg, le)
        sg, se = _state(g), _state(e)
        for part, a, b in zip(("params", "grads", "m", "v"), sg[:4], se[:4]):
            np.testing.assert_array_equal(a, b, err_msg=f"step {step} {part}")
        assert sg[4] == se[4]
    n = C.c_int32()
    check(dev.h, L.gn_model_graph_count(g.h, C.byref(n)))
    assert n.value == 1
    g.Close()
    e.Close()
