"""GPU tests of the reference's batch-loop semantics around the hot path:
training flags across Predict and worker clones, batches larger than the
buffers were made for, samples skipped on an Embedding index error, MoE
routing indices, and the per-layer Dense entry points.  All against the
oracle (or float64 numpy for the single-layer ops) through the C ABI."""
import ctypes as C

import numpy as np
import pytest

from cfgutil import max_rel, norm_rel, oracle_net, tensor_parts
from gpuutil import DBuf, TOL, compare_step, log, random_block

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ training flags
@pytest.mark.parametrize("workers", [1, 4])
def test_predict_then_train_keeps_flags_off(gn, oracle, workers):
    """Sequential.Predict turns every layer's training flag off and leaves it
    off (sequential.go:118-122); TrainBatch does not turn it back on.  With
    W = 1 the next step runs Dropout as identity.  With W = 4 the first
    TrainBatch made the worker clones with Dropout on, and SetTraining never
    reaches them (net.go:129-152, 187-193), so after Predict the parallel
    step still drops units.  Then Fit-style SetTraining(true)."""
    from goneuron_amd import configs
    cfg = configs.mlp()
    x, y = configs.inputs(cfg)
    B = cfg["B"]
    model = configs.build(cfg, workers=workers)
    net = oracle_net(oracle, cfg, workers=workers)
    parts = tensor_parts(cfg, net)

    def step(tag):
        lg = model.TrainBatch(x, y)
        lo = net.accumulate_batch(x, y, B)
        g, r = model.Gradients(), net.grads.copy()
        assert abs(lg - lo) <= TOL * abs(lo), (tag, lg, lo)
        bad = {n: e for n, sl in parts if (e := max_rel(g[sl], r[sl])) > TOL}
        assert not bad, (tag, bad)
        net.step()
        p = model.Params()
        assert norm_rel(p, net.params) <= TOL, tag
        net.params[:] = p
        return g

    g_train = step("fresh")
    assert model.IsTraining(1)
    out = model.PredictBatch(x[:8])
    net.set_training(False)  # what Predict does to the network
    assert not model.IsTraining(1)
    ref = np.stack([net.forward(x[b]) for b in range(8)])
    assert max_rel(out, ref) <= TOL
    g_after = step("after predict")
    # W = 1: dropout off changes the first layer's gradient; W = 4: the clones still drop
    sl = parts[0][1]
    if workers == 1:
        assert max_rel(g_after[sl], g_train[sl]) > 1e-3
    model.SetTraining(True)
    net.set_training(True)
    step("after SetTraining(true)")


def test_moe_starts_without_training_mode(gn, oracle):
    """NewMoE leaves its training flag false, so a bare TrainBatch routes
    without gate noise and adds no load-balancing gradient; Dropout and
    BatchNorm2D start in training mode."""
    from goneuron_amd.configs import dense
    cfg = dict(num=16, name="moe_flag", B=24, loss="ce", lr=1e-3, x="normal", in_len=12, classes=4,
               layers=[dense(12, 16, "relu"), {"kind": "dropout", "p": 0.3, "n": 16},
                       {"kind": "moe", "in": 16, "out": 8, "E": 4, "k": 2},
                       dense(8, 4, "softmax", True)])
    model, _ = compare_step(gn, oracle, cfg, steps=2,
                            perturb=lambda p: (p + np.random.default_rng(3).normal(size=p.size)
                                               .astype(np.float32) * 0.2))
    assert model.IsTraining(1) and not model.IsTraining(2)


# ------------------------------------------------------------------ batch above max_batch
def test_batch_above_max_batch_keeps_state(gn, oracle):
    """TrainBatch / PredictBatch with more samples than the model's buffers
    hold grow them and keep parameters, Adam moments and timestep: three
    steps at B = 40, 96, 40 and a 300-sample PredictBatch against the oracle
    doing the same."""
    from goneuron_amd import configs
    from goneuron_amd.configs import dense
    cfg = dict(num=3, name="grow", B=96, loss="ce", lr=1e-3, x="normal", in_len=48, classes=9,
               layers=[dense(48, 64, "relu"), {"kind": "dropout", "p": 0.25, "n": 64},
                       dense(64, 9, "softmax", True)])
    x, y = configs.inputs(cfg, B=300)
    model = configs.build(cfg, workers=1, max_batch=40)
    net = oracle_net(oracle, cfg)
    assert model.max_batch == 40
    for B in (40, 96, 40):
        lg = model.TrainBatch(x[:B], y[:B])
        lo = net.train_batch(x[:B], y[:B], B)
        assert abs(lg - lo) <= TOL * abs(lo), (B, lg, lo)
        p = model.Params()
        assert norm_rel(p, net.params) <= TOL, B
        net.params[:] = p
    assert model.max_batch == 96
    m, v, t = model.AdamState()
    assert t == net.timestep == 3
    assert norm_rel(m, net.adam_m) <= TOL and norm_rel(v, net.adam_v) <= TOL
    out = model.PredictBatch(x)
    assert model.max_batch == 300
    net.set_training(False)
    ref = np.stack([net.forward(x[b]) for b in range(300)])
    assert max_rel(out, ref) <= TOL


# ------------------------------------------------------------------ embedding index errors
@pytest.mark.parametrize("workers,bad", [(1, [1]), (1, [0, 3]), (2, [1]), (2, [0, 5]), (3, [4])])
def test_embedding_bad_index_skips_samples(gn, oracle, workers, bad):
    """An out-of-range token makes Embedding.Forward fail; the batch loop
    skips the sample (trainBatchSequential: that sample only; a
    trainBatchParallel worker: the rest of its chunk, and the chunk's loss is
    lost) and the step still applies.  Loss, every gradient tensor (Q12's
    last-sample embedding gradient included) and the updated weights against
    the oracle, with a random block; SkippedSamples counts the skipped ones;
    inference on the same batch reports GN_ERR_INDEX."""
    from goneuron_amd import configs
    cfg = configs.gpt(B=6, T=8, vocab=23, dim=16, heads=2, ff=24)
    x, y = configs.inputs(cfg)
    for b in bad:
        x[b, 3] = 23 + b  # outside [0, 23)
    model, _ = compare_step(gn, oracle, cfg, steps=2, workers=workers, perturb=random_block(cfg),
                            xy=(x, y))
    W = min(workers, 6)
    if W == 1:
        want = len(bad)
    else:
        chunk = (6 + W - 1) // W
        want = 0
        for c0 in range(0, 6, chunk):
            first = [b for b in bad if c0 <= b < c0 + chunk]
            want += (min(6, c0 + chunk) - min(first)) if first else 0
    assert model.SkippedSamples() == want
    with pytest.raises(gn.GNError) as e:
        model.PredictBatch(x)
    assert e.value.code == -8
    assert model.SkippedSamples() == 0  # the last pass was inference


# ------------------------------------------------------------------ MoE routes
@pytest.mark.parametrize("workers", [1, 4])
def test_moe_routes_bit_exact(gn, oracle, workers):
    """Top-k routing indices (moe.go:140-234: noisy softmax in training mode,
    descending stable order) equal the oracle's for every sample, in training
    mode over two steps (the noise streams run on) and in inference."""
    from goneuron_amd import configs
    E, K, B = 12, 3, 64
    cfg = dict(num=16, name="moe_routes", B=B, loss="mse", lr=1e-3, x="normal", in_len=20, classes=6,
               layers=[{"kind": "moe", "in": 20, "out": 10, "E": E, "k": K},
                       {"kind": "dense", "in": 10, "out": 6, "act": "linear", "ptr": False}])
    x, y = configs.inputs(cfg)
    model = configs.build(cfg, workers=workers)
    net = oracle_net(oracle, cfg, workers=workers)
    rng = np.random.default_rng(8)
    sl = net.layer_slice(0)
    p = net.params.copy()
    p[sl] = (rng.normal(size=sl.stop - sl.start) * 0.3).astype(np.float32)
    net.params[:] = p
    model.SetParams(p)
    model.SetTraining(True)
    net.set_training(True)
    net.routes(0)  # start the oracle's route log
    for s in range(2):
        model.TrainBatch(x, y)
        net.accumulate_batch(x, y, B)
        got = model.LayerArgmax(0, B * K)
        ref = net.routes(0)
        log(f"  step {s}: {int((got != ref).sum())} of {B * K} routes differ")
        np.testing.assert_array_equal(got, ref)
        net.step()
        net.params[:] = model.Params()
    model.PredictBatch(x)
    net.set_training(False)
    for b in range(B):
        net.forward(x[b])
    np.testing.assert_array_equal(model.LayerArgmax(0, B * K), net.routes(0))


# ------------------------------------------------------------------ per-layer Dense ops
def _dact(out, act):
    if act == 1:
        return (out > 0).astype(np.float64)
    if act == 2:
        return out * (1 - out)
    if act == 3:
        return 1 - out * out
    return np.ones_like(out)


@pytest.mark.parametrize("act,ptr", [(1, 0), (2, 0), (3, 0), (6, 0), (4, 1), (5, 1)])
@pytest.mark.parametrize("B,I,O", [(64, 784, 128), (37, 91, 53), (256, 512, 1000)])
def test_dense_ops(gn, dev, act, ptr, B, I, O):
    """gn_dense_forward / gn_dense_backward (Dense.Forward / Backward over a
    batch, layer.go:346-667) against float64: out = act(b + x W^T), dz = g *
    act'(out) (Softmax / LogSoftmax pointers: their Jacobians), gradW = s dz^T
    x, gradB = s colsum(dz), gin = dz W."""
    from goneuron_amd._lib import lib, check
    rng = np.random.default_rng(B + I + O + act)
    x = rng.normal(size=(B, I)).astype(np.float32)
    W = (rng.normal(size=(O, I)) * 0.05).astype(np.float32)
    b = (rng.normal(size=O) * 0.1).astype(np.float32)
    g = rng.normal(size=(B, O)).astype(np.float32)
    dx, dW, db, dg = DBuf(dev, x), DBuf(dev, W), DBuf(dev, b), DBuf(dev, g)
    dout = DBuf(dev, np.zeros((B, O), np.float32))
    check(dev.h, lib().gn_dense_forward(dev.h, dx.p, dW.p, db.p, dout.p, B, I, O, act, ptr))
    out = dout.get()
    z = x.astype(np.float64) @ W.T.astype(np.float64) + b
    if act == 1:
        ref = np.maximum(z, 0)
    elif act == 2:
        ref = 1 / (1 + np.exp(-z))
    elif act == 3:
        ref = np.tanh(z)
    elif act == 4:
        e = np.exp(z - z.max(1, keepdims=True))
        ref = e / e.sum(1, keepdims=True)
    elif act == 5:
        ref = z - z.max(1, keepdims=True) - np.log(np.exp(z - z.max(1, keepdims=True)).sum(1, keepdims=True))
    else:
        ref = z
    assert max_rel(out, ref) <= 1e-5, max_rel(out, ref)
    dgW, dgB = DBuf(dev, np.zeros((O, I), np.float32)), DBuf(dev, np.zeros(O, np.float32))
    dgin, dz = DBuf(dev, np.zeros((B, I), np.float32)), DBuf(dev, np.zeros((B, O), np.float32))
    scale = np.float32(1.0) / np.float32(B)
    check(dev.h, lib().gn_dense_backward(dev.h, dx.p, dW.p, dout.p, dg.p, dgW.p, dgB.p, dgin.p, dz.p,
                                         B, I, O, act, ptr, C.c_float(scale)))
    o64 = out.astype(np.float64)
    g64 = g.astype(np.float64)
    if act == 4:
        dzr = o64 * g64 - o64 * (g64 * o64).sum(1, keepdims=True)
    elif act == 5:
        dzr = g64 - np.exp(o64) * g64.sum(1, keepdims=True)
    else:
        dzr = g64 * _dact(o64, act)
    for name, got, want in (("gradW", dgW.get(), float(scale) * dzr.T @ x.astype(np.float64)),
                            ("gradB", dgB.get(), float(scale) * dzr.sum(0)),
                            ("gin", dgin.get(), dzr @ W.astype(np.float64))):
        assert max_rel(got, want) <= TOL, (name, max_rel(got, want))
