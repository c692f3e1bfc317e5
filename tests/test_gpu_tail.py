"""GPU parity of the fused output-layer kernels.

A training pass whose output layer is a Dense with at most 32 outputs and an
input width that is a multiple of 4 runs that layer as two kernels: the
forward product fused with the loss rows (activation, loss, loss gradient
through the Jacobian / derivative, layer.go:405-470 + loss.go), and one
backward kernel for dW, db and dX with the dX GEMM's epilogue (a Dropout's
factor, act' of the layer below), which also sums the bias and weight
gradients of a Dense whose dz that dX is.

Each case:
  - runs two training steps against the oracle (gpuutil.compare_step, every
    tensor to 1e-4, with the worker split W of the case);
  - checks from the per-launch timing records that the fused kernels ran, and
    that gn_debug_fused_tail(0) gives the GEMM / loss-row path instead;
  - compares the two paths' loss and gradients with each other (to 1e-5:
    both are float32 products over the same terms in different orders).

The cases cover the three kernel shapes (outputs <= 4, <= 16, <= 32), the
split-K partials of the Dense below summed by the output kernel (with and
without a Dropout between), a batch
that leaves the last block of rows partial, batches beyond one 64-row chunk
of the backward, each kind of layer below (a Dense with its act', a Dropout
over a Dense, a Flatten over pooling) and Embedding index errors under a
W-worker split."""
import ctypes as C

import numpy as np
import pytest

from gpuutil import compare_step, log

pytestmark = pytest.mark.gpu


def _dense(i, o, act, ptr=False):
    return {"kind": "dense", "in": i, "out": o, "act": act, "ptr": ptr}


def _onehot(rng, B, C_):
    y = np.zeros((B, C_), np.float32)
    y[np.arange(B), rng.integers(0, C_, size=B)] = 1
    return y


def cases():
    """name -> (config, workers, (x, y) or None)"""
    from goneuron_amd import configs
    rng = np.random.default_rng(11)
    out = {}
    out["mlp_w4"] = (configs.mlp(), 4, None)
    out["mlp_w1"] = (configs.mlp(), 1, None)
    # one output (the 4-wide kernels, 16 rows a block: 37 rows leave 5 in the last)
    B = 37
    out["mse_one_output"] = (dict(num=41, name="mse_one_output", B=B, loss="mse", lr=1e-3, x="normal", in_len=12,
                                  layers=[_dense(12, 24, "sigmoid"), _dense(24, 1, "linear")]),
                             1, (rng.normal(size=(B, 12)).astype(np.float32),
                                 rng.normal(size=(B, 1)).astype(np.float32)))
    # 20 classes (the 32-wide kernels) under a Dropout over a ReLU Dense
    B = 5
    out["softmax_20"] = (dict(num=42, name="softmax_20", B=B, loss="ce", lr=1e-3, x="normal", in_len=16,
                              classes=20,
                              layers=[_dense(16, 32, "relu"), {"kind": "dropout", "p": 0.25, "n": 32},
                                      _dense(32, 20, "softmax", True)]),
                         1, (rng.normal(size=(B, 16)).astype(np.float32), _onehot(rng, B, 20)))
    # 130 rows in three chunks of the backward, three workers
    B = 130
    out["logsoftmax_16"] = (dict(num=43, name="logsoftmax_16", B=B, loss="ce", lr=1e-3, x="normal", in_len=20,
                                 classes=16,
                                 layers=[_dense(20, 64, "tanh"), _dense(64, 16, "logsoftmax", True)]),
                            3, (rng.normal(size=(B, 20)).astype(np.float32), _onehot(rng, B, 16)))
    # an element-wise output activation with the MSE loss
    B = 6
    out["sigmoid_out"] = (dict(num=44, name="sigmoid_out", B=B, loss="mse", lr=1e-3, x="normal", in_len=8,
                               layers=[_dense(8, 24, "relu"), _dense(24, 5, "sigmoid")]),
                          1, (rng.normal(size=(B, 8)).astype(np.float32),
                              rng.uniform(size=(B, 5)).astype(np.float32)))
    # a Dense below with K = 1024 (its GEMM splits K): the output kernel sums
    # the partials, applies the bias and tanh, and writes that layer's output
    B = 40
    out["split_below"] = (dict(num=46, name="split_below", B=B, loss="mse", lr=1e-3, x="normal", in_len=1024,
                               layers=[_dense(1024, 48, "tanh"), _dense(48, 5, "sigmoid")]),
                          3, (rng.normal(size=(B, 1024)).astype(np.float32),
                              rng.uniform(size=(B, 5)).astype(np.float32)))
    # three Dense layers: the middle one's weight gradient comes from the
    # output kernel, its input gradient from its own dX GEMM
    B = 70
    out["three_dense"] = (dict(num=47, name="three_dense", B=B, loss="ce", lr=1e-3, x="normal", in_len=10,
                               classes=3,
                               layers=[_dense(10, 16, "relu"), _dense(16, 24, "tanh"),
                                       _dense(24, 3, "softmax", True)]),
                          2, (rng.normal(size=(B, 10)).astype(np.float32), _onehot(rng, B, 3)))
    # C2's layers at a small batch: the input gradient goes to a Flatten over MaxPool2D
    out["cnn_small"] = (configs.cnn(B=9), 1, None)
    # Embedding index errors under two workers: the skipped samples' rows and chunk losses
    B = 8
    ids = rng.integers(0, 15, size=(B, 5)).astype(np.float32)
    ids[2, 3] = 21.0
    out["embedding_bad_ids"] = (dict(num=45, name="embedding_bad_ids", B=B, loss="ce", lr=1e-3, x="ids",
                                     in_len=5, classes=3,
                                     layers=[{"kind": "embedding", "vocab": 15, "dim": 4, "T": 5},
                                             {"kind": "flatten", "n": 20},
                                             _dense(20, 3, "softmax", True)]),
                                2, (ids, _onehot(rng, B, 3)))
    return out


def _set_tail(model, on):
    from goneuron_amd._lib import lib
    assert lib().gn_debug_fused_tail(model.h, 1 if on else 0) == 0


def _kernel_names(dev, model, x, y):
    from goneuron_amd._lib import KernelStat, lib
    L = lib()
    assert L.gn_timing_enable(dev.h, 1) == 0
    try:
        model.TrainBatch(x, y)
        cap = 256
        arr = (KernelStat * cap)()
        n = C.c_int32()
        assert L.gn_timing_kernels(dev.h, arr, cap, C.byref(n)) == 0
        return {arr[i].name.decode() for i in range(min(n.value, cap))}
    finally:
        assert L.gn_timing_enable(dev.h, 0) == 0


@pytest.mark.parametrize("name", sorted(cases()))
def test_fused_output_layer(gn, oracle, dev, name):
    from goneuron_amd import configs
    cfg, workers, xy = cases()[name]
    x, y = configs.inputs(cfg) if xy is None else xy
    compare_step(gn, oracle, cfg, steps=2, workers=workers, xy=xy)
    on = configs.build(cfg, workers=workers)
    off = configs.build(cfg, workers=workers)
    _set_tail(off, False)
    k_on, k_off = _kernel_names(dev, on, x, y), _kernel_names(dev, off, x, y)
    log(f"{name}: fused {sorted(k_on)}; unfused {sorted(k_off)}")
    assert {"tail_fwd", "tail_bwd"} <= k_on and "out_rows" not in k_on
    assert not ({"tail_fwd", "tail_bwd"} & k_off) and "out_rows" in k_off
    # the next step on both paths from equal weights (the gradients and the
    # loss do not depend on the Adam moments)
    off.SetParams(on.Params())
    lon, loff = on.TrainBatch(x, y), off.TrainBatch(x, y)
    assert abs(lon - loff) <= 1e-5 * max(abs(loff), 1e-30), (lon, loff)
    g_on, g_off = on.Gradients(), off.Gradients()
    scale = float(np.abs(g_off).max())
    assert float(np.abs(g_on - g_off).max()) <= 1e-5 * scale, float(np.abs(g_on - g_off).max()) / scale
    on.Close()
    off.Close()
