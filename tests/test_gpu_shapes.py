"""GPU parity for layer arrangements the reference accepts beyond the benchmark
configs: a SequenceUnroller (LSTM or GRU) or an Embedding below other layers,
unrollers that return every state, and output layers that are not Dense.

  - SequenceUnroller not first: it hands the layer below dx_t = Wx^T dG_t for
    every step (lstm.go:642-663, gru.go:481-500, stacked by
    unroller.go:200-206), from the unclipped deltas;
  - Embedding not first: floor() of the layer below's outputs are its ids, and
    the layer below gets a zero gradient (embedding.go:156-163);
  - SequenceUnroller(returnSequences = true) outputs every step's state and
    adds each step's own gradient to the carried one (unroller.go:115-119,
    192-198);
  - a non-Dense output layer receives the loss gradient itself (Network.Forward
    hands its output to the loss, net.go:212-223).

Each case runs two training steps on the GPU and the oracle from the same
weights, every parameter tensor to 1e-4 (gpuutil.compare_step)."""
import numpy as np
import pytest

from gpuutil import compare_step

pytestmark = pytest.mark.gpu


def _dense(i, o, act, ptr=False):
    return {"kind": "dense", "in": i, "out": o, "act": act, "ptr": ptr}


def _normal(rng, *shape):
    return rng.normal(size=shape).astype(np.float32)


def _onehot(rng, B, C):
    y = np.zeros((B, C), np.float32)
    y[np.arange(B), rng.integers(0, C, size=B)] = 1
    return y


def cases():
    """name -> (config, (x, y))"""
    rng = np.random.default_rng(5)
    out = {}
    B = 6
    # Dense -> LSTM -> Dense (the unroller's input is the Dense output, T x I)
    out["dense_lstm"] = (dict(num=21, name="dense_lstm", B=B, loss="mse", lr=1e-3, x="normal", in_len=10,
                              layers=[_dense(10, 5 * 4, "tanh"),
                                      {"kind": "lstm", "in": 4, "hidden": 8, "T": 5},
                                      _dense(8, 1, "linear")]),
                         (_normal(rng, B, 10), _normal(rng, B, 1)))
    # Conv2D -> Flatten -> SequenceUnroller(LSTM, T = 1) -> Dense (examples/stock_prediction_cnn_lstm)
    out["conv_lstm"] = (dict(num=22, name="conv_lstm", B=B, loss="mse", lr=1e-3, x="normal", in_len=36,
                             layers=[{"kind": "conv2d", "inC": 1, "outC": 2, "k": 3, "s": 1, "p": 1,
                                      "act": "relu"},
                                     {"kind": "flatten", "n": 72},
                                     {"kind": "lstm", "in": 72, "hidden": 6, "T": 1},
                                     _dense(6, 1, "linear")]),
                        (_normal(rng, B, 36), _normal(rng, B, 1)))
    # Dense -> GRU -> Dense
    out["dense_gru"] = (dict(num=23, name="dense_gru", B=B, loss="mse", lr=1e-3, x="normal", in_len=9,
                             layers=[_dense(9, 3 * 4, "sigmoid"),
                                     {"kind": "gru", "in": 4, "hidden": 5, "T": 3},
                                     _dense(5, 1, "linear")]),
                        (_normal(rng, B, 9), _normal(rng, B, 1)))
    # Embedding -> LSTM -> Dense(Softmax) + CE (the unroller second, fed by the table rows)
    V, T, D = 30, 7, 6
    out["embedding_lstm"] = (dict(num=24, name="embedding_lstm", B=B, loss="ce", lr=1e-3, x="ids", in_len=T,
                                  classes=3,
                                  layers=[{"kind": "embedding", "vocab": V, "dim": D},
                                          {"kind": "lstm", "in": D, "hidden": 8, "T": T},
                                          _dense(8, 3, "softmax", True)]),
                             (rng.integers(0, V, size=(B, T)).astype(np.float32), _onehot(rng, B, 3)))
    # Dense(ReLU) -> Embedding (ids = floor of the ReLU outputs) -> Flatten -> Dense
    out["dense_embedding"] = (dict(num=25, name="dense_embedding", B=B, loss="mse", lr=1e-3, x="normal",
                                   in_len=4,
                                   layers=[_dense(4, 5, "relu"),
                                           {"kind": "embedding", "vocab": 12, "dim": 3, "T": 5},
                                           {"kind": "flatten", "n": 15},
                                           _dense(15, 2, "linear")]),
                              ((_normal(rng, B, 4) * 3).astype(np.float32), _normal(rng, B, 2)))
    # SequenceUnroller(returnSequences = true): every state out, every step's gradient in
    out["lstm_seq"] = (dict(num=29, name="lstm_seq", B=B, loss="mse", lr=1e-3, x="normal", in_len=5 * 3,
                            layers=[{"kind": "lstm", "in": 3, "hidden": 6, "T": 5, "seq": True},
                                    _dense(30, 1, "linear")]),
                       (_normal(rng, B, 15), _normal(rng, B, 1)))
    # H = 32: the cooperative BPTT kernel with the per-step gradients; then a
    # second unroller on the state sequence (examples/stock_prediction_bilstm stacks them)
    out["lstm_seq_coop_stack"] = (dict(num=30, name="lstm_seq_coop_stack", B=8, loss="mse", lr=1e-3,
                                       x="normal", in_len=7 * 4,
                                       layers=[{"kind": "lstm", "in": 4, "hidden": 32, "T": 7, "seq": True},
                                               {"kind": "lstm", "in": 32, "hidden": 8, "T": 7},
                                               _dense(8, 2, "linear")]),
                                  (_normal(rng, 8, 28), _normal(rng, 8, 2)))
    out["gru_seq"] = (dict(num=31, name="gru_seq", B=B, loss="mse", lr=1e-3, x="normal", in_len=4 * 3,
                           layers=[{"kind": "gru", "in": 3, "hidden": 5, "T": 4, "seq": True},
                                   _dense(20, 2, "linear")]),
                      (_normal(rng, B, 12), _normal(rng, B, 2)))
    # Conv2D -> MaxPool2D -> Flatten -> Dropout -> Dense: Dropout above a Flatten
    out["flatten_dropout"] = (dict(num=32, name="flatten_dropout", B=B, loss="ce", lr=1e-3, x="normal",
                                   in_len=2 * 6 * 6, classes=3,
                                   layers=[{"kind": "conv2d", "inC": 2, "outC": 3, "k": 3, "s": 1, "p": 1,
                                            "act": "relu"},
                                           {"kind": "maxpool2d", "k": 2, "s": 2, "p": 0, "inC": 3},
                                           {"kind": "flatten", "n": 27},
                                           {"kind": "dropout", "p": 0.25, "n": 27},
                                           _dense(27, 3, "softmax", True)]),
                              (_normal(rng, B, 72), _onehot(rng, B, 3)))
    # output layers that are not Dense
    out["dropout_out"] = (dict(num=26, name="dropout_out", B=B, loss="mse", lr=1e-3, x="normal", in_len=10,
                               layers=[_dense(10, 6, "relu"), {"kind": "dropout", "p": 0.3, "n": 6}]),
                          (_normal(rng, B, 10), _normal(rng, B, 6)))
    out["lstm_out"] = (dict(num=27, name="lstm_out", B=B, loss="mse", lr=1e-3, x="normal", in_len=5 * 3,
                            layers=[{"kind": "lstm", "in": 3, "hidden": 4, "T": 5}]),
                       (_normal(rng, B, 15), _normal(rng, B, 4)))
    out["conv_out"] = (dict(num=28, name="conv_out", B=B, loss="mse", lr=1e-3, x="normal", in_len=2 * 5 * 5,
                            layers=[_dense(50, 50, "tanh"),
                                    {"kind": "conv2d", "inC": 2, "outC": 3, "k": 3, "s": 1, "p": 1,
                                     "act": "sigmoid"}]),
                       (_normal(rng, B, 50), _normal(rng, B, 75)))
    return out


@pytest.mark.parametrize("name", sorted(cases()))
def test_layer_arrangements(gn, oracle, name):
    cfg, xy = cases()[name]
    compare_step(gn, oracle, cfg, steps=2, xy=xy)
