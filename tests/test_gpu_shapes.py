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
    hands its output to the loss, net.go:212-223);
  - standalone LayerNorm, MultiHeadAttention and GlobalAveragePooling1D
    (goneuron.go:220-227, 369-381), hidden Softmax / LogSoftmax Dense layers
    (layer.go:504-560) and a second Embedding.

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
    # standalone LayerNorm between Dense layers (rows of 8 in a 16-wide sample)
    out["layernorm_mlp"] = (dict(num=33, name="layernorm_mlp", B=B, loss="ce", lr=1e-3, x="normal", in_len=12,
                                 classes=3,
                                 layers=[_dense(12, 16, "relu"),
                                         {"kind": "layernorm", "n": 8, "len": 16},
                                         _dense(16, 3, "softmax", True)]),
                            (_normal(rng, B, 12), _onehot(rng, B, 3)))
    # Embedding -> PositionalEncoding -> MultiHeadAttention -> LayerNorm ->
    # GlobalAveragePooling1D -> Dense(Softmax): the standalone attention layer
    V, T, D = 20, 6, 8
    out["mha_gap"] = (dict(num=34, name="mha_gap", B=B, loss="ce", lr=1e-3, x="ids", in_len=T, classes=4,
                           layers=[{"kind": "embedding", "vocab": V, "dim": D},
                                   {"kind": "posenc", "T": T, "dim": D},
                                   {"kind": "mha", "heads": 2, "T": T, "causal": True, "dim": D},
                                   {"kind": "layernorm", "n": D, "len": T * D},
                                   {"kind": "gap1d", "T": T, "dim": D},
                                   _dense(D, 4, "softmax", True)]),
                      (rng.integers(0, V, size=(B, T)).astype(np.float32), _onehot(rng, B, 4)))
    # non-causal attention with heads wider than 32 (the batched-GEMM path), last
    out["mha_wide_out"] = (dict(num=35, name="mha_wide_out", B=B, loss="mse", lr=1e-3, x="normal",
                                in_len=5 * 80,
                                layers=[{"kind": "mha", "heads": 2, "T": 5, "causal": False, "dim": 80}]),
                           (_normal(rng, B, 400), _normal(rng, B, 400)))
    # hidden Softmax / LogSoftmax Dense layers: the row Jacobian on the
    # gradient from above (layer.go:504-560)
    out["hidden_softmax"] = (dict(num=36, name="hidden_softmax", B=B, loss="ce", lr=1e-3, x="normal",
                                  in_len=10, classes=3,
                                  layers=[_dense(10, 8, "softmax", True), _dense(8, 6, "relu"),
                                          _dense(6, 3, "logsoftmax", True)]),
                             (_normal(rng, B, 10), _onehot(rng, B, 3)))
    out["hidden_logsoftmax_dropout"] = (dict(num=37, name="hidden_logsoftmax_dropout", B=B, loss="mse", lr=1e-3,
                                             x="normal", in_len=10,
                                             layers=[_dense(10, 8, "logsoftmax", True),
                                                     {"kind": "dropout", "p": 0.25, "n": 8},
                                                     _dense(8, 2, "tanh")]),
                                        (_normal(rng, B, 10), _normal(rng, B, 2)))
    # two Embeddings: the second reads floor() of ReLU outputs as ids, some
    # out of range (those samples are skipped, as is one with a bad first id)
    x2 = rng.integers(0, 15, size=(8, 5)).astype(np.float32)
    x2[3, 1] = 17.0
    out["two_embeddings"] = (dict(num=38, name="two_embeddings", B=8, loss="mse", lr=1e-3, x="ids", in_len=5,
                                  classes=15,
                                  layers=[{"kind": "embedding", "vocab": 15, "dim": 4, "T": 5},
                                          {"kind": "flatten", "n": 20},
                                          _dense(20, 6, "relu"),
                                          {"kind": "embedding", "vocab": 9, "dim": 3, "T": 6},
                                          {"kind": "flatten", "n": 18},
                                          _dense(18, 2, "linear")]),
                             (x2, _normal(rng, 8, 2)))
    return out


def _perturb_mha(cfg):
    """MultiHeadAttention starts at zero (Q11): random weights, so attention
    and its gradients are live from the first step."""
    offs, o = [], 0
    for d in cfg["layers"]:
        n = 0
        if d["kind"] == "dense":
            n = d["in"] * d["out"] + d["out"]
        elif d["kind"] == "embedding":
            n = d["vocab"] * d["dim"]
        elif d["kind"] == "posenc":
            n = d["T"] * d["dim"]
        elif d["kind"] == "layernorm":
            n = 2 * d["n"]
        elif d["kind"] == "mha":
            n = 4 * (d["dim"] * d["dim"] + d["dim"])
            offs.append((o, n, d["dim"]))
        o += n

    def f(p):
        rng = np.random.default_rng(41)
        for o0, n, D in offs:
            p[o0:o0 + n] = (rng.normal(size=n) * (0.7 / np.sqrt(D))).astype(np.float32)
        return p
    return f


@pytest.mark.parametrize("name", sorted(cases()))
def test_layer_arrangements(gn, oracle, name):
    cfg, xy = cases()[name]
    perturb = _perturb_mha(cfg) if any(d["kind"] == "mha" for d in cfg["layers"]) else None
    compare_step(gn, oracle, cfg, steps=2, xy=xy, perturb=perturb)


@pytest.mark.parametrize("dim", [16, 320])
def test_transformer_batch_times_heads_beyond_grid(gn, oracle, dim):
    """A TransformerBlock training step over 8,200 samples x 8 heads (more
    (sample, head) pairs than a grid dimension holds): heads 2 wide take the
    fused kernels (pairs on the grid's x dimension), heads 40 wide the
    batched GEMMs in chunks of samples.  The batch repeats 10 distinct
    samples 820 times, so its loss and batch-averaged gradients equal the
    10-sample batch's, which the oracle computes; the last sample (the one
    the embedding gradient comes from, Q12) is the 10th distinct one."""
    from cfgutil import max_rel, oracle_net, tensor_parts
    from goneuron_amd import configs
    from gpuutil import TOL, log, random_block
    nd, reps = 10, 820
    small = configs.gpt(B=nd, T=4, vocab=11, dim=dim, heads=8, ff=12)
    big = configs.gpt(B=nd * reps, T=4, vocab=11, dim=dim, heads=8, ff=12)
    log(f"transformer B={big['B']} heads=8 dim={dim}: {big['B'] * 8} (sample, head) pairs")
    x, y = configs.inputs(small)
    model = configs.build(big, workers=1)
    net = oracle_net(oracle, small)
    p = random_block(small, scale=0.1)(net.params.copy())
    net.params[:] = p
    model.SetParams(p)
    lg = model.TrainBatch(np.tile(x, (reps, 1)), np.tile(y, (reps, 1)))
    lo = net.accumulate_batch(x, y, nd)
    # float32 sums over 8,200 samples (in sample order, as the reference's
    # batch loop) round to about B * 2^-24 of their value; the oracle's
    # 10-sample sums hardly at all
    gtol = max(TOL, big["B"] * 2.0 ** -24)
    assert abs(lg - lo) <= gtol * abs(lo), (lg, lo)
    g, r = model.Gradients(), net.grads
    for name, sl in tensor_parts(small, net):
        ref = r[sl]
        got = g[sl]
        if name.endswith("embedding.E"):
            # Q12: the last sample's rows alone, times 1/B (embedding.go:152-154)
            got = got * np.float32(big["B"] / nd)
        if np.abs(ref).max() <= 1e-6 * np.abs(r).max():
            continue
        assert max_rel(got, ref) <= gtol, (name, max_rel(got, ref))
    model.Close()
