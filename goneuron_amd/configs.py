"""The five BASELINE training-step configurations and their synthetic inputs.

Layers are described neutrally (dicts) so that the same description builds the
GPU model (``build``) and, in tests, the CPU oracle.  Inputs come from the
reference's LCG (layer.go:61-81) with seeds 1000 + config number (inputs) and
2000 + config number (targets).
"""
from __future__ import annotations

import numpy as np

from . import (CrossEntropy, MSE, Adam, Dense, Dropout, Conv2D, MaxPool2D, AvgPool2D, BatchNorm2D, MoE,
               RMSNorm, LayerNorm, MultiHeadAttention, GlobalAveragePooling1D,
               SwiGLU, Flatten, TransformerBlockExt, ActReLU, ActSwiGLU, ActGELU, NormLN, NormRMS,
               Embedding,
               PositionalEncoding, TransformerBlock, CLSPooling, LSTM, GRU, SequenceUnroller, ReLU,
               Sigmoid, Tanh, Linear, GELU, Softmax, LogSoftmax, Ref, NewSequential, fill_normal,
               fill_uniform, fill_class_ids)

BLOCK_ACTS = {"relu": ActReLU, "swiglu": ActSwiGLU, "gelu": ActGELU}
BLOCK_NORMS = {"ln": NormLN, "rms": NormRMS}
_ACTS = {"relu": ReLU, "sigmoid": Sigmoid, "tanh": Tanh, "linear": Linear, "softmax": Softmax,
         "logsoftmax": LogSoftmax, "gelu": GELU}


def dense(i, o, act, ptr=False):
    return {"kind": "dense", "in": i, "out": o, "act": act, "ptr": ptr}


def mlp(hidden=128):
    return dict(num=1, name="mlp", B=64, loss="ce", lr=1e-3, x="uniform", in_len=784,
                classes=10,
                layers=[dense(784, hidden, "relu"), {"kind": "dropout", "p": 0.2, "n": hidden},
                        dense(hidden, 10, "softmax", True)])


def cnn(B=128):
    return dict(num=2, name="cnn", B=B, loss="ce", lr=1e-3, x="normal", in_len=3 * 32 * 32,
                classes=10,
                layers=[{"kind": "conv2d", "inC": 3, "outC": 16, "k": 3, "s": 1, "p": 1, "act": "relu"},
                        {"kind": "maxpool2d", "k": 2, "s": 2, "p": 0, "inC": 16},
                        {"kind": "flatten", "n": 4096},
                        dense(4096, 10, "softmax", True)])


def wide(width=4096, classes=1000, depth=4, B=1024):
    ls = [dense(width, width, "relu") for _ in range(depth)]
    ls.append(dense(width, classes, "logsoftmax", True))
    return dict(num=3, name="wide", B=B, loss="ce", lr=1e-3, x="normal", in_len=width,
                classes=classes, layers=ls)


def gpt(B=32, T=128, vocab=8000, dim=256, heads=8, ff=1024, causal=True, act="relu", norm="ln",
        rope=False):
    """C4; act / norm / rope select TransformerBlockExt's feed-forward
    ("relu", "swiglu", "gelu"), norms ("ln", "rms") and rotary embeddings."""
    return dict(num=4, name="gpt", B=B, loss="ce", lr=1e-3, x="ids", in_len=T, classes=vocab,
                layers=[{"kind": "embedding", "vocab": vocab, "dim": dim},
                        {"kind": "posenc", "T": T, "dim": dim},
                        {"kind": "transformer", "dim": dim, "heads": heads, "T": T, "ff": ff,
                         "causal": causal, "act": act, "norm": norm, "rope": rope},
                        {"kind": "clspool", "T": T, "dim": dim},
                        dense(dim, vocab, "logsoftmax", True)])


def lstm(B=64, T=100, inp=64, hidden=256):
    return dict(num=5, name="lstm", B=B, loss="mse", lr=1e-3, x="normal", in_len=T * inp,
                classes=None, targets="normal",
                layers=[{"kind": "lstm", "in": inp, "hidden": hidden, "T": T},
                        dense(hidden, 1, "linear")])


def gru(B=64, T=100, inp=64, hidden=256):
    """C5's shape with a GRU in the SequenceUnroller (not a BASELINE config)."""
    return dict(num=6, name="gru", B=B, loss="mse", lr=1e-3, x="normal", in_len=T * inp,
                classes=None, targets="normal",
                layers=[{"kind": "gru", "in": inp, "hidden": hidden, "T": T},
                        dense(hidden, 1, "linear")])


def cnn2(B=128):
    """C2 with a second 16 -> 16 Conv2D below the pooling (not a BASELINE
    config): the second conv's input gradient runs every step."""
    return dict(num=7, name="cnn2", B=B, loss="ce", lr=1e-3, x="normal", in_len=3 * 32 * 32,
                classes=10,
                layers=[{"kind": "conv2d", "inC": 3, "outC": 16, "k": 3, "s": 1, "p": 1, "act": "relu"},
                        {"kind": "conv2d", "inC": 16, "outC": 16, "k": 3, "s": 1, "p": 1, "act": "relu"},
                        {"kind": "maxpool2d", "k": 2, "s": 2, "p": 0, "inC": 16},
                        {"kind": "flatten", "n": 4096},
                        dense(4096, 10, "softmax", True)])


def gpt_long(B=16):
    """C4 with sequences of 256 tokens (not a BASELINE config): beyond the
    fused attention kernels' 128, so attention runs as batched GEMMs over the
    (sample, head) pairs with materialised scores."""
    cfg = gpt(B=B, T=256)
    cfg.update(num=8, name="gpt_long")
    return cfg


CONFIGS = {"mlp": mlp, "cnn": cnn, "wide": wide, "gpt": gpt, "lstm": lstm}
# further workloads bench.py times on request (--config), outside the default line
EXTRA = {"gru": gru, "cnn2": cnn2, "gpt_long": gpt_long}


def get(name):
    return (CONFIGS.get(name) or EXTRA[name])()


def inputs(cfg, B=None):
    """(x, y) float32 arrays, B x in_len and B x out_len."""
    B = B or cfg["B"]
    n = B * cfg["in_len"]
    seed_x, seed_y = 1000 + cfg["num"], 2000 + cfg["num"]
    if cfg["x"] == "uniform":
        x = fill_uniform(n, seed_x)
    elif cfg["x"] == "normal":
        x = fill_normal(n, seed_x)
    else:
        x = fill_class_ids(n, cfg["classes"], seed_x).astype(np.float32)
    x = x.reshape(B, cfg["in_len"])
    if cfg.get("targets") == "normal":
        y = fill_normal(B, seed_y).reshape(B, 1)
    else:
        ids = fill_class_ids(B, cfg["classes"], seed_y)
        y = np.zeros((B, cfg["classes"]), np.float32)
        y[np.arange(B), ids] = 1.0
    return x, y


def product_layers(cfg):
    out = []
    for d in cfg["layers"]:
        k = d["kind"]
        if k == "dense":
            act = _ACTS[d["act"]]
            out.append(Dense(d["in"], d["out"], Ref(act) if d["ptr"] else act))
        elif k == "dropout":
            out.append(Dropout(d["p"], d["n"]))
        elif k == "flatten":
            out.append(Flatten(d["n"]))
        elif k == "conv2d":
            out.append(Conv2D(d["inC"], d["outC"], d["k"], d["s"], d["p"], _ACTS[d["act"]]))
        elif k == "maxpool2d":
            out.append(MaxPool2D(d["k"], d["s"], d["p"], d["inC"]))
        elif k == "avgpool2d":
            out.append(AvgPool2D(d["k"], d["s"], d["p"], d["inC"]))
        elif k == "rmsnorm":
            out.append(RMSNorm(d["n"]))
        elif k == "layernorm":
            out.append(LayerNorm(d["n"]))
        elif k == "mha":
            out.append(MultiHeadAttention(d["heads"], d["T"], d["causal"], d["dim"]))
        elif k == "gap1d":
            out.append(GlobalAveragePooling1D(d["T"], d["dim"]))
        elif k == "batchnorm2d":
            out.append(BatchNorm2D(d["C"]))
        elif k == "moe":
            out.append(MoE(d["out"], d["E"], d["k"], d["in"]))
        elif k == "swiglu":
            out.append(SwiGLU(d["out"], d["in"]))
        elif k == "embedding":
            out.append(Embedding(d["vocab"], d["dim"]))
        elif k == "posenc":
            out.append(PositionalEncoding(d["T"], d["dim"]))
        elif k == "transformer":
            if d.get("act", "relu") == "relu" and d.get("norm", "ln") == "ln" and not d.get("rope"):
                out.append(TransformerBlock(d["dim"], d["heads"], d["T"], d["ff"], d["causal"]))
            else:
                out.append(TransformerBlockExt(d["heads"], d["T"], d["ff"], d["causal"],
                                               BLOCK_ACTS[d.get("act", "relu")],
                                               BLOCK_NORMS[d.get("norm", "ln")], d.get("rope", False),
                                               d["dim"]))
        elif k == "clspool":
            out.append(CLSPooling(d["T"], d["dim"]))
        elif k == "lstm":
            out.append(SequenceUnroller(LSTM(d["hidden"], d["in"]), d["T"], d.get("seq", False)))
        elif k == "gru":
            out.append(SequenceUnroller(GRU(d["hidden"], d["in"]), d["T"], d.get("seq", False)))
        else:
            raise ValueError(k)
    # the first layer carries the per-sample input length (an LSTM carries its
    # per-step input size and sequence length instead)
    if cfg["layers"][0]["kind"] in ("conv2d", "embedding") or out[0].desc.in_size <= 0:
        out[0].desc.in_size = cfg["in_len"]
    return out


def gpu_workers(B):
    """The worker count Network.TrainBatch gives a device of Type() == GPU:
    trainBatchParallel for B >= 64 (net.go:425-433) with at most 4 workers
    (net.go:594-604), trainBatchSequential (W = 1) below that."""
    return min(4, B) if B >= 64 else 1


def build(cfg, device=None, workers=None, max_batch=None):
    """workers=None selects gpu_workers(cfg["B"]), the reference's own
    semantics for a GPU device."""
    if workers is None:
        workers = gpu_workers(cfg["B"])
    m = NewSequential(*product_layers(cfg), device=device)
    m.Compile(Adam(cfg["lr"]), CrossEntropy if cfg["loss"] == "ce" else MSE,
              max_batch=max_batch or cfg["B"], workers=workers)
    return m
