"""Network.Save / net.Load on the device (gn_model_save_gob / gn_model_load_gob).

Save: the file must equal, byte for byte, what Go's Network.Encode
(net.go:1008-1075) writes for the same network in a process whose first gob
use it is.  The expected bytes come from goformats.network_encode, a gob
encoder restated from the gob specification and pinned by the reference's own
gob file (test_goformats.py), with ExtractLayerConfig (net.go:1426-1505) and
Adam.GobState (opt.go:312-322) restated on the test side from the layer
descriptions:

  - Conv2D records outC x oH x oW output channels and MaxPool2D C H W / k^2
    input channels once the network's own layers have run a forward pass
    (Predict, or training with one worker, trainBatchSequential); with
    several workers only clones run (net.go:588-716) and they record outC / 0;
  - Adam's moments are in the file only for networks of at most 1000
    parameters (opt.go:129-153); layers without a LayerConfig type are
    "Unknown".

Load: net.Load's checks in its order (the reference's TestLoadSecurity cases:
bad magic, version, too many layers; the 256M-parameter case needs a 1 GiB
file and is left out), a parameter count that does not match, then the layers
CreateLayer (net.go:1512-1588) builds, with value activations, and a fresh
Adam(0.001).  Files written with other type numbers (a Go process that used
gob before) load the same."""
import struct

import numpy as np
import pytest

import goformats as G
from gpuutil import log

pytestmark = pytest.mark.gpu

ACT_CODES = {"relu": 1, "sigmoid": 2, "tanh": 3, "softmax": 4, "logsoftmax": 5, "linear": 6, "gelu": 7}


def _infer_hw(n):
    h = int(np.sqrt(n))
    return (h, h) if h * h == n else (h, n // h)


def geometry(cfg):
    """Per-layer dicts for goformats.layer_config, from the config's layers
    and the per-sample input length, as the layers infer their sizes."""
    out, n = [], cfg["in_len"]
    for d in cfg["layers"]:
        k = d["kind"]
        if k == "dense":
            L = dict(kind=G.DENSE, in_size=d["in"], out_size=d["out"], act=ACT_CODES[d["act"]])
            n = d["out"]
        elif k == "dropout":
            L = dict(kind=G.DROPOUT, in_size=d["n"], prob=d["p"])
        elif k == "flatten":
            L = dict(kind=G.FLATTEN)
        elif k == "conv2d":
            H, W = _infer_hw(n // d["inC"])
            oH, oW = (H + 2 * d["p"] - d["k"]) // d["s"] + 1, (W + 2 * d["p"] - d["k"]) // d["s"] + 1
            L = dict(kind=G.CONV2D, in_channels=d["inC"], out_channels=d["outC"], k=d["k"], s=d["s"], p=d["p"],
                     act=ACT_CODES[d["act"]], oH=oH, oW=oW)
            n = d["outC"] * oH * oW
        elif k in ("maxpool2d", "avgpool2d"):
            C = d["inC"] if d["inC"] > 0 else 1
            H, W = _infer_hw(n // C)
            oH, oW = (H + 2 * d["p"] - d["k"]) // d["s"] + 1, (W + 2 * d["p"] - d["k"]) // d["s"] + 1
            L = dict(kind=G.MAXPOOL2D if k == "maxpool2d" else G.AVGPOOL2D, in_channels=d["inC"], C=C, H=H, W=W,
                     k=d["k"], s=d["s"], p=d["p"])
            n = C * oH * oW
        elif k == "batchnorm2d":
            L = dict(kind=G.BATCHNORM2D, in_channels=d["C"], eps=1e-5, affine=True)
        elif k == "embedding":
            L = dict(kind=G.EMBEDDING, vocab=d["vocab"], dim=d["dim"])
            n = n * d["dim"]
        elif k == "lstm":
            L = dict(kind=G.LSTM)
            n = d["hidden"]
        elif k == "layernorm":
            L = dict(kind=G.LAYERNORM, n=d["n"], eps=1e-5)
        elif k == "mha":
            L = dict(kind=G.MHA)
        elif k == "gap1d":
            L = dict(kind=G.GAP1D)
            n = d["dim"]
        else:
            raise ValueError(k)
        out.append(L)
    return out


def _cnn_all(B=8):
    return dict(num=51, name="gob_cnn", B=B, loss="ce", lr=2e-3, x="normal", in_len=2 * 8 * 8, classes=4,
                layers=[{"kind": "conv2d", "inC": 2, "outC": 4, "k": 3, "s": 1, "p": 1, "act": "tanh"},
                        {"kind": "batchnorm2d", "C": 4},
                        {"kind": "maxpool2d", "k": 2, "s": 2, "p": 0, "inC": 4},
                        {"kind": "avgpool2d", "k": 2, "s": 2, "p": 0, "inC": -1},
                        {"kind": "flatten", "n": 16},
                        {"kind": "dropout", "p": 0.2, "n": 16},
                        {"kind": "dense", "in": 16, "out": 4, "act": "softmax", "ptr": True}])


def _mlp_big(B=8):
    return dict(num=52, name="gob_mlp", B=B, loss="mse", lr=1e-3, x="normal", in_len=64, classes=8,
                layers=[{"kind": "dense", "in": 64, "out": 32, "act": "tanh", "ptr": False},
                        {"kind": "dense", "in": 32, "out": 8, "act": "sigmoid", "ptr": False}])


def _emb(B=8):
    return dict(num=53, name="gob_emb", B=B, loss="ce", lr=1e-3, x="ids", in_len=5, classes=6,
                layers=[{"kind": "embedding", "vocab": 6, "dim": 4},
                        {"kind": "flatten", "n": 20},
                        {"kind": "dense", "in": 20, "out": 6, "act": "linear", "ptr": False}])


def _lstm(B=4):
    return dict(num=54, name="gob_lstm", B=B, loss="mse", lr=1e-3, x="normal", in_len=3 * 2, classes=None,
                targets="normal",
                layers=[{"kind": "lstm", "in": 2, "hidden": 4, "T": 3},
                        {"kind": "dense", "in": 4, "out": 1, "act": "linear", "ptr": False}])


def _norm(B=8):
    # a Tanh output: CreateLayer rebuilds activations as values, which for
    # Softmax would predict the identity (net.go:1512-1588)
    return dict(num=55, name="gob_norm", B=B, loss="ce", lr=1e-3, x="normal", in_len=12, classes=3,
                layers=[{"kind": "dense", "in": 12, "out": 8, "act": "relu", "ptr": False},
                        {"kind": "layernorm", "n": 4, "len": 8},
                        {"kind": "dense", "in": 8, "out": 3, "act": "tanh", "ptr": False}])


def _attn(B=4):
    return dict(num=56, name="gob_attn", B=B, loss="mse", lr=1e-3, x="normal", in_len=3 * 4, classes=None,
                targets="normal",
                layers=[{"kind": "mha", "heads": 2, "T": 3, "causal": True, "dim": 4},
                        {"kind": "gap1d", "T": 3, "dim": 4},
                        {"kind": "dense", "in": 4, "out": 1, "act": "linear", "ptr": False}])


MODELS = {"cnn_all": _cnn_all, "mlp_big": _mlp_big, "emb": _emb, "lstm": _lstm, "norm": _norm,
          "attn": _attn}


def expected_file(cfg, model, dims_known, types=None):
    p = model.Params()
    m, v, t = model.AdamState()
    lp = [p[model.LayerParams(i)] for i in range(len(cfg["layers"]))]
    o = model.opt
    return G.network_encode(geometry(cfg), lp, p, "CrossEntropy" if cfg["loss"] == "ce" else "MSE",
                            (o.LearningRate, o.Beta1, o.Beta2, o.Epsilon), t, m, v, dims_known, types)


@pytest.mark.parametrize("name", sorted(MODELS))
@pytest.mark.parametrize("mode", ["fresh", "w1_trained", "w4_trained", "w4_predicted"])
def test_save_is_go_encoding(gn, tmp_path, name, mode):
    from goneuron_amd import configs
    cfg = MODELS[name]()
    workers = 1 if mode in ("fresh", "w1_trained") else 4
    model = configs.build(cfg, workers=workers)
    x, y = configs.inputs(cfg)
    if mode != "fresh":
        for _ in range(2):
            model.TrainBatch(x, y)
    if mode == "w4_predicted":
        model.Predict(x[0])
    path = tmp_path / "net.gob"
    model.Save(path)
    got = path.read_bytes()
    want = expected_file(cfg, model, dims_known=mode in ("w1_trained", "w4_predicted"))
    log(f"  {name}/{mode}: {len(got)} bytes, {model.nparams} parameters")
    if got != want:
        k = next(i for i in range(min(len(got), len(want))) if got[i] != want[i])
        raise AssertionError(f"first difference at byte {k} of {len(got)} / {len(want)}: "
                             f"{got[k:k + 16].hex()} vs {want[k:k + 16].hex()}")
    model.Close()


def _expected_descs(cfg, dims_known):
    """CreateLayer (net.go:1512-1588) of each saved config, as (kind, fields)."""
    out = []
    for L in geometry(cfg):
        c = G.layer_config(L, [], dims_known)
        t = c["Type"]
        if t == "Dense":
            out.append((G.DENSE, dict(in_size=c["InSize"], out_size=c["OutSize"], act=L["act"], act_is_ptr=0)))
        elif t == "Conv2D":
            out.append((G.CONV2D, dict(in_channels=c["InChannels"], out_channels=c["OutChannels"],
                                       kernel=c["KernelSize"], stride=c["Stride"], padding=c["Padding"])))
        elif t in ("MaxPool2D", "AvgPool2D"):
            out.append((G.MAXPOOL2D if t == "MaxPool2D" else G.AVGPOOL2D,
                        dict(in_channels=c["InChannels"], kernel=c["KernelSize"], stride=c["Stride"])))
        elif t == "BatchNorm2D":
            out.append((G.BATCHNORM2D, dict(in_channels=c["InChannels"], no_affine=0)))
        elif t == "Dropout":
            out.append((G.DROPOUT, dict(in_size=c["InSize"])))
        elif t == "Embedding":
            out.append((G.EMBEDDING, dict(vocab=c["InSize"], dim=c["OutSize"])))
        elif t == "LayerNorm":
            out.append((G.LAYERNORM, dict(dim=c["NormalizedShape"])))
        else:
            out.append((G.FLATTEN, {}))
    return out


@pytest.mark.parametrize("name", ["cnn_all", "mlp_big", "emb", "norm"])
def test_load_rebuilds_the_network(gn, tmp_path, name):
    """Saved after training with four workers (sizes unknown to the network's
    own layers), loaded back: the layers CreateLayer builds, the parameters,
    the loss, a fresh Adam(0.001); the loaded network predicts as the saved
    one (their activations are the same values) and trains."""
    from goneuron_amd import configs, Load
    cfg = MODELS[name]()
    model = configs.build(cfg, workers=4)
    x, y = configs.inputs(cfg)
    model.TrainBatch(x, y)
    path = tmp_path / "net.gob"
    model.Save(path)
    loaded, loss = Load(path, in_len=cfg["in_len"], max_batch=cfg["B"], workers=4)
    assert loss.kind == (2 if cfg["loss"] == "ce" else 1)
    assert len(loaded.layers) == len(cfg["layers"])
    for i, (kind, fields) in enumerate(_expected_descs(cfg, False)):
        d = loaded.layers[i].desc
        assert d.kind == kind, (i, d.kind, kind)
        for f, val in fields.items():
            assert getattr(d, f) == val, (i, f, getattr(d, f), val)
    np.testing.assert_array_equal(loaded.Params(), model.Params())
    m, v, t = loaded.AdamState()
    assert t == 0 and not m.any() and not v.any()
    if name != "cnn_all":  # the saved MaxPool2D config has 0 channels: the loaded one pools one plane
        np.testing.assert_array_equal(loaded.PredictBatch(x), model.PredictBatch(x))
    before = loaded.Params()
    lo = loaded.TrainBatch(x, y)
    assert np.isfinite(lo) and not np.array_equal(loaded.Params(), before)
    # a fresh model of the same layers, Adam(0.001) and parameters takes the same step
    ref = gn.NewSequential(*loaded.layers)
    ref.Compile(gn.Adam(0.001), loss, max_batch=cfg["B"], workers=4)
    ref.SetParams(before)
    assert ref.TrainBatch(x, y) == lo
    np.testing.assert_array_equal(ref.Params(), loaded.Params())
    for mm in (model, loaded, ref):
        mm.Close()


def _gob_file(configs_, params, loss="MSE", opt="Adam", nlayers=None, types=None):
    e = G.Encoder(types or G.Types())
    e.encode("int", len(configs_) if nlayers is None else nlayers)
    e.encode("string", loss)
    e.encode("string", opt)
    for c in configs_:
        e.encode(G.LAYER_CONFIG, c)
    e.encode(G.F32S, list(map(float, params)))
    return b"GONN" + struct.pack("<i", 1) + bytes(e.out)


def _dense_cfg(i, o, act="Tanh", params=None):
    n = i * o + o
    p = list(np.linspace(-0.5, 0.5, n).astype(np.float32)) if params is None else params
    return {"Type": "Dense", "InSize": i, "OutSize": o, "Activation": act, "Params": [float(v) for v in p]}


def test_load_errors(gn, tmp_path):
    from goneuron_amd import configs, Load, GNError
    cases = {}
    good = _gob_file([_dense_cfg(3, 2)], np.linspace(-0.5, 0.5, 8).astype(np.float32))
    cases["bad_magic"] = (b"BAD!" + good[4:], -1, "invalid magic number")
    cases["version"] = (good[:4] + struct.pack("<i", 999) + good[8:], -1, "unsupported version")
    e = G.Encoder(G.Types())
    e.encode("int", 2000)
    cases["too_many_layers"] = (b"GONN" + struct.pack("<i", 1) + bytes(e.out), -1, "invalid number of layers")
    cases["count_mismatch"] = (_gob_file([_dense_cfg(3, 2)], [0.5, 1.0]), -1, "parameter count mismatch")
    cases["truncated"] = (good[:len(good) - 5], -1, "failed to read parameters")
    cases["unknown_type"] = (_gob_file([{"Type": "Unknown", "InSize": -1, "OutSize": -1, "Params": [1.0]}], [1.0]),
                             -4, "unsupported layer type: Unknown")
    cases["huber"] = (_gob_file([_dense_cfg(3, 2)], _dense_cfg(3, 2)["Params"], loss="Huber"), -4, "Huber")
    cases["sgd"] = (_gob_file([_dense_cfg(3, 2)], _dense_cfg(3, 2)["Params"], opt="SGD"), -4, "SGD")
    cases["leaky"] = (_gob_file([_dense_cfg(3, 2, "LeakyReLU")], _dense_cfg(3, 2)["Params"]), -4, "LeakyReLU")
    # Conv2D saved after a forward pass: OutChannels = outC x oH x oW
    cfg = _cnn_all()
    model = configs.build(cfg, workers=1)
    x, y = configs.inputs(cfg)
    model.TrainBatch(x, y)
    model.Save(tmp_path / "dims.gob")
    cases["conv_dims_known"] = ((tmp_path / "dims.gob").read_bytes(), -4, "parameters")
    model.Close()
    cfg = _lstm()
    model = configs.build(cfg)
    model.Save(tmp_path / "lstm.gob")
    cases["lstm_unknown"] = ((tmp_path / "lstm.gob").read_bytes(), -4, "unsupported layer type: Unknown")
    model.Close()
    for name, (buf, code, text) in cases.items():
        path = tmp_path / f"{name}.gob"
        path.write_bytes(buf)
        with pytest.raises(GNError) as ei:
            Load(path, max_batch=4)
        log(f"  {name}: {ei.value}")
        assert ei.value.code == code and text in str(ei.value), (name, str(ei.value))
    # the good file loads; an unknown loss name is MSE (net.go:966-976)
    (tmp_path / "good.gob").write_bytes(_gob_file([_dense_cfg(3, 2)], _dense_cfg(3, 2)["Params"], loss="L1"))
    m, loss = Load(tmp_path / "good.gob", max_batch=4)
    assert loss.kind == 1 and m.layers[0].desc.act == 3
    m.Close()


def test_load_other_type_numbers(gn, tmp_path):
    """A file from a Go process that used gob before numbers its types from
    70: the definitions in the file are what counts."""
    from goneuron_amd import configs, Load
    cfg = _mlp_big()
    model = configs.build(cfg, workers=4)
    x, y = configs.inputs(cfg)
    model.TrainBatch(x, y)
    buf = expected_file(cfg, model, False, types=G.Types(first=70))
    assert buf != expected_file(cfg, model, False)
    (tmp_path / "t70.gob").write_bytes(buf)
    loaded, _ = Load(tmp_path / "t70.gob", max_batch=cfg["B"])
    np.testing.assert_array_equal(loaded.Params(), model.Params())
    np.testing.assert_array_equal(loaded.PredictBatch(x), model.PredictBatch(x))
    loaded.Close()
    model.Close()
