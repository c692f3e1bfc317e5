"""Checkpoint formats around the device-resident arena: SaveBinaryWeights and
its reader, GGUF v3 (F32 / F16) and the resume state file.  The files are
parsed here by readers written from the formats (net.go:1119-1392, gguf.go),
not by the library."""
import os
import struct

import numpy as np
import pytest

import goformats

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gn():
    import goneuron_amd as gn
    gn.GetDefaultDevice()
    return gn


def _cnn_bn():
    return dict(num=21, name="ckpt_cnn", B=12, loss="ce", lr=1e-3, x="normal", in_len=2 * 8 * 8, classes=4,
                layers=[{"kind": "conv2d", "inC": 2, "outC": 3, "k": 3, "s": 1, "p": 1, "act": "relu"},
                        {"kind": "batchnorm2d", "C": 3},
                        {"kind": "maxpool2d", "k": 2, "s": 2, "p": 0, "inC": 3},
                        {"kind": "flatten", "n": 48},
                        {"kind": "dense", "in": 48, "out": 4, "act": "softmax", "ptr": True}])


def _read_gonn(path):
    with open(path, "rb") as f:
        buf = f.read()
    assert buf[:4] == b"GONN"
    ver, count = struct.unpack_from("<ii", buf, 4)
    pos, out = 12, []
    for _ in range(count):
        (nl,) = struct.unpack_from("<i", buf, pos)
        name = buf[pos + 4:pos + 4 + nl].decode()
        pos += 4 + nl
        (rank,) = struct.unpack_from("<i", buf, pos)
        shape = struct.unpack_from("<%di" % rank, buf, pos + 4)
        pos += 4 + 4 * rank
        (n,) = struct.unpack_from("<i", buf, pos)
        data = np.frombuffer(buf, "<f4", n, pos + 4)
        pos += 4 + 4 * n
        out.append((name, tuple(shape), data))
    assert pos == len(buf)
    return ver, out


def test_binary_weights_layout_and_round_trip(gn, tmp_path):
    """SaveBinaryWeights (net.go:1119-1214): names layer_<i>_<type>_<param>
    from ExtractLayerConfig and NamedParams (BatchNorm2D's running statistics
    included), shapes, data; loading it into a fresh model restores the
    parameters and running statistics exactly; a model of another shape
    rejects the file."""
    from goneuron_amd import configs, GNError
    cfg = _cnn_bn()
    x, y = configs.inputs(cfg)
    model = configs.build(cfg)
    model.TrainBatch(x, y)
    path = str(tmp_path / "w.gonn")
    model.SaveBinaryWeights(path)
    ver, ts = _read_gonn(path)
    assert ver == 1
    # byte for byte what net.go:1119-1214 writes for these tensors
    assert open(path, "rb").read() == goformats.binary_weights([(n, s, d) for n, s, d in ts])
    assert [(n, s) for n, s, _ in ts] == [
        ("layer_0_Conv2D_weights", (3, 2, 3, 3)), ("layer_0_Conv2D_biases", (3,)),
        ("layer_1_BatchNorm2D_running_mean", (3,)), ("layer_1_BatchNorm2D_running_var", (3,)),
        ("layer_1_BatchNorm2D_gamma", (3,)), ("layer_1_BatchNorm2D_beta", (3,)),
        ("layer_4_Dense_weights", (4, 48)), ("layer_4_Dense_biases", (4,))]
    p = model.Params()
    rm, rv = model.RunningStats(1)
    flat = np.concatenate([d for n, _, d in ts if "running" not in n])
    np.testing.assert_array_equal(flat, p)
    np.testing.assert_array_equal(ts[2][2], rm)
    np.testing.assert_array_equal(ts[3][2], rv)
    assert not np.array_equal(rm, np.zeros(3))  # one training step moved them
    fresh = configs.build(cfg)
    fresh.SetParams(np.zeros_like(p))
    fresh.LoadBinaryWeights(path)
    np.testing.assert_array_equal(fresh.Params(), p)
    m2, v2 = fresh.RunningStats(1)
    np.testing.assert_array_equal(m2, rm)
    np.testing.assert_array_equal(v2, rv)
    other = dict(cfg, layers=cfg["layers"][:4] + [
        {"kind": "dense", "in": 48, "out": 5, "act": "softmax", "ptr": True}], classes=5)
    with pytest.raises(GNError):
        configs.build(other).LoadBinaryWeights(path)


def _read_gguf(path):
    with open(path, "rb") as f:
        buf = f.read()
    magic, ver, nt, nkv = struct.unpack_from("<IIQQ", buf, 0)
    assert magic == 0x46554747 and ver == 3
    pos = 24

    def s():
        nonlocal pos
        (n,) = struct.unpack_from("<Q", buf, pos)
        v = buf[pos + 8:pos + 8 + n].decode()
        pos += 8 + n
        return v
    kv = {}
    for _ in range(nkv):
        k = s()
        (t,) = struct.unpack_from("<I", buf, pos)
        pos += 4
        if t == 8:
            kv[k] = s()
        else:
            assert t == 4
            (kv[k],) = struct.unpack_from("<I", buf, pos)
            pos += 4
    infos = []
    for _ in range(nt):
        name = s()
        (rank,) = struct.unpack_from("<I", buf, pos)
        dims = struct.unpack_from("<%dQ" % rank, buf, pos + 4)
        pos += 4 + 8 * rank
        typ, off = struct.unpack_from("<IQ", buf, pos)
        pos += 12
        infos.append((name, tuple(reversed(dims)), typ, off))
    start = (pos + 31) // 32 * 32
    out = []
    for name, shape, typ, off in infos:
        assert off % 32 == 0
        n = int(np.prod(shape))
        data = np.frombuffer(buf, "<f4" if typ == 0 else "<f2", n, start + off)
        out.append((name, shape, typ, data))
    return kv, out


@pytest.mark.parametrize("f16", [0, 1])
def test_gguf_export(gn, tmp_path, f16):
    """SaveGGUFExt (net.go:1222-1392): GGUF v3 header, the five metadata
    keys, tensor names blk.<i>.<mapped name> with dims last-first and 32-byte
    aligned offsets, for a TransformerBlockExt GPT (SwiGLU, RMSNorm, RoPE);
    F32 data equal to the parameters; F16 data is Float32ToFloat16's
    truncation: never larger in magnitude and within one half-precision step."""
    from goneuron_amd import configs
    cfg = configs.gpt(B=2, T=8, vocab=13, dim=16, heads=2, ff=24, act="swiglu", norm="rms", rope=True)
    model = configs.build(cfg)
    rng = np.random.default_rng(3)
    p = (rng.normal(size=model.nparams) * 0.3).astype(np.float32)
    model.SetParams(p)
    path = str(tmp_path / "m.gguf")
    model.SaveGGUFExt(path, f16)
    kv, ts = _read_gguf(path)
    assert kv == {"general.architecture": "goneuron", "general.name": "GoNeuron Model",
                  "general.alignment": 32, "goneuron.layer_count": 5,
                  "goneuron.loss_type": "loss.CrossEntropy"}
    names = [n for n, _, _, _ in ts]
    assert names[:2] == ["blk.0.weight", "blk.1.weight"]
    assert names[2:8] == ["blk.2.attn_q.weight", "blk.2.attn_q.bias", "blk.2.attn_k.weight",
                          "blk.2.attn_k.bias", "blk.2.attn_v.weight", "blk.2.attn_v.bias"]
    assert names[8:] == ["blk.2.attn_output.weight", "blk.2.attn_output.bias", "blk.2.attn_norm.weight",
                         "blk.2.ffn_norm.weight", "blk.2.ffn_up.w", "blk.2.ffn_up.v",
                         "blk.2.ffn_down.weight", "blk.2.ffn_down.bias", "blk.4.weight", "blk.4.bias"]
    assert ts[0][1] == (13, 16) and ts[1][1] == (8, 16) and ts[12][1] == (24, 16)
    assert ts[14][1] == (16, 24)
    assert all(t == f16 for _, _, t, _ in ts)
    # byte for byte what net.go:1222-1392 writes: the same tensors as
    # NamedParams (consecutive slices of the parameters, names before the
    # GGUF mapping), header, metadata, 32-byte alignment, F16 truncation
    named = [[("weights", (13, 16))], [("weights", (8, 16))],
             [(f"mha_{w}_{b}", (16, 16) if b == "weights" else (16,)) for w in ("wQ", "wK", "wV", "wOut")
              for b in ("weights", "biases")] +
             [("norm1_gamma", (16,)), ("norm2_gamma", (16,)), ("ff1_w", (24, 16)), ("ff1_v", (24, 16)),
              ("ff2_weights", (16, 24)), ("ff2_biases", (16,))],
             ("flat", p[:0]), [("weights", (13, 16)), ("biases", (13,))]]
    off, layer_tensors = 0, []
    for lt in named:
        if isinstance(lt, tuple):
            layer_tensors.append(lt)
            continue
        cur = []
        for n, shape in lt:
            k = int(np.prod(shape))
            cur.append((n, shape, p[off:off + k]))
            off += k
        layer_tensors.append(cur)
    assert off == p.size
    want = goformats.gguf(layer_tensors, 5, "loss.CrossEntropy", f16)
    assert open(path, "rb").read() == want
    got = np.concatenate([d.astype(np.float32) for _, _, _, d in ts])
    if not f16:
        np.testing.assert_array_equal(got, p)
    else:
        big = np.abs(p) >= 6.2e-5  # normal half range
        assert (np.abs(got) <= np.abs(p)).all()
        step = 2.0 ** (np.floor(np.log2(np.abs(p[big]))) - 10)
        assert (np.abs(p[big] - got[big]) < step).all()
        assert (np.sign(got[big]) == np.sign(p[big])).all()


def test_resume_state_continues_bit_exactly(gn, tmp_path):
    """SaveState / LoadState: parameters, Adam moments and timestep,
    BatchNorm2D running statistics and MoE noise streams; a model restored
    from the file and trained one more step matches the original run
    bit for bit."""
    from goneuron_amd import configs
    cfg = dict(num=22, name="ckpt_moe", B=16, loss="ce", lr=1e-3, x="normal", in_len=12, classes=3,
               layers=[{"kind": "dense", "in": 12, "out": 16, "act": "relu", "ptr": False},
                       {"kind": "moe", "in": 16, "out": 10, "E": 4, "k": 2},
                       {"kind": "dense", "in": 10, "out": 3, "act": "softmax", "ptr": True}])
    for c in (cfg, _cnn_bn()):
        x, y = configs.inputs(c)
        a = configs.build(c)
        a.TrainBatch(x, y)
        a.TrainBatch(x, y)
        path = str(tmp_path / ("s_" + c["name"]))
        a.SaveState(path)
        a.TrainBatch(x, y)
        b = configs.build(c)
        b.LoadState(path)
        b.TrainBatch(x, y)
        np.testing.assert_array_equal(b.Params(), a.Params())
        ma, va, ta = a.AdamState()
        mb, vb, tb = b.AdamState()
        assert ta == tb == 3
        np.testing.assert_array_equal(mb, ma)
        np.testing.assert_array_equal(vb, va)
    assert os.path.getsize(path) > 0
