"""The test-side format restatements (goformats.py) pinned before they are used
to check the library's writers:

  - gob: the one gob file the reference holds (a Go process's []float32 of
    15103 parameters, examples/portuguese_gpt/main.go:332-339) decodes and
    re-encodes to the same 88723 bytes; the gob package documentation's worked
    example (Point{22, 33}) encodes to the bytes the documentation lists;
  - Float32ToFloat16 (gguf.go:178-210): truncation onto the half-precision
    grid, checked against the largest half value not above |x| found by
    search over all finite halves;
  - Network.Encode: the definitions come in the order gob numbers them
    (LayerConfig 64, []float32 65, adamGobState 66, [][]float32 67) and a
    second, independent decode returns every field.
"""
import os
import struct

import numpy as np

import goformats as G

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "gob", "portuguese_gpt_params.gob")


def test_gob_fixture_decodes_and_reencodes_byte_for_byte():
    buf = open(FIXTURE, "rb").read()
    d = G.Decoder(buf)
    tid, v = d.value()
    assert d.value() is None
    assert d.defs == [(64, ("slice", 4, ""))]  # []float32 met at top level: no name
    assert tid == 64 and v.shape == (15103,)
    assert np.isfinite(v).all() and 0.001 < np.abs(v).mean() < 1.0
    assert (v.astype(np.float32).astype(np.float64) == v).all()  # float32 values widened
    e = G.Encoder(G.Types())
    e.encode(G.F32S, [float(x) for x in v])  # name "" at top level
    assert bytes(e.out) == buf


def test_gob_documentation_point_example():
    """encoding/gob package documentation: `type Point struct {X, Y int}`,
    Encode(Point{22, 33}) in a program where Point is type 65."""
    want = bytes.fromhex("1fff810301010550 6f696e7401ff8200 0102010158010400 0101590104000000"
                         "07ff82012c014200".replace(" ", ""))
    e = G.Encoder(G.Types(first=65))
    e.encode(("struct", "Point", [("X", "int"), ("Y", "int")]), {"X": 22, "Y": 33})
    assert bytes(e.out) == want
    d = G.Decoder(want)
    assert d.value() == (65, {"X": 22, "Y": 33})


def test_gob_primitives():
    assert G.enc_uint(0) == b"\x00" and G.enc_uint(127) == b"\x7f"
    assert G.enc_uint(128) == b"\xff\x80" and G.enc_uint(256) == b"\xfe\x01\x00"
    assert [G.enc_int(i) for i in (0, -1, 1, -64, 64)] == [0, 1, 2, 127, 128]
    assert G.enc_uint(G.float_bits(1.0)) == b"\xfe\xf0\x3f"  # 0x3ff0000000000000 reversed
    assert G.enc_uint(G.float_bits(0.0)) == b"\x00"


def _largest_half_not_above(a):
    grid = np.arange(0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)  # finite, >= 0
    idx = np.searchsorted(grid, a, side="right") - 1
    return np.arange(0x7C00, dtype=np.uint16)[idx]


def test_f32_to_f16_truncates_onto_the_half_grid():
    rng = np.random.default_rng(7)
    mags = np.concatenate([
        np.exp(rng.uniform(np.log(1e-9), np.log(65535.0), 4000)),   # subnormal to max half range
        [0.0, 2.0 ** -25, 2.0 ** -24, 1.5 * 2 ** -24, 2.0 ** -14, 65504.0, 65519.0, 65535.9, 1.0, 1 - 2 ** -24],
    ]).astype(np.float32)
    for sign in (1.0, -1.0):
        x = (mags * sign).astype(np.float32)
        got = np.array([G.f32_to_f16(v) for v in x], np.uint16)
        want = _largest_half_not_above(np.abs(x).astype(np.float64))
        if sign < 0:
            want = want | 0x8000
        np.testing.assert_array_equal(got, want)
    # beyond the half range, infinities and NaN
    assert G.f32_to_f16(np.float32(65536.0)) == 0x7C00 and G.f32_to_f16(np.float32(-1e30)) == 0xFC00
    assert G.f32_to_f16(np.float32(np.inf)) == 0x7C00
    h = G.f32_to_f16(np.float32(np.nan))
    assert h & 0x7C00 == 0x7C00 and h & 1 and h & 0x3FF
    assert G.f32_to_f16(np.float32(1e-40)) == 0  # float32 subnormal


def _small_net():
    layers = [dict(kind=G.DENSE, in_size=4, out_size=3, act=1),
              dict(kind=G.DROPOUT, in_size=3, prob=0.25),
              dict(kind=G.LSTM)]
    lp = [np.arange(15, dtype=np.float32) / 7, np.zeros(0, np.float32), np.array([0.5, -2.0], np.float32)]
    return layers, lp


def test_network_encode_definitions_and_values():
    layers, lp = _small_net()
    flat = np.concatenate(lp)
    m = np.linspace(-1, 1, flat.size).astype(np.float32)
    buf = G.network_encode(layers, lp, flat, "CrossEntropy", (1e-3, 0.9, 0.999, 1e-8), 3, m, m * m, False)
    assert buf[:4] == b"GONN" and struct.unpack_from("<i", buf, 4)[0] == 1
    d = G.Decoder(buf, 8)
    vals = []
    while (nv := d.value()) is not None:
        vals.append(nv)
    assert [i for i, _ in d.defs] == [64, 65, 66, 67]
    assert d.defs[1][1] == ("slice", 4, "[]float32") and d.defs[3][1] == ("slice", 65, "[][]float32")
    assert d.defs[0][1][1] == "LayerConfig" and [f for f, _ in d.defs[0][1][2]][:4] == [
        "Type", "InSize", "OutSize", "Params"]
    assert vals[0] == (2, 3) and vals[1] == (6, "CrossEntropy") and vals[2] == (6, "Adam")
    c0, c1, c2 = (v for _, v in vals[3:6])
    assert c0["Type"] == "Dense" and c0["InSize"] == 4 and c0["OutSize"] == 3 and c0["Activation"] == "ReLU"
    np.testing.assert_array_equal(c0["Params"], lp[0])
    assert c1 == {"Type": "Dropout", "InSize": 3, "OutSize": -1, "Prob": 0.25}
    assert c2["Type"] == "Unknown" and c2["InSize"] == -1 and list(c2["Params"]) == [0.5, -2.0]
    np.testing.assert_array_equal(vals[6][1], flat)
    st = vals[7][1]
    assert st["Timestep"] == 3 and abs(st["LearningRate"] - 1e-3) < 1e-10 and len(st["Momentum1"]) == 1
    np.testing.assert_array_equal(st["Momentum1"][0], m)
