"""Test-side restatements of the reference's file formats, written from their
specifications, to check the library's writers byte for byte:

  - encoding/gob (the Go standard library; its package documentation is the
    spec): a generic encoder over Go type descriptions with gob's per-process
    type numbering and per-encoder definition sending, and a generic decoder
    driven by the definitions it reads;
  - Network.Encode (net.go:1008-1075) on top of it, with ExtractLayerConfig
    (net.go:1425-1505) and Adam.GobState (opt.go:312-322);
  - SaveBinaryWeights (net.go:1119-1214) and SaveGGUFExt (net.go:1222-1392,
    gguf.go:79-210).

Type descriptions: "bool", "int", "uint", "float", "string", ("slice", elem,
go_name), ("struct", name, [(field, type), ...]).  go_name is what Go's
reflect gives the slice type where it is first met: its String() as a struct
field ("[]float32"), its Name() ("") at top level or as a slice element.
"""
from __future__ import annotations

import struct

import numpy as np

BASIC = {"bool": 1, "int": 2, "uint": 3, "float": 4, "bytes": 5, "string": 6}

# gob's own description types (type ids 16-23), used to send definitions
COMMON = ("struct", "CommonType", [("Name", "string"), ("Id", "int")])
FIELD = ("struct", "fieldType", [("Name", "string"), ("Id", "int")])
SLICE_T = ("struct", "sliceType", [("CommonType", COMMON), ("Elem", "int")])
STRUCT_T = ("struct", "structType", [("CommonType", COMMON), ("Field", ("slice", FIELD, ""))])
WIRE = ("struct", "wireType", [("ArrayT", "ptr"), ("SliceT", SLICE_T), ("StructT", STRUCT_T)])


# ---------------------------------------------------------------- primitives
def enc_uint(x: int) -> bytes:
    if x < 128:
        return bytes([x])
    b = x.to_bytes(8, "big").lstrip(b"\0")
    return bytes([256 - len(b)]) + b


def enc_int(i: int) -> int:
    return ((~i) << 1) | 1 if i < 0 else i << 1


def float_bits(f: float) -> int:
    """float64 bits with their bytes reversed (gob sends floats that way)."""
    return int.from_bytes(struct.pack("<d", float(f)), "big")


class Types:
    """The process-wide type table: ids from 64 in the order types are first
    met, a struct before its fields' types, a slice after its element."""

    def __init__(self, first=64):
        self.next = first
        self.ids = {}     # key -> id
        self.names = {}   # key -> name recorded when first met

    @staticmethod
    def key(t):
        if isinstance(t, str):
            return t
        if t[0] == "slice":
            return ("slice", Types.key(t[1]))
        return ("struct", t[1])

    def id(self, t, name=""):
        if isinstance(t, str):
            return BASIC[t]
        k = self.key(t)
        if k in self.ids:
            return self.ids[k]
        if t[0] == "struct":
            self.ids[k] = self.next
            self.names[k] = t[1]
            self.next += 1
            for _, ft in t[2]:
                fname = ft[2] if not isinstance(ft, str) and ft[0] == "slice" else ""
                self.id(ft, fname)
            return self.ids[k]
        self.id(t[1], "")           # the element first (reflect Name() of it)
        self.ids[k] = self.next
        self.names[k] = name
        self.next += 1
        return self.ids[k]


class Encoder:
    """gob.NewEncoder: each Encode sends the definitions this encoder has not
    sent yet (a struct's before its fields' types), then the value message."""

    def __init__(self, types: Types):
        self.types = types
        self.sent = set()
        self.out = bytearray()

    # -- values
    def _value(self, t, v, top=False) -> bytes:
        if t == "int":
            return enc_uint(enc_int(int(v)))
        if t == "uint":
            return enc_uint(int(v))
        if t == "bool":
            return enc_uint(1 if v else 0)
        if t == "float":
            return enc_uint(float_bits(v))
        if t == "string":
            b = v.encode()
            return enc_uint(len(b)) + b
        if t[0] == "slice":
            return enc_uint(len(v)) + b"".join(self._value(t[1], e) for e in v)
        return self._struct(t, v)

    @staticmethod
    def _zero(t, v):
        if v is None:
            return True
        if isinstance(t, str):
            return v == 0 or v == "" or v is False
        if t[0] == "slice":
            return len(v) == 0
        return False  # struct-valued fields are always sent

    def _struct(self, t, v) -> bytes:
        out, last = bytearray(), -1
        for k, (name, ft) in enumerate(t[2]):
            val = v.get(name)
            if ft == "ptr" or self._zero(ft, val):
                continue
            out += enc_uint(k - last)
            last = k
            out += self._value(ft, val)
        out += b"\0"
        return bytes(out)

    # -- definitions
    def _send_type(self, t, name=""):
        if isinstance(t, str):
            return
        tid = self.types.id(t, name)
        if tid in self.sent:
            return
        k = Types.key(t)
        common = {"Name": self.types.names[k], "Id": tid}
        if t[0] == "struct":
            wire = {"StructT": {"CommonType": common,
                                "Field": [{"Name": f, "Id": self.types.id(ft, ft[2] if not isinstance(ft, str)
                                                                          and ft[0] == "slice" else "")}
                                          for f, ft in t[2]]}}
        else:
            wire = {"SliceT": {"CommonType": common, "Elem": self.types.id(t[1])}}
        self._message(enc_uint(enc_int(-tid)) + self._struct(WIRE, wire))
        self.sent.add(tid)
        if t[0] == "struct":
            for _, ft in t[2]:
                self._send_type(ft, ft[2] if not isinstance(ft, str) and ft[0] == "slice" else "")
        else:
            self._send_type(t[1])

    def _message(self, m: bytes):
        self.out += enc_uint(len(m)) + m

    def encode(self, t, v, name=""):
        self._send_type(t, name)
        tid = self.types.id(t, name)
        if isinstance(t, str) or t[0] != "struct":
            self._message(enc_uint(enc_int(tid)) + b"\0" + self._value(t, v))
        else:
            self._message(enc_uint(enc_int(tid)) + self._struct(t, v))


# ---------------------------------------------------------------- decoding
class Reader:
    def __init__(self, buf, pos=0, end=None):
        self.b, self.p, self.e = buf, pos, len(buf) if end is None else end

    def uint(self):
        c = self.b[self.p]
        self.p += 1
        if c < 128:
            return c
        n = 256 - c
        assert n <= 8 and self.p + n <= self.e, "bad uint"
        v = int.from_bytes(self.b[self.p:self.p + n], "big")
        self.p += n
        return v

    def int(self):
        x = self.uint()
        return ~(x >> 1) if x & 1 else x >> 1

    def float(self):
        return struct.unpack("<d", self.uint().to_bytes(8, "big"))[0]

    def bytes(self):
        n = self.uint()
        v = bytes(self.b[self.p:self.p + n])
        self.p += n
        return v


class Decoder:
    """Reads a gob stream: definitions are recorded as they come, values are
    decoded by their wire type.  Structs decode to dicts by field name, []float
    to float64 numpy arrays."""

    def __init__(self, buf, pos=0):
        self.r = Reader(buf, pos)
        self.wire = {}  # id -> ("slice", elem, name) | ("struct", name, [(field, id)])
        self.defs = []  # (id, definition) in stream order

    def _struct_fields(self, m, handlers):
        f = -1
        while True:
            d = m.uint()
            if d == 0:
                return
            f += d
            handlers(f)

    def _common(self, m):
        out = {"Name": "", "Id": 0}

        def h(f):
            if f == 0:
                out["Name"] = m.bytes().decode()
            elif f == 1:
                out["Id"] = m.int()
            else:
                raise ValueError("CommonType field")
        self._struct_fields(m, h)
        return out

    def _definition(self, m):
        res = {}

        def outer(f):
            kind = {1: "slice", 2: "struct"}.get(f)
            if kind is None:
                raise ValueError(f"wireType field {f} not handled")
            res["kind"] = kind
            res["fields"] = []

            def inner(g):
                if g == 0:
                    res.update(self._common(m))
                elif kind == "slice" and g == 1:
                    res["elem"] = m.int()
                elif kind == "struct" and g == 1:
                    for _ in range(m.uint()):
                        fl = {"Name": "", "Id": 0}

                        def fh(h):
                            if h == 0:
                                fl["Name"] = m.bytes().decode()
                            else:
                                fl["Id"] = m.int()
                        self._struct_fields(m, fh)
                        res["fields"].append((fl["Name"], fl["Id"]))
                else:
                    raise ValueError("definition field")
            self._struct_fields(m, inner)
        self._struct_fields(m, outer)
        if res["kind"] == "slice":
            return ("slice", res["elem"], res["Name"]), res["Id"]
        return ("struct", res["Name"], res["fields"]), res["Id"]

    def _value(self, m, tid):
        if tid == 1:
            return m.uint() != 0
        if tid == 2:
            return m.int()
        if tid == 3:
            return m.uint()
        if tid == 4:
            return m.float()
        if tid in (5, 6):
            v = m.bytes()
            return v.decode() if tid == 6 else v
        w = self.wire[tid]
        if w[0] == "slice":
            n = m.uint()
            if w[1] == 4:
                return np.array([m.float() for _ in range(n)], np.float64)
            return [self._value(m, w[1]) for _ in range(n)]
        out, f = {}, -1
        while True:
            d = m.uint()
            if d == 0:
                return out
            f += d
            name, ftid = w[2][f]
            out[name] = self._value(m, ftid)

    def value(self):
        """(type id, value) of the next value; None at the end."""
        while self.r.p < self.r.e:
            n = self.r.uint()
            m = Reader(self.r.b, self.r.p, self.r.p + n)
            self.r.p += n
            tid = m.int()
            if tid < 0:
                d, did = self._definition(m)
                assert did == -tid, (did, tid)
                self.wire[did] = d
                self.defs.append((did, d))
                continue
            if self.wire.get(tid, ("",))[0] != "struct":
                assert m.uint() == 0, "singleton delta"
            v = self._value(m, tid)
            assert m.p == m.e, "message not consumed"
            return tid, v
        return None


# ---------------------------------------------------------------- Network.Encode
F32S = ("slice", "float", "[]float32")
LAYER_CONFIG = ("struct", "LayerConfig", [
    ("Type", "string"), ("InSize", "int"), ("OutSize", "int"), ("Params", F32S), ("Activation", "string"),
    ("Alpha", "float"), ("KernelSize", "int"), ("Stride", "int"), ("Padding", "int"), ("InChannels", "int"),
    ("OutChannels", "int"), ("Prob", "float"), ("Eps", "float"), ("Affine", "bool"),
    ("NormalizedShape", "int"), ("NumCenters", "int"), ("Gamma", "float")])
ADAM_STATE = ("struct", "adamGobState", [
    ("LearningRate", "float"), ("Beta1", "float"), ("Beta2", "float"), ("Epsilon", "float"),
    ("Momentum1", ("slice", F32S, "[][]float32")), ("Momentum2", ("slice", F32S, "[][]float32")),
    ("Timestep", "int")])

# kind codes of goneuron_hip.h
DENSE, DROPOUT, CONV2D, MAXPOOL2D, FLATTEN, EMBEDDING, POSENC, TRANSFORMER, CLSPOOL, LSTM, AVGPOOL2D, \
    RMSNORM, SWIGLU, BATCHNORM2D, GRU, MOE, MHA, LAYERNORM, GAP1D = range(1, 20)
ACT_NAMES = {2: "Sigmoid", 3: "Tanh", 4: "Softmax", 5: "LogSoftmax", 6: "Linear", 7: "GELU"}
TYPE_NAMES = {DENSE: "Dense", CONV2D: "Conv2D", DROPOUT: "Dropout", MAXPOOL2D: "MaxPool2D",
              AVGPOOL2D: "AvgPool2D", EMBEDDING: "Embedding", FLATTEN: "Flatten", BATCHNORM2D: "BatchNorm2D",
              LAYERNORM: "LayerNorm"}


def f32(x):
    return float(np.float32(x))


def layer_config(L, params, dims_known):
    """ExtractLayerConfig (net.go:1426-1505) of one layer.  L: dict with the
    layer's kind and geometry (in_size, out_size, act, in_channels,
    out_channels, k, s, p, prob, eps, affine, vocab, dim, H, W, oH, oW, C)."""
    cfg = {"Type": TYPE_NAMES.get(L["kind"], "Unknown"), "InSize": -1, "OutSize": -1, "Params": params}
    k = L["kind"]
    if k == DENSE:
        cfg.update(InSize=L["in_size"], OutSize=L["out_size"], Activation=ACT_NAMES.get(L["act"], "ReLU"))
    elif k == CONV2D:
        out = L["out_channels"] * L["oH"] * L["oW"] if dims_known else L["out_channels"]
        cfg.update(InChannels=L["in_channels"], OutChannels=out, KernelSize=L["k"], Stride=L["s"],
                   Padding=L["p"], Activation=ACT_NAMES.get(L["act"], "ReLU"))
    elif k == DROPOUT:
        cfg.update(Prob=f32(L["prob"]), InSize=L["in_size"])
    elif k == BATCHNORM2D:
        cfg.update(InChannels=L["in_channels"], Eps=f32(L["eps"]), Affine=L["affine"])
    elif k == MAXPOOL2D:
        insize = L["C"] * L["H"] * L["W"] if dims_known else 0
        cfg.update(InChannels=insize // (L["k"] * L["k"]), KernelSize=L["k"], Stride=L["s"], Padding=L["p"])
    elif k == AVGPOOL2D:
        ch = 1 if dims_known and L["in_channels"] <= 0 else L["in_channels"]
        cfg.update(InChannels=ch, KernelSize=L["k"], Stride=L["s"], Padding=L["p"])
    elif k == EMBEDDING:
        cfg.update(InSize=L["vocab"], OutSize=L["dim"])
    elif k == LAYERNORM:  # net.go:1469-1473
        cfg.update(NormalizedShape=L["n"], Eps=f32(L["eps"]), Affine=True)
    return cfg


def network_encode(layers, layer_params, params, loss, adam, timestep, m, v, dims_known, types=None):
    """Network.Encode (net.go:1008-1075) -> bytes.  adam = (lr, beta1, beta2,
    eps); m / v the flat Adam moments."""
    types = types or Types()
    e = Encoder(types)
    e.encode("int", len(layers))
    e.encode("string", loss)
    e.encode("string", "Adam")
    for L, p in zip(layers, layer_params):
        e.encode(LAYER_CONFIG, layer_config(L, [f32(x) for x in p], dims_known))
    e.encode(F32S, [f32(x) for x in params])
    st = {"LearningRate": f32(adam[0]), "Beta1": f32(adam[1]), "Beta2": f32(adam[2]), "Epsilon": f32(adam[3]),
          "Timestep": timestep}
    n = len(params)
    if timestep > 0 and n <= 1000:  # opt.go:129-153: one moment slice for the flat buffer
        if n:
            st["Momentum1"], st["Momentum2"] = [list(map(f32, m))], [list(map(f32, v))]
        else:
            st["Momentum1"] = st["Momentum2"] = [[] for _ in layers]
    e.encode(ADAM_STATE, st)
    return b"GONN" + struct.pack("<i", 1) + bytes(e.out)


# ---------------------------------------------------------------- binary weights / GGUF
def binary_weights(tensors):
    """SaveBinaryWeights (net.go:1119-1214); tensors: [(name, shape, data)]."""
    out = bytearray(b"GONN" + struct.pack("<ii", 1, len(tensors)))
    for name, shape, data in tensors:
        nb = name.encode()
        out += struct.pack("<i", len(nb)) + nb + struct.pack("<i", len(shape))
        out += struct.pack("<%di" % len(shape), *shape)
        d = np.asarray(data, "<f4")
        out += struct.pack("<i", d.size) + d.tobytes()
    return bytes(out)


def f32_to_f16(x):
    """Float32ToFloat16 (gguf.go:178-210) on one value: mantissa truncated,
    exponents below the half range shifted into a subnormal or flushed, NaN
    keeps a set low bit."""
    bits = int(np.float32(x).view(np.uint32))
    s = (bits >> 16) & 0x8000
    e = (bits >> 23) & 0xFF
    m = bits & 0x7FFFFF
    if e == 0:
        return s
    if e == 0xFF:
        return s | 0x7C00 if m == 0 else s | 0x7C00 | (m >> 13) | 1
    e -= 127 - 15
    if e >= 31:
        return s | 0x7C00
    if e <= 0:
        if e < -10:
            return s
        m = (m | 0x800000) >> (1 - e)
        return s | (m >> 13)
    return s | (e << 10) | (m >> 13)


GGUF_NAME_MAP = [("weights", "weight"), ("biases", "bias"), ("gamma", "weight"), ("beta", "bias"),
                 ("mha_wQ_", "attn_q."), ("mha_wK_", "attn_k."), ("mha_wV_", "attn_v."),
                 ("mha_wOut_", "attn_output."), ("ff1_", "ffn_up."), ("ff2_", "ffn_down."),
                 ("norm1_", "attn_norm."), ("norm2_", "ffn_norm.")]


def gguf(layer_tensors, nlayers, loss_type, f16):
    """SaveGGUFExt (net.go:1222-1392).  layer_tensors: per layer, either
    [(NamedParams name, shape, data)] or ("flat", data) for a layer without
    NamedParams; loss_type is Go's %T of the loss ("loss.CrossEntropy")."""
    tensors = []
    for i, lt in enumerate(layer_tensors):
        if isinstance(lt, tuple) and lt and lt[0] == "flat":
            if len(lt[1]):
                tensors.append((f"blk.{i}.weight", [len(lt[1])], lt[1]))
            continue
        for name, shape, data in lt:
            for a, b in GGUF_NAME_MAP:
                name = name.replace(a, b)
            tensors.append((f"blk.{i}.{name}", list(shape), data))

    def s(v):
        b = v.encode()
        return struct.pack("<Q", len(b)) + b
    kv = [("general.architecture", 8, "goneuron"), ("general.name", 8, "GoNeuron Model"),
          ("general.alignment", 4, 32), ("goneuron.layer_count", 4, nlayers), ("goneuron.loss_type", 8, loss_type)]
    out = bytearray(struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kv)))
    for k, t, v in kv:
        out += s(k) + struct.pack("<I", t) + (s(v) if t == 8 else struct.pack("<I", v))
    off, tsize = 0, 2 if f16 else 4
    for name, shape, data in tensors:
        out += s(name) + struct.pack("<I", len(shape)) + struct.pack("<%dQ" % len(shape), *reversed(shape))
        out += struct.pack("<IQ", 1 if f16 else 0, off)
        off += len(data) * tsize
        off = (off + 31) // 32 * 32
    for _, _, data in tensors:
        out += b"\0" * ((32 - len(out) % 32) % 32)
        d = np.asarray(data, np.float32)
        if f16:
            out += np.array([f32_to_f16(x) for x in d], "<u2").tobytes()
        else:
            out += d.astype("<f4").tobytes()
    return bytes(out)
