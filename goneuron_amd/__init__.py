"""goneuron_amd — MI355X (gfx950) training backend for GoNeuron's Sequential API.

A Python mirror of the Go facade (goneuron/goneuron.go) over the C ABI of
libgoneuron_hip.so.  Names, argument meaning and error behaviour follow the
reference so that code and tests read the same:

    model = NewSequential(Dense(784, 128, ReLU), Dropout(0.2, 128),
                          Dense(128, 10, Ref(Softmax)))
    model.Compile(Adam(1e-3), CrossEntropy)
    loss = model.TrainBatch(batchX, batchY)

Every step runs on the GPU (hand-written HIP kernels); there is no CPU path.
"""
from __future__ import annotations

import atexit
import ctypes as C
import weakref

import numpy as np

from . import _lib
from ._lib import GNError, LayerDesc, AdamDesc, check, lib

__all__ = [
    "NewSequential", "Sequential", "Dense", "DenseE", "Dropout", "Flatten", "Conv2D", "MaxPool2D",
    "AvgPool2D", "BatchNorm2D", "RMSNorm", "SwiGLU", "MoE", "Embedding", "PositionalEncoding", "TransformerBlock",
    "TransformerBlockExt", "ActReLU", "ActSwiGLU", "ActGELU", "NormLN", "NormRMS", "CLSPooling",
    "LSTM", "GRU", "SequenceUnroller",
    "ReLU", "Sigmoid", "Tanh", "Softmax", "LogSoftmax", "Linear", "GELU", "Ref", "Adam", "MSE",
    "CrossEntropy", "HIPDevice", "GetDefaultDevice", "GNError", "GGMLTypeF32", "GGMLTypeF16", "Load",
]

# ---------------------------------------------------------------- activations
ACT_NIL, ACT_RELU, ACT_SIGMOID, ACT_TANH, ACT_SOFTMAX, ACT_LOGSOFTMAX, ACT_LINEAR, ACT_GELU = range(8)


class Activation:
    """An activation object.  ``is_ptr`` mirrors Go's &activations.X{} versus
    activations.X{}: Dense only applies Softmax/LogSoftmax (and their
    Jacobians) for pointers (layer.go:183-205); the facade's values
    (goneuron.go:30-40) run as identity forward with a NaN derivative."""

    __slots__ = ("kind", "is_ptr", "name")

    def __init__(self, kind, is_ptr, name):
        self.kind, self.is_ptr, self.name = kind, is_ptr, name

    def __repr__(self):
        return ("&" if self.is_ptr else "") + f"activations.{self.name}{{}}"


ReLU = Activation(ACT_RELU, False, "ReLU")
Sigmoid = Activation(ACT_SIGMOID, False, "Sigmoid")
Tanh = Activation(ACT_TANH, False, "Tanh")
Softmax = Activation(ACT_SOFTMAX, False, "Softmax")
LogSoftmax = Activation(ACT_LOGSOFTMAX, False, "LogSoftmax")
Linear = Activation(ACT_LINEAR, False, "Linear")
GELU = Activation(ACT_GELU, False, "GELU")


def Ref(act: Activation) -> Activation:
    """``&act`` — the pointer form of an activation value."""
    return Activation(act.kind, True, act.name)


# ---------------------------------------------------------------- layers
(LAYER_DENSE, LAYER_DROPOUT, LAYER_CONV2D, LAYER_MAXPOOL2D, LAYER_FLATTEN, LAYER_EMBEDDING,
 LAYER_POSENC, LAYER_TRANSFORMER, LAYER_CLSPOOL, LAYER_LSTM_UNROLLER, LAYER_AVGPOOL2D,
 LAYER_RMSNORM, LAYER_SWIGLU, LAYER_BATCHNORM2D, LAYER_GRU_UNROLLER, LAYER_MOE, LAYER_MHA,
 LAYER_LAYERNORM, LAYER_GAP1D) = range(1, 20)


class Layer:
    def __init__(self, kind, **fields):
        self.desc = LayerDesc()
        self.desc.kind = kind
        self.desc.in_channels = -1
        for k, v in fields.items():
            setattr(self.desc, k, v)

    def InSize(self):
        return self.desc.in_size

    def __repr__(self):
        return f"{type(self).__name__}({self.desc.in_size}->{self.desc.out_size})"


class _Dense(Layer):
    pass


def DenseE(*args):
    """goneuron.DenseE (goneuron.go:68-113): (in, out, act) or (out, act, in).
    The lazy form (out, act) is rejected: Dense.Build has no error return, so
    Sequential.Build never resolves it (sequential.go:68-74)."""
    if len(args) == 3 and isinstance(args[1], int):
        i, o, act = args
    elif len(args) == 3:
        o, act, i = args
    elif len(args) == 2:
        raise GNError(-1, "Dense(out, act): lazy input size is not resolved by Sequential.Build")
    else:
        raise GNError(-1, f"Dense expects 2 or 3 arguments, got {len(args)}")
    if not isinstance(act, Activation):
        raise GNError(-1, f"Dense: activation must be an Activation, got {type(act).__name__}")
    if i <= 0 or o <= 0:
        raise GNError(-1, f"invalid sizes in={i} out={o}")
    return _Dense(LAYER_DENSE, in_size=i, out_size=o, act=act.kind, act_is_ptr=int(act.is_ptr))


def Dense(*args):
    return DenseE(*args)


def Dropout(prob: float, *in_size):
    """goneuron.Dropout (goneuron.go:211-218) -> layer.NewDropout (dropout.go:47-53),
    which requires an input size."""
    if not in_size or in_size[0] <= 0:
        raise GNError(-1, "Dropout needs an input size (NewDropout rejects inSize <= 0)")
    if prob < 0 or prob > 1:
        raise GNError(-1, f"invalid dropout probability {prob}")
    return Layer(LAYER_DROPOUT, in_size=in_size[0], out_size=in_size[0], p=prob)


def Flatten(*in_size):
    return Layer(LAYER_FLATTEN, in_size=in_size[0] if in_size else 0)


def Conv2D(*args):
    """goneuron.Conv2DE (goneuron.go:131-182): (inC, outC, k, s, p, act)."""
    if len(args) == 6 and isinstance(args[5], Activation):
        ic, oc, k, s, p, act = args
    elif len(args) == 6:
        oc, k, s, p, act, ic = args
    else:
        raise GNError(-1, "Conv2D expects (inC, outC, k, s, p, act)")
    return Layer(LAYER_CONV2D, in_channels=ic, out_channels=oc, kernel=k, stride=s, padding=p,
                 act=act.kind, act_is_ptr=int(act.is_ptr))


def MaxPool2D(kernel, stride, padding, *in_channels):
    return Layer(LAYER_MAXPOOL2D, kernel=kernel, stride=stride, padding=padding,
                 in_channels=in_channels[0] if in_channels else -1)


def AvgPool2D(kernel, stride, padding, *in_channels):
    """goneuron.AvgPool2D (goneuron.go:256): average over the in-bounds cells of
    each window (padding not counted)."""
    return Layer(LAYER_AVGPOOL2D, kernel=kernel, stride=stride, padding=padding,
                 in_channels=in_channels[0] if in_channels else -1)


def BatchNorm2D(*in_channels, eps=1e-5, momentum=0.1, affine=True):
    """goneuron.BatchNorm2D (goneuron.go:211-218): NewBatchNorm2D(in, 1e-5,
    0.1, true).  Training normalises each sample's channel planes by their own
    statistics (one sample per Forward) and advances the running mean / var
    once per sample; inference uses the running statistics.  The lazy form is
    rejected: BatchNorm2D.Build has no error return, so Sequential.Build
    (sequential.go:68-73) never resolves it."""
    if not in_channels or in_channels[0] <= 0:
        raise GNError(-1, "BatchNorm2D needs the channel count (the lazy form is never built)")
    if eps < 0 or not (0 <= momentum <= 1):
        raise GNError(-1, f"invalid eps {eps} / momentum {momentum}")
    return Layer(LAYER_BATCHNORM2D, in_channels=int(in_channels[0]), eps=float(eps) if eps > 0 else 0.0,
                 momentum=float(momentum), no_affine=int(not affine))


def RMSNorm(*normalized_shape, eps=1e-5):
    """goneuron.RMSNorm (goneuron.go:229-236): y = x / sqrt(mean(x^2) + eps) *
    gamma over rows of normalizedShape, gamma starting at 1 (rmsnorm.go:73-96).
    The lazy form RMSNorm() is rejected: RMSNorm.Build has no error return, so
    Sequential.Build (sequential.go:68-73) never resolves its size."""
    if not normalized_shape or normalized_shape[0] <= 0:
        raise GNError(-1, "RMSNorm needs normalizedShape > 0 (the lazy form is never built)")
    if eps < 0:
        raise GNError(-1, f"invalid eps {eps}: must be >= 0")
    return Layer(LAYER_RMSNORM, dim=int(normalized_shape[0]), eps=float(eps) if eps > 0 else 0.0)


def LayerNorm(*normalized_shape, eps=1e-5):
    """goneuron.LayerNorm (goneuron.go:220-227) -> layer.NewLayerNorm(in, 1e-5,
    true): y = gamma (x - mean) / sqrt(var + eps) + beta over rows of
    normalizedShape, gamma 1 and beta 0 at the start (layernorm.go:57-118).
    The lazy form LayerNorm() is rejected: LayerNorm.Build has no error
    return, so Sequential.Build (sequential.go:68-73) never resolves it."""
    if not normalized_shape or normalized_shape[0] <= 0:
        raise GNError(-1, "LayerNorm needs normalizedShape > 0 (the lazy form is never built)")
    if eps < 0:
        raise GNError(-1, f"invalid eps {eps}: must be >= 0")
    return Layer(LAYER_LAYERNORM, dim=int(normalized_shape[0]), eps=float(eps) if eps > 0 else 0.0)


def MultiHeadAttention(num_heads, seq_len, causal, *dim):
    """goneuron.MultiHeadAttention (goneuron.go:369-376) ->
    layer.NewMultiHeadAttentionE(dim, numHeads, seqLen, causal): per-token
    wQ, wK, wV, wOut Linear Dense layers around scaled dot-product attention,
    all parameters starting at 0 (Build rebinds them to a fresh zero buffer,
    transformer.go:318-394).  Without dim the layer takes input / seq_len."""
    if num_heads <= 0 or seq_len <= 0:
        raise GNError(-1, f"invalid numHeads {num_heads} / seqLen {seq_len}")
    d = int(dim[0]) if dim else -1
    if d != -1 and (d <= 0 or d % num_heads):
        raise GNError(-1, f"dim {d} must be positive and divisible by numHeads {num_heads}")
    return Layer(LAYER_MHA, dim=d, num_heads=int(num_heads), seq_len=int(seq_len), causal=int(causal))


def GlobalAveragePooling1D(seq_len, dim):
    """goneuron.GlobalAveragePooling1D (goneuron.go:378-381): the mean over the
    seq_len rows of dim (transformer.go:1524-1600)."""
    if seq_len <= 0 or dim <= 0:
        raise GNError(-1, f"invalid seqLen {seq_len} / dim {dim}")
    return Layer(LAYER_GAP1D, seq_len=int(seq_len), dim=int(dim))


def SwiGLU(out, *in_size):
    """goneuron.SwiGLU (goneuron.go:238-245): y = swish(W x) * (V x), no
    biases.  The lazy form SwiGLU(out) is rejected: SwiGLU.Build has no error
    return, so Sequential.Build (sequential.go:68-73) never resolves its size."""
    if not in_size or in_size[0] <= 0:
        raise GNError(-1, "SwiGLU needs an input size (the lazy form is never built)")
    if out <= 0:
        raise GNError(-1, f"invalid outSize {out}: must be > 0")
    return Layer(LAYER_SWIGLU, in_size=int(in_size[0]), out_size=int(out))


def MoE(out, num_experts, k, *in_size):
    """goneuron.MoE (goneuron.go:398-405): a Linear gating Dense and
    num_experts Dense(in, out, LeakyReLU 0.1) experts, top-k routing by the
    gate softmax, all parameters starting at 0 (moe.go:122-135).  Training
    mode adds the RNG(42) gate noise and the load-balancing gradient.  The
    lazy form is rejected (the input size must be known)."""
    if not in_size or in_size[0] <= 0:
        raise GNError(-1, "MoE needs an input size")
    if out <= 0 or num_experts <= 0 or not (0 < k <= num_experts):
        raise GNError(-1, f"invalid MoE sizes out={out} experts={num_experts} k={k}")
    return Layer(LAYER_MOE, in_size=int(in_size[0]), out_size=int(out), num_experts=int(num_experts),
                 top_k=int(k))


def Embedding(num, dim):
    return Layer(LAYER_EMBEDDING, vocab=num, dim=dim)


def PositionalEncoding(seq_len, *dim):
    return Layer(LAYER_POSENC, seq_len=seq_len, dim=dim[0] if dim else -1)


def TransformerBlock(dim, heads, seq_len, ff_dim, causal):
    return Layer(LAYER_TRANSFORMER, dim=dim, num_heads=heads, seq_len=seq_len, ff_dim=ff_dim,
                 causal=int(causal))


# GGUF tensor types (gguf.go:57-66)
GGMLTypeF32, GGMLTypeF16 = 0, 1

# TransformerBlockExt options (goneuron.go:352-358, transformer.go:199-210)
ActReLU, ActSwiGLU, ActGELU = 0, 1, 2
NormLN, NormRMS = 0, 1


def TransformerBlockExt(heads, seq_len, ff_dim, causal, act_type, norm_type, use_rope, *dim):
    """goneuron.TransformerBlockExt (goneuron.go:342-350): feed-forward ReLU,
    SwiGLU or GELU, LayerNorm or RMSNorm, optional rotary embeddings on Q and
    K.  The model dimension is required: with dim = -1 the reference leaves
    the RMSNorm and SwiGLU sub-layers unbuilt (their Build has no error
    return, transformer.go:987-1005)."""
    if not dim or dim[0] <= 0:
        raise GNError(-1, "TransformerBlockExt needs the model dimension")
    if act_type not in (ActReLU, ActSwiGLU, ActGELU):
        raise GNError(-1, f"unknown activation type {act_type}")
    if norm_type not in (NormLN, NormRMS):
        raise GNError(-1, f"unknown norm type {norm_type}")
    return Layer(LAYER_TRANSFORMER, dim=int(dim[0]), num_heads=heads, seq_len=seq_len, ff_dim=ff_dim,
                 causal=int(causal), block_act=int(act_type), block_norm=int(norm_type),
                 use_rope=int(bool(use_rope)))


def CLSPooling(seq_len, dim):
    return Layer(LAYER_CLSPOOL, seq_len=seq_len, dim=dim)


class _LSTMSpec:
    def __init__(self, out, inp):
        self.out, self.inp = out, inp


class _GRUSpec(_LSTMSpec):
    pass


def LSTM(out, *inp):
    return _LSTMSpec(out, inp[0] if inp else -1)


def GRU(out, *inp):
    """goneuron.GRU (goneuron.go:193-200): NewGRU(in, out), usable through
    SequenceUnroller."""
    return _GRUSpec(out, inp[0] if inp else -1)


def SequenceUnroller(l, seq_len, return_sequences):
    """goneuron.SequenceUnroller over an LSTM or a GRU (unroller.go:57-213)."""
    if not isinstance(l, _LSTMSpec):
        raise GNError(-4, "SequenceUnroller is built for LSTM and GRU only")
    kind = LAYER_GRU_UNROLLER if isinstance(l, _GRUSpec) else LAYER_LSTM_UNROLLER
    return Layer(kind, in_size=l.inp, out_size=l.out, seq_len=seq_len,
                 return_sequences=int(return_sequences))


# ---------------------------------------------------------------- optimizer / loss
class Adam:
    """opt.NewAdam (opt.go:117-126): beta1 0.9, beta2 0.999, eps 1e-8."""

    def __init__(self, lr, beta1=0.9, beta2=0.999, eps=1e-8):
        self.LearningRate, self.Beta1, self.Beta2, self.Epsilon = lr, beta1, beta2, eps


LOSS_MSE, LOSS_CE = 1, 2


class _Loss:
    def __init__(self, kind, name):
        self.kind, self.name = kind, name

    def __repr__(self):
        return f"loss.{self.name}{{}}"


MSE = _Loss(LOSS_MSE, "MSE")
CrossEntropy = _Loss(LOSS_CE, "CrossEntropy")


# ---------------------------------------------------------------- device
class HIPDevice:
    """One HIP context (stream + scratch) on a GPU ordinal: the MI355X
    counterpart of layer.MetalDevice (metal.go:67-98)."""

    def __init__(self, ordinal=0):
        h = C.c_void_p()
        rc = lib().gn_init(ordinal, C.byref(h))
        if rc != 0:
            raise GNError(rc, "gn_init failed (no HIP device?)")
        self.h = h

    def Type(self):
        return "GPU"

    def IsAvailable(self):
        return True

    def sync(self):
        check(self.h, lib().gn_sync(self.h))

    def info(self):
        inf = _lib.Info()
        check(self.h, lib().gn_device_info(self.h, C.byref(inf)))
        return {"arch": inf.arch.decode(), "cu_count": inf.cu_count, "hbm_bytes": inf.hbm_bytes,
                "peak_fp32_mfma_tflops": inf.peak_fp32_mfma_tflops,
                "peak_hbm_gbps": inf.peak_hbm_gbps}

    def close(self):
        if getattr(self, "h", None):
            lib().gn_shutdown(self.h)
            self.h = None


_default = None
_live_models = weakref.WeakSet()


def _teardown():
    """At interpreter exit: destroy every live model, then shut the default
    device down, in that order and before module finalisation, so no HIP call
    runs from a finalizer after the runtime has started to unload."""
    global _default
    for m in list(_live_models):
        try:
            m.Close()
        except Exception:
            pass
    if _default is not None:
        try:
            _default.close()
        except Exception:
            pass
        _default = None


atexit.register(_teardown)


def GetDefaultDevice() -> HIPDevice:
    """layer.GetDefaultDevice (device.go:39-48): the HIP device.  Raises when
    no GPU is present (no CPU fallback)."""
    global _default
    if _default is None:
        if not lib().gn_available():
            raise GNError(-7, "no HIP device available")
        _default = HIPDevice(0)
    return _default


# ---------------------------------------------------------------- model
def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


class Sequential:
    """net.Sequential (sequential.go:11-212) running on one HIP device."""

    def __init__(self, *layers, device=None):
        self.layers = list(layers)
        self.device = device
        self.h = None
        self.opt = None
        self.loss = None
        self.workers = 1
        self.max_batch = 0

    # Compile (sequential.go:26-37) + Build/initBuffers (:41-87, net.go:91-127)
    def Compile(self, optimizer, loss_fn, max_batch=1024, workers=1):
        self.opt, self.loss = optimizer, loss_fn
        self.workers = workers
        self._create(max_batch)
        return None

    def _create(self, max_batch):
        if self.device is None:
            self.device = GetDefaultDevice()
        if self.h is not None:
            lib().gn_model_destroy(self.h)
            self.h = None
        descs = (LayerDesc * len(self.layers))(*[l.desc for l in self.layers])
        ad = AdamDesc(self.opt.LearningRate, self.opt.Beta1, self.opt.Beta2, self.opt.Epsilon)
        h = C.c_void_p()
        check(self.device.h, lib().gn_model_create(self.device.h, descs, len(self.layers), self.loss.kind,
                                                   C.byref(ad), max_batch, self.workers, C.byref(h)))
        self.h = h
        self.max_batch = max_batch
        _live_models.add(self)
        n = C.c_int64()
        check(self.device.h, lib().gn_model_nparams(self.h, C.byref(n)))
        self.nparams = n.value
        o = C.c_int32()
        check(self.device.h, lib().gn_model_out_size(self.h, C.byref(o)))
        self.out_size = o.value

    def _ck(self, rc):
        return check(self.device.h, rc)

    def SetDevice(self, device):
        self.device = device

    def SetTraining(self, training):
        """Network.SetTraining (net.go:187-193)."""
        self._ck(lib().gn_model_set_training(self.h, int(training)))

    def IsTraining(self, i):
        t = C.c_int32()
        self._ck(lib().gn_model_get_training(self.h, i, C.byref(t)))
        return bool(t.value)

    def _reserve(self, B):
        """Batch-sized buffers for B samples; every other piece of state stays."""
        if B > self.max_batch:
            self._ck(lib().gn_model_reserve(self.h, B))
            self.max_batch = B

    def SkippedSamples(self):
        """Samples the last TrainBatch skipped (Embedding index out of range;
        the reference's batch loop drops them, net.go:738-741)."""
        n = C.c_int32()
        self._ck(lib().gn_model_skipped_samples(self.h, C.byref(n)))
        return n.value

    def TrainBatch(self, batchX, batchY) -> float:
        """Network.TrainBatch (net.go:412-436): fwd + bwd + Adam; returns mean loss."""
        x = _f32(batchX)
        y = _f32(batchY)
        B = x.shape[0]
        if B == 0:
            return 0.0  # net.go:414-417
        self._reserve(B)
        loss = C.c_float()
        self._ck(lib().gn_model_train_step(self.h, _fp(x), _fp(y), B, C.byref(loss)))
        return loss.value

    def Fit(self, trainX, trainY, epochs, batchSize, callbacks=()):
        """Network.Fit (net.go:351-408) without callbacks' side effects: sets
        training mode, then TrainBatch over the batches of every epoch."""
        self.SetTraining(True)
        x = _f32(trainX)
        y = _f32(trainY)
        n = x.shape[0]
        nb = (n + batchSize - 1) // batchSize
        hist = []
        for _ in range(epochs):
            tot = np.float32(0)
            for b in range(nb):
                tot += np.float32(self.TrainBatch(x[b * batchSize:(b + 1) * batchSize],
                                                  y[b * batchSize:(b + 1) * batchSize]))
            hist.append(float(tot / np.float32(nb)))
        return hist

    def PredictBatch(self, x):
        x = _f32(x)
        B = x.shape[0]
        self._reserve(B)
        out = np.empty((B, self.out_size), np.float32)
        self._ck(lib().gn_model_predict(self.h, _fp(x), B, _fp(out)))
        return out

    def Predict(self, x):
        """Sequential.Predict (sequential.go:118-122): inference mode."""
        return self.PredictBatch(_f32(x).reshape(1, -1))[0]

    # flat arena views (net.go:787-846)
    def Params(self):
        out = np.empty(self.nparams, np.float32)
        self._ck(lib().gn_model_get_params(self.h, _fp(out), 0, self.nparams))
        return out

    def SetParams(self, p):
        p = _f32(p)
        self._ck(lib().gn_model_set_params(self.h, _fp(p), 0, p.size))

    def Gradients(self):
        out = np.empty(self.nparams, np.float32)
        self._ck(lib().gn_model_get_grads(self.h, _fp(out), 0, self.nparams))
        return out

    def AdamState(self):
        m = np.empty(self.nparams, np.float32)
        v = np.empty(self.nparams, np.float32)
        t = C.c_int32()
        self._ck(lib().gn_model_get_adam(self.h, _fp(m), _fp(v), 0, self.nparams, C.byref(t)))
        return m, v, t.value

    def LayerParams(self, i):
        off, cnt = C.c_int64(), C.c_int64()
        self._ck(lib().gn_model_layer_params(self.h, i, C.byref(off), C.byref(cnt)))
        return slice(off.value, off.value + cnt.value)

    def LayerOutput(self, i, n):
        out = np.empty(n, np.float32)
        self._ck(lib().gn_model_layer_output(self.h, i, _fp(out), n))
        return out

    # ---- checkpoints (net.go:863-1392) ----
    def Save(self, filename):
        """Network.Save (net.go:863-871): the "GONN" gob file net.Load reads."""
        self._ck(lib().gn_model_save_gob(self.h, str(filename).encode()))

    def SaveBinaryWeights(self, filename):
        """Network.SaveBinaryWeights (net.go:1119-1214)."""
        self._ck(lib().gn_model_save_binary_weights(self.h, str(filename).encode()))

    def LoadBinaryWeights(self, filename):
        """Reads a SaveBinaryWeights file into this model (names and sizes checked)."""
        self._ck(lib().gn_model_load_binary_weights(self.h, str(filename).encode()))

    def SaveGGUF(self, filename):
        """Network.SaveGGUF (net.go:1217-1220): GGUF v3, F32 tensors."""
        self.SaveGGUFExt(filename, GGMLTypeF32)

    def SaveGGUFExt(self, filename, tensor_type):
        """Network.SaveGGUFExt (net.go:1222-1392): F32 or F16 tensors."""
        self._ck(lib().gn_model_save_gguf(self.h, str(filename).encode(), int(tensor_type)))

    def SaveState(self, filename):
        """Parameters, Adam moments and timestep, BatchNorm2D running stats and
        MoE noise streams, for resuming training."""
        self._ck(lib().gn_model_save_state(self.h, str(filename).encode()))

    def LoadState(self, filename):
        self._ck(lib().gn_model_load_state(self.h, str(filename).encode()))

    def RunningStats(self, i):
        """BatchNorm2D.GetRunningMean / GetRunningVar (batchnorm2d.go:837-838)."""
        n = self.layers[i].desc.in_channels
        m, v = np.empty(n, np.float32), np.empty(n, np.float32)
        self._ck(lib().gn_model_get_running_stats(self.h, i, _fp(m), _fp(v), n))
        return m, v

    def SetRunningStats(self, i, mean, var):
        m, v = _f32(mean).ravel(), _f32(var).ravel()
        self._ck(lib().gn_model_set_running_stats(self.h, i, _fp(m), _fp(v), m.size))

    def LayerArgmax(self, i, n):
        out = np.empty(n, np.int32)
        self._ck(lib().gn_model_layer_argmax(self.h, i, out.ctypes.data_as(C.POINTER(C.c_int32)), n))
        return out

    def Close(self):
        if self.h is not None:
            lib().gn_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.Close()
        except Exception:
            pass


def NewSequential(*layers, device=None) -> Sequential:
    return Sequential(*layers, device=device)


def Load(filename, in_len=0, max_batch=1024, workers=1, device=None):
    """goneuron.Load (goneuron.go:491-497, net.Load net.go:875-1005): the model
    a Save file describes, with its parameters, the saved loss and a fresh
    Adam(0.001); returns (model, loss).  in_len is the per-sample input length,
    needed when the first layer is not Dense or Dropout."""
    device = device or GetDefaultDevice()
    h = C.c_void_p()
    lk = C.c_int32()
    check(device.h, lib().gn_model_load_gob(device.h, str(filename).encode(), int(in_len), int(max_batch),
                                            int(workers), C.byref(h), C.byref(lk)))
    n = C.c_int32()
    check(device.h, lib().gn_model_layer_count(h, C.byref(n)))
    layers = []
    for i in range(n.value):
        d = LayerDesc()
        check(device.h, lib().gn_model_layer_desc(h, i, C.byref(d)))
        layer = Layer(d.kind)
        layer.desc = d
        layers.append(layer)
    m = Sequential(*layers, device=device)
    m.opt = Adam(0.001)
    m.loss = CrossEntropy if lk.value == LOSS_CE else MSE
    m.workers = int(workers)
    m.h = h
    m.max_batch = int(max_batch)
    _live_models.add(m)
    cnt = C.c_int64()
    check(device.h, lib().gn_model_nparams(h, C.byref(cnt)))
    m.nparams = cnt.value
    check(device.h, lib().gn_model_out_size(h, C.byref(n)))
    m.out_size = n.value
    return m, m.loss


# ---------------------------------------------------------------- synthetic data
def fill_uniform(n, seed):
    a = np.empty(n, np.float32)
    check(None, lib().gn_fill_uniform(_fp(a), n, seed))
    return a


def fill_normal(n, seed):
    a = np.empty(n, np.float32)
    check(None, lib().gn_fill_normal(_fp(a), n, seed))
    return a


def fill_class_ids(n, nclass, seed):
    a = np.empty(n, np.int32)
    check(None, lib().gn_fill_class_ids(a.ctypes.data_as(C.POINTER(C.c_int32)), n, nclass, seed))
    return a
