"""ctypes wrapper for the CPU parity oracle (``oracle/librefcpu.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, as the checker or the timed CPU
baseline.  The product (``goneuron_amd``) never imports this module.

The library restates GoNeuron's pure-Go float32 per-sample training step
(internal/net/net.go:588-784 and the layer files cited in ``refcpu.h``).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "librefcpu.so")

(ACT_NIL, ACT_RELU, ACT_SIGMOID, ACT_TANH, ACT_SOFTMAX, ACT_LOGSOFTMAX, ACT_LINEAR, ACT_GELU,
 ACT_LEAKYRELU) = range(9)
(LAYER_DENSE, LAYER_DROPOUT, LAYER_CONV2D, LAYER_MAXPOOL2D, LAYER_FLATTEN, LAYER_EMBEDDING,
 LAYER_POSENC, LAYER_TRANSFORMER, LAYER_CLSPOOL, LAYER_LSTM_UNROLLER, LAYER_AVGPOOL2D,
 LAYER_RMSNORM, LAYER_SWIGLU, LAYER_BATCHNORM2D, LAYER_GRU_UNROLLER, LAYER_MOE, LAYER_MHA,
 LAYER_LAYERNORM, LAYER_GAP1D) = range(1, 20)
LOSS_MSE, LOSS_CE = 1, 2


class LayerSpec(C.Structure):
    _fields_ = [
        ("kind", C.c_int32), ("in_size", C.c_int32), ("out_size", C.c_int32),
        ("act", C.c_int32), ("act_is_ptr", C.c_int32),
        ("in_channels", C.c_int32), ("out_channels", C.c_int32),
        ("kernel", C.c_int32), ("stride", C.c_int32), ("padding", C.c_int32),
        ("p", C.c_float),
        ("seq_len", C.c_int32), ("num_heads", C.c_int32), ("ff_dim", C.c_int32),
        ("causal", C.c_int32), ("vocab", C.c_int32), ("dim", C.c_int32),
        ("return_sequences", C.c_int32), ("eps", C.c_float),
        ("block_act", C.c_int32), ("block_norm", C.c_int32), ("use_rope", C.c_int32),
        ("momentum", C.c_float), ("no_affine", C.c_int32),
        ("num_experts", C.c_int32), ("top_k", C.c_int32),
    ]


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        f32p = C.POINTER(C.c_float)
        i32p = C.POINTER(C.c_int32)
        L.gno_rand_float.argtypes = [C.POINTER(C.c_uint64)]
        L.gno_rand_float.restype = C.c_float
        L.gno_fill_uniform.argtypes = [f32p, C.c_int64, C.c_uint64]
        L.gno_fill_normal.argtypes = [f32p, C.c_int64, C.c_uint64]
        L.gno_fill_class_ids.argtypes = [i32p, C.c_int64, C.c_int32, C.c_uint64]
        L.gno_net_create.argtypes = [C.POINTER(LayerSpec), C.c_int32, C.c_int32, C.c_float, C.c_int32]
        L.gno_net_create.restype = C.c_void_p
        L.gno_net_destroy.argtypes = [C.c_void_p]
        for name in ("gno_net_nparams",):
            getattr(L, name).argtypes = [C.c_void_p]
            getattr(L, name).restype = C.c_int64
        L.gno_net_layer_param_offset.argtypes = [C.c_void_p, C.c_int32]
        L.gno_net_layer_param_offset.restype = C.c_int64
        L.gno_net_layer_param_count.argtypes = [C.c_void_p, C.c_int32]
        L.gno_net_layer_param_count.restype = C.c_int64
        for name in ("gno_net_params", "gno_net_grads", "gno_net_adam_m", "gno_net_adam_v"):
            getattr(L, name).argtypes = [C.c_void_p]
            getattr(L, name).restype = f32p
        L.gno_net_adam_timestep.argtypes = [C.c_void_p]
        L.gno_net_adam_timestep.restype = C.c_int32
        L.gno_net_train_batch.argtypes = [C.c_void_p, f32p, f32p, C.c_int32]
        L.gno_net_train_batch.restype = C.c_float
        L.gno_net_accumulate_batch.argtypes = [C.c_void_p, f32p, f32p, C.c_int32]
        L.gno_net_accumulate_batch.restype = C.c_float
        L.gno_net_step.argtypes = [C.c_void_p]
        L.gno_net_accumulate_grad.argtypes = [C.c_void_p, f32p, f32p, C.c_int32, C.c_int32, f32p, f32p]
        L.gno_net_forward.argtypes = [C.c_void_p, f32p, f32p]
        L.gno_net_forward.restype = C.c_int32
        L.gno_net_set_training.argtypes = [C.c_void_p, C.c_int32]
        L.gno_net_out_size.argtypes = [C.c_void_p]
        L.gno_net_out_size.restype = C.c_int32
        L.gno_net_layer_argmax.argtypes = [C.c_void_p, C.c_int32, i32p, C.c_int32]
        L.gno_net_layer_argmax.restype = C.c_int32
        L.gno_net_layer_routes.argtypes = [C.c_void_p, C.c_int32, i32p, C.c_int32]
        L.gno_net_layer_routes.restype = C.c_int32
        L.gno_net_layer_preact.argtypes = [C.c_void_p, C.c_int32, f32p, C.c_int32]
        L.gno_net_layer_preact.restype = C.c_int32
        L.gno_activate_batch.argtypes = [C.c_int32, f32p, C.c_int32]
        L.gno_activate.argtypes = [C.c_int32, C.c_float]
        L.gno_activate.restype = C.c_float
        L.gno_derivative.argtypes = [C.c_int32, C.c_float]
        L.gno_derivative.restype = C.c_float
        L.gno_loss_forward.argtypes = [C.c_int32, f32p, f32p, C.c_int32]
        L.gno_loss_forward.restype = C.c_float
        L.gno_loss_backward.argtypes = [C.c_int32, f32p, f32p, f32p, C.c_int32]
        L.gno_adam_step_inplace.argtypes = [f32p, f32p, f32p, f32p, C.c_int64, C.c_float, C.c_float,
                                            C.c_float, C.c_float, C.c_int32]
        L.gno_matmul.argtypes = [f32p, f32p, f32p, f32p, C.c_int32, C.c_int32, C.c_int32]
        L.gno_avgpool2d.argtypes = [f32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                    f32p, f32p, f32p]
        L.gno_avgpool2d.restype = C.c_int32
        L.gno_rmsnorm.argtypes = [f32p, C.c_int32, C.c_int32, C.c_float, f32p, f32p, f32p, f32p,
                                  f32p]
        L.gno_rmsnorm.restype = C.c_int32
        L.gno_swiglu.argtypes = [f32p, C.c_int32, C.c_int32, f32p, f32p, f32p, f32p, f32p]
        L.gno_rope.argtypes = [f32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32]
        L.gno_moe.argtypes = [f32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, f32p, C.c_int32,
                              C.POINTER(C.c_uint64), f32p, i32p, f32p, f32p, f32p]
        L.gno_moe.restype = C.c_int32
        L.gno_gru_sequence.argtypes = [f32p, C.c_int32, C.c_int32, C.c_int32, f32p, f32p, f32p, f32p,
                                       f32p]
        L.gno_batchnorm2d.argtypes = [f32p, C.c_int32, C.c_int32, C.c_int32, C.c_float, C.c_float,
                                      C.c_int32, f32p, C.c_int32, f32p, f32p, f32p, f32p, f32p, f32p]
        L.gno_net_layer_running_stats.argtypes = [C.c_void_p, C.c_int32, f32p, f32p]
        L.gno_net_layer_running_stats.restype = C.c_int32
        _lib = L
    return _lib


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_float))


def iptr(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def fill_uniform(n, seed):
    a = np.empty(n, np.float32)
    lib().gno_fill_uniform(fptr(a), n, seed)
    return a


def fill_normal(n, seed):
    a = np.empty(n, np.float32)
    lib().gno_fill_normal(fptr(a), n, seed)
    return a


def fill_class_ids(n, nclass, seed):
    a = np.empty(n, np.int32)
    lib().gno_fill_class_ids(iptr(a), n, nclass, seed)
    return a


def spec(kind, **kw) -> LayerSpec:
    s = LayerSpec()
    s.kind = kind
    s.in_channels = -1
    for k, v in kw.items():
        setattr(s, k, v)
    return s


class Net:
    """Owns an oracle network; exposes flat params/grads/m/v as numpy views."""

    def __init__(self, specs, loss_kind, lr=1e-3, workers=1):
        arr = (LayerSpec * len(specs))(*specs)
        self._keep = arr
        self.h = lib().gno_net_create(arr, len(specs), loss_kind, lr, workers)
        self.n = lib().gno_net_nparams(self.h)
        self.nlayers = len(specs)

    def _view(self, fn):
        p = fn(self.h)
        return np.ctypeslib.as_array(p, shape=(self.n,))

    @property
    def params(self):
        return self._view(lib().gno_net_params)

    @property
    def grads(self):
        return self._view(lib().gno_net_grads)

    @property
    def adam_m(self):
        return self._view(lib().gno_net_adam_m)

    @property
    def adam_v(self):
        return self._view(lib().gno_net_adam_v)

    @property
    def timestep(self):
        return lib().gno_net_adam_timestep(self.h)

    def layer_slice(self, i):
        off = lib().gno_net_layer_param_offset(self.h, i)
        cnt = lib().gno_net_layer_param_count(self.h, i)
        return slice(off, off + cnt)

    def train_batch(self, x, y, B):
        x = np.ascontiguousarray(x, np.float32)
        y = np.ascontiguousarray(y, np.float32)
        return lib().gno_net_train_batch(self.h, fptr(x), fptr(y), B)

    def accumulate_batch(self, x, y, B):
        x = np.ascontiguousarray(x, np.float32)
        y = np.ascontiguousarray(y, np.float32)
        return lib().gno_net_accumulate_batch(self.h, fptr(x), fptr(y), B)

    def accumulate_grad(self, x, gout, B, in_len, out_len):
        """Batch pass with given output gradients: returns (outputs, input
        gradients); self.grads holds the averaged parameter gradients."""
        x = np.ascontiguousarray(x, np.float32)
        gout = np.ascontiguousarray(gout, np.float32)
        out = np.zeros((B, out_len), np.float32)
        gin = np.zeros((B, in_len), np.float32)
        lib().gno_net_accumulate_grad(self.h, fptr(x), fptr(gout), B, out_len, fptr(out), fptr(gin))
        return out, gin

    def step(self):
        lib().gno_net_step(self.h)

    def forward(self, x, out_cap=1 << 20):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(out_cap, np.float32)
        n = lib().gno_net_forward(self.h, fptr(x), fptr(out))
        if n < 0:
            raise ValueError("Forward failed (embedding index out of range)")
        return out[:n].copy()

    def set_training(self, t):
        lib().gno_net_set_training(self.h, int(t))

    def argmax(self, layer, cap=1 << 20):
        a = np.empty(cap, np.int32)
        n = lib().gno_net_layer_argmax(self.h, layer, iptr(a), cap)
        return a[:n].copy()

    def routes(self, layer, cap=1 << 20):
        """MoE routes logged since the previous call (the first call starts the log)."""
        a = np.empty(cap, np.int32)
        n = lib().gno_net_layer_routes(self.h, layer, iptr(a), cap)
        return a[:n].copy()

    def running_stats(self, layer, cap=1 << 16):
        m = np.empty(cap, np.float32)
        v = np.empty(cap, np.float32)
        n = lib().gno_net_layer_running_stats(self.h, layer, fptr(m), fptr(v))
        return m[:n].copy(), v[:n].copy()

    def preact(self, layer, cap=1 << 20):
        a = np.empty(cap, np.float32)
        n = lib().gno_net_layer_preact(self.h, layer, fptr(a), cap)
        return a[:n].copy()

    def __del__(self):
        try:
            lib().gno_net_destroy(self.h)
        except Exception:
            pass


def avgpool2d(x, in_channels, kernel, stride, padding, g=None):
    """AvgPool2D of one sample; returns out, or (out, grad_in) when g is given."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size, np.float32)
    if g is None:
        n = lib().gno_avgpool2d(fptr(x), x.size, in_channels, kernel, stride, padding, fptr(out),
                                None, None)
        return out[:n].copy()
    g = np.ascontiguousarray(g, np.float32)
    gin = np.empty(x.size, np.float32)
    n = lib().gno_avgpool2d(fptr(x), x.size, in_channels, kernel, stride, padding, fptr(out),
                            fptr(g), fptr(gin))
    return out[:n].copy(), gin


def rmsnorm(x, n, gamma=None, g=None, eps=1e-5):
    """RMSNorm of one sample over rows of n; returns out, or (out, grad_in,
    grad_gamma) when g is given (grad_gamma accumulated from zero)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    gamma = np.ones(n, np.float32) if gamma is None else np.ascontiguousarray(gamma, np.float32)
    out = np.empty(x.size, np.float32)
    if g is None:
        if lib().gno_rmsnorm(fptr(x), x.size, n, eps, fptr(gamma), fptr(out), None, None, None) < 0:
            raise ValueError("n must divide the input length")
        return out
    g = np.ascontiguousarray(g, np.float32).ravel()
    gin = np.empty(x.size, np.float32)
    gg = np.zeros(n, np.float32)
    if lib().gno_rmsnorm(fptr(x), x.size, n, eps, fptr(gamma), fptr(out), fptr(g), fptr(gin),
                         fptr(gg)) < 0:
        raise ValueError("n must divide the input length")
    return out, gin, gg


def swiglu(x, out, params, g=None):
    """SwiGLU of one sample (params [W | V], each out x in); returns y, or
    (y, grad_in, grad_params) when g is given (grad_params from zero)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    params = np.ascontiguousarray(params, np.float32).ravel()
    assert params.size == 2 * x.size * out
    y = np.empty(out, np.float32)
    if g is None:
        lib().gno_swiglu(fptr(x), x.size, out, fptr(params), fptr(y), None, None, None)
        return y
    g = np.ascontiguousarray(g, np.float32).ravel()
    gin = np.empty(x.size, np.float32)
    gp = np.zeros(params.size, np.float32)
    lib().gno_swiglu(fptr(x), x.size, out, fptr(params), fptr(y), fptr(g), fptr(gin), fptr(gp))
    return y, gin, gp


def batchnorm2d(x, N, C, HW, training=True, gamma_beta=None, rm=None, rv=None, g=None, eps=1e-5,
                momentum=0.1):
    """BatchNorm2D over N samples of C x HW.  Returns (out, rm, rv) or, with
    g (training), (out, rm, rv, grad_in, grad_gamma_beta)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    affine = gamma_beta is not None
    gb = np.ascontiguousarray(gamma_beta if affine else np.zeros(2 * C), np.float32)
    rm = np.zeros(C, np.float32) if rm is None else np.array(rm, np.float32)
    rv = np.ones(C, np.float32) if rv is None else np.array(rv, np.float32)
    out = np.empty(x.size, np.float32)
    gin = np.empty(x.size, np.float32)
    ggb = np.zeros(2 * C, np.float32)
    gg = None if g is None else np.ascontiguousarray(g, np.float32).ravel()
    lib().gno_batchnorm2d(fptr(x), N, C, HW, eps, momentum, int(affine), fptr(gb), int(training),
                          fptr(out), fptr(rm), fptr(rv), None if gg is None else fptr(gg),
                          None if gg is None else fptr(gin), fptr(ggb))
    if gg is None:
        return out, rm, rv
    return out, rm, rv, gin, ggb


def gru_sequence(x, I, H, T, params, g=None):
    """SequenceUnroller(GRU) of one sample; returns h_T, or (h_T, grad_x,
    grad_params) when g (dL/dh_T) is given."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    params = np.ascontiguousarray(params, np.float32).ravel()
    out = np.empty(H, np.float32)
    if g is None:
        lib().gno_gru_sequence(fptr(x), I, H, T, fptr(params), fptr(out), None, None, None)
        return out
    g = np.ascontiguousarray(g, np.float32).ravel()
    gin = np.empty(T * I, np.float32)
    gp = np.zeros(params.size, np.float32)
    lib().gno_gru_sequence(fptr(x), I, H, T, fptr(params), fptr(out), fptr(g), fptr(gin), fptr(gp))
    return out, gin, gp


def moe(x, O, E, K, params, training=False, rng=42, g=None):
    """MoE of one sample; returns (out, active, rng) or, with g,
    (out, active, rng, grad_in, grad_params)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    params = np.ascontiguousarray(params, np.float32).ravel()
    st = C.c_uint64(rng)
    out = np.empty(O, np.float32)
    act = np.empty(K, np.int32)
    gin = np.empty(x.size, np.float32)
    gp = np.zeros(params.size, np.float32)
    gg = None if g is None else np.ascontiguousarray(g, np.float32).ravel()
    rc = lib().gno_moe(fptr(x), x.size, O, E, K, fptr(params), int(training), C.byref(st), fptr(out),
                       iptr(act), None if gg is None else fptr(gg), None if gg is None else fptr(gin),
                       fptr(gp))
    if rc < 0:
        raise ValueError("bad MoE sizes")
    if gg is None:
        return out, act, st.value
    return out, act, st.value, gin, gp


def rope(x, T, nh, hd, conj=False):
    """applyRoPE of x ([T, nh*hd] row major) into a new array."""
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().gno_rope(fptr(y), T, nh, hd, int(conj))
    return y


def matmul(x, w, b):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    B, I = x.shape
    O = w.shape[0]
    out = np.empty((B, O), np.float32)
    lib().gno_matmul(fptr(x), fptr(w), fptr(b), fptr(out), B, I, O)
    return out


def activate_batch(act, x):
    x = np.array(x, np.float32).copy()
    lib().gno_activate_batch(act, fptr(x), x.size)
    return x


def adam_step(params, grads, m, v, lr, b1, b2, eps, timestep):
    lib().gno_adam_step_inplace(fptr(params), fptr(grads), fptr(m), fptr(v), params.size, lr, b1, b2,
                                eps, timestep)


def loss_forward(kind, pred, y):
    pred = np.ascontiguousarray(pred, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    return lib().gno_loss_forward(kind, fptr(pred), fptr(y), pred.size)


def loss_backward(kind, pred, y):
    pred = np.ascontiguousarray(pred, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    g = np.empty_like(pred)
    lib().gno_loss_backward(kind, fptr(pred), fptr(y), fptr(g), pred.size)
    return g
