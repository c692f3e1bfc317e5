"""ctypes binding of libgoneuron_hip.so (the C ABI in include/goneuron_hip.h).

The library is the only compute path: if it is missing, loading fails with an
error that says how to build it.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgoneuron_hip.so")

GN_OK = 0
ERRORS = {
    -1: "GN_ERR_INVALID", -2: "GN_ERR_HIP", -3: "GN_ERR_OOM", -4: "GN_ERR_UNSUPPORTED",
    -5: "GN_ERR_SHAPE", -6: "GN_ERR_INJECTED", -7: "GN_ERR_NO_DEVICE", -8: "GN_ERR_INDEX",
}


class GNError(RuntimeError):
    def __init__(self, code, msg=""):
        self.code = code
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")


class LayerDesc(C.Structure):
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


class AdamDesc(C.Structure):
    _fields_ = [("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float)]


class KernelStat(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("cls", C.c_int32), ("launches", C.c_int64), ("ms", C.c_double),
                ("units", C.c_double)]


class Info(C.Structure):
    _fields_ = [("arch", C.c_char * 64), ("cu_count", C.c_int32), ("hbm_bytes", C.c_int64),
                ("peak_fp32_mfma_tflops", C.c_double), ("peak_hbm_gbps", C.c_double)]


f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int32)
vp = C.c_void_p

# name -> (restype, argtypes)
SIGNATURES = {
    "gn_available": (C.c_int, []),
    "gn_init": (C.c_int, [C.c_int, C.POINTER(vp)]),
    "gn_shutdown": (None, [vp]),
    "gn_last_error": (C.c_char_p, [vp]),
    "gn_device_info": (C.c_int, [vp, C.POINTER(Info)]),
    "gn_sync": (C.c_int, [vp]),
    "gn_debug_fail_next": (C.c_int, [vp, C.c_int]),
    "gn_debug_lstm_spin_limit": (C.c_int, [vp, C.c_int32]),
    "gn_debug_lstm_clip_bail": (C.c_int, [vp, C.c_int32]),
    "gn_debug_fused_tail": (C.c_int, [vp, C.c_int32]),
    "gn_debug_step_update": (C.c_int, [vp, C.c_int32]),
    "gn_debug_side_streams": (C.c_int, [vp, C.c_int32]),
    "gn_malloc": (C.c_int, [vp, C.c_size_t, C.POINTER(vp)]),
    "gn_free": (C.c_int, [vp, vp]),
    "gn_memcpy_h2d": (C.c_int, [vp, vp, vp, C.c_size_t]),
    "gn_memcpy_d2h": (C.c_int, [vp, vp, vp, C.c_size_t]),
    "gn_memset_zero": (C.c_int, [vp, vp, C.c_size_t]),
    "gn_model_create": (C.c_int, [vp, C.POINTER(LayerDesc), C.c_int32, C.c_int32, C.POINTER(AdamDesc),
                                  C.c_int32, C.c_int32, C.POINTER(vp)]),
    "gn_model_destroy": (None, [vp]),
    "gn_model_nparams": (C.c_int, [vp, C.POINTER(C.c_int64)]),
    "gn_model_layer_params": (C.c_int, [vp, C.c_int32, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "gn_model_out_size": (C.c_int, [vp, i32p]),
    "gn_model_layer_count": (C.c_int, [vp, i32p]),
    "gn_model_layer_desc": (C.c_int, [vp, C.c_int32, C.POINTER(LayerDesc)]),
    "gn_model_loss_kind": (C.c_int, [vp, i32p]),
    "gn_model_get_params": (C.c_int, [vp, f32p, C.c_int64, C.c_int64]),
    "gn_model_set_params": (C.c_int, [vp, f32p, C.c_int64, C.c_int64]),
    "gn_model_get_grads": (C.c_int, [vp, f32p, C.c_int64, C.c_int64]),
    "gn_model_get_adam": (C.c_int, [vp, f32p, f32p, C.c_int64, C.c_int64, i32p]),
    "gn_model_arena": (C.c_int, [vp, C.POINTER(vp), C.POINTER(vp), C.POINTER(vp), C.POINTER(vp)]),
    "gn_model_train_step": (C.c_int, [vp, f32p, f32p, C.c_int32, f32p]),
    "gn_model_train_step_device": (C.c_int, [vp, vp, vp, C.c_int32]),
    "gn_model_accumulate_device": (C.c_int, [vp, vp, vp, C.c_int32]),
    "gn_model_step": (C.c_int, [vp]),
    "gn_model_read_loss": (C.c_int, [vp, f32p]),
    "gn_model_predict": (C.c_int, [vp, f32p, C.c_int32, f32p]),
    "gn_model_predict_device": (C.c_int, [vp, vp, C.c_int32, vp]),
    "gn_model_set_training": (C.c_int, [vp, C.c_int32]),
    "gn_model_get_training": (C.c_int, [vp, C.c_int32, i32p]),
    "gn_model_reserve": (C.c_int, [vp, C.c_int32]),
    "gn_model_set_graphs": (C.c_int, [vp, C.c_int32]),
    "gn_model_graph_count": (C.c_int, [vp, i32p]),
    "gn_model_skipped_samples": (C.c_int, [vp, i32p]),
    "gn_model_layer_output": (C.c_int, [vp, C.c_int32, f32p, C.c_int64]),
    "gn_model_layer_argmax": (C.c_int, [vp, C.c_int32, i32p, C.c_int64]),
    "gn_model_get_running_stats": (C.c_int, [vp, C.c_int32, f32p, f32p, C.c_int32]),
    "gn_model_set_adam": (C.c_int, [vp, f32p, f32p, C.c_int64, C.c_int64, C.c_int32]),
    "gn_model_save_binary_weights": (C.c_int, [vp, C.c_char_p]),
    "gn_model_load_binary_weights": (C.c_int, [vp, C.c_char_p]),
    "gn_model_save_gguf": (C.c_int, [vp, C.c_char_p, C.c_int32]),
    "gn_model_save_state": (C.c_int, [vp, C.c_char_p]),
    "gn_model_load_state": (C.c_int, [vp, C.c_char_p]),
    "gn_model_save_gob": (C.c_int, [vp, C.c_char_p]),
    "gn_model_load_gob": (C.c_int, [vp, C.c_char_p, C.c_int32, C.c_int32, C.c_int32, C.POINTER(vp), i32p]),
    "gn_model_set_running_stats": (C.c_int, [vp, C.c_int32, f32p, f32p, C.c_int32]),
    "gn_dense_forward": (C.c_int, [vp, vp, vp, vp, vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                   C.c_int32]),
    "gn_dense_backward": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, vp, C.c_int32, C.c_int32,
                                    C.c_int32, C.c_int32, C.c_int32, C.c_float]),
    "gn_dense_backward_noalloc": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, C.c_int32, C.c_int32,
                                            C.c_int32, C.c_int32, C.c_int32, C.c_float]),
    "gn_conv2d_forward": (C.c_int, [vp, vp, vp, vp] + [C.c_int32] * 9),
    "gn_conv2d_backward": (C.c_int, [vp] + [vp] * 6 + [C.c_int32] * 9 + [C.c_float]),
    "gn_maxpool2d_forward": (C.c_int, [vp, vp, vp, vp] + [C.c_int32] * 7),
    "gn_maxpool2d_backward": (C.c_int, [vp, vp, vp, vp] + [C.c_int32] * 7),
    "gn_dropout_forward": (C.c_int, [vp, vp, vp, vp, C.c_int32, C.c_int32, C.c_float, C.c_int32]),
    "gn_dropout_backward": (C.c_int, [vp, vp, vp, vp, C.c_int32, C.c_int32, C.c_float, C.c_int32]),
    "gn_softmax_ce_backward": (C.c_int, [vp, vp, vp, vp, vp] + [C.c_int32] * 5),
    "gn_layernorm_forward": (C.c_int, [vp] + [vp] * 5 + [C.c_int32, C.c_int32, C.c_float]),
    "gn_layernorm_backward": (C.c_int, [vp] + [vp] * 8 + [C.c_int32, C.c_int32, C.c_float]),
    "gn_mha_workspace": (C.c_int, [C.c_int32] * 5 + [C.POINTER(C.c_int64)]),
    "gn_mha_forward": (C.c_int, [vp] + [vp] * 4 + [C.c_int32] * 6),
    "gn_mha_backward": (C.c_int, [vp] + [vp] * 6 + [C.c_int32] * 6 + [C.c_float]),
    "gn_lstm_workspace": (C.c_int, [C.c_int32] * 5 + [C.POINTER(C.c_int64)]),
    "gn_lstm_seq_forward": (C.c_int, [vp] + [vp] * 4 + [C.c_int32] * 5),
    "gn_lstm_seq_backward": (C.c_int, [vp] + [vp] * 6 + [C.c_int32] * 5 + [C.c_float, C.c_int32]),
    "gn_embedding_forward": (C.c_int, [vp] + [vp] * 5 + [C.c_int32] * 4),
    "gn_embedding_backward": (C.c_int, [vp] + [vp] * 4 + [C.c_int32] * 5 + [C.c_float]),
    "gn_avgpool2d_forward": (C.c_int, [vp] + [vp] * 2 + [C.c_int32] * 7),
    "gn_avgpool2d_backward": (C.c_int, [vp] + [vp] * 2 + [C.c_int32] * 7),
    "gn_rmsnorm_forward": (C.c_int, [vp] + [vp] * 4 + [C.c_int32, C.c_int32, C.c_float]),
    "gn_rmsnorm_backward": (C.c_int, [vp] + [vp] * 7 + [C.c_int32, C.c_int32, C.c_float]),
    "gn_swiglu_workspace": (C.c_int, [C.c_int32, C.c_int32, C.POINTER(C.c_int64)]),
    "gn_swiglu_forward": (C.c_int, [vp] + [vp] * 4 + [C.c_int32] * 3),
    "gn_swiglu_backward": (C.c_int, [vp] + [vp] * 6 + [C.c_int32] * 3 + [C.c_float]),
    "gn_batchnorm2d_forward": (C.c_int, [vp] + [vp] * 6 + [C.c_int32] * 3 + [C.c_float, C.c_float, C.c_int32]),
    "gn_batchnorm2d_backward": (C.c_int, [vp] + [vp] * 8 + [C.c_int32] * 3 + [C.c_float, C.c_int32, C.c_float]),
    "gn_gru_workspace": (C.c_int, [C.c_int32] * 4 + [C.POINTER(C.c_int64)]),
    "gn_gru_seq_forward": (C.c_int, [vp] + [vp] * 4 + [C.c_int32] * 5),
    "gn_gru_seq_backward": (C.c_int, [vp] + [vp] * 6 + [C.c_int32] * 4 + [C.c_float, C.c_int32]),
    "gn_moe_workspace": (C.c_int, [C.c_int32] * 5 + [C.POINTER(C.c_int64)]),
    "gn_moe_forward": (C.c_int, [vp] + [vp] * 4 + [C.c_int32] * 6 + [C.POINTER(C.c_uint64)]),
    "gn_moe_backward": (C.c_int, [vp] + [vp] * 6 + [C.c_int32] * 6 + [C.c_float]),
    "gn_gemm": (C.c_int, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_float, vp,
                          C.c_int32, vp, C.c_int32, vp, C.c_int32]),
    "gn_adam_step": (C.c_int, [vp, vp, vp, vp, vp, C.c_int64, C.c_float, C.c_float, C.c_float,
                               C.c_float, C.c_int32]),
    "gn_fill_uniform": (C.c_int, [f32p, C.c_int64, C.c_uint64]),
    "gn_fill_normal": (C.c_int, [f32p, C.c_int64, C.c_uint64]),
    "gn_fill_class_ids": (C.c_int, [i32p, C.c_int64, C.c_int32, C.c_uint64]),
    "gn_timing_enable": (C.c_int, [vp, C.c_int]),
    "gn_timing_report": (C.c_int, [vp, C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_double)]),
    "gn_timing_kernels": (C.c_int, [vp, C.POINTER(KernelStat), C.c_int32, i32p]),
    "gn_timing_floor": (C.c_int, [vp, C.c_int32, C.c_int32]),
}

_lib = None


def lib():
    """Loads the in-tree library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m goneuron_amd.build` "
                "(hipcc, gfx950). goneuron_amd has no CPU fallback.")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(ctx, rc):
    if rc != GN_OK:
        msg = lib().gn_last_error(ctx) if ctx else b""
        raise GNError(rc, (msg or b"").decode(errors="replace"))
    return rc
