"""ctypes binding of libcpb_moe.so (the C ABI in include/cpb_moe.h,
include/cpb_gguf.h, include/cpb_head.h, include/cpb_attn.h and include/cpb_synth.h).  Loading fails loudly when the library is missing: there
is no CPU fallback for the HIP path."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libcpb_moe.so"

f32p = C.POINTER(C.c_float)
i8p = C.POINTER(C.c_int8)
i32p = C.POINTER(C.c_int32)
u8p = C.POINTER(C.c_uint8)

CPB_OK, CPB_EINVAL, CPB_ENOMEM, CPB_ENODEV, CPB_ESTATE = 0, -22, -12, -19, -71
ROUTER_TOPK_SOFTMAX, ROUTER_SOFTMAX_TOPK = 0, 1
ACT_SWIGLU_OAI, ACT_SILU = 0, 1
NORM_GPTOSS, NORM_QWEN = 0, 1
GGUF_MXFP4, GGUF_Q4_K, GGUF_Q6_K = 39, 12, 14


class MoeCfg(C.Structure):
    _fields_ = [("d", C.c_int), ("n_expert", C.c_int), ("top_k", C.c_int), ("d_ff", C.c_int),
                ("n_layer", C.c_int), ("router", C.c_int), ("act", C.c_int), ("norm", C.c_int),
                ("norm_nt", C.c_int), ("alpha", C.c_float), ("limit", C.c_float), ("rms_eps", C.c_float),
                ("wtype_gate_up", C.c_int), ("wtype_down", C.c_int), ("has_bias", C.c_int),
                ("max_tokens", C.c_int)]


class MoeTrace(C.Structure):
    _fields_ = [("xn", f32p), ("xq", i8p), ("xsb", f32p), ("xsum", i32p), ("logits", f32p),
                ("ids", i32p), ("wts", f32p), ("gu", f32p), ("gu_sums", i32p), ("h", f32p), ("hq", i8p),
                ("hsb", f32p), ("hsum", i32p), ("dn", f32p), ("dn_sums", i32p),
                ("exact_router_fallbacks", C.c_int32)]


class GgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_int32), ("n_dims", C.c_int32), ("dims", C.c_uint64 * 4),
                ("n_elements", C.c_uint64), ("offset", C.c_uint64), ("n_bytes", C.c_uint64), ("data", C.c_void_p)]


class GgufHparams(C.Structure):
    _fields_ = [("arch", C.c_char * 32), ("n_embd", C.c_int64), ("n_layer", C.c_int64), ("n_head", C.c_int64),
                ("n_head_kv", C.c_int64), ("head_dim", C.c_int64), ("n_expert", C.c_int64),
                ("n_expert_used", C.c_int64), ("n_ff_exp", C.c_int64), ("sliding_window", C.c_int64),
                ("n_vocab", C.c_int64), ("context_length", C.c_int64), ("rope_freq_base", C.c_double),
                ("rms_eps", C.c_double)]


class HeadCfg(C.Structure):
    _fields_ = [("d", C.c_int), ("n_vocab", C.c_int), ("n_slices", C.c_int), ("n_cand", C.c_int),
                ("rms_eps", C.c_float)]


class HeadTrace(C.Structure):
    _fields_ = [("cand_ids", i32p), ("cand_screen", f32p), ("cand_logits", f32p), ("xq", i8p), ("xsb", f32p),
                ("screen", f32p)]


class AttnCfg(C.Structure):
    _fields_ = [("d", C.c_int), ("n_head", C.c_int), ("n_head_kv", C.c_int), ("head_dim", C.c_int),
                ("n_layer", C.c_int), ("max_seq", C.c_int), ("sliding_window", C.c_int), ("rope_base", C.c_float),
                ("rms_eps", C.c_float)]


class AttnTrace(C.Structure):
    _fields_ = [("xq", i8p), ("xsb", f32p), ("q", f32p), ("k", f32p), ("v", f32p), ("ao", f32p), ("aq", i8p),
                ("asb", f32p)]


# every symbol the public headers declare, with its ctypes signature
SIGNATURES = {
    "cpb_moe_create": (C.c_int, [C.POINTER(MoeCfg), C.c_int, C.POINTER(C.c_void_p)]),
    "cpb_moe_load_layer": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                     f32p, f32p, f32p, f32p, f32p, f32p]),
    "cpb_moe_load_layer_typed": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                           C.c_void_p, f32p, f32p, f32p, f32p, f32p, f32p]),
    "cpb_moe_forward": (C.c_int, [C.c_void_p, C.c_int, f32p, C.c_int, C.c_int, C.POINTER(MoeTrace)]),
    "cpb_moe_forward_device": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int]),
    "cpb_moe_forward_device_noalloc": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int]),
    "cpb_moe_set_stream": (C.c_int, [C.c_void_p, C.c_void_p]),
    "cpb_moe_sync": (C.c_int, [C.c_void_p]),
    "cpb_moe_destroy": (None, [C.c_void_p]),
    "cpb_moe_last_error": (C.c_char_p, []),
    "cpb_moe_layer_bytes": (C.c_int, [C.POINTER(MoeCfg), C.POINTER(C.c_size_t)]),
    "cpb_moe_timing": (C.c_int, [C.c_void_p, C.c_int]),
    "cpb_moe_kernel_times": (C.c_int, [C.c_void_p, C.POINTER(C.c_double), C.POINTER(C.c_long)]),
    "cpb_moe_grouped_sums": (C.c_int, [C.c_void_p, C.c_int, f32p, C.c_int, C.c_int, i32p, i32p]),
    "cpb_moe_config": (C.c_int, [C.c_void_p, C.POINTER(MoeCfg)]),
    "cpb_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "cpb_gguf_close": (None, [C.c_void_p]),
    "cpb_gguf_version": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "cpb_gguf_n_tensors": (C.c_int, [C.c_void_p, C.POINTER(C.c_int64)]),
    "cpb_gguf_tensor_at": (C.c_int, [C.c_void_p, C.c_int64, C.POINTER(GgufTensor)]),
    "cpb_gguf_find": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(GgufTensor)]),
    "cpb_gguf_meta_i64": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_int64)]),
    "cpb_gguf_meta_f64": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_double)]),
    "cpb_gguf_meta_str": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_char_p)]),
    "cpb_gguf_hparams_get": (C.c_int, [C.c_void_p, C.POINTER(GgufHparams)]),
    "cpb_gguf_write_manifest": (C.c_int, [C.c_void_p, C.c_char_p]),
    "cpb_moe_load_gguf_layer": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int]),
    "cpb_head_create": (C.c_int, [C.POINTER(HeadCfg), C.c_int, C.POINTER(C.c_void_p)]),
    "cpb_head_load": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint16), f32p]),
    "cpb_head_forward": (C.c_int, [C.c_void_p, f32p, i32p, C.POINTER(HeadTrace)]),
    "cpb_head_forward_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "cpb_head_set_screen": (C.c_int, [C.c_void_p, C.c_int]),
    "cpb_head_set_stream": (C.c_int, [C.c_void_p, C.c_void_p]),
    "cpb_head_sync": (C.c_int, [C.c_void_p]),
    "cpb_head_destroy": (None, [C.c_void_p]),
    "cpb_head_bytes": (C.c_int, [C.POINTER(HeadCfg), C.POINTER(C.c_size_t)]),
    "cpb_attn_create": (C.c_int, [C.POINTER(AttnCfg), C.c_int, C.POINTER(C.c_void_p)]),
    "cpb_attn_load_layer": (C.c_int, [C.c_void_p, C.c_int, f32p, C.POINTER(C.c_uint16), C.POINTER(C.c_uint16), C.POINTER(C.c_uint16), C.POINTER(C.c_uint16),
                                      f32p, f32p, f32p, f32p, f32p]),
    "cpb_attn_forward": (C.c_int, [C.c_void_p, C.c_int, C.c_int, f32p, C.POINTER(AttnTrace)]),
    "cpb_attn_forward_device": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "cpb_attn_reset": (C.c_int, [C.c_void_p]),
    "cpb_attn_set_stream": (C.c_int, [C.c_void_p, C.c_void_p]),
    "cpb_attn_sync": (C.c_int, [C.c_void_p]),
    "cpb_attn_destroy": (None, [C.c_void_p]),
    "cpb_synth_u64": (C.c_uint64, [C.c_uint64, C.c_uint64, C.c_uint64]),
    "cpb_synth_mxfp4": (None, [u8p, C.c_size_t, C.c_int, C.c_int, C.c_uint64, C.c_uint64]),
    "cpb_synth_normal": (None, [f32p, C.c_size_t, C.c_float, C.c_float, C.c_uint64, C.c_uint64]),
    "cpb_synth_q4k": (None, [u8p, C.c_size_t, C.c_float, C.c_uint64, C.c_uint64]),
    "cpb_synth_q6k": (None, [u8p, C.c_size_t, C.c_float, C.c_uint64, C.c_uint64]),
    "cpb_synth_zipf_bias": (None, [f32p, C.c_int, C.c_float, C.c_uint64, C.c_uint64]),
    "cpb_f32_to_half": (C.c_uint16, [C.c_float]),
}

_LIB = None


class CpbError(RuntimeError):
    def __init__(self, code: int, where: str, msg: str):
        super().__init__(f"{where} failed ({code}): {msg}")
        self.code = code


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m cpubrrr_amd.build` (hipcc, gfx950)")
        # One HIP runtime per process: PyTorch-ROCm ships its own
        # libamdhip64.so.7.  Loaded after ours, torch would bind to the system
        # runtime already in the process and find no device; loaded first, the
        # library binds to torch's copy.  So torch (when installed) goes first.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(code: int, where: str) -> None:
    if code != 0:
        raise CpbError(code, where, lib().cpb_moe_last_error().decode(errors="replace"))
