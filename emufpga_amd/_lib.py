"""ctypes binding of libemuhip.so (the C ABI declared in include/emuhip.h).

The native library is the product: if it is missing this module raises
instead of falling back to any CPU path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libemuhip.so"

# emu_status (include/emuhip.h)
EMU_OK = 0
EMU_E_SHORT = 1
EMU_E_SHAPE = 2
EMU_E_ACTIVATION_LEN = 3
EMU_E_TRUNCATED = 4
EMU_E_UNSUPPORTED = 5
EMU_E_CONTEXT_FULL = 6
EMU_E_CONFIG = 7
EMU_E_HIP = 8
EMU_E_ARG = 9
EMU_E_NOMEM = 10
EMU_E_FORMAT = 11
EMU_E_IO = 12

# GGUF dtype ids (spm-gguf/src/parse.rs:10-29)
F32, F16, Q8_0, Q2_K, Q5_K, Q6_K = 0, 1, 8, 10, 13, 14
ENCODINGS = {"F32": F32, "F16": F16, "Q8_0": Q8_0, "Q2_K": Q2_K, "Q5_K": Q5_K, "Q6_K": Q6_K}

EMU_MV_ACCUMULATE = 1
EMU_MV_LANE_MAJOR = 2
EMU_MV_MFMA_MAJOR = 4
EMU_MV_F32_ACT = 8
EMU_MOE_F32_ACT = 1
EMU_SESSION_F32_ACT = 1
EMU_SESSION_DIRECT = 2
EMU_ROPE_NEOX = 0
EMU_ROPE_INTERLEAVED = 1
EMU_ROPE_NEOX_FMA = 2
EMU_STYLE_QWEN3 = 0
EMU_STYLE_SMOL = 1
EMU_STYLE_GRANITE = 2
(EMU_T_LAYER, EMU_T_EMBED, EMU_T_OUTPUT, EMU_T_ATTN_NORM, EMU_T_FFN_NORM, EMU_T_Q_NORM,
 EMU_T_K_NORM, EMU_T_OUT_NORM, EMU_T_FFN_NORM2) = range(9)


class EmuError(RuntimeError):
    """A non-OK status from the native library."""

    def __init__(self, status: int, what: str, detail: str = ""):
        self.status = status
        msg = f"{what}: {strerror(status)} (status {status})"
        if detail:
            msg += f" [{detail}]"
        super().__init__(msg)


class DecodeError(EmuError):
    """spm-codec-any DecodeError (decode.rs:8-19)."""


class Short(DecodeError):
    """Partial block (tensor.rs:105-107)."""


class Unsupported(DecodeError):
    """Encoding without a decoder (decode.rs:43-45)."""


class LinearError(EmuError):
    """spm-linear LinearError (resident.rs:6-34)."""


class WeightCount(LinearError):
    pass


class ActivationLen(LinearError):
    pass


class Truncated(LinearError):
    pass


class ContextFull(EmuError):
    """KvCache::append on a full context (spm-kv/src/cache.rs:50-54)."""


class ConfigError(EmuError):
    """Configuration errors the reference panics on (attend.rs:82-85)."""


class HipError(EmuError):
    pass


class ArgumentError(EmuError):
    pass


_ERRORS = {
    EMU_E_SHORT: Short,
    EMU_E_SHAPE: WeightCount,
    EMU_E_ACTIVATION_LEN: ActivationLen,
    EMU_E_TRUNCATED: Truncated,
    EMU_E_UNSUPPORTED: Unsupported,
    EMU_E_CONTEXT_FULL: ContextFull,
    EMU_E_CONFIG: ConfigError,
    EMU_E_HIP: HipError,
    EMU_E_ARG: ArgumentError,
    EMU_E_NOMEM: EmuError,
    EMU_E_FORMAT: EmuError,
    EMU_E_IO: EmuError,
}


EMU_ACT_SILU, EMU_ACT_GELU_TANH = 0, 1


class ExpertCacheStats(C.Structure):
    _fields_ = [("hits", C.c_uint64), ("misses", C.c_uint64), ("loads", C.c_uint64), ("evictions", C.c_uint64),
                ("streamed", C.c_uint64), ("bytes_uploaded", C.c_uint64), ("resident", C.c_uint32),
                ("bytes_streamed", C.c_uint64)]


class MoeDesc(C.Structure):
    _fields_ = [
        ("enc_gate_up", C.c_int32), ("enc_down", C.c_int32), ("d_gate", C.c_void_p), ("d_up", C.c_void_p),
        ("d_down", C.c_void_p), ("d_down_scale", C.c_void_p), ("n_experts", C.c_uint32),
        ("width", C.c_uint32), ("ff", C.c_uint32), ("k", C.c_uint32), ("act", C.c_int32),
        ("flags", C.c_uint32),
    ]


class ModelConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("heads", C.c_uint32), ("kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("ffn", C.c_uint32), ("vocab", C.c_uint32),
        ("layers", C.c_uint32), ("rope_theta", C.c_float), ("eps", C.c_float),
        ("style", C.c_int32), ("encoding", C.c_int32), ("tied", C.c_int32),
        ("qk_norm", C.c_int32), ("n_experts", C.c_uint32), ("experts_used", C.c_uint32),
        ("expert_ff", C.c_uint32), ("expert_encoding", C.c_int32), ("embed_scale", C.c_float),
        ("residual_scale", C.c_float), ("logit_div", C.c_float), ("score_mul", C.c_float),
        ("rope_neox", C.c_int32), ("gemma", C.c_int32), ("expert_down_encoding", C.c_int32),
        ("shared_ff", C.c_uint32), ("window", C.c_uint32), ("global_every", C.c_uint32),
        ("rope_theta_global", C.c_float), ("logit_softcap", C.c_float),
    ]


class GgufTensorInfo(C.Structure):
    _fields_ = [("name", C.c_void_p), ("name_len", C.c_size_t), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 8), ("dtype", C.c_uint32),
                ("offset", C.c_uint64), ("len", C.c_uint64)]


class SpmDescriptor(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("cols", C.c_uint32), ("group_size", C.c_uint32), ("encoding", C.c_uint32),
                ("lane_count", C.c_uint32)]


class SpmGroup(C.Structure):
    _fields_ = [("stream", C.c_uint32), ("scale", C.c_float), ("count", C.c_uint32),
                ("packed", C.POINTER(C.c_uint8)), ("packed_len", C.c_size_t)]


P = C.c_void_p
U32 = C.c_uint32
U64 = C.c_uint64
SZ = C.c_size_t
I = C.c_int
F = C.c_float
FP = C.POINTER(C.c_float)

# name -> argtypes; every function returns int (emu_status) unless listed in _RESTYPE
SIGNATURES = {
    "emu_strerror": [I],
    "emu_last_error": [P],
    "emu_ctx_create": [I, C.POINTER(P)],
    "emu_ctx_destroy": [P],
    "emu_ctx_sync": [P],
    "emu_ctx_stream": [P, C.POINTER(P)],
    "emu_device_info": [P, C.POINTER(I), C.c_char_p, SZ],
    "emu_malloc": [P, SZ, C.POINTER(P)],
    "emu_free": [P, P],
    "emu_memcpy_htod": [P, P, P, SZ],
    "emu_memcpy_dtoh": [P, P, P, SZ],
    "emu_memcpy_dtod": [P, P, P, SZ],
    "emu_memset": [P, P, I, SZ],
    "emu_event_record": [P, I],
    "emu_event_elapsed": [P, I, I, FP],
    "emu_block_layout": [I, C.POINTER(U32), C.POINTER(U32)],
    "emu_dequant": [P, I, P, SZ, P],
    "emu_qmatvec": [P, I, P, SZ, U32, U32, P, SZ, U32, P, U32],
    "emu_qmatvec_fused": [P, I, P, P, U32, U32, P, U32, P, F, P, U32],
    "emu_quantize_act": [P, P, U32, U32, P, P],
    "emu_block_dots": [P, I, P, SZ, U32, U32, P, U32, P],
    "emu_qmatvec_i8": [P, I, P, SZ, U32, U32, P, P, U32, P],
    "emu_rms_norm": [P, P, P, U32, U32, F, P],
    "emu_rope_table": [P, U32, U32, F, P],
    "emu_weights_lane_major": [P, I, P, SZ, P],
    "emu_weights_mfma_major": [P, I, P, SZ, U32, U32, P],
    "emu_weights_mfma_major_bytes": [U32, U32],
    "emu_model_sync": [P],
    "emu_host_alloc": [P, SZ, C.POINTER(P)],
    "emu_host_free": [P, P],
    "emu_expert_cache_create": [P, U32, U32, SZ, U32, U32, I, C.POINTER(P)],
    "emu_expert_cache_destroy": [P],
    "emu_expert_cache_set_source": [P, U32, U32, P],
    "emu_expert_cache_stats": [P, P],
    "emu_expert_cache_slot": [P, U32, U32, P],
    "emu_moe_ffn_cached": [P, P, P, U32, P, U32, P, P, P, P, SZ, P],
    "emu_expert_cache_policy_trace": [U32, I, P, P, P, U32, P, P],
    "emu_session_route_zipf": [P, F, C.c_uint64],
    "emu_session_set_options": [P, U32],
    "emu_session_time_layers": [P, P, U32],
    "emu_model_resident_bytes": [P, C.POINTER(C.c_uint64)],
    "emu_session_attach_expert_cache": [P, P],
    "emu_host_device_pointer": [P, P, C.POINTER(P)],
    "emu_expert_cache_load_model": [P, P, P, SZ],
    "emu_hbm_read_rate": [P, P, SZ, U32, P],
    "emu_session_route_trace": [P, U32],
    "emu_session_read_routes": [P, U32, P, P],
    "emu_model_tensor_lane_major": [P, I, U32, C.POINTER(P), C.POINTER(SZ)],
    "emu_rope_table_style": [P, I, U32, U32, F, P],
    "emu_rope": [P, P, U32, U32, U32, P, P, U32, I],
    "emu_attend_cached": [P, P, P, P, I, U32, U32, U32, U32, F, P],
    "emu_attend_cached_noalloc": [P, P, P, P, I, U32, U32, U32, U32, F, P],
    "emu_route": [P, P, U32, U32, U32, P, P],
    "emu_argmax": [P, P, U32, U32, I, P],
    "emu_moe_workspace_bytes": [U32, U32, U32, U32],
    "emu_moe_ffn": [P, C.POINTER(MoeDesc), P, U32, P, P, P, SZ, P],
    "emu_model_create": [P, C.POINTER(ModelConfig), C.POINTER(P)],
    "emu_model_destroy": [P],
    "emu_model_tensor": [P, I, U32, C.POINTER(P), C.POINTER(SZ)],
    "emu_model_synth": [P, C.c_uint64],
    "emu_model_weight_bytes": [P, C.POINTER(C.c_uint64)],
    "emu_session_create": [P, U32, U32, I, C.POINTER(P)],
    "emu_session_destroy": [P],
    "emu_session_reset": [P],
    "emu_session_reset_client": [P, U32],
    "emu_decode_step": [P, P, P, P],
    "emu_generate": [P, P, U32, U32, P],
    "emu_time_decode": [P, U32, FP],
    "emu_session_positions": [P, P],
    "emu_session_read_kv": [P, U32, U32, I, P, U32],
    "emu_gguf_open": [C.c_char_p, C.POINTER(P), C.c_char_p, SZ],
    "emu_gguf_close": [P],
    "emu_gguf_error": [P],
    "emu_gguf_summary": [P, C.POINTER(U32), C.POINTER(U64), C.POINTER(U64), C.POINTER(U64)],
    "emu_gguf_metadata_at": [P, U64, C.POINTER(P), C.POINTER(SZ), C.POINTER(P), C.POINTER(SZ)],
    "emu_gguf_metadata_number": [P, C.c_char_p, C.POINTER(C.c_double)],
    "emu_gguf_tensor_at": [P, U64, C.POINTER(GgufTensorInfo)],
    "emu_gguf_find": [P, C.c_char_p, C.POINTER(U64)],
    "emu_gguf_read_range": [P, U64, U64, U64, U64, P],
    "emu_gguf_upload": [P, P, U64, U64, U64, P],
    "emu_model_load_gguf": [P, P],
    "emu_spm_bytes_for": [U32, U64, C.POINTER(U64)],
    "emu_spm_parse": [P, SZ, C.POINTER(P), C.c_char_p, SZ],
    "emu_spm_close": [P],
    "emu_spm_error": [P],
    "emu_spm_header": [P, C.POINTER(C.c_uint16), C.POINTER(C.c_uint16), C.POINTER(U32)],
    "emu_spm_descriptor_at": [P, U32, C.POINTER(SpmDescriptor)],
    "emu_spm_position": [P, C.POINTER(U32), C.POINTER(U64)],
    "emu_spm_next_group": [P, C.POINTER(I), C.POINTER(SpmGroup)],
    "emu_spm_upload_stream": [P, P, P, SZ, C.POINTER(U32)],
    "emu_spm_writer_create": [C.POINTER(SpmDescriptor), U32, C.POINTER(P)],
    "emu_spm_write_raw_group": [P, F, P, SZ, U64],
    "emu_spm_writer_finish": [P, C.POINTER(C.POINTER(C.c_uint8)), C.POINTER(SZ)],
    "emu_spm_writer_error": [P],
    "emu_spm_writer_destroy": [P],
}
_RESTYPE = {"emu_strerror": C.c_char_p, "emu_last_error": C.c_char_p, "emu_moe_workspace_bytes": C.c_size_t,
            "emu_weights_mfma_major_bytes": C.c_size_t,
            "emu_gguf_error": C.c_char_p, "emu_spm_error": C.c_char_p, "emu_spm_writer_error": C.c_char_p}

_lib = None


def load() -> C.CDLL:
    """Load libemuhip.so (built by ``python -m emufpga_amd.build``)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m emufpga_amd.build` "
            "(the HIP library is the only implementation; there is no fallback)")
    lib = C.CDLL(str(LIB_PATH))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, C.c_int)
    _lib = lib
    return lib


def strerror(status: int) -> str:
    return load().emu_strerror(status).decode()


def check(status: int, what: str, ctx=None) -> None:
    if status == EMU_OK:
        return
    detail = ""
    if ctx is not None:
        try:
            detail = load().emu_last_error(ctx).decode()
        except Exception:  # pragma: no cover - diagnostic only
            detail = ""
    raise _ERRORS.get(status, EmuError)(status, what, detail)
