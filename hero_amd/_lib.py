"""ctypes binding of libhero_amd.so (include/hero_kernels.h, include/hero_model.h,
include/hero_gemma4.h).

The library is built in-tree (``python -c "import __graft_entry__ as g; g.build()"``
or ``make -C hero_amd``). There is no CPU fallback: if the library is missing,
importing this module raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint64, c_void_p

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhero_amd.so")

HERO_OK, HERO_EINVAL, HERO_EHIP, HERO_ERANGE, HERO_ENOMEM, HERO_EIO = range(6)
HERO_STATE_KV_FP16 = 1  # hero_batch_state_create flag: fp16 paged attention cache
HERO_STATE_GDN_CHUNKED = 2  # hero_batch_state_create flag: chunked delta-net prefill
HERO_STATE_KV_Q8_0 = 4  # hero_batch_state_create flag: Q8_0 paged attention cache


class HeroError(RuntimeError):
    """A non-zero status from the C ABI; .code is the HERO_E* value."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class ContextExhausted(HeroError):
    """HERO_ERANGE: the reference's std::length_error (nm/src/qwen35.hpp:289)."""


class GdnDecodeArgs(ctypes.Structure):
    _fields_ = [
        ("proj", c_void_p), ("proj_stride", c_int64), ("z_off", c_int64), ("beta_off", c_int64), ("alpha_off", c_int64),
        ("conv_taps", c_void_p), ("conv_hist", c_void_p), ("state", c_void_p), ("dt_bias", c_void_p), ("decay", c_void_p),
        ("norm_gamma", c_void_p), ("eps", c_float), ("positions", c_void_p), ("act_out", c_void_p), ("out_f32", c_void_p),
        ("b", c_int32), ("hk", c_int32), ("hv", c_int32), ("dk", c_int32), ("dv", c_int32), ("conv_width", c_int32),
    ]


class AttnDecodeArgs(ctypes.Structure):
    _fields_ = [
        ("proj", c_void_p), ("proj_stride", c_int64), ("k_off", c_int64), ("v_off", c_int64),
        ("q_gamma", c_void_p), ("k_gamma", c_void_p), ("eps", c_float), ("rope_cs", c_void_p),
        ("k_cache", c_void_p), ("v_cache", c_void_p), ("max_ctx", c_int64), ("positions", c_void_p),
        ("scores", c_void_p), ("q_rot", c_void_p), ("score_scale", c_float), ("window", c_int32), ("act_out", c_void_p), ("out_f32", c_void_p),
        ("b", c_int32), ("hq", c_int32), ("hkv", c_int32), ("dh", c_int32),
    ]


class AttnPagedArgs(ctypes.Structure):
    _fields_ = [
        ("a", AttnDecodeArgs), ("pages", c_void_p), ("page_table", c_void_p),
        ("page_size", c_int32), ("max_pages", c_int32), ("work", c_void_p), ("work_bytes", c_int64),
        ("q8", c_int32),
    ]


class ModelDims(ctypes.Structure):
    _fields_ = [
        ("vocab", c_int64), ("d_model", c_int64), ("layers", c_int64), ("ctx", c_int64),
        ("q_heads", c_int64), ("kv_heads", c_int64), ("head_dim", c_int64), ("rotary_dims", c_int64),
        ("key_head_dim", c_int64), ("value_head_dim", c_int64), ("key_heads", c_int64), ("value_heads", c_int64),
        ("conv_width", c_int64), ("ffn", c_int64), ("tied", c_int64), ("rope_base", c_double), ("rms_eps", c_float),
        ("device_bytes", c_int64),
    ]


class SynthConfig(ctypes.Structure):
    _fields_ = [
        ("vocab", c_int64), ("d_model", c_int64), ("layers", c_int64), ("ffn", c_int64),
        ("q_heads", c_int64), ("kv_heads", c_int64), ("head_dim", c_int64),
        ("key_head_dim", c_int64), ("value_head_dim", c_int64), ("key_heads", c_int64), ("value_heads", c_int64),
        ("conv_width", c_int64), ("ctx", c_int64), ("rope_base", c_double), ("tied", c_int32), ("seed", c_uint64),
        ("weight_mix", c_int32),
    ]


class Gemma4Dims(ctypes.Structure):
    _fields_ = [
        ("vocab", c_int64), ("d_model", c_int64), ("layers", c_int64), ("ctx", c_int64), ("ffn", c_int64),
        ("q_heads", c_int64), ("kv_heads", c_int64), ("local_head_dim", c_int64), ("full_head_dim", c_int64),
        ("per_layer_input", c_int64), ("window", c_int64), ("shared_kv_layers", c_int64),
        ("rms_eps", c_float), ("logit_softcap", c_float), ("device_bytes", c_int64),
    ]


class Gemma4SynthConfig(ctypes.Structure):
    _fields_ = [
        ("vocab", c_int64), ("d_model", c_int64), ("layers", c_int64), ("ffn", c_int64),
        ("q_heads", c_int64), ("kv_heads", c_int64), ("local_head_dim", c_int64), ("full_head_dim", c_int64),
        ("per_layer_input", c_int64), ("window", c_int64), ("shared_kv_layers", c_int64), ("ctx", c_int64),
        ("seed", c_uint64),
    ]


# name -> (restype, argtypes); every symbol of include/hero_*.h
SIGNATURES = {
    "hero_last_error": (c_char_p, []),
    "hero_version": (c_char_p, []),
    "hero_q8_0_packed_bytes": (c_int64, [c_int64, c_int64]),
    "hero_q8_0_act_bytes": (c_int64, [c_int64, c_int64]),
    "hero_q8_0_pack": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "hero_q8_0_quantize": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "hero_q8_0_gemv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "hero_rmsnorm_q8_0_gemv": (c_int, [c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "hero_swiglu_q8_0_gemv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "hero_q8_0_pack_interleaved": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "hero_rmsnorm_q8_0_gemv_swiglu": (c_int, [c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_int64, c_int64, c_void_p]),
    "hero_q8_0_gemm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "hero_q8_0_gemm_plan": (c_int, [c_int64, c_int64, c_int64, c_void_p]),
    "hero_q8_0_block_sums": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "hero_rmsnorm_quant": (c_int, [c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "hero_swiglu_quant": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "hero_q8_0_embed": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p]),
    "hero_argmax": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p]),
    "hero_argmax_noalloc": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "hero_math_eval": (c_int, [c_void_p, c_void_p, c_int64, c_void_p]),
    "hero_sample_topk": (c_int, [c_void_p, c_int64, c_int32, c_float, c_float, c_float, c_void_p, c_void_p]),
    "hero_sample_work_bytes": (c_int64, [c_int64]),
    "hero_sample": (c_int, [c_void_p, c_int64, c_int32, c_float, c_float, c_float, c_void_p, c_int64, c_void_p, c_void_p]),
    "hero_q8_K_act_bytes": (c_int64, [c_int64, c_int64]),
    "hero_q8_K_quantize": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "hero_kquant_gemm": (c_int, [c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "hero_kquant_packed_bytes": (c_int64, [c_int32, c_int64, c_int64]),
    "hero_kquant_pack": (c_int, [c_int32, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "hero_q5_K_gemm": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "hero_kquant_dequant_rows": (c_int, [c_int32, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p]),
    "hero_gdn_decode": (c_int, [POINTER(GdnDecodeArgs), c_void_p]),
    "hero_gdn_decode_cols": (c_int, [POINTER(GdnDecodeArgs), c_void_p, c_void_p, c_void_p]),
    "hero_gdn_norm_gate": (c_int, [c_void_p, POINTER(GdnDecodeArgs), c_void_p]),
    "hero_headgate_q8_0_gemv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "hero_gdn_prefill_work_bytes": (c_int64, [c_int64, c_int32, c_int32]),
    "hero_gdn_prefill": (c_int, [POINTER(GdnDecodeArgs), c_void_p, c_int64, c_void_p]),
    "hero_gdn_prefill_chunked": (c_int, [POINTER(GdnDecodeArgs), c_void_p, c_int64, c_void_p]),
    "hero_attn_decode": (c_int, [POINTER(AttnDecodeArgs), c_void_p]),
    "hero_attn_prefill": (c_int, [POINTER(AttnDecodeArgs), c_void_p]),
    "hero_attn_paged_work_bytes": (c_int64, [c_int64, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "hero_attn_page_bytes": (c_int64, [c_int32, c_int32, c_int32, c_int32]),
    "hero_read_probe": (c_int, [c_void_p, c_int64, c_int32, c_void_p, c_void_p]),
    "hero_q8_0_gemv_prefetch": (c_int, [c_void_p, c_int64, c_int64, c_void_p]),
    "hero_attn_decode_paged": (c_int, [POINTER(AttnPagedArgs), c_void_p]),
    "hero_model_open": (c_int, [c_char_p, POINTER(c_void_p)]),
    "hero_model_open_image": (c_int, [c_void_p, c_size_t, POINTER(c_void_p)]),
    "hero_model_close": (None, [c_void_p]),
    "hero_model_dims_get": (c_int, [c_void_p, POINTER(ModelDims)]),
    "hero_state_create": (c_int, [c_void_p, c_int64, POINTER(c_void_p)]),
    "hero_state_destroy": (None, [c_void_p]),
    "hero_state_reset": (c_int, [c_void_p]),
    "hero_state_tokens": (c_int64, [c_void_p]),
    "hero_batch_state_create": (c_int, [c_void_p, c_int64, c_int32, ctypes.c_uint32, POINTER(c_void_p)]),
    "hero_state_batch": (c_int64, [c_void_p]),
    "hero_state_seq_tokens": (c_int64, [c_void_p, c_int32]),
    "hero_model_forward_seq": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "hero_model_decode_batch": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "hero_model_embed": (c_int, [c_void_p, c_void_p, c_int64, c_void_p]),
    "hero_model_forward": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "hero_model_decode_greedy": (c_int, [c_void_p, c_void_p, c_int32, c_int64, c_void_p, c_void_p]),
    "hero_model_last_decode_seconds": (c_double, [c_void_p]),
    "hero_model_time_gemvs": (c_int, [c_void_p, c_void_p, c_int32, POINTER(c_double), POINTER(c_int64), POINTER(c_int64)]),
    "hero_synth_qwen35_size": (c_int64, [POINTER(SynthConfig)]),
    "hero_synth_qwen35_image": (c_int, [POINTER(SynthConfig), c_void_p, c_size_t]),
    "hero_synth_qwen35_file": (c_int, [POINTER(SynthConfig), c_char_p]),
    "hero_gemma_math_eval": (c_int, [c_void_p, c_void_p, c_int64, c_float, c_void_p]),
    "hero_gemma4_open": (c_int, [c_char_p, POINTER(c_void_p)]),
    "hero_gemma4_open_image": (c_int, [c_void_p, c_size_t, POINTER(c_void_p)]),
    "hero_gemma4_close": (None, [c_void_p]),
    "hero_gemma4_dims_get": (c_int, [c_void_p, POINTER(Gemma4Dims)]),
    "hero_gemma4_state_create": (c_int, [c_void_p, c_int64, POINTER(c_void_p)]),
    "hero_gemma4_state_destroy": (None, [c_void_p]),
    "hero_gemma4_state_reset": (c_int, [c_void_p]),
    "hero_gemma4_state_tokens": (c_int64, [c_void_p]),
    "hero_gemma4_embed": (c_int, [c_void_p, c_void_p, c_int64, c_void_p]),
    "hero_gemma4_forward": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "hero_gemma4_decode_greedy": (c_int, [c_void_p, c_void_p, c_int32, c_int64, c_void_p, c_void_p]),
    "hero_gemma4_last_decode_seconds": (c_double, [c_void_p]),
    "hero_synth_gemma4_size": (c_int64, [POINTER(Gemma4SynthConfig)]),
    "hero_synth_gemma4_image": (c_int, [POINTER(Gemma4SynthConfig), c_void_p, c_size_t]),
    "hero_synth_gemma4_file": (c_int, [POINTER(Gemma4SynthConfig), c_char_p]),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() or make -C hero_amd")
    # One HIP runtime per process. PyTorch-ROCm ships its own libamdhip64 and
    # loads it by file name, so a runtime loaded earlier by this library would
    # not be shared: two runtimes would each own the device, and pointers from
    # one are invalid in the other. Loading torch first makes this library's
    # libamdhip64.so.7 / libhsa-runtime64.so.1 resolve to torch's copies.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(status: int) -> None:
    if status != HERO_OK:
        msg = lib.hero_last_error().decode(errors="replace")
        if status == HERO_ERANGE:
            raise ContextExhausted(status, msg)
        raise HeroError(status, msg)
