"""ctypes binding of ``libmindpipe_amd.so`` (the C ABI in ``include/mindpipe_amd.h``).

There is no fallback: if the library is missing or a symbol is absent, loading
raises.  The product path never computes on the CPU.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("MINDPIPE_AMD_LIB", Path(__file__).resolve().parent / "libmindpipe_amd.so"))

MP_F16, MP_BF16, MP_F32, MP_I8 = 0, 1, 2, 3
MP_SCALE_FP32, MP_SCALE_FAKE = 0, 1
MP_SCALE_FP16 = MP_SCALE_FAKE  # older name of the fake rule
ABI_VERSION = 2

_vp, _i64, _i32, _sz = C.c_void_p, C.c_int64, C.c_int, C.c_size_t

# name -> (restype, argtypes); mirrors include/mindpipe_amd.h one to one.
SIGNATURES = {
    "mp_strerror": (C.c_char_p, [_i32]),
    "mp_abi_version": (_i32, []),
    "mp_w4_quantize_awq": (_i32, [_vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "mp_awq_pseudo_quantize": (_i32, [_vp, _i32, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "mp_w4_quantize_gptq_rtn": (_i32, [_vp, _i32, _i64, _i64, _i32, _vp, _vp, _vp, _vp]),
    "mp_pack_int4": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "mp_unpack_int4": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "mp_w4a16_gemm": (_i32, [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _vp]),
    "mp_w4a16_gemm_swiglu": (_i32, [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _vp]),
    "mp_w4a16_gemv_rmsnorm": (_i32, [_vp, _vp, _vp, C.c_float, _vp, _i64, _vp, _i64, _vp, _vp, _i32, _vp, _i32,
                                     _vp, _i32, _vp]),
    "mp_quant_per_token_i8": (_i32, [_vp, _i64, _i64, _i32, _vp, _vp, _i32, _vp]),
    "mp_add_rms_norm_quant": (_i32, [_vp, _vp, _vp, C.c_float, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp]),
    "mp_decode_rope_append": (_i32, [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp]),
    "mp_prefill_rope_split": (_i32, [_vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _i64, _vp, _vp, _vp, _vp]),
    "mp_decode_attention_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "mp_decode_attention": (_i32, [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _i64, _i32, C.c_float, _vp, _vp, _sz,
                                   _vp]),
    "mp_decode_rope_attention": (_i32, [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _i64, _vp, _vp, _i32, C.c_float,
                                        _vp, _vp, _sz, _vp]),
    "mp_silu_mul": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp]),
    "mp_argmax_rows": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "mp_w8a8_gemm_quant_out_workspace_bytes": (_sz, [_i64, _i64]),
    "mp_w8a8_gemm_quant_out": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _vp, _vp,
                                      _vp, _sz, _vp]),
    "mp_colmax_abs": (_i32, [_vp, _i32, _i64, _i64, _i32, _vp, _vp]),
    "mp_smooth_scales": (_i32, [_vp, _vp, _i64, C.c_double, _i32, _vp, _vp]),
    "mp_scale_columns": (_i32, [_vp, _i32, _i64, _i64, _vp, _i32, _vp]),
    "mp_w8_quantize_per_channel": (_i32, [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _i32, _vp, _vp]),
    "mp_w8a8_gemm": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _vp]),
    "mp_moe_route_workspace_bytes": (_sz, [_i64, _i64, _i32]),
    "mp_moe_permute_quant": (_i32, [_vp, _i32, _vp, _i64, _i64, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _sz,
                                    _vp]),
    "mp_moe_gmm1_workspace_bytes": (_sz, [_i64, _i64]),
    "mp_i8_gemm_swiglu_requant": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _vp, _vp,
                                         _sz, _vp]),
    "mp_i8_gemm_swiglu_requant_noalloc": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp,
                                                 _vp, _vp]),
    "mp_w8a8_grouped_gemm": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _i32, _vp]),
    "mp_w8a8_gemm_fake": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _vp]),
    "mp_dq_linear": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _vp]),
    "mp_fake_quant_rows": (_i32, [_vp, _i32, _i64, _i64, _i32, _vp, _vp, _vp]),
    "mp_moe_unpermute_combine": (_i32, [_vp, _vp, _vp, _i64, _i32, _i64, _i32, _vp, _i32, _vp]),
}

_LIB = None


def load() -> C.CDLL:
    """Load the HIP library once; raise if it is missing or incomplete."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise ImportError(
            f"mindpipe_amd: HIP library {LIB_PATH} is not built "
            "(run `python -m mindpipe_amd.build`); there is no CPU fallback")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is missing
        fn.restype = res
        fn.argtypes = args
    if lib.mp_abi_version() != ABI_VERSION:
        raise ImportError("mindpipe_amd: ABI version mismatch")
    _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().mp_strerror(rc).decode()
        raise RuntimeError(f"{what}: {msg} (status {rc})")
