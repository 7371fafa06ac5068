"""hyper_amd: MI355X (gfx950) quantized MoE expert-FFN path behind a C ABI (include/hymoe.h).

The product is libhymoe.so (HIP kernels + C entry points).  This package loads it with ctypes and
mirrors the reference's expert-compute API (hyper src/kernels4.cuh:45-91, src/experts.h:20-50) on
torch device tensors (torch is used for device memory and streams only).  There is no fallback: if
the library is missing or a call fails, an exception is raised.
"""
import ctypes
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libhymoe.so"

HY_OK, HY_EUNSUPPORTED_TYPE, HY_EBAD_SHAPE, HY_EHIP, HY_EINVAL = 0, 1, 2, 3, 4


class HyError(RuntimeError):
    """A non-zero status from libhymoe (the reference throws std::runtime_error at the same places)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[hymoe {code}] {msg}")
        self.code = code


class hy_moe_dev(ctypes.Structure):
    """C layout of hy_moe_dev (include/hymoe.h; replaces MoeDev, src/kernels4.cuh:56-63)."""
    _fields_ = [("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
                ("tg", ctypes.c_int32), ("td", ctypes.c_int32),
                ("gate_bytes", ctypes.c_size_t), ("down_bytes", ctypes.c_size_t),
                ("slot", ctypes.c_void_p), ("ff", ctypes.c_int32), ("n", ctypes.c_int32),
                ("clamp", ctypes.c_float), ("n_expert", ctypes.c_int32), ("n_local", ctypes.c_int32)]


class hy_expert_tensors(ctypes.Structure):
    _fields_ = [("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
                ("gb", ctypes.c_size_t), ("db", ctypes.c_size_t), ("E", ctypes.c_int32),
                ("tg", ctypes.c_int32), ("td", ctypes.c_int32)]


class hy_gguf_tensor_info(ctypes.Structure):
    """C layout of hy_gguf_tensor_info (include/hymoe.h; replaces GTensor, src/gguf.h:22-32)."""
    _fields_ = [("name", ctypes.c_char_p), ("data", ctypes.c_void_p), ("nbytes", ctypes.c_size_t),
                ("type", ctypes.c_int32), ("n_dims", ctypes.c_int32), ("ne", ctypes.c_int64 * 4)]


_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_DEV = ctypes.POINTER(hy_moe_dev)

# name -> (restype, argtypes); every function declared in include/hymoe.h
SIGNATURES = {
    "hy_last_error": (ctypes.c_char_p, []),
    "hy_abi_version": (_I, []),
    "hy_block_bytes": (ctypes.c_size_t, [_I]),
    "hy_block_elems": (_I, [_I]),
    "hy_vec_dot_type": (_I, [_I]),
    "hy_q8_row_bytes": (ctypes.c_size_t, [_I, _I]),
    "hy_upload_experts": (_I, [ctypes.POINTER(hy_expert_tensors), _P, ctypes.c_int32, ctypes.c_int32, _F, _DEV]),
    "hy_free_experts": (_I, [_DEV]),
    "hy_gguf_open": (_I, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]),
    "hy_gguf_close": (_I, [_P]),
    "hy_gguf_arch": (ctypes.c_char_p, [_P]),
    "hy_gguf_has": (_I, [_P, ctypes.c_char_p]),
    "hy_gguf_get_int": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    "hy_gguf_get_float": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "hy_gguf_get_str": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]),
    "hy_gguf_get_int_arr": (_I, [_P, ctypes.c_char_p, _P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]),
    "hy_gguf_get_float_arr": (_I, [_P, ctypes.c_char_p, _P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]),
    "hy_gguf_n_tensors": (_I, [_P]),
    "hy_gguf_tensor_at": (_I, [_P, _I, ctypes.POINTER(hy_gguf_tensor_info)]),
    "hy_gguf_tensor": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(hy_gguf_tensor_info)]),
    "hy_gguf_expert_tensors": (_I, [_P, _I, _I, ctypes.POINTER(hy_expert_tensors)]),
    "hy_gemv_f32": (_I, [_P, _I, _I, _P, _I, _P, _I, _I, _P, _I, _P]),
    "hy_gemv_bf16w": (_I, [_P, _I, _I, _P, _I, _P, _I, _I, _P, _I, _P]),
    "hy_bf16_to_f32": (_I, [_P, ctypes.c_size_t, _P, _P]),
    "hy_moe_route": (_I, [_P, _I, _I, _I, _P, _P, _P, _I, _P]),
    "hy_moe_route_sig": (_I, [_P, _I, _P, _I, _I, _F, _P, _P, _P, _I, _P]),
    "hy_moe_route_sqrtsp": (_I, [_P, _I, _P, _I, _I, _F, _P, _P, _I, _P]),
    "hy_moe_order": (_I, [_DEV, _P, _I, _I, _P, _P, _P, _P]),
    "hy_q8_quantize": (_I, [_I, _P, _I, _I, _I, _P, _P]),
    "hy_q8k_quantize_host": (_I, [_P, _P, ctypes.c_int64]),
    "hy_moe_gate_up": (_I, [_DEV, _P, _I, _P, _I, _P, _I, _P, _P, _P]),
    "hy_moe_down": (_I, [_DEV, _P, _P, _P, _I, _P, _I, _P, _P, _P]),
    "hy_moe_gemm_gate_up": (_I, [_DEV, _P, _I, _I, _P, _P, _P, _I, _P, _P]),
    "hy_moe_gemm_down": (_I, [_DEV, _P, _I, _P, _P, _P, _I, _P, _P, _P]),
    "hy_moe_reduce": (_I, [_P, _P, _P, _I, _P, _I, _I, _P, _P]),
    "hy_moe_reduce_residual": (_I, [_P, _P, _P, _I, _P, _I, _I, _P, _P]),
    "hy_moe_down_reduce": (_I, [_DEV, _P, _P, _P, _I, _P, _P, _P, _I, _P]),
    "hy_moe_down_reduce_residual": (_I, [_DEV, _P, _P, _P, _I, _P, _P, _P, _I, _P]),
    "hy_moe_router_q8": (_I, [_P, _I, _I, _P, _I, _P, _I, _P, _I, _I, _P, _I, _P]),
    "hy_moe_router_q8_bf16w": (_I, [_P, _I, _I, _P, _I, _P, _I, _P, _I, _I, _P, _I, _P]),
    "hy_moe_route_gate_up": (_I, [_DEV, _P, _I, _I, _I, _P, _P, _P, _P, _P, _I, _P]),
    "hy_moe_route_gate_up_q8": (_I, [_DEV, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _P]),
    "hy_moe_shared_gate_up": (_I, [_DEV, _P, _P, _I, _P]),
    "hy_moe_shared_down": (_I, [_DEV, _P, _P, _I, _P]),
    "hy_moe_down_reduce_q8": (_I, [_DEV, _P, _P, _P, _I, _P, _P, _P, _I, _I, _P]),
    "hy_moe_decode_ws_bytes": (ctypes.c_size_t, [_DEV, _I, _I, _DEV, _I]),
    "hy_moe_decode": (_I, [_DEV, _P, _I, _P, _I, _P, _I, _I, _DEV, _P, _I, _I, _P, ctypes.c_size_t, _P]),
    "hy_moe_decode_noalloc": (_I, [_DEV, _P, _I, _P, _I, _P, _I, _I, _DEV, _P, _I, _I, _P]),
    "hy_dequant_row": (_I, [_I, _P, _I, _P, _P]),
    "hy_block_ints": (_I, [_I, _P, ctypes.c_size_t, _I, _P, _I, _P, _P, _P]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded libhymoe.so (built by __graft_entry__.build() / python -m hyper_amd.build)."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("HYMOE_LIB", LIB_PATH))
        if not path.exists():
            raise ImportError(f"libhymoe.so not built at {path}: run `python -m hyper_amd.build`")
        L = ctypes.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != HY_OK:
        raise HyError(rc, lib().hy_last_error().decode(errors="replace"))


from .formats import GType, block_bytes, block_elems, vec_dot_type, q8_row_bytes  # noqa: E402,F401
