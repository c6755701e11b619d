"""ctypes binding of ``blog_amd/libqlin.so`` (the C ABI declared in ``include/qlin.h``).

Plumbing for the tests and the benchmark: device memory comes from torch tensors, every compute
call goes through the C ABI into the HIP kernels.  There is no fallback of any kind: if the
library is missing or a call is rejected, this module raises.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libqlin.so")

Q4_0, Q5_0, Q8_0, Q8_1, Q4_K, Q6_K = 2, 6, 8, 9, 12, 14
STATUS = {0: "QLIN_OK", 1: "QLIN_ERR_UNSUPPORTED_TYPE", 2: "QLIN_ERR_SHAPE", 3: "QLIN_ERR_NULL",
          4: "QLIN_ERR_ROW_BYTES", 5: "QLIN_ERR_LIMIT", 6: "QLIN_ERR_LAUNCH", 7: "QLIN_ERR_ALIGN",
          8: "QLIN_ERR_IO", 9: "QLIN_ERR_FORMAT", 10: "QLIN_ERR_NOT_FOUND", 11: "QLIN_ERR_ALLOC"}

P, I, I64, SZ, F = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_float
S, U32, U64 = C.c_char_p, C.c_uint32, C.c_uint64
PP, PI, PI64, PU64, PSZ, PD = (C.POINTER(C.c_void_p), C.POINTER(C.c_int), C.POINTER(C.c_int64),
                               C.POINTER(C.c_uint64), C.POINTER(C.c_size_t), C.POINTER(C.c_double))


class GgufTensorInfo(C.Structure):
    """struct qlin_gguf_tensor (include/qlin_gguf.h)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("n_dims", C.c_int), ("shape", C.c_int64 * 4),
                ("nbytes", C.c_uint64), ("offset", C.c_uint64), ("data", C.c_void_p)]

# name -> (restype, argtypes); every symbol of include/qlin.h
SIGNATURES = {
    "qlin_status_string": (C.c_char_p, [I]),
    "qlin_version": (C.c_char_p, []),
    "qlin_set_stream": (I, [P]),
    "qlin_get_stream": (P, []),
    "qlin_block_elems": (I, [I]),
    "qlin_block_bytes": (I, [I]),
    "qlin_row_bytes": (SZ, [I, I]),
    "qlin_launch_quant_gemv": (I, [I, P, SZ, P, P, I, I, I]),
    "qlin_launch_quant_gemv_add": (I, [I, P, SZ, P, P, I, I]),
    "qlin_launch_quant_matmul": (I, [I, P, SZ, P, P, I, I, I]),
    "qlin_launch_quant_matmul_add": (I, [I, P, SZ, P, P, I, I, I]),
    "qlin_launch_quant_gemv_q8_1": (I, [I, P, SZ, P, P, I, I]),
    "qlin_launch_moe_accumulate": (I, [P, F, P, I]),
    "qlin_launch_moe_accumulate_device": (I, [P, P, P, I]),
    "qlin_launch_argmax": (I, [P, I, P]),
    "qlin_launch_quantize_q8_1_mmq": (I, [P, P, I, I, I]),
    "qlin_launch_quant_matmul_q8_1_mmq": (I, [I, P, SZ, P, P, I, I, I]),
    "qlin_launch_quant_swiglu_indexed_block": (I, [I, P, P, SZ, SZ, SZ, SZ, P, P, P, I, I, I, I]),
    "qlin_launch_quant_swiglu_indexed_q8_1": (I, [I, P, P, SZ, SZ, SZ, SZ, P, P, P, I, I, I]),
    "qlin_launch_quant_down_q8_1_indexed_accum": (I, [I, P, SZ, SZ, P, P, P, P, I, I, I]),
    "qlin_launch_quant_down_q8_1_indexed_accum_shared": (I, [I, P, SZ, SZ, P, P, P, P, I, I, I]),
    "qlin_launch_quant_down_f32_indexed_accum": (I, [I, P, SZ, SZ, P, P, P, P, I, I, I]),
    "qlin_launch_quant_swiglu_rows": (I, [I, P, P, SZ, SZ, P, P, I, I, I]),
    "qlin_launch_quant_gemv_multi": (I, [I, I, P, SZ, P, P, P, I]),
    "qlin_q8_1_row_bytes": (SZ, [I]),
    "qlin_launch_quantize_q8_1": (I, [P, P, I, I, I]),
    "qlin_launch_quant_matmul_q8_1": (I, [I, P, SZ, P, P, I, I, I]),
    "qlin_launch_quant_swiglu": (I, [I, P, P, SZ, SZ, P, P, I, I]),
    "qlin_launch_quant_swiglu_indexed": (I, [I, P, P, SZ, SZ, SZ, SZ, P, P, P, I, I, I]),
    "qlin_launch_quant_down_f32_indexed_accum_ordered": (I, [I, P, SZ, SZ, P, P, P, P, I, I, I]),
    "qlin_launch_moe_router_topk": (I, [P, P, P, I, I, I, F]),
    "qlin_launch_dequantize_to_f16": (I, [I, P, P, I64]),
    "qlin_launch_dequantize_q4k_to_f16": (I, [P, P, I64]),
    "qlin_launch_dequantize_q80_to_f16": (I, [P, P, I64]),
    "qlin_launch_dequantize_q50_to_f16": (I, [P, P, I64]),
    "qlin_launch_dequantize_q6k_to_f16": (I, [P, P, I64]),
    "qlin_launch_dequantize_to_f32": (I, [I, P, P, I64]),
    "qlin_gemm": (I, [I, P, SZ, P, P, I, I, I]),
    "qlin_moe_routed_decode_indexed": (I, [I, P, P, SZ, I, P, SZ, I, I, I, I, P, P, P, P, P, I]),
    "qlin_moe_routed_decode_indexed_logits": (I, [I, P, P, SZ, I, P, SZ, I, I, I, I, P, P, F, P, P, P, P, I]),
    "qlin_moe_ffn_decode_indexed_logits": (I, [I, P, P, SZ, I, P, SZ, I, I, I, I, I, P, P, SZ, P, SZ, I, P, P, F, P, P,
                                               P, P, I]),
    "qlin_moe_grouped_workspace_bytes": (SZ, [I, I, I, I, I]),
    "qlin_moe_routed_decode_grouped": (I, [I, P, P, SZ, I, P, SZ, I, I, I, I, P, P, P, P, SZ, P, I, I]),
    "qlin_moe_routed_decode_grouped_logits": (I, [I, P, P, SZ, I, P, SZ, I, I, I, I, P, P, F, P, P, P, SZ, P, I, I]),
    "qlin_moe_ffn_workspace_bytes": (SZ, [I, I, I, I, I, I]),
    "qlin_moe_ffn_decode_grouped_logits": (I, [I, P, P, SZ, I, P, SZ, I, I, I, I, I, P, P, SZ, P, SZ, I, P, P, F, P, P,
                                               P, SZ, P, I, I]),
    "qlin_moe_routed_decode_grouped_noalloc": (I, [I, P, P, SZ, I, P, SZ, I, I, I, I, P, P, P, P, I, I]),
    # include/qlin_decoder.h
    "qlin_launch_rms_norm": (I, [P, P, P, I, I, I, F, I]),
    "qlin_launch_rope_store_kv": (I, [P, P, P, P, P, I, I, I, I, I, P, F]),
    "qlin_launch_attend": (I, [P, P, P, P, I, I, I, I, I, P]),
    "qlin_launch_rope_attend": (I, [P, P, P, P, P, P, I, I, I, I, P, F]),
    "qlin_launch_rms_norm_quant_gemv_multi": (I, [I, I, P, SZ, P, P, I, F, I, P, P, I]),
    "qlin_launch_rms_norm_quant_swiglu": (I, [I, P, P, SZ, P, P, I, F, I, P, I, I]),
    "qlin_launch_quant_gemv_argmax": (I, [I, P, SZ, P, P, I, F, I, P, I, I, P, P]),
    "qlin_launch_quant_embedding": (I, [I, P, P, P, SZ, I, I]),
    "qlin_launch_mla_absorb_q_nope": (I, [I, P, P, SZ, P, I, I, I, I, I]),
    "qlin_launch_mla_absorb_q4_xsum_delta": (I, [P, P, SZ, P, I, I, I, I, I]),
    "qlin_launch_mla_absorb_v": (I, [I, P, SZ, P, P, P, I, I, I, I]),
    "qlin_launch_mla_store_latent_q8_1_device_pos": (I, [P, P, I, I, SZ, P]),
    "qlin_launch_mla_absorb_scores_device_pos": (I, [P, P, P, SZ, P, P, P, I, I, I, I, P, I, F]),
    "qlin_launch_mla_absorb_context_device_pos": (I, [P, P, SZ, P, P, I, I, P, I]),
    "qlin_launch_mla_absorb_attend_device_pos": (I, [P, P, P, SZ, P, P, P, P, I, I, I, I, P, I, F]),
    "qlin_launch_mla_project_v_device_pos": (I, [I, P, SZ, P, SZ, P, I, I, I, I, P]),
    "qlin_launch_mla_absorb_context_v_device_pos": (I, [P, P, P, I, I, I, P, I]),
    # include/qlin_gguf.h
    "qlin_gguf_open": (I, [S, PP]),
    "qlin_gguf_close": (None, [P]),
    "qlin_gguf_version": (U32, [P]),
    "qlin_gguf_alignment": (U32, [P]),
    "qlin_gguf_tensor_count": (I64, [P]),
    "qlin_gguf_find_tensor": (I64, [P, S]),
    "qlin_gguf_tensor_info": (I, [P, I64, C.POINTER(GgufTensorInfo)]),
    "qlin_gguf_metadata_count": (I64, [P]),
    "qlin_gguf_metadata_key": (S, [P, I64]),
    "qlin_gguf_metadata_type": (I, [P, S]),
    "qlin_gguf_get_i64": (I, [P, S, PI64]),
    "qlin_gguf_get_f64": (I, [P, S, PD]),
    "qlin_gguf_get_str": (I, [P, S, PP, PSZ]),
    "qlin_gguf_get_array_info": (I, [P, S, PI, PI64]),
    "qlin_gguf_get_array_i64": (I, [P, S, I64, PI64]),
    "qlin_gguf_get_array_f64": (I, [P, S, I64, PD]),
    "qlin_gguf_get_array_str": (I, [P, S, I64, PP, PSZ]),
    "qlin_pool_create": (I, [PP]),
    "qlin_pool_destroy": (None, [P]),
    "qlin_pool_weight": (I, [P, P, S, PP, PU64]),
    "qlin_pool_expert_view": (I, [P, P, S, I, PP, PU64, PI64, PI64]),
    "qlin_pool_resident_bytes": (U64, [P]),
}


class QlinError(RuntimeError):
    def __init__(self, fn: str, rc: int):
        super().__init__(f"{fn} returned {rc} ({STATUS.get(rc, '?')})")
        self.rc = rc


_lib = None


def lib() -> C.CDLL:
    """Loads the HIP library; raises if it has not been built (no fallback path exists)."""
    global _lib
    if _lib is None:
        # torch ships its own HIP runtime (torch/lib/libamdhip64.so, soname libamdhip64.so.7).  Loaded
        # first, it satisfies this library's libamdhip64.so.7 dependency, so the process has one HIP
        # runtime; loaded after, it would bring a second one next to /opt/rocm's, and device memory of
        # one is unusable from the other.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `python -m blog_amd.build` (HIP/gfx950 build)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def ptr(t) -> int:
    """Device address of a torch tensor (or an int address, or None -> 0)."""
    if t is None:
        return 0
    if isinstance(t, int):
        return t
    return t.data_ptr()


def call(name: str, *args) -> int:
    """Calls an entry point with tensors converted to addresses; raises on a non-zero status."""
    rc = getattr(lib(), name)(*[ptr(a) if not isinstance(a, (float, bool)) and hasattr(a, "data_ptr") else a
                                for a in args])
    if rc != 0:
        raise QlinError(name, rc)
    return rc


def status(name: str, *args) -> int:
    """Calls an entry point and returns its status without raising."""
    return getattr(lib(), name)(*[ptr(a) if hasattr(a, "data_ptr") else a for a in args])


def set_stream(stream) -> None:
    """Launch on a torch.cuda.Stream (or a raw hipStream_t address, or None)."""
    handle = 0 if stream is None else (stream if isinstance(stream, int) else stream.cuda_stream)
    lib().qlin_set_stream(handle or None)


def row_bytes(qtype: int, in_dim: int) -> int:
    return int(lib().qlin_row_bytes(qtype, in_dim))


# ---- convenience wrappers (tensors in, launches on the current library stream) --------------

def quant_gemv(qtype, w, rb, x, y, out_dim, in_dim, m=1):
    call("qlin_launch_quant_gemv", qtype, w, rb, x, y, out_dim, in_dim, m)


def quant_gemv_add(qtype, w, rb, x, y, out_dim, in_dim):
    call("qlin_launch_quant_gemv_add", qtype, w, rb, x, y, out_dim, in_dim)


def quant_gemv_multi(qtype, ws, rb, x, ys, out_dims, in_dim):
    """Several GEMVs sharing x in one launch (lists of tensors / device addresses)."""
    n = len(ws)
    wa = (C.c_void_p * n)(*[ptr(w) for w in ws])
    ya = (C.c_void_p * n)(*[ptr(y) for y in ys])
    da = (C.c_int * n)(*out_dims)
    call("qlin_launch_quant_gemv_multi", qtype, n, C.addressof(wa), rb, x, C.addressof(ya), C.addressof(da), in_dim)


def rms_norm_quant_gemv_multi(qtype, ws, rb, x, norm_w, norm_type, eps, one_plus, ys, out_dims, in_dim):
    """quant_gemv_multi of rms_norm(x), in one launch (lists of tensors / device addresses)."""
    n = len(ws)
    wa = (C.c_void_p * n)(*[ptr(w) for w in ws])
    ya = (C.c_void_p * n)(*[ptr(y) for y in ys])
    da = (C.c_int * n)(*out_dims)
    call("qlin_launch_rms_norm_quant_gemv_multi", qtype, n, C.addressof(wa), rb, x, norm_w, norm_type, eps, one_plus,
         C.addressof(ya), C.addressof(da), in_dim)


def quant_swiglu(qtype, wg, wu, g_rb, u_rb, x, act, ffn_dim, in_dim):
    call("qlin_launch_quant_swiglu", qtype, wg, wu, g_rb, u_rb, x, act, ffn_dim, in_dim)


def quant_matmul(qtype, w, rb, x, y, out_dim, in_dim, m):
    call("qlin_launch_quant_matmul", qtype, w, rb, x, y, out_dim, in_dim, m)


def quant_matmul_add(qtype, w, rb, x, y, out_dim, in_dim, m):
    call("qlin_launch_quant_matmul_add", qtype, w, rb, x, y, out_dim, in_dim, m)


def quant_swiglu_rows(qtype, wg, wu, g_rb, u_rb, x, act, ffn_dim, in_dim, m):
    call("qlin_launch_quant_swiglu_rows", qtype, wg, wu, g_rb, u_rb, x, act, ffn_dim, in_dim, m)


def quantize_q8_1(x, xq, in_dim, m, store_raw_sum=False):
    call("qlin_launch_quantize_q8_1", x, xq, in_dim, m, int(store_raw_sum))


def quant_matmul_q8_1(qtype, w, rb, xq, y, out_dim, in_dim, m):
    call("qlin_launch_quant_matmul_q8_1", qtype, w, rb, xq, y, out_dim, in_dim, m)


def dequantize(qtype, src, out, n, f16=True):
    if f16:
        call("qlin_launch_dequantize_to_f16", qtype, src, out, n)
    else:
        call("qlin_launch_dequantize_to_f32", qtype, src, out, n)
