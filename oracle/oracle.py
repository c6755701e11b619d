"""ctypes front end of the CPU oracle (``oracle/liboracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, always as the checker.  The product (``blog_amd``) never imports it.

Every function restates reference arithmetic; the C source cites the reference lines
(``AI/codes/local-llm/src/backend/cuda/ops/kernel.cu``).  Arrays are numpy, C-contiguous.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q4_0, Q5_0, Q8_0, Q8_1, Q4_K, Q6_K = 0, 1, 2, 6, 8, 9, 12, 14
BLOCK = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q8_1: (32, 36), Q4_K: (256, 144), Q6_K: (256, 210)}
NAMES = {Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}

_lib = None
_lib_lock = threading.Lock()


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> C.CDLL:
    """The loaded library, its signatures declared.  Safe from several threads at once: the library is
    published only after every signature is set (a call through an undeclared function would pass its
    pointer arguments as 32-bit ints)."""
    global _lib
    if _lib is None:
        with _lib_lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    build()
                L = C.CDLL(LIB_PATH)
                _declare(L)
                _lib = L
    return _lib


P = C.c_void_p
I = C.c_int
I64 = C.c_int64
SZ = C.c_size_t


def _declare(L: C.CDLL) -> None:
    sig = {
        "orc_block_elems": (I, [I]),
        "orc_block_bytes": (I, [I]),
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
        "orc_f16_to_f32_array": (None, [P, P, I64]),
        "orc_f32_to_f16_array": (None, [P, P, I64]),
        "orc_q4k_scale_min": (None, [I, P, P, P]),
        "orc_dequant_f32": (I, [I, P, I64, P]),
        "orc_dequant_f16": (I, [I, P, I64, P]),
        "orc_matmul_f64": (I, [I, P, SZ, P, P, I, I, I]),
        "orc_matmul_f32": (I, [I, P, SZ, P, P, I, I, I, I]),
        "orc_matmul_lane32": (I, [I, P, SZ, P, P, I, I, I]),
        "orc_gemv_add": (I, [I, P, SZ, P, P, I, I]),
        "orc_q8_1_row_bytes": (SZ, [I]),
        "orc_quantize_q8_1": (None, [P, P, I, I, I]),
        "orc_matmul_q8_1": (I, [I, P, SZ, P, P, I, I, I]),
        "orc_matmul_q8_1_mt": (I, [I, P, SZ, P, P, I, I, I, I]),
        "orc_router_topk": (None, [P, P, P, I, I, I, C.c_float]),
        "orc_swiglu": (I, [I, P, P, SZ, SZ, P, P, I, I]),
        "orc_swiglu_indexed": (I, [I, P, P, SZ, SZ, SZ, SZ, P, P, P, I, I, I]),
        "orc_down_indexed_ordered": (I, [I, P, SZ, SZ, P, P, P, P, I, I, I]),
        "orc_argmax": (I, [P, I]),
        "orc_qwen2_logits": (I, [P, P, P, P, P, I, I, P, I]),
        "orc_quant_embedding": (I, [I, P, I, P, SZ, I, P]),
        "orc_mla_absorb_q_nope": (I, [I, P, P, SZ, P, I, I, I, I, I]),
        "orc_mla_absorb_q4_xsum_delta": (I, [P, P, SZ, P, I, I, I, I, I]),
        "orc_mla_absorb_v": (I, [I, P, SZ, P, P, P, I, I, I, I]),
        "orc_quantize_q8_1_mmq": (None, [P, P, I, I, I]),
        "orc_matmul_q8_1_mmq": (I, [I, P, SZ, P, P, I, I, I]),
        "orc_swiglu_indexed_q8_1": (I, [I, P, P, SZ, SZ, SZ, SZ, P, P, P, I, I, I]),
        "orc_down_q8_1_indexed_accum": (I, [I, P, SZ, SZ, P, P, P, P, I, I, I]),
        "orc_down_f32_indexed_accum": (I, [I, P, SZ, SZ, P, P, P, P, I, I, I]),
        "orc_mla_store_latent_q8_1": (I, [P, P, I, I, SZ, I]),
        "orc_mla_absorb_scores": (I, [P, P, P, SZ, P, P, P, I, I, I, I, I, I, C.c_float]),
        "orc_mla_absorb_context": (I, [P, P, SZ, P, P, I, I, I, I]),
        "orc_mla_absorb_attend": (I, [P, P, P, SZ, P, P, P, P, I, I, I, I, I, I, C.c_float]),
        "orc_mla_project_v": (I, [I, P, SZ, P, SZ, P, I, I, I, I, I]),
        "orc_mla_absorb_context_v": (I, [P, P, P, I, I, I, I, I]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _ok(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what}: unsupported type or shape")


def row_bytes(qtype: int, in_dim: int) -> int:
    be, bb = BLOCK[qtype]
    assert in_dim % be == 0
    return in_dim // be * bb


# ---- f16 ----------------------------------------------------------------------------------
def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(f), _p(out), f.size)
    return out


def q4k_scale_min(j: int, scales: bytes) -> tuple[int, int]:
    s = np.frombuffer(bytes(scales), np.uint8).copy()
    sc, m = C.c_int(), C.c_int()
    lib().orc_q4k_scale_min(j, _p(s), C.addressof(sc), C.addressof(m))
    return sc.value, m.value


# ---- dequant -------------------------------------------------------------------------------
def dequant_f32(qtype: int, src: np.ndarray, n: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(n, np.float32)
    _ok(lib().orc_dequant_f32(qtype, _p(src), n, _p(out)), "dequant_f32")
    return out


def dequant_f16(qtype: int, src: np.ndarray, n: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(n, np.uint16)
    _ok(lib().orc_dequant_f16(qtype, _p(src), n, _p(out)), "dequant_f16")
    return out


# ---- GEMV / matmul -------------------------------------------------------------------------
def matmul_f64(qtype: int, w: np.ndarray, rb: int, x: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_dim)
    m = x.shape[0]
    y = np.empty((m, out_dim), np.float64)
    _ok(lib().orc_matmul_f64(qtype, _p(w), rb, _p(x), _p(y), out_dim, in_dim, m), "matmul_f64")
    return y


def matmul_f32(qtype: int, w: np.ndarray, rb: int, x: np.ndarray, out_dim: int, in_dim: int,
               nthreads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_dim)
    m = x.shape[0]
    y = np.empty((m, out_dim), np.float32)
    _ok(lib().orc_matmul_f32(qtype, _p(w), rb, _p(x), _p(y), out_dim, in_dim, m, nthreads), "matmul_f32")
    return y


def matmul_lane32(qtype: int, w: np.ndarray, rb: int, x: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_dim)
    m = x.shape[0]
    y = np.empty((m, out_dim), np.float32)
    _ok(lib().orc_matmul_lane32(qtype, _p(w), rb, _p(x), _p(y), out_dim, in_dim, m), "matmul_lane32")
    return y


def gemv_add(qtype: int, w: np.ndarray, rb: int, x: np.ndarray, y: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.array(y, dtype=np.float32, copy=True)
    _ok(lib().orc_gemv_add(qtype, _p(w), rb, _p(x), _p(y), out_dim, in_dim), "gemv_add")
    return y


# ---- Q8_1 ----------------------------------------------------------------------------------
def q8_1_row_bytes(in_dim: int) -> int:
    return int(lib().orc_q8_1_row_bytes(in_dim))


def quantize_q8_1(x: np.ndarray, in_dim: int, store_raw_sum: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_dim)
    m = x.shape[0]
    out = np.zeros(m * q8_1_row_bytes(in_dim), np.uint8)
    lib().orc_quantize_q8_1(_p(x), _p(out), in_dim, m, int(store_raw_sum))
    return out


def matmul_q8_1(qtype: int, w: np.ndarray, rb: int, xq: np.ndarray, out_dim: int, in_dim: int, m: int,
                threads: int = 1) -> np.ndarray:
    """threads: OpenMP threads over the rows (<= 0: all); the results do not depend on it."""
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    y = np.empty((m, out_dim), np.float64)
    _ok(lib().orc_matmul_q8_1_mt(qtype, _p(w), rb, _p(xq), _p(y), out_dim, in_dim, m, threads), "matmul_q8_1")
    return y


# ---- MoE -----------------------------------------------------------------------------------
def router_topk(logits: np.ndarray, k: int, routed_scaling: float = 1.0):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    tokens, n_experts = logits.shape
    idx = np.empty((tokens, k), np.int32)
    w = np.empty((tokens, k), np.float32)
    lib().orc_router_topk(_p(logits), _p(idx), _p(w), tokens, n_experts, k, routed_scaling)
    return idx, w


def swiglu(qtype, wg, wu, g_rb, u_rb, x, ffn_dim, in_dim) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    act = np.empty(ffn_dim, np.float32)
    _ok(lib().orc_swiglu(qtype, _p(wg), _p(wu), g_rb, u_rb, _p(x), _p(act), ffn_dim, in_dim), "swiglu")
    return act


def swiglu_indexed(qtype, wg, wu, g_eb, u_eb, g_rb, u_rb, x, expert_ids, ffn_dim, in_dim) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(expert_ids, dtype=np.int32)
    k = ids.size
    act = np.empty((k, ffn_dim), np.float32)
    _ok(lib().orc_swiglu_indexed(qtype, _p(wg), _p(wu), g_eb, u_eb, g_rb, u_rb, _p(x), _p(ids), _p(act),
                                 k, ffn_dim, in_dim), "swiglu_indexed")
    return act


def down_indexed_ordered(qtype, wd, d_eb, d_rb, act, expert_ids, route_w, out, hidden, ffn_dim) -> np.ndarray:
    act = np.ascontiguousarray(act, dtype=np.float32)
    ids = np.ascontiguousarray(expert_ids, dtype=np.int32)
    rw = np.ascontiguousarray(route_w, dtype=np.float32)
    out = np.array(out, dtype=np.float32, copy=True)
    _ok(lib().orc_down_indexed_ordered(qtype, _p(wd), d_eb, d_rb, _p(act), _p(ids), _p(rw), _p(out),
                                       ids.size, hidden, ffn_dim), "down_indexed_ordered")
    return out


class Qwen2Cfg(C.Structure):
    """orc_qwen2_cfg (qlin_oracle.h)."""
    _fields_ = [("layers", C.c_int), ("hidden", C.c_int), ("n_heads", C.c_int), ("kv_heads", C.c_int),
                ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int), ("wtype", C.c_int),
                ("eps", C.c_double), ("theta", C.c_double)]


class Qwen2Layer(C.Structure):
    """orc_qwen2_layer (qlin_oracle.h)."""
    _fields_ = [(n, C.c_void_p) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "attn_norm", "ffn_norm")]


def qwen2_logits(cfg: dict, layers: list, final_norm: np.ndarray, table: np.ndarray, tokens, first: int,
                 threads: int = 0) -> np.ndarray:
    """The decoder twin: logits [len(tokens) - first, vocab] of positions first.., teacher-forced.

    cfg: layers, hidden, n_heads, kv_heads, head_dim, ffn, vocab, wtype, eps, theta; layers: dicts of
    numpy arrays wq, wk, wv, wo, wg, wu, wd (packed bytes) and attn_norm, ffn_norm (float32)."""
    c = Qwen2Cfg(**cfg)
    keep = []

    def ptr(a, dtype):
        a = np.ascontiguousarray(a, dtype=dtype)
        keep.append(a)
        return a.ctypes.data

    arr = (Qwen2Layer * len(layers))()
    for i, L in enumerate(layers):
        for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
            setattr(arr[i], n, ptr(L[n], np.uint8))
        arr[i].attn_norm = ptr(L["attn_norm"], np.float32)
        arr[i].ffn_norm = ptr(L["ffn_norm"], np.float32)
    toks = np.ascontiguousarray(tokens, np.int32)
    out = np.empty((len(toks) - first, cfg["vocab"]), np.float32)
    threads = threads or (os.cpu_count() or 1)
    _ok(lib().orc_qwen2_logits(C.byref(c), arr, ptr(final_norm, np.float32), ptr(table, np.uint8), _p(toks),
                               len(toks), first, _p(out), threads), "orc_qwen2_logits")
    return out


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(lib().orc_argmax(_p(v), v.size))


def quant_embedding(qtype: int, ids: np.ndarray, table: np.ndarray, rb: int, hidden: int) -> np.ndarray:
    ids = np.ascontiguousarray(ids, np.int32)
    out = np.zeros((len(ids), hidden), np.float32)
    _ok(lib().orc_quant_embedding(qtype, _p(ids), len(ids), _p(table), rb, hidden, _p(out)), "orc_quant_embedding")
    return out


def mla_absorb_q_nope(qtype, q, w, rb, n_heads, qk_nope, qk_rope, v_head, kv_lora) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    out = np.zeros(n_heads * kv_lora, np.float64)
    _ok(lib().orc_mla_absorb_q_nope(qtype, _p(q), _p(w), rb, _p(out), n_heads, qk_nope, qk_rope, v_head, kv_lora),
        "orc_mla_absorb_q_nope")
    return out


def mla_absorb_q4_xsum_delta(q, w, rb, n_heads, qk_nope, qk_rope, v_head, kv_lora) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    out = np.zeros(n_heads * ((kv_lora + 31) // 32), np.float64)
    _ok(lib().orc_mla_absorb_q4_xsum_delta(_p(q), _p(w), rb, _p(out), n_heads, qk_nope, qk_rope, v_head, kv_lora),
        "orc_mla_absorb_q4_xsum_delta")
    return out


def mla_absorb_v(qtype, w, rb, latent, delta, n_heads, qk_nope, v_head, kv_lora) -> np.ndarray:
    latent = np.ascontiguousarray(latent, np.float32)
    delta = np.ascontiguousarray(delta if delta is not None else np.zeros(1), np.float32)
    out = np.zeros(n_heads * v_head, np.float64)
    _ok(lib().orc_mla_absorb_v(qtype, _p(w), rb, _p(latent), _p(delta), _p(out), n_heads, qk_nope, v_head, kv_lora),
        "orc_mla_absorb_v")
    return out


# ---- MLA over the Q8_1 latent cache --------------------------------------------------------------
def mla_store_latent_q8_1(kv_cache, cache, kv_lora, qk_rope, row_bytes, pos) -> np.ndarray:
    """cache (uint8 [rows, row_bytes]) with row pos rewritten; returns a new array."""
    kv_cache = np.ascontiguousarray(kv_cache, np.float32)
    out = np.array(cache, np.uint8, copy=True)
    _ok(lib().orc_mla_store_latent_q8_1(_p(kv_cache), _p(out), kv_lora, qk_rope, row_bytes, pos),
        "orc_mla_store_latent_q8_1")
    return out


def mla_absorb_scores(q_abs, q, cache, crb, delta, kv_cache, n_heads, qk_nope, qk_rope, kv_lora, pos, max_seq,
                      scale) -> np.ndarray:
    """[n_heads, max_seq] float64; entries past pos are NaN."""
    args = [np.ascontiguousarray(a, np.float32) for a in (q_abs, q, delta, kv_cache)]
    cache = np.ascontiguousarray(cache, np.uint8)
    out = np.full((n_heads, max_seq), np.nan, np.float64)
    _ok(lib().orc_mla_absorb_scores(_p(args[0]), _p(args[1]), _p(cache), crb, _p(args[2]), _p(args[3]), _p(out),
                                    n_heads, qk_nope, qk_rope, kv_lora, pos, max_seq, scale), "orc_mla_absorb_scores")
    return out


def mla_absorb_context(scores, cache, crb, n_heads, kv_lora, pos, max_seq):
    """(attn_latent [n_heads, kv_lora], attn_xsum_delta [n_heads, ceil(kv_lora / 32)]) in float64."""
    scores = np.ascontiguousarray(scores, np.float32)
    cache = np.ascontiguousarray(cache, np.uint8)
    lat = np.zeros((n_heads, kv_lora), np.float64)
    dl = np.zeros((n_heads, (kv_lora + 31) // 32), np.float64)
    _ok(lib().orc_mla_absorb_context(_p(scores), _p(cache), crb, _p(dl), _p(lat), n_heads, kv_lora, pos, max_seq),
        "orc_mla_absorb_context")
    return lat, dl


def mla_project_v(qtype, w, rb, cache, crb, kv_b_cache, n_heads, qk_nope, v_head, kv_lora, pos) -> np.ndarray:
    """kv_b_cache (float64 copy) with the v rows of position pos written."""
    cache = np.ascontiguousarray(cache, np.uint8)
    out = np.array(kv_b_cache, np.float64, copy=True)
    _ok(lib().orc_mla_project_v(qtype, _p(w), rb, _p(cache), crb, _p(out), n_heads, qk_nope, v_head, kv_lora, pos),
        "orc_mla_project_v")
    return out


def mla_absorb_context_v(scores, kv_b_cache, n_heads, qk_nope, v_head, pos, max_seq) -> np.ndarray:
    scores = np.ascontiguousarray(scores, np.float32)
    kvb = np.ascontiguousarray(kv_b_cache, np.float32)
    out = np.zeros((n_heads, v_head), np.float64)
    _ok(lib().orc_mla_absorb_context_v(_p(scores), _p(kvb), _p(out), n_heads, qk_nope, v_head, pos, max_seq),
        "orc_mla_absorb_context_v")
    return out


def mla_absorb_attend(q_abs, q, cache, crb, delta, kv_cache, n_heads, qk_nope, qk_rope, kv_lora, pos, max_seq, scale):
    """(attn_latent, attn_xsum_delta) of the fused form (softmax without the 1e-9 term), float64."""
    args = [np.ascontiguousarray(a, np.float32) for a in (q_abs, q, delta, kv_cache)]
    cache = np.ascontiguousarray(cache, np.uint8)
    lat = np.zeros((n_heads, kv_lora), np.float64)
    dl = np.zeros((n_heads, (kv_lora + 31) // 32), np.float64)
    _ok(lib().orc_mla_absorb_attend(_p(args[0]), _p(args[1]), _p(cache), crb, _p(args[2]), _p(dl), _p(args[3]),
                                    _p(lat), n_heads, qk_nope, qk_rope, kv_lora, pos, max_seq, scale),
        "orc_mla_absorb_attend")
    return lat, dl


# ---- Q8_1-activation variants ----------------------------------------------------------------------
def quantize_q8_1_mmq(x: np.ndarray, in_dim: int, store_raw_sum: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_dim)
    m = x.shape[0]
    out = np.zeros(((in_dim + 127) // 128) * m * 144, np.uint8)
    lib().orc_quantize_q8_1_mmq(_p(x), _p(out), in_dim, m, int(store_raw_sum))
    return out


def matmul_q8_1_mmq(qtype, w, rb, xq, out_dim, in_dim, m) -> np.ndarray:
    xq = np.ascontiguousarray(xq, np.uint8)
    y = np.empty((m, out_dim), np.float64)
    _ok(lib().orc_matmul_q8_1_mmq(qtype, _p(w), rb, _p(xq), _p(y), out_dim, in_dim, m), "matmul_q8_1_mmq")
    return y


def swiglu_indexed_q8_1(qtype, wg, wu, g_eb, u_eb, g_rb, u_rb, xq, expert_ids, ffn_dim, in_dim) -> np.ndarray:
    ids = np.ascontiguousarray(expert_ids, np.int32)
    xq = np.ascontiguousarray(xq, np.uint8)
    act = np.empty((ids.size, ffn_dim), np.float64)
    _ok(lib().orc_swiglu_indexed_q8_1(qtype, _p(wg), _p(wu), g_eb, u_eb, g_rb, u_rb, _p(xq), _p(ids), _p(act),
                                      ids.size, ffn_dim, in_dim), "swiglu_indexed_q8_1")
    return act


def down_q8_1_indexed_accum(qtype, wd, d_eb, d_rb, act, expert_ids, route_w, out, hidden, ffn_dim, f32_act=False):
    """out (float64 copy) += the routed down products; act is Q8_1 bytes or, with f32_act, f32 rows."""
    ids = np.ascontiguousarray(expert_ids, np.int32)
    rw = np.ascontiguousarray(route_w, np.float32)
    res = np.array(out, np.float64, copy=True)
    if f32_act:
        a = np.ascontiguousarray(act, np.float32)
        fn = lib().orc_down_f32_indexed_accum
    else:
        a = np.ascontiguousarray(act, np.uint8)
        fn = lib().orc_down_q8_1_indexed_accum
    _ok(fn(qtype, _p(wd), d_eb, d_rb, _p(a), _p(ids), _p(rw), _p(res), ids.size, hidden, ffn_dim),
        "down_q8_1_indexed_accum")
    return res
