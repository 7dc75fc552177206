"""numpy front end of the CPU oracle (oracle/m27q_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker.  The product library
(libm27q.so) never imports or calls it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libm27q_oracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libofficial_dequant.so")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, IQ4_XS = 0, 1, 8, 12, 13, 14, 15, 23
TYPE_SIZE = {F32: 4, F16: 2, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292, IQ4_XS: 136}
BLOCK_ELEMS = {F32: 1, F16: 1, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256, IQ4_XS: 256}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P, I, I64, D = C.c_void_p, C.c_int, C.c_int64, C.c_double
        sig = {
            "ora_fp16_to_fp32_n": (None, [P, P, C.c_size_t]),
            "ora_fp32_to_fp16_n": (None, [P, P, C.c_size_t]),
            "ora_dequant_rows": (I, [I, P, I, I, P]),
            "ora_quantize_row_q4_K": (None, [P, P, I64]),
            "ora_quantize_row_q5_K": (None, [P, P, I64]),
            "ora_quantize_row_q6_K": (None, [P, P, I64]),
            "ora_quantize_row_q8_0": (None, [P, P, I64]),
            "ora_quantize_row_iq4_xs": (None, [P, P, I64]),
            "ora_quant_act": (None, [P, I64, P, P, P]),
            "ora_quant_act_gated": (None, [P, P, I64, P, P, P]),
            "ora_exp_cw_n": (None, [P, P, C.c_size_t]),
            "ora_gated_n": (None, [P, P, P, C.c_size_t]),
            "ora_vec_dot_q4_K_q8_K": (C.c_float, [I, P, P]),
            "ora_vec_dot_q6_K_q8_K": (C.c_float, [I, P, P]),
            "ora_vec_dot_q8_0_q8_0": (C.c_float, [I, P, P]),
            "ora_dot_act": (D, [I, P, I, P, P, P, P]),
            "ora_gemv_act": (I, [I, P, I, I, P, P, P, P, P]),
            "ora_gemv_f64": (I, [I, P, I, I, P, P]),
            "ora_quant_q8_1": (None, [P, I64, P]),
            "ora_ref_vec_dot_q4_K_q8_1": (C.c_float, [P, P, I]),
            "ora_ref_vec_dot_q5_K_q8_1": (C.c_float, [P, P, I]),
            "ora_ref_vec_dot_q6_K_q8_1": (C.c_float, [P, P, I]),
            "ora_ref_vec_dot_q8_0_q8_1": (C.c_float, [P, P, I]),
            "ora_ref_vec_dot_iq4_xs_q8_1": (C.c_float, [P, P, I]),
            "ora_quantize_row_q8_K": (None, [P, P, I64]),
            "ora_sample": (I, [P, P, I, C.c_float, C.c_float, C.c_float, C.c_float]),
            "ora_quantize_row_q8_0_act": (None, [P, P, I64]),
            "ora_gemv_cpu": (I, [I, P, I, I, P, P, I]),
            "ora_gemv_cpu_simd": (I, [I, P, I, I, P, P, I]),
            "ora_simd_vec_dot_q4_K_q8_K": (C.c_float, [I, P, P]),
            "ora_simd_vec_dot_q6_K_q8_K": (C.c_float, [I, P, P]),
            "ora_simd_vec_dot_q8_0_q8_0": (C.c_float, [I, P, P]),
            "ora_topk": (I, [P, I, I, P, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ------------------------------------------------------------------ fp16 --

def fp16_to_fp32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().ora_fp16_to_fp32_n(_p(h), _p(out), h.size)
    return out


def fp32_to_fp16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().ora_fp32_to_fp16_n(_p(f), _p(out), f.size)
    return out


# ------------------------------------------------------------ weights --

def row_bytes(type_: int, k: int) -> int:
    be = BLOCK_ELEMS[type_]
    assert k % be == 0
    return k // be * TYPE_SIZE[type_]


def quantize(type_: int, w: np.ndarray) -> np.ndarray:
    """fp32 [rc, K] -> GGUF blocks as uint8 [rc, row_bytes]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rc, k = w.shape
    if type_ == F32:
        return w.view(np.uint8).reshape(rc, k * 4).copy()
    if type_ == F16:
        return fp32_to_fp16(w).view(np.uint8).reshape(rc, k * 2).copy()
    out = np.empty((rc, row_bytes(type_, k)), np.uint8)
    fn = {Q4_K: lib().ora_quantize_row_q4_K, Q5_K: lib().ora_quantize_row_q5_K, Q6_K: lib().ora_quantize_row_q6_K,
          Q8_0: lib().ora_quantize_row_q8_0, IQ4_XS: lib().ora_quantize_row_iq4_xs}[type_]
    fn(_p(w), _p(out), w.size)  # rows are contiguous: one call quantizes them all
    return out


def dequant(type_: int, blocks: np.ndarray, rb: int, rc: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks)
    out = np.empty((rc, rb * BLOCK_ELEMS[type_]), np.float32)
    assert blocks.nbytes >= rc * rb * TYPE_SIZE[type_]
    rc_ = lib().ora_dequant_rows(type_, _p(blocks), rb, rc, _p(out))
    assert rc_ == 0
    return out


def synth_weights(type_: int, rc: int, k: int, seed: int, std: float = 0.02) -> np.ndarray:
    """Seeded N(0, std) fp32 weights quantized to GGUF blocks (chunked)."""
    rng = np.random.default_rng(seed)
    out = np.empty((rc, row_bytes(type_, k)), np.uint8)
    step = max(1, (1 << 24) // k)
    for r0 in range(0, rc, step):
        r1 = min(rc, r0 + step)
        w = (rng.standard_normal((r1 - r0, k), dtype=np.float32) * np.float32(std))
        out[r0:r1] = quantize(type_, w)
    return out


# -------------------------------------------------------- activations --

def quant_act(x: np.ndarray):
    """fp32 [..., K] -> (codes int8 [..., K], d f32 [..., K/32], s u32 [..., K/32])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    assert k % 32 == 0
    q = np.empty(x.shape, np.int8)
    d = np.empty(x.shape[:-1] + (k // 32,), np.float32)
    s = np.empty(x.shape[:-1] + (k // 32,), np.uint32)
    lib().ora_quant_act(_p(x), x.size, _p(q), _p(d), _p(s))
    return q, d, s


def quant_act_gated(x: np.ndarray, g: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(g, dtype=np.float32)
    k = x.shape[-1]
    q = np.empty(x.shape, np.int8)
    d = np.empty(x.shape[:-1] + (k // 32,), np.float32)
    s = np.empty(x.shape[:-1] + (k // 32,), np.uint32)
    lib().ora_quant_act_gated(_p(x), _p(g), x.size, _p(q), _p(d), _p(s))
    return q, d, s


def exp_cw(t: np.ndarray) -> np.ndarray:
    """The build's fixed exp (ora_exp_cw), elementwise on float32."""
    t = np.ascontiguousarray(t, dtype=np.float32)
    out = np.empty(t.shape, np.float32)
    lib().ora_exp_cw_n(_p(t), _p(out), t.size)
    return out


def gated(x: np.ndarray, g: np.ndarray) -> np.ndarray:
    """x * (1 / (1 + e^-g)) with the fixed exp (ora_gated), elementwise."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(g, dtype=np.float32)
    out = np.empty(x.shape, np.float32)
    lib().ora_gated_n(_p(x), _p(g), _p(out), x.size)
    return out


def gemv_act(type_: int, blocks: np.ndarray, rb: int, rc: int, q, d, s):
    """Integer-dot oracle in fp64; returns (y, norm) each float64 [rc]."""
    blocks = np.ascontiguousarray(blocks)
    y = np.empty(rc, np.float64)
    nrm = np.empty(rc, np.float64)
    q, d, s = (np.ascontiguousarray(a) for a in (q, d, s))
    assert lib().ora_gemv_act(type_, _p(blocks), rb, rc, _p(q), _p(d), _p(s), _p(y), _p(nrm)) == 0
    return y, nrm


def gemv_f64(type_: int, blocks: np.ndarray, rb: int, rc: int, x: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rc, np.float64)
    assert lib().ora_gemv_f64(type_, _p(blocks), rb, rc, _p(x), _p(y)) == 0
    return y


# ------------------------------------ the reference's q8_1 formulation --

Q8_1_DTYPE = np.dtype([("d", "<u2"), ("s", "<u2"), ("qs", "i1", 32)])


def quant_q8_1(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 32, Q8_1_DTYPE)
    lib().ora_quant_q8_1(_p(x), x.size, out.ctypes.data)
    return out


def ref_vec_dot_q8_1(type_: int, wrow: np.ndarray, xq: np.ndarray, rb: int) -> float:
    wrow = np.ascontiguousarray(wrow)
    fn = {Q4_K: lib().ora_ref_vec_dot_q4_K_q8_1, Q5_K: lib().ora_ref_vec_dot_q5_K_q8_1,
          Q6_K: lib().ora_ref_vec_dot_q6_K_q8_1,
          Q8_0: lib().ora_ref_vec_dot_q8_0_q8_1, IQ4_XS: lib().ora_ref_vec_dot_iq4_xs_q8_1}[type_]
    return float(fn(_p(wrow), xq.ctypes.data, rb))


# ---------------------------------------- ggml CPU path (q8_K, q8_0) --

def quant_cpu_act(type_: int, x: np.ndarray) -> np.ndarray:
    """Activation in the format ggml's CPU dot pairs with the weight type."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if type_ == Q8_0:
        out = np.empty(x.size // 32 * 34, np.uint8)
        lib().ora_quantize_row_q8_0_act(_p(x), _p(out), x.size)
    else:
        out = np.empty(x.size // 256 * 292, np.uint8)
        lib().ora_quantize_row_q8_K(_p(x), _p(out), x.size)
    return out


Q8_K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
Q8_0_DTYPE = np.dtype([("d", "<u2"), ("qs", "i1", 32)])


def cpu_act_values(type_: int, xq: np.ndarray) -> np.ndarray:
    """The activation a q8_K / q8_0 buffer stands for, d * q, in float64."""
    if type_ == Q8_0:
        b = np.frombuffer(np.ascontiguousarray(xq).tobytes(), Q8_0_DTYPE)
        d = fp16_to_fp32(b["d"]).astype(np.float64)
    else:
        b = np.frombuffer(np.ascontiguousarray(xq).tobytes(), Q8_K_DTYPE)
        d = b["d"].astype(np.float64)
    return (d[:, None] * b["qs"].astype(np.float64)).reshape(-1)


def vec_dot_cpu(type_: int, wrow: np.ndarray, xq: np.ndarray, n: int) -> float:
    """One row of ggml_vec_dot_{q4_K_q8_K, q6_K_q8_K, q8_0_q8_0} (restated)."""
    fn = {Q4_K: lib().ora_vec_dot_q4_K_q8_K, Q6_K: lib().ora_vec_dot_q6_K_q8_K,
          Q8_0: lib().ora_vec_dot_q8_0_q8_0}[type_]
    wrow = np.ascontiguousarray(wrow)
    xq = np.ascontiguousarray(xq)
    return float(fn(n, _p(wrow), _p(xq)))


def gemv_cpu(type_: int, blocks: np.ndarray, rb: int, rc: int, xq: np.ndarray, nthreads: int = 1,
             simd: bool = False) -> np.ndarray:
    """ggml's CPU path as restated: scalar C, or the AVX2 build (simd)."""
    blocks = np.ascontiguousarray(blocks)
    y = np.empty(rc, np.float32)
    fn = lib().ora_gemv_cpu_simd if simd else lib().ora_gemv_cpu
    assert fn(type_, _p(blocks), rb, rc, _p(xq), _p(y), nthreads) == 0
    return y


# ---------------------------------------------------------------- top-k --

def sample(idx: np.ndarray, val: np.ndarray, temperature: float, min_p: float, top_p: float, u: float) -> int:
    idx = np.ascontiguousarray(idx, np.int32)
    val = np.ascontiguousarray(val, np.float32)
    return int(lib().ora_sample(_p(idx), _p(val), idx.size, temperature, min_p, top_p, u))


def topk(v: np.ndarray, k: int):
    v = np.ascontiguousarray(v, dtype=np.float32)
    idx = np.empty(k, np.int32)
    val = np.empty(k, np.float32)
    assert lib().ora_topk(_p(v), v.size, k, _p(idx), _p(val)) == 0
    return idx, val


# ------------------------------------- the reference's own C (oracle/_ref) --

def ref_lib():
    """dequantize_row_q4_K built from the reference's debug/official_dequant.c,
    or None where that build is absent (it is made only where the reference
    checkout exists)."""
    if not os.path.exists(REF_LIB_PATH):
        return None
    L = C.CDLL(REF_LIB_PATH)
    L.dequantize_row_q4_K.restype = None
    L.dequantize_row_q4_K.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    return L
