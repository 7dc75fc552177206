"""ctypes binding of libm27q.so (include/m27q.h) for Python callers.

Device buffers are torch tensors (PyTorch supplies device memory and streams);
every call goes through the C ABI.  There is no fallback: if the library is
not built, loading fails with an error.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "libm27q.so")
HEADER = os.path.join(ROOT, "include", "m27q.h")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS = 0, 1, 8, 12, 13, 14, 23
GGUF, TILED = 0, 1
BLOCK_ELEMS = {F32: 1, F16: 1, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ4_XS: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ4_XS: 136}

STATUS = {0: "M27Q_OK", 1: "M27Q_ERR_NULL", 2: "M27Q_ERR_SHAPE", 3: "M27Q_ERR_TYPE",
          4: "M27Q_ERR_LAYOUT", 5: "M27Q_ERR_SCRATCH", 6: "M27Q_ERR_RANGE", 7: "M27Q_ERR_HIP", 8: "M27Q_ERR_IO"}


class M27QError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: {STATUS.get(status, status)}")
        self.status = status


class WeightDesc(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("ggml_type", C.c_uint32), ("row_blocks", C.c_uint32),
                ("row_count", C.c_uint32), ("layout", C.c_uint32)]


class BlobTensor(C.Structure):
    """m27q_blob_tensor: one entry of a .m27b weights section."""
    _fields_ = [("name", C.c_char * 64), ("ggml_type", C.c_uint32), ("source_model", C.c_uint32),
                ("role", C.c_uint32), ("row_elems", C.c_uint32), ("row_count", C.c_uint32),
                ("layout", C.c_uint32), ("row_blocks", C.c_uint32), ("pad", C.c_uint32),
                ("file_offset", C.c_uint64), ("bytes", C.c_uint64)]


_P, _I, _SZ, _U32 = C.c_void_p, C.c_int, C.c_size_t, C.c_uint32
_SIGS = {
    "m27q_status_string": (C.c_char_p, [_I]),
    "m27q_row_size": (_SZ, [_U32, _U32]),
    "m27q_weight_bytes": (_SZ, [_U32, _U32, _U32, _U32]),
    "m27q_repack": (_I, [_U32, _U32, _U32, _P, _P]),
    "m27q_unpack": (_I, [_U32, _U32, _U32, _P, _P]),
    "m27q_retile_blob": (_I, [C.c_char_p, C.c_char_p]),
    "m27q_blob_tensors": (_I, [C.c_char_p, C.POINTER(BlobTensor), _I, C.POINTER(_I)]),
    "m27q_blob_load": (_I, [C.c_char_p, C.POINTER(BlobTensor), _P, _SZ, C.POINTER(WeightDesc)]),
    "m27q_act_bytes": (_SZ, [_I, _I]),
    "m27q_act_d_offset": (_SZ, [_I, _I]),
    "m27q_act_s_offset": (_SZ, [_I, _I]),
    "m27q_quant_act": (_I, [_P, _I, _I, _P, _P]),
    "m27q_quant_act_gated": (_I, [_P, _P, _I, _I, _P, _P]),
    "m27q_matvec_q8": (_I, [C.POINTER(WeightDesc), _P, _P, _P, _P, _P]),
    "m27q_matvec_q8_multi": (_I, [_I, C.POINTER(WeightDesc), _P, C.POINTER(_P), _P]),
    "m27q_matvec_multi": (_I, [_I, C.POINTER(WeightDesc), _P, C.POINTER(_P), _P]),
    "m27q_ffn_swiglu": (_I, [C.POINTER(WeightDesc), C.POINTER(WeightDesc), _P, _P, _P, _P]),
    "m27q_ffn_swiglu_q8": (_I, [C.POINTER(WeightDesc), C.POINTER(WeightDesc), _P, _P, _P, _P]),
    "m27q_matvec_f32": (_I, [C.POINTER(WeightDesc), _P, _P, _P, _P]),
    "m27q_matvec": (_I, [C.POINTER(WeightDesc), _P, _P, _P, _P, _P]),
    "m27q_matmul_q8": (_I, [C.POINTER(WeightDesc), _I, _P, _P, _P, _P]),
    "m27q_matmul_q8_multi": (_I, [_I, C.POINTER(WeightDesc), _I, _P, C.POINTER(_P), _P]),
    "m27q_dequant_rows": (_I, [C.POINTER(WeightDesc), _I, _I, _P, _P]),
    "m27q_embed_rows": (_I, [C.POINTER(WeightDesc), _P, _I, _P, _P, _P]),
    "m27q_embed_token": (_I, [C.POINTER(WeightDesc), C.c_int32, _P, _P]),
    "m27q_topk_scratch_bytes": (_SZ, [_I, _I]),
    "m27q_topk": (_I, [_P, _I, _I, _P, _P, _P, _SZ, _P]),
    "m27q_topk_noalloc": (_I, [_P, _I, _I, _P, _P, _P]),
    "m27q_sample": (_I, [_P, _P, _I, C.c_float, C.c_float, C.c_float, _P, _P, _P]),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"M27Q_API\s+[\w\s\*]*?\b(m27q_\w+)\s*\(", text)))


def check(status: int, what: str) -> None:
    if status != 0:
        raise M27QError(status, what)


# ------------------------------------------------------------ host side --

def row_size(type_: int, ne: int) -> int:
    return lib().m27q_row_size(type_, ne)


def weight_bytes(type_: int, rb: int, rc: int, layout: int) -> int:
    return lib().m27q_weight_bytes(type_, rb, rc, layout)


def repack(type_: int, rb: int, rc: int, gguf: np.ndarray) -> np.ndarray:
    gguf = np.ascontiguousarray(gguf, dtype=np.uint8)
    out = np.empty(weight_bytes(type_, rb, rc, TILED), np.uint8)
    check(lib().m27q_repack(type_, rb, rc, gguf.ctypes.data, out.ctypes.data), "m27q_repack")
    return out


def unpack(type_: int, rb: int, rc: int, tiled: np.ndarray) -> np.ndarray:
    tiled = np.ascontiguousarray(tiled, dtype=np.uint8)
    out = np.empty(rc * rb * BLOCK_BYTES[type_], np.uint8)
    check(lib().m27q_unpack(type_, rb, rc, tiled.ctypes.data, out.ctypes.data), "m27q_unpack")
    return out


def retile_blob(in_path: str, out_path: str) -> None:
    """Copy a .m27b blob with its quantized matrices re-tiled (host, pack time)."""
    check(lib().m27q_retile_blob(in_path.encode(), out_path.encode()), "m27q_retile_blob")


def blob_tensors(path: str) -> list:
    """The entry table of a .m27b blob as BlobTensor records (host only)."""
    n = C.c_int(0)
    check(lib().m27q_blob_tensors(path.encode(), None, 0, C.byref(n)), "m27q_blob_tensors")
    out = (BlobTensor * n.value)()
    check(lib().m27q_blob_tensors(path.encode(), out, n.value, C.byref(n)), "m27q_blob_tensors")
    return list(out)


def act_bytes(M: int, K: int) -> int:
    return lib().m27q_act_bytes(M, K)


def act_offsets(M: int, K: int):
    return lib().m27q_act_d_offset(M, K), lib().m27q_act_s_offset(M, K)


# ----------------------------------------------------------- device side --

def _torch():
    import torch
    return torch


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


class Weight:
    """A quantized weight resident in device memory."""

    def __init__(self, data, type_: int, rb: int, rc: int, layout: int):
        self.data, self.type, self.rb, self.rc, self.layout = data, type_, rb, rc, layout

    @property
    def K(self) -> int:
        return self.rb * BLOCK_ELEMS[self.type]

    @property
    def nbytes_gguf(self) -> int:
        return self.rb * self.rc * BLOCK_BYTES[self.type]

    def desc(self) -> WeightDesc:
        return WeightDesc(self.data.data_ptr(), self.type, self.rb, self.rc, self.layout)

    @staticmethod
    def upload(gguf_rows: np.ndarray, type_: int, rb: int, rc: int, layout: int = TILED, device="cuda"):
        torch = _torch()
        host = np.ascontiguousarray(gguf_rows, dtype=np.uint8).reshape(-1)
        if layout == TILED:
            host = repack(type_, rb, rc, host)
        data = torch.from_numpy(host).to(device)
        return Weight(data, type_, rb, rc, layout)


def blob_load(path: str, t: BlobTensor, device="cuda") -> Weight:
    """Upload one blob tensor (m27q_blob_load) into a new device buffer."""
    torch = _torch()
    data = torch.empty(max(1, int(t.bytes)), dtype=torch.uint8, device=device)
    d = WeightDesc()
    check(lib().m27q_blob_load(path.encode(), C.byref(t), data.data_ptr(), data.numel(), C.byref(d)),
          "m27q_blob_load")
    return Weight(data, d.ggml_type, d.row_blocks, d.row_count, d.layout)


class Act:
    """A quantized activation buffer (codes, scales, sums) for M rows of K."""

    def __init__(self, M: int, K: int, device="cuda"):
        torch = _torch()
        self.M, self.K = M, K
        self.buf = torch.zeros(act_bytes(M, K), dtype=torch.uint8, device=device)

    def parts(self):
        """(codes int8 [M,K], d f32 [M,K/32], sums u32-as-int32 [M,K/32]) views."""
        torch = _torch()
        d_off, s_off = act_offsets(self.M, self.K)
        n = self.M * self.K
        g = self.M * (self.K // 32)
        codes = self.buf[:n].view(torch.int8).view(self.M, self.K)
        d = self.buf[d_off:d_off + 4 * g].view(torch.float32).view(self.M, self.K // 32)
        s = self.buf[s_off:s_off + 4 * g].view(torch.int32).view(self.M, self.K // 32)
        return codes, d, s


def quant_act(x, act: Act, gate=None, stream=None) -> None:
    if gate is None:
        check(lib().m27q_quant_act(_ptr(x), act.M, act.K, _ptr(act.buf), _stream(stream)), "m27q_quant_act")
    else:
        check(lib().m27q_quant_act_gated(_ptr(x), _ptr(gate), act.M, act.K, _ptr(act.buf), _stream(stream)),
              "m27q_quant_act_gated")


def matvec_q8(w: Weight, act: Act, y, residual=None, yq: Act | None = None, stream=None) -> None:
    d = w.desc()
    check(lib().m27q_matvec_q8(C.byref(d), _ptr(act.buf), _ptr(y), _ptr(residual),
                               None if yq is None else _ptr(yq.buf), _stream(stream)), "m27q_matvec_q8")


def matvec_q8_multi(ws: list[Weight], act: Act, ys: list, stream=None) -> None:
    n = len(ws)
    descs = (WeightDesc * n)(*[w.desc() for w in ws])
    yp = (C.c_void_p * n)(*[_ptr(y) for y in ys])
    check(lib().m27q_matvec_q8_multi(n, descs, _ptr(act.buf), yp, _stream(stream)), "m27q_matvec_q8_multi")


def matvec_multi(ws: list[Weight], x, ys: list, stream=None) -> None:
    """fp32 activation x shared by up to 4 weights (quantized inside the kernel)."""
    n = len(ws)
    descs = (WeightDesc * n)(*[w.desc() for w in ws])
    yp = (C.c_void_p * n)(*[_ptr(y) for y in ys])
    check(lib().m27q_matvec_multi(n, descs, _ptr(x), yp, _stream(stream)), "m27q_matvec_multi")


def ffn_swiglu_q8(gate: Weight, up: Weight, act: Act, y, yq: Act | None = None, stream=None) -> None:
    g, u = gate.desc(), up.desc()
    check(lib().m27q_ffn_swiglu_q8(C.byref(g), C.byref(u), _ptr(act.buf), _ptr(y),
                                   None if yq is None else _ptr(yq.buf), _stream(stream)), "m27q_ffn_swiglu_q8")


def ffn_swiglu(gate: Weight, up: Weight, x, y, yq: Act | None = None, stream=None) -> None:
    """fp32 activation x (quantized inside the kernel)."""
    g, u = gate.desc(), up.desc()
    check(lib().m27q_ffn_swiglu(C.byref(g), C.byref(u), _ptr(x), _ptr(y),
                                None if yq is None else _ptr(yq.buf), _stream(stream)), "m27q_ffn_swiglu")


def matvec_f32(w: Weight, x, y, residual=None, stream=None) -> None:
    d = w.desc()
    check(lib().m27q_matvec_f32(C.byref(d), _ptr(x), _ptr(y), _ptr(residual), _stream(stream)), "m27q_matvec_f32")


def matvec(w: Weight, x, y, residual=None, yq: Act | None = None, stream=None) -> None:
    """fp32 activation x (quantized inside the kernel); F16/F32 weights take the fp32 path."""
    d = w.desc()
    check(lib().m27q_matvec(C.byref(d), _ptr(x), _ptr(y), _ptr(residual), None if yq is None else _ptr(yq.buf),
                            _stream(stream)), "m27q_matvec")


def matmul_q8(w: Weight, act: Act, Y, residual=None, stream=None) -> None:
    d = w.desc()
    check(lib().m27q_matmul_q8(C.byref(d), act.M, _ptr(act.buf), _ptr(Y), _ptr(residual), _stream(stream)),
          "m27q_matmul_q8")


def matmul_q8_multi(ws: list[Weight], act: Act, Ys: list, stream=None) -> None:
    n = len(ws)
    descs = (WeightDesc * n)(*[w.desc() for w in ws])
    yp = (C.c_void_p * n)(*[_ptr(y) for y in Ys])
    check(lib().m27q_matmul_q8_multi(n, descs, act.M, _ptr(act.buf), yp, _stream(stream)), "m27q_matmul_q8_multi")


def dequant_rows(w: Weight, row0: int, nrows: int, out, stream=None) -> None:
    d = w.desc()
    check(lib().m27q_dequant_rows(C.byref(d), row0, nrows, _ptr(out), _stream(stream)), "m27q_dequant_rows")


def embed_rows(w: Weight, ids, out, bad=None, stream=None) -> None:
    d = w.desc()
    check(lib().m27q_embed_rows(C.byref(d), _ptr(ids), ids.numel(), _ptr(out), _ptr(bad), _stream(stream)),
          "m27q_embed_rows")


def embed_token(w: Weight, token_id: int, out, stream=None) -> None:
    d = w.desc()
    check(lib().m27q_embed_token(C.byref(d), token_id, _ptr(out), _stream(stream)), "m27q_embed_token")


def topk_scratch_bytes(n: int, k: int) -> int:
    return lib().m27q_topk_scratch_bytes(n, k)


def sample(idx, val, k: int, temperature: float, min_p: float, top_p: float, u, token, stream=None) -> None:
    """token[0] <- the candidate sample() picks for the uniform u[0] (device tensors)."""
    check(lib().m27q_sample(_ptr(idx), _ptr(val), k, temperature, min_p, top_p, _ptr(u), _ptr(token),
                            _stream(stream)), "m27q_sample")


def topk(logits, k: int, idx, val, scratch, stream=None) -> None:
    n = logits.numel()
    check(lib().m27q_topk(_ptr(logits), n, k, _ptr(idx), _ptr(val), _ptr(scratch),
                          scratch.numel() * scratch.element_size(), _stream(stream)), "m27q_topk")


def topk_noalloc(logits, k: int, idx, val, stream=None) -> None:
    """m27q_topk on the library's static scratch (no scratch argument)."""
    check(lib().m27q_topk_noalloc(_ptr(logits), logits.numel(), k, _ptr(idx), _ptr(val), _stream(stream)),
          "m27q_topk_noalloc")
