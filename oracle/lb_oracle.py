"""ctypes binding of liblb_oracle.so — the CPU restatement of the reference path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product (lbhip) never
imports it.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "liblb_oracle.so"

F32, Q4_K, Q5_K, Q8_K, IQ3_S, IQ2_S = 0, 12, 13, 15, 21, 22
BLOCK_BYTES = {F32: 4, Q4_K: 144, Q5_K: 176, IQ2_S: 82, IQ3_S: 110, Q8_K: 292}
MODE_DEQUANT_F32, MODE_LLAMA_Q8K, MODE_CPU_PARALLEL_Q8K = 0, 1, 2

STATUS = {
    0: "Ok", 1: "UnsupportedType", 2: "ZeroLogicalElements", 3: "LogicalElementsNotDivisible",
    4: "ArithmeticOverflow", 6: "EncodedLengthMismatch", 7: "OutputLengthMismatch",
    8: "NonFiniteScale", 9: "NonFiniteActivation", 10: "NonFiniteQ8Scale",
    20: "DimensionMismatch", 21: "ScratchTooSmall", 22: "NonFiniteValue",
    23: "RoutedExpertOrder", 24: "DuplicateRoutedExpert", 25: "InvalidParameter",
}


class LboError(C.Structure):
    _fields_ = [("status", C.c_int32), ("ty", C.c_int32), ("index", C.c_uint64),
                ("expected", C.c_uint64), ("actual", C.c_uint64), ("bits", C.c_uint32),
                ("field", C.c_uint32)]


class LboMatrix(C.Structure):
    _fields_ = [("ty", C.c_int32), ("rows", C.c_uint64), ("k", C.c_uint64),
                ("bytes", C.c_void_p)]


class LboExec(C.Structure):
    _fields_ = [("mode", C.c_int32), ("threads", C.c_int32), ("avx2", C.c_int32)]


class LboExpert(C.Structure):
    _fields_ = [("gate", LboMatrix), ("up", LboMatrix), ("down", LboMatrix)]


class OracleError(Exception):
    def __init__(self, err: LboError):
        self.status = STATUS.get(err.status, str(err.status))
        self.index, self.expected, self.actual = err.index, err.expected, err.actual
        self.bits, self.field, self.ty = err.bits, err.field, err.ty
        super().__init__(f"{self.status}(ty={self.ty}, index={self.index}, expected={self.expected}, "
                         f"actual={self.actual}, bits={self.bits:#x}, field={self.field})")


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built (run `make -C oracle`)")
        L = C.CDLL(str(LIB_PATH))
        p = C.c_void_p
        L.lbo_quantize_row_q8_k.argtypes = [p, C.c_size_t, p, C.c_size_t, C.POINTER(LboError)]
        L.lbo_vec_dot_q8_k.argtypes = [C.c_int, p, C.c_size_t, p, C.c_size_t, C.c_size_t, p, C.POINTER(LboError)]
        L.lbo_vec_dot_q8_k_avx2.argtypes = L.lbo_vec_dot_q8_k.argtypes
        L.lbo_dot_scalar.argtypes = [C.c_int, p, p, C.c_size_t]
        L.lbo_dot_scalar.restype = C.c_float
        L.lbo_dot_avx2.argtypes = [C.c_int, p, p, C.c_size_t]
        L.lbo_dot_avx2.restype = C.c_float
        L.lbo_block_sums.argtypes = [C.c_int, p, p, C.c_size_t, p]
        L.lbo_decode_row.argtypes = [C.c_int, p, C.c_size_t, C.c_size_t, p, C.c_size_t, C.POINTER(LboError)]
        L.lbo_gemv.argtypes = [C.POINTER(LboExec), C.POINTER(LboMatrix), p, C.c_size_t, p, C.c_size_t,
                               p, C.c_size_t, C.POINTER(LboError)]
        L.lbo_gemv_accumulate.argtypes = [C.POINTER(LboExec), C.POINTER(LboMatrix), p, C.c_size_t, p,
                                          C.c_size_t, C.c_float, p, C.c_size_t, C.POINTER(LboError)]
        L.lbo_gemv_prequantized.argtypes = [C.POINTER(LboExec), C.POINTER(LboMatrix), p, p]
        L.lbo_apply_swiglu.argtypes = [p, p, C.c_size_t]
        L.lbo_apply_swiglu.restype = C.c_int64
        L.lbo_moe_routed_by_id.argtypes = [C.POINTER(LboExec), p, p, C.c_size_t, C.POINTER(LboExpert),
                                           C.c_size_t, C.POINTER(LboExpert), p, p, C.c_int,
                                           C.POINTER(LboError)]
        L.lbo_residual_add_in_place.argtypes = [p, C.c_size_t, p, C.c_size_t, C.POINTER(LboError)]
        L.lbo_route_sigmoid_bias.argtypes = [p, p, C.c_size_t, C.c_size_t, C.c_float, p, p, C.POINTER(LboError)]
        L.lbo_route_softmax_topk.argtypes = [p, C.c_size_t, C.c_size_t, p, p, C.POINTER(LboError)]
        L.lbo_router_logits_f32.argtypes = [p, C.c_size_t, C.c_size_t, p, p]
        L.lbo_router_logits_f32.restype = None
        L.lbo_f16_to_f32.argtypes = [C.c_uint16]
        L.lbo_f16_to_f32.restype = C.c_float
        L.lbo_expf.argtypes = [C.c_float]
        L.lbo_expf.restype = C.c_float
        L.lbo_expf_array.argtypes = [p, p, C.c_size_t]
        L.lbo_expf_array.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _check(st: int, err: LboError) -> None:
    if st != 0:
        raise OracleError(err)


def quantize_row_q8_k_into(x: np.ndarray, encoded: np.ndarray) -> None:
    """Mirror of quantize_row_q8_k_into (q8_k.rs:16-76); encoded untouched on error."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert encoded.dtype == np.uint8 and encoded.flags.c_contiguous
    err = LboError()
    _check(lib().lbo_quantize_row_q8_k(_ptr(x), x.size, _ptr(encoded), encoded.size, C.byref(err)), err)


def quantize_q8_k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.zeros(x.size // 256 * 292, np.uint8)
    quantize_row_q8_k_into(x, out)
    return out


def vec_dot_q8_k(ty: int, w: np.ndarray, q8: np.ndarray, n: int, avx2: bool = False) -> float:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    q8 = np.ascontiguousarray(q8, dtype=np.uint8)
    out = np.zeros(1, np.float32)
    err = LboError()
    fn = lib().lbo_vec_dot_q8_k_avx2 if avx2 else lib().lbo_vec_dot_q8_k
    _check(fn(ty, _ptr(w), w.size, _ptr(q8), q8.size, n, _ptr(out), C.byref(err)), err)
    return out


def block_sums(ty: int, w_row: np.ndarray, q8: np.ndarray) -> np.ndarray:
    blocks = q8.size // 292
    per = 9 if ty in (Q4_K, Q5_K) else 1
    out = np.zeros(blocks * per, np.int32)
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    q8 = np.ascontiguousarray(q8, dtype=np.uint8)
    assert lib().lbo_block_sums(ty, _ptr(w_row), _ptr(q8), blocks, _ptr(out)) == 0
    return out.reshape(blocks, per) if per > 1 else out


def decode_row(ty: int, w: np.ndarray, n: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.zeros(n, np.float32)
    err = LboError()
    _check(lib().lbo_decode_row(ty, _ptr(w), w.size, n, _ptr(out), out.size, C.byref(err)), err)
    return out


def make_matrix(ty: int, rows: int, k: int, data: np.ndarray) -> LboMatrix:
    m = LboMatrix(ty, rows, k, _ptr(data))
    m._keep = data  # keep the bytes alive
    return m


def make_exec(mode: int = MODE_LLAMA_Q8K, threads: int = 1, avx2: bool = False) -> LboExec:
    return LboExec(mode, threads, 1 if avx2 else 0)


def gemv(ex: LboExec, m: LboMatrix, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(m.rows, np.float32)
    q8 = np.zeros(max(m.k // 256 * 292, 1), np.uint8)
    err = LboError()
    _check(lib().lbo_gemv(C.byref(ex), C.byref(m), _ptr(x), x.size, _ptr(y), y.size, _ptr(q8),
                          q8.size if m.k % 256 == 0 else 0, C.byref(err)), err)
    return y


def gemv_accumulate(ex: LboExec, m: LboMatrix, x: np.ndarray, dest: np.ndarray, scale: float) -> None:
    x = np.ascontiguousarray(x, dtype=np.float32)
    q8 = np.zeros(max(m.k // 256 * 292, 1), np.uint8)
    err = LboError()
    _check(lib().lbo_gemv_accumulate(C.byref(ex), C.byref(m), _ptr(x), x.size, _ptr(dest), dest.size,
                                     scale, _ptr(q8), q8.size, C.byref(err)), err)


def gemv_prequantized(ex: LboExec, m: LboMatrix, q8: np.ndarray) -> np.ndarray:
    q8 = np.ascontiguousarray(q8, dtype=np.uint8)
    y = np.zeros(m.rows, np.float32)
    assert lib().lbo_gemv_prequantized(C.byref(ex), C.byref(m), _ptr(q8), _ptr(y)) == 0
    return y


def make_expert(gate: LboMatrix, up: LboMatrix, down: LboMatrix) -> LboExpert:
    e = LboExpert(gate, up, down)
    e._keep = (gate._keep, up._keep, down._keep)
    return e


def moe_routed_by_id(ex: LboExec, ids, coefs, experts: list, shared: LboExpert, x: np.ndarray,
                     preflight: bool = True) -> np.ndarray:
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    coefs = np.ascontiguousarray(coefs, dtype=np.float32)
    arr = (LboExpert * len(experts))(*experts)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(shared.down.rows, np.float32)
    err = LboError()
    _check(lib().lbo_moe_routed_by_id(C.byref(ex), _ptr(ids), _ptr(coefs), ids.size, arr, len(experts),
                                      C.byref(shared), _ptr(x), _ptr(out), 1 if preflight else 0,
                                      C.byref(err)), err)
    return out


def moe_routed_by_id_status(ex: LboExec, ids, coefs, experts: list, shared: LboExpert, x: np.ndarray,
                            out: np.ndarray, preflight: bool = True) -> LboError:
    """As moe_routed_by_id, but returns the error record and leaves `out` as the
    reference leaves its output (unchanged, or partially accumulated)."""
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    coefs = np.ascontiguousarray(coefs, dtype=np.float32)
    arr = (LboExpert * len(experts))(*experts)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    err = LboError()
    lib().lbo_moe_routed_by_id(C.byref(ex), _ptr(ids), _ptr(coefs), ids.size, arr, len(experts), C.byref(shared),
                               _ptr(x), _ptr(out), 1 if preflight else 0, C.byref(err))
    return err


def residual_add_in_place(destination: np.ndarray, residual) -> None:
    """residual_add_in_place (norm.rs:83-98): destination += residual; untouched on error."""
    assert destination.dtype == np.float32 and destination.flags.c_contiguous
    residual = np.ascontiguousarray(residual, dtype=np.float32)
    err = LboError()
    _check(lib().lbo_residual_add_in_place(_ptr(destination), destination.size, _ptr(residual), residual.size,
                                           C.byref(err)), err)


def route_sigmoid_bias(logits, bias, top_k: int, weight_scale: float):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    ids = np.zeros(top_k, np.uint32)
    coefs = np.zeros(top_k, np.float32)
    err = LboError()
    _check(lib().lbo_route_sigmoid_bias(_ptr(logits), _ptr(bias), logits.size, top_k, weight_scale,
                                        _ptr(ids), _ptr(coefs), C.byref(err)), err)
    return ids, coefs


def route_softmax_topk(logits, top_k: int):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.zeros(top_k, np.uint32)
    coefs = np.zeros(top_k, np.float32)
    err = LboError()
    _check(lib().lbo_route_softmax_topk(_ptr(logits), logits.size, top_k, _ptr(ids), _ptr(coefs),
                                        C.byref(err)), err)
    return ids, coefs


def router_logits_f32(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    n_experts = w.size // x.size
    out = np.zeros(n_experts, np.float32)
    lib().lbo_router_logits_f32(_ptr(w), n_experts, x.size, _ptr(x), _ptr(out))
    return out


def apply_swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.array(gate, dtype=np.float32, copy=True)
    u = np.ascontiguousarray(up, dtype=np.float32)
    bad = lib().lbo_apply_swiglu(_ptr(g), _ptr(u), g.size)
    if bad >= 0:
        raise OracleError(LboError(22, 0, bad, 0, 0, 0, 5))
    return g


def expf_array(x: np.ndarray) -> np.ndarray:
    """The host C library's expf (what the reference's f32::exp links) over an array."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().lbo_expf_array(_ptr(x), _ptr(out), x.size)
    return out


def default_threads() -> int:
    """recommended_thread_count (crates/bridge-kernels-cpu/src/lib.rs:121-126)."""
    n = os.cpu_count() or 1
    return max(1, (n + 1) // 2)
