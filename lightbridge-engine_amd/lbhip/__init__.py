"""Python mirror of the reference's quantized-dot API over the HIP C ABI.

The names, argument meanings and error variants follow the reference crates:
``quantize_row_q8_k_into`` (crates/bridge-quant-layout/src/q8_k.rs:16),
``gemv_into`` / ``gemv_accumulate_scaled_into``
(crates/bridge-kernels-reference/src/gemv.rs:88, :117), and the backend object
mirrors ``CpuBackend`` (crates/bridge-kernels-cpu/src/lib.rs:59-119).  Device
buffers are torch CUDA tensors (PyTorch is only the allocator and stream
provider); every call goes through liblightbridge_hip.so.  There is no CPU
fallback: if the library or a gfx950 device is missing, construction raises.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_DIR / "liblightbridge_hip.so"

F32, Q4_K, Q5_K, Q8_K, IQ3_S, IQ2_S = 0, 12, 13, 15, 21, 22
Q8_K_BLOCK_ELEMENTS, Q8_K_BLOCK_BYTES = 256, 292
BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, IQ2_S: 82, IQ3_S: 110}

STATUS = {
    0: "Ok", 1: "UnsupportedType", 2: "ZeroLogicalElements", 3: "LogicalElementsNotDivisible",
    4: "ArithmeticOverflow", 6: "EncodedLengthMismatch", 7: "OutputLengthMismatch",
    8: "NonFiniteScale", 9: "NonFiniteActivation", 10: "NonFiniteQ8Scale",
    20: "DimensionMismatch", 21: "ScratchTooSmall", 22: "NonFiniteValue",
    23: "RoutedExpertOrder", 24: "DuplicateRoutedExpert", 25: "InvalidParameter",
    36: "SourceReadFailed",
    100: "HipError", 101: "NullArgument", 102: "UnsupportedShape", 103: "DeviceTimeout", 104: "ScratchInUse",
}
QUANT_ERRORS = {1, 2, 3, 4, 6, 7, 8, 9, 10}


class LbhError(C.Structure):
    _fields_ = [("status", C.c_int32), ("ty", C.c_int32), ("index", C.c_uint64), ("expected", C.c_uint64),
                ("actual", C.c_uint64), ("bits", C.c_uint32), ("field", C.c_uint32), ("row", C.c_uint64),
                ("hip_error", C.c_int32), ("reserved", C.c_int32)]


class BackendError(Exception):
    """Base of the mirrored error enums; ``variant`` is the reference variant name."""

    def __init__(self, err: LbhError):
        self.code = err.status
        self.variant = STATUS.get(err.status, str(err.status))
        self.ty, self.index, self.expected, self.actual = err.ty, err.index, err.expected, err.actual
        self.bits, self.field, self.row, self.hip_error = err.bits, err.field, err.row, err.hip_error
        super().__init__(f"{self.variant}(ty={self.ty}, index={self.index}, expected={self.expected}, "
                         f"actual={self.actual}, bits={self.bits:#x}, field={self.field}, row={self.row}, "
                         f"hip={self.hip_error})")


class QuantError(BackendError):
    """crates/bridge-quant-layout/src/error.rs:6-65."""


class KernelError(BackendError):
    """crates/bridge-kernels-reference/src/error.rs:7-59."""


def _raise(err: LbhError) -> None:
    raise (QuantError if err.status in QUANT_ERRORS else KernelError)(err)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"HIP backend library missing: {LIB_PATH} (build with __graft_entry__.build())")
        L = C.CDLL(str(LIB_PATH))
        p, sz, i32, u32 = C.c_void_p, C.c_size_t, C.c_int32, C.c_uint32
        E = C.POINTER(LbhError)
        sig = {
            "lbh_backend_name": ([], C.c_char_p),
            "lbh_device_count": ([], i32),
            "lbh_ctx_create": ([i32, p, C.POINTER(p), E], i32),
            "lbh_ctx_destroy": ([p], i32),
            "lbh_ctx_set_stream": ([p, p], i32),
            "lbh_ctx_synchronize": ([p, E], i32),
            "lbh_ctx_set_tuning": ([p, i32, i32], i32),
            "lbh_ctx_cu_count": ([p], i32),
            "lbh_quantize_row_q8_k_into": ([p, p, sz, p, sz, E], i32),
            "lbh_quantize_q8_k_rows": ([p, p, sz, sz, p], i32),
            "lbh_matrix_create": ([p, i32, sz, sz, p, sz, i32, C.POINTER(p), E], i32),
            "lbh_matrix_destroy": ([p], i32),
            "lbh_matrix_read_ggml": ([p, p, p, sz, E], i32),
            "lbh_matrix_rows": ([p], sz),
            "lbh_matrix_k": ([p], sz),
            "lbh_matrix_type": ([p], i32),
            "lbh_matrix_bytes": ([p], sz),
            "lbh_matrix_device_bytes": ([p], sz),
            "lbh_gemv_into": ([p, p, p, sz, p, sz, p, sz, E], i32),
            "lbh_gemv_accumulate_scaled_into": ([p, p, p, sz, p, sz, C.c_float, p, sz, E], i32),
            "lbh_gemv_q8_k": ([p, p, p, p, C.c_float, i32], i32),
            "lbh_gemv_f32": ([p, p, p, p, p, C.c_float, i32], i32),
            "lbh_gemv_block_sums": ([p, p, p, p], i32),
            "lbh_validate_vec_dot_q8_k": ([p, i32, p, sz, sz, p, sz, sz, E], i32),
            "lbh_vec_dot_q8_k_into": ([p, i32, p, sz, sz, p, sz, sz, p, sz, E], i32),
            "lbh_gemv_q8_k_into": ([p, p, p, sz, p, sz, C.c_float, i32, E], i32),
            "lbh_gemv_dequant_into": ([p, p, p, sz, p, sz, E], i32),
            "lbh_gemv_dequant_accumulate_scaled_into": ([p, p, p, sz, p, sz, C.c_float, E], i32),
            "lbh_gemv_dequant_f32": ([p, p, p, p, C.c_float, i32], i32),
            "lbh_debug_f16_to_f32": ([p, p, p, sz, E], i32),
            "lbh_debug_empty_kernel": ([p], i32),
            "lbh_debug_read_matrix": ([p, p, p, i32, i32, i32], i32),
            "lbh_moe_create": ([p, p, p, p, sz, p, p, p, C.POINTER(p), E], i32),
            "lbh_moe_destroy": ([p], i32),
            "lbh_moe_set_tiles": ([p, i32, i32, i32], i32),
            "lbh_moe_set_streams": ([p, i32], i32),
            "lbh_moe_routed_by_id_into": ([p, p, p, p, sz, p, sz, p, sz, E], i32),
            "lbh_moe_routed_by_id_dequant_f32_into": ([p, p, p, p, sz, p, sz, p, sz, E], i32),
            "lbh_moe_forward": ([p, p, p, p, sz, p, p], i32),
            "lbh_debug_expf": ([p, p, p, sz, i32, p, E], i32),
            "lbh_debug_expf_host": ([p, p, sz, i32, p], None),
            "lbh_router_create": ([p, p, sz, sz, p, i32, C.POINTER(p), E], i32),
            "lbh_router_destroy": ([p], i32),
            "lbh_router_take_status": ([p, p, C.POINTER(C.c_uint64), E], i32),
            "lbh_router_set_spin_limit": ([p, C.c_int64], i32),
            "lbh_router_route_into": ([p, p, p, sz, sz, i32, C.c_float, p, p, p, E], i32),
            "lbh_moe_block_forward": ([p, p, p, p, sz, i32, C.c_float, p], i32),
            "lbh_moe_block_forward_residual": ([p, p, p, p, sz, i32, C.c_float, p], i32),
            "lbh_moe_forward_batch_residual": ([p, p, p, p, sz, sz, p, p], i32),
            "lbh_moe_reserve_batch": ([p, sz, sz, E], i32),
            "lbh_matrix_prepare_gemm": ([p, p, E], i32),
            "lbh_gemm_workspace_bytes": ([sz, sz], sz),
            "lbh_gemm_q8_k": ([p, p, p, sz, p, p, sz], i32),
            "lbh_gemm_q8_k_noalloc": ([p, p, p, sz, p, E], i32),
            "lbh_moe_set_batch_tiles": ([p, i32, i32, i32, i32, i32], i32),
            "lbh_moe_set_batch_engine": ([p, i32, i32, i32], i32),
            "lbh_moe_make_batch_tile_copies": ([p, p, p, sz, E], i32),
            "lbh_moe_batch_tile_copy_bytes": ([p], sz),
            "lbh_moe_forward_batch": ([p, p, p, p, sz, sz, p, p], i32),
            "lbh_moe_routed_by_id_batch_into": ([p, p, p, p, sz, sz, p, sz, p, sz, E], i32),
            "lbh_route_experts_batch": ([p, p, sz, sz, sz, i32, C.c_float, p, p, p], i32),
            "lbh_expert_cache_create": ([p, p, u32, u32, i32, i32, C.POINTER(p), E], i32),
            "lbh_expert_cache_destroy": ([p], i32),
            "lbh_expert_cache_entry_bytes": ([p], C.c_uint64),
            "lbh_expert_cache_get_or_load": ([p, u32, u32, p, p, p, E], i32),
            "lbh_expert_cache_get": ([p, u32, u32, p, p], i32),
            "lbh_expert_cache_release": ([p, p], i32),
            "lbh_expert_cache_stats": ([p, p], i32),
            "lbh_expert_cache_clear_unpinned": ([p, p], i32),
            "lbh_expert_cache_read_record": ([p, p, p, sz, E], i32),
            "lbh_moe_create_cached": ([p, p, p, p, p, C.POINTER(p), E], i32),
            "lbh_moe_forward_leased": ([p, p, p, p, sz, p, p], i32),
            "lbh_matrix_create_streamed": ([p, i32, sz, sz, p, p, C.POINTER(p), E], i32),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes, fn.restype = args, res
        _lib = L
    return _lib


def _dev_ptr(t) -> int:
    import torch
    assert isinstance(t, torch.Tensor) and t.is_cuda and t.is_contiguous(), "expected a contiguous CUDA tensor"
    return t.data_ptr()


def _call(fn, *args) -> None:
    err = LbhError()
    st = fn(*args, C.byref(err))
    if st != 0:
        if err.status == 0:
            err.status = st
        _raise(err)


def backend_name() -> str:
    return lib().lbh_backend_name().decode()


class HipBackend:
    """Counterpart of CpuBackend (crates/bridge-kernels-cpu/src/lib.rs:59-119) for gfx950.

    ``execution_mode`` is the extra ReferenceExecutionMode this backend adds
    beside DequantF32 / LlamaQ8K / CpuParallelQ8K (gemv.rs:12-16)."""

    execution_mode = "HipQ8K"

    def __init__(self, device: int = 0, stream=None):
        import torch
        if not torch.cuda.is_available():
            raise RuntimeError("HipBackend needs a ROCm GPU")
        self.device = device
        torch.cuda.set_device(device)
        self._stream = stream if stream is not None else torch.cuda.current_stream(device)
        h = C.c_void_p()
        _call(lib().lbh_ctx_create, device, C.c_void_p(self._stream.cuda_stream), C.byref(h))
        self.ctx = h

    def backend_name(self) -> str:
        return backend_name()

    def set_stream(self, stream) -> None:
        """Order subsequent work on `stream` (a torch.cuda.Stream), e.g. for graph capture."""
        self._stream = stream
        lib().lbh_ctx_set_stream(self.ctx, C.c_void_p(stream.cuda_stream))

    TUNE_GEMV_LPU, TUNE_GEMV_MAX_BLOCKS, TUNE_GEMM_SHAPE, TUNE_GEMV_DEPTH = 1, 2, 3, 4

    def set_tuning(self, key: int, value: int) -> None:
        """Launch-shape knob (lanes per unit, workgroup cap); 0 restores the default."""
        st = lib().lbh_ctx_set_tuning(self.ctx, key, value)
        if st:
            raise KernelError(LbhError(status=st))

    def cu_count(self) -> int:
        return lib().lbh_ctx_cu_count(self.ctx)

    def simd_active(self) -> bool:
        return True

    def synchronize(self) -> None:
        _call(lib().lbh_ctx_synchronize, self.ctx)

    def close(self) -> None:
        if self.ctx:
            lib().lbh_ctx_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- matrices -----------------------------------------------------------------
    def upload(self, ty: int, rows: int, k: int, data) -> "DeviceMatrix":
        return DeviceMatrix(self, ty, rows, k, data)

    # -- Q8_K ---------------------------------------------------------------------
    def quantize_row_q8_k_into(self, x, encoded) -> None:
        _call(lib().lbh_quantize_row_q8_k_into, self.ctx, _dev_ptr(x), x.numel(), _dev_ptr(encoded), encoded.numel())

    def quantize_q8_k_rows(self, x, encoded, rows: int, n: int) -> None:
        st = lib().lbh_quantize_q8_k_rows(self.ctx, _dev_ptr(x), rows, n, _dev_ptr(encoded))
        if st:
            raise KernelError(LbhError(status=st))

    # -- matvec ---------------------------------------------------------------------
    def gemv_into(self, m: "DeviceMatrix", x, y, q8_scratch) -> None:
        _call(lib().lbh_gemv_into, self.ctx, m.handle, _dev_ptr(x), x.numel(), _dev_ptr(y), y.numel(),
              _dev_ptr(q8_scratch), q8_scratch.numel())

    def gemv_accumulate_scaled_into(self, m: "DeviceMatrix", x, dest, scale: float, q8_scratch) -> None:
        _call(lib().lbh_gemv_accumulate_scaled_into, self.ctx, m.handle, _dev_ptr(x), x.numel(), _dev_ptr(dest),
              dest.numel(), scale, _dev_ptr(q8_scratch), q8_scratch.numel())

    def gemv_q8_k(self, m: "DeviceMatrix", q8, y, coef: float = 0.0, accumulate: bool = False) -> None:
        st = lib().lbh_gemv_q8_k(self.ctx, m.handle, _dev_ptr(q8), _dev_ptr(y), coef, 1 if accumulate else 0)
        if st:
            raise KernelError(LbhError(status=st))

    def gemv_f32(self, m: "DeviceMatrix", x, y, q8_out=None, coef: float = 0.0, accumulate: bool = False) -> None:
        """Quantize x to Q8_K inside the matvec kernel and compute y (= or +=)."""
        q8p = _dev_ptr(q8_out) if q8_out is not None else None
        st = lib().lbh_gemv_f32(self.ctx, m.handle, _dev_ptr(x), q8p, _dev_ptr(y), coef, 1 if accumulate else 0)
        if st:
            raise KernelError(LbhError(status=st))

    def gemv_q8_k_into(self, m: "DeviceMatrix", q8, y, coef: float = 0.0, accumulate: bool = False) -> None:
        """Checked matvec over caller-supplied Q8_K bytes (validate_q8_scales,
        crates/bridge-quant-layout/src/q8_k.rs:208-222, before any write)."""
        _call(lib().lbh_gemv_q8_k_into, self.ctx, m.handle, _dev_ptr(q8), q8.numel(), _dev_ptr(y), y.numel(), coef,
              1 if accumulate else 0)

    # -- the reference's dot API over raw GGML rows (q8_k.rs:80-101, :172-186) --------------
    def validate_vec_dot_q8_k(self, ty: int, weights, q8, logical_elements: int, rows: int = 1) -> None:
        _call(lib().lbh_validate_vec_dot_q8_k, self.ctx, ty, _dev_ptr(weights), weights.numel(), rows, _dev_ptr(q8),
              q8.numel(), logical_elements)

    def vec_dot_q8_k_into(self, ty: int, weights, q8, logical_elements: int, out, rows: int = 1) -> None:
        """out[r] = vec_dot_q8_k(ty, row r of `weights`, q8, logical_elements)."""
        _call(lib().lbh_vec_dot_q8_k_into, self.ctx, ty, _dev_ptr(weights), weights.numel(), rows, _dev_ptr(q8),
              q8.numel(), logical_elements, _dev_ptr(out), out.numel())

    def vec_dot_q8_k(self, ty: int, weights, q8, logical_elements: int) -> float:
        import torch
        out = torch.zeros(1, dtype=torch.float32, device=weights.device)
        self.vec_dot_q8_k_into(ty, weights, q8, logical_elements, out)
        return float(out.item())

    def vec_dot_q4_k_q8_k(self, weights, q8, logical_elements: int) -> float:
        return self.vec_dot_q8_k(Q4_K, weights, q8, logical_elements)

    def vec_dot_q5_k_q8_k(self, weights, q8, logical_elements: int) -> float:
        return self.vec_dot_q8_k(Q5_K, weights, q8, logical_elements)

    def vec_dot_iq2_s_q8_k(self, weights, q8, logical_elements: int) -> float:
        return self.vec_dot_q8_k(IQ2_S, weights, q8, logical_elements)

    def vec_dot_iq3_s_q8_k(self, weights, q8, logical_elements: int) -> float:
        return self.vec_dot_q8_k(IQ3_S, weights, q8, logical_elements)

    # -- DequantF32 execution mode (gemv.rs:12-16, :305-328) ------------------------------
    def gemv_dequant_into(self, m: "DeviceMatrix", x, y) -> None:
        _call(lib().lbh_gemv_dequant_into, self.ctx, m.handle, _dev_ptr(x), x.numel(), _dev_ptr(y), y.numel())

    def gemv_dequant_accumulate_scaled_into(self, m: "DeviceMatrix", x, dest, scale: float) -> None:
        _call(lib().lbh_gemv_dequant_accumulate_scaled_into, self.ctx, m.handle, _dev_ptr(x), x.numel(),
              _dev_ptr(dest), dest.numel(), scale)

    def gemv_dequant_f32(self, m: "DeviceMatrix", x, y, coef: float = 0.0, accumulate: bool = False) -> None:
        st = lib().lbh_gemv_dequant_f32(self.ctx, m.handle, _dev_ptr(x), _dev_ptr(y), coef, 1 if accumulate else 0)
        if st:
            raise KernelError(LbhError(status=st))

    def gemm_q8_k(self, m: "DeviceMatrix", q8, n_tokens: int, y, workspace) -> None:
        """y[t, r] = vec_dot_q8_k(row r, token t) for a batch of Q8_K rows on the
        matrix cores (the matrix must be prepared with DeviceMatrix.prepare_gemm)."""
        st = lib().lbh_gemm_q8_k(self.ctx, m.handle, _dev_ptr(q8), n_tokens, _dev_ptr(y), _dev_ptr(workspace),
                                 workspace.numel() * workspace.element_size())
        if st:
            raise KernelError(LbhError(status=st))

    def gemm_q8_k_noalloc(self, m: "DeviceMatrix", q8, n_tokens: int, y) -> None:
        """gemm_q8_k staging its activation tiles in the library's static per-GPU
        scratch (no workspace, no allocation); an eager call on another stream
        while the last one is pending raises ScratchInUse."""
        _call(lib().lbh_gemm_q8_k_noalloc, self.ctx, m.handle, _dev_ptr(q8), n_tokens, _dev_ptr(y))

    NOALLOC_SCRATCH_BYTES = 8 << 20

    @staticmethod
    def gemm_workspace_bytes(n_tokens: int, k: int) -> int:
        return lib().lbh_gemm_workspace_bytes(n_tokens, k)

    def block_sums(self, m: "DeviceMatrix", q8, out) -> None:
        st = lib().lbh_gemv_block_sums(self.ctx, m.handle, _dev_ptr(q8), _dev_ptr(out))
        if st:
            raise KernelError(LbhError(status=st))

    def empty_kernel(self) -> None:
        """One empty kernel launch (the launch floor of a matvec)."""
        lib().lbh_debug_empty_kernel(self.ctx)

    READ_MAX_GRID = 65536

    def read_matrix(self, m: "DeviceMatrix", sink, grid: int, unroll: int = 4, slab: bool = False) -> None:
        """A plain read of the matrix's device bytes with 16-byte non-temporal loads (its matvec's memory
        floor) in one launch shape; sink: int32 device tensor of at least 4 * grid words."""
        st = lib().lbh_debug_read_matrix(self.ctx, m.handle, _dev_ptr(sink), grid, unroll, int(slab))
        if st:
            raise KernelError(LbhError(status=st))

    def f16_to_f32(self, src, dst) -> None:
        _call(lib().lbh_debug_f16_to_f32, self.ctx, _dev_ptr(src), _dev_ptr(dst), src.numel())

    def expf(self, x, out, up=None) -> None:
        """Device expf (or the SwiGLU element when `up` is given)."""
        _call(lib().lbh_debug_expf, self.ctx, _dev_ptr(x), _dev_ptr(out), x.numel(), 1 if up is not None else 0,
              _dev_ptr(up) if up is not None else None)

    # -- MoE ------------------------------------------------------------------------
    def moe_create(self, experts, shared=None) -> "MoeLayer":
        """experts: list of (gate, up, down) DeviceMatrix; shared: the same triple or None."""
        return MoeLayer(self, experts, shared)

    def moe_routed_by_id_into(self, moe: "MoeLayer", ids, coefs, x, y) -> None:
        """moe_routed_by_id_into (crates/bridge-kernels-reference/src/moe.rs:64-147)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        coefs = np.ascontiguousarray(coefs, dtype=np.float32)
        _call(lib().lbh_moe_routed_by_id_into, self.ctx, moe.handle, C.c_void_p(ids.ctypes.data),
              C.c_void_p(coefs.ctypes.data), ids.size, _dev_ptr(x), x.numel(), _dev_ptr(y), y.numel())

    def moe_routed_by_id_dequant_f32_into(self, moe: "MoeLayer", ids, coefs, x, y) -> None:
        """moe_routed_by_id_into in the DequantF32 execution mode (moe.rs:64-147;
        every matvec dot_dequant_row, gemv.rs:33-41)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        coefs = np.ascontiguousarray(coefs, dtype=np.float32)
        _call(lib().lbh_moe_routed_by_id_dequant_f32_into, self.ctx, moe.handle, C.c_void_p(ids.ctypes.data),
              C.c_void_p(coefs.ctypes.data), ids.size, _dev_ptr(x), x.numel(), _dev_ptr(y), y.numel())

    def moe_forward_batch(self, moe: "MoeLayer", ids, coefs, x, y) -> None:
        """Batched decode (asynchronous, unchecked): ids/coefs device tensors
        [n_tokens, top_k] (uint32 as int32 storage / float32), x and y [n_tokens, hidden]."""
        n, k = ids.shape
        st = lib().lbh_moe_forward_batch(self.ctx, moe.handle, _dev_ptr(ids), _dev_ptr(coefs), n, k, _dev_ptr(x),
                                         _dev_ptr(y))
        if st:
            raise KernelError(LbhError(status=st))

    def moe_forward_batch_residual(self, moe: "MoeLayer", ids, coefs, x, hidden) -> None:
        """moe_forward_batch adding each token's block output to hidden [n_tokens, hidden]
        in place (residual_add_in_place, crates/bridge-kernels-reference/src/norm.rs:83-98)."""
        n, k = ids.shape
        st = lib().lbh_moe_forward_batch_residual(self.ctx, moe.handle, _dev_ptr(ids), _dev_ptr(coefs), n, k,
                                                  _dev_ptr(x), _dev_ptr(hidden))
        if st:
            raise KernelError(LbhError(status=st))

    def moe_routed_by_id_batch_into(self, moe: "MoeLayer", ids, coefs, x, y) -> None:
        """Checked batched decode with host routing [n_tokens, top_k] (each token as
        moe_routed_by_id_into, crates/bridge-kernels-reference/src/moe.rs:64-147)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        coefs = np.ascontiguousarray(coefs, dtype=np.float32)
        n, k = ids.shape
        _call(lib().lbh_moe_routed_by_id_batch_into, self.ctx, moe.handle, C.c_void_p(ids.ctypes.data),
              C.c_void_p(coefs.ctypes.data), n, k, _dev_ptr(x), x.numel(), _dev_ptr(y), y.numel())

    def route_experts_batch(self, logits, top_k: int, ids, coefs, mode: int = 0, weight_scale: float = 1.0,
                            bias=None) -> None:
        """Top-k selection of every token from device logits [n_tokens, n_experts]
        (route_experts_into, crates/bridge-model-hy3/src/routing.rs:25-107, for mode 1)."""
        n, ne = logits.shape
        st = lib().lbh_route_experts_batch(self.ctx, _dev_ptr(logits), n, ne, top_k, mode, weight_scale,
                                           _dev_ptr(bias) if bias is not None else None, _dev_ptr(ids),
                                           _dev_ptr(coefs))
        if st:
            raise KernelError(LbhError(status=st))

    def moe_forward(self, moe: "MoeLayer", ids, coefs, x, y) -> None:
        """Unchecked, asynchronous form (graph capturable)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        coefs = np.ascontiguousarray(coefs, dtype=np.float32)
        st = lib().lbh_moe_forward(self.ctx, moe.handle, C.c_void_p(ids.ctypes.data), C.c_void_p(coefs.ctypes.data),
                                   ids.size, _dev_ptr(x), _dev_ptr(y))
        if st:
            raise KernelError(LbhError(status=st))


class Router:
    """The F32 MoE router resident in HBM: weights [n_experts][hidden] (GGML F32
    [hidden, n_experts]) and an optional selection bias (routing.rs:25-107)."""

    SOFTMAX, SIGMOID_BIAS = 0, 1

    def __init__(self, be: HipBackend, weights: np.ndarray, bias: np.ndarray | None = None):
        w = np.ascontiguousarray(weights, dtype=np.float32)
        b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
        self.be, self.n_experts, self.hidden = be, w.shape[0], w.shape[1]
        h = C.c_void_p()
        _call(lib().lbh_router_create, be.ctx, C.c_void_p(w.ctypes.data), self.n_experts, self.hidden,
              C.c_void_p(b.ctypes.data) if b is not None else None, 0, C.byref(h))
        self.handle = h

    def route_into(self, x, top_k: int, mode: int = 0, weight_scale: float = 1.0, want_logits: bool = False):
        """Host (ids, coefs[, logits]) of one token; ids ascending."""
        ids = np.zeros(top_k, np.uint32)
        coefs = np.zeros(top_k, np.float32)
        logits = np.zeros(self.n_experts, np.float32) if want_logits else None
        _call(lib().lbh_router_route_into, self.be.ctx, self.handle, _dev_ptr(x), x.numel(), top_k, mode,
              weight_scale, C.c_void_p(ids.ctypes.data), C.c_void_p(coefs.ctypes.data),
              C.c_void_p(logits.ctypes.data) if logits is not None else None)
        return (ids, coefs, logits) if want_logits else (ids, coefs)

    def set_spin_limit(self, limit: int) -> None:
        """Polls of the router chains' bounded waits (0 default, < 0 give up at once: a test knob)."""
        lib().lbh_router_set_spin_limit(self.handle, limit)

    def take_status(self) -> int:
        """Rejected block-decode steps since the last call (then cleared); raises the first
        rejection's error (DeviceTimeout or NonFiniteValue) like route_experts_into."""
        n = C.c_uint64(0)
        _call(lib().lbh_router_take_status, self.be.ctx, self.handle, C.byref(n))
        return int(n.value)

    def close(self) -> None:
        if self.handle:
            lib().lbh_router_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def moe_block_forward(be: HipBackend, moe: "MoeLayer", router: Router, x, y, top_k: int, mode: int = 0,
                      weight_scale: float = 1.0) -> None:
    """Device router + top-k + MoE experts of one token (asynchronous, unchecked)."""
    st = lib().lbh_moe_block_forward(be.ctx, moe.handle, router.handle, _dev_ptr(x), top_k, mode, weight_scale,
                                     _dev_ptr(y))
    if st:
        raise KernelError(LbhError(status=st))


def moe_block_forward_residual(be: HipBackend, moe: "MoeLayer", router: Router, x, hidden, top_k: int, mode: int = 0,
                               weight_scale: float = 1.0) -> None:
    """moe_block_forward ending with hidden += ffn_delta in place (layer.rs:464)."""
    st = lib().lbh_moe_block_forward_residual(be.ctx, moe.handle, router.handle, _dev_ptr(x), top_k, mode,
                                              weight_scale, _dev_ptr(hidden))
    if st:
        raise KernelError(LbhError(status=st))


def expf_host(x: np.ndarray, up: np.ndarray | None = None) -> np.ndarray:
    """The device expf / SwiGLU arithmetic compiled for the host CPU."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    u = np.ascontiguousarray(up, dtype=np.float32) if up is not None else None
    lib().lbh_debug_expf_host(C.c_void_p(x.ctypes.data), C.c_void_p(out.ctypes.data), x.size,
                              1 if u is not None else 0, C.c_void_p(u.ctypes.data) if u is not None else None)
    return out


class MoeLayer:
    """A resident routed + shared SwiGLU MoE layer (moe.rs:17-21 RoutedMoeSelection)."""

    def __init__(self, be: HipBackend, experts, shared=None):
        n = len(experts)
        arr = [(C.c_void_p * n)(*[e[i].handle for e in experts]) for i in range(3)]
        sh = [shared[i].handle if shared is not None else None for i in range(3)]
        h = C.c_void_p()
        _call(lib().lbh_moe_create, be.ctx, arr[0], arr[1], arr[2], n, sh[0], sh[1], sh[2], C.byref(h))
        self.be, self.handle = be, h
        self._keep = (experts, shared)
        self.n_experts = n

    def reserve_batch(self, max_tokens: int, top_k: int) -> None:
        """Scratch of batched calls (allocated once)."""
        _call(lib().lbh_moe_reserve_batch, self.handle, max_tokens, top_k)

    def set_batch_tiles(self, tokens_per_chunk: int = 8, rows_gate_up_routed: int = 128,
                        rows_gate_up_shared: int = 128, rows_down_routed: int = 320, rows_down_shared: int = 128) -> None:
        st = lib().lbh_moe_set_batch_tiles(self.handle, tokens_per_chunk, rows_gate_up_routed, rows_gate_up_shared,
                                           rows_down_routed, rows_down_shared)
        if st:
            raise KernelError(LbhError(status=st))

    def set_batch_engine(self, mx_min_tokens: int = 4, mx_rows_gate_up: int = 0, mx_rows_down: int = 0) -> None:
        """Batched IQ chunks of at least mx_min_tokens tokens on the matrix cores, the
        rest on the VALU dot4 path (0: all on the VALU); resets the batch launch shapes
        to their defaults."""
        st = lib().lbh_moe_set_batch_engine(self.handle, mx_min_tokens, mx_rows_gate_up, mx_rows_down)
        if st:
            raise KernelError(LbhError(status=st))

    def make_batch_tile_copies(self, experts=None) -> None:
        """16-row tile copies of the routed IQ matrices of `experts` (None: all; an
        empty list drops them) for the batched matrix-core streams."""
        if experts is None:
            _call(lib().lbh_moe_make_batch_tile_copies, self.be.ctx, self.handle, None, 0)
            return
        ids = np.ascontiguousarray(experts, dtype=np.uint32)
        buf = ids if ids.size else np.zeros(1, np.uint32)   # a list, possibly empty: never NULL
        _call(lib().lbh_moe_make_batch_tile_copies, self.be.ctx, self.handle, C.c_void_p(buf.ctypes.data), ids.size)

    @property
    def batch_tile_copy_bytes(self) -> int:
        """HBM bytes of the tile copies (0 when none)."""
        return int(lib().lbh_moe_batch_tile_copy_bytes(self.handle))

    def set_streams(self, two_streams: bool) -> None:
        """Shared expert on a second stream beside the routed experts, or (default) all on one."""
        st = lib().lbh_moe_set_streams(self.handle, 1 if two_streams else 0)
        if st:
            raise KernelError(LbhError(status=st))

    def set_tiles(self, wg_routed: int, wg_shared: int, tile_d: int = 16) -> None:
        """Workgroups of the routed / shared gate-up streams, output rows per down workgroup."""
        st = lib().lbh_moe_set_tiles(self.handle, wg_routed, wg_shared, tile_d)
        if st:
            raise KernelError(LbhError(status=st))

    def close(self) -> None:
        if self.handle:
            lib().lbh_moe_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceMatrix:
    """A PackedMatrix (crates/bridge-kernels-reference/src/matrix.rs:102-186) resident in HBM."""

    def __init__(self, be: HipBackend, ty: int, rows: int, k: int, data):
        import torch
        self.be, self.ty, self.rows, self.k = be, ty, rows, k
        h = C.c_void_p()
        if isinstance(data, torch.Tensor):
            assert data.is_cuda and data.dtype == torch.uint8
            data = data.contiguous()
            _call(lib().lbh_matrix_create, be.ctx, ty, rows, k, C.c_void_p(data.data_ptr()), data.numel(), 1,
                  C.byref(h))
        else:
            arr = np.ascontiguousarray(data).reshape(-1).view(np.uint8)   # the GGML bytes (F32: the floats' bytes)
            _call(lib().lbh_matrix_create, be.ctx, ty, rows, k, C.c_void_p(arr.ctypes.data), arr.size, 0,
                  C.byref(h))
        self.handle = h
        self.nbytes = lib().lbh_matrix_bytes(h)

    @classmethod
    def streamed(cls, be: HipBackend, ty: int, rows: int, k: int, reader) -> "DeviceMatrix":
        """A matrix whose GGML bytes come from `reader` (a ctypes lbh_byte_reader
        callback), streamed through pinned chunks straight to HBM."""
        self = cls.__new__(cls)
        self.be, self.ty, self.rows, self.k = be, ty, rows, k
        h = C.c_void_p()
        self.handle = None
        _call(lib().lbh_matrix_create_streamed, be.ctx, ty, rows, k, C.cast(reader, C.c_void_p), None, C.byref(h))
        self.handle = h
        self.nbytes = lib().lbh_matrix_bytes(h)
        return self

    def prepare_gemm(self) -> None:
        """Build the MFMA-ready copy used by gemm_q8_k (Q4_K / Q5_K)."""
        _call(lib().lbh_matrix_prepare_gemm, self.be.ctx, self.handle)

    @property
    def device_bytes(self) -> int:
        """HBM bytes held: the packed planes plus the MFMA-ready copy once prepared."""
        return lib().lbh_matrix_device_bytes(self.handle)

    def read_ggml(self) -> np.ndarray:
        out = np.zeros(self.nbytes, np.uint8)
        _call(lib().lbh_matrix_read_ggml, self.be.ctx, self.handle, C.c_void_p(out.ctypes.data), out.size)
        return out

    def close(self) -> None:
        if self.handle:
            lib().lbh_matrix_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
