"""Python mirror of the HBM expert cache (lbh_expert_cache_* in liblightbridge_hip.so).

Names follow the reference's CompressedCache (crates/bridge-cache/src/lib.rs):
``get_or_try_insert(key, loader)`` returns a lease that pins the entry until
``release()`` (CacheLease's drop, lib.rs:419-443); ``get``, ``stats`` and
``clear_unpinned`` as lib.rs:101-322.  Keys are ``ExpertKey(layer, expert)``.
A loader is a callable returning the expert's tight record (gate | up | down
GGML bytes), or, for zero-copy loads, a callable ``fill(dst) -> length`` marked
with ``into=True`` that writes the record into the cache's pinned staging
memory (``Sidecar.read_into``).  Errors raise the mirrored QuantError /
KernelError, or ``CacheError`` (lib.rs:496-516) / ``LoaderError``
(LoadError::Loader, carrying the loader's own exception).
"""
from __future__ import annotations

import ctypes as C
import itertools
import threading

import numpy as np

from . import LbhError, _dev_ptr, _raise, lib
from .sidecar import ExpertKey

CACHE_ERRORS = {30: "ZeroCapacity", 31: "ZeroAdmissionThreshold", 32: "EntryTooLarge", 33: "CapacityPinned",
                34: "LoadedSizeMismatch", 35: "Loader"}
_LEASE_LIVE = 0x4C454153


class CacheConfig(C.Structure):
    _fields_ = [("capacity_bytes", C.c_uint64), ("admit_after_requests", C.c_uint64)]


class CacheStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "capacity_bytes", "used_bytes", "reserved_bytes", "resident_entries", "pinned_entries", "loading_entries",
        "heat_entries", "hits", "misses", "loads", "waits", "evictions", "entry_bytes", "slots", "bytes_uploaded")]

    def as_dict(self) -> dict:
        return {n: getattr(self, n) for n, _ in self._fields_}


class Lease(C.Structure):
    _fields_ = [("layer", C.c_uint32), ("expert", C.c_uint32), ("slot", C.c_int32), ("reserved", C.c_int32)]


LOADER = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint8), C.c_size_t,
                     C.POINTER(C.c_size_t))


class CacheError(Exception):
    """CacheError (lib.rs:496-516): ``variant`` and the error payload."""

    def __init__(self, err: LbhError):
        self.variant = CACHE_ERRORS.get(err.status, str(err.status))
        self.expected, self.actual = err.expected, err.actual
        super().__init__(f"{self.variant}(expected={err.expected}, actual={err.actual})")


class LoaderError(Exception):
    """LoadError::Loader (lib.rs:518-524): the loader failed; ``__cause__`` is its exception."""


_registry: dict = {}
_ids = itertools.count(1)
_reg_lock = threading.Lock()


@LOADER
def _trampoline(user, layer, expert, dst, cap, written):
    entry = _registry.get(int(user or 0))
    if entry is None:
        return -1
    fn, into, box = entry
    try:
        if into:
            n = int(fn(memoryview((C.c_uint8 * cap).from_address(C.cast(dst, C.c_void_p).value)).cast("B")))
        else:
            data = fn()
            buf = np.ascontiguousarray(np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray)
                                       else data.reshape(-1).view(np.uint8))
            n = buf.size
            if n <= cap:
                C.memmove(dst, buf.ctypes.data, n)
        written[0] = n
        return 0
    except Exception as e:   # surfaces as LoaderError after the call returns
        box.append(e)
        return 1


def _addr(obj) -> C.c_void_p:
    return C.c_void_p(C.addressof(obj))


_TRAMPOLINE_PTR = C.cast(_trampoline, C.c_void_p)


def _check(st: int, err: LbhError, box=None) -> None:
    if st == 0:
        return
    if err.status == 0:
        err.status = st
    if err.status == 35:
        raise LoaderError(f"loader failed for expert {err.index} (code {err.actual})") from (box[0] if box else None)
    if err.status in CACHE_ERRORS:
        raise CacheError(err)
    _raise(err)


class CacheLease:
    """A pinned cache entry (CacheLease, lib.rs:396-443)."""

    def __init__(self, cache: "ExpertCache", lease: Lease):
        self.cache, self.lease = cache, lease
        self.key = ExpertKey(lease.layer, lease.expert)

    @property
    def live(self) -> bool:
        return self.lease.reserved == _LEASE_LIVE

    def release(self) -> None:
        if self.live:
            st = lib().lbh_expert_cache_release(self.cache.handle, _addr(self.lease))
            if st:
                raise CacheError(LbhError(status=st))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.release()


class ExpertCache:
    """CompressedCache<ExpertKey> resident in HBM for one routed-expert shape."""

    def __init__(self, be, capacity_bytes: int, admit_after_requests: int, hidden: int, ffn: int,
                 gate_up_type: int, down_type: int):
        cfg = CacheConfig(capacity_bytes, admit_after_requests)
        h = C.c_void_p()
        err = LbhError()
        _check(lib().lbh_expert_cache_create(be.ctx, _addr(cfg), hidden, ffn, gate_up_type, down_type, C.byref(h),
                                             C.byref(err)), err)
        self.be, self.handle = be, h
        self.hidden, self.ffn, self.gate_up_type, self.down_type = hidden, ffn, gate_up_type, down_type
        self.entry_bytes = int(lib().lbh_expert_cache_entry_bytes(h))

    def get_or_try_insert(self, key: ExpertKey, loader, into: bool = False) -> CacheLease:
        box: list = []
        with _reg_lock:
            uid = next(_ids)
            _registry[uid] = (loader, into, box)
        lease, err = Lease(), LbhError()
        try:
            st = lib().lbh_expert_cache_get_or_load(self.handle, key.layer, key.expert, _TRAMPOLINE_PTR,
                                                    C.c_void_p(uid), _addr(lease), C.byref(err))
        finally:
            with _reg_lock:
                del _registry[uid]
        _check(st, err, box)
        return CacheLease(self, lease)

    def get(self, key: ExpertKey) -> CacheLease | None:
        lease, found = Lease(), C.c_int32(0)
        st = lib().lbh_expert_cache_get(self.handle, key.layer, key.expert, _addr(lease), _addr(found))
        if st:
            raise CacheError(LbhError(status=st))
        return CacheLease(self, lease) if found.value else None

    def stats(self) -> dict:
        s = CacheStats()
        lib().lbh_expert_cache_stats(self.handle, _addr(s))
        return s.as_dict()

    def clear_unpinned(self) -> int:
        n = C.c_uint64(0)
        lib().lbh_expert_cache_clear_unpinned(self.handle, _addr(n))
        return n.value

    def read_record(self, lease: CacheLease) -> np.ndarray:
        """The entry's tight record read back from HBM (device layout inverted)."""
        out = np.zeros(self.entry_bytes, np.uint8)
        err = LbhError()
        _check(lib().lbh_expert_cache_read_record(self.handle, _addr(lease.lease), C.c_void_p(out.ctypes.data),
                                                  out.size, C.byref(err)), err)
        return out

    def close(self) -> None:
        if self.handle:
            lib().lbh_expert_cache_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class CachedMoeLayer:
    """A MoE layer whose routed experts stream through an ExpertCache
    (the runtime's streaming MoE, crates/bridge-runtime/src/hy3_scalar.rs:561-626)."""

    def __init__(self, be, cache: ExpertCache, shared=None):
        sh = [shared[i].handle if shared is not None else None for i in range(3)]
        h = C.c_void_p()
        err = LbhError()
        _check(lib().lbh_moe_create_cached(be.ctx, cache.handle, sh[0], sh[1], sh[2], C.byref(h), C.byref(err)), err)
        self.be, self.cache, self.handle = be, cache, h
        self._keep = shared

    def forward_leased(self, leases, coefs, x, y) -> None:
        """Routed experts = the leases (ascending expert ids) with coefficients `coefs`."""
        arr = (Lease * len(leases))(*[l.lease for l in leases])
        cf = np.ascontiguousarray(coefs, dtype=np.float32)
        st = lib().lbh_moe_forward_leased(self.be.ctx, self.handle, _addr(arr), C.c_void_p(cf.ctypes.data), len(leases),
                                          _dev_ptr(x), _dev_ptr(y))
        if st:
            _raise(LbhError(status=st))

    def close(self) -> None:
        if self.handle:
            lib().lbh_moe_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
