"""GPU tests of the HBM expert cache (lbh_expert_cache_*, mirror lbhip.cache).

The cache semantics are the reference's CompressedCache tests
(crates/bridge-cache/tests/cache.rs) restated against the device cache: LRU
eviction under the byte ceiling, pins blocking a reservation before the loader
runs, concurrent misses deduplicated, hysteretic admission, a bad loader
releasing its reservation.  Beyond them: the record read back from HBM equals
the loader's bytes for every type, non-finite scales are rejected with the
reference's payload, and the streaming MoE forward over leased experts
(crates/bridge-runtime/src/hy3_scalar.rs:561-626) equals the CPU oracle's
moe_routed_by_id bit for bit, also while slots are evicted and refilled behind
queued kernels.  The records come from sidecar files (lbhip.sidecar) written
from seeded synthetic experts.
"""
import threading
import time

import numpy as np
import pytest

from lbhip import sidecar as sc
from lbhip import synth
from moe_helpers import dev, host

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
Q4_K, Q5_K, IQ3_S, IQ2_S = 12, 13, 21, 22
NAMES = {Q4_K: "Q4_K", Q5_K: "Q5_K", IQ3_S: "IQ3_S", IQ2_S: "IQ2_S"}
HID, FFN = 512, 256


@pytest.fixture(scope="module")
def be():
    import lbhip
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    b = lbhip.HipBackend(0)
    yield b
    b.close()


def expert_np(e, tg=IQ2_S, td=IQ3_S, hidden=HID, ffn=FFN, seed=0):
    return (synth.random_matrix(tg, ffn, hidden, seed + 3 * e), synth.random_matrix(tg, ffn, hidden, seed + 3 * e + 1),
            synth.random_matrix(td, hidden, ffn, seed + 3 * e + 2))


def record(e, **kw):
    g, u, d = expert_np(e, **kw)
    return np.concatenate([g.reshape(-1), u.reshape(-1), d.reshape(-1)])


def entry_bytes(tg=IQ2_S, td=IQ3_S, hidden=HID, ffn=FFN):
    """Tight record length: gate and up [ffn x hidden], down [hidden x ffn]."""
    return 2 * ffn * (hidden // 256) * synth.BLOCK_BYTES[tg] + hidden * (ffn // 256) * synth.BLOCK_BYTES[td]


def make_cache(be, entries, admit=1, tg=IQ2_S, td=IQ3_S, hidden=HID, ffn=FFN):
    from lbhip.cache import ExpertCache
    c = ExpertCache(be, entries * entry_bytes(tg, td, hidden, ffn), admit, hidden, ffn, tg, td)
    assert c.entry_bytes == entry_bytes(tg, td, hidden, ffn) and c.stats()["slots"] == entries
    return c


K = sc.ExpertKey


def test_lru_eviction_stays_within_the_fixed_ceiling(be):
    c = make_cache(be, 2)
    c.get_or_try_insert(K(0, 1), lambda: record(1)).release()
    c.get_or_try_insert(K(0, 2), lambda: record(2)).release()
    c.get(K(0, 1)).release()
    c.get_or_try_insert(K(0, 3), lambda: record(3)).release()
    st = c.stats()
    assert st["used_bytes"] == 2 * c.entry_bytes and st["resident_entries"] == 2 and st["evictions"] == 1
    assert c.get(K(0, 1)) is not None and c.get(K(0, 2)) is None and c.get(K(0, 3)) is not None
    c.close()


def test_pinned_entries_block_reservation_before_loader_runs(be):
    from lbhip.cache import CacheError
    c = make_cache(be, 1)
    lease = c.get_or_try_insert(K(0, 1), lambda: record(1))
    calls = []
    with pytest.raises(CacheError) as e:
        c.get_or_try_insert(K(0, 2), lambda: calls.append(1) or record(2))
    assert e.value.variant == "CapacityPinned" and e.value.expected == c.entry_bytes
    assert not calls
    assert np.array_equal(c.read_record(lease), record(1))
    lease.release()
    c.close()


def test_concurrent_misses_are_deduplicated(be):
    c = make_cache(be, 4)
    loads, gate = [], threading.Barrier(2)
    leases = [None, None]

    def loader():
        loads.append(1)
        time.sleep(0.2)   # the second caller arrives while this load is in flight
        return record(7)

    def run(i):
        gate.wait()
        leases[i] = c.get_or_try_insert(K(1, 7), loader)

    ts = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert len(loads) == 1
    assert np.array_equal(c.read_record(leases[0]), record(7)) and np.array_equal(c.read_record(leases[1]), record(7))
    assert c.stats()["waits"] >= 1
    for lease in leases:
        lease.release()
    c.close()


def test_hysteretic_admission_requires_reuse(be):
    c = make_cache(be, 4, admit=2)
    n = []
    load = lambda: n.append(1) or record(1)  # noqa: E731
    c.get_or_try_insert(K(0, 1), load).release()
    assert c.stats()["resident_entries"] == 0 and c.get(K(0, 1)) is None   # ephemeral: gone with its last pin
    c.get_or_try_insert(K(0, 1), load).release()
    assert c.stats()["resident_entries"] == 1
    hit = c.get(K(0, 1))
    assert hit is not None and np.array_equal(c.read_record(hit), record(1))
    hit.release()
    assert len(n) == 2
    c.close()


def test_bad_loader_size_releases_the_reservation(be):
    from lbhip.cache import CacheError, LoaderError
    c = make_cache(be, 2)
    with pytest.raises(CacheError) as e:
        c.get_or_try_insert(K(0, 1), lambda: record(1)[:-1])
    assert e.value.variant == "LoadedSizeMismatch" and e.value.expected == c.entry_bytes
    assert e.value.actual == c.entry_bytes - 1
    assert c.stats()["reserved_bytes"] == 0 and c.stats()["used_bytes"] == 0

    def broken():
        raise IOError("disk gone")
    with pytest.raises(LoaderError) as le:
        c.get_or_try_insert(K(0, 1), broken)
    assert isinstance(le.value.__cause__, IOError)
    lease = c.get_or_try_insert(K(0, 1), lambda: record(1))
    assert np.array_equal(c.read_record(lease), record(1))
    lease.release()
    c.close()


@pytest.mark.parametrize("segment", [0, 1, 2])
def test_non_finite_scale_is_rejected_with_the_reference_payload(be, segment):
    import lbhip
    c = make_cache(be, 2, tg=Q4_K, td=Q5_K)
    rec = record(2, tg=Q4_K, td=Q5_K)
    g, u, d = expert_np(2, tg=Q4_K, td=Q5_K)
    seg_off = [0, g.size, g.size + u.size][segment]
    nb, bb = (HID // 256, 144) if segment < 2 else (FFN // 256, 176)
    row, blk, field = 5, nb - 1, 1
    pos = seg_off + (row * nb + blk) * bb + 2 * field
    rec[pos:pos + 2] = np.array([0x7c01], np.uint16).view(np.uint8)   # NaN dmin
    with pytest.raises(lbhip.QuantError) as e:
        c.get_or_try_insert(K(0, 2), lambda: rec)
    err = e.value
    assert err.variant == "NonFiniteScale" and err.expected == segment and err.row == row
    assert err.index == blk and err.field == field and err.bits == 0x7c01
    assert c.stats()["reserved_bytes"] == 0 and c.get(K(0, 2)) is None
    c.close()


@pytest.mark.parametrize("tg,td", [(IQ2_S, IQ3_S), (Q4_K, Q5_K), (IQ3_S, IQ2_S), (Q5_K, Q4_K)])
def test_record_read_back_from_hbm_is_the_loaders(be, tg, td):
    c = make_cache(be, 3, tg=tg, td=td)
    leases = [c.get_or_try_insert(K(2, e), lambda e=e: record(e, tg=tg, td=td)) for e in range(3)]
    for e, lease in enumerate(leases):
        assert np.array_equal(c.read_record(lease), record(e, tg=tg, td=td))
        lease.release()
    c.close()


# ---------------------------------------------------------------- streaming MoE

class Streamed:
    """A sidecar of n experts (IQ2_S gate/up, IQ3_S down), the oracle's view of
    them and a Q4_K/Q5_K shared expert resident on the device."""

    def __init__(self, be, oracle, tmp, n, hidden=HID, ffn=FFN, ffn_s=512, seed=40):
        self.hidden = hidden
        self.np = [expert_np(e, hidden=hidden, ffn=ffn, seed=seed) for e in range(n)]
        self.path, self.mpath = tmp / "experts.sidecar", tmp / "experts.json"
        sc.write_sidecar(self.path, self.mpath,
                         [(K(4, e), tuple(m.tobytes() for m in self.np[e]), ("IQ2_S", "IQ2_S", "IQ3_S"))
                          for e in range(n)], sc.FUSED_GATE_UP, 4096)
        self.sidecar = sc.Sidecar(self.path, self.mpath)
        self.orc = [oracle.make_expert(oracle.make_matrix(IQ2_S, ffn, hidden, g), oracle.make_matrix(IQ2_S, ffn, hidden, u),
                                       oracle.make_matrix(IQ3_S, hidden, ffn, d)) for g, u, d in self.np]
        sh = (synth.random_matrix(Q4_K, ffn_s, hidden, seed + 901), synth.random_matrix(Q4_K, ffn_s, hidden, seed + 902),
              synth.random_matrix(Q5_K, hidden, ffn_s, seed + 903))
        self.shared_np = sh
        self.shared = (be.upload(Q4_K, ffn_s, hidden, sh[0]), be.upload(Q4_K, ffn_s, hidden, sh[1]),
                       be.upload(Q5_K, hidden, ffn_s, sh[2]))
        self.orc_shared = oracle.make_expert(oracle.make_matrix(Q4_K, ffn_s, hidden, sh[0]),
                                             oracle.make_matrix(Q4_K, ffn_s, hidden, sh[1]),
                                             oracle.make_matrix(Q5_K, hidden, ffn_s, sh[2]))

    def lease(self, cache, e):
        return cache.get_or_try_insert(K(4, e), lambda dst: self.sidecar.read_into(K(4, e), dst), into=True)

    def want(self, oracle, ids, coefs, x):
        ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
        return oracle.moe_routed_by_id(ex, ids, coefs, self.orc, self.orc_shared, x, preflight=False)


def test_forward_leased_matches_oracle_with_evictions_behind_queued_work(be, oracle, tmp_path):
    """12 experts through a 5-entry cache, 10 tokens of top-4: every token's
    leases are released right after its (asynchronous) forward is queued, so
    later misses evict and refill slots that queued kernels still read; every
    token must still equal the oracle."""
    from lbhip.cache import CachedMoeLayer
    s = Streamed(be, oracle, tmp_path, 12)
    cache = make_cache(be, 5)
    layer = CachedMoeLayer(be, cache, s.shared)
    rng = np.random.default_rng(8)
    xs = rng.standard_normal((10, HID)).astype(np.float32)
    ys = torch.full((10, HID), float("nan"), device="cuda")
    routes = []
    for t in range(10):
        ids = np.sort(rng.choice(12, 4, replace=False)).astype(np.uint32)
        coefs = rng.random(4).astype(np.float32)
        routes.append((ids, coefs))
        leases = [s.lease(cache, int(e)) for e in ids]
        layer.forward_leased(leases, coefs, dev(xs[t]), ys[t])
        for lease in leases:
            lease.release()
    got = host(ys)
    for t, (ids, coefs) in enumerate(routes):
        want = s.want(oracle, ids, coefs, xs[t])
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), f"token {t}"
    st = cache.stats()
    assert st["evictions"] > 0 and st["hits"] > 0 and st["pinned_entries"] == 0
    layer.close()
    cache.close()


def test_forward_leased_equals_the_resident_layer(be, oracle, tmp_path):
    """The same experts resident (lbh_moe_forward) and streamed (leases): same bits."""
    from lbhip.cache import CachedMoeLayer
    s = Streamed(be, oracle, tmp_path, 6)
    dev_exp = [tuple(be.upload(t, r, k, m) for t, r, k, m in ((IQ2_S, FFN, HID, g), (IQ2_S, FFN, HID, u),
                                                             (IQ3_S, HID, FFN, d))) for g, u, d in s.np]
    resident = be.moe_create(dev_exp, s.shared)
    cache = make_cache(be, 6)
    layer = CachedMoeLayer(be, cache, s.shared)
    x = dev(np.random.default_rng(3).standard_normal(HID).astype(np.float32))
    ids, coefs = np.array([0, 2, 3, 5], np.uint32), np.array([0.1, 0.4, 0.2, 0.3], np.float32)
    y1 = torch.zeros(HID, device="cuda")
    y2 = torch.zeros(HID, device="cuda")
    be.moe_forward(resident, ids, coefs, x, y1)
    leases = [s.lease(cache, int(e)) for e in ids]
    layer.forward_leased(leases, coefs, x, y2)
    assert np.array_equal(host(y1).view(np.uint32), host(y2).view(np.uint32))
    for lease in leases:
        lease.release()
    layer.close()
    resident.close()
    cache.close()


def test_forward_leased_rejects_bad_leases(be, oracle, tmp_path):
    import lbhip
    from lbhip.cache import CachedMoeLayer
    s = Streamed(be, oracle, tmp_path, 3)
    cache = make_cache(be, 3)
    layer = CachedMoeLayer(be, cache, s.shared)
    x, y = dev(np.ones(HID, np.float32)), torch.zeros(HID, device="cuda")
    a, b = s.lease(cache, 0), s.lease(cache, 1)
    with pytest.raises(lbhip.KernelError, match="RoutedExpertOrder"):
        layer.forward_leased([b, a], [0.5, 0.5], x, y)
    with pytest.raises(lbhip.KernelError, match="DuplicateRoutedExpert"):
        layer.forward_leased([a, a], [0.5, 0.5], x, y)
    b.release()
    with pytest.raises(lbhip.KernelError, match="InvalidParameter"):
        layer.forward_leased([a, b], [0.5, 0.5], x, y)
    a.release()
    # a cache-fed layer has no resident expert table
    with pytest.raises(lbhip.KernelError):
        be.moe_forward(layer, np.array([0], np.uint32), np.array([1.0], np.float32), x, y)
    layer.close()
    cache.close()


def test_forward_leased_on_another_stream_keeps_slots_until_read(be, oracle, tmp_path):
    """The layer runs on a second stream (its own context) while the cache was
    created on the first: each slot's last use is recorded on the stream that
    reads it, so a refill on the copy stream waits for the second stream's
    queued forward, not for the cache context's idle stream.  A bounded spin
    before each forward keeps the readers queued while later misses evict."""
    import lbhip
    from lbhip.cache import CachedMoeLayer
    s = Streamed(be, oracle, tmp_path, 12)
    cache = make_cache(be, 5)
    side = torch.cuda.Stream()
    be2 = lbhip.HipBackend(0, stream=side)
    layer = CachedMoeLayer(be2, cache, s.shared)
    rng = np.random.default_rng(21)
    xs = rng.standard_normal((10, HID)).astype(np.float32)
    xd = dev(xs)
    ys = torch.full((10, HID), float("nan"), device="cuda")
    torch.cuda.synchronize()
    routes = []
    for t in range(10):
        ids = np.sort(rng.choice(12, 4, replace=False)).astype(np.uint32)
        coefs = rng.random(4).astype(np.float32)
        routes.append((ids, coefs))
        leases = [s.lease(cache, int(e)) for e in ids]
        with torch.cuda.stream(side):
            if hasattr(torch.cuda, "_sleep"):
                torch.cuda._sleep(2_000_000)      # ~1 ms of bounded spinning on the side stream
        layer.forward_leased(leases, coefs, xd[t], ys[t])
        for lease in leases:
            lease.release()
    torch.cuda.synchronize()
    got = ys.cpu().numpy()
    for t, (ids, coefs) in enumerate(routes):
        want = s.want(oracle, ids, coefs, xs[t])
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), f"token {t}"
    assert cache.stats()["evictions"] > 0
    layer.close()
    cache.close()
    be2.close()
