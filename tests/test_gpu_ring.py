"""GPU ring-queue and lifecycle scenarios with analytically known results.

All-pass fixture (the scenario the reference's GPU tests use,
tests/gpu_cpu_ring_queue_test.cpp:17-50): identity rotation, zero centroids, zero sign
codes, f_add = -1e6 so every vector passes the filter, zero ex-codes and f_ex_rescale = 0
so the refined distance is f_ex_add + ||q||^2. The expected top-k is the k vectors with
the smallest f_ex_add, and every (query, vector) pair must be published exactly once,
through ring wraps, HBM spills, vanguard seeding/recovery and query chunking.
"""
import sys

import numpy as np
import pytest

import coraanns_amd as ca

pytestmark = pytest.mark.gpu
F32_MAX = np.finfo(np.float32).max


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class AllPass:
    def __init__(self, count=32768, k=100, clusters=8, queries=5, dim=96, padded=128):
        self.count, self.k, self.clusters, self.queries = count, k, clusters, queries
        self.dim, self.padded = dim, padded
        self.centroids = np.zeros((clusters, padded), np.float32)
        self.rotation = np.zeros((dim, padded), np.float32)
        self.rotation[np.arange(dim), np.arange(dim)] = 1
        self.short = np.zeros(count * padded // 32, np.uint32)
        self.sf = np.zeros((count, 3), np.float32)
        self.sf[:, 0] = -1e6
        self.long = np.zeros((count, padded * 7 // 8), np.uint8)
        self.lf = np.zeros((count, 2), np.float32)
        self.lf[:, 0] = 0.01 * ((np.arange(count) * 7919) % count)
        self.ids = np.arange(count, dtype=np.uint32)
        self.sizes = np.full(clusters, count // clusters, np.uint64)
        self.query = np.array([[0.01 * (1 + (q + d) % 7) for d in range(dim)] for q in range(queries)],
                              np.float32)
        order = np.argsort(self.lf[:, 0], kind="stable")
        self.expected = np.sort(order[:k]).astype(np.uint32)

    def engine(self, capacity, spill, vanguard, **kw):
        # the reference's ring scenarios: every candidate reaches the CPU, so the GPU
        # ex-code stages (seed thresholds, refined pre-filter) are off unless asked for
        kw.setdefault("gpu_seed_refine", False)
        kw.setdefault("gpu_refine_filter", False)
        e = ca.HybridIndex(0, queue_capacity=capacity, queue_spill_capacity=spill,
                           vanguard_size=vanguard, candidate_stats=True, **kw)
        e.load_from_raw_pointers(self.count, self.dim, self.padded, self.clusters, 7, self.centroids,
                                 self.rotation, self.short, self.sf, self.long, self.lf, self.ids,
                                 self.sizes)
        e.prepare_workspace(self.queries, self.k, self.clusters)
        return e

    def check(self, e, chunk, batch_q=4, expect_all_consumed=False, expect_all_published=True):
        ids = np.zeros((self.queries, self.k), np.uint32)
        dists = np.zeros((self.queries, self.k), np.float32)
        for b in range(0, self.queries, chunk):
            q = self.query[b:b + chunk]
            e.reset_buffer(q)
            d, i = e.search(q, self.k, self.clusters, batch_q)
            st = e.stats()
            if expect_all_published:
                assert st["submitted"] == q.shape[0] * self.count, "dropped or duplicated candidates"
            else:
                assert st["submitted"] <= q.shape[0] * self.count, "duplicated candidates"
            if expect_all_consumed:
                assert st["refined"] == q.shape[0] * self.count
            ids[b:b + chunk], dists[b:b + chunk] = i, d
        for q in range(self.queries):
            assert np.array_equal(np.sort(ids[q]), self.expected), "wrong nearest ids"
            norm = float((self.query[q].astype(np.float32) ** 2).sum())
            want = self.lf[ids[q], 0] + norm
            assert np.all(np.abs(dists[q] - want) < 1e-3), "torn or stale payload"


@pytest.fixture(scope="module")
def allpass():
    return AllPass()


@pytest.mark.parametrize("capacity", [8192, 262144])
@pytest.mark.parametrize("vanguard", [0, 5])
def test_all_pass_wraps_threads_secondary_chunks(allpass, capacity, vanguard):
    say(f"[gpu] all-pass capacity={capacity} vanguard={vanguard}")
    e = allpass.engine(capacity, 262144, vanguard)
    for threads in (1, 4, 16):
        for secondary in (False, True):
            e.configure(vanguard_size=vanguard, cpu_secondary_filter=secondary, candidate_stats=True,
                        cpu_threads=threads)
            for _ in range(2):
                allpass.check(e, allpass.queries, 4, not secondary)
                if capacity > allpass.queries * allpass.count:
                    assert e.stats()["spilled"] == 0
                allpass.check(e, 2, 4, not secondary)


@pytest.mark.parametrize("capacity", [8192, 262144])
@pytest.mark.parametrize("pair_seeds", [False, True])
def test_all_pass_with_gpu_excode_stages(allpass, capacity, pair_seeds):
    """The same scenarios with the GPU ex-code stages on (the fused vanguard pass, or the
    per-pair seed thresholds, and the refined pre-filter): fewer candidates reach the
    CPU, the top-k and its distances are unchanged."""
    say(f"[gpu] all-pass with GPU ex-code stages, capacity={capacity}, pair_seeds={pair_seeds}")
    for threads in (1, 16):
        e = allpass.engine(capacity, 262144, 5, gpu_seed_refine=True, gpu_refine_filter=True,
                           cpu_threads=threads, extra_flags=ca.FLAG_PAIR_SEEDS if pair_seeds else 0)
        allpass.check(e, allpass.queries, 4, False, False)
        assert e.stats()["submitted"] < allpass.queries * allpass.count
        allpass.check(e, 2, 4, False, False)


def test_forced_spill_and_refill():
    say("[gpu] forced spill")
    f = AllPass(count=1032, k=10)
    spilled = False
    for capacity in (32, 8192):
        e = f.engine(capacity, 8192, 0)
        for _ in range(3):
            f.check(e, f.queries)
            spilled |= e.stats()["spilled"] > 0
    assert spilled, "capacity 32 never exercised the HBM spill path"


@pytest.mark.parametrize("batch_q", [1, 2, 3, 5, 6, 7, 8, 24, 64])
def test_all_pass_batch_q(allpass, batch_q):
    say(f"[gpu] all-pass batch_q={batch_q}")
    e = allpass.engine(8192, 262144, 5)
    allpass.check(e, allpass.queries, batch_q)


def test_zero_candidates():
    say("[gpu] zero candidates")
    f = AllPass()
    f.sf[:, 0] = F32_MAX
    e = f.engine(8192, 1024, 0)
    for _ in range(3):
        e.reset_buffer(f.query)
        d, i = e.search(f.query, f.k, f.clusters)
        assert e.stats()["submitted"] == 0
        assert np.all(d == F32_MAX)


def test_spill_exhaustion_reports_error_then_recovers(allpass):
    say("[gpu] spill exhaustion")
    e = allpass.engine(32, 0, 0)
    e.reset_buffer(allpass.query)
    with pytest.raises(ca.EngineError) as err:
        e.search(allpass.query, allpass.k, allpass.clusters)
    assert "spill capacity exhausted" in str(err.value)
    e.reset_buffer(allpass.query)
    e.seed_thresholds(np.full(allpass.queries, -F32_MAX, np.float32))
    e.search(allpass.query, allpass.k, allpass.clusters)
    assert e.stats()["submitted"] == 0


@pytest.mark.parametrize("k", [10, 100, 513, 1024])
@pytest.mark.parametrize("stages", [False, True])
def test_high_k_vanguard_on_off_identical(k, stages):
    """The reference's high-k scenario (tests/gpu_cpu_highk_vanguard_test.cpp:81-90) with the
    vanguard pairs on and off; with the GPU ex-code stages on (stages), the vanguard pairs run
    in the fused pass, above top-128 in its staged form."""
    say(f"[gpu] high-k k={k} stages={stages}")
    f = AllPass(k=1024)
    e = f.engine(1 << 20, 1 << 20, 5, gpu_seed_refine=stages, gpu_refine_filter=stages)
    order = np.argsort(f.lf[:, 0], kind="stable")
    expected = np.sort(order[:k])
    results = []
    for vanguard in (0, 5):
        e.set_vanguard_size(vanguard)
        for chunk in (f.queries, 2):
            ids = []
            dists = []
            for b in range(0, f.queries, chunk):
                q = f.query[b:b + chunk]
                e.reset_buffer(q)
                d, i = e.search(q, k, f.clusters)
                mode = e.stats()["vanguard_mode"]
                if vanguard == 0:
                    assert mode == 0, mode
                elif not stages:
                    assert mode == 1, mode
                else:
                    assert mode == (4 if k > 128 else 2), mode
                ids.append(i)
                dists.append(d)
            ids = np.vstack(ids)
            dists = np.vstack(dists)
            for q in range(f.queries):
                assert np.array_equal(np.sort(ids[q]), expected)
            results.append((np.sort(ids, axis=1), np.sort(dists, axis=1)))
    for r in results[1:]:
        assert np.array_equal(r[0], results[0][0])
        assert np.allclose(r[1], results[0][1], rtol=1e-6)


def test_lifecycle_and_shape_errors():
    say("[gpu] lifecycle")
    dim, count, nq = 128, 32, 2
    q = np.zeros((nq, dim), np.float32)
    e = ca.HybridIndex(0, vanguard_size=0)
    with pytest.raises(ca.LogicError):
        e.prepare_workspace(nq, 10, 1)
    with pytest.raises(ca.LogicError):
        e.reset_buffer(q)
    with pytest.raises(ca.LogicError):
        e.search(q, 10, 1)
    rot = np.eye(dim, dtype=np.float32)
    sf = np.zeros((count, 3), np.float32)
    sf[:, 0] = 1e6
    e.load_from_raw_pointers(count, dim, dim, 1, 7, np.zeros((1, dim), np.float32), rot,
                             np.zeros(count * dim // 32, np.uint32), sf,
                             np.zeros((count, dim * 7 // 8), np.uint8), np.zeros((count, 2), np.float32),
                             np.arange(count, dtype=np.uint32), np.array([count], np.uint64))
    with pytest.raises(ca.LogicError):
        e.load_from_raw_pointers(count, dim, dim, 1, 7, np.zeros((1, dim), np.float32), rot,
                                 np.zeros(count * dim // 32, np.uint32), sf,
                                 np.zeros((count, dim * 7 // 8), np.uint8),
                                 np.zeros((count, 2), np.float32), np.arange(count, dtype=np.uint32),
                                 np.array([count], np.uint64))
    e.configure(queue_capacity=32, queue_spill_capacity=1024, vanguard_size=0)
    with pytest.raises(ca.InvalidArgument):
        e.prepare_workspace(65536, 10, 1)
    e.prepare_workspace(nq, 10, 1)
    with pytest.raises(ca.InvalidArgument):
        e.reset_buffer(np.zeros((nq + 1, dim), np.float32))
    with pytest.raises(ca.InvalidArgument):
        e.search(np.zeros((nq + 1, dim), np.float32), 10, 1)
    with pytest.raises(ca.InvalidArgument):
        e.search(q, 11, 1)
    with pytest.raises(ca.InvalidArgument):
        e.search(q, 10, 2)
    with pytest.raises(ca.InvalidArgument):
        e.search(q, 10, 1, 65)
    with pytest.raises(ca.InvalidArgument):
        e.search(q, 10, 1, 0)
    with pytest.raises(ca.LogicError):
        e.set_vanguard_size(1)
    for it in range(3):
        e.reset_buffer(q)
        e.seed_thresholds(np.full(nq, -1, np.float32))
        e.search(q, 10, 1)
        e.free_workspace()
        e.free_workspace()
        with pytest.raises(ca.LogicError):
            e.reset_buffer(q)
        e.set_vanguard_size(1 if it == 0 else 0)
        e.prepare_workspace(nq, 10, 1)


def test_unconsumed_ring_is_cleared_before_the_next_search(allpass):
    """A search whose records the CPU never consumed (the host stopped after the GPU side
    finished) leaves complete records in the ring. The next reset must clear them: else
    the next consumer takes them for its own search's records at the same positions."""
    say("[gpu] unconsumed ring, then a full search")
    e = allpass.engine(262144, 262144, 0)
    gpu, lib = e.gpu, ca._load()[0]
    e.reset_buffer(allpass.query)
    # GPU side only: 2 of the 8 clusters per query (positions the next search reuses)
    flags = ca.FLAG_CROSS_QUERY_REUSE | ca.FLAG_NO_GPU_SEED | ca.FLAG_NO_GPU_PREFILTER
    args = ca.cora_search_args(allpass.queries, allpass.k, 2, 4, 0, flags, 1.0)
    ca._gpu_check(gpu, lib.cora_gpu_launch_search(gpu, ca.C.byref(args)))
    st = ca.cora_search_stats()
    ca._gpu_check(gpu, lib.cora_gpu_sync(gpu, ca.C.byref(st)))
    assert st.produced == allpass.queries * 2 * (allpass.count // allpass.clusters)
    for _ in range(2):
        allpass.check(e, allpass.queries, 4)
