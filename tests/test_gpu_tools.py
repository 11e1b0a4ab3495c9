"""GPU index-build and evaluation tools (cora_tool_*): rotation, nearest-centroid
assignment, k-means and the exhaustive top-k that produces the benchmarks' ground truth.

Distances on the GPU are FP32 GEMM results, so near-ties may order differently from an
FP64 brute force; the checks compare what is fixed regardless of rounding: the FP64
distances of the returned neighbours against the FP64 optimum, to FP32 accuracy.
"""
import sys

import numpy as np
import pytest

import coraanns_amd as ca

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def fp64_scores(base, queries, metric):
    b = base.astype(np.float64)
    q = queries.astype(np.float64)
    if metric == 1:
        return -(q @ b.T)
    return (q * q).sum(1)[:, None] + (b * b).sum(1)[None, :] - 2.0 * (q @ b.T)


def check_topk(base, queries, k, metric, ids):
    assert ids.shape == (queries.shape[0], k)
    assert ids.max() < base.shape[0]
    for r in ids:  # no id twice
        assert len(np.unique(r)) == k
    s = fp64_scores(base, queries, metric)
    got = np.sort(np.take_along_axis(s, ids.astype(np.int64), axis=1), axis=1)
    best = np.sort(s, axis=1)[:, :k]
    scale = np.abs(s).max(axis=1, keepdims=True) + 1e-30
    assert np.all(np.abs(got - best) <= 1e-5 * scale), np.abs(got - best).max()
    # the returned order is ascending in distance up to FP32 rounding
    own = np.take_along_axis(s, ids.astype(np.int64), axis=1)
    assert np.all(np.diff(own, axis=1) >= -1e-5 * scale)


@pytest.mark.parametrize("metric", [0, 1])
def test_topk_single_block(metric):
    rng = np.random.default_rng(11 + metric)
    base = rng.standard_normal((5000, 72)).astype(np.float32)
    q = rng.standard_normal((70, 72)).astype(np.float32)
    say(f"[tools] topk single block metric={metric}")
    check_topk(base, q, 26, metric, ca.gpu_topk(base, q, 26, metric))


@pytest.mark.parametrize("metric", [0, 1])
def test_topk_two_level_blocks(metric):
    """More than 2^20 base rows: blocks of the base selected separately and merged; the
    true neighbours are planted in the last block, across the block boundary and in the
    first block, so a merge that drops a block fails."""
    rng = np.random.default_rng(5 + metric)
    nb, dim, nq, k = (1 << 21) + 777, 16, 24, 26
    base = rng.standard_normal((nb, dim)).astype(np.float32)
    q = rng.standard_normal((nq, dim)).astype(np.float32)
    blk = (nb + 2) // 3  # three blocks of the tool's split
    for i in range(nq):
        where = [nb - 1 - i, blk - 1 - i, blk + i, i][i % 4]
        base[where] = q[i] * (1.5 if metric == 1 else 1.0)
    say(f"[tools] topk two-level metric={metric} nb={nb}")
    ids = ca.gpu_topk(base, q, k, metric)
    check_topk(base, q, k, metric, ids)
    for i in range(nq):
        where = [nb - 1 - i, blk - 1 - i, blk + i, i][i % 4]
        assert where in ids[i]


def test_topk_k_equals_nb():
    rng = np.random.default_rng(3)
    base = rng.standard_normal((40, 64)).astype(np.float32)
    q = rng.standard_normal((5, 64)).astype(np.float32)
    ids = ca.gpu_topk(base, q, 40, 0)
    assert np.all(np.sort(ids, axis=1) == np.arange(40))
    check_topk(base, q, 40, 0, ids)


def test_assign_and_rotate():
    rng = np.random.default_rng(21)
    x = rng.standard_normal((20000, 96)).astype(np.float32)
    c = rng.standard_normal((300, 96)).astype(np.float32)
    say("[tools] assign + rotate")
    a = ca.gpu_assign(x, c)
    s = fp64_scores(c, x, 0)
    got = s[np.arange(x.shape[0]), a.astype(np.int64)]
    scale = np.abs(s).max(axis=1)
    assert np.all(got - s.min(axis=1) <= 1e-5 * scale)
    R = np.linalg.qr(rng.standard_normal((128, 128)))[0][:96].astype(np.float32)
    xr = ca.gpu_rotate(x, R)
    ref = x.astype(np.float64) @ R.astype(np.float64)
    assert np.allclose(xr, ref, rtol=0, atol=1e-4)


def test_kmeans_reduces_inertia():
    rng = np.random.default_rng(8)
    centers = rng.standard_normal((32, 48)).astype(np.float32) * 4
    lab = rng.integers(0, 32, 30000)
    x = (centers[lab] + rng.standard_normal((30000, 48)).astype(np.float32)).astype(np.float32)
    say("[tools] kmeans")
    c1 = ca.gpu_kmeans(x, 32, 1, seed=4)
    c20 = ca.gpu_kmeans(x, 32, 20, seed=4)

    def inertia(c):
        return fp64_scores(c, x, 0).min(axis=1).sum()

    assert np.isfinite(c20).all()
    assert inertia(c20) <= inertia(c1) * (1 + 1e-6)


def test_kmeans_reseeds_empty_clusters():
    """Well-separated unit-norm clusters (the 20M x 768 configuration's shape, scaled down)
    with twice as many centroids as true clusters: random initialisation leaves some true
    clusters without a centroid and the absorbing centroids drift to the origin, emptying
    others. Empty clusters are re-seeded by splitting populated ones, so at the end every
    centroid owns training rows and none sits near the origin."""
    rng = np.random.default_rng(9)
    ntrue, k, dim, n = 64, 128, 256, 32768
    centers = rng.standard_normal((ntrue, dim)).astype(np.float32)
    x = centers[rng.integers(0, ntrue, n)] + 0.5 * rng.standard_normal((n, dim)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    say("[tools] kmeans re-seeds empty clusters")
    c = ca.gpu_kmeans(x, k, 20, seed=5)
    a = ca.gpu_assign(x, c)
    sizes = np.bincount(a, minlength=k)
    assert sizes.min() >= 1, np.sort(sizes)[:8]
    # a populated centroid is the mean of one true cluster's unit vectors (norm ~0.9)
    assert np.linalg.norm(c, axis=1).min() > 0.5


@pytest.mark.parametrize("dim,P,metric", [(128, 128, 0), (128, 128, 1), (250, 256, 0), (768, 768, 1)])
def test_gpu_builder_matches_host_builder(dim, P, metric, tmp_path):
    """The GPU quantiser (cora_build_ivf_gpu) writes the same index file, byte for byte, as
    the host builder (cora_build_ivf, itself pinned to the reference builder's codes) on the
    GPU-rotated rows: sign codes, all factors, ex-codes, ids."""
    rng = np.random.default_rng(dim + metric)
    n, nl = 3000, 12
    centers = rng.standard_normal((nl, dim)).astype(np.float32)
    x = (centers[rng.integers(0, nl, n)] + 0.6 * rng.standard_normal((n, dim))).astype(np.float32)
    if metric == 1:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
    x[7] = centers[0]  # a row equal to its centre's neighbourhood, ties in |o|
    R = np.linalg.qr(rng.standard_normal((P, P)))[0][:dim].astype(np.float32)
    cent = ca.gpu_kmeans(x, nl, 5, seed=3)
    assign = ca.gpu_assign(x, cent)
    cr = (cent.astype(np.float64) @ R.astype(np.float64)).astype(np.float32)
    say(f"[tools] GPU builder vs host builder, dim {dim} P {P} metric {metric}")
    ca.build_ivf(tmp_path / "host.index", ca.gpu_rotate(x, R), cr, assign, R, metric=metric)
    ca.build_ivf_gpu(tmp_path / "gpu.index", x, cr, assign, R, metric=metric)
    a, b = (tmp_path / "host.index").read_bytes(), (tmp_path / "gpu.index").read_bytes()
    assert len(a) == len(b)
    if a != b:
        ha, hb = ca.IvfIndex(tmp_path / "host.index"), ca.IvfIndex(tmp_path / "gpu.index")
        for name in ("short_data", "short_factors", "long_codes", "ex_factors", "ids"):
            u, v = getattr(ha, name), getattr(hb, name)
            bad = np.nonzero((u != v).reshape(u.shape[0], -1).any(1))[0]
            assert bad.size == 0, (name, bad[:8], bad.size)
        assert a == b


def test_topk_l2_beyond_2_32_work_items():
    """More than 2^32 / 64 base rows (70M x 4, L2): every row's norm takes part (a launch of
    one 64-lane workgroup per row would exceed the dispatch's 32-bit work-item count and
    leave the last rows without norms, which then look nearest)."""
    rng = np.random.default_rng(70)
    nb, dim, nq, k = 70_000_000, 4, 4, 10
    base = rng.standard_normal((nb, dim), dtype=np.float32)
    q = rng.standard_normal((nq, dim), dtype=np.float32)
    plant = [3, 20_000_001, 45_000_007, nb - 2]
    for i, w in enumerate(plant):
        base[w] = q[i]
    say(f"[tools] topk L2 over {nb:,} rows")
    ids = ca.gpu_topk(base, q, k, 0)
    for i, w in enumerate(plant):
        assert ids[i, 0] == w, (i, ids[i, :3])
        d = ((base.astype(np.float64) - q[i]) ** 2).sum(1) if i == 0 else None
        if d is not None:
            want = np.argsort(d, kind="stable")[:k]
            assert set(want.tolist()) == set(ids[i].tolist())
