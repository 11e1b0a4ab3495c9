"""GPU parity tests: every stage of the HIP path against the CPU oracle, through the C-ABI.

Each stage is checked on the GPU's own inputs for that stage (e.g. the quantiser on the
GPU-rotated queries), so integer results are compared bit-exactly and floating-point
ones within 1e-5 relative (scaled by the magnitude of the terms), as the north star asks.
"""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import cora_oracle as orc
import coraanns_amd as ca
from conftest import GOLDEN, read_fbin

pytestmark = pytest.mark.gpu

F32_MAX = np.finfo(np.float32).max


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def planes_to_bits(planes):
    """GPU q-planes [nq][8][W] (dim 32w+l at bit l) -> qint bit planes [nq][8][P]."""
    nq, B, W = planes.shape
    sh = np.arange(32, dtype=np.uint32)
    return ((planes[:, :, :, None] >> sh) & 1).reshape(nq, B, W * 32).astype(np.uint8)


def qint_from_planes(planes):
    bits = planes_to_bits(planes).astype(np.int64)
    u = sum(bits[:, j, :] << j for j in range(8))
    return np.where(u >= 128, u - 256, u).astype(np.int32)


class Case:
    def __init__(self, path, queries, base=None):
        self.path = path
        self.queries = np.ascontiguousarray(queries, np.float32)
        self.base = base
        self.file = orc.read_ivf(path)
        self.sd = orc.search_data(self.file)
        self.ivf = ca.IvfIndex(path)


def make_engine(case, nprobe, topk, vanguard=0, frozen=True, secondary=False, reuse=True,
                lower_bound_scale=1.0, **kw):
    """lower_bound_scale 1.0: the reference Bitwise producer's bound, whose candidate sets
    the oracle restates."""
    eng = ca.HybridIndex(0, vanguard_size=vanguard, frozen_thresholds=frozen,
                         cpu_secondary_filter=secondary, cross_query_reuse=reuse,
                         metric=case.file.metric, gpu_filter_timing=True,
                         lower_bound_scale=lower_bound_scale, **kw)
    eng.load_ivf(case.ivf)
    eng.prepare_workspace(case.queries.shape[0], topk, nprobe)
    return eng


@pytest.fixture(scope="module")
def golden_l2():
    return Case(GOLDEN / "l2_d96" / "ivf.index", read_fbin(GOLDEN / "l2_d96" / "queries.fbin"),
                read_fbin(GOLDEN / "l2_d96" / "base.fbin"))


@pytest.fixture(scope="module")
def golden_ip():
    return Case(GOLDEN / "ip_d64" / "ivf.index", read_fbin(GOLDEN / "ip_d64" / "queries.fbin"),
                read_fbin(GOLDEN / "ip_d64" / "base.fbin"))


@pytest.fixture(scope="module")
def synth(tmp_path_factory):
    """20,000 x 128 (P = 128), 64 clusters, 96 queries, built by this repository's builder."""
    rng = np.random.default_rng(7)
    n, dim, nl, nq = 20000, 128, 64, 96
    centers = rng.normal(0, 1, (nl, dim))
    lab = rng.integers(0, nl, n)
    x = (centers[lab] + rng.normal(0, 0.4, (n, dim))).astype(np.float32)
    q = (centers[rng.integers(0, nl, nq)] + rng.normal(0, 0.4, (nq, dim))).astype(np.float32)
    d = ((x[:, None, :] - centers[None]) ** 2).sum(2)
    assign = d.argmin(1).astype(np.uint32)
    cent = np.stack([x[assign == c].mean(0) for c in range(nl)])
    a = rng.normal(size=(dim, dim))
    R = np.linalg.qr(a)[0].T.astype(np.float32)
    path = tmp_path_factory.mktemp("synth") / "synth.index"
    ca.build_ivf(path, (x.astype(np.float64) @ R).astype(np.float32),
                 (cent @ R).astype(np.float32), assign, R, metric=0)
    return Case(path, q, x)


@pytest.fixture(scope="module")
def synth_ip768(tmp_path_factory):
    """6,000 x 768 unit vectors (P = 768, 24 words per code), 24 clusters, inner product,
    48 queries: the embedding shape of the 20M x 768 configuration."""
    rng = np.random.default_rng(768)
    n, dim, nl, nq = 6000, 768, 24, 48
    centers = rng.normal(0, 1, (nl, dim))
    x = centers[rng.integers(0, nl, n)] + rng.normal(0, 0.5, (n, dim))
    x = (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)
    q = centers[rng.integers(0, nl, nq)] + rng.normal(0, 0.5, (nq, dim))
    q = (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)
    assign = (x @ centers.T).argmax(1).astype(np.uint32)
    cent = np.stack([x[assign == c].mean(0) for c in range(nl)])
    R = np.linalg.qr(rng.normal(size=(dim, dim)))[0].T.astype(np.float32)
    path = tmp_path_factory.mktemp("synth768") / "synth768.index"
    ca.build_ivf(path, (x.astype(np.float64) @ R).astype(np.float32),
                 (cent @ R).astype(np.float32), assign, R, metric=1)
    return Case(path, q, x)



def _small_case(tmp_path_factory, name, seed, n, dim, nl, nq, metric):
    """n x dim Gaussian-mixture vectors in nl clusters (unit norm for inner product), nq
    queries from the same mixture, clustered by nearest center and built by this
    repository's builder."""
    rng = np.random.default_rng(seed)
    centers = rng.normal(0, 1, (nl, dim))
    x = centers[rng.integers(0, nl, n)] + rng.normal(0, 0.5, (n, dim))
    q = centers[rng.integers(0, nl, nq)] + rng.normal(0, 0.5, (nq, dim))
    if metric == 1:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        q /= np.linalg.norm(q, axis=1, keepdims=True)
        assign = (x @ centers.T).argmax(1).astype(np.uint32)
    else:
        assign = ((x[:, None, :] - centers[None]) ** 2).sum(2).argmin(1).astype(np.uint32)
    x, q = x.astype(np.float32), q.astype(np.float32)
    cent = np.stack([x[assign == c].mean(0) for c in range(nl)])
    R = np.linalg.qr(rng.normal(size=(dim, dim)))[0].T.astype(np.float32)
    path = tmp_path_factory.mktemp(name) / f"{name}.index"
    ca.build_ivf(path, (x.astype(np.float64) @ R).astype(np.float32),
                 (cent @ R).astype(np.float32), assign, R, metric=metric)
    return Case(path, q, x)


@pytest.fixture(scope="module")
def synth_l2_256(tmp_path_factory):
    """4,000 x 256 (P = 256, 8 words per code), 16 clusters, L2, 32 queries: the
    matrix-core kernels at W = 8."""
    return _small_case(tmp_path_factory, "synth256", 256, 4000, 256, 16, 32, 0)


@pytest.fixture(scope="module")
def synth_l2_192(tmp_path_factory):
    """4,000 x 192 (P = 192, 6 words per code), 16 clusters, L2, 32 queries: the
    16x16x32 matrix-core kernel at W = 6."""
    return _small_case(tmp_path_factory, "synth192", 192, 4000, 192, 16, 32, 0)


@pytest.fixture(scope="module")
def synth_ip1024(tmp_path_factory):
    """4,000 x 1,024 unit vectors (P = 1,024, 32 words per code), 16 clusters, inner
    product, 24 queries: the matrix-core kernels at W = 32."""
    return _small_case(tmp_path_factory, "synth1024", 1024, 4000, 1024, 16, 24, 1)


@pytest.fixture(scope="module")
def synth_ip512(tmp_path_factory):
    """4,000 x 512 unit vectors (P = 512, 16 words per code), 16 clusters, inner product, 32
    queries: the matrix-core kernels at W = 16, with LUT4 on the matrix cores."""
    return _small_case(tmp_path_factory, "synth512", 512, 4000, 512, 16, 32, 1)

def run_frozen(case, nprobe, topk, thresholds=None, **kw):
    eng = make_engine(case, nprobe, topk, **kw)
    nq = case.queries.shape[0]
    eng.reset_buffer(case.queries)
    if thresholds is not None:
        eng.seed_thresholds(thresholds)
    d, i = eng.search(case.queries, topk, nprobe)
    return eng, d, i


def gpu_intermediates(eng, case, nprobe):
    nq, P = case.queries.shape[0], case.file.padded_dim
    W = P // 32
    g = {
        "qr": eng.debug_read(ca.DBG_ROTATED_QUERIES, (nq, P), np.float32),
        "k1": eng.debug_read(ca.DBG_K1XSUMQ, (nq,), np.float32),
        "kb": eng.debug_read(ca.DBG_KBXSUMQ, (nq,), np.float32),
        "width": eng.debug_read(ca.DBG_Q_WIDTH, (nq,), np.float32),
        "width2": eng.debug_read(ca.DBG_Q_WIDTH2, (nq,), np.float32),
        "planes": eng.debug_read(ca.DBG_Q_PLANES, (nq, 16, W), np.uint32),
        "pidx": eng.debug_read(ca.DBG_PROBE_IDX, (nq, nprobe), np.int32),
        "gadd": eng.debug_read(ca.DBG_PROBE_GADD, (nq, nprobe), np.float32),
        "gerr": eng.debug_read(ca.DBG_PROBE_GERR, (nq, nprobe), np.float32),
    }
    return g


CASES = ["golden_l2", "golden_ip", "synth", "synth_ip768"]
# P = 192, 256, 512 and 1,024: the matrix-core kernels' other code widths
CASES_WIDE = ["synth_l2_192", "synth_l2_256", "synth_ip512", "synth_ip1024"]


@pytest.mark.parametrize("case_name", CASES)
def test_query_preparation(case_name, request):
    case = request.getfixturevalue(case_name)
    say(f"[gpu] query prep parity on {case_name}")
    nprobe = min(4, case.file.nlist)
    eng, _, _ = run_frozen(case, nprobe, 10)
    g = gpu_intermediates(eng, case, nprobe)
    qr_ref = orc.rotate(case.queries, case.sd.rotator)
    scale = np.abs(case.queries).sum(1, keepdims=True) * np.abs(case.sd.rotator).max()
    assert np.all(np.abs(g["qr"] - qr_ref) <= 1e-5 * scale)
    # k1/kb from the GPU-rotated queries
    k1, kb = orc.query_factors(g["qr"], case.file.ex_bits)
    s = np.abs(g["qr"]).sum(1) + 1e-30
    assert np.all(np.abs(g["k1"] - k1) <= 1e-5 * s)
    assert np.all(np.abs(g["kb"] - kb) <= 1e-5 * 127.5 * s)
    # Bq=8 quantisation and its residual: bit-exact on the same rotated input
    qint, width = orc.quantize_query_bitwise(g["qr"])
    assert np.array_equal(g["width"].view(np.uint32), width.view(np.uint32))
    assert np.array_equal(qint_from_planes(g["planes"][:, :8]), qint)
    qres, width2 = orc.quantize_query_residual(g["qr"], qint, width)
    assert np.array_equal(g["width2"].view(np.uint32), width2.view(np.uint32))
    assert np.array_equal(qint_from_planes(g["planes"][:, 8:]), qres)


def test_bq8_quantiser_at_rounding_boundaries(tmp_path):
    """The GPU's Bq=8 query quantisation on rows placed at its rounding boundaries: exact
    ties with width 2^-3, and components where q * f32(1/width) and q / width round to
    different integers. The index's rotator is the identity and the FP32 GEMM rotates, so
    the quantiser sees the rows unchanged; the expected codes come from exact rational
    arithmetic (query_kernels.cuh:158-176: __float2int_rn(q * inv_width))."""
    from test_oracle import bq8_expected, f32_round, rint_even
    from fractions import Fraction
    dim = 64
    rng = np.random.default_rng(31)
    rows = []
    tie = np.zeros(dim, np.float32)
    tie[0] = np.float32(127.0 / 8.0)
    tie[1:9] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5], np.float32) / np.float32(8.0)
    rows.append(tie)
    while len(rows) < 24:
        row = np.zeros(dim, np.float32)
        row[0] = np.float32(rng.uniform(0.1, 50.0))
        _, width, inv = bq8_expected(row[:1])
        cases = []
        for k in range(-120, 121, 3):
            c = np.float32((k + 0.5) * float(width))
            for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
                a = rint_even(Fraction(float(f32_round(Fraction(float(cand)) * Fraction(float(inv))))))
                b = rint_even(Fraction(float(f32_round(Fraction(float(cand)) / Fraction(float(width))))))
                if a != b:
                    cases.append(cand)
        if cases:
            row[1:1 + min(dim - 1, len(cases))] = cases[:dim - 1]
            rows.append(row)
    q = np.stack(rows).astype(np.float32)
    nq = q.shape[0]
    base = rng.normal(0, 1, (256, dim)).astype(np.float32)
    R = np.eye(dim, dtype=np.float32)
    path = tmp_path / "eye.index"
    ca.build_ivf(path, base, base[:2].copy(), (np.arange(256) % 2).astype(np.uint32), R, metric=0)
    case = Case(path, q)
    say(f"[gpu] Bq=8 quantiser on {nq} boundary rows")
    eng, _, _ = run_frozen(case, 2, 10, extra_flags=ca.FLAG_FP32_GEMM)
    g = gpu_intermediates(eng, case, 2)
    assert np.array_equal(g["qr"].view(np.uint32), q.view(np.uint32))  # the identity rotation is exact
    got = qint_from_planes(g["planes"][:, :8])
    for r in range(nq):
        want, width, _ = bq8_expected(q[r])
        assert g["width"][r] == width, r
        assert np.array_equal(got[r], want), r
    eng.close()


@pytest.mark.parametrize("case_name", CASES)
@pytest.mark.parametrize("fp32", [False, True])
def test_coarse_probe(case_name, fp32, request):
    """Probe selection from the split-FP16 distance GEMM (default) and the FP32 one."""
    case = request.getfixturevalue(case_name)
    nprobe = min(6, case.file.nlist)
    say(f"[gpu] coarse probe parity on {case_name} nprobe={nprobe} fp32={fp32}")
    eng, _, _ = run_frozen(case, nprobe, 10, extra_flags=ca.FLAG_FP32_GEMM if fp32 else 0)
    g = gpu_intermediates(eng, case, nprobe)
    idx, gadd, gerr, l2 = orc.coarse_probe(g["qr"], case.sd.centroids, case.file.nlist, case.file.metric)
    for q in range(idx.shape[0]):
        got = g["pidx"][q]
        # ascending exact distance; the selected set equals the oracle's up to ties at 1e-5
        d_all = dict(zip(idx[q].tolist(), l2[q].tolist()))
        dg = np.array([d_all[c] for c in got])
        assert np.all(np.diff(dg) >= -1e-5 * (np.abs(dg).max() + 1))
        kth = l2[q][nprobe - 1]
        strict = set(idx[q][l2[q] < kth - 1e-5 * (abs(kth) + 1)].tolist())
        assert strict <= set(got.tolist())
        assert len(set(got.tolist())) == nprobe
        # g_add / g_error of the selected probes
        qq = g["qr"][q].astype(np.float64)
        c = case.sd.centroids[got].astype(np.float64)
        l2x = ((qq - c) ** 2).sum(1)
        ipx = c @ qq
        want = l2x if case.file.metric == 0 else -ipx
        sc = (qq ** 2).sum() + (c ** 2).sum(1)
        assert np.all(np.abs(g["gadd"][q] - want) <= 1e-5 * sc)
        assert np.all(np.abs(g["gerr"][q] - np.sqrt(l2x)) <= 1e-5 * np.sqrt(sc))


@pytest.mark.parametrize("case_name", CASES)
def test_probe_distance_matrix(case_name, request):
    """The whole coarse-probe distance matrix ||q'||^2 + ||c'||^2 - 2 <q',c'> of the
    split-FP16 GEMM (default) and of the FP32 one against FP64 from the same rotated
    queries, relative to ||q'||^2 + ||c'||^2: within 1e-6 (FP32 rounding of the three terms
    and of the sum, plus at most 3 * 2^-22 per product term for the split operands). A GEMM
    on plain FP16 operands (the lo halves dropped) errs by ~2^-11 per term, 1e-5 and more
    here, and fails."""
    case = request.getfixturevalue(case_name)
    nprobe = min(4, case.file.nlist)
    nq, P, nl = case.queries.shape[0], case.file.padded_dim, case.file.nlist
    c = case.sd.centroids.astype(np.float64)
    for name, flags in (("split-fp16", 0), ("fp32", ca.FLAG_FP32_GEMM)):
        say(f"[gpu] probe distance matrix on {case_name}, {name} GEMM")
        eng, _, _ = run_frozen(case, nprobe, 10, extra_flags=flags)
        q = eng.debug_read(ca.DBG_ROTATED_QUERIES, (nq, P), np.float32).astype(np.float64)
        d = eng.debug_read(ca.DBG_PROBE_DIST, (nq, nl), np.float32)
        qn, cn = (q ** 2).sum(1)[:, None], (c ** 2).sum(1)[None]
        want = qn + cn - 2 * q @ c.T
        err = np.abs(d - want) / (qn + cn)
        assert err.max() <= 1e-6, (name, float(err.max()))


def order_keys(d):
    """The select's total order on FP32 distances: IEEE bits made monotone as unsigned."""
    u = np.ascontiguousarray(d, dtype=np.float32).view(np.uint32)
    return np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint32)


@pytest.mark.parametrize("nlist,distinct,nprobe", [(12000, 0, 16), (16384, 0, 32), (16384, 0, 64),
                                                   (16384, 40, 32), (12000, 7, 64), (20000, 0, 32),
                                                   (40000, 0, 16), (65536, 0, 64), (65536, 0, 33),
                                                   (40000, 50, 64),
                                                   # the fused select's wide slots (16 keys per tile)
                                                   (16384, 0, 128), (16384, 0, 512), (16384, 40, 256),
                                                   (40000, 50, 300), (65536, 0, 1024),
                                                   # beyond the LDS-held selects: up to the reference's 65,536
                                                   (16384, 0, 8192), (12000, 7, 5000), (40000, 50, 20000),
                                                   (65536, 0, 65536)])
def test_select_exact_on_gpu_distances(nlist, distinct, nprobe, tmp_path):
    """The probe select over the materialised distance matrix (8,192 < nlist <= 16,384:
    distances in registers; beyond: two streaming passes; either way per-wave candidates
    below a bound from minima, ranked by (distance, cluster id); heavy ties fall back to the
    radix select; nprobe > 4,096: radix select of the k-th key, ordered compaction, stable
    radix sort in global scratch) against an exact sort of the GPU's own distance matrix by
    (distance key, cluster id); then, where the fused select applies (nprobe <= 64, or up to
    1,024 with at most ~4.5 probes per 128-cluster tile on average), the default search, whose
    GEMM epilogue keeps 8 (16 above nprobe 64) keys per 128-cluster tile and whose merge
    selects from them (above nprobe 64 a bitwise search for the k-th key, then a sort of the
    keys up to it), must give the same probe lists. distinct > 0 repeats that many
    centroids over the whole list, so every distance is tied nlist / distinct times: the
    fused select cannot settle such queries from its candidates and sends them to its
    fallback (the query's distance row computed again, the generic select)."""
    rng = np.random.default_rng(nlist + distinct)
    dim, nq = 64, 40
    n = 2 * nlist
    cent = rng.normal(0, 1, (nlist, dim)).astype(np.float32)
    if distinct:
        cent = cent[np.arange(nlist) % distinct]
    assign = rng.integers(0, nlist, n).astype(np.uint32)
    x = (cent[assign] + rng.normal(0, 0.1, (n, dim))).astype(np.float32)
    q = (cent[rng.integers(0, nlist, nq)] + rng.normal(0, 0.1, (nq, dim))).astype(np.float32)
    R = np.linalg.qr(rng.normal(size=(dim, dim)))[0].T.astype(np.float32)
    path = tmp_path / "sel.index"
    ca.build_ivf(path, (x.astype(np.float64) @ R).astype(np.float32), (cent.astype(np.float64) @ R).astype(np.float32),
                 assign, R, metric=0)
    case = Case(path, q)
    say(f"[gpu] select on GPU distances, nlist={nlist} distinct={distinct} nprobe={nprobe}")
    eng, _, _ = run_frozen(case, nprobe, 10, extra_flags=ca.FLAG_UNFUSED_PROBE)
    d = eng.debug_read(ca.DBG_PROBE_DIST, (nq, nlist), np.float32)
    pidx = eng.debug_read(ca.DBG_PROBE_IDX, (nq, nprobe), np.int32)
    fb = eng.debug_read(ca.DBG_PROBE_FALLBACK, (nq + 1,), np.uint32)
    eng.close()
    assert fb[0] == 0
    keys = order_keys(d)
    ids = np.arange(nlist)
    want = np.stack([np.lexsort((ids, keys[qi]))[:nprobe] for qi in range(nq)])
    for qi in range(nq):
        assert np.array_equal(pidx[qi], want[qi]), qi
    fused_applies = 8192 <= nlist <= 65536 and (nprobe <= 64 or (
        nprobe <= 1024 and nprobe * 256 <= 9 * nlist and -(-nlist // 128) * 16 <= 8192))
    if not fused_applies:
        return
    say(f"[gpu] fused select, nlist={nlist} distinct={distinct} nprobe={nprobe}")
    eng, _, _ = run_frozen(case, nprobe, 10)
    fused = eng.debug_read(ca.DBG_PROBE_IDX, (nq, nprobe), np.int32)
    fb = eng.debug_read(ca.DBG_PROBE_FALLBACK, (nq + 1,), np.uint32)
    with pytest.raises(ca.EngineError):
        eng.debug_read(ca.DBG_PROBE_DIST, (nq, nlist), np.float32)
    eng.close()
    for qi in range(nq):
        assert np.array_equal(fused[qi], want[qi]), qi
    rows = fb[1:1 + fb[0]]
    assert len(set(rows.tolist())) == len(rows) and np.all(rows < nq)
    if 0 < distinct < 16:
        # every 128-cluster tile holds 8 or more copies of the nearest centroid: more than the
        # epilogue keeps (nprobe <= 64)
        assert fb[0] > 0, "tied distances never reached the fallback"
    elif not distinct:
        assert fb[0] <= nq // 4, "the merge settled too few queries"


def test_fused_probe_fallback_sweep(tmp_path):
    """More fallback queries than the fallback GEMM's grid holds (1,024 rows per sweep): 10
    centroids repeated over 10,000 clusters (each 128-cluster tile holds 12 or 13 copies of a
    query's nearest, more than the 8 keys per tile the epilogue keeps, so no query is settled
    by the merge), 2,500 queries, against the select over the materialised matrix."""
    rng = np.random.default_rng(2500)
    nlist, distinct, dim, nq, nprobe = 10000, 10, 64, 2500, 40
    cent = rng.normal(0, 1, (distinct, dim)).astype(np.float32)[np.arange(nlist) % distinct]
    n = 2 * nlist
    assign = rng.integers(0, nlist, n).astype(np.uint32)
    x = (cent[assign] + rng.normal(0, 0.1, (n, dim))).astype(np.float32)
    q = (cent[rng.integers(0, nlist, nq)] + rng.normal(0, 0.1, (nq, dim))).astype(np.float32)
    R = np.linalg.qr(rng.normal(size=(dim, dim)))[0].T.astype(np.float32)
    path = tmp_path / "sweep.index"
    ca.build_ivf(path, (x.astype(np.float64) @ R).astype(np.float32), (cent.astype(np.float64) @ R).astype(np.float32),
                 assign, R, metric=0)
    case = Case(path, q)
    say(f"[gpu] fused select fallback sweep, nq={nq} nlist={nlist}")
    eng, _, _ = run_frozen(case, nprobe, 10, extra_flags=ca.FLAG_UNFUSED_PROBE)
    want = eng.debug_read(ca.DBG_PROBE_IDX, (nq, nprobe), np.int32)
    eng.close()
    eng, _, _ = run_frozen(case, nprobe, 10)
    got = eng.debug_read(ca.DBG_PROBE_IDX, (nq, nprobe), np.int32)
    fb = eng.debug_read(ca.DBG_PROBE_FALLBACK, (nq + 1,), np.uint32)
    eng.close()
    assert fb[0] > 1024, int(fb[0])
    assert np.array_equal(np.sort(fb[1:1 + fb[0]]), np.unique(fb[1:1 + fb[0]]))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dim,metric", [(96, 0), (768, 1)])
def test_sliced_upload_matches_one_pass(dim, metric, tmp_path):
    """Queries uploaded from the staging buffer in slices (4,100 queries: three slices of
    512 / 1,920 / 1,668 rows, each rotated, prepared and probed as it lands) give the
    same rotated queries, query factors, Bq=8 planes, probe lists and frozen top-k, bit for
    bit, as the same queries searched in chunks of 1,400 that upload and run in one pass."""
    rng = np.random.default_rng(4100 + dim)
    nlist, n, nq, nprobe, topk = 8192, 40000, 4100, 16, 10
    cent = rng.normal(0, 1, (nlist, dim)).astype(np.float32)
    assign = rng.integers(0, nlist, n).astype(np.uint32)
    x = (cent[assign] + rng.normal(0, 0.3, (n, dim))).astype(np.float32)
    q = (cent[rng.integers(0, nlist, nq)] + rng.normal(0, 0.3, (nq, dim))).astype(np.float32)
    if metric == 1:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        q /= np.linalg.norm(q, axis=1, keepdims=True)
    P = (dim + 63) // 64 * 64  # the rotator is [dim][P]: orthonormal rows, padded to whole 64s
    R = np.linalg.qr(rng.normal(size=(P, P)))[0][:dim].astype(np.float32)
    path = tmp_path / "sliced.index"
    ca.build_ivf(path, (x.astype(np.float64) @ R).astype(np.float32), (cent.astype(np.float64) @ R).astype(np.float32),
                 assign, R, metric=metric)
    case = Case(path, q)
    say(f"[gpu] sliced upload vs one pass, nq={nq} dim={dim} nlist={nlist}")
    eng, d, i = run_frozen(case, nprobe, topk, vanguard=3)
    g = gpu_intermediates(eng, case, nprobe)
    eng.close()
    for c0 in range(0, nq, 1400):
        sub = Case(path, q[c0:c0 + 1400])
        e2, d2, i2 = run_frozen(sub, nprobe, topk, vanguard=3)
        g2 = gpu_intermediates(e2, sub, nprobe)
        e2.close()
        for key, v in g2.items():
            assert np.array_equal(g[key][c0:c0 + 1400], v), (key, c0)
        assert np.array_equal(i[c0:c0 + 1400], i2) and np.array_equal(d[c0:c0 + 1400], d2), c0


def test_end_to_end_nprobe_8192(tmp_path):
    """nprobe 8,192 (beyond the LDS-held selects) end to end with frozen infinite thresholds:
    probe lists against the oracle's FP64 coarse probe, every vector of every probed
    cluster a candidate exactly once, and the top-k of the oracle's restatement."""
    rng = np.random.default_rng(8192)
    nlist, dim, n, nq, nprobe, topk = 16384, 128, 60000, 24, 8192, 10
    cent = rng.normal(0, 1, (nlist, dim)).astype(np.float32)
    assign = rng.integers(0, nlist, n).astype(np.uint32)
    x = (cent[assign] + rng.normal(0, 0.3, (n, dim))).astype(np.float32)
    q = (cent[rng.integers(0, nlist, nq)] + rng.normal(0, 0.3, (nq, dim))).astype(np.float32)
    R = np.linalg.qr(rng.normal(size=(dim, dim)))[0].T.astype(np.float32)
    path = tmp_path / "np8192.index"
    ca.build_ivf(path, (x.astype(np.float64) @ R).astype(np.float32), (cent.astype(np.float64) @ R).astype(np.float32),
                 assign, R, metric=0)
    case = Case(path, q)
    say(f"[gpu] end-to-end at nprobe {nprobe}, nlist {nlist}")
    eng, d, i = run_frozen(case, nprobe, topk, vanguard=5)
    st = eng.stats()
    g = gpu_intermediates(eng, case, nprobe)
    idx, _, _, l2 = orc.coarse_probe(g["qr"], case.sd.centroids, nprobe, case.file.metric)
    for qi in range(nq):
        got = g["pidx"][qi]
        assert len(set(got.tolist())) == nprobe
        kth = float(l2[qi][-1])
        band = 1e-5 * (abs(kth) + 1)
        # every cluster clearly inside the oracle's top-nprobe is probed, ascending order
        assert set(idx[qi][l2[qi] < kth - band].tolist()) <= set(got.tolist()), qi
        cd = ((g["qr"][qi].astype(np.float64) - case.sd.centroids[got].astype(np.float64)) ** 2).sum(1)
        assert np.all(np.diff(cd) >= -band), qi
    od, oi, cands = oracle_topk_from_gpu(case, g, nprobe, topk)
    assert st["submitted"] == sum(len(c) for c in cands)
    assert_topk_equal(d, i, od, oi)
    eng.close()


@pytest.mark.parametrize("nlist", [9000, 20000, 40000])
def test_coarse_probe_large_nlist(nlist, tmp_path):
    """Top-nprobe selection over nlist above the LDS-staged select (register-staged select,
    1,024 threads per query) against the oracle's FP64 probe distances."""
    rng = np.random.default_rng(nlist)
    dim, nq, nprobe = 64, 64, 16
    n = 2 * nlist
    cent = rng.normal(0, 1, (nlist, dim)).astype(np.float32)
    assign = rng.integers(0, nlist, n).astype(np.uint32)
    x = (cent[assign] + rng.normal(0, 0.1, (n, dim))).astype(np.float32)
    q = (cent[rng.integers(0, nlist, nq)] + rng.normal(0, 0.1, (nq, dim))).astype(np.float32)
    R = np.linalg.qr(rng.normal(size=(dim, dim)))[0].T.astype(np.float32)
    path = tmp_path / "wide.index"
    ca.build_ivf(path, (x.astype(np.float64) @ R).astype(np.float32), (cent.astype(np.float64) @ R).astype(np.float32),
                 assign, R, metric=0)
    case = Case(path, q)
    say(f"[gpu] coarse probe parity, nlist={nlist}")
    eng, _, _ = run_frozen(case, nprobe, 10)
    g = gpu_intermediates(eng, case, nprobe)
    for qi in range(nq):
        if qi % 8 == 0:  # oracle distances to every cluster, 8 queries at a time
            idx, _, _, l2 = orc.coarse_probe(g["qr"][qi:qi + 8], case.sd.centroids, case.file.nlist,
                                             case.file.metric)
            idx, l2 = {qi + r: idx[r] for r in range(idx.shape[0])}, {qi + r: l2[r] for r in range(l2.shape[0])}
        got = g["pidx"][qi]
        d_all = dict(zip(idx[qi].tolist(), l2[qi].tolist()))
        dg = np.array([d_all[c] for c in got])
        assert np.all(np.diff(dg) >= -1e-5 * (np.abs(dg).max() + 1)), qi
        kth = l2[qi][nprobe - 1]
        strict = set(idx[qi][l2[qi] < kth - 1e-5 * (abs(kth) + 1)].tolist())
        assert strict <= set(got.tolist()), qi
        assert len(set(got.tolist())) == nprobe


@pytest.mark.parametrize("case_name", CASES + CASES_WIDE)
@pytest.mark.parametrize("mfma,vanguard", [(True, 0), (False, 0), (True, 4)])
def test_popcount_estimator_bit_exact(case_name, mfma, vanguard, request):
    """ip_int and ip_res of every (vector, probe) bit-exact, the lower bound within 1e-5,
    from the scan kernels the search ran: the matrix-core one (int8 MFMA) or the popcount
    one; with vanguard pairs, the matrix-core kernel over the vanguard units of up to 16
    pairs that the vanguard lows pass scanned."""
    case = request.getfixturevalue(case_name)
    nprobe = min(8, case.file.nlist)
    vanguard = min(vanguard, nprobe - 1)
    say(f"[gpu] dense estimator parity on {case_name} nprobe={nprobe} mfma={mfma} vanguard={vanguard}")
    flags = (0 if mfma else ca.FLAG_NO_MFMA_SCAN) | \
        (ca.FLAG_GPU_SEED_FROZEN | ca.FLAG_VANGUARD_MFMA if vanguard else 0)
    eng, _, _ = run_frozen(case, nprobe, 10, extra_flags=flags, vanguard=vanguard)
    g = gpu_intermediates(eng, case, nprobe)
    maxc = case.ivf.max_cluster
    ip, ipr, low = eng.debug_dense(case.queries.shape[0], nprobe, maxc)
    qint = qint_from_planes(g["planes"][:, :8])
    qres = qint_from_planes(g["planes"][:, 8:])
    sd = case.sd
    checked = 0
    for q in range(case.queries.shape[0]):
        for p in range(nprobe):
            c = int(g["pidx"][q, p])
            s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
            want_ip = orc.ip_int_direct(sd.bits[s:s + n], qint[q])
            assert np.array_equal(ip[q, p, :n].astype(np.int64), want_ip), (q, p, c)
            want_res = orc.ip_int_direct(sd.bits[s:s + n], qres[q])
            assert np.array_equal(ipr[q, p, :n].astype(np.int64), want_res), (q, p, c)
            # the reference's bit-plane popcount restatement on the reference word layout
            words = sd.short_data[s * (sd.bits.shape[1] // 32):(s + n) * (sd.bits.shape[1] // 32)]
            words = words.reshape(-1, n).T
            planes_msb = orc.query_planes_msb(qint[q:q + 1])[0]
            assert np.array_equal(orc.ip_int_planes(np.ascontiguousarray(words), planes_msb), want_ip)
            ex = orc.exact_ip_bitwise(want_ip, g["width"][q])
            f = sd.short_factors[s:s + n]
            want_low = orc.low_dist(f[:, 0], f[:, 1], f[:, 2], g["gadd"][q, p], g["gerr"][q, p], ex, g["k1"][q])
            sc = np.abs(f[:, 0]) + abs(g["gadd"][q, p]) + np.abs(f[:, 1] * (ex + g["k1"][q])) + \
                np.abs(f[:, 2] * g["gerr"][q, p])
            assert np.all(np.abs(low[q, p, :n] - want_low) <= 1e-5 * sc)
            checked += n
    assert checked > 0


def oracle_topk_from_gpu(case, g, nprobe, topk, thresholds=None, luts=None):
    """Final top-k restated by the oracle from the GPU's query-side intermediates; with
    luts (the LUT4 tables [nq][P/4][16]) the LUT4 estimate is the bound's and refinement's
    exact_ip."""
    sd, P = case.sd, case.file.padded_dim
    qint = qint_from_planes(g["planes"][:, :8])
    qres = qint_from_planes(g["planes"][:, 8:])
    nq = case.queries.shape[0]
    out_d = np.full((nq, topk), F32_MAX, np.float32)
    out_i = np.zeros((nq, topk), np.uint32)
    cands = []
    for q in range(nq):
        items, cset = [], set()
        thr = F32_MAX if thresholds is None else thresholds[q]
        for p in range(nprobe):
            c = int(g["pidx"][q, p])
            s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
            if luts is not None:
                ex = orc.lut4_ip(cluster_words(sd, s, n), luts[q])
            else:
                ipi = orc.ip_int_direct(sd.bits[s:s + n], qint[q])
                ex = orc.exact_ip_bitwise(ipi, g["width"][q])
            f = sd.short_factors[s:s + n]
            low = orc.low_dist(f[:, 0], f[:, 1], f[:, 2], g["gadd"][q, p], g["gerr"][q, p], ex, g["k1"][q])
            keep = np.nonzero(low < thr)[0]
            gids = s + keep
            if luts is not None:
                ex2 = ex[keep]
            else:
                ipr = orc.ip_int_direct(sd.bits[gids], qres[q])
                ex2 = orc.exact_ip_two_stage(ipi[keep], ipr, g["width"][q], g["width2"][q])
            ip2 = orc.excode_ip(g["qr"][q], sd.long_codes[gids], P)
            rd = orc.refine_dist(sd.ex_factors[gids, 0], sd.ex_factors[gids, 1], g["gadd"][q, p], ex2, ip2,
                                 g["kb"][q], case.file.ex_bits)
            cset.update(int(x) for x in gids)
            items += list(zip(rd.tolist(), sd.ids[gids].tolist()))
        items.sort()
        items = [t for t in items if t[0] < thr][:topk]
        for r, (dv, pid) in enumerate(items):
            out_d[q, r], out_i[q, r] = dv, pid
        cands.append(cset)
    return out_d, out_i, cands


def cluster_words(sd, s, n):
    """Sign-code words [n][P/32] of the cluster starting at s (reference word layout)."""
    W = sd.bits.shape[1] // 32
    return np.ascontiguousarray(sd.short_data[s * W:(s + n) * W].reshape(W, n).T)


def assert_topk_equal(d, i, od, oi, rtol=1e-5):
    for q in range(d.shape[0]):
        scale = np.abs(od[q][od[q] < F32_MAX]).max() + 1 if (od[q] < F32_MAX).any() else 1
        assert np.allclose(d[q], od[q], rtol=0, atol=rtol * scale), q
        # ids equal except where neighbouring distances tie within tolerance
        for r in range(d.shape[1]):
            if i[q, r] != oi[q, r]:
                close = np.abs(od[q] - d[q, r]) <= rtol * scale
                assert i[q, r] in set(oi[q][close].tolist()), (q, r)


@pytest.mark.parametrize("case_name", CASES + CASES_WIDE)
@pytest.mark.parametrize("vanguard", [0, 3])
def test_end_to_end_frozen_infinite_thresholds(case_name, vanguard, request):
    case = request.getfixturevalue(case_name)
    nprobe, topk = min(8, case.file.nlist), 10
    say(f"[gpu] end-to-end frozen parity on {case_name} vanguard={vanguard}")
    eng, d, i = run_frozen(case, nprobe, topk, vanguard=vanguard)
    st = eng.stats()
    g = gpu_intermediates(eng, case, nprobe)
    od, oi, cands = oracle_topk_from_gpu(case, g, nprobe, topk)
    # every vector of every probed cluster is a candidate exactly once
    assert st["submitted"] == sum(len(c) for c in cands)
    assert st["refined"] == st["submitted"]
    assert_topk_equal(d, i, od, oi)


@pytest.mark.parametrize("case_name", ["golden_l2", "synth"])
def test_filter_candidate_set_with_frozen_thresholds(case_name, request):
    case = request.getfixturevalue(case_name)
    nprobe, topk = min(8, case.file.nlist), 10
    say(f"[gpu] frozen-threshold candidate count on {case_name}")
    eng, _, _ = run_frozen(case, nprobe, topk)
    g = gpu_intermediates(eng, case, nprobe)
    od, oi, _ = oracle_topk_from_gpu(case, g, nprobe, topk)
    thr = (od[:, topk - 1] * np.float32(1.02)).astype(np.float32)
    eng2, d, i = run_frozen(case, nprobe, topk, thresholds=thr)
    st = eng2.stats()
    # candidate count equals the oracle's {low < thr} up to lows within 1e-5 of thr
    _, _, low = eng2.debug_dense(case.queries.shape[0], nprobe, case.ivf.max_cluster)
    lo = hi = 0
    for q in range(case.queries.shape[0]):
        for p in range(nprobe):
            n = int(case.sd.cluster_sizes[int(g["pidx"][q, p])])
            l = low[q, p, :n].astype(np.float64)
            lo += int((l < thr[q] - 1e-5 * abs(thr[q])).sum())
            hi += int((l < thr[q] + 1e-5 * abs(thr[q])).sum())
    assert lo <= st["submitted"] <= hi
    od2, oi2, _ = oracle_topk_from_gpu(case, g, nprobe, topk, thresholds=thr)
    assert_topk_equal(d, i, od2, oi2)


@pytest.mark.parametrize("batch_q", [1, 2, 3, 4, 6, 8, 16, 64])
def test_batch_q_and_reuse_do_not_change_results(synth, batch_q):
    say(f"[gpu] batch_q={batch_q}")
    nprobe, topk = 12, 10
    _, d0, i0 = run_frozen(synth, nprobe, topk, reuse=False)
    eng, d, i = run_frozen(synth, nprobe, topk, reuse=True)
    eng.reset_buffer(synth.queries)
    d, i = eng.search(synth.queries, topk, nprobe, batch_q)
    assert np.array_equal(i, i0)
    assert np.allclose(d, d0, rtol=1e-6)


@pytest.mark.parametrize("mode", ["fused", "fused_lows", "staged", "pair", "none"])
@pytest.mark.parametrize("topk", [10, 100])
def test_live_thresholds_match_frozen_results(synth, mode, topk):
    """Default production mode (live thresholds, secondary filter, vanguard 5; the fused
    vanguard pass in one per-query kernel, with or without the lows pass before it, the
    staged pass, the per-pair seed and recovery passes, or no GPU seed thresholds) returns
    the same top-k as the exhaustive frozen search, except where refine distances tie."""
    nprobe = 16
    say(f"[gpu] live vs frozen, vanguard mode {mode}")
    _, d0, i0 = run_frozen(synth, nprobe, topk, vanguard=0)
    eng = make_engine(synth, nprobe, topk, vanguard=5, frozen=False, secondary=True,
                      gpu_seed_refine=mode != "none",
                      extra_flags={"pair": ca.FLAG_PAIR_SEEDS,
                                   "fused_lows": ca.FLAG_VANGUARD_MFMA | ca.FLAG_VANGUARD_ONE_PASS,
                                   "staged": ca.FLAG_VANGUARD_MFMA | ca.FLAG_VANGUARD_STAGED}.get(mode, 0))
    eng.reset_buffer(synth.queries)
    d, i = eng.search(synth.queries, topk, nprobe, 4)
    st = eng.stats()
    want_mode = {"fused": 2, "fused_lows": 3, "staged": 4, "pair": 1}.get(mode)
    if want_mode is not None:
        assert st["vanguard_mode"] == want_mode, st["vanguard_mode"]
    say(f"[gpu]   candidates per query {st['submitted'] / synth.queries.shape[0]:.1f}")
    assert st["submitted"] < synth.queries.shape[0] * 20000  # the filter prunes
    same = np.mean([len(set(a) & set(b)) / topk for a, b in zip(i.tolist(), i0.tolist())])
    assert same >= 0.99, same


@pytest.mark.parametrize("case_name", ["synth", "synth_ip768"])
@pytest.mark.parametrize("topk", [10, 100])
@pytest.mark.parametrize("lows", [False, True, "staged"])
def test_gpu_final_topk_matches_cpu_refinement(case_name, topk, lows, request):
    """GPU-final top-k (the GPU forms the final top-k from the refined distances it computed
    on the HBM ex-codes; nothing published to the ring) against the CPU consumer's top-k of
    the same search: distances within the rounding bound of the two evaluations, ids equal
    except where distances tie within it. Frozen thresholds in the GPU-seeded test mode, so
    both searches start from the same thresholds.

    The lower bound's error term is tripled (lower_bound_scale 3): at the reference's bound
    an estimate occasionally exceeds the vector's refined distance, and whether the fused
    pass refines such a vector depends on how far its threshold has fallen when the vector's
    turn comes, i.e. on the order its waves fill the candidate window, which differs between
    runs. With every bound valid, both searches return the exact top-k of the probed
    vectors, which the oracle's exhaustive top-k also checks."""
    case = request.getfixturevalue(case_name)
    nprobe, nq = 16, case.queries.shape[0]
    say(f"[gpu] GPU-final top-{topk} vs CPU refinement on {case_name} lows={lows}")
    flags = ca.FLAG_GPU_SEED_FROZEN | (ca.FLAG_VANGUARD_MFMA if lows else 0) | \
        (ca.FLAG_VANGUARD_ONE_PASS if lows is True else ca.FLAG_VANGUARD_STAGED if lows else 0)
    res = {}
    for final in (False, True):
        eng = make_engine(case, nprobe, topk, vanguard=5, frozen=True, extra_flags=flags, gpu_final_topk=final,
                          lower_bound_scale=3.0)
        eng.reset_buffer(case.queries)
        res[final] = eng.search(case.queries, topk, nprobe)
        st = eng.stats()
        if final:
            assert st["refined"] == 0 and st["submitted"] > 0
            g = gpu_intermediates(eng, case, nprobe)
        eng.close()
    (dc, ic), (dg, ig) = res[False], res[True]
    od, oi, _ = oracle_topk_from_gpu(case, g, nprobe, topk)
    assert_topk_equal(dg, ig, od, oi, rtol=2e-4)
    for q in range(nq):
        scale = np.abs(dc[q][dc[q] < F32_MAX]).max() + 1
        tol = 2e-4 * scale  # both sides' rounding bounds of the refined distance
        assert np.allclose(dg[q], dc[q], rtol=0, atol=tol), q
        for r in range(topk):
            if ig[q, r] != ic[q, r]:
                close = np.abs(dc[q] - dg[q, r]) <= tol
                assert ig[q, r] in set(ic[q][close].tolist()), (q, r)


def test_gpu_final_topk_rejects_unsupported_modes(synth):
    eng = make_engine(synth, 8, 10, vanguard=5, frozen=True, gpu_final_topk=True)
    eng.reset_buffer(synth.queries)
    with pytest.raises(ca.LogicError):  # frozen thresholds without the GPU-seeded test mode
        eng.search(synth.queries, 10, 8)
    eng.configure(vanguard_size=5, frozen_thresholds=False, metric=synth.file.metric, gpu_final_topk=True,
                  extra_flags=ca.FLAG_PAIR_SEEDS)
    eng.reset_buffer(synth.queries)
    with pytest.raises(ca.LogicError):  # the per-pair passes publish unrefined seeds
        eng.search(synth.queries, 10, 8)
    eng.configure(vanguard_size=0, metric=synth.file.metric, gpu_final_topk=True)
    eng.reset_buffer(synth.queries)
    with pytest.raises(ca.LogicError):  # no vanguard pass: no refined threshold for any query
        eng.search(synth.queries, 10, 8)
    eng.configure(vanguard_size=5, metric=synth.file.metric, gpu_final_topk=True)
    eng.reset_buffer(synth.queries)
    d, i = eng.search(synth.queries, 10, 8)  # live thresholds: supported
    assert np.all(d[:, 0] < F32_MAX)
    eng.close()


def test_vanguard_mode_reported(synth):
    """Which vanguard passes ran is reported: top-k above 128 in the staged pass (the
    workspace prepared for it), or the per-pair passes where the staged pass cannot run."""
    nprobe = 16
    eng = make_engine(synth, nprobe, 129, vanguard=5, frozen=False, secondary=True)
    for topk, flags, mode in [(10, 0, 2), (10, ca.FLAG_VANGUARD_MFMA | ca.FLAG_VANGUARD_ONE_PASS, 3),
                              (10, ca.FLAG_VANGUARD_MFMA, 3), (10, ca.FLAG_VANGUARD_MFMA | ca.FLAG_VANGUARD_STAGED, 4),
                              (100, ca.FLAG_VANGUARD_MFMA, 3), (100, ca.FLAG_VANGUARD_MFMA | ca.FLAG_VANGUARD_STAGED, 4),
                              (129, 0, 4), (129, ca.FLAG_NO_VANGUARD_MFMA, 1),
                              (10, ca.FLAG_PAIR_SEEDS, 1)]:
        eng.configure(vanguard_size=5, cpu_secondary_filter=True, metric=synth.file.metric, gpu_filter_timing=True,
                      extra_flags=flags, lower_bound_scale=1.0)
        eng.reset_buffer(synth.queries)
        eng.search(synth.queries, topk, nprobe)
        st = eng.stats()
        assert st["vanguard_mode"] == mode, (topk, flags, st["vanguard_mode"])
        assert all(t > 0 for t in st["phase_ms"]), st["phase_ms"]
        assert (st["vanguard_refine_ms"] > 0) == (mode == 4), st["vanguard_refine_ms"]
        assert st["vanguard_refine_bytes"] == (st["gpu_refined"] * (synth.file.padded_dim + 32) if mode == 4 else 0)
    eng.configure(vanguard_size=0, metric=synth.file.metric)
    eng.reset_buffer(synth.queries)
    eng.search(synth.queries, 10, nprobe)
    assert eng.stats()["vanguard_mode"] == 0
    eng.close()


@pytest.mark.parametrize("prefilter", [False, True])
def test_gpu_seed_thresholds_frozen_parity(synth, prefilter):
    """Per-pair vanguard passes (the reference's structure), GPU ex-code stages in their
    deterministic test mode (frozen snapshot lowered by the
    seed thresholds): seed choice and refined seed distances vs the oracle, the seeded
    threshold vs the oracle's rule and its safety, the candidate count of the far and
    recovery passes against it (with the refined pre-filter: low below the threshold and
    refined distance within the rounding bound of it), the seeds published after the
    threshold (refined distance within their bound of it), and an unchanged final top-k."""
    nprobe, topk, van = 8, 10, 3
    keep = max(topk, 20)
    say(f"[gpu] GPU seed thresholds, frozen parity, prefilter={prefilter}")
    case = synth
    nq, P = case.queries.shape[0], case.file.padded_dim
    eng = make_engine(case, nprobe, topk, vanguard=van, frozen=True,
                      extra_flags=ca.FLAG_GPU_SEED_FROZEN | ca.FLAG_PAIR_SEEDS,
                      gpu_refine_filter=prefilter)
    eng.reset_buffer(case.queries)
    d, i = eng.search(case.queries, topk, nprobe)
    st = eng.stats()
    g = gpu_intermediates(eng, case, nprobe)
    sdist = eng.debug_read(ca.DBG_SEED_DIST, (nq, van, keep), np.float32)
    thr = eng.debug_read(ca.DBG_THRESHOLDS, (nq,), np.float32)
    qint = qint_from_planes(g["planes"][:, :8])
    qres = qint_from_planes(g["planes"][:, 8:])
    sd = case.sd
    lo_cnt = hi_cnt = 0
    od = np.full((nq, topk), F32_MAX, np.float32)
    oi = np.zeros((nq, topk), np.uint32)
    for q in range(nq):
        dists, lows, errs, l1 = [], [], [], float(np.abs(g["qr"][q]).sum())
        pair_lows, seed_sets = [], []
        for p in range(nprobe):
            c = int(g["pidx"][q, p])
            s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
            ipi = orc.ip_int_direct(sd.bits[s:s + n], qint[q])
            f = sd.short_factors[s:s + n]
            low = orc.low_dist(f[:, 0], f[:, 1], f[:, 2], g["gadd"][q, p], g["gerr"][q, p],
                               orc.exact_ip_bitwise(ipi, g["width"][q]), g["k1"][q])
            pair_lows.append(low)
            if p >= van:
                seed_sets.append(None)
                continue
            seeds = orc.vanguard_seeds(low, keep, F32_MAX)
            seed_sets.append(set(seeds.tolist()))
            gids = s + seeds
            ipr = orc.ip_int_direct(sd.bits[gids], qres[q])
            ex2 = orc.exact_ip_two_stage(ipi[seeds], ipr, g["width"][q], g["width2"][q])
            ipx = orc.excode_ip(g["qr"][q], sd.long_codes[gids], P)
            fa, fr = sd.ex_factors[gids, 0], sd.ex_factors[gids, 1]
            rd = orc.refine_dist(fa, fr, g["gadd"][q, p], ex2, ipx, g["kb"][q], 7)
            err = orc.refine_error_bound(fa, fr, g["gadd"][q, p], ex2, l1, g["kb"][q], 7, P)
            got = sdist[q, p][np.isfinite(sdist[q, p])]
            assert got.size == seeds.size, (q, p)
            assert np.all(np.abs(np.sort(got) - np.sort(rd)) <= np.sort(err)[::-1][0]), (q, p)
            dists.append(rd)
            lows.append(low[seeds])
            errs.append(err)
        dists, lows, errs = np.concatenate(dists), np.concatenate(lows), np.concatenate(errs)
        want = orc.seed_threshold(dists, lows, errs, topk)
        assert want is not None
        assert abs(float(thr[q]) - float(want)) <= 2e-5 * (abs(float(want)) + 1) + float(errs.max()), q
        # safety: the topk best seeds stay strictly below the threshold, lows included
        best = np.argsort(dists, kind="stable")[:topk]
        assert np.all(dists[best] < thr[q]) and np.all(lows[best] < thr[q]), q
        # published: every seed, plus non-seeds (vanguard) and far vectors with low < thr;
        # the oracle's top-k over that candidate set is what the CPU must return
        band = 1e-5 * (abs(float(thr[q])) + 1)
        items = []
        for p in range(nprobe):
            c = int(g["pidx"][q, p])
            s = int(sd.cluster_start[c])
            low = pair_lows[p].astype(np.float64)
            mask = np.ones(low.size, bool)
            idx = None
            if seed_sets[p] is not None:
                idx = np.fromiter(seed_sets[p], np.int64, len(seed_sets[p]))
                mask[idx] = False
            # refined distance and rounding bound of every vector of the pair
            gall = s + np.arange(low.size)
            ipa = orc.ip_int_direct(sd.bits[gall], qint[q])
            ipra = orc.ip_int_direct(sd.bits[gall], qres[q])
            exa = orc.exact_ip_two_stage(ipa, ipra, g["width"][q], g["width2"][q])
            fa, fr = sd.ex_factors[gall, 0], sd.ex_factors[gall, 1]
            rda = orc.refine_dist(fa, fr, g["gadd"][q, p], exa,
                                  orc.excode_ip(g["qr"][q], sd.long_codes[gall], P), g["kb"][q], 7)
            erra = orc.refine_error_bound(fa, fr, g["gadd"][q, p], exa, l1, g["kb"][q], 7, P)
            if idx is not None:
                # seeds refined on the GPU are published when within their bound of the threshold
                lo_cnt += int((rda[idx] <= thr[q] + 0.9 * erra[idx]).sum())
                hi_cnt += int((rda[idx] <= thr[q] + 1.1 * erra[idx]).sum())
            lo_ok = low < thr[q] - band
            hi_ok = low < thr[q] + band
            if prefilter:
                lo_ok &= rda <= thr[q] + 0.9 * erra
                hi_ok &= rda <= thr[q] + 1.1 * erra
            lo_cnt += int((mask & lo_ok).sum())
            hi_cnt += int((mask & hi_ok).sum())
            # top-k over the seeds and the vectors with low below the threshold: the
            # pre-filter only drops refined distances above the threshold
            sel = np.nonzero(~mask | (low < thr[q] - band))[0]
            items += list(zip(rda[sel].tolist(), sd.ids[gall[sel]].tolist()))
        items.sort()
        for r, (dv, pid) in enumerate(items[:topk]):
            od[q, r], oi[q, r] = dv, pid
    assert lo_cnt <= st["submitted"] <= hi_cnt, (lo_cnt, st["submitted"], hi_cnt)
    assert (st["prefilter_dropped"] > 0) == prefilter
    assert_topk_equal(d, i, od, oi)
    # against the exhaustive search: seeding pruned, and only rare RaBitQ lower-bound
    # misses (low above the refined distance) differ
    ed, ei, cands = oracle_topk_from_gpu(case, g, nprobe, topk)
    assert st["submitted"] < sum(len(c) for c in cands)
    same = np.mean([len(set(a) & set(b)) / topk for a, b in zip(i.tolist(), ei.tolist())])
    say(f"[gpu]   candidates {st['submitted']} of {sum(len(c) for c in cands)}, top-k overlap {same:.4f}")
    assert same >= 0.99, same


def probed_vectors(case, g, q, nprobe):
    """Every vector of the query's probed clusters: probe rank, global index, oracle lower
    bound, refined distance (CPU formula) and its rounding bound."""
    sd, P = case.sd, case.file.padded_dim
    qint = qint_from_planes(g["planes"][q:q + 1, :8])[0]
    qres = qint_from_planes(g["planes"][q:q + 1, 8:])[0]
    l1 = float(np.abs(g["qr"][q]).sum())
    out = []
    for p in range(nprobe):
        c = int(g["pidx"][q, p])
        s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
        gid = s + np.arange(n)
        ipi = orc.ip_int_direct(sd.bits[gid], qint)
        f = sd.short_factors[gid]
        low = orc.low_dist(f[:, 0], f[:, 1], f[:, 2], g["gadd"][q, p], g["gerr"][q, p],
                           orc.exact_ip_bitwise(ipi, g["width"][q]), g["k1"][q])
        ex2 = orc.exact_ip_two_stage(ipi, orc.ip_int_direct(sd.bits[gid], qres), g["width"][q], g["width2"][q])
        fa, fr = sd.ex_factors[gid, 0], sd.ex_factors[gid, 1]
        rd = orc.refine_dist(fa, fr, g["gadd"][q, p], ex2, orc.excode_ip(g["qr"][q], sd.long_codes[gid], P),
                             g["kb"][q], 7)
        err = orc.refine_error_bound(fa, fr, g["gadd"][q, p], ex2, l1, g["kb"][q], 7, P)
        out.append((p, gid, low.astype(np.float64), rd.astype(np.float64), err.astype(np.float64)))
    return out


@pytest.mark.parametrize("case_name", ["synth", "synth_ip768"] + CASES_WIDE)
@pytest.mark.parametrize("vanguard", [5, 16])
def test_vanguard_lows_pass_matches_oracle(case_name, vanguard, request):
    """The matrix-core vanguard lows pass (vanguard units of up to 16 same-cluster pairs):
    every (vector, vanguard pair) lower bound it writes equals the oracle's Bitwise bound
    (filter_kernels.cuh:79-114) within 1e-5 of the magnitude of its terms."""
    nprobe, topk = 16, 10
    case = request.getfixturevalue(case_name)
    nq = case.queries.shape[0]
    say(f"[gpu] vanguard lows pass vs oracle, {case_name} vanguard={vanguard}")
    eng = make_engine(case, nprobe, topk, vanguard=vanguard, frozen=True,
                      extra_flags=ca.FLAG_GPU_SEED_FROZEN | ca.FLAG_VANGUARD_MFMA)
    eng.reset_buffer(case.queries)
    eng.search(case.queries, topk, nprobe)
    st = eng.stats()
    assert st["vanguard_lows_bytes"] > 0
    g = gpu_intermediates(eng, case, nprobe)
    stride = (case.ivf.max_cluster + 255) // 256 * 256
    lows = eng.debug_read(ca.DBG_VANGUARD_LOWS, (nq, vanguard, stride), np.float32)
    sd = case.sd
    qint = qint_from_planes(g["planes"][:, :8])
    checked = 0
    for q in range(nq):
        for p in range(vanguard):
            c = int(g["pidx"][q, p])
            s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
            ex = orc.exact_ip_bitwise(orc.ip_int_direct(sd.bits[s:s + n], qint[q]), g["width"][q])
            f = sd.short_factors[s:s + n]
            want = orc.low_dist(f[:, 0], f[:, 1], f[:, 2], g["gadd"][q, p], g["gerr"][q, p], ex, g["k1"][q])
            sc = np.abs(f[:, 0]) + abs(g["gadd"][q, p]) + np.abs(f[:, 1] * (ex + g["k1"][q])) + \
                np.abs(f[:, 2] * g["gerr"][q, p])
            assert np.all(np.abs(lows[q, p, :n] - want) <= 1e-5 * sc), (q, p, c)
            checked += n
    assert checked > 0
    # the lows pass reads each cluster once per unit of up to 16 of its vanguard pairs and
    # writes a 4-byte bound per (vector, vanguard pair)
    P = case.file.padded_dim
    m = np.bincount(g["pidx"][:, :vanguard].reshape(-1), minlength=case.file.nlist)
    sizes = sd.cluster_sizes.astype(np.int64)
    assert st["vanguard_lows_bytes"] == (int((-(-m // 16) * sizes).sum()) * (P // 8 + 12) +
                                         4 * int((m * sizes).sum()))
    eng.close()


@pytest.mark.parametrize("case_name", ["synth", "synth_ip768"])
@pytest.mark.parametrize("vanguard,topk", [(3, 10), (8, 10), (5, 100), (10, 100)])
@pytest.mark.parametrize("lows", [True, False, "staged"])
def test_fused_vanguard_frozen_parity(case_name, vanguard, topk, lows, request):
    """Fused per-query vanguard pass in its deterministic test mode (frozen snapshot,
    lowered by the pass): the threshold is backed by topk published vanguard vectors below
    it; the vanguard pass publishes every vector with low and refined distance below the
    threshold and nothing beyond its rounding bound; the far pass publishes exactly the
    vectors with low < threshold and refined distance within the bound; the final top-k is
    the top-k of that candidate set by the CPU consumer's distance. lows: the bounds come
    from the matrix-core lows pass, else from the per-query pass itself; "staged": after
    the lows pass, the staged pass (per-query select, grid-wide refinement, per-query
    merge and publication) instead of the one per-query kernel. Top-100 with
    vanguard 10 is the 100M configuration's mode (top-k window, held list and threshold
    over many refinement rounds)."""
    nprobe = 16
    case = request.getfixturevalue(case_name)
    nq = case.queries.shape[0]
    say(f"[gpu] fused vanguard pass, frozen parity, {case_name} vanguard={vanguard} lows={lows}")
    eng = make_engine(case, nprobe, topk, vanguard=vanguard, frozen=True,
                      extra_flags=ca.FLAG_GPU_SEED_FROZEN | (ca.FLAG_VANGUARD_MFMA if lows else ca.FLAG_NO_VANGUARD_MFMA) |
                      (ca.FLAG_VANGUARD_ONE_PASS if lows is True else ca.FLAG_VANGUARD_STAGED if lows else 0))
    eng.reset_buffer(case.queries)
    d, i = eng.search(case.queries, topk, nprobe)
    st = eng.stats()
    assert st["vanguard_mode"] == (4 if lows == "staged" else 3 if lows else 2), st["vanguard_mode"]
    g = gpu_intermediates(eng, case, nprobe)
    thr = eng.debug_read(ca.DBG_THRESHOLDS, (nq,), np.float32)
    assert st["seeded_queries"] == nq
    assert st["recovery_ms"] == 0.0
    van_lo = van_hi = far_lo = far_hi = 0
    sd = case.sd
    for q in range(nq):
        T = float(thr[q])
        assert np.isfinite(T), q
        band = 1e-5 * (abs(T) + 1)
        vecs = probed_vectors(case, g, q, nprobe)
        backing = 0
        info = {}
        for p, gid, low, rd, err in vecs:
            if p < vanguard:
                # the GPU's k best are within their rounding bound of the CPU's values, and
                # the threshold sits above d_k plus the largest such bound and above their
                # largest lower bound (+1 ulp), which the oracle's lower bound matches within
                # the band, not bit for bit
                backing += int(((rd < T) & (low < T + band)).sum())
                van_lo += int(((low < T - band) & (rd <= T + 0.9 * err)).sum())
                van_hi += int((rd <= T + 1.1 * err).sum())
            else:
                far_lo += int(((low < T - band) & (rd <= T + 0.9 * err)).sum())
                far_hi += int(((low < T + band) & (rd <= T + 1.1 * err)).sum())
            for k in range(gid.size):
                info[int(sd.ids[gid[k]])] = (p, low[k], rd[k], err[k])
        assert backing >= topk, (q, backing)
        # the returned list: oracle distances, at or below the threshold
        scale = abs(T) + 1
        for r in range(topk):
            p, low, rd, err = info[int(i[q, r])]
            assert abs(float(d[q, r]) - rd) <= 1e-5 * scale + err, (q, r)
            # every candidate passed the filter: low below the threshold, or a vanguard
            # vector refined before the threshold fell, within its bound of the threshold
            assert low < T + band or (p < vanguard and rd <= T + 1.1 * err), (q, r)
        assert float(d[q, topk - 1]) <= T + band, q
        # completeness: every vector below the threshold closer than the returned k-th
        got = set(i[q].tolist())
        kth = float(d[q, topk - 1])
        for pid, (p, low, rd, err) in info.items():
            if low < T - band and rd < kth - 1e-5 * scale - 2 * err:
                assert pid in got, (q, pid)
    produced = st["pass_produced"]
    say(f"[gpu]   vanguard published {produced[0]} in [{van_lo}, {van_hi}], far "
        f"{produced[1] - produced[0]} in [{far_lo}, {far_hi}], refined on the GPU {st['gpu_refined']}")
    assert van_lo <= produced[0] <= van_hi
    assert far_lo <= produced[1] - produced[0] <= far_hi
    assert produced[2] == produced[1]
    assert st["gpu_refined"] >= produced[0]
    # against the exhaustive search: only rare RaBitQ lower-bound misses differ
    ed, ei, cands = oracle_topk_from_gpu(case, g, nprobe, topk)
    same = np.mean([len(set(a) & set(b)) / topk for a, b in zip(i.tolist(), ei.tolist())])
    say(f"[gpu]   candidates {st['submitted']} of {sum(len(c) for c in cands)}, top-k overlap {same:.4f}")
    assert same >= 0.99, same


@pytest.mark.parametrize("case_name", ["synth", "synth_ip768"])
@pytest.mark.parametrize("topk", [10, 100])
def test_staged_vanguard_pool_overflow(case_name, topk, request, monkeypatch):
    """The staged vanguard pass with per-query regions too small for many queries: the
    queries whose seeds or candidate list do not fit are listed and run by the one-pass
    kernel afterwards; every query still gets its GPU threshold, and the top-k matches the
    staged pass with regions that fit (frozen thresholds, GPU-seeded test mode)."""
    nprobe, vanguard = 16, 5
    case = request.getfixturevalue(case_name)
    nq = case.queries.shape[0]
    flags = ca.FLAG_GPU_SEED_FROZEN | ca.FLAG_VANGUARD_MFMA | ca.FLAG_VANGUARD_STAGED
    say(f"[gpu] staged vanguard pass, pool overflow, {case_name} top-{topk}")
    eng = make_engine(case, nprobe, topk, vanguard=vanguard, frozen=True, extra_flags=flags)
    eng.reset_buffer(case.queries)
    d0, i0 = eng.search(case.queries, topk, nprobe)
    st0 = eng.stats()
    counts0 = eng.debug_read(ca.DBG_STAGED_COUNTS, (4,), np.uint64)
    eng.close()
    assert st0["vanguard_mode"] == 4
    # every query's seeds and list fit their regions: each refined vector is a seed or listed
    assert counts0[3] == 0 and counts0[0] + counts0[1] == st0["gpu_refined"], counts0
    # regions of 128 entries: top-100 seeds (at least 200) do not fit
    monkeypatch.setenv("CORA_VANGUARD_REGION_CAP", "128")
    eng = make_engine(case, nprobe, topk, vanguard=vanguard, frozen=True, extra_flags=flags)
    eng.reset_buffer(case.queries)
    d1, i1 = eng.search(case.queries, topk, nprobe)
    st1 = eng.stats()
    counts1 = eng.debug_read(ca.DBG_STAGED_COUNTS, (4,), np.uint64)
    eng.close()
    say(f"[gpu]   queries left to the one-pass kernel: {counts1[3]} of {nq}")
    if topk == 100:
        assert counts1[3] > 0, counts1
    assert st1["vanguard_mode"] == 4 and st1["seeded_queries"] == nq
    # the two passes refine the same vectors below the final threshold; they differ only on
    # the rare vector whose lower bound misses (above its refined distance)
    same = np.mean([len(set(a) & set(b)) / topk for a, b in zip(i1.tolist(), i0.tolist())])
    say(f"[gpu]   top-k overlap with the pool that fits {same:.4f}")
    assert same >= 0.99, same


@pytest.mark.parametrize("case_name", CASES)
def test_recall_against_brute_force(case_name, request):
    case = request.getfixturevalue(case_name)
    nprobe, topk = case.file.nlist if case.file.nlist <= 8 else 24, 10
    say(f"[gpu] recall on {case_name}")
    eng = make_engine(case, nprobe, topk, vanguard=5, frozen=False, secondary=True)
    d, i = eng.search_all(case.queries, topk, nprobe)
    gt = orc.brute_force_gt(case.base, case.queries, topk, case.file.metric)
    r = orc.recall_at_k(i, gt, topk)
    assert r >= 0.9, r


REF_DUMP = Path(__file__).resolve().parent.parent / "oracle" / "_ref" / "ref_dump"


@pytest.mark.skipif(not REF_DUMP.exists(), reason="oracle/_ref/ref_dump not built (needs /root/reference)")
@pytest.mark.parametrize("case_name", ["synth", "synth_ip768"])
def test_topk_and_recall_match_reference_cpu_path(case_name, request, tmp_path):
    """Final top-k ids and recall against the reference's own CPU search (rabitqlib
    IVF::search with the FastScan-hacc estimator, ivf.hpp:670-732, run by the ref_dump
    checker built from the reference sources) on the same index file, same queries and
    same nprobe; production mode (live thresholds, vanguard 5, secondary filter)."""
    from coraanns_amd.workloads import write_fbin

    synth = request.getfixturevalue(case_name)
    nprobes, topk = [4, 8, 16], 10
    say(f"[gpu] top-k vs reference IVF::search on {case_name}")
    qf = tmp_path / "q.fbin"
    write_fbin(qf, synth.queries)
    out = tmp_path / "ref"
    out.mkdir()
    subprocess.run([str(REF_DUMP), "index", str(synth.path), str(qf), str(out), str(topk)] +
                   [str(n) for n in nprobes], check=True, capture_output=True, timeout=300)
    ref_ids = np.fromfile(out / "search_ids.bin", np.uint32).reshape(len(nprobes), -1, topk)
    gt = orc.brute_force_gt(synth.base, synth.queries, topk, synth.file.metric)
    eng = make_engine(synth, max(nprobes), topk, vanguard=5, frozen=False, secondary=True)
    for li, nprobe in enumerate(nprobes):
        _, ids = eng.search_all(synth.queries, topk, nprobe)
        agree = np.mean([len(set(a) & set(b)) / topk for a, b in zip(ids.tolist(), ref_ids[li].tolist())])
        r_gpu = orc.recall_at_k(ids, gt, topk)
        r_ref = orc.recall_at_k(ref_ids[li], gt, topk)
        say(f"[gpu]   nprobe={nprobe}: id agreement {agree:.4f}, recall gpu {r_gpu:.4f} ref {r_ref:.4f}")
        assert agree >= 0.98, (nprobe, agree)
        assert abs(r_gpu - r_ref) <= 0.01, (nprobe, r_gpu, r_ref)


def _mixture_index(tmp_path, n, dim, n_centers, nlist, nq, metric, sd, seed):
    """A Gaussian-mixture index of the benchmark configurations' kind, built here (GPU
    k-means and assignment, host RaBitQ builder) with exact ground truth."""
    from coraanns_amd import workloads as wl

    rng = np.random.default_rng(seed)
    centers = rng.normal(0, 1, (n_centers, dim)).astype(np.float32)

    def draw(m):
        x = centers[rng.integers(0, n_centers, m)] + rng.normal(0, sd, (m, dim)).astype(np.float32)
        if metric == 1:
            x /= np.linalg.norm(x, axis=1, keepdims=True)
        return np.ascontiguousarray(x, np.float32)

    x, q = draw(n), draw(nq)
    sample = x[rng.choice(n, min(n, 256 * nlist), replace=False)]
    cent = ca.gpu_kmeans(sample, nlist, 20, seed)
    assign = ca.gpu_assign(x, cent)
    R = wl.rotation(dim, (dim + 63) // 64 * 64, seed + 1)
    path = tmp_path / "mix.index"
    ca.build_ivf(path, ca.gpu_rotate(x, R), (cent.astype(np.float64) @ R.astype(np.float64)).astype(np.float32),
                 assign, R, metric=metric)
    gt = wl.ground_truth(x, q, 10, metric)
    return path, q, gt


@pytest.mark.skipif(not REF_DUMP.exists(), reason="oracle/_ref/ref_dump not built (needs /root/reference)")
@pytest.mark.parametrize("n,dim,n_centers,nlist,nq,metric,sd", [
    (200_000, 128, 256, 256, 2000, 0, 0.3),   # config 2's kind (1M x 128 L2) at a fifth of its size
    (100_000, 768, 512, 128, 1000, 1, 0.5),   # config 4's kind (20M x 768 IP, unit norm)
])
def test_recall_at_least_reference_cpu_path(n, dim, n_centers, nlist, nq, metric, sd, tmp_path):
    """Production mode (live thresholds, vanguard 5, secondary filter, the default lower-bound
    scale): recall@10 at least the reference CPU search's (rabitqlib IVF::search, FastScan
    hacc, ivf.hpp:670-732, run by ref_dump from the reference sources) minus 0.001, at every
    nprobe, on the same index file and queries. With the reference Bitwise bound (scale 1)
    the GPU filter tests every vector against a nearly final threshold, where the CPU
    search tests early vectors against a looser running one, and recall trails by ~0.004."""
    from coraanns_amd.workloads import write_fbin

    say(f"[gpu] recall vs reference CPU path, {n} x {dim} {'IP' if metric else 'L2'}, nlist {nlist}")
    path, q, gt = _mixture_index(tmp_path, n, dim, n_centers, nlist, nq, metric, sd, 11 + dim)
    nprobes, topk = [4, 8, 16], 10
    qf = tmp_path / "q.fbin"
    write_fbin(qf, q)
    out = tmp_path / "ref"
    out.mkdir()
    subprocess.run([str(REF_DUMP), "index", str(path), str(qf), str(out), str(topk)] +
                   [str(v) for v in nprobes], check=True, capture_output=True, timeout=600)
    ref_ids = np.fromfile(out / "search_ids.bin", np.uint32).reshape(len(nprobes), -1, topk)
    ivf = ca.IvfIndex(path)
    eng = ca.HybridIndex(0, vanguard_size=5, cpu_secondary_filter=True, metric=metric)
    eng.load_ivf(ivf)
    eng.prepare_workspace(nq, topk, max(nprobes))
    for li, nprobe in enumerate(nprobes):
        eng.reset_buffer(q)
        _, ids = eng.search(q, topk, nprobe)
        r_gpu = orc.recall_at_k(ids, gt, topk)
        r_ref = orc.recall_at_k(ref_ids[li], gt, topk)
        agree = np.mean([len(set(a) & set(b)) / topk for a, b in zip(ids.tolist(), ref_ids[li].tolist())])
        say(f"[gpu]   nprobe={nprobe}: recall gpu {r_gpu:.4f} ref {r_ref:.4f}, id agreement {agree:.4f}")
        assert r_gpu >= r_ref - 0.001, (nprobe, r_gpu, r_ref)
        # the two top-k lists differ only where one of them misses a true neighbour (measured:
        # 0.9975 at 200k x 128 against recalls 0.9865 / 0.9848; 0.9522 at 100k x 768, where the
        # reference's FastScan search has recall 0.9357 against 0.9823)
        assert agree >= min(r_gpu, r_ref) - 0.005, (nprobe, agree, r_gpu, r_ref)
    eng.close()


@pytest.mark.parametrize("dim,metric,nlist", [(128, 0, 16384), (768, 1, 16384), (128, 0, 40000)])
def test_pair_schedule_and_scan_bytes_large_nlist(dim, metric, nlist, tmp_path):
    """Pair scheduling at nlist 16,384 (the 10M/20M configurations' nlist: LDS bucket
    histograms) and 40,000 (global-atomic bucket counting, a bucket scan over 79 workgroups)
    and the scan statistics the benchmark's roofline is computed from: the scheduled pairs
    are exactly the probe lists, vanguard pairs first; the far-pass bytes are sum over
    clusters of ceil(m_c / unit) * n_c * (P/8 + 12), the vanguard bytes ceil(m_c / 16) * n_c *
    (P/8 + 12) + 4 m_c n_c for the vanguard lows pass and 4 m_c n_c plus the refined vectors'
    (P + 8) for the per-query vanguard pass. A second, smaller search on the same engine checks that
    the bucket counts and cursors the first one left behind were cleared."""
    rng = np.random.default_rng(dim + nlist)
    n, nq, nprobe, vanguard = 40000, 192, 32, 5
    cent = rng.normal(0, 1, (nlist, dim)).astype(np.float32)
    assign = rng.integers(0, nlist, n).astype(np.uint32)
    x = (cent[assign] + rng.normal(0, 0.3, (n, dim))).astype(np.float32)
    q = (cent[rng.integers(0, nlist, nq)] + rng.normal(0, 0.3, (nq, dim))).astype(np.float32)
    if metric == 1:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        q /= np.linalg.norm(q, axis=1, keepdims=True)
    R = np.linalg.qr(rng.normal(size=(dim, dim)))[0].T.astype(np.float32)
    path = tmp_path / "sched.index"
    ca.build_ivf(path, (x.astype(np.float64) @ R).astype(np.float32),
                 (cent.astype(np.float64) @ R).astype(np.float32), assign, R, metric=metric)
    case = Case(path, q)
    P = case.file.padded_dim
    sizes = case.sd.cluster_sizes.astype(np.int64)
    bpv = P // 8 + 12
    unit = 16 if (P // 32) in (2, 4, 6, 8, 16, 24, 32) else 4  # matrix-core far scan, else batch-q 4
    eng = make_engine(case, nprobe, 10, vanguard=vanguard, frozen=False, secondary=True,
                      gpu_seed_refine=True, gpu_refine_filter=True, extra_flags=ca.FLAG_VANGUARD_MFMA)
    for nqs in (nq, 77):
        say(f"[gpu] pair schedule + scan bytes, nlist={nlist} P={P} nq={nqs}")
        qs = np.ascontiguousarray(q[:nqs])
        eng.reset_buffer(qs)
        eng.search(qs, 10, nprobe)
        st = eng.stats()
        pidx = eng.debug_read(ca.DBG_PROBE_IDX, (nqs, nprobe), np.int32)
        pairs = eng.debug_read(ca.DBG_PAIRS, (nqs * nprobe, 3), np.int32)
        assert pidx.min() >= 0 and pidx.max() < nlist
        # the scheduled pairs are the probe lists (as a multiset), vanguard pairs first
        want = np.stack([pidx.reshape(-1), np.repeat(np.arange(nqs), nprobe), np.tile(np.arange(nprobe), nqs)], 1)
        key = lambda a: np.lexsort((a[:, 2], a[:, 1], a[:, 0]))
        assert np.array_equal(pairs[key(pairs)], want[key(want)])
        nvan = nqs * vanguard
        assert np.all(pairs[:nvan, 2] < vanguard) and np.all(pairs[nvan:, 2] >= vanguard)
        assert np.all(np.diff(pairs[nvan:, 0]) >= 0)  # far pairs grouped by cluster
        far_m = np.bincount(pidx[:, vanguard:].reshape(-1), minlength=nlist)
        van_m = np.bincount(pidx[:, :vanguard].reshape(-1), minlength=nlist)
        assert st["scan_vectors"] == int((far_m * sizes).sum())
        assert st["scan_bytes"] == int((-(-far_m // unit) * sizes).sum()) * bpv
        # the vanguard lows pass reads each cluster once per unit of up to 16 vanguard pairs
        # and writes one 4-byte bound per (vector, pair), which the per-query pass streams,
        # plus the refined vectors' sign code, ex-code and ex-factors
        assert st["vanguard_lows_bytes"] == (int((-(-van_m // 16) * sizes).sum()) * bpv +
                                             4 * int((van_m * sizes).sum()))
        assert st["vanguard_bytes"] == 4 * int((van_m * sizes).sum()) + st["gpu_refined"] * (P + 8)
    eng.close()


# ---------------------------------------------------------------------------------------
# LUT4 estimator (HybridIndex::set_ip_kernel_type(Lut4Bit), CORA_FLAG_LUT4)
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("case_name", CASES + CASES_WIDE)
@pytest.mark.parametrize("vanguard", [0, 3])
def test_lut4_tables_and_estimator_bit_exact(case_name, vanguard, request):
    """The FP16 nibble tables equal the oracle's (precompute_lut_fp16_kernel,
    query_kernels.cuh:199-221) from the GPU's rotated queries bit for bit; the LUT4 estimate
    of every probed vector (filter_kernels.cuh:655-708) likewise; the lower bound within
    1e-5 of the oracle's expression on it."""
    case = request.getfixturevalue(case_name)
    nprobe = min(8, case.file.nlist)
    vanguard = min(vanguard, nprobe - 1)
    nq, P = case.queries.shape[0], case.file.padded_dim
    say(f"[gpu] LUT4 dense parity on {case_name} nprobe={nprobe} vanguard={vanguard}")
    eng, _, _ = run_frozen(case, nprobe, 10, vanguard=vanguard, ip_kernel_type="lut4")
    g = gpu_intermediates(eng, case, nprobe)
    lut = eng.debug_read(ca.DBG_LUT, (nq, P // 4, 16), np.uint16)
    want = orc.lut4_table(g["qr"])
    assert np.array_equal(lut, want.view(np.uint16))
    ip, ipr, low = eng.debug_dense(nq, nprobe, case.ivf.max_cluster)
    ipf = ip.view(np.float32)
    sd = case.sd
    checked = 0
    for q in range(nq):
        for p in range(nprobe):
            c = int(g["pidx"][q, p])
            s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
            w = orc.lut4_ip(cluster_words(sd, s, n), want[q])
            assert np.array_equal(ipf[q, p, :n].view(np.uint32), w.view(np.uint32)), (q, p, c)
            assert not ipr[q, p, :n].any()
            f = sd.short_factors[s:s + n]
            want_low = orc.low_dist(f[:, 0], f[:, 1], f[:, 2], g["gadd"][q, p], g["gerr"][q, p], w, g["k1"][q])
            sc = np.abs(f[:, 0]) + abs(g["gadd"][q, p]) + np.abs(f[:, 1] * (w + g["k1"][q])) + \
                np.abs(f[:, 2] * g["gerr"][q, p])
            assert np.all(np.abs(low[q, p, :n] - want_low) <= 1e-5 * sc)
            checked += n
    assert checked > 0
    eng.close()


@pytest.mark.parametrize("case_name", CASES)
@pytest.mark.parametrize("vanguard", [0, 3])
def test_lut4_end_to_end_frozen(case_name, vanguard, request):
    """LUT4 search with frozen infinite thresholds: every probed vector is a candidate once
    (seed and recovery passes with vanguard pairs), and the final top-k equals the oracle's
    with the LUT4 estimate as refinement's exact_ip."""
    case = request.getfixturevalue(case_name)
    nprobe, topk = min(8, case.file.nlist), 10
    vanguard = min(vanguard, nprobe - 1)
    nq, P = case.queries.shape[0], case.file.padded_dim
    say(f"[gpu] LUT4 end-to-end frozen parity on {case_name} vanguard={vanguard}")
    eng, d, i = run_frozen(case, nprobe, topk, vanguard=vanguard, ip_kernel_type="lut4")
    st = eng.stats()
    g = gpu_intermediates(eng, case, nprobe)
    luts = eng.debug_read(ca.DBG_LUT, (nq, P // 4, 16), np.uint16).view(np.float16)
    od, oi, cands = oracle_topk_from_gpu(case, g, nprobe, topk, luts=luts)
    assert st["submitted"] == sum(len(c) for c in cands)
    assert st["refined"] == st["submitted"]
    assert_topk_equal(d, i, od, oi)
    eng.close()


@pytest.mark.parametrize("case_name", ["synth", "synth_ip768"])
@pytest.mark.parametrize("topk", [10, 100])
def test_lut4_live_thresholds_match_frozen(case_name, topk, request):
    """LUT4 in the production setting (live thresholds, secondary filter, vanguard 5, the GPU
    seed thresholds and refined pre-filter on the HBM ex-codes, batch-q 4) returns the top-k
    of the exhaustive frozen LUT4 search, and GPU-final top-k is refused for it. At P = 768
    the matrix-core lows pass and far scan (lowered Bitwise bounds, exact LUT4 bounds of the
    survivors) and the staged vanguard pass run it; at P = 128 the per-pair passes."""
    case = request.getfixturevalue(case_name)
    nprobe = 16
    say(f"[gpu] LUT4 live vs frozen on {case_name} top-{topk}")
    _, d0, i0 = run_frozen(case, nprobe, topk, vanguard=0, ip_kernel_type="lut4")
    eng = make_engine(case, nprobe, topk, vanguard=5, frozen=False, secondary=True, ip_kernel_type="lut4")
    eng.reset_buffer(case.queries)
    d, i = eng.search(case.queries, topk, nprobe, 4)
    st = eng.stats()
    assert st["vanguard_mode"] == (4 if case.file.padded_dim >= 512 else 1), st["vanguard_mode"]
    assert st["submitted"] < case.queries.shape[0] * case.file.num  # the filter prunes
    same = np.mean([len(set(a) & set(b)) / topk for a, b in zip(i.tolist(), i0.tolist())])
    assert same >= 0.99, same
    eng.configure(vanguard_size=5, metric=case.file.metric, gpu_final_topk=True, ip_kernel_type="lut4")
    eng.reset_buffer(case.queries)
    with pytest.raises(ca.LogicError):
        eng.search(case.queries, topk, nprobe)
    eng.close()


def probed_vectors_lut(case, g, q, nprobe, lut):
    """probed_vectors with the LUT4 estimate (the query's FP16 tables lut) as the bound's and
    refinement's exact_ip."""
    sd, P = case.sd, case.file.padded_dim
    l1 = float(np.abs(g["qr"][q]).sum())
    out = []
    for p in range(nprobe):
        c = int(g["pidx"][q, p])
        s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
        gid = s + np.arange(n)
        ex = orc.lut4_ip(cluster_words(sd, s, n), lut)
        f = sd.short_factors[gid]
        low = orc.low_dist(f[:, 0], f[:, 1], f[:, 2], g["gadd"][q, p], g["gerr"][q, p], ex, g["k1"][q])
        fa, fr = sd.ex_factors[gid, 0], sd.ex_factors[gid, 1]
        rd = orc.refine_dist(fa, fr, g["gadd"][q, p], ex, orc.excode_ip(g["qr"][q], sd.long_codes[gid], P),
                             g["kb"][q], 7)
        err = orc.refine_error_bound(fa, fr, g["gadd"][q, p], ex, l1, g["kb"][q], 7, P)
        out.append((p, gid, low.astype(np.float64), rd.astype(np.float64), err.astype(np.float64)))
    return out


@pytest.mark.parametrize("topk", [10, 100])
def test_lut4_staged_vanguard_frozen_parity(topk, synth_ip768):
    """LUT4 on the matrix cores with the staged vanguard pass, in its deterministic test mode
    (frozen snapshot lowered by the pass; vanguard 5): the lows pass writes Bitwise bounds
    lowered by the query's LUT4 margin, the staged pass refines with the LUT4 estimate and
    evaluates each refined vector's LUT4 bound, and the far scan publishes exactly the vectors
    whose LUT4 bound lies below the threshold (within the refined pre-filter's rounding bound),
    all against the oracle's LUT4 restatement (filter_kernels.cuh:655-708): the threshold is
    backed by topk vanguard vectors below it, the publication counts lie in the oracle's bands,
    and the final top-k are oracle distances at or below the threshold, complete below it, and
    the exhaustive LUT4 top-k of the probed clusters."""
    case, nprobe, vanguard = synth_ip768, 16, 5
    nq, P = case.queries.shape[0], case.file.padded_dim
    say(f"[gpu] LUT4 staged vanguard pass, frozen parity, top-{topk}")
    eng = make_engine(case, nprobe, topk, vanguard=vanguard, frozen=True, ip_kernel_type="lut4",
                      extra_flags=ca.FLAG_GPU_SEED_FROZEN)
    eng.reset_buffer(case.queries)
    d, i = eng.search(case.queries, topk, nprobe)
    st = eng.stats()
    assert st["vanguard_mode"] == 4, st["vanguard_mode"]
    g = gpu_intermediates(eng, case, nprobe)
    luts = eng.debug_read(ca.DBG_LUT, (nq, P // 4, 16), np.uint16).view(np.float16)
    thr = eng.debug_read(ca.DBG_THRESHOLDS, (nq,), np.float32)
    assert st["seeded_queries"] == nq
    van_lo = van_hi = far_lo = far_hi = 0
    sd = case.sd
    for q in range(nq):
        T = float(thr[q])
        assert np.isfinite(T), q
        band = 1e-5 * (abs(T) + 1)
        backing = 0
        info = {}
        for p, gid, low, rd, err in probed_vectors_lut(case, g, q, nprobe, luts[q]):
            if p < vanguard:
                backing += int(((rd < T) & (low < T + band)).sum())
                van_lo += int(((low < T - band) & (rd <= T + 0.9 * err)).sum())
                van_hi += int((rd <= T + 1.1 * err).sum())
            else:
                far_lo += int(((low < T - band) & (rd <= T + 0.9 * err)).sum())
                far_hi += int(((low < T + band) & (rd <= T + 1.1 * err)).sum())
            for k in range(gid.size):
                info[int(sd.ids[gid[k]])] = (p, low[k], rd[k], err[k])
        assert backing >= topk, (q, backing)
        scale = abs(T) + 1
        for r in range(topk):
            p, low, rd, err = info[int(i[q, r])]
            assert abs(float(d[q, r]) - rd) <= 1e-5 * scale + err, (q, r)
            assert low < T + band or (p < vanguard and rd <= T + 1.1 * err), (q, r)
        assert float(d[q, topk - 1]) <= T + band, q
        got = set(i[q].tolist())
        kth = float(d[q, topk - 1])
        for pid, (p, low, rd, err) in info.items():
            if low < T - band and rd < kth - 1e-5 * scale - 2 * err:
                assert pid in got, (q, pid)
    produced = st["pass_produced"]
    say(f"[gpu]   vanguard published {produced[0]} in [{van_lo}, {van_hi}], far "
        f"{produced[1] - produced[0]} in [{far_lo}, {far_hi}], refined on the GPU {st['gpu_refined']}")
    assert van_lo <= produced[0] <= van_hi
    assert far_lo <= produced[1] - produced[0] <= far_hi
    assert produced[2] == produced[1]
    ed, ei, _ = oracle_topk_from_gpu(case, g, nprobe, topk, luts=luts)
    same = np.mean([len(set(a) & set(b)) / topk for a, b in zip(i.tolist(), ei.tolist())])
    say(f"[gpu]   top-k overlap with the exhaustive LUT4 search {same:.4f}")
    assert same >= 0.99, same
    eng.close()


@pytest.mark.parametrize("case_name", ["synth", "synth_ip768"])
@pytest.mark.parametrize("vanguard,topk", [(16, 513), (5, 1024), (16, 1024)])
def test_high_k_staged_vanguard(case_name, vanguard, topk, request):
    """Top-k above the one-pass kernel's limit (128) with the GPU ex-code stages on: the
    staged pass serves it (mode 4). GPU-final top-k in the GPU-seeded frozen mode (bound
    scale 3, every bound valid) against the oracle's exhaustive top-k of the probed vectors;
    the default live-threshold search with the CPU consumer against the exhaustive frozen
    search without vanguard pairs."""
    case = request.getfixturevalue(case_name)
    nprobe, nq = 16, case.queries.shape[0]
    say(f"[gpu] high-k staged on {case_name} vanguard={vanguard} topk={topk}")
    eng = make_engine(case, nprobe, topk, vanguard=vanguard, frozen=True, extra_flags=ca.FLAG_GPU_SEED_FROZEN,
                      gpu_final_topk=True, lower_bound_scale=3.0)
    eng.reset_buffer(case.queries)
    dg, ig = eng.search(case.queries, topk, nprobe)
    st = eng.stats()
    assert st["vanguard_mode"] == 4, st["vanguard_mode"]
    assert st["refined"] == 0 and st["submitted"] > 0
    g = gpu_intermediates(eng, case, nprobe)
    eng.close()
    od, oi, _ = oracle_topk_from_gpu(case, g, nprobe, topk)
    assert_topk_equal(dg, ig, od, oi, rtol=2e-4)
    _, d0, i0 = run_frozen(case, nprobe, topk, vanguard=0)
    eng = make_engine(case, nprobe, topk, vanguard=vanguard, frozen=False, secondary=True)
    eng.reset_buffer(case.queries)
    d, i = eng.search(case.queries, topk, nprobe, 4)
    st = eng.stats()
    eng.close()
    assert st["vanguard_mode"] == 4, st["vanguard_mode"]
    if vanguard == nprobe:  # every probed vector is a vanguard vector: at least topk of them
        assert st["seeded_queries"] == nq, st["seeded_queries"]
    same = np.mean([len(set(a) & set(b)) / topk for a, b in zip(i.tolist(), i0.tolist())])
    assert same >= 0.99, same
