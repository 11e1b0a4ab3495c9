"""CPU tests of the native host library (libcoraanns) and the C-ABI exports.

No GPU is touched: the libraries are loaded and only host entry points are called.
"""
import os
import re
import shutil
import subprocess
import sys

import numpy as np
import pytest

import cora_oracle as orc
import coraanns_amd as ca
from conftest import GOLDEN, REPO, read_fbin


def declared(header):
    text = (REPO / "include" / header).read_text()
    return sorted(set(re.findall(r"\b(cora_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header,which", [("cora_gpu.h", 0), ("cora_host.h", 1)])
def test_library_exports_every_declared_symbol(header, which):
    lib = ca.libs()[which]
    names = declared(header)
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares a signature for every exported entry point
    sigs = ca.GPU_SIGNATURES if which == 0 else ca.HOST_SIGNATURES
    assert set(names) <= set(sigs), set(names) - set(sigs)


@pytest.mark.parametrize("name", ["l2_d96", "ip_d64"])
def test_ivf_reader_matches_reference_searchdata(golden, name):
    ref = golden(f"{name}/ref")
    ivf = ca.IvfIndex(GOLDEN / name / "ivf.index")
    n, dim, P, nl, ex, metric = (int(x) for x in ref["meta"])
    assert (ivf.num, ivf.dim, ivf.padded_dim, ivf.nlist, ivf.ex_bits, ivf.metric) == (n, dim, P, nl, ex, metric)
    assert np.array_equal(ivf.short_data, ref["short_data"].reshape(-1))
    assert np.array_equal(ivf.short_factors.view(np.uint32), ref["short_factors"].view(np.uint32))
    assert np.array_equal(ivf.long_codes, ref["long_codes"])
    assert np.array_equal(ivf.ex_factors.view(np.uint32), ref["ex_factors"].view(np.uint32))
    assert np.array_equal(ivf.ids, ref["ids"])
    assert np.array_equal(ivf.cluster_sizes, ref["cluster_sizes"])
    assert np.array_equal(ivf.centroids, ref["centroids"])
    assert np.array_equal(ivf.rotator, ref["rotator"])
    assert ivf.max_cluster == int(ref["cluster_sizes"].max())


def test_ivf_reader_rejects_truncated_file(tmp_path):
    raw = (GOLDEN / "l2_d96" / "ivf.index").read_bytes()
    bad = tmp_path / "bad.index"
    bad.write_bytes(raw[:-100])
    with pytest.raises(ca.EngineError):
        ca.IvfIndex(bad)


@pytest.mark.parametrize("metric,tag", [(0, "l2"), (1, "ip")])
def test_quantizer_matches_reference(golden, metric, tag):
    g = golden("quant_d128")
    rows = np.fromfile(GOLDEN / "quant_d128" / "rows.f32", dtype=np.float32).reshape(-1, 128)
    bits, f1, ex, f2 = ca.quantize_rows(rows[1:], rows[0], metric=metric)
    assert np.array_equal(bits.astype(np.int32), g[f"bits_{tag}"])
    # ex-codes come from a rescale search over |o|/||o||; reductions are summed in a
    # different order than the reference's Eigen code, so allow rare last-step flips
    mism = (ex != g[f"excode_{tag}"]).mean()
    assert mism <= 0.002, mism
    assert np.allclose(f1, g[f"f1_{tag}"], rtol=1e-5, atol=1e-5 * np.abs(g[f"f1_{tag}"]).max())
    assert np.allclose(f2[:, 0], g[f"f2_{tag}"][:, 0], rtol=1e-4, atol=1e-4 * np.abs(g[f"f2_{tag}"][:, 0]).max())
    assert np.allclose(f2[:, 1], g[f"f2_{tag}"][:, 1], rtol=1e-4)


def test_excode_ip7_matches_reference_and_oracle(golden):
    g = golden("quant_d128")
    q = np.fromfile(GOLDEN / "quant_d128" / "rows.f32", dtype=np.float32)[:128]
    ip = ca.excode_ip7(q, g["packed7"])
    sc = np.abs(q).sum() * 127
    assert np.all(np.abs(ip - g["ip_fxu7"]) <= 1e-6 * sc)
    rng = np.random.default_rng(3)
    for P in (64, 128, 768):
        codes = rng.integers(0, 128, (20, P)).astype(np.uint8)
        packed = orc.pack_excode7(codes)
        qq = rng.normal(0, 1, P).astype(np.float32)
        got = ca.excode_ip7(qq, packed)
        want = codes.astype(np.float64) @ qq.astype(np.float64)
        assert np.all(np.abs(got - want) <= 1e-5 * np.abs(qq).sum() * 127)


def _random_rotation(dim, P, rng):
    a = rng.normal(size=(P, P))
    q, _ = np.linalg.qr(a)
    return q.T[:dim].astype(np.float32)


def _build_small(tmp_path, metric=0, n=700, dim=40, nl=5, seed=0):
    rng = np.random.default_rng(seed)
    P = (dim + 63) // 64 * 64
    centers = rng.normal(0, 2, (nl, dim))
    x = (centers[rng.integers(0, nl, n)] + rng.normal(0, 1, (n, dim))).astype(np.float32)
    if metric == 1:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
    d = ((x[:, None, :] - centers[None]) ** 2).sum(2)
    assign = d.argmin(1).astype(np.uint32)
    cent = np.stack([x[assign == c].mean(0) if (assign == c).any() else centers[c] for c in range(nl)])
    R = _random_rotation(dim, P, rng)
    xr = (x.astype(np.float64) @ R).astype(np.float32)
    cr = (cent.astype(np.float64) @ R).astype(np.float32)
    path = tmp_path / f"built_{metric}.index"
    ca.build_ivf(path, xr, cr, assign, R, metric=metric, threads=4)
    return path, x, xr, cr, assign, R


@pytest.mark.parametrize("metric", [0, 1])
def test_builder_writes_reference_format(tmp_path, metric):
    path, x, xr, cr, assign, R = _build_small(tmp_path, metric)
    f = orc.read_ivf(path)
    sd = orc.search_data(f)
    assert f.metric == metric and f.ex_bits == 7 and f.num == x.shape[0]
    assert np.array_equal(f.cluster_sizes, np.bincount(assign, minlength=cr.shape[0]).astype(np.uint64))
    # ids are grouped by cluster in ascending order within a cluster
    for c in range(f.nlist):
        s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
        ids = f.ids[s:s + n]
        assert np.all(assign[ids] == c) and np.all(np.diff(ids.astype(np.int64)) > 0)
        # sign bits / factors / ex-codes equal the quantizer's output for those rows
        bits, f1, ex, f2 = ca.quantize_rows(xr[ids], cr[c], metric=metric)
        assert np.array_equal(sd.bits[s:s + n], bits)
        assert np.array_equal(sd.short_factors[s:s + n].view(np.uint32), f1.view(np.uint32))
        assert np.array_equal(orc.unpack_excode7(sd.long_codes[s:s + n], f.padded_dim), ex)
        assert np.array_equal(sd.ex_factors[s:s + n].view(np.uint32), f2.view(np.uint32))
    # the C++ reader agrees with the oracle reader
    ivf = ca.IvfIndex(path)
    assert np.array_equal(ivf.short_data, sd.short_data)
    assert np.array_equal(ivf.long_codes, sd.long_codes)


@pytest.mark.skipif(not (REPO / "oracle" / "_ref" / "ref_dump").exists(),
                    reason="reference CPU path not built (make -C oracle ref)")
def test_reference_code_reads_built_index(tmp_path):
    """The reference's own IVF::load + SearchData read an index written by this builder."""
    path, x, xr, cr, assign, R = _build_small(tmp_path, 0, n=500, dim=96, nl=4)
    q = x[:6]
    qf = tmp_path / "q.fbin"
    with open(qf, "wb") as fh:
        fh.write(np.array(q.shape, np.uint32).tobytes())
        fh.write(q.astype(np.float32).tobytes())
    out = tmp_path / "dump"
    out.mkdir()
    subprocess.run([str(REPO / "oracle" / "_ref" / "ref_dump"), "index", str(path), str(qf), str(out),
                    "5", "4"], check=True, capture_output=True)
    from conftest import load_golden
    import conftest
    old = conftest.GOLDEN
    try:
        conftest.GOLDEN = tmp_path
        ref = load_golden("dump")
    finally:
        conftest.GOLDEN = old
    ivf = ca.IvfIndex(path)
    assert np.array_equal(ivf.short_data, ref["short_data"].reshape(-1))
    assert np.array_equal(ivf.long_codes, ref["long_codes"])
    # the reference CPU search finds the query vectors themselves (queries are base rows)
    assert np.all(ref["search_ids"][0][:, 0] == np.arange(6))


@pytest.mark.parametrize("capacity,spill,producers,consumers", [
    (8192, 262144, 4, 4),
    (262144, 262144, 2, 1),
    (1024, 1 << 16, 8, 16),
    (64, 1 << 16, 4, 4),   # forced spill and refill through the drain
])
@pytest.mark.parametrize("secondary", [False, True])
def test_ring_protocol_cpu_emulated_producer(capacity, spill, producers, consumers, secondary):
    nq, per, k = 5, 3000, 50
    t, d, i = ca.ring_test(capacity, spill, producers, consumers, nq, per, k, secondary)
    assert t.overflow == 0
    assert t.submitted == nq * per
    if not secondary:
        assert t.refined == nq * per
    for q in range(nq):
        r = np.arange(per)
        dist = (0.01 * ((r * 7919 + q * 31) % per) + 1.0).astype(np.float32)
        order = np.argsort(dist, kind="stable")[:k]
        assert np.all(np.diff(d[q]) >= 0)  # ascending, as the consumer keeps it
        assert np.allclose(d[q], dist[order])
        assert set(int(v) for v in i[q]) == set(int(q * per + v) for v in order)
    if capacity < nq * per:
        assert t.spilled > 0 or capacity >= 8192


def test_ring_protocol_overflow_is_reported_without_hang():
    t, d, i = ca.ring_test(32, 0, 2, 2, 5, 1000, 10, False)
    assert t.overflow == 1


def test_ring_protocol_zero_candidates():
    t, d, i = ca.ring_test(64, 64, 2, 2, 3, 0, 4, False)
    assert t.submitted == 0 and t.overflow == 0
    assert np.all(d == np.finfo(np.float32).max) and np.all(i == 0)


CPP_TESTS = ["release_tracker_test.cpp", "parameters_test.cpp", "recall_evaluator_test.cpp", "huge_pages_test.cpp"]


@pytest.mark.parametrize("src", CPP_TESTS)
def test_cpp_unit(tmp_path, src):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / src.replace(".cpp", "")
    subprocess.run([gxx, "-O1", "-std=c++17", "-pthread", f"-I{REPO / 'include'}",
                    str(REPO / "tests" / "cpp" / src), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout


def test_excode_ip7_avx2_and_dispatched_paths_agree(golden, tmp_path):
    """The CPU refinement's inner product gives the same values on its AVX-512 path (when
    the CPU has it) and its AVX2 path (CORA_CPU_ISA=avx2, checked in a child process)."""
    g = golden("quant_d128")
    packed = np.ascontiguousarray(g["packed7"])
    rng = np.random.default_rng(31)
    q = rng.normal(0, 1, 128).astype(np.float32)
    np.save(tmp_path / "q.npy", q)
    np.save(tmp_path / "packed.npy", packed)
    code = (
        "import sys, numpy as np; sys.path.insert(0, sys.argv[1]); import coraanns_amd as ca; "
        "q = np.load(sys.argv[2]); p = np.load(sys.argv[3]); "
        "np.save(sys.argv[4], ca.excode_ip7(q, p)); print(ca.cpu_refine_isa())")
    outs = {}
    for isa in ("", "avx2"):
        env = dict(os.environ, CORA_CPU_ISA=isa)
        out = tmp_path / f"ip_{isa or 'auto'}.npy"
        r = subprocess.run([sys.executable, "-c", code, str(REPO / "cgcl-coraanns_amd"), str(tmp_path / "q.npy"),
                            str(tmp_path / "packed.npy"), str(out)], env=env, capture_output=True, text=True,
                           check=True)
        outs[isa or "auto"] = (int(r.stdout.strip()), np.load(out))
    assert outs["avx2"][0] == 256
    want = orc.excode_ip(q, packed, 128)
    for isa, (width, ip) in outs.items():
        assert np.all(np.abs(ip - want) <= 1e-6 * np.abs(q).sum() * 127), isa


@pytest.mark.parametrize("P", [64, 128, 256])
def test_builder_excodes_equal_reference_rescale_search(P):
    """The builder's rescale search (events bucket-sorted on t, then swept) gives exactly the
    ex-codes of the oracle's priority-queue restatement of the reference's search."""
    import cora_oracle as orc
    rng = np.random.default_rng(P)
    rows = rng.normal(size=(24, P)).astype(np.float32)
    cent = (0.2 * rng.normal(size=P)).astype(np.float32)
    rows[3, :5] = cent[:5]  # a few zero residual coordinates
    _, _, ex, _ = ca.quantize_rows(rows, cent, metric=0)
    want = np.stack([orc.quantize_excode(r, cent, 7) for r in rows])
    assert np.array_equal(ex, want)


def test_gaussian_mixture_generator():
    """Counter-based benchmark rows: thread-count invariant, prefix-stable, standard normal
    noise (moments, and a chi-square fit of the mixture labels), unit norm when asked."""
    rng = np.random.default_rng(1)
    centers = rng.standard_normal((8, 64)).astype(np.float32) * 5
    sd = np.full(64, 0.5, np.float32)
    a = ca.gaussian_mixture(centers, sd, 20000, seed=99, threads=1)
    b = ca.gaussian_mixture(centers, sd, 20000, seed=99, threads=8)
    assert np.array_equal(a, b)
    assert np.array_equal(ca.gaussian_mixture(centers, sd, 500, seed=99), a[:500])
    assert not np.array_equal(ca.gaussian_mixture(centers, sd, 500, seed=98), a[:500])
    lab = np.argmin(((a[:, None, :] - centers[None]) ** 2).sum(-1), axis=1)
    z = ((a - centers[lab]) / sd).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.var() - 1) < 0.01
    assert abs((z ** 4).mean() - 3) < 0.05  # normal kurtosis
    counts = np.bincount(lab, minlength=8)
    chi2 = ((counts - 2500.0) ** 2 / 2500.0).sum()
    assert chi2 < 24.3  # 7 dof, p = 0.001
    u = ca.gaussian_mixture(centers, sd, 1000, seed=3, normalize=True)
    assert np.allclose(np.linalg.norm(u, axis=1), 1, atol=1e-6)
    with pytest.raises(ValueError):
        ca.gaussian_mixture(centers[:, :63], sd[:63], 10, seed=1)
