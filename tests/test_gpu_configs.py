"""The benchmark configurations at their real sizes, on the GPU.

- Config 1 (4,096 x 128, 100 queries, nlist 16, nprobe 4/8/16): the frozen exhaustive search
  against the oracle's restatement at every nprobe, and production recall@10 against the
  reference CPU path (rabitq_cpu, built from the reference sources) on the same index file.
- Config 2 (1M x 128, 10,000 queries, nlist 1,024): production recall@10 at least the
  reference CPU path's on the same 2,000 queries over the whole nprobe grid, at batch-q 64 and
  4; live against frozen results and the frozen-threshold candidate count against the oracle's
  band on a 64-query sample.
- Configs 3-5 (10M x 96, 20M x 768 inner product, 100M x 96 at top-100 with vanguard 10):
  the full index built; production recall on a 256-query sample at the grid's first nprobe,
  at least rabitq_cpu's on the same queries minus 0.001 (config 4 also at top-100, with CPU
  refinement and with the GPU-final top-k); config 4's vanguard pass in its frozen test mode
  with the matrix-core lows pass, its publication bands and top-k checked on 16 queries; and
  the exhaustive frozen top-k of 4 queries against the oracle. The oracle reads only the
  probed clusters of the index file (open_ivf_lazy / cluster_data).
"""
import dataclasses
import os
import re
import subprocess
import sys
import time
from pathlib import Path

import numpy as np
import pytest

import cora_oracle as orc
import coraanns_amd as ca
from coraanns_amd import workloads as wl

pytestmark = pytest.mark.gpu
REPO = Path(__file__).resolve().parent.parent
RABITQ_CPU = REPO / "oracle" / "_ref" / "rabitq_cpu"
F32_MAX = np.finfo(np.float32).max


def say(msg):
    """Progress on stdout and, where the run's output directory exists, in a progress file
    there (index builds of the large configurations run for minutes)."""
    print(msg, flush=True)
    sys.stdout.flush()
    root = os.environ.get("GRAFT_REPO_ROOT")
    if root and os.path.isdir(os.path.join(root, "gpurun_out")):
        with open(os.path.join(root, "gpurun_out", "test_progress.log"), "a") as f:
            f.write(f"{time.strftime('%H:%M:%S')} {msg}\n")


def qint_from_planes(planes):
    nq, B, W = planes.shape
    sh = np.arange(32, dtype=np.uint32)
    bits = ((planes[:, :, :, None] >> sh) & 1).reshape(nq, B, W * 32).astype(np.int64)
    u = sum(bits[:, j, :] << j for j in range(8))
    return np.where(u >= 128, u - 256, u).astype(np.int32)


def query_side(eng, nq, P, nprobe):
    W = P // 32
    return {
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


def oracle_topk(lz, g, nprobe, topk, thresholds=None, queries=None):
    """The oracle's top-k of each query over its probed clusters (the GPU's probe lists and
    query-side values), reading only those clusters of the index file; also the count of
    vectors whose lower bound is below thresholds -/+ a 1e-5 band."""
    P = lz.padded_dim
    qint = qint_from_planes(g["planes"][:, :8])
    qres = qint_from_planes(g["planes"][:, 8:])
    queries = range(g["qr"].shape[0]) if queries is None else queries
    out = {}
    lo = hi = 0
    for q in queries:
        items = []
        thr = float(F32_MAX) if thresholds is None else float(thresholds[q])
        band = 1e-5 * (abs(thr) + 1)
        for p in range(nprobe):
            bits, f, lc, exf, ids, _ = orc.cluster_data(lz, int(g["pidx"][q, p]))
            if bits.shape[0] == 0:
                continue
            ipi = orc.ip_int_direct(bits, qint[q])
            low = orc.low_dist(f[:, 0], f[:, 1], f[:, 2], g["gadd"][q, p], g["gerr"][q, p],
                               orc.exact_ip_bitwise(ipi, g["width"][q]), g["k1"][q])
            low64 = low.astype(np.float64)  # the band around FLT_MAX does not fit FP32
            lo += int((low64 < thr - band).sum())
            hi += int((low64 < thr + band).sum())
            keep = np.nonzero(low < thr)[0]
            ex2 = orc.exact_ip_two_stage(ipi[keep], orc.ip_int_direct(bits[keep], qres[q]), g["width"][q],
                                         g["width2"][q])
            rd = orc.refine_dist(exf[keep, 0], exf[keep, 1], g["gadd"][q, p], ex2,
                                 orc.excode_ip(g["qr"][q], lc[keep], P), g["kb"][q], lz.ex_bits)
            items += list(zip(rd.tolist(), ids[keep].tolist()))
        items.sort()
        items = [t for t in items if t[0] < thr][:topk]
        out[q] = items
    return out, lo, hi


def assert_matches_oracle(d, i, want, rtol=1e-5):
    """GPU top-k distances within 1e-5 of the oracle's, ids equal except at ties."""
    for q, items in want.items():
        od = np.array([t[0] for t in items], np.float64)
        oi = [t[1] for t in items]
        scale = np.abs(od).max() + 1 if od.size else 1
        k = len(items)
        assert np.allclose(d[q, :k], od, rtol=0, atol=rtol * scale), q
        for r in range(k):
            if int(i[q, r]) != oi[r]:
                close = np.abs(od - d[q, r]) <= rtol * scale
                assert int(i[q, r]) in {oi[j] for j in np.nonzero(close)[0]}, (q, r)


def rabitq_cpu_recall(index_path, q, gt, topk, nprobes, tmp, threads=16):
    """recall@topk of the reference CPU path per nprobe (its own evaluator, ID mode)."""
    if not RABITQ_CPU.exists():
        pytest.skip("oracle/_ref/rabitq_cpu not built (needs /root/reference)")
    qf, gf = tmp / "rq.fbin", tmp / "rgt.ibin"
    wl.write_fbin(qf, q)
    wl.write_fbin(gf, gt[:, :topk], np.uint32)
    r = subprocess.run([str(RABITQ_CPU), str(index_path), str(qf), str(gf), "--topk", str(topk), "--nprobes",
                        ",".join(str(n) for n in nprobes), "--threads", str(threads), "--warmup", "0",
                        "--rounds", "1", "--hacc", "true"], capture_output=True, text=True, timeout=600,
                       env=dict(os.environ, OMP_NUM_THREADS=str(threads)))
    assert r.returncode == 0, r.stderr[-1000:]
    rows = re.findall(r"^(\d+)\t([\d.eE+-]+)\t([\d.eE+-]+)\s*$", r.stdout, re.M)
    return {int(n): float(rec) for n, _, rec in rows}


def engine(path, metric, nq, topk, nprobe, vanguard, **kw):
    ivf = ca.IvfIndex(path)
    eng = ca.HybridIndex(0, vanguard_size=vanguard, metric=metric, gpu_filter_timing=True, **kw)
    eng.load_ivf(ivf)
    eng.prepare_workspace(nq, topk, nprobe)
    return ivf, eng


def test_config1_exact(tmp_path):
    c = wl.CONFIGS[1]
    say(f"[gpu] {c.describe()}")
    base, q = wl.generate(c)
    path = tmp_path / "cfg1.index"
    wl.build_index(c, base, path, log=say)
    gt = orc.brute_force_gt(base, q, 10, c.metric)
    lz = orc.open_ivf_lazy(path)
    nq = q.shape[0]
    # frozen exhaustive search against the oracle at every nprobe of the grid
    ivf, eng = engine(path, c.metric, nq, c.topk, max(c.nprobes), 0, frozen_thresholds=True,
                      cpu_secondary_filter=False, lower_bound_scale=1.0)
    for nprobe in c.nprobes:
        eng.reset_buffer(q)
        d, i = eng.search(q, c.topk, nprobe)
        want, _, _ = oracle_topk(lz, query_side(eng, nq, c.padded_dim, nprobe), nprobe, c.topk)
        assert_matches_oracle(d, i, want)
    eng.close()
    # production mode against the reference CPU path on the same index file
    ref = rabitq_cpu_recall(path, q, gt, c.topk, c.nprobes, tmp_path)
    ivf, eng = engine(path, c.metric, nq, c.topk, max(c.nprobes), c.vanguard)
    for nprobe in c.nprobes:
        eng.reset_buffer(q)
        _, i = eng.search(q, c.topk, nprobe)
        r = orc.recall_at_k(i, gt, c.topk)
        say(f"[gpu]   cfg1 nprobe={nprobe}: recall@10 gpu {r:.4f} rabitq_cpu {ref[nprobe]:.4f}")
        assert r >= ref[nprobe] - 0.001, (nprobe, r, ref[nprobe])
    eng.close()


def test_config2_full_size(tmp_path):
    c = wl.CONFIGS[2]
    say(f"[gpu] {c.describe()}")
    base, q = wl.generate(c)
    path = tmp_path / "cfg2.index"
    wl.build_index(c, base, path, log=say)
    gt = wl.ground_truth(base, q, 10, c.metric)
    del base
    nq, sample, nprobes = q.shape[0], 2000, list(c.nprobes)
    ref = rabitq_cpu_recall(path, q[:sample], gt[:sample], 10, nprobes, tmp_path)
    ivf, eng = engine(path, c.metric, nq, c.topk, max(nprobes), c.vanguard, cpu_secondary_filter=True)
    live = {}
    # the whole nprobe grid at the configuration's batch-q 64, and the reference's own batch-q
    # range (1..6) at 4
    for batch_q in (c.batch_q, 4):
        for nprobe in nprobes:
            eng.reset_buffer(q)
            _, i = eng.search(q, c.topk, nprobe, batch_q)
            if batch_q == c.batch_q:
                live[nprobe] = i
            r_all = orc.recall_at_k(i, gt, 10)
            r = orc.recall_at_k(i[:sample], gt[:sample], 10)
            say(f"[gpu]   cfg2 nprobe={nprobe} batch-q {batch_q}: recall@10 gpu {r:.4f} (all {r_all:.4f}) "
                f"rabitq_cpu {ref[nprobe]:.4f} on the same {sample} queries")
            assert r >= ref[nprobe] - 0.001, (nprobe, batch_q, r, ref[nprobe])
            assert r_all >= 0.98
    eng.close()
    # a 64-query sample: frozen exhaustive vs live results, and the frozen candidate count
    qs = q[:64]
    lz = orc.open_ivf_lazy(path)
    ivf, eng = engine(path, c.metric, 64, c.topk, 8, 0, frozen_thresholds=True, cpu_secondary_filter=False,
                      lower_bound_scale=1.0)
    eng.reset_buffer(qs)
    d0, i0 = eng.search(qs, c.topk, 8)
    g = query_side(eng, 64, c.padded_dim, 8)
    want, _, _ = oracle_topk(lz, g, 8, c.topk)
    assert_matches_oracle(d0, i0, want)
    same = np.mean([len(set(a) & set(b)) / c.topk for a, b in zip(live[8][:64].tolist(), i0.tolist())])
    assert same >= 0.99, same
    thr = np.array([want[j][c.topk - 1][0] * 1.02 for j in range(64)], np.float32)
    eng.reset_buffer(qs)
    eng.seed_thresholds(thr)
    eng.search(qs, c.topk, 8)
    sub = eng.stats()["submitted"]
    _, lo, hi = oracle_topk(lz, g, 8, c.topk, thresholds=thr)
    say(f"[gpu]   cfg2 frozen candidates {sub} in the oracle's band [{lo}, {hi}]")
    assert lo <= sub <= hi
    eng.close()


class LazyProbed:
    """Every vector of a query's probed clusters, from the index file (only those clusters
    are read): probe rank, external ids, oracle lower bound, refined distance (the CPU
    consumer's formula) and its rounding bound; cluster slices are cached."""

    def __init__(self, lz, g):
        self.lz, self.g, self.cache = lz, g, {}
        self.qint = qint_from_planes(g["planes"][:, :8])
        self.qres = qint_from_planes(g["planes"][:, 8:])

    def __call__(self, q, nprobe):
        g, P = self.g, self.lz.padded_dim
        l1 = float(np.abs(g["qr"][q]).sum())
        out = []
        for p in range(nprobe):
            c = int(g["pidx"][q, p])
            if c not in self.cache:
                self.cache[c] = orc.cluster_data(self.lz, c)
            bits, f, lc, exf, ids, _ = self.cache[c]
            if bits.shape[0] == 0:
                continue
            ipi = orc.ip_int_direct(bits, self.qint[q])
            low = orc.low_dist(f[:, 0], f[:, 1], f[:, 2], g["gadd"][q, p], g["gerr"][q, p],
                               orc.exact_ip_bitwise(ipi, g["width"][q]), g["k1"][q])
            ex2 = orc.exact_ip_two_stage(ipi, orc.ip_int_direct(bits, self.qres[q]), g["width"][q], g["width2"][q])
            fa, fr = exf[:, 0], exf[:, 1]
            rd = orc.refine_dist(fa, fr, g["gadd"][q, p], ex2, orc.excode_ip(g["qr"][q], lc, P), g["kb"][q],
                                 self.lz.ex_bits)
            err = orc.refine_error_bound(fa, fr, g["gadd"][q, p], ex2, l1, g["kb"][q], self.lz.ex_bits, P)
            out.append((p, ids, low.astype(np.float64), rd.astype(np.float64), err.astype(np.float64)))
        return out


def check_frozen_vanguard_bands(eng, lz, nq, P, nprobe, vanguard, topk, d, i):
    """The vanguard pass's deterministic test mode (frozen snapshot lowered by the pass) on
    the index file: the threshold is backed by topk vanguard vectors below it; the vanguard
    pass publishes every vector with lower bound and refined distance below the threshold and
    nothing beyond its rounding bound; the far pass exactly the vectors with lower bound below
    the threshold and refined distance within the bound; the returned top-k are oracle
    distances at or below the threshold and miss no closer vector below it; and they agree
    with the oracle's exhaustive top-k over the probed clusters."""
    st = eng.stats()
    g = query_side(eng, nq, P, nprobe)
    thr = eng.debug_read(ca.DBG_THRESHOLDS, (nq,), np.float32)
    assert st["seeded_queries"] == nq
    probed = LazyProbed(lz, g)
    van_lo = van_hi = far_lo = far_hi = 0
    overlap = []
    for q in range(nq):
        T = float(thr[q])
        assert np.isfinite(T), q
        band = 1e-5 * (abs(T) + 1)
        backing = 0
        info = {}
        items = []
        for p, ids, low, rd, err in probed(q, nprobe):
            if p < vanguard:
                backing += int(((rd < T) & (low < T + band)).sum())
                van_lo += int(((low < T - band) & (rd <= T + 0.9 * err)).sum())
                van_hi += int((rd <= T + 1.1 * err).sum())
            else:
                far_lo += int(((low < T - band) & (rd <= T + 0.9 * err)).sum())
                far_hi += int(((low < T + band) & (rd <= T + 1.1 * err)).sum())
            for k in range(ids.size):
                info[int(ids[k])] = (p, low[k], rd[k], err[k])
            items += list(zip(rd.tolist(), ids.tolist()))
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
        items.sort()
        overlap.append(len(got & {pid for _, pid in items[:topk]}) / topk)
    produced = st["pass_produced"]
    say(f"[gpu]   frozen bands on {nq} queries: vanguard published {produced[0]} in [{van_lo}, {van_hi}], far "
        f"{produced[1] - produced[0]} in [{far_lo}, {far_hi}], exhaustive top-{topk} overlap {np.mean(overlap):.4f}")
    assert van_lo <= produced[0] <= van_hi
    assert far_lo <= produced[1] - produced[0] <= far_hi
    assert produced[2] == produced[1]
    assert np.mean(overlap) >= 0.99


@pytest.mark.parametrize("cfg", [3, 4, 5])
def test_large_config_full_size(cfg, tmp_path):
    """Production recall on a 256-query sample at the grid's first nprobe, at least the
    reference CPU path's (rabitq_cpu on the same index file and queries) minus 0.001;
    config 4 also at top-100 with CPU refinement and with the GPU-final top-k, and the
    vanguard pass's frozen bands on 16 queries with the matrix-core lows pass on; then the
    exhaustive frozen top-k of 4 queries against the oracle."""
    c = dataclasses.replace(wl.CONFIGS[cfg], nq=256)
    say(f"[gpu] {c.describe()}: generating and building the full index")
    base, q = wl.generate(c)
    path = tmp_path / f"cfg{cfg}.index"
    kmax = 100 if cfg == 4 else c.topk
    try:
        wl.build_index(c, base, path, log=say)
        gt = wl.ground_truth(base, q, kmax, c.metric)
        del base
        nprobe = c.nprobes[0]
        nq = q.shape[0]
        ref = rabitq_cpu_recall(path, q, gt, c.topk, [nprobe], tmp_path)[nprobe]
        say(f"[gpu]   cfg{cfg}: loading the index")
        prod = dict(vanguard_size=c.vanguard, metric=c.metric, gpu_filter_timing=True, cpu_secondary_filter=True)
        ivf = ca.IvfIndex(path)
        eng = ca.HybridIndex(0, **prod)
        eng.load_ivf(ivf)
        eng.prepare_workspace(nq, kmax, nprobe)
        eng.reset_buffer(q)
        _, i = eng.search(q, c.topk, nprobe, c.batch_q)
        r10, rk = orc.recall_at_k(i, gt, 10), orc.recall_at_k(i, gt, c.topk)
        say(f"[gpu]   cfg{cfg} nprobe={nprobe}: recall@10 {r10:.4f} recall@{c.topk} {rk:.4f}, rabitq_cpu "
            f"recall@{c.topk} {ref:.4f} (vanguard mode {eng.stats()['vanguard_mode']})")
        assert rk >= ref - 0.001 and r10 >= 0.9
        if cfg == 4:
            ref100 = rabitq_cpu_recall(path, q, gt, 100, [nprobe], tmp_path)[nprobe]
            for final in (False, True):
                eng.configure(**dict(prod, gpu_final_topk=final))
                eng.reset_buffer(q)
                _, i = eng.search(q, 100, nprobe, c.batch_q)
                r100 = orc.recall_at_k(i, gt, 100)
                say(f"[gpu]   cfg4 top-100 ({'GPU-final' if final else 'CPU refinement'}): recall@100 {r100:.4f}, "
                    f"rabitq_cpu {ref100:.4f}")
                assert r100 >= ref100 - 0.001, (final, r100, ref100)
        eng.close()
        lz = orc.open_ivf_lazy(path)
        if cfg == 4:
            qs = q[:16]
            eng = ca.HybridIndex(0, vanguard_size=5, metric=c.metric, gpu_filter_timing=True, frozen_thresholds=True,
                                 cpu_secondary_filter=False, lower_bound_scale=1.0,
                                 extra_flags=ca.FLAG_GPU_SEED_FROZEN | ca.FLAG_VANGUARD_MFMA)
            eng.load_ivf(ivf)
            eng.prepare_workspace(16, c.topk, nprobe)
            eng.reset_buffer(qs)
            d, i = eng.search(qs, c.topk, nprobe)
            assert eng.stats()["vanguard_mode"] in (3, 4), eng.stats()["vanguard_mode"]
            check_frozen_vanguard_bands(eng, lz, 16, c.padded_dim, nprobe, 5, c.topk, d, i)
            eng.close()
        # four queries: the exhaustive frozen search against the oracle over their probe lists
        qs = q[:4]
        ivf, eng = engine(path, c.metric, 4, c.topk, nprobe, 0, frozen_thresholds=True,
                          cpu_secondary_filter=False, lower_bound_scale=1.0)
        eng.reset_buffer(qs)
        d, i = eng.search(qs, c.topk, nprobe)
        want, _, _ = oracle_topk(lz, query_side(eng, 4, c.padded_dim, nprobe), nprobe, c.topk)
        assert_matches_oracle(d, i, want)
        eng.close()
        say(f"[gpu]   cfg{cfg}: frozen top-{c.topk} of 4 queries matches the oracle")
    finally:
        if path.exists():
            path.unlink()
