"""The coraanns_search driver end to end (bin/coraanns_search, the reference driver's
command line and output, apps/search.cpp): the scenario of the reference's
tests/smoke_gpu.py:19-47 (known nearest vectors must be found with recall 1.0 through a
256-slot ring that wraps, with and without --exact-base), and the final table parsed the
way the reference's experiment runner parses it (tools/run_experiment.py:130-146)."""
import math
import os
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import coraanns_amd as ca
from coraanns_amd.workloads import rotation, write_fbin

pytestmark = pytest.mark.gpu
REPO = Path(__file__).resolve().parent.parent
DRIVER = REPO / "cgcl-coraanns_amd" / "bin" / "coraanns_search"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def parse_summary(text, expected):
    """The final nprobe/QPS/recall table: one row per requested nprobe, in order, finite
    QPS > 0 and recall in [0, 1]."""
    marker = "nprobe\tQPS\trecall"
    assert marker in text, "no final table"
    rows = []
    for line in text.rsplit(marker, 1)[1].splitlines():
        f = line.split()
        if len(f) != 3 or not f[0].isdigit():
            continue
        nprobe, qps, rec = int(f[0]), float(f[1]), float(f[2])
        assert math.isfinite(qps) and qps > 0 and math.isfinite(rec) and 0 <= rec <= 1
        rows.append((nprobe, qps, rec))
    assert [r[0] for r in rows] == expected, rows
    return rows


def write_fvecs(path, arr):
    arr = np.ascontiguousarray(arr, np.float32)
    out = np.empty((arr.shape[0], arr.shape[1] + 1), np.float32)
    out[:, 0] = np.array([arr.shape[1]], np.int32).view(np.float32)[0]
    out[:, 1:] = arr
    out.tofile(path)


@pytest.fixture(scope="module")
def known_neighbours(tmp_path_factory):
    """1,024 vectors of dim 96 around 4 centres (sd 0.1), vector i in cluster i % 4;
    the queries are five of the base vectors, each its own nearest neighbour."""
    rng = np.random.default_rng(42)
    dim, count, nlist = 96, 1024, 4
    centers = rng.uniform(-4, 4, (nlist, dim)).astype(np.float32)
    assign = (np.arange(count) % nlist).astype(np.uint32)
    base = (centers[assign] + rng.normal(0, 0.1, (count, dim))).astype(np.float32)
    selected = np.array([3, 17, 205, 511, 1001])
    d = tmp_path_factory.mktemp("driver")
    R = rotation(dim, 128, 5)
    ca.build_ivf(d / "ivf.index", (base.astype(np.float64) @ R).astype(np.float32),
                 (centers.astype(np.float64) @ R).astype(np.float32), assign, R, metric=0)
    write_fbin(d / "base.fbin", base)
    write_fvecs(d / "base.fvecs", base)
    write_fbin(d / "queries.fbin", base[selected])
    write_fbin(d / "gt.ibin", selected[:, None], np.uint32)
    return d


def run_driver(args, timeout=120):
    r = subprocess.run([str(DRIVER)] + [str(a) for a in args], capture_output=True, text=True,
                       timeout=timeout, env=dict(os.environ, OMP_NUM_THREADS="2", OMP_DYNAMIC="FALSE"))
    return r


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("recall_base", ["base.fbin", "base.fvecs"])
def test_driver_recovers_known_neighbours(known_neighbours, exact, recall_base):
    d = known_neighbours
    say(f"[gpu] coraanns_search exact={exact} recall_base={recall_base}")
    args = [d / "ivf.index", d / "queries.fbin", d / "gt.ibin", "--topk", 1, "--nprobes", 4,
            "--threads", 2, "--warmup", 0, "--rounds", 1, "--query-chunk", 2, "--queue-capacity", 256,
            "--queue-spill-capacity", 8192, "--recall-base", d / recall_base, "--candidate-stats", "true"]
    if exact:
        args += ["--exact-base", d / "base.fbin"]
    r = run_driver(args)
    assert r.returncode == 0, r.stdout + r.stderr
    rows = parse_summary(r.stdout, [4])
    assert rows[0][2] == 1.0, r.stdout
    assert "[Recall] mode=distance-aware" in r.stdout
    runs = re.findall(r"^\[Run\] round=1 nprobe=4 QPS=([\d.eE+-]+) recall=([\d.eE+-]+)$", r.stdout, re.M)
    assert len(runs) == 1 and float(runs[0][1]) == 1.0
    # every (query, vector) pair of the 4 probed clusters is a candidate of the all-probe
    # search (1,024 per query) unless the filter drops it; none may be lost to the ring wraps
    qs = re.findall(r"^\[QueueStats\] round=1 nprobe=4 submitted=(\d+) spilled=(\d+) wraps=(\d+)$",
                    r.stdout, re.M)
    assert len(qs) == 1 and 0 < int(qs[0][0]) <= 5 * 1024


def test_driver_multiple_nprobes_and_recall_once(known_neighbours):
    d = known_neighbours
    say("[gpu] coraanns_search nprobe grid, --recall-once")
    r = run_driver([d / "ivf.index", d / "queries.fbin", d / "gt.ibin", "--topk", 1, "--nprobes", "1,2,4",
                    "--warmup", 1, "--rounds", 2, "--recall-once", "true", "--profile", "true",
                    "--gpu-filter-timing", "true"])
    assert r.returncode == 0, r.stdout + r.stderr
    rows = parse_summary(r.stdout, [1, 2, 4])
    assert rows[-1][2] == 1.0
    assert len(re.findall(r"^\[RecallPoint\] nprobe=\d+ source_round=1 recall=", r.stdout, re.M)) == 3
    assert len(re.findall(r"^\[GPUFilter\] round=\d+ nprobe=\d+ ", r.stdout, re.M)) == 6
    # the reference's per-search profile phases (hybrid.cu:479, 500, 516, 679-685)
    for phase in ["0~2. Initial Matrix Math", "3. Select Top-nprobe Clusters", "4. Flatten Pairs",
                  "7~9. Single-Stage Global Task Pool Pipeline (BITWISE_DECOMP)"]:
        times = re.findall(r"^\[Profile\] " + re.escape(phase) + r" time: ([\d.eE+-]+) ms$", r.stdout, re.M)
        assert len(times) == 9 and all(float(t) >= 0 for t in times), (phase, len(times))
    assert r.stdout.count("------------------------------------------") == 9


@pytest.mark.parametrize("bad", [
    ["--topk", "0"], ["--nprobes", "5"], ["--nprobes", "2,2"], ["--batch-q", "65"], ["--batch-q", "0"], ["--rounds", "x"],
    ["--unknown", "1"], ["--queue-capacity", "300"], ["--lower-bound-scale", "0"],
])
def test_driver_rejects_invalid_options(known_neighbours, bad):
    d = known_neighbours
    r = run_driver([d / "ivf.index", d / "queries.fbin", d / "gt.ibin"] + bad)
    assert r.returncode == 1 and "coraanns_search failed" in r.stderr, (bad, r.stdout, r.stderr)


def test_driver_reads_hnsw_sidecar_index(known_neighbours, tmp_path):
    """An index whose centroids live in an hnswlib sidecar (the reference's form for
    nlist >= 20000, ivf.hpp:487-520), labels stored out of order: at nprobe 1 every query
    must probe its own cluster, so a wrong label-to-centroid mapping loses the recall."""
    from test_ivf_storage import write_sidecar
    d = known_neighbours
    side = tmp_path / "side.index"
    write_sidecar(d / "ivf.index", side, np.array([2, 0, 3, 1]))
    say("[gpu] coraanns_search on an HNSW-sidecar index")
    r = run_driver([side, d / "queries.fbin", d / "gt.ibin", "--topk", 1, "--nprobes", "1,4", "--warmup", 0,
                    "--rounds", 1])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Centroids: HNSW sidecar" in r.stdout
    rows = parse_summary(r.stdout, [1, 4])
    assert rows[0][2] == 1.0 and rows[1][2] == 1.0, r.stdout
