"""Write the golden fixtures under tests/golden/ from the reference's own CPU code.

Runs in the build container only (it needs /root/reference): compiles nothing itself,
it drives the binaries that oracle/Makefile builds into oracle/_ref/ from the reference
sources:

* ``coraanns_build_index`` (reference apps/build_index.cpp) builds an IVF-RaBitQ index
  in the reference's on-disk format (ivf.hpp:403-445) from seeded synthetic data and
  k-means centroids/assignments computed here with numpy;
* ``ref_dump index`` dumps the SearchData arrays, rotated queries, centroid
  distances, FastScan-hacc estimates, ex-distances and IVF::search top-k ids;
* ``ref_dump quant`` dumps RaBitQ 1-bit / ex-bit codes and factors, the 7-bit ex-code
  packing, the AVX2 ex-code inner product and FastScan code packing;
* ``rabitq_cpu`` (reference apps/baselines/cpu.cpp) prints its nprobe/QPS/recall table,
  kept as text.

Every fixture is data (inputs and the reference's outputs); no reference source is
copied. Usage: python tests/golden/make_golden.py
"""
import os
import shutil
import struct
import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
REF_BIN = REPO / "oracle" / "_ref"


def write_fbin(path, arr, dtype):
    arr = np.ascontiguousarray(arr, dtype=dtype)
    with open(path, "wb") as f:
        f.write(struct.pack("<II", arr.shape[0], arr.shape[1]))
        f.write(arr.tobytes())


def write_vecs(path, arr, dtype):
    arr = np.ascontiguousarray(arr, dtype=dtype)
    with open(path, "wb") as f:
        for row in arr:
            f.write(struct.pack("<I", row.shape[0]))
            f.write(row.tobytes())


def kmeans(x, k, iters, seed):
    rng = np.random.default_rng(seed)
    c = x[rng.choice(x.shape[0], k, replace=False)].astype(np.float64)
    for _ in range(iters):
        d = (x * x).sum(1)[:, None] - 2 * x @ c.T + (c * c).sum(1)[None, :]
        a = d.argmin(1)
        for j in range(k):
            m = a == j
            if m.any():
                c[j] = x[m].mean(0)
    d = (x * x).sum(1)[:, None] - 2 * x @ c.T + (c * c).sum(1)[None, :]
    return c.astype(np.float32), d.argmin(1).astype(np.uint32)


def mixture(rng, n, dim, centers, sd):
    lab = rng.integers(0, centers.shape[0], n)
    return (centers[lab] + rng.normal(0.0, sd, (n, dim))).astype(np.float32)


def make_index_fixture(name, n, dim, nlist, nq, metric, normalize, seed, nprobes, topk):
    out = HERE / name
    if out.exists():
        shutil.rmtree(out)
    out.mkdir(parents=True)
    rng = np.random.default_rng(seed)
    centers = rng.normal(0.0, 2.0, (max(nlist * 2, 16), dim))
    base = mixture(rng, n, dim, centers, 1.0)
    queries = mixture(rng, nq, dim, centers, 1.0)
    if normalize:
        base /= np.linalg.norm(base, axis=1, keepdims=True)
        queries /= np.linalg.norm(queries, axis=1, keepdims=True)
    cent, assign = kmeans(base.astype(np.float64), nlist, 15, seed + 1000)
    write_fbin(out / "base.fbin", base, np.float32)
    write_fbin(out / "queries.fbin", queries, np.float32)
    write_vecs(out / "centroids.fvecs", cent, np.float32)
    write_vecs(out / "assign.ivecs", assign[:, None], np.uint32)
    # exact ground truth (top-100 or n) by brute force in float64
    b64, q64 = base.astype(np.float64), queries.astype(np.float64)
    if metric == "ip":
        score = -(q64 @ b64.T)
    else:
        score = (q64 * q64).sum(1)[:, None] - 2 * q64 @ b64.T + (b64 * b64).sum(1)[None, :]
    gt = np.argsort(score, axis=1, kind="stable")[:, : min(100, n)].astype(np.uint32)
    write_fbin(out / "gt.ibin", gt, np.uint32)
    env = dict(os.environ, OMP_NUM_THREADS="1", OMP_DYNAMIC="FALSE")
    subprocess.run([str(REF_BIN / "coraanns_build_index"), str(out / "base.fbin"),
                    str(out / "centroids.fvecs"), str(out / "assign.ivecs"), "8",
                    str(out / "ivf.index"), metric, "false"],
                   check=True, env=env, stdout=subprocess.DEVNULL)
    dump = out / "ref"
    dump.mkdir()
    subprocess.run([str(REF_BIN / "ref_dump"), "index", str(out / "ivf.index"),
                    str(out / "queries.fbin"), str(dump), str(topk)] + [str(p) for p in nprobes],
                   check=True, env=env, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    table = subprocess.run([str(REF_BIN / "rabitq_cpu"), str(out / "ivf.index"),
                            str(out / "queries.fbin"), str(out / "gt.ibin"), "--topk", str(topk),
                            "--nprobes", ",".join(str(p) for p in nprobes), "--threads", "1",
                            "--warmup", "0", "--rounds", "1"],
                           check=True, env=env, capture_output=True, text=True).stdout
    lines = table.strip().splitlines()
    start = max(i for i, l in enumerate(lines) if l.startswith("nprobe\tQPS"))
    (out / "rabitq_cpu_table.txt").write_text("\n".join(lines[start:]) + "\n")
    for f in ["centroids.fvecs", "assign.ivecs"]:
        (out / f).unlink()


def make_quant_fixture(name, n, dim, seed):
    out = HERE / name
    if out.exists():
        shutil.rmtree(out)
    out.mkdir(parents=True)
    rng = np.random.default_rng(seed)
    centroid = rng.normal(0.0, 1.0, (1, dim))
    rows = centroid + rng.normal(0.0, 0.5, (n, dim))
    # a few rows with exact zeros in the residual to exercise the (o > 0) / (o >= 0) split
    rows[0, :8] = centroid[0, :8]
    allrows = np.vstack([centroid, rows]).astype(np.float32)
    allrows.tofile(out / "rows.f32")
    subprocess.run([str(REF_BIN / "ref_dump"), "quant", str(out / "rows.f32"), str(n), str(dim),
                    str(out)], check=True, stdout=subprocess.DEVNULL)


def main():
    if not (REF_BIN / "ref_dump").exists():
        sys.exit("build the reference CPU path first: make -C oracle ref")
    make_index_fixture("l2_d96", n=512, dim=96, nlist=8, nq=24, metric="l2", normalize=False,
                       seed=11, nprobes=[1, 2, 4, 8], topk=10)
    make_index_fixture("ip_d64", n=384, dim=64, nlist=6, nq=16, metric="ip", normalize=True,
                       seed=12, nprobes=[1, 3, 6], topk=10)
    make_quant_fixture("quant_d128", n=40, dim=128, seed=13)
    print("golden fixtures written under", HERE)


if __name__ == "__main__":
    main()
