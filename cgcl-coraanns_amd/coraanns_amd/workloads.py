"""Seeded synthetic workloads for the benchmark configurations.

Data generation is numpy (seeded); k-means, nearest-centroid assignment, rotation and the
exhaustive ground truth run on the GPU through the engine's cora_tool_* entry points; the
IVF-RaBitQ index is written in the reference's on-disk format by the C++ builder.
Seeds follow the measurement plan: base = cfg, queries = 1000 + cfg, k-means = 2000 + cfg,
rotation = 3000 + cfg. Configurations of more than 2^31 values (4 and 5) draw base and
queries from the engine's counter-based generator (cora_gaussian_mixture) in parallel.
"""
from __future__ import annotations

import os
import struct
import time
from dataclasses import dataclass, field

import numpy as np

from . import build_ivf, build_ivf_gpu, gaussian_mixture, gpu_assign, gpu_kmeans, gpu_rotate, gpu_topk


@dataclass
class Config:
    cfg: int
    n: int
    dim: int
    n_centers: int
    nlist: int
    nq: int
    metric: int  # 0 = L2, 1 = IP
    topk: int
    nprobes: list
    center_scale: float
    within_sd: float
    anisotropic: bool = False
    normalize: bool = False
    batch_q: int = 4
    vanguard: int = 5
    secondary_filter: bool = True
    notes: str = ""

    @property
    def padded_dim(self):
        return (self.dim + 63) // 64 * 64

    def describe(self):
        return (f"cfg{self.cfg}: {self.n:,} x {self.dim} {'IP' if self.metric else 'L2'}, "
                f"nlist {self.nlist}, {self.nq:,} queries, top-{self.topk}")


CONFIGS = {
    1: Config(1, 4096, 128, 16, 16, 100, 0, 10, [4, 8, 16], 2.0, 1.0),
    2: Config(2, 1_000_000, 128, 1024, 1024, 10_000, 0, 10, [8, 16, 32, 64, 128], 1.0, 0.3,
              batch_q=64, notes="batch-q 64 as configured (the reference driver accepts 1..6)"),
    3: Config(3, 10_000_000, 96, 4096, 16384, 10_000, 0, 10, [16, 32, 64, 128, 256], 1.0, 0.5,
              anisotropic=True),
    4: Config(4, 20_000_000, 768, 8192, 16384, 10_000, 1, 10, [32, 64, 128, 256, 512], 1.0, 0.5,
              normalize=True),
    5: Config(5, 100_000_000, 96, 65536, 65536, 10_000, 0, 100, [64, 128, 256, 512, 1024], 1.0, 0.5,
              anisotropic=True, vanguard=10),
}


def _normal(rng, shape, chunk=1 << 22):
    out = np.empty(shape, np.float32)
    flat = out.reshape(-1)
    for s in range(0, flat.size, chunk):
        flat[s:s + chunk] = rng.standard_normal(min(chunk, flat.size - s), dtype=np.float32)
    return out


def generate(c: Config, n=None, nq=None, queries_only=False):
    """Base vectors and queries from the config's Gaussian mixture (base None when
    queries_only: the queries depend only on the centres and their own seed)."""
    n = c.n if n is None else n
    nq = c.nq if nq is None else nq
    rng_c = np.random.default_rng(c.cfg)
    var = (1.0 / (1.0 + np.arange(c.dim) / 8.0)).astype(np.float32) if c.anisotropic else \
        np.ones(c.dim, np.float32)
    centers = (_normal(rng_c, (c.n_centers, c.dim)) * (c.center_scale * np.sqrt(var))).astype(np.float32)

    def draw(rng, m, rows=1 << 18):
        lab = rng.integers(0, c.n_centers, m)
        x = _normal(rng, (m, c.dim))
        sd = (c.within_sd * np.sqrt(var))[None, :]
        for s in range(0, m, rows):  # in row blocks: no full-size temporaries
            blk = x[s:s + rows]
            blk *= sd
            blk += centers[lab[s:s + rows]]
            if c.normalize:
                blk /= np.linalg.norm(blk, axis=1, keepdims=True)
        return x

    if c.n * c.dim > 1 << 31:
        # configurations of billions of values: counter-based rows generated in parallel
        # (the numpy stream runs at ~60 M values/s on one core)
        sd = (c.within_sd * np.sqrt(var)).astype(np.float32)
        base = None if queries_only else gaussian_mixture(centers, sd, n, c.cfg + 10_000, c.normalize)
        return base, gaussian_mixture(centers, sd, nq, 1000 + c.cfg, c.normalize)
    base = None if queries_only else draw(np.random.default_rng(c.cfg + 10_000), n)
    queries = draw(np.random.default_rng(1000 + c.cfg), nq)
    return base, queries


def rotation(dim, P, seed):
    """Random orthonormal rows: first dim rows of Q^T for Q from QR of a P x P Gaussian
    (the construction of the reference MatrixRotator, rotator.hpp:57-71, seeded here)."""
    a = np.random.default_rng(seed).standard_normal((P, P))
    q, r = np.linalg.qr(a)
    q *= np.sign(np.diag(r))[None, :]
    return np.ascontiguousarray(q.T[:dim], np.float32)


def ground_truth(base, queries, k, metric, device=0, extra=16):
    """Exact top-k: GPU FP32 candidates (k + extra), re-ranked in FP64 on the host."""
    kk = min(base.shape[0], k + extra)
    cand = gpu_topk(base, queries, kk, metric, device)
    out = np.empty((queries.shape[0], k), np.uint32)
    q64 = queries.astype(np.float64)
    for s in range(0, queries.shape[0], 2048):
        b = base[cand[s:s + 2048]].astype(np.float64)  # [m, kk, dim]
        qq = q64[s:s + 2048, None, :]
        score = -(b * qq).sum(-1) if metric == 1 else ((b - qq) ** 2).sum(-1)
        order = np.lexsort((cand[s:s + 2048], score), axis=1)[:, :k]
        out[s:s + 2048] = np.take_along_axis(cand[s:s + 2048], order, axis=1)
    return out


def build_index(c: Config, base, path, device=0, log=print, kmeans_iters=20, threads=0, gpu_quantize=True):
    P = c.padded_dim
    R = rotation(c.dim, P, 3000 + c.cfg)
    t = time.time()
    sample_n = min(base.shape[0], 256 * c.nlist)
    rng = np.random.default_rng(2000 + c.cfg)
    sample = base[np.sort(rng.choice(base.shape[0], sample_n, replace=False))] if sample_n < base.shape[0] else base
    cent = gpu_kmeans(sample, c.nlist, kmeans_iters, 2000 + c.cfg, device)
    assign = gpu_assign(base, cent, device)
    log(f"[build] k-means {c.nlist} x {kmeans_iters} it on {sample_n:,} + assign {base.shape[0]:,}: "
        f"{time.time() - t:.1f}s")
    t = time.time()
    cr = (cent.astype(np.float64) @ R.astype(np.float64)).astype(np.float32)
    if gpu_quantize:
        # rotation and RaBitQ quantisation on the GPU, packing on the host
        build_ivf_gpu(path, base, cr, assign, R, metric=c.metric, device=device, threads=threads)
    else:
        build_ivf(path, gpu_rotate(base, R, device), cr, assign, R, metric=c.metric, threads=threads)
    log(f"[build] rotate + RaBitQ quantise ({'GPU' if gpu_quantize else 'host'}) + write {path}: "
        f"{time.time() - t:.1f}s")
    return R, cent, assign


def write_fbin(path, arr, dtype=np.float32):
    arr = np.ascontiguousarray(arr, dtype)
    with open(path, "wb") as f:
        f.write(struct.pack("<II", arr.shape[0], arr.shape[1]))
        f.write(arr.tobytes())
