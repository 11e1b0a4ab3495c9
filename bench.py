#!/usr/bin/env python3
"""Benchmark: QPS at recall@10 >= 0.9 of the MI355X GPU-filter / CPU-refine IVF-RaBitQ
search on one GPU, plus the RaBitQ scan kernel's HBM roofline and the reference CPU path
(rabitq_cpu) timed on the same host.

A step is what the reference driver times per query chunk (apps/search.cpp:230,251-253):
reset_buffer (query upload, queue and threshold reset) followed by search() over the
workload's full query set (one chunk of <= 65,535 queries), with the index resident in
HBM. The rate of search() alone is reported as config.qps_search_only. The
headline nprobe is the smallest of the configuration's nprobe grid whose recall@10 reaches
the target. Prints one JSON line on stdout; progress goes to stderr.

--copy-calibration runs only a plain device copy of a known size (torch) so that
rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE can be scaled to bytes.
"""
import argparse
import json
import os
import re
import shutil
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "cgcl-coraanns_amd"))

HBM_PEAK_GBPS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
FP16_MFMA_PEAK_TFLOPS = 2500.0  # dense


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def recall_at_k(ids, gt, k):
    hits = 0
    for r, g in zip(ids[:, :k], gt[:, :k]):
        hits += len(np.intersect1d(r, g))
    return hits / (ids.shape[0] * k)


def cpu_baseline(index_path, queries, gt, topk, nprobe, threads, workdir, sample):
    """rabitq_cpu (the reference CPU path) on the first `sample` queries, 1 warmup + 3
    rounds; None when it is not built, fails or exceeds its time limit."""
    exe = REPO / "oracle" / "_ref" / "rabitq_cpu"
    if not exe.exists():
        return None
    queries, gt = queries[:sample], gt[:sample]
    from coraanns_amd.workloads import write_fbin
    qf, gf = Path(workdir) / "bq.fbin", Path(workdir) / "bgt.ibin"
    write_fbin(qf, queries)
    write_fbin(gf, gt[:, :topk], np.uint32)
    env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_DYNAMIC="FALSE")
    # the reference's measurement recipe runs it with memory interleaved over NUMA nodes
    # (README.md:100, docs/REPRODUCIBILITY.md:71); numactl is used when the host has it
    numactl = shutil.which("numactl")
    cmd = ([numactl, "--interleave=all"] if numactl else []) + [str(exe), str(index_path), str(qf), str(gf), "--topk", str(topk), "--nprobes", str(nprobe),
           "--threads", str(threads), "--warmup", "1", "--rounds", "3", "--hacc", "true"]
    t = time.time()
    try:
        out = subprocess.run(cmd, capture_output=True, text=True, env=env, timeout=600)
    except subprocess.TimeoutExpired:
        log("[cpu_baseline] rabitq_cpu exceeded 600 s; no baseline")
        return None
    if out.returncode != 0:
        log(f"[cpu_baseline] rabitq_cpu failed: {out.stderr[-500:]}")
        return None
    rows = re.findall(r"^(\d+)\t([\d.eE+-]+)\t([\d.eE+-]+)\s*$", out.stdout, re.M)
    if not rows:
        return None
    _, qps, rec = rows[-1]
    log(f"[cpu_baseline] rabitq_cpu nprobe={nprobe} threads={threads}: QPS={float(qps):.1f} "
        f"recall={float(rec):.4f} ({time.time() - t:.1f}s)")
    return {"value": round(float(qps), 1), "unit": "queries/s", "cores": threads, "kind": "reference",
            "recall": round(float(rec), 4),
            "numactl_interleave": bool(numactl),
            "sample": f"{queries.shape[0]} queries x 3 rounds (1 warmup) at nprobe {nprobe}, top-{topk}, "
                      f"same index file, rabitq_cpu --hacc true built -mavx2 -mfma"
                      f"{', numactl --interleave=all' if numactl else ' (no numactl on this host)'}"}


def hbm_traffic(run, kernel):
    """HBM bytes per launch of the kernel (FETCH_SIZE + WRITE_SIZE, each scaled by the
    reading of a 1 GiB copy) from the committed rocprofv3 summary whose "match" block names
    exactly this run's workload and mode (config, nprobe, top-k, batch-q, estimator, GPU-final
    top-k, vanguard mode), or None when no summary matches."""
    for f in sorted((REPO / "profiles").glob("hbm_traffic_*.json")):
        data = json.loads(f.read_text())
        if data.get("match") != run:
            continue
        for v in data.get("kernels", {}).values():
            if v.get("role") == kernel:
                return int(v["fetch_bytes"] + v["write_bytes"])
    return None


def extra_lines(eng, eng_cfg, queries, gt, c, nprobe, args, traffic_key):
    """Two further measurements on the resident index at the headline nprobe, each 1 warmup +
    args.extra_steps timed searches:
    - scan_q1: the RaBitQ popcount scan at Q = 1 (cross-query reuse off, every far
      (query, probe) pair a unit of its own), its HIP-event time and algorithmic bytes
      sum n_c (P/8 + 12) over the units, against the HBM peak;
    - reference_structure: the reference's structure, GPU filter -> ring -> CPU refinement of
      every candidate (GPU seed thresholds and GPU refined pre-filter off), its QPS and recall.
    The engine is configured back to eng_cfg afterwards."""
    import coraanns_amd as ca

    def timed(cfg, batch_q, chunk=None):
        eng.configure(**cfg)
        rows = []
        for it in range(1 + args.extra_steps):
            t0 = time.perf_counter()
            if chunk:
                _, ids = eng.search_all(queries, c.topk, nprobe, batch_q, chunk=chunk)
            else:
                eng.reset_buffer(queries)
                _, ids = eng.search(queries, c.topk, nprobe, batch_q)
            dt = time.perf_counter() - t0
            if it:
                rows.append((dt, ids, eng.stats()))
        return rows

    out = {}
    W = c.padded_dim // 32
    rows = timed(dict(eng_cfg, cross_query_reuse=False), 1)
    ms = float(np.mean([st["scan_ms"] for _, _, st in rows]))
    nbytes = float(np.mean([st["scan_bytes"] for _, _, st in rows]))
    ach = nbytes / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
    key = dict(traffic_key, batch_q=1, mode="scan_q1")
    out["scan_q1"] = {"kernel": f"scan_kernel<{W}, 1, 0, {1 if args.ip_kernel == 'lut4' else 0}> "
                                "(far-pair RaBitQ scan, one (query, probe) pair per unit, cross-query reuse off)",
                      "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                      "frac": round(ach / HBM_PEAK_GBPS, 4), "bytes_per_launch": int(nbytes),
                      "avg_launch_ms": round(ms, 4), "traffic": hbm_traffic(key, "scan_q1"),
                      "recall_at_10": round(float(np.mean([recall_at_k(i, gt, 10) for _, i, _ in rows])), 4),
                      "qps": round(queries.shape[0] * len(rows) / sum(dt for dt, _, _ in rows), 1)}
    log(f"[scan_q1] nprobe={nprobe} scan {ms:.3f}ms {nbytes / 1e6:.1f}MB -> {ach:.1f} GB/s "
        f"({ach / HBM_PEAK_GBPS:.3f} of peak)")
    if args.no_reference_structure:
        eng.configure(**eng_cfg)
        return out
    # every candidate goes to the ring: when a chunk of all queries publishes more than the
    # ring and its HBM spill hold (the reference's default sizes), the queries go in smaller
    # chunks, as the reference driver's --query-chunk does
    ref_cfg = dict(eng_cfg, gpu_seed_refine=False, gpu_refine_filter=False, gpu_final_topk=False)
    chunk = None
    for chunk in (None, 2048, 512):
        try:
            rows = timed(ref_cfg, args.batch_q or c.batch_q, chunk)
            break
        except ca.EngineError as e:
            if e.code != 4 or chunk == 512:  # CORA_ERR_SPILL_EXHAUSTED
                raise
            log(f"[reference_structure] {e}; query chunks of {2048 if chunk is None else 512}")
    qps = queries.shape[0] * len(rows) / sum(dt for dt, _, _ in rows)
    out["reference_structure"] = {
        "what": "GPU filter -> ring -> CPU refinement of every candidate (--no-gpu-seed --no-gpu-prefilter), "
                "the reference's structure, same index, queries, nprobe and batch-q",
        "qps": round(qps, 1), "ms_per_step": round(1000.0 * sum(dt for dt, _, _ in rows) / len(rows), 3),
        "query_chunk": chunk or queries.shape[0],
        "recall_at_10": round(float(np.mean([recall_at_k(i, gt, 10) for _, i, _ in rows])), 4),
        f"recall_at_{c.topk}": round(float(np.mean([recall_at_k(i, gt, c.topk) for _, i, _ in rows])), 4),
        "candidates_per_query": round(float(np.mean([st["submitted"] for _, _, st in rows])) / queries.shape[0], 1)}
    log(f"[reference_structure] nprobe={nprobe} QPS={qps:.1f} "
        f"recall@10={out['reference_structure']['recall_at_10']:.4f}")
    eng.configure(**eng_cfg)
    return out


def copy_calibration():
    """A plain device-to-device copy of 1 GiB, 5 times: the reference kernel for scaling
    the FETCH_SIZE / WRITE_SIZE counters (each launch reads and writes 1 GiB)."""
    import torch

    src = torch.empty(1 << 28, dtype=torch.float32, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": src.numel() * 4, "launches": 5}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=4,
                    help="BASELINE configuration (default 4: 20M x 768 inner product, the headline workload)")
    ap.add_argument("--nprobe", type=int, default=0, help="0: smallest grid nprobe reaching the recall target")
    ap.add_argument("--topk", type=int, default=0, help="override the configuration's top-k (config 4: 10 and 100)")
    ap.add_argument("--recall-target", type=float, default=0.9)
    ap.add_argument("--batch-q", type=int, default=0)
    ap.add_argument("--vanguard", type=int, default=-1, help="vanguard size (default: the configuration's)")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-queries", type=int, default=0,
                    help="queries in the CPU baseline sample (0: all at P <= 128, 2,000 above)")
    ap.add_argument("--n", type=int, default=0, help="override base size (testing only)")
    ap.add_argument("--nq", type=int, default=0, help="override query count (testing only)")
    ap.add_argument("--no-gpu-seed", action="store_true",
                    help="CPU-only thresholds (the reference's behaviour), no GPU seed thresholds")
    ap.add_argument("--no-gpu-prefilter", action="store_true", help="no GPU refined pre-filter")
    ap.add_argument("--lower-bound-scale", type=float, default=0.0,
                    help="multiplier of the filter's error term (0: the engine's default; 1: the "
                         "reference Bitwise producer's bound)")
    ap.add_argument("--gpu-final", action="store_true",
                    help="GPU-final top-k: the GPU forms the final top-k from its refined distances, no CPU refinement")
    ap.add_argument("--no-vanguard-mfma", action="store_true",
                    help="vanguard lower bounds inside the per-query pass instead of the matrix-core lows pass")
    ap.add_argument("--vanguard-one-pass", action="store_true",
                    help="after the lows pass, run the vanguard pairs in the one per-query kernel (the default "
                         "with the Bitwise estimator up to top-128)")
    ap.add_argument("--vanguard-staged", action="store_true",
                    help="after the lows pass, run the staged vanguard pass (per-query select and merge around "
                         "grid-wide refinement; the default with LUT4 and above top-128)")
    ap.add_argument("--vanguard-mfma", action="store_true",
                    help="run the matrix-core vanguard lows pass whatever the index size and dimension")
    ap.add_argument("--ip-kernel", choices=["bitwise", "lut4"], default="bitwise",
                    help="estimator: bitwise (Bq=8 popcount bound, the default here) or lut4 (the reference's "
                         "FP16 nibble-LUT estimator, set_ip_kernel_type(Lut4Bit))")
    ap.add_argument("--unfused-probe", action="store_true",
                    help="coarse probe through the whole distance matrix and a select pass over it, instead of "
                         "the select fused into the GEMM epilogue")
    ap.add_argument("--fp32-gemm", action="store_true",
                    help="query rotation and coarse-probe distances from the FP32 matrix-core GEMMs instead of the split-FP16 ones")
    ap.add_argument("--workdir", default="",
                    help="keep the built index and ground truth in this directory and reuse them")
    ap.add_argument("--no-extra-lines", action="store_true",
                    help="configs 4 and 5: skip the Q=1 scan roofline and the reference-structure line")
    ap.add_argument("--extra-steps", type=int, default=3, help="timed steps of each extra line (after 1 warmup)")
    ap.add_argument("--no-reference-structure", action="store_true",
                    help="of the extra lines, measure the Q=1 scan only")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (PMC byte-count calibration)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU runs are not part of it "
                                   "(N GPUs would each hold the whole index and search 1/N of the queries)",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import coraanns_amd as ca
    from coraanns_amd import workloads as wl

    c = wl.CONFIGS[args.config]
    if args.topk:  # config 4 is specified at top-10 and top-100
        import dataclasses
        c = dataclasses.replace(c, topk=args.topk)
    # CPU refinement threads: at top-10 the GPU bounds the step and 12 of the box's 16-CPU
    # share leave room for the submitting thread and the HIP runtime's threads (with 16
    # spinning consumers a search now and then waited a scheduler tick, ~4 ms); at top-100
    # the CPU refinement of ~190 candidates per query bounds it and takes all 16; with the
    # GPU-final top-k the CPU refines nothing (its threads copy the queries and map the
    # result ids), and 16 threads left 7 of 10 steps 6-9 ms longer
    threads = args.cpu_threads or min(12 if c.topk <= 10 or args.gpu_final else 16, os.cpu_count() or 16)
    batch_q = args.batch_q or c.batch_q
    workdir = args.workdir or tempfile.mkdtemp(prefix="cora_bench_")
    os.makedirs(workdir, exist_ok=True)
    index_path = Path(workdir) / f"cfg{c.cfg}.index"
    gt_path = Path(workdir) / (f"cfg{c.cfg}_gt.npy" if not args.topk else f"cfg{c.cfg}_gt_top{c.topk}.npy")
    t0 = time.time()
    if args.workdir and index_path.exists() and gt_path.exists():
        _, queries = wl.generate(c, n=args.n or None, nq=args.nq or None, queries_only=True)
        gt = np.load(gt_path)
        log(f"[data] {c.describe()}: index and ground truth reused from {workdir}")
    else:
        base, queries = wl.generate(c, n=args.n or None, nq=args.nq or None)
        log(f"[data] {c.describe()}: generated {base.shape} + {queries.shape} in {time.time() - t0:.1f}s")
        if args.workdir and index_path.exists():
            log(f"[data] index reused from {workdir}; ground truth for top-{c.topk} computed")
        else:
            wl.build_index(c, base, index_path, log=log)
        t = time.time()
        gt = wl.ground_truth(base, queries, c.topk, c.metric)
        log(f"[gt] exact top-{c.topk} (GPU FP32 + FP64 re-rank): {time.time() - t:.1f}s")
        del base
        if args.workdir:
            np.save(gt_path, gt)

    ivf = ca.IvfIndex(index_path)
    vanguard = c.vanguard if args.vanguard < 0 else args.vanguard
    eng_cfg = dict(vanguard_size=vanguard, cpu_secondary_filter=c.secondary_filter,
                   cross_query_reuse=True, gpu_filter_timing=True, metric=c.metric,
                   cpu_threads=threads, gpu_seed_refine=not args.no_gpu_seed,
                   gpu_refine_filter=not args.no_gpu_prefilter,
                   extra_flags=(ca.FLAG_FP32_GEMM if args.fp32_gemm else 0) |
                               (ca.FLAG_NO_VANGUARD_MFMA if args.no_vanguard_mfma else 0) |
                               (ca.FLAG_VANGUARD_MFMA if args.vanguard_mfma else 0) |
                               (ca.FLAG_VANGUARD_ONE_PASS if args.vanguard_one_pass else 0) |
                               (ca.FLAG_VANGUARD_STAGED if args.vanguard_staged else 0) |
                               (ca.FLAG_UNFUSED_PROBE if args.unfused_probe else 0),
                   lower_bound_scale=args.lower_bound_scale or None, gpu_final_topk=args.gpu_final,
                   ip_kernel_type=args.ip_kernel)
    eng = ca.HybridIndex(0, **eng_cfg)
    eng.load_ivf(ivf)
    chunk = min(queries.shape[0], 65535)
    eng.prepare_workspace(chunk, c.topk, max(c.nprobes))
    log(f"[engine] index resident in HBM: {ivf.num:,} vectors, max cluster {ivf.max_cluster}, "
        f"cpu refine threads {threads}, batch_q {batch_q}")

    assert queries.shape[0] <= chunk, "one search() per step"

    def step(nprobe):
        # reset_buffer + search, as the reference driver times each chunk
        t0 = time.perf_counter()
        eng.reset_buffer(queries)
        t = time.perf_counter()
        d, i = eng.search(queries, c.topk, nprobe, batch_q)
        t1 = time.perf_counter()
        step.search_only = t1 - t
        return t1 - t0, i, eng.stats()

    sweep = []
    for nprobe in ([] if args.nprobe else c.nprobes):  # --nprobe: measure that one only
        step(nprobe)
        dt, ids, st = step(nprobe)
        r = recall_at_k(ids, gt, 10)
        sweep.append({"nprobe": nprobe, "qps": round(queries.shape[0] / dt, 1), "recall": round(r, 4),
                      f"recall_at_{c.topk}": round(recall_at_k(ids, gt, c.topk), 4),
                      "candidates_per_query": round(st["submitted"] / queries.shape[0], 1),
                      "seed_ms": round(st["seed_ms"], 3), "scan_ms": round(st["scan_ms"], 3),
                      "recovery_ms": round(st["recovery_ms"], 3), "filter_ms": round(st["gpu_filter_ms"], 3)})
        pp = st["pass_produced"]
        log(f"[sweep] nprobe={nprobe} QPS={queries.shape[0] / dt:.1f} recall@10={r:.4f} "
            f"recall@{c.topk}={recall_at_k(ids, gt, c.topk):.4f} "
            f"cand/q={st['submitted'] / queries.shape[0]:.1f} (seed {pp[0] / queries.shape[0]:.1f}, "
            f"far {(pp[1] - pp[0]) / queries.shape[0]:.1f}, recovery {(pp[2] - pp[1]) / queries.shape[0]:.1f}; "
            f"gpu-seeded queries {st['seeded_queries']}, pre-filter dropped "
            f"{st['prefilter_dropped'] / queries.shape[0]:.1f}) seed={st['seed_ms']:.3f}ms far={st['scan_ms']:.3f}ms "
            f"recovery={st['recovery_ms']:.3f}ms filter={st['gpu_filter_ms']:.3f}ms")
    nprobe = args.nprobe
    if not nprobe:
        ok = [s["nprobe"] for s in sweep if s["recall"] >= args.recall_target]
        nprobe = ok[0] if ok else c.nprobes[-1]

    for _ in range(args.warmup):
        step(nprobe)
    times, times_search, scan_ms, scan_bytes, recalls, probe_ms, probe_flops = [], [], [], [], [], [], []
    select_ms = []
    recalls_k = []
    van_ms, van_bytes, lows_ms, lows_bytes, ref_ms, ref_bytes, van_modes = [], [], [], [], [], [], []
    refined, pair_vectors = [], []
    cands = []
    staged_counts = []
    last_ids = None
    for _ in range(args.steps):
        dt, ids, st = step(nprobe)
        last_ids = ids
        times.append(dt)
        times_search.append(step.search_only)
        probe_ms.append(st["probe_ms"])
        select_ms.append(st["phase_ms"][1])
        probe_flops.append(st["probe_flops"])
        scan_ms.append(st["scan_ms"])
        scan_bytes.append(st["scan_bytes"])
        van_ms.append(st["vanguard_ms"])
        van_bytes.append(st["vanguard_bytes"])
        lows_ms.append(st["vanguard_lows_ms"])
        lows_bytes.append(st["vanguard_lows_bytes"])
        ref_ms.append(st["vanguard_refine_ms"])
        ref_bytes.append(st["vanguard_refine_bytes"])
        van_modes.append(st["vanguard_mode"])
        refined.append(st["gpu_refined"])
        if st["vanguard_lows_ms"] > 0:
            # with the lows pass the per-query pass's bytes are 4 per vanguard (query, vector)
            # bound plus P + 8 per refined vector: the (query, vector) count of the vanguard pairs
            pair_vectors.append((st["vanguard_bytes"] - st["gpu_refined"] * (c.padded_dim + 8)) / 4)
        cands.append(st["submitted"])
        if st["vanguard_mode"] == 4 and not staged_counts:
            staged_counts.extend(int(x) for x in eng.debug_read(ca.DBG_STAGED_COUNTS, (4,), np.uint64))
            log(f"[staged] seeds {staged_counts[0]}, list {staged_counts[1]}, lists from a second pass "
                f"{staged_counts[2]}, queries left to the one-pass kernel {staged_counts[3]}")
        recalls.append(recall_at_k(ids, gt, 10))
        recalls_k.append(recall_at_k(ids, gt, c.topk))
    total = sum(times)
    qps = queries.shape[0] * args.steps / total
    ms_step = 1000.0 * total / args.steps
    avg_scan_ms = float(np.mean(scan_ms))
    bytes_per_launch = float(np.mean(scan_bytes))
    achieved = bytes_per_launch / (avg_scan_ms * 1e-3) / 1e9 if avg_scan_ms > 0 else 0.0
    avg_van_ms = float(np.mean(van_ms))
    van_bpl = float(np.mean(van_bytes))
    van_achieved = van_bpl / (avg_van_ms * 1e-3) / 1e9 if avg_van_ms > 0 else 0.0
    avg_lows_ms = float(np.mean(lows_ms))
    lows_bpl = float(np.mean(lows_bytes))
    lows_achieved = lows_bpl / (avg_lows_ms * 1e-3) / 1e9 if avg_lows_ms > 0 else 0.0
    avg_ref_ms = float(np.mean(ref_ms))
    ref_bpl = float(np.mean(ref_bytes))
    ref_achieved = ref_bpl / (avg_ref_ms * 1e-3) / 1e9 if avg_ref_ms > 0 else 0.0
    staged = avg_ref_ms > 0
    avg_probe_ms = float(np.mean(probe_ms))
    probe_tflops = float(np.mean(probe_flops)) / (avg_probe_ms * 1e-3) / 1e12 if avg_probe_ms > 0 else 0.0
    if args.fp32_gemm:
        probe_line = {"kernel": "dist_gemm_kernel (coarse-probe L2 distances, 128x128 tiles, v_mfma_f32_16x16x4f32)",
                      "flops_per_launch": int(np.mean(probe_flops)), "avg_launch_ms": round(avg_probe_ms, 4),
                      "achieved": round(probe_tflops, 3), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                      "frac": round(probe_tflops / FP32_MFMA_PEAK_TFLOPS, 4)}
    else:
        # three FP16 products per term: the matrix cores execute 3x the GEMM's 2 nq P nlist
        # flops; the time includes the split of the queries into FP16 pairs
        probe_line = {"kernel": "split_f16_kernel + dist_gemm_f16x3_kernel (coarse-probe L2 distances, "
                                "split-FP16 operands, 3 x v_mfma_f32_16x16x32_f16 per term, 128x128 tiles)",
                      "flops_per_launch": 3 * int(np.mean(probe_flops)),
                      "gemm_flops": int(np.mean(probe_flops)), "avg_launch_ms": round(avg_probe_ms, 4),
                      "achieved": round(3 * probe_tflops, 3), "peak": FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                      "frac": round(3 * probe_tflops / FP16_MFMA_PEAK_TFLOPS, 4),
                      "fp32_equivalent_tflops": round(probe_tflops, 3)}
    probe_line["select_and_gadd_ms"] = round(float(np.mean(select_ms)), 4)
    log(f"[timed] nprobe={nprobe} steps={args.steps} QPS={qps:.1f} recall={np.mean(recalls):.4f} "
        f"cand/q={np.mean(cands) / queries.shape[0]:.1f} refined/q={np.mean(refined) / queries.shape[0]:.1f} "
        f"vanguard lows={avg_lows_ms:.3f}ms {lows_bpl / 1e6:.1f}MB -> {lows_achieved:.1f} GB/s; "
        f"vanguard={avg_van_ms:.3f}ms {van_bpl / 1e6:.1f}MB -> {van_achieved:.1f} GB/s "
        f"(mode {van_modes[-1] if van_modes else 0}; refinement {avg_ref_ms:.3f}ms {ref_bpl / 1e6:.1f}MB -> "
        f"{ref_achieved:.1f} GB/s); "
        f"far scan={avg_scan_ms:.3f}ms {bytes_per_launch / 1e6:.1f}MB -> {achieved:.1f} GB/s; "
        f"probe GEMM {avg_probe_ms:.3f}ms -> {probe_tflops:.2f} TFLOP/s; "
        f"probe select + g_add {float(np.mean(select_ms)):.3f}ms")

    # the dominant scan kernel of the step (HIP events on the engine stream around it)
    W = c.padded_dim // 32
    lut = args.ip_kernel == "lut4"
    # the engine's matrix-core far scan (cross-query reuse is on; Bitwise estimator only)
    mfma_far = W in (2, 4, 6, 8, 16, 24, 32) and not lut
    narrow = W in (2, 6)  # P = 64, 192: the 16x16x32 kernel; the other widths the 16x16x64 one
    far_name = (f"far_mfma_kernel<{W}, 0> (far-pair RaBitQ scan, int8 MFMA 16x16x32 ip_int/ip_res" if narrow else
                f"far_mfma_wide_kernel<{W}, 0> (far-pair RaBitQ scan, int8 MFMA 16x16x64 ip_int, popcount "
                "ip_res for survivors")
    lows_name = (f"far_mfma_kernel<{W}, 2>" if narrow else f"far_mfma_wide_kernel<{W}, 2>")
    kernels = {
        "vanguard_query_kernel": {
            "kernel": f"vanguard_query_kernel<{W}, {'true' if avg_lows_ms > 0 else 'false'}> (fused per-query "
                      f"vanguard pass: {'streamed lower bounds' if avg_lows_ms > 0 else 'popcount lower bounds'}, "
                      "GPU refinement, top-k threshold)",
            "avg_launch_ms": round(avg_van_ms, 4), "bytes_per_launch": int(van_bpl), "achieved": van_achieved},
        "vs_refine_kernel": {
            "kernel": f"vs_refine_kernel<{W}> (staged vanguard pass: grid-wide refinement of the seeds and of the "
                      "candidate list, two launches; time and bytes are their sum)",
            "avg_launch_ms": round(avg_ref_ms, 4), "bytes_per_launch": int(ref_bpl), "achieved": ref_achieved},
        "vanguard_lows": {
            "kernel": f"{lows_name} (vanguard lower bounds on the matrix cores, cluster-major, units of 16 "
                      "same-cluster pairs)",
            "avg_launch_ms": round(avg_lows_ms, 4), "bytes_per_launch": int(lows_bpl), "achieved": lows_achieved,
            # of which written: a 4-byte bound per vanguard (query, vector), and for the staged
            # pass the minimum of each 4 of them
            "pair_vectors": int(np.mean(pair_vectors)) if pair_vectors else 0,
            "bytes_written": int((5 if van_modes and van_modes[-1] == 4 else 4) * np.mean(pair_vectors))
            if pair_vectors else 0},
        "far_mfma_kernel" if mfma_far else "scan_kernel": {
            "kernel": f"{far_name}, units of 16 same-cluster pairs)" if mfma_far else
                      f"scan_kernel<0, {4 if batch_q > 1 else 1}, 0, 1> (far-pair LUT4 scan, FP16 nibble tables in LDS)"
                      if lut else f"scan_kernel<{W}, {8 if batch_q > 1 else 1}, 0, 0> (far-pair RaBitQ popcount scan)",
            "avg_launch_ms": round(avg_scan_ms, 4), "bytes_per_launch": int(bytes_per_launch),
            "achieved": achieved},
    }
    if staged:
        # the staged pass is five kernels: its whole time and bytes are reported beside the
        # kernels, and its refinement kernel competes for the dominant one
        staged_pass = dict(kernels.pop("vanguard_query_kernel"))
        staged_pass["kernel"] = (f"staged vanguard pass (vs_seed_kernel, vs_refine_kernel<{W}> x2, vs_list_kernel, "
                                 "vs_merge_kernel): streamed lower bounds, GPU refinement, top-k threshold")
    else:
        kernels.pop("vs_refine_kernel")
    dom = max(kernels, key=lambda k: kernels[k]["avg_launch_ms"])
    # the counter profile applies to exactly this workload and mode
    traffic_key = {"config": args.config, "nprobe": nprobe, "topk": c.topk, "batch_q": batch_q,
                   "ip_kernel": args.ip_kernel, "gpu_final": bool(args.gpu_final),
                   "vanguard_mode": int(van_modes[-1]) if van_modes else 0}
    d = kernels[dom]
    roofline = {"bound": "hbm", "achieved": round(d["achieved"], 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(d["achieved"] / HBM_PEAK_GBPS, 4),
                "traffic": hbm_traffic(traffic_key, dom), "kernel": d["kernel"],
                "bytes_per_launch": d["bytes_per_launch"], "avg_launch_ms": d["avg_launch_ms"],
                "other": [dict(v, achieved=round(v["achieved"], 1)) for k, v in kernels.items() if k != dom] +
                         ([dict(staged_pass, achieved=round(staged_pass["achieved"], 1))] if staged else [])}

    extra = {}
    if not args.no_extra_lines and c.cfg in (4, 5):
        extra = extra_lines(eng, eng_cfg, queries, gt, c, nprobe, args, traffic_key)

    baseline = None
    if not args.no_cpu_baseline:
        sample = args.cpu_queries or (queries.shape[0] if c.padded_dim <= 128 else 2000)
        # the reference CPU path gets the whole 16-CPU share (nothing else runs beside it)
        baseline = cpu_baseline(index_path, queries, gt, c.topk, nprobe, args.cpu_threads or min(16, os.cpu_count() or 16),
                                workdir, sample)
        if baseline is not None:
            # the GPU's recall on exactly the queries the CPU baseline ran
            n_s = min(sample, queries.shape[0])
            baseline["gpu_recall_same_sample"] = round(recall_at_k(last_ids[:n_s], gt[:n_s], c.topk), 4)
            baseline["gpu_recall_at_10_same_sample"] = round(recall_at_k(last_ids[:n_s], gt[:n_s], 10), 4)

    line = {
        "metric": "QPS at recall@10>=0.9 (1 GPU)",
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic",
        "config": {"workload": c.describe(), "nprobe": nprobe, "recall_at_10": round(float(np.mean(recalls)), 4),
                   f"recall_at_{c.topk}": round(float(np.mean(recalls_k)), 4),
                   "qps_search_only": round(queries.shape[0] * args.steps / sum(times_search), 1),
                   "step_ms": [round(1000.0 * t, 3) for t in times],
                   "batch_q": batch_q, "vanguard": vanguard, "cpu_secondary_filter": c.secondary_filter,
                   "vanguard_mode": {0: "none", 1: "per-pair seed and recovery passes", 2: "fused per-query pass",
                                     3: "lows pass + fused per-query pass",
                                     4: "lows pass + staged pass"}.get(van_modes[-1] if van_modes else 0),
                   "lower_bound_scale": eng.lower_bound_scale, "gpu_final_topk": args.gpu_final,
                   "ip_kernel_type": args.ip_kernel,
                   "cpu_refine_threads": threads, "cpu_refine_isa": f"avx{ca.cpu_refine_isa()}",
                   "gpu_seed_thresholds": not args.no_gpu_seed, "gpu_refined_prefilter": not args.no_gpu_prefilter,
                   "query_chunk": chunk, "sweep": sweep},
        "roofline": roofline,
        **extra,
        "probe_mfma": probe_line,
        "cpu_baseline": baseline,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
