"""Python binding (ctypes) of the MI355X IVF-RaBitQ GPU-filter / CPU-refine engine.

Loads the in-tree shared libraries built by ``make -C cgcl-coraanns_amd``:

* ``lib/libcora_gpu.so`` — HIP kernels for gfx950 behind the C-ABI in include/cora_gpu.h;
* ``lib/libcoraanns.so`` — the C++ host (HybridIndex, CPU ex-code refinement, IVF file
  reader, index builder) behind the C-ABI in include/cora_host.h.

There is no fallback: if a library is missing every entry point raises
``EngineUnavailable``. This module only marshals arrays; all computation happens in the
native libraries.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_DIR = PKG_ROOT / "lib"
GPU_LIB = LIB_DIR / "libcora_gpu.so"
HOST_LIB = LIB_DIR / "libcoraanns.so"

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_LOGIC = 2
ERR_RUNTIME = 3
ERR_SPILL_EXHAUSTED = 4
ERR_OUT_OF_MEMORY = 5
ERR_QUEUE_STALLED = 6

FLAG_FROZEN_THRESHOLDS = 1
FLAG_FILTER_TIMING = 2
FLAG_CROSS_QUERY_REUSE = 4

DBG_ROTATED_QUERIES, DBG_K1XSUMQ, DBG_KBXSUMQ, DBG_Q_WIDTH, DBG_Q_PLANES = range(5)
DBG_PROBE_IDX, DBG_PROBE_GADD, DBG_PROBE_GERR, DBG_PAIRS, DBG_Q_WIDTH2 = range(5, 10)
DBG_SEED_DIST, DBG_THRESHOLDS, DBG_PROBE_DIST, DBG_VANGUARD_LOWS, DBG_LUT = 10, 11, 12, 13, 14
DBG_PROBE_FALLBACK = 15
DBG_STAGED_COUNTS = 16
FLAG_NO_GPU_SEED, FLAG_GPU_SEED_FROZEN, FLAG_NO_GPU_PREFILTER = 1 << 3, 1 << 4, 1 << 5
FLAG_PAIR_SEEDS = 1 << 6
FLAG_NO_MFMA_SCAN = 1 << 7
FLAG_FP32_GEMM = 1 << 8
FLAG_NO_VANGUARD_MFMA = 1 << 9
FLAG_VANGUARD_MFMA = 1 << 10
FLAG_GPU_FINAL = 1 << 11
FLAG_LUT4 = 1 << 12
FLAG_UNFUSED_PROBE = 1 << 13
FLAG_VANGUARD_ONE_PASS = 1 << 14
FLAG_VANGUARD_STAGED = 1 << 15
KERNEL_TYPES = {None: 0, "lut4": 1, "bitwise": 2}


class EngineUnavailable(RuntimeError):
    pass


class EngineError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class InvalidArgument(EngineError, ValueError):
    pass


class LogicError(EngineError):
    pass


def _raise(code, msg):
    if code == ERR_INVALID_ARGUMENT:
        raise InvalidArgument(code, msg)
    if code == ERR_LOGIC:
        raise LogicError(code, msg)
    raise EngineError(code, msg)


class cora_search_args(C.Structure):
    _fields_ = [("num_queries", C.c_uint32), ("topk", C.c_uint32), ("nprobe", C.c_uint32),
                ("batch_q", C.c_uint32), ("vanguard", C.c_uint32), ("flags", C.c_uint32),
                ("bound_scale", C.c_float)]


class cora_search_stats(C.Structure):
    _fields_ = [("produced", C.c_uint64), ("spilled", C.c_uint64), ("overflow", C.c_int32),
                ("stalled", C.c_int32), ("filter_ms", C.c_float), ("scan_ms", C.c_float),
                ("scan_bytes", C.c_uint64), ("scan_units", C.c_uint64),
                ("scan_vectors", C.c_uint64), ("probe_ms", C.c_float), ("probe_flops", C.c_uint64),
                ("pass_produced", C.c_uint64 * 3), ("seeded_queries", C.c_uint64),
                ("prefilter_dropped", C.c_uint64), ("seed_ms", C.c_float), ("recovery_ms", C.c_float),
                ("gpu_refined", C.c_uint64), ("vanguard_ms", C.c_float), ("vanguard_bytes", C.c_uint64),
                ("vanguard_lows_ms", C.c_float), ("vanguard_lows_bytes", C.c_uint64),
                ("vanguard_mode", C.c_int32), ("phase_ms", C.c_float * 4),
                ("vanguard_refine_ms", C.c_float), ("vanguard_refine_bytes", C.c_uint64)]


class cora_queue_view(C.Structure):
    _fields_ = [("items", C.c_void_p), ("progress", C.c_void_p), ("capacity", C.c_uint64),
                ("thresholds", C.POINTER(C.c_float)), ("abort_flag", C.POINTER(C.c_int))]


class cora_hybrid_config(C.Structure):
    _fields_ = [("profiling", C.c_int), ("candidate_stats", C.c_int),
                ("gpu_filter_timing", C.c_int), ("cross_query_reuse", C.c_int),
                ("cpu_secondary_filter", C.c_int), ("vanguard_size", C.c_uint64),
                ("queue_capacity", C.c_uint64), ("queue_spill_capacity", C.c_uint64),
                ("metric", C.c_int), ("frozen_thresholds", C.c_int), ("cpu_threads", C.c_int),
                ("gpu_seed_refine", C.c_int), ("gpu_refine_filter", C.c_int), ("extra_flags", C.c_uint32),
                ("lower_bound_scale", C.c_float), ("gpu_final_topk", C.c_int), ("ip_kernel_type", C.c_int)]


class cora_hybrid_stats(C.Structure):
    _fields_ = [("submitted", C.c_uint64), ("spilled", C.c_uint64), ("refined", C.c_uint64),
                ("gpu_filter_ms", C.c_float), ("scan_ms", C.c_float), ("scan_bytes", C.c_uint64),
                ("scan_units", C.c_uint64), ("scan_vectors", C.c_uint64), ("probe_ms", C.c_float),
                ("probe_flops", C.c_uint64), ("pass_produced", C.c_uint64 * 3),
                ("seeded_queries", C.c_uint64), ("prefilter_dropped", C.c_uint64),
                ("seed_ms", C.c_float), ("recovery_ms", C.c_float), ("gpu_refined", C.c_uint64),
                ("vanguard_ms", C.c_float), ("vanguard_bytes", C.c_uint64),
                ("vanguard_lows_ms", C.c_float), ("vanguard_lows_bytes", C.c_uint64),
                ("vanguard_mode", C.c_int32), ("phase_ms", C.c_float * 4),
                ("vanguard_refine_ms", C.c_float), ("vanguard_refine_bytes", C.c_uint64)]


class cora_ivf_info(C.Structure):
    _fields_ = [("num", C.c_uint64), ("dim", C.c_uint64), ("padded_dim", C.c_uint64),
                ("nlist", C.c_uint64), ("ex_bits", C.c_uint64), ("max_cluster", C.c_uint64),
                ("metric", C.c_int), ("centroid_storage", C.c_int)]


class cora_ivf_arrays(C.Structure):
    _fields_ = [("centroids", C.c_void_p), ("rotator", C.c_void_p), ("short_data", C.c_void_p),
                ("short_factors", C.c_void_p), ("long_codes", C.c_void_p),
                ("ex_factors", C.c_void_p), ("ids", C.c_void_p), ("cluster_sizes", C.c_void_p)]


class cora_ring_test(C.Structure):
    _fields_ = [("capacity", C.c_uint64), ("spill_capacity", C.c_uint64),
                ("producers", C.c_uint32), ("consumers", C.c_uint32), ("queries", C.c_uint32),
                ("per_query", C.c_uint32), ("topk", C.c_uint32), ("secondary_filter", C.c_int),
                ("submitted", C.c_uint64), ("spilled", C.c_uint64), ("refined", C.c_uint64),
                ("overflow", C.c_int)]


_P = C.c_void_p
_U64 = C.c_uint64
_I = C.c_int

GPU_SIGNATURES = {
    "cora_gpu_create": [C.POINTER(C.c_void_p), _I],
    "cora_gpu_destroy": [_P],
    "cora_gpu_last_error": [_P, C.c_char_p, C.c_size_t],
    "cora_gpu_load_index": [_P, _U64, _U64, _U64, _U64, _U64, _I, _P, _P, _P, _P, _P],
    "cora_gpu_load_excodes": [_P, _P, _P],
    "cora_gpu_set_queue": [_P, _U64, _U64],
    "cora_gpu_prepare_workspace": [_P, _U64, _U64, _U64, _U64],
    "cora_gpu_free_workspace": [_P],
    "cora_gpu_queue_view": [_P, C.POINTER(cora_queue_view)],
    "cora_gpu_reset": [_P, _P, _U64],
    "cora_gpu_query_staging": [_P, C.POINTER(_P)],
    "cora_gpu_final_results": [_P, _P, _P],
    "cora_gpu_launch_search": [_P, C.POINTER(cora_search_args)],
    "cora_gpu_wait_host_inputs": [_P, C.POINTER(_P), C.POINTER(_P), C.POINTER(_P)],
    "cora_gpu_sync": [_P, C.POINTER(cora_search_stats)],
    "cora_gpu_capture_thresholds": [_P, _P, _U64],
    "cora_gpu_seed_thresholds": [_P, _P, _U64],
    "cora_gpu_index_info": [_P, _P, _P, _P, _P, _P],
    "cora_gpu_debug_read": [_P, _I, _P, _U64],
    "cora_gpu_debug_dense": [_P, _P, _P, _P, _U64],
    "cora_tool_last_error": [],
    "cora_tool_rotate": [_P, _U64, _U64, _P, _U64, _P, _I],
    "cora_tool_quantize": [_P, _U64, _U64, _P, _U64, _P, _U64, _P, _I, _P, _P, _P, _P, _I],
    "cora_tool_kmeans": [_P, _U64, _U64, _U64, C.c_uint32, _U64, _P, _I],
    "cora_tool_assign": [_P, _U64, _U64, _P, _U64, _P, _I],
    "cora_tool_topk": [_P, _U64, _P, _U64, _U64, _U64, _I, _P, _I],
    "cora_tool_assign_noalloc": [_P, _U64, _U64, _P, _U64, _P, _I],
}

HOST_SIGNATURES = {
    "cora_host_last_error": [],
    "cora_hybrid_create": [C.POINTER(C.c_void_p), _I],
    "cora_hybrid_destroy": [_P],
    "cora_hybrid_configure": [_P, C.POINTER(cora_hybrid_config)],
    "cora_hybrid_load": [_P, _U64, _U64, _U64, _U64, _U64, _P, _P, _P, _P, _P, _P, _P, _P],
    "cora_hybrid_enable_exact_refine": [_P, _P, _U64, _U64, _U64, _U64],
    "cora_hybrid_prepare": [_P, _U64, _U64, _U64],
    "cora_hybrid_free_workspace": [_P],
    "cora_hybrid_reset": [_P, _P, _U64],
    "cora_hybrid_search": [_P, _P, _U64, _U64, _U64, _P, _P, _I],
    "cora_hybrid_stats_get": [_P, C.POINTER(cora_hybrid_stats)],
    "cora_hybrid_capture_thresholds": [_P, _P, _U64],
    "cora_hybrid_seed_thresholds": [_P, _P, _U64],
    "cora_hybrid_set_vanguard_size": [_P, _U64],
    "cora_hybrid_gpu": [_P],
    "cora_hybrid_lower_bound_scale": [_P],
    "cora_ivf_load": [C.c_char_p, _I, C.POINTER(C.c_void_p)],
    "cora_ivf_info_get": [_P, C.POINTER(cora_ivf_info)],
    "cora_ivf_arrays_get": [_P, C.POINTER(cora_ivf_arrays)],
    "cora_ivf_free": [_P],
    "cora_build_ivf": [_P, _P, _P, _P, _U64, _U64, _U64, _U64, _U64, _I, _I, C.c_char_p],
    "cora_build_ivf_gpu": [_P, _P, _P, _P, _U64, _U64, _U64, _U64, _U64, _I, _I, _I, C.c_char_p],
    "cora_quantize_rows": [_P, _P, _U64, _U64, _U64, _I, _P, _P, _P, _P],
    "cora_excode_ip7": [_P, _P, _U64, _U64, _P],
    "cora_cpu_refine_isa": [],
    "cora_gaussian_mixture": [_P, _U64, _U64, _P, _U64, _U64, _I, _I, _P, _P],
    "cora_test_ring": [C.POINTER(cora_ring_test), _P, _P],
}

_gpu = None
_host = None


def _load():
    global _gpu, _host
    if _host is not None:
        return _gpu, _host
    for p in (GPU_LIB, HOST_LIB):
        if not p.exists():
            raise EngineUnavailable(f"{p} is not built; run __graft_entry__.build() or make -C cgcl-coraanns_amd")
    gpu = C.CDLL(str(GPU_LIB), mode=C.RTLD_GLOBAL)
    host = C.CDLL(str(HOST_LIB))
    for lib, sigs in ((gpu, GPU_SIGNATURES), (host, HOST_SIGNATURES)):
        for name, args in sigs.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = C.c_int
    host.cora_host_last_error.restype = C.c_char_p
    gpu.cora_tool_last_error.restype = C.c_char_p
    host.cora_hybrid_gpu.restype = C.c_void_p
    host.cora_hybrid_lower_bound_scale.restype = C.c_float
    _gpu, _host = gpu, host
    return gpu, host


def libs():
    return _load()


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _host_check(rc):
    if rc != OK:
        _raise(rc, _load()[1].cora_host_last_error().decode())


def _gpu_check(engine, rc):
    if rc != OK:
        buf = C.create_string_buffer(512)
        _load()[0].cora_gpu_last_error(engine, buf, 512)
        _raise(rc, buf.value.decode())


class IvfIndex:
    """An IVF-RaBitQ index file (reference on-disk format) adapted like SearchData."""

    def __init__(self, path, include_extended=True):
        _, host = _load()
        h = C.c_void_p()
        _host_check(host.cora_ivf_load(str(path).encode(), 1 if include_extended else 0, C.byref(h)))
        self._h = h
        info = cora_ivf_info()
        host.cora_ivf_info_get(h, C.byref(info))
        self.num, self.dim, self.padded_dim = info.num, info.dim, info.padded_dim
        self.nlist, self.ex_bits, self.max_cluster, self.metric = (info.nlist, info.ex_bits,
                                                                   info.max_cluster, info.metric)
        self.centroid_storage = "hnsw_sidecar" if info.centroid_storage == 1 else "embedded"
        ar = cora_ivf_arrays()
        host.cora_ivf_arrays_get(h, C.byref(ar))
        P, n, nl = self.padded_dim, self.num, self.nlist
        lc = P * self.ex_bits // 8

        def view(ptr, ctype, count, shape):
            if not ptr:
                return None
            buf = (ctype * count).from_address(ptr)
            return np.frombuffer(buf, dtype=np.dtype(ctype)).reshape(shape)

        self.centroids = view(ar.centroids, C.c_float, nl * P, (nl, P))
        self.rotator = view(ar.rotator, C.c_float, self.dim * P, (self.dim, P))
        self.short_data = view(ar.short_data, C.c_uint32, n * P // 32, (n * P // 32,))
        self.short_factors = view(ar.short_factors, C.c_float, n * 3, (n, 3))
        self.long_codes = view(ar.long_codes, C.c_uint8, n * lc, (n, lc))
        self.ex_factors = view(ar.ex_factors, C.c_float, n * 2, (n, 2))
        self.ids = view(ar.ids, C.c_uint32, n, (n,))
        self.cluster_sizes = view(ar.cluster_sizes, C.c_uint64, nl, (nl,))

    def close(self):
        if getattr(self, "_h", None):
            _load()[1].cora_ivf_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HybridIndex:
    """coraanns::HybridIndex through the host C-ABI (include/cora_host.h)."""

    def __init__(self, device=0, *, profiling=False, candidate_stats=False, gpu_filter_timing=False,
                 cross_query_reuse=True, cpu_secondary_filter=True, vanguard_size=5,
                 queue_capacity=None, queue_spill_capacity=None, metric=0, frozen_thresholds=False,
                 cpu_threads=0, gpu_seed_refine=True, gpu_refine_filter=True, extra_flags=0,
                 lower_bound_scale=None, gpu_final_topk=False, ip_kernel_type=None):
        _, host = _load()
        h = C.c_void_p()
        _host_check(host.cora_hybrid_create(C.byref(h), device))
        self._h = h
        self._keep = []
        self.configure(profiling=profiling, candidate_stats=candidate_stats,
                       gpu_filter_timing=gpu_filter_timing, cross_query_reuse=cross_query_reuse,
                       cpu_secondary_filter=cpu_secondary_filter, vanguard_size=vanguard_size,
                       queue_capacity=queue_capacity, queue_spill_capacity=queue_spill_capacity,
                       metric=metric, frozen_thresholds=frozen_thresholds, cpu_threads=cpu_threads,
                       gpu_seed_refine=gpu_seed_refine, gpu_refine_filter=gpu_refine_filter,
                       extra_flags=extra_flags, lower_bound_scale=lower_bound_scale,
                       gpu_final_topk=gpu_final_topk, ip_kernel_type=ip_kernel_type)

    def configure(self, *, profiling=False, candidate_stats=False, gpu_filter_timing=False,
                  cross_query_reuse=True, cpu_secondary_filter=True, vanguard_size=5,
                  queue_capacity=None, queue_spill_capacity=None, metric=0, frozen_thresholds=False,
                  cpu_threads=0, gpu_seed_refine=True, gpu_refine_filter=True, extra_flags=0,
                  lower_bound_scale=None, gpu_final_topk=False, ip_kernel_type=None):
        """lower_bound_scale: multiplier of the filter's error term (None keeps the
        engine's default; 1.0 is the reference Bitwise producer's bound). ip_kernel_type:
        None keeps the current one (Bitwise by default), "lut4" or "bitwise"."""
        cfg = cora_hybrid_config(int(profiling), int(candidate_stats), int(gpu_filter_timing),
                                 int(cross_query_reuse), int(cpu_secondary_filter), int(vanguard_size),
                                 int(queue_capacity or 0),
                                 (1 << 64) - 1 if queue_spill_capacity is None else int(queue_spill_capacity),
                                 int(metric), int(frozen_thresholds), int(cpu_threads),
                                 int(gpu_seed_refine), int(gpu_refine_filter), int(extra_flags),
                                 float(lower_bound_scale or 0.0), int(gpu_final_topk),
                                 KERNEL_TYPES[ip_kernel_type])
        _host_check(_load()[1].cora_hybrid_configure(self._h, C.byref(cfg)))

    def load_from_raw_pointers(self, num_vecs, dim, padded_dim, n_centroids, ex_bits, centroids,
                               rotator, short_data, short_factors, long_codes, ex_factors, ids,
                               cluster_sizes):
        arrs = [np.ascontiguousarray(centroids, np.float32), np.ascontiguousarray(rotator, np.float32),
                np.ascontiguousarray(short_data, np.uint32), np.ascontiguousarray(short_factors, np.float32),
                None if long_codes is None else np.ascontiguousarray(long_codes, np.uint8),
                None if ex_factors is None else np.ascontiguousarray(ex_factors, np.float32),
                np.ascontiguousarray(ids, np.uint32), np.ascontiguousarray(cluster_sizes, np.uint64)]
        self._keep.append(arrs)  # long codes / ex factors / ids are borrowed by the engine
        _host_check(_load()[1].cora_hybrid_load(self._h, num_vecs, dim, padded_dim, n_centroids, ex_bits,
                                                *[_ptr(a) for a in arrs]))

    def load_ivf(self, ivf: IvfIndex):
        self._keep.append(ivf)
        self.load_from_raw_pointers(ivf.num, ivf.dim, ivf.padded_dim, ivf.nlist, ivf.ex_bits,
                                    ivf.centroids, ivf.rotator, ivf.short_data, ivf.short_factors,
                                    ivf.long_codes, ivf.ex_factors, ivf.ids, ivf.cluster_sizes)

    def enable_exact_refine(self, base: np.ndarray):
        base = np.ascontiguousarray(base, np.float32)
        self._keep.append(base)
        _host_check(_load()[1].cora_hybrid_enable_exact_refine(
            self._h, _ptr(base.view(np.uint8)), base.shape[0], base.shape[1], base.shape[1] * 4, 0))

    def prepare_workspace(self, max_queries, max_topk, max_nprobe):
        _host_check(_load()[1].cora_hybrid_prepare(self._h, max_queries, max_topk, max_nprobe))

    def free_workspace(self):
        _load()[1].cora_hybrid_free_workspace(self._h)

    def set_vanguard_size(self, size):
        _host_check(_load()[1].cora_hybrid_set_vanguard_size(self._h, size))

    def reset_buffer(self, queries):
        q = np.ascontiguousarray(queries, np.float32)
        _host_check(_load()[1].cora_hybrid_reset(self._h, _ptr(q), q.shape[0]))

    def search(self, queries, topk, nprobe, batch_q=4):
        q = np.ascontiguousarray(queries, np.float32)
        nq = q.shape[0]
        d = np.empty((nq, topk), np.float32)
        i = np.empty((nq, topk), np.uint32)
        _host_check(_load()[1].cora_hybrid_search(self._h, _ptr(q), nq, topk, nprobe, _ptr(d), _ptr(i),
                                                  batch_q))
        return d, i

    def search_all(self, queries, topk, nprobe, batch_q=4, chunk=65535):
        """reset_buffer + search per query chunk (reference apps/search.cpp:223-241)."""
        q = np.ascontiguousarray(queries, np.float32)
        ds, ids = [], []
        for b in range(0, q.shape[0], chunk):
            self.reset_buffer(q[b:b + chunk])
            d, i = self.search(q[b:b + chunk], topk, nprobe, batch_q)
            ds.append(d)
            ids.append(i)
        return np.vstack(ds), np.vstack(ids)

    def stats(self):
        s = cora_hybrid_stats()
        _load()[1].cora_hybrid_stats_get(self._h, C.byref(s))
        out = {k: getattr(s, k) for k, _ in cora_hybrid_stats._fields_}
        out["pass_produced"] = list(out["pass_produced"])
        out["phase_ms"] = list(out["phase_ms"])
        return out

    def capture_thresholds(self, nq):
        out = np.empty(nq, np.float32)
        _host_check(_load()[1].cora_hybrid_capture_thresholds(self._h, _ptr(out), nq))
        return out

    def seed_thresholds(self, thr):
        t = np.ascontiguousarray(thr, np.float32)
        _host_check(_load()[1].cora_hybrid_seed_thresholds(self._h, _ptr(t), t.shape[0]))

    @property
    def lower_bound_scale(self):
        return float(_load()[1].cora_hybrid_lower_bound_scale(self._h))

    @property
    def gpu(self):
        return _load()[1].cora_hybrid_gpu(self._h)

    def debug_read(self, which, shape, dtype):
        out = np.empty(shape, dtype)
        eng = self.gpu
        _gpu_check(eng, _load()[0].cora_gpu_debug_read(eng, which, _ptr(out), out.nbytes))
        return out

    def debug_dense(self, nq, nprobe, max_cluster):
        """ip_int <b,qint>, residual <b,qres> and low distance of every probed vector,
        [nq][nprobe][max_cluster]."""
        ip = np.full((nq, nprobe, max_cluster), -(1 << 30), np.int32)
        ip2 = np.full((nq, nprobe, max_cluster), -(1 << 30), np.int32)
        low = np.full((nq, nprobe, max_cluster), np.nan, np.float32)
        eng = self.gpu
        _gpu_check(eng, _load()[0].cora_gpu_debug_dense(eng, _ptr(ip), _ptr(ip2), _ptr(low), ip.size))
        return ip, ip2, low

    def close(self):
        if getattr(self, "_h", None):
            _load()[1].cora_hybrid_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def build_ivf(path, rotated_data, rotated_centroids, assignments, rotator, metric=0, threads=0):
    """Write an IVF-RaBitQ index (reference format, 8-bit: 1 sign + 7 ex bits)."""
    x = np.ascontiguousarray(rotated_data, np.float32)
    c = np.ascontiguousarray(rotated_centroids, np.float32)
    a = np.ascontiguousarray(assignments, np.uint32)
    r = np.ascontiguousarray(rotator, np.float32)
    _host_check(_load()[1].cora_build_ivf(_ptr(x), _ptr(c), _ptr(a), _ptr(r), x.shape[0], r.shape[0],
                                          x.shape[1], c.shape[0], 7, metric, threads, str(path).encode()))


def build_ivf_gpu(path, data, rotated_centroids, assignments, rotator, metric=0, device=0, threads=0):
    """The same index as build_ivf(path, data @ rotator, ...) with the rotation and the RaBitQ
    quantisation on the GPU (bit-identical to build_ivf on the GPU-rotated rows)."""
    x = np.ascontiguousarray(data, np.float32)
    c = np.ascontiguousarray(rotated_centroids, np.float32)
    a = np.ascontiguousarray(assignments, np.uint32)
    r = np.ascontiguousarray(rotator, np.float32)
    _host_check(_load()[1].cora_build_ivf_gpu(_ptr(x), _ptr(c), _ptr(a), _ptr(r), x.shape[0], x.shape[1],
                                              r.shape[1], c.shape[0], 7, metric, device, threads,
                                              str(path).encode()))


def quantize_rows(rows, centroid, metric=0, ex_bits=7):
    rows = np.ascontiguousarray(rows, np.float32)
    centroid = np.ascontiguousarray(centroid, np.float32)
    n, P = rows.shape
    bits = np.empty((n, P), np.uint8)
    f1 = np.empty((n, 3), np.float32)
    ex = np.empty((n, P), np.uint8)
    f2 = np.empty((n, 2), np.float32)
    _host_check(_load()[1].cora_quantize_rows(_ptr(rows), _ptr(centroid), n, P, ex_bits, metric,
                                              _ptr(bits), _ptr(f1), _ptr(ex), _ptr(f2)))
    return bits, f1, ex, f2


def gaussian_mixture(centers, sd, n, seed, normalize=False, threads=0):
    """n rows centers[label] + sd * z (z standard normal), optionally L2-normalised, from
    counter-based streams: the same output for any thread count."""
    centers = np.ascontiguousarray(centers, np.float32)
    sd = np.ascontiguousarray(sd, np.float32)
    k, dim = centers.shape
    if dim % 2 or sd.shape != (dim,):
        raise ValueError("gaussian_mixture: dim must be even and sd of length dim")
    out = np.empty((n, dim), np.float32)
    _host_check(_load()[1].cora_gaussian_mixture(_ptr(centers), k, dim, _ptr(sd), n, seed,
                                                 int(normalize), threads, _ptr(out), None))
    return out


def excode_ip7(q, packed):
    q = np.ascontiguousarray(q, np.float32)
    packed = np.ascontiguousarray(packed, np.uint8)
    out = np.empty(packed.shape[0], np.float32)
    _host_check(_load()[1].cora_excode_ip7(_ptr(q), _ptr(packed), packed.shape[0], q.shape[0], _ptr(out)))
    return out


def ring_test(capacity, spill_capacity, producers, consumers, queries, per_query, topk,
              secondary_filter=False):
    t = cora_ring_test(capacity, spill_capacity, producers, consumers, queries, per_query, topk,
                       int(secondary_filter), 0, 0, 0, 0)
    d = np.empty((queries, topk), np.float32)
    i = np.empty((queries, topk), np.uint32)
    rc = _load()[1].cora_test_ring(C.byref(t), _ptr(d), _ptr(i))
    _host_check(rc)
    return t, d, i


def _tool_check(rc):
    if rc != OK:
        _raise(rc, _load()[0].cora_tool_last_error().decode())


def gpu_rotate(x, R, device=0):
    x = np.ascontiguousarray(x, np.float32)
    R = np.ascontiguousarray(R, np.float32)
    out = np.empty((x.shape[0], R.shape[1]), np.float32)
    _tool_check(_load()[0].cora_tool_rotate(_ptr(x), x.shape[0], x.shape[1], _ptr(R), R.shape[1], _ptr(out),
                                            device))
    return out


def gpu_kmeans(x, k, iters=20, seed=0, device=0):
    x = np.ascontiguousarray(x, np.float32)
    c = np.empty((k, x.shape[1]), np.float32)
    _tool_check(_load()[0].cora_tool_kmeans(_ptr(x), x.shape[0], x.shape[1], k, iters, seed, _ptr(c), device))
    return c


def gpu_assign(x, centroids, device=0):
    x = np.ascontiguousarray(x, np.float32)
    c = np.ascontiguousarray(centroids, np.float32)
    a = np.empty(x.shape[0], np.uint32)
    _tool_check(_load()[0].cora_tool_assign(_ptr(x), x.shape[0], x.shape[1], _ptr(c), c.shape[0], _ptr(a),
                                            device))
    return a


def gpu_topk(base, queries, k, metric=0, device=0):
    b = np.ascontiguousarray(base, np.float32)
    q = np.ascontiguousarray(queries, np.float32)
    ids = np.empty((q.shape[0], k), np.uint32)
    _tool_check(_load()[0].cora_tool_topk(_ptr(b), b.shape[0], _ptr(q), q.shape[0], q.shape[1], k, metric,
                                          _ptr(ids), device))
    return ids


def cpu_refine_isa():
    """Vector width (512 or 256) of the CPU refinement's ex-code inner product."""
    return _load()[1].cora_cpu_refine_isa()


def gpu_available():
    """True when a HIP device is visible (does not initialise torch)."""
    try:
        gpu, _ = _load()
    except EngineUnavailable:
        return False
    h = C.c_void_p()
    if gpu.cora_gpu_create(C.byref(h), 0) != OK:
        return False
    gpu.cora_gpu_destroy(h)
    return True
