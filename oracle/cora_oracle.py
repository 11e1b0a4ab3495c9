"""CPU oracle for the IVF-RaBitQ GPU-filter / CPU-refine search path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker: the product path
(cgcl-coraanns_amd/) never imports, links or runs anything under oracle/.

Each function restates one step of the reference's algorithm in numpy, citing the
reference file:line it follows (paths relative to the reference repository root).
How each function is pinned (golden vectors written by the reference's own code,
closed forms, brute force) is listed in the PINNED table at the end of this module;
a function not listed there is "parity unpinned".
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

F32_MAX = np.float32(np.finfo(np.float32).max)

# FastScan interleave of 16 vectors inside a 32-vector block
# (third_party/rabitq/include/rabitqlib/fastscan/fastscan.hpp:40-42).
K_PERM0 = np.array([0, 8, 1, 9, 2, 10, 3, 11, 4, 12, 5, 13, 6, 14, 7, 15], dtype=np.int64)


# --------------------------------------------------------------------------------------
# On-disk IVF format (third_party/rabitq/include/rabitqlib/index/ivf/ivf.hpp:403-539,
# quantization/data_layout.hpp:57-176)
# --------------------------------------------------------------------------------------
@dataclass
class IVFFile:
    num: int
    dim: int
    padded_dim: int
    nlist: int
    ex_bits: int
    rotator_type: int
    metric: int  # 0 = L2, 1 = IP (defines.hpp:65)
    cluster_sizes: np.ndarray  # u64 [nlist]
    rotator: np.ndarray  # f32 [dim, padded_dim], row-major; q' = q @ R (rotator.hpp:108-112)
    centroids: np.ndarray  # f32 [nlist, padded_dim] (rotated)
    batch_data: np.ndarray  # u8, per cluster ceil(n/32) blocks of (P*4 + 32*12) bytes
    ex_data: np.ndarray  # u8 [num, P*ex/8 + 8]
    ids: np.ndarray  # u32 [num], cluster order


def round_up(x, m):
    return (x + m - 1) // m * m


HNSW_HEADER = struct.Struct("<6QiI3QdQ")  # hnswlib saveIndex header (hnswalg.h:689-702)


def read_hnsw_centroids(path, nlist: int, P: int) -> np.ndarray:
    """Centroids of an HNSW sidecar ("<index>.hnsw", HNSWInitializer::save/load,
    initializer.hpp:255-279). hnswlib's saveIndex (hnswalg.h:685-713) writes a header of
    offsetLevel0_, max_elements_, cur_element_count, size_data_per_element_, label_offset_,
    offsetData_ (size_t), maxlevel_ (int), enterpoint_node_ (u32), maxM_, maxM0_, M_ (size_t),
    mult_ (double), ef_construction_ (size_t); then cur_element_count level-0 elements of
    size_data_per_element_ bytes (vector at offsetData_, size_t label at label_offset_); then
    per element a u32 byte count and its upper-level links. Centroid c is the vector labelled
    c (rebuild_label_to_internal, initializer.hpp:181-198)."""
    raw = np.fromfile(path, dtype=np.uint8)
    if raw.size < HNSW_HEADER.size:
        raise ValueError("Index seems to be corrupted or unsupported")
    (_, _, count, per, label_off, data_off, _, _, _, _, _, _, _) = HNSW_HEADER.unpack_from(raw.tobytes(), 0)
    if count != nlist:
        raise ValueError("HNSW centroid count does not match the IVF cluster count")
    if label_off - data_off != 4 * P or label_off + 8 > per:
        raise ValueError("HNSW sidecar vectors are not padded_dim floats")
    off = HNSW_HEADER.size
    if off + count * per > raw.size:
        raise ValueError("Index seems to be corrupted or unsupported")
    # the loadIndex check (hnswalg.h:754-770): the link lists end exactly at the file end
    pos = off + count * per
    for _ in range(count):
        if pos + 4 > raw.size:
            raise ValueError("Index seems to be corrupted or unsupported")
        pos += 4 + int(raw[pos:pos + 4].view(np.uint32)[0])
    if pos != raw.size:
        raise ValueError("Index seems to be corrupted or unsupported")
    el = raw[off:off + count * per].reshape(count, per)
    labels = el[:, label_off:label_off + 8].copy().view(np.uint64).reshape(count)
    if np.any(labels >= nlist) or np.unique(labels).size != count:
        raise ValueError("Invalid or duplicate HNSW centroid label")
    cent = np.empty((nlist, P), np.float32)
    cent[labels.astype(np.int64)] = el[:, data_off:data_off + 4 * P].copy().view(np.float32).reshape(count, P)
    return cent


def _centroid_layout(remaining: int, payload: int, nlist: int, P: int) -> str:
    """Stored centroid representation from the bytes left after the rotator
    (ivf.hpp:487-520)."""
    if remaining == payload + 4 * P * nlist:
        return "embedded"
    if remaining == payload:
        return "hnsw_sidecar"
    raise ValueError("IVF index size does not match a supported centroid layout")


def read_ivf(path) -> IVFFile:
    """IVF::load (ivf.hpp:447-539): header of four size_t + two u8, cluster sizes,
    MatrixRotator [dim x P] (rotator.hpp:89-94), the centroids (embedded flat centroids,
    initializer.hpp:147-169, or none here and an HNSW sidecar "<path>.hnsw"), batch data,
    ex data, ids. P = round_up(dim, 64) (ivf.hpp:242, rotator.hpp:375-405)."""
    raw = np.fromfile(path, dtype=np.uint8)
    num, dim, nlist, ex_bits = struct.unpack_from("<4Q", raw, 0)
    rtype, metric = raw[32], raw[33]
    off = 34
    sizes = np.frombuffer(raw, dtype=np.uint64, count=nlist, offset=off).copy()
    off += 8 * nlist
    P = round_up(dim, 64)
    rot = np.frombuffer(raw, dtype=np.float32, count=dim * P, offset=off).reshape(dim, P).copy()
    off += 4 * dim * P
    blocks = int(sum((int(s) + 31) // 32 for s in sizes))
    batch_bytes = blocks * (P * 32 // 8 + 32 * 12)
    ex_stride = P * ex_bits // 8 + 8 if ex_bits > 0 else 0
    payload = batch_bytes + ex_stride * num + 4 * num
    if _centroid_layout(raw.size - off, payload, nlist, P) == "embedded":
        cent = np.frombuffer(raw, dtype=np.float32, count=nlist * P, offset=off).reshape(nlist, P).copy()
        off += 4 * P * nlist
    else:
        cent = read_hnsw_centroids(str(path) + ".hnsw", nlist, P)
    batch = raw[off:off + batch_bytes].copy()
    off += batch_bytes
    ex = raw[off:off + ex_stride * num].reshape(num, ex_stride).copy()
    off += ex_stride * num
    ids = np.frombuffer(raw, dtype=np.uint32, count=num, offset=off).copy()
    if int(sizes.sum()) != num:
        raise ValueError("cluster sizes do not sum to num")
    return IVFFile(num, dim, P, nlist, ex_bits, int(rtype), int(metric), sizes, rot, cent, batch, ex, ids)


def fastscan_pack(compact: np.ndarray, P: int) -> np.ndarray:
    """fastscan::pack_codes (fastscan.hpp:69-106). compact: u8 [n, P/8] big-endian bit
    packing of the sign code (space.hpp pack_binary: dim j -> bit 7-j%8 of byte j/8).
    Returns blocks of 32 vectors x P/8 columns, each column 32 bytes."""
    n = compact.shape[0]
    nrd = round_up(n, 32)
    cols = P // 8
    padded = np.zeros((nrd, cols), dtype=np.uint8)
    padded[:n] = compact
    out = np.zeros((nrd // 32, cols, 32), dtype=np.uint8)
    for b in range(nrd // 32):
        blk = padded[b * 32:(b + 1) * 32]  # [32, cols]
        hi = blk >> 4
        lo = blk & 15
        for j in range(16):
            out[b, :, j] = hi[K_PERM0[j]] | (hi[K_PERM0[j] + 16] << 4)
            out[b, :, j + 16] = lo[K_PERM0[j]] | (lo[K_PERM0[j] + 16] << 4)
    return out.reshape(-1)


def unpack_fastscan_bits(codes: np.ndarray, P: int, batch_len: int) -> np.ndarray:
    """Sign bits of one 32-vector FastScan block as u8 {0,1} [batch_len, P]
    (search_data.cpp:60-72): byte = codes[(d/8)*32 + (d%8 < 4 ? 0 : 16) + invPerm0[v%16]],
    nibble = v < 16 ? low : high, bit = (nibble >> (3 - d%4)) & 1."""
    inv = np.empty(16, dtype=np.int64)
    inv[K_PERM0] = np.arange(16)
    d = np.arange(P)
    v = np.arange(batch_len)
    byte_idx = (d[None, :] // 8) * 32 + np.where(d[None, :] % 8 < 4, 0, 16) + inv[v[:, None] % 16]
    byte = codes[byte_idx]
    nib = np.where(v[:, None] < 16, byte & 0x0F, byte >> 4)
    return ((nib >> (3 - (d[None, :] % 4))) & 1).astype(np.uint8)


def bits_to_words_msb(bits: np.ndarray) -> np.ndarray:
    """u8 {0,1} [n, P] -> u32 [n, P/32], dim 32w+l at bit 31-l of word w
    (search_data.cpp:71; query_kernels.cuh:115-116 'dimension-0-at-bit-31')."""
    n, P = bits.shape
    b = bits.reshape(n, P // 32, 32).astype(np.uint64)
    sh = (31 - np.arange(32)).astype(np.uint64)
    return (b << sh).sum(axis=2).astype(np.uint32)


def words_msb_to_bits(words: np.ndarray) -> np.ndarray:
    n, W = words.shape
    sh = (31 - np.arange(32)).astype(np.uint32)
    return ((words[:, :, None] >> sh) & 1).reshape(n, W * 32).astype(np.uint8)


@dataclass
class SearchData:
    centroids: np.ndarray  # f32 [nl, P]
    rotator: np.ndarray  # f32 [dim, P]
    short_data: np.ndarray  # u32 [N*P/32], per-cluster word-major: [start*W + w*n + i]
    short_factors: np.ndarray  # f32 [N, 3] (f_add, f_rescale, f_error)
    long_codes: np.ndarray  # u8 [N, P*ex/8]
    ex_factors: np.ndarray  # f32 [N, 2] (f_add_ex, f_rescale_ex)
    ids: np.ndarray  # u32 [N]
    cluster_sizes: np.ndarray  # u64 [nl]
    cluster_start: np.ndarray  # i64 [nl]
    bits: np.ndarray  # u8 [N, P] sign bits in cluster order (derived, for checking)


def search_data(ivf: IVFFile) -> SearchData:
    """SearchData::SearchData (search_data.cpp:9-127): unpack each cluster's FastScan
    blocks into per-cluster word-major u32 words (MSB = lowest dim), AoS factors,
    and compact the ex-codes (drop the two trailing ex factors of each record)."""
    P, W = ivf.padded_dim, ivf.padded_dim // 32
    N = ivf.num
    block_bytes = P * 4 + 32 * 12
    bits = np.zeros((N, P), dtype=np.uint8)
    factors = np.zeros((N, 3), dtype=np.float32)
    short = np.zeros(N * W, dtype=np.uint32)
    starts = np.zeros(ivf.nlist, dtype=np.int64)
    g = 0
    boff = 0
    for c in range(ivf.nlist):
        n = int(ivf.cluster_sizes[c])
        starts[c] = g
        for i in range(0, n, 32):
            blen = min(32, n - i)
            blk = ivf.batch_data[boff:boff + block_bytes]
            fl = blk[P * 4:].view(np.float32)
            bits[g + i:g + i + blen] = unpack_fastscan_bits(blk[:P * 4], P, blen)
            factors[g + i:g + i + blen, 0] = fl[0:blen]
            factors[g + i:g + i + blen, 1] = fl[32:32 + blen]
            factors[g + i:g + i + blen, 2] = fl[64:64 + blen]
            boff += block_bytes
        words = bits_to_words_msb(bits[g:g + n])  # [n, W]
        short[g * W:(g + n) * W] = words.T.reshape(-1)  # word-major within the cluster
        g += n
    lc = (P * ivf.ex_bits + 7) // 8
    long_codes = ivf.ex_data[:, :lc].copy()
    exf = ivf.ex_data[:, lc:lc + 8].copy().view(np.float32).reshape(N, 2)
    return SearchData(ivf.centroids, ivf.rotator, short, factors, long_codes, exf.copy(), ivf.ids,
                      ivf.cluster_sizes, starts, bits)


@dataclass
class LazyIVF:
    """An IVF file mapped, not read: header arrays in memory, batch data, ex data and ids as
    memory maps, with the per-cluster offsets of search_data (for indexes too large to
    unpack whole in numpy)."""
    num: int
    dim: int
    padded_dim: int
    nlist: int
    ex_bits: int
    metric: int
    cluster_sizes: np.ndarray
    rotator: np.ndarray
    centroids: np.ndarray
    batch_data: np.ndarray  # memmap u8
    ex_data: np.ndarray  # memmap u8 [num, stride]
    ids: np.ndarray  # memmap u32
    cluster_start: np.ndarray  # i64 [nlist]: first vector (cluster order)
    block_start: np.ndarray  # i64 [nlist]: first 32-vector FastScan block


def open_ivf_lazy(path) -> LazyIVF:
    """The layout read_ivf follows (ivf.hpp:403-539), memory-mapped."""
    raw = np.memmap(path, dtype=np.uint8, mode="r")
    num, dim, nlist, ex_bits = struct.unpack_from("<4Q", raw[:32].tobytes(), 0)
    metric = int(raw[33])
    off = 34
    sizes = np.frombuffer(raw[off:off + 8 * nlist].tobytes(), dtype=np.uint64).copy()
    off += 8 * nlist
    P = round_up(dim, 64)
    rot = np.frombuffer(raw[off:off + 4 * dim * P].tobytes(), dtype=np.float32).reshape(dim, P).copy()
    off += 4 * dim * P
    nblk = (sizes.astype(np.int64) + 31) // 32
    blocks = int(nblk.sum())
    batch_bytes = blocks * (P * 32 // 8 + 32 * 12)
    ex_stride = P * ex_bits // 8 + 8
    if _centroid_layout(raw.size - off, batch_bytes + ex_stride * num + 4 * num, nlist, P) == "embedded":
        cent = np.frombuffer(raw[off:off + 4 * P * nlist].tobytes(), dtype=np.float32).reshape(nlist, P).copy()
        off += 4 * P * nlist
    else:
        cent = read_hnsw_centroids(str(path) + ".hnsw", nlist, P)
    batch = raw[off:off + batch_bytes]
    off += batch_bytes
    ex = raw[off:off + ex_stride * num].reshape(num, ex_stride)
    off += ex_stride * num
    ids = raw[off:off + 4 * num].view(np.uint32)
    starts = np.concatenate([[0], np.cumsum(sizes.astype(np.int64))[:-1]])
    bstarts = np.concatenate([[0], np.cumsum(nblk)[:-1]])
    return LazyIVF(int(num), int(dim), P, int(nlist), int(ex_bits), metric, sizes, rot, cent, batch, ex, ids,
                   starts, bstarts)


def cluster_data(ivf: LazyIVF, c: int):
    """One cluster's slice of search_data: sign bits u8 [n, P], short factors f32 [n, 3],
    packed ex-codes u8 [n, P*ex/8], ex factors f32 [n, 2], ids u32 [n] and the global index
    of its first vector."""
    P = ivf.padded_dim
    n = int(ivf.cluster_sizes[c])
    start = int(ivf.cluster_start[c])
    block_bytes = P * 4 + 32 * 12
    bits = np.zeros((n, P), np.uint8)
    fac = np.zeros((n, 3), np.float32)
    b0 = int(ivf.block_start[c]) * block_bytes
    for i in range(0, n, 32):
        blen = min(32, n - i)
        blk = np.asarray(ivf.batch_data[b0 + (i // 32) * block_bytes:b0 + (i // 32 + 1) * block_bytes])
        fl = blk[P * 4:].view(np.float32)
        bits[i:i + blen] = unpack_fastscan_bits(blk[:P * 4], P, blen)
        fac[i:i + blen, 0] = fl[0:blen]
        fac[i:i + blen, 1] = fl[32:32 + blen]
        fac[i:i + blen, 2] = fl[64:64 + blen]
    lc = (P * ivf.ex_bits + 7) // 8
    ex = np.asarray(ivf.ex_data[start:start + n])
    return (bits, fac, ex[:, :lc].copy(), ex[:, lc:lc + 8].copy().view(np.float32).reshape(n, 2),
            np.asarray(ivf.ids[start:start + n]).copy(), start)


def cluster_bits_from_short(short: np.ndarray, start: int, n: int, W: int) -> np.ndarray:
    """Inverse of the per-cluster word-major layout (filter_kernels.cuh:90-91)."""
    words = short[start * W:(start + n) * W].reshape(W, n).T
    return words_msb_to_bits(np.ascontiguousarray(words))


# --------------------------------------------------------------------------------------
# Query preparation (src/search/hybrid.cu:436-463, src/search/query_kernels.cuh)
# --------------------------------------------------------------------------------------
def rotate(q: np.ndarray, R: np.ndarray) -> np.ndarray:
    """Q' = Q . R with R [dim, P] row-major (hybrid.cu:436-440, rotator.hpp:108-112).
    Accumulated in float64 and rounded once."""
    return (q.astype(np.float64) @ R.astype(np.float64)).astype(np.float32)


def query_factors(qr: np.ndarray, ex_bits: int):
    """computeQueryFactorsWarpKernel (query_kernels.cuh:73-103):
    k1xSumq = -0.5 * sum(q'), kbxSumq = -(2^(ex+1) - 1)/2 * sum(q')."""
    s = qr.astype(np.float64).sum(axis=1)
    c1 = -0.5
    cb = -float((1 << (ex_bits + 1)) - 1) / 2.0
    return (s * c1).astype(np.float32), (s * cb).astype(np.float32)


BQ = 8  # RABITQ_BQ (kernel_types.cuh:13)


def quantize_query_bitwise(qr: np.ndarray):
    """quantize_query_bitwise_kernel (query_kernels.cuh:117-197): symmetric Bq=8
    quantisation. width = max(amax/127, 1e-30); qint = clamp(rint(q' * (1/width)),
    -128, 127) with IEEE single-precision arithmetic and round-half-even.
    Returns qint int32 [nq, P], width f32 [nq]."""
    qr = np.asarray(qr, dtype=np.float32)
    amax = np.abs(qr).max(axis=1).astype(np.float32)
    width = np.maximum(amax / np.float32(127.0), np.float32(1e-30)).astype(np.float32)
    inv = (np.float32(1.0) / width).astype(np.float32)
    prod = (qr * inv[:, None]).astype(np.float32)
    qint = np.rint(prod).astype(np.int64)
    qint = np.clip(qint, -128, 127).astype(np.int32)
    return qint, width


def quantize_query_residual(qr: np.ndarray, qint: np.ndarray, width: np.ndarray):
    """Second-stage query quantisation of this engine (no counterpart in the reference's
    Bitwise producer; it replaces the precision the reference's default FP16-LUT producer
    gives the <q',b> it hands to CPU refinement, query_kernels.cuh:199-221):
    r = fma(-width, qint, q') (the exact difference rounded once to f32; in float64 the
    product of an f32 and an 8-bit integer and this difference are exact), width2 =
    width/254, qres = clamp(rint(r * (1/width2)), -127, 127).
    Returns qres int32 [nq, P], width2 f32."""
    qr = np.asarray(qr, dtype=np.float32)
    width = np.asarray(width, dtype=np.float32)
    r = (qr.astype(np.float64) - width[:, None].astype(np.float64) * qint.astype(np.float64)).astype(np.float32)
    width2 = (width / np.float32(254.0)).astype(np.float32)
    inv2 = (np.float32(1.0) / width2).astype(np.float32)
    qres = np.clip(np.rint((r * inv2[:, None]).astype(np.float32)), -127, 127).astype(np.int32)
    return qres, width2


def exact_ip_two_stage(ip_int, ip_res, width, width2):
    """<q',b> carried to CPU refinement: fl(fl(width*ip_int) + width2*ip_res), one
    rounding for the multiply-add (float64 evaluation of an exact product)."""
    e1 = (np.float32(width) * np.asarray(ip_int, dtype=np.float32)).astype(np.float32)
    v = np.float64(np.float32(width2)) * np.asarray(ip_res, np.float64) + e1.astype(np.float64)
    return v.astype(np.float32)


def query_planes_msb(qint: np.ndarray) -> np.ndarray:
    """Bit planes of (qint & 0xFF): plane j word w bit (31-l) = bit j of dim 32w+l
    (query_kernels.cuh:171-188). Returns u32 [nq, 8, P/32]."""
    u = (qint.astype(np.int64) & 0xFF).astype(np.uint8)
    nq, P = u.shape
    planes = np.zeros((nq, BQ, P // 32), dtype=np.uint32)
    for j in range(BQ):
        planes[:, j, :] = bits_to_words_msb(((u >> j) & 1).astype(np.uint8))
    return planes


def popcount32(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.uint64)
    x = x - ((x >> 1) & 0x55555555)
    x = (x & 0x33333333) + ((x >> 2) & 0x33333333)
    x = (x + (x >> 4)) & 0x0F0F0F0F
    return ((x * 0x01010101) & 0xFFFFFFFF) >> 24


def ip_int_planes(words: np.ndarray, planes: np.ndarray) -> np.ndarray:
    """Bitwise popcount estimator (filter_kernels.cuh:79-107):
    ip_int = sum_{j<7} 2^j popc(x & q_j) - 2^7 popc(x & q_7) over all words.
    words u32 [n, W], planes u32 [8, W] -> int64 [n]."""
    acc = np.zeros(words.shape[0], dtype=np.int64)
    for j in range(BQ):
        pc = popcount32(words & planes[j][None, :]).sum(axis=1).astype(np.int64)
        acc += (pc << j) if j < BQ - 1 else -(pc << (BQ - 1))
    return acc


def ip_int_direct(bits: np.ndarray, qint: np.ndarray) -> np.ndarray:
    """Definition the popcount identity must reproduce: sum_i b_i * qint_i (exact)."""
    return bits.astype(np.int64) @ qint.astype(np.int64)


def exact_ip_bitwise(ip_int, width):
    """exact_ip = delta_q * ip_int + q_min * popc(x), q_min = 0 (filter_kernels.cuh:109,
    query_kernels.cuh:162-165)."""
    return (np.float32(width) * np.asarray(ip_int, dtype=np.float32)).astype(np.float32)


def lut4_table(qr: np.ndarray) -> np.ndarray:
    """FP16 nibble tables of the Lut4Bit estimator, precompute_lut_fp16_kernel
    (query_kernels.cuh:199-221): for nibble group g and pattern m, start from 0.0f and add
    in FP32, in this order, q'[4g] if m & 8, q'[4g+1] if m & 4, q'[4g+2] if m & 2,
    q'[4g+3] if m & 1, then round to FP16 (__float2half: nearest even). [nq, P/4, 16] f16."""
    qr = np.atleast_2d(np.asarray(qr, np.float32))
    nq, P = qr.shape
    v = qr.reshape(nq, P // 4, 4)
    m = np.arange(16)
    s = np.zeros((nq, P // 4, 16), np.float32)
    for i, bit in enumerate((8, 4, 2, 1)):
        add = np.where((m & bit) != 0, 1, 0).astype(bool)
        s = np.where(add[None, None, :], (s + v[:, :, i:i + 1]).astype(np.float32), s)
    with np.errstate(over="ignore"):  # beyond the FP16 range: +-inf, as __float2half gives
        return s.astype(np.float16)


def lut4_ip(words: np.ndarray, lut: np.ndarray) -> np.ndarray:
    """<q',b> of the Lut4Bit producers (filter_kernels.cuh:283-306, 655-708) for codes in
    the reference word layout (words [n, P/32], dimension 32w+l at bit 31-l): nibble
    j = 8w + i of word w is (word >> (28 - 4i)) & 15; FP32 accumulators a0 (even j) and
    a1 (odd j) each add float(lut[j, nibble]) in increasing j, and the estimate is a0 + a1.
    Returns f32 [n]."""
    words = np.atleast_2d(np.asarray(words, np.uint32))
    n, W = words.shape
    tab = np.asarray(lut, np.float16).astype(np.float32)  # exact
    a = [np.zeros(n, np.float32), np.zeros(n, np.float32)]
    for w in range(W):
        for i in range(8):
            j = 8 * w + i
            nib = (words[:, w] >> np.uint32(28 - 4 * i)) & np.uint32(15)
            a[j & 1] = (a[j & 1] + tab[j, nib]).astype(np.float32)
    return (a[0] + a[1]).astype(np.float32)


def low_dist(f_add, f_rescale, f_error, g_add, g_error, exact_ip, k1):
    """low = f_add + g_add + f_rescale*(exact_ip + k1) - f_error*g_error
    (filter_kernels.cuh:113-114; estimator.hpp:315-318). float64, rounded once."""
    f_add, f_rescale, f_error = (np.asarray(a, np.float64) for a in (f_add, f_rescale, f_error))
    v = f_add + np.float64(g_add) + f_rescale * (np.asarray(exact_ip, np.float64) + np.float64(k1)) \
        - f_error * np.float64(g_error)
    return v.astype(np.float32)


def est_dist(f_add, f_rescale, g_add, exact_ip, k1):
    """est = f_add + g_add + f_rescale*(ip + k1) (estimator.hpp:315-316)."""
    v = np.asarray(f_add, np.float64) + np.float64(g_add) + np.asarray(f_rescale, np.float64) * (
        np.asarray(exact_ip, np.float64) + np.float64(k1))
    return v.astype(np.float32)


# --------------------------------------------------------------------------------------
# Coarse probing (hybrid.cu:465-498; initializer.hpp:128-145; query.hpp:537-545)
# --------------------------------------------------------------------------------------
def coarse_probe(qr: np.ndarray, cent: np.ndarray, nprobe: int, metric: int):
    """Per query: the nprobe clusters nearest in L2 over rotated vectors, ascending,
    ties by cluster index (RAFT select_k tie order is unpinned; hybrid.cu:485-493).
    g_add = ||q'-c'||^2 (L2) or -<q',c'> (IP); g_error = ||q'-c'||
    (query.hpp:537-545; the hybrid GPU path uses L2 only, filter_kernels.cuh:359-361).
    Returns idx int32 [nq, nprobe], g_add f32, g_error f32, l2 f32."""
    q = qr.astype(np.float64)
    c = cent.astype(np.float64)
    d = ((q[:, None, :] - c[None, :, :]) ** 2).sum(axis=2)
    idx = np.argsort(d, axis=1, kind="stable")[:, :nprobe].astype(np.int32)
    l2 = np.take_along_axis(d, idx, axis=1)
    ip = np.einsum("qp,qkp->qk", q, c[idx])
    g_error = np.sqrt(np.maximum(l2, 0.0))
    g_add = l2 if metric == 0 else -ip
    return idx, g_add.astype(np.float32), g_error.astype(np.float32), l2.astype(np.float32)


def pair_order(probe_idx: np.ndarray, vanguard: int):
    """flatten_pairs_kernel + thrust::sort(PairSortCompare) (query_kernels.cuh:105-113,
    kernel_types.cuh:34-60): vanguard pairs (probe < vanguard) first, then by
    cluster, probe, query. Returns int64 [npairs, 3] rows (cluster, query, probe)."""
    nq, npb = probe_idx.shape
    qq, pp = np.meshgrid(np.arange(nq), np.arange(npb), indexing="ij")
    cl = probe_idx.reshape(-1).astype(np.int64)
    qq = qq.reshape(-1)
    pp = pp.reshape(-1)
    far = (pp >= vanguard).astype(np.int64)
    order = np.lexsort((qq, pp, cl, far))
    return np.stack([cl[order], qq[order], pp[order]], axis=1)


# --------------------------------------------------------------------------------------
# Ex-code refinement (cpu_refinement.cpp:183-192; pack_excode.hpp:216-265;
# space.hpp:677-761; estimator.hpp:333-351)
# --------------------------------------------------------------------------------------
def unpack_excode7(packed: np.ndarray, P: int) -> np.ndarray:
    """Inverse of packing_7bit_excode (pack_excode.hpp:216-265). Per 64 dims (56 bytes):
    bytes 0-15 / 16-31 / 32-47 hold the low 6 bits of dims 0-15 / 16-31 / 32-47 and in
    their top 2 bits bits (0-1) / (2-3) / (4-5) of dims 48-63; bytes 48-55 are a u64
    whose bit 8*(d%8) + d/8 is bit 6 of dim d. packed u8 [n, 56*P/64] -> u8 [n, P]."""
    n = packed.shape[0]
    out = np.zeros((n, P), dtype=np.uint8)
    for g in range(P // 64):
        blk = packed[:, g * 56:(g + 1) * 56].astype(np.uint16)
        low = np.zeros((n, 64), dtype=np.uint16)
        low[:, 0:16] = blk[:, 0:16] & 0x3F
        low[:, 16:32] = blk[:, 16:32] & 0x3F
        low[:, 32:48] = blk[:, 32:48] & 0x3F
        low[:, 48:64] = ((blk[:, 0:16] >> 6) & 3) | (((blk[:, 16:32] >> 6) & 3) << 2) | \
            (((blk[:, 32:48] >> 6) & 3) << 4)
        top = blk[:, 48:56].astype(np.uint64)
        top64 = np.zeros(n, dtype=np.uint64)
        for b in range(8):
            top64 |= top[:, b] << np.uint64(8 * b)
        d = np.arange(64, dtype=np.uint64)
        sh = np.uint64(8) * (d % np.uint64(8)) + d // np.uint64(8)
        bit6 = ((top64[:, None] >> sh[None, :]) & np.uint64(1)).astype(np.uint16)
        out[:, g * 64:(g + 1) * 64] = (low | (bit6 << 6)).astype(np.uint8)
    return out


def pack_excode7(codes: np.ndarray) -> np.ndarray:
    """packing_7bit_excode (pack_excode.hpp:216-265), u8 [n, P] -> u8 [n, 56*P/64]."""
    n, P = codes.shape
    out = np.zeros((n, 56 * P // 64), dtype=np.uint8)
    c = codes.astype(np.uint16)
    for g in range(P // 64):
        v = c[:, g * 64:(g + 1) * 64]
        hi = v[:, 48:64]
        o = out[:, g * 56:(g + 1) * 56]
        o[:, 0:16] = ((v[:, 0:16] & 0x3F) | ((hi << 6) & 0xC0)).astype(np.uint8)
        o[:, 16:32] = ((v[:, 16:32] & 0x3F) | ((hi << 4) & 0xC0)).astype(np.uint8)
        o[:, 32:48] = ((v[:, 32:48] & 0x3F) | ((hi << 2) & 0xC0)).astype(np.uint8)
        top = np.zeros(n, dtype=np.uint64)
        for i in range(0, 64, 8):
            for b in range(8):
                bit = ((v[:, i + b] >> 6) & 1).astype(np.uint64)
                top |= bit << np.uint64(8 * b + i // 8)
        for b in range(8):
            o[:, 48 + b] = ((top >> np.uint64(8 * b)) & np.uint64(0xFF)).astype(np.uint8)
    return out


def excode_ip(qr_row: np.ndarray, packed: np.ndarray, P: int) -> np.ndarray:
    """<q', ex_code> over all P dims (space.hpp:677-761), float64 then rounded."""
    codes = unpack_excode7(packed, P).astype(np.float64)
    return (codes @ qr_row.astype(np.float64)).astype(np.float32)


def refine_dist(f_ex_add, f_ex_rescale, g_add, exact_ip, ip2, kb, ex_bits):
    """refine = f_ex_add + g_add + f_ex_rescale*(2^ex * exact_ip + ip2 + kbxSumq)
    (cpu_refinement.cpp:183-192; estimator.hpp:344-348)."""
    v = np.asarray(f_ex_add, np.float64) + np.float64(g_add) + np.asarray(f_ex_rescale, np.float64) * (
        float(1 << ex_bits) * np.asarray(exact_ip, np.float64) + np.asarray(ip2, np.float64) + np.float64(kb))
    return v.astype(np.float32)


# --------------------------------------------------------------------------------------
# End-to-end hybrid search with frozen thresholds (hybrid.cu:398-689,
# cpu_refinement.cpp:71-284) — deterministic restatement for candidate-set and top-k
# parity. thresholds: f32 [nq] read by the GPU filter (low < thr) and never tightened
# (the engine's frozen-threshold mode); the CPU side then keeps the topk smallest
# refine distances per query (insertion under refine < current k-th,
# cpu_refinement.cpp:197-229).
# --------------------------------------------------------------------------------------
@dataclass
class HybridResult:
    dists: np.ndarray  # f32 [nq, topk] (FLT_MAX pad)
    ids: np.ndarray  # u32 [nq, topk] (0 pad)
    candidates: list  # per query: set of (gid) published by the filter
    low: dict  # (q, gid) -> low distance (f32)
    exact_ip: dict  # (q, gid) -> exact_ip (f32)


def hybrid_search(sd: SearchData, queries: np.ndarray, topk: int, nprobe: int, metric: int,
                  ex_bits: int, thresholds=None, estimator: str = "bitwise") -> HybridResult:
    """estimator "bitwise": Bq=8 lower bound, two-stage exact_ip for refinement (this
    engine's Bitwise mode); "lut4": the FP16 nibble-LUT estimate for both (the reference's
    Lut4Bit producers)."""
    P = sd.centroids.shape[1]
    W = P // 32
    nq = queries.shape[0]
    qr = rotate(queries, sd.rotator)
    k1, kb = query_factors(qr, ex_bits)
    qint, width = quantize_query_bitwise(qr)
    qres, width2 = quantize_query_residual(qr, qint, width)
    planes = query_planes_msb(qint)
    luts = lut4_table(qr) if estimator == "lut4" else None
    idx, g_add, g_err, _ = coarse_probe(qr, sd.centroids, nprobe, metric)
    thr = np.full(nq, F32_MAX, np.float32) if thresholds is None else np.asarray(thresholds, np.float32)
    dists = np.full((nq, topk), F32_MAX, np.float32)
    out_ids = np.zeros((nq, topk), np.uint32)
    cands, lows, eips = [], {}, {}
    for q in range(nq):
        items = []
        cset = set()
        for p in range(nprobe):
            c = int(idx[q, p])
            n = int(sd.cluster_sizes[c])
            s = int(sd.cluster_start[c])
            if n == 0:
                continue
            words = np.ascontiguousarray(sd.short_data[s * W:(s + n) * W].reshape(W, n).T)
            if luts is not None:
                eip = lut4_ip(words, luts[q])
            else:
                ipi = ip_int_planes(words, planes[q])
                eip = exact_ip_bitwise(ipi, width[q])
            f = sd.short_factors[s:s + n]
            low = low_dist(f[:, 0], f[:, 1], f[:, 2], g_add[q, p], g_err[q, p], eip, k1[q])
            keep = np.nonzero(low < thr[q])[0]
            if keep.size == 0:
                continue
            gids = s + keep
            if luts is not None:
                eip2 = eip[keep]
            else:
                ipr = ip_int_direct(sd.bits[gids], qres[q])
                eip2 = exact_ip_two_stage(ipi[keep], ipr, width[q], width2[q])
            ip2 = excode_ip(qr[q], sd.long_codes[gids], P)
            rd = refine_dist(sd.ex_factors[gids, 0], sd.ex_factors[gids, 1], g_add[q, p], eip2,
                             ip2, kb[q], ex_bits)
            for j, gid in enumerate(gids):
                cset.add(int(gid))
                lows[(q, int(gid))] = low[keep[j]]
                eips[(q, int(gid))] = eip2[j]
                items.append((float(rd[j]), int(sd.ids[gid])))
        cands.append(cset)
        items.sort(key=lambda t: t[0])
        items = [t for t in items if t[0] < thr[q]][:topk]
        for r, (dv, pid) in enumerate(items):
            dists[q, r] = dv
            out_ids[q, r] = pid
    return HybridResult(dists, out_ids, cands, lows, eips)


def vanguard_seeds(low: np.ndarray, keep: int, cutoff) -> np.ndarray:
    """Seeds of one vanguard pair (filter_kernels.cuh:308-468, whose CUB radix sort keeps
    max(topk, 20) lowest bounds below the cutoff): the min(keep, #valid) smallest lows
    below the cutoff, ties to the lower index (this engine's radix select; CUB's tie order
    is unpinned). Returns local indices in ascending low order."""
    valid = np.nonzero(np.asarray(low) < np.float32(cutoff))[0]
    return valid[np.argsort(np.asarray(low)[valid], kind="stable")][:keep]


def refine_error_scale(padded_dim: int) -> float:
    """Per unit of magnitude, the bound on the difference between two FP32 evaluations of
    refine_dist (cpu_refinement.cpp:183-192) in any summation orders: each lies within
    gamma_n = n u / (1 - n u), u = 2^-24, of the exact value times the magnitude of its terms,
    n = P + 8 the longest chain of roundings a term passes (the P products and sums of the
    ex-code dot product, fused or not, and the outer formula's five); two differ by at most
    2 gamma_n, and 2.002 covers the FP32 rounding of the magnitude. The engine's kernels use
    the same constant (refine_err_scale, engine_internal.h)."""
    n = float(padded_dim) + 8.0
    u = 2.0 ** -24
    return float(np.float32(2.002 * n * u / (1.0 - n * u)))


def refine_error_bound(f_ex_add, f_ex_rescale, g_add, exact_ip, q_l1, kb, ex_bits, padded_dim):
    """Bound on the rounding difference between two FP32 evaluations of refine_dist in
    different summation orders (GPU refinement vs the CPU consumer): refine_error_scale(P)
    times the magnitude of its terms, |f_add| + |g_add| + |f_rescale| (2^ex |ip| +
    (2^ex - 1) ||q'||_1 + |kb|). The ex-code inner product is at most (2^ex - 1) ||q'||_1.
    Pinned by test_refine_error_bound_covers_f32_evaluation (sequential FP32 order against
    FP64, and two FP32 orders against each other, at half and the full bound)."""
    s = float(1 << ex_bits)
    mag = np.abs(np.asarray(f_ex_add, np.float64)) + abs(float(g_add)) + np.abs(
        np.asarray(f_ex_rescale, np.float64)) * (s * np.abs(np.asarray(exact_ip, np.float64)) +
                                                 (s - 1) * float(q_l1) + abs(float(kb)))
    return (refine_error_scale(padded_dim) * mag).astype(np.float32)


def seed_threshold(dists, lows, errs, topk: int):
    """GPU seed threshold of this engine (no counterpart in the reference, whose CPU
    consumer alone publishes thresholds, cpu_refinement.cpp:207-230): with d_k the topk-th
    smallest refined seed distance, e the largest rounding bound and l the largest lower
    bound among the seeds with distance <= d_k, thr = nextafter(max(d_k + e, l), +inf)
    in FP32. None when fewer than topk seeds exist."""
    d = np.asarray(dists, np.float32)
    fin = np.isfinite(d)
    if fin.sum() < topk:
        return None
    kth = np.sort(d[fin])[topk - 1]
    sel = fin & (d <= kth)
    e = np.float32(np.asarray(errs, np.float32)[sel].max())
    l = np.float32(np.asarray(lows, np.float32)[sel].max())
    return np.nextafter(np.float32(max(np.float32(kth + e), l)), np.float32(np.inf))


def brute_force_gt(base: np.ndarray, queries: np.ndarray, k: int, metric: int) -> np.ndarray:
    """Exact top-k by float64 brute force (tools/data/generate_gt_gpu.py semantics)."""
    b = base.astype(np.float64)
    q = queries.astype(np.float64)
    if metric == 1:
        score = -(q @ b.T)
    else:
        score = (q * q).sum(1)[:, None] - 2 * q @ b.T + (b * b).sum(1)[None, :]
    return np.argsort(score, axis=1, kind="stable")[:, :k].astype(np.uint32)


def recall_at_k(result_ids: np.ndarray, gt: np.ndarray, k: int) -> float:
    """ID recall (include/coraanns/benchmark/recall.hpp:74-128): |R ∩ G_k| / (nq*k)."""
    hits = 0
    for r, g in zip(result_ids, gt):
        hits += len(set(int(x) for x in r[:k]) & set(int(x) for x in g[:k]))
    return hits / (result_ids.shape[0] * k)


# How each function is pinned (see tests/test_oracle.py):
_TIGHT_START = [0.0, 0.15, 0.20, 0.52, 0.59, 0.71, 0.75, 0.77, 0.81]  # rabitq_impl.hpp:263-273


def excode_residual_abs(x: np.ndarray, c: np.ndarray) -> np.ndarray:
    """|o| / ||o|| in the builder's arithmetic (quantize_ex_bits): o = x - c in f32,
    ||o||^2 accumulated sequentially in f64 and rounded to f32, sqrt and division in f32."""
    o = (np.asarray(x, np.float32) - np.asarray(c, np.float32)).astype(np.float32)
    acc = 0.0
    for v in o.tolist():
        acc += v * v
    norm = np.sqrt(np.float32(acc))
    return o, np.abs((o / norm).astype(np.float32))


def best_rescale_factor(o_abs: np.ndarray, ex_bits: int) -> float:
    """The reference's rescale search (rabitq_impl.hpp:276-333): a min-priority queue of
    (t, coordinate) increment points, t from t_start = t_end * tight_start[ex] up to
    t_end = (2^ex - 1 + 10) / max|o|; each pop increments the coordinate's code, updates
    <code + 1/2, |o|> and ||code + 1/2||^2 in double, and keeps the first t of the largest
    ratio; the coordinate's next point is pushed while its code is below 2^ex - 1 and the
    point is below t_end."""
    import heapq
    import math
    eps, n_enum = 1e-5, 10
    cap = (1 << ex_bits) - 1
    oa = [float(v) for v in o_abs]
    max_o = max(oa)
    t_end = (cap + n_enum) / max_o
    t_start = t_end * _TIGHT_START[ex_bits]
    cur = [int(t_start * v + eps) for v in oa]
    sqr_den = len(oa) * 0.25
    num = 0.0
    for c, v in zip(cur, oa):
        sqr_den += c * c + c
        num += (c + 0.5) * v
    heap = [((c + 1) / v if v != 0 else math.inf, i) for i, (c, v) in enumerate(zip(cur, oa))]
    heapq.heapify(heap)
    best_ip, best_t = 0.0, 0.0
    while heap:
        t, i = heapq.heappop(heap)
        cur[i] += 1
        v = cur[i]
        sqr_den += 2 * v
        num += oa[i]
        ip = num / math.sqrt(sqr_den)
        if ip > best_ip:
            best_ip, best_t = ip, t
        if v < cap:
            tn = (v + 1) / oa[i] if oa[i] != 0 else math.inf
            if tn < t_end:
                heapq.heappush(heap, (tn, i))
    return best_t


def quantize_excode(x: np.ndarray, c: np.ndarray, ex_bits: int) -> np.ndarray:
    """7-bit ex-code of one vector (rabitq_impl.hpp:336-360, 423-429): floor(t |o_i| + eps)
    capped, bitwise complement on negative residual coordinates."""
    o, oa = excode_residual_abs(x, c)
    t = best_rescale_factor(oa, ex_bits)
    cap = (1 << ex_bits) - 1
    code = np.array([min(int(t * float(v) + 1e-5), cap) for v in oa], np.int64)
    code = np.where(o < 0, (~code) & cap, code)
    return code.astype(np.uint8)


PINNED = {
    "read_ivf": "golden: ref_dump meta/ids/centroids/rotator (reference IVF::load)",
    "lut4_table": "closed forms: single-bit entries, pattern bit 3 = first dimension, FP16 "
                  "round-half-even and overflow to inf",
    "lut4_ip": "closed forms: split even/odd FP32 accumulators (1 + n_odd 2^-24 case), one-hot "
               "nibble layout, exact integer inner products for representable values",
    "read_hnsw_centroids": "reference-built sidecar index (coraanns_build_index, nlist 20000): centroids "
                           "equal ref_dump's (reference IVF::load + HNSWInitializer); permuted-label "
                           "sidecars equal the embedded centroids; corrupt files rejected",
    "search_data": "golden: ref_dump short_data/short_factors/long_codes/ex_factors (reference SearchData)",
    "open_ivf_lazy": "equals read_ivf on the golden indexes (header arrays, maps, offsets)",
    "cluster_data": "equals the per-cluster slices of search_data on the golden indexes",
    "fastscan_pack": "golden: ref_dump fastscan_blocks (reference pack_codes) + unpack round trip",
    "unpack_fastscan_bits": "round trip with fastscan_pack on random bits; golden short_data",
    "rotate": "golden: ref_dump rotated_queries (reference MatrixRotator::rotate), 1e-5",
    "query_factors": "golden: ref_dump est_qvals k1xsumq/kbxsumq (reference SplitBatchQuery), 1e-5",
    "quantize_query_bitwise": "closed forms: zero query, +-amax -> +-127, half-even ties at width 1 and "
                              "2^-3, |err|<=width/2; exact rational arithmetic at rounding boundaries "
                              "where q*(1/width) and q/width round apart",
    "quantize_query_residual": "closed forms: |q' - width*qint - width2*qres| <= width2/2 (+ f32 rounding), "
                               "zero query -> 0, exact multiples of width -> qres 0",
    "exact_ip_two_stage": "bound: |two_stage - <q',b>_f64| <= popc(b)*width2/2 (+ f32 rounding) on random data",
    "ip_int_planes": "brute force: equals ip_int_direct on random bits / qint, incl. -128",
    "low_dist": "golden: reproduces reference est_low from est_ipx0 (estimator.hpp:315-318), 1e-5",
    "est_dist": "golden: reproduces reference est_dist from est_ipx0, 1e-5",
    "coarse_probe": "golden: ref_dump centroid_dist/centroid_ip and est_qvals g_add/g_error, 1e-5",
    "pair_order": "comparator KAT against PairSortCompare cases",
    "unpack_excode7": "golden: ref_dump packed7 vs excode_l2 (reference packing_7bit_excode)",
    "pack_excode7": "golden: equals ref_dump packed7 byte for byte",
    "excode_ip": "golden: ref_dump ip_fxu7 (reference ip64_fxu7_avx), 1e-5",
    "refine_dist": "golden: reproduces reference est_exdist from est_ipx0 (split_distance_boosting), 1e-5",
    "hybrid_search": "composition of the pinned functions; top-k ids vs brute force on all-probe search",
    "vanguard_seeds": "brute force: equals the first min(keep, #valid) of a full stable sort of valid lows",
    "refine_error_bound": "property: two FP32 orders of refine_dist on golden ex-codes each within half of it "
                          "of FP64, and the all-positive worst case of sequential summation at P = 1,024",
    "refine_error_scale": "closed form 2.002 gamma_{P+8}; covered by the refine_error_bound property test",
    "seed_threshold": "properties: >= topk seeds strictly below it with lows below it; >= true topk-th",
    "excode_residual_abs": "golden: quantize_excode reproduces the reference builder's ex-codes (quant_d128)",
    "best_rescale_factor": "golden: quantize_excode reproduces the reference builder's ex-codes (quant_d128); "
                           "brute force over every increment point on small dims",
    "quantize_excode": "golden: the reference builder's ex-codes of quant_d128 (rows vs centroid row 0)",
}
