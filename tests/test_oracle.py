"""Pin the CPU oracle against the reference's own outputs (tests/golden, written by
tests/golden/make_golden.py from the reference CPU code), closed forms and brute force.
CPU only."""
import numpy as np
import pytest

import cora_oracle as orc
from conftest import GOLDEN, read_fbin

FIXTURES = ["l2_d96", "ip_d64"]


def rel_close(a, b, rtol=1e-5, scale=None):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    s = np.maximum(np.abs(b), 1.0 if scale is None else scale)
    return np.all(np.abs(a - b) <= rtol * s)


@pytest.fixture(scope="module", params=FIXTURES)
def fx(request, golden):
    name = request.param
    ref = golden(f"{name}/ref")
    ivf = orc.read_ivf(GOLDEN / name / "ivf.index")
    sd = orc.search_data(ivf)
    q = read_fbin(GOLDEN / name / "queries.fbin")
    return name, ref, ivf, sd, q


def test_ivf_header_and_payload(fx):
    _, ref, ivf, sd, _ = fx
    n, dim, P, nl, ex, metric = (int(x) for x in ref["meta"])
    assert (ivf.num, ivf.dim, ivf.padded_dim, ivf.nlist, ivf.ex_bits, ivf.metric) == (n, dim, P, nl, ex, metric)
    assert np.array_equal(ivf.ids, ref["ids"])
    assert np.array_equal(ivf.cluster_sizes, ref["cluster_sizes"])
    assert np.array_equal(sd.centroids.view(np.uint32), ref["centroids"].view(np.uint32))
    assert np.array_equal(sd.rotator.view(np.uint32), ref["rotator"].view(np.uint32))


def test_search_data_unpack_bit_exact(fx):
    _, ref, ivf, sd, _ = fx
    assert np.array_equal(sd.short_data, ref["short_data"].reshape(-1))
    assert np.array_equal(sd.short_factors.view(np.uint32), ref["short_factors"].view(np.uint32))
    assert np.array_equal(sd.long_codes, ref["long_codes"])
    assert np.array_equal(sd.ex_factors.view(np.uint32), ref["ex_factors"].view(np.uint32))
    # word-major layout inverse
    W = ivf.padded_dim // 32
    for c in range(ivf.nlist):
        s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
        assert np.array_equal(orc.cluster_bits_from_short(sd.short_data, s, n, W), sd.bits[s:s + n])


def test_lazy_reader_matches_search_data(fx):
    """The memory-mapped per-cluster reader (for indexes too large to unpack whole) gives
    exactly the search_data slices of every cluster."""
    name, _, ivf, sd, _ = fx
    lz = orc.open_ivf_lazy(GOLDEN / name / "ivf.index")
    assert (lz.num, lz.dim, lz.padded_dim, lz.nlist, lz.ex_bits, lz.metric) == \
        (ivf.num, ivf.dim, ivf.padded_dim, ivf.nlist, ivf.ex_bits, ivf.metric)
    assert np.array_equal(lz.rotator, ivf.rotator) and np.array_equal(lz.centroids, ivf.centroids)
    assert np.array_equal(lz.cluster_start, sd.cluster_start)
    for c in range(ivf.nlist):
        bits, fac, lc, exf, ids, start = orc.cluster_data(lz, c)
        s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
        assert start == s
        assert np.array_equal(bits, sd.bits[s:s + n])
        assert np.array_equal(fac.view(np.uint32), sd.short_factors[s:s + n].view(np.uint32))
        assert np.array_equal(lc, sd.long_codes[s:s + n])
        assert np.array_equal(exf.view(np.uint32), sd.ex_factors[s:s + n].view(np.uint32))
        assert np.array_equal(ids, sd.ids[s:s + n])


def test_fastscan_pack_golden_and_round_trip(golden):
    g = golden("quant_d128")
    compact = g["compact_bits"]
    blocks = orc.fastscan_pack(compact, 128)
    assert np.array_equal(blocks, g["fastscan_blocks"])
    n = compact.shape[0]
    bits_ref = np.unpackbits(compact, axis=1)  # MSB first == pack_binary order
    got = []
    for b in range(0, n, 32):
        blen = min(32, n - b)
        got.append(orc.unpack_fastscan_bits(blocks[(b // 32) * 512:(b // 32 + 1) * 512], 128, blen))
    assert np.array_equal(np.vstack(got), bits_ref)
    # random round trip, ragged last block
    rng = np.random.default_rng(5)
    for n, P in [(1, 64), (33, 128), (70, 192)]:
        bits = rng.integers(0, 2, (n, P), dtype=np.uint8)
        blocks = orc.fastscan_pack(np.packbits(bits, axis=1), P)
        out = [orc.unpack_fastscan_bits(blocks[(b // 32) * 4 * P:(b // 32 + 1) * 4 * P], P, min(32, n - b))
               for b in range(0, n, 32)]
        assert np.array_equal(np.vstack(out), bits)


def test_rotation_and_query_factors(fx):
    _, ref, ivf, sd, q = fx
    qr = orc.rotate(q, sd.rotator)
    scale = np.abs(q).sum(1, keepdims=True) * np.abs(sd.rotator).max()
    assert np.all(np.abs(qr - ref["rotated_queries"]) <= 1e-5 * scale)
    k1, kb = orc.query_factors(ref["rotated_queries"], ivf.ex_bits)
    s = np.abs(ref["rotated_queries"]).sum(1)
    assert np.all(np.abs(k1 - ref["est_qvals"][:, 0]) <= 1e-5 * s)
    assert np.all(np.abs(kb - ref["est_qvals"][:, 1]) <= 1e-5 * 127.5 * s)


def test_coarse_probe_distances(fx):
    _, ref, ivf, sd, _ = fx
    qr = ref["rotated_queries"]
    nl = ivf.nlist
    idx, g_add, g_err, l2 = orc.coarse_probe(qr, sd.centroids, nl, ivf.metric)
    # order agrees with the reference flat initializer's distances
    cd = ref["centroid_dist"]
    for qi in range(qr.shape[0]):
        d_sorted = cd[qi, idx[qi]]
        assert np.all(np.diff(d_sorted.astype(np.float64)) >= -1e-5 * d_sorted.max())
        assert rel_close(np.sqrt(l2[qi]), cd[qi, idx[qi]])
    # g_add / g_error of the estimate cluster match SplitBatchQuery::set_g_add
    for qi in range(qr.shape[0]):
        c = int(ref["est_cluster"][qi])
        p = int(np.nonzero(idx[qi] == c)[0][0])
        assert rel_close(g_add[qi, p], ref["est_qvals"][qi, 2], scale=1.0)
        assert rel_close(g_err[qi, p], ref["est_qvals"][qi, 3])


def _est_rows(ref, sd, qi):
    c = int(ref["est_cluster"][qi])
    s, n = int(sd.cluster_start[c]), int(sd.cluster_sizes[c])
    off = int(sum(int(sd.cluster_sizes[int(ref["est_cluster"][j])]) for j in range(qi)))
    return c, s, n, off


def test_low_and_est_reproduce_reference_estimator(fx):
    _, ref, ivf, sd, _ = fx
    for qi in range(ref["rotated_queries"].shape[0]):
        c, s, n, off = _est_rows(ref, sd, qi)
        k1, kb, gadd, gerr = ref["est_qvals"][qi, :4]
        ipx0 = ref["est_ipx0"][off:off + n]
        f = sd.short_factors[s:s + n]
        est = orc.est_dist(f[:, 0], f[:, 1], gadd, ipx0, k1)
        low = orc.low_dist(f[:, 0], f[:, 1], f[:, 2], gadd, gerr, ipx0, k1)
        sc = np.abs(f[:, 1] * (ipx0 + k1)) + abs(gadd) + np.abs(f[:, 0]) + np.abs(f[:, 2] * gerr)
        assert np.all(np.abs(est - ref["est_dist"][off:off + n]) <= 2e-5 * sc)
        assert np.all(np.abs(low - ref["est_low"][off:off + n]) <= 2e-5 * sc)


def test_refine_reproduces_reference_ex_distance(fx):
    _, ref, ivf, sd, _ = fx
    P = ivf.padded_dim
    for qi in range(ref["rotated_queries"].shape[0]):
        c, s, n, off = _est_rows(ref, sd, qi)
        k1, kb, gadd, gerr = ref["est_qvals"][qi, :4]
        ipx0 = ref["est_ipx0"][off:off + n]
        ip2 = orc.excode_ip(ref["rotated_queries"][qi], sd.long_codes[s:s + n], P)
        rd = orc.refine_dist(sd.ex_factors[s:s + n, 0], sd.ex_factors[s:s + n, 1], gadd, ipx0, ip2, kb,
                             ivf.ex_bits)
        sc = np.abs(sd.ex_factors[s:s + n, 1]) * (128 * np.abs(ipx0) + np.abs(ip2) + abs(kb)) \
            + abs(gadd) + np.abs(sd.ex_factors[s:s + n, 0])
        assert np.all(np.abs(rd - ref["est_exdist"][off:off + n]) <= 2e-5 * sc)


def test_excode_pack_unpack_and_ip(golden):
    g = golden("quant_d128")
    codes = g["excode_l2"]
    packed = g["packed7"]
    assert np.array_equal(orc.unpack_excode7(packed, 128), codes)
    assert np.array_equal(orc.pack_excode7(codes), packed)
    centroid = np.fromfile(GOLDEN / "quant_d128" / "rows.f32", dtype=np.float32)[:128]
    ip = orc.excode_ip(centroid, packed, 128)
    sc = np.abs(centroid).sum() * 127
    assert np.all(np.abs(ip - g["ip_fxu7"]) <= 1e-6 * sc)


def test_quantize_query_closed_forms():
    # zero query: width clamps to 1e-30, qint = 0
    qint, w = orc.quantize_query_bitwise(np.zeros((1, 64), np.float32))
    assert w[0] == np.float32(1e-30) and not qint.any()
    # +-amax map to +-127, ties round half to even
    v = np.zeros((1, 64), np.float32)
    v[0, 0], v[0, 1] = 127.0, -127.0
    v[0, 2], v[0, 3], v[0, 4], v[0, 5] = 0.5, 1.5, 2.5, -0.5
    qint, w = orc.quantize_query_bitwise(v)
    assert w[0] == 1.0
    assert list(qint[0, :6]) == [127, -127, 0, 2, 2, 0]
    # random: reconstruction error within width/2
    rng = np.random.default_rng(1)
    x = rng.normal(0, 3, (20, 128)).astype(np.float32)
    qint, w = orc.quantize_query_bitwise(x)
    assert np.all(np.abs(x - qint * w[:, None]) <= 0.5 * w[:, None] * (1 + 1e-5))
    assert qint.min() >= -127 and qint.max() <= 127


def test_residual_quantize_closed_forms():
    # zero query: residual 0
    z = np.zeros((1, 64), np.float32)
    qint, w = orc.quantize_query_bitwise(z)
    qres, w2 = orc.quantize_query_residual(z, qint, w)
    assert not qres.any() and w2[0] == np.float32(1e-30) / np.float32(254.0)
    # integer queries with amax 127: width 1, q' = qint exactly, residual 0
    rng = np.random.default_rng(11)
    v = rng.integers(-127, 128, (3, 128)).astype(np.float32)
    v[:, 0] = 127.0
    qint, w = orc.quantize_query_bitwise(v)
    qres, w2 = orc.quantize_query_residual(v, qint, w)
    assert np.all(w == 1.0) and not qres.any()
    assert np.all(w2 == np.float32(1.0) / np.float32(254.0))
    # random: two-stage reconstruction within width2/2 (plus f32 rounding of q')
    x = rng.normal(0, 3, (20, 128)).astype(np.float32)
    qint, w = orc.quantize_query_bitwise(x)
    qres, w2 = orc.quantize_query_residual(x, qint, w)
    recon = qint * w[:, None].astype(np.float64) + qres * w2[:, None].astype(np.float64)
    err = np.abs(x.astype(np.float64) - recon)
    assert np.all(err <= 0.5 * w2[:, None] + 4e-7 * np.abs(x))
    assert qres.min() >= -127 and qres.max() <= 127
    # the residual really refines: the one-stage error is about 127x larger on average
    assert np.abs(x - qint * w[:, None]).mean() > 50 * err.mean()
    # a plausible mistake (residual step = width instead of width / 254) breaks the bound
    bad = np.clip(np.rint((x - qint * w[:, None]) / w[:, None]), -127, 127)
    recon_bad = qint * w[:, None] + bad * w2[:, None]
    assert not np.all(np.abs(x - recon_bad) <= 0.5 * w2[:, None] + 4e-7 * np.abs(x))


def test_two_stage_inner_product_error_bound():
    rng = np.random.default_rng(12)
    for P in (64, 128, 768):
        x = rng.normal(0, 1, (4, P)).astype(np.float32)
        bits = rng.integers(0, 2, (200, P), dtype=np.uint8)
        qint, w = orc.quantize_query_bitwise(x)
        qres, w2 = orc.quantize_query_residual(x, qint, w)
        for q in range(x.shape[0]):
            ip1 = orc.ip_int_direct(bits, qint[q])
            ipr = orc.ip_int_direct(bits, qres[q])
            est = orc.exact_ip_two_stage(ip1, ipr, w[q], w2[q]).astype(np.float64)
            exact = bits.astype(np.float64) @ x[q].astype(np.float64)
            pc = bits.sum(1)
            bound = pc * 0.5 * w2[q] + 2e-7 * (np.abs(est) + pc * np.abs(x[q]).max())
            assert np.all(np.abs(est - exact) <= bound), P
            # the Bq=8 estimate alone violates the same bound (the refinement matters)
            one = orc.exact_ip_bitwise(ip1, w[q]).astype(np.float64)
            assert not np.all(np.abs(one - exact) <= bound)


def test_popcount_planes_equal_direct_inner_product():
    rng = np.random.default_rng(2)
    for P in (64, 128, 768):
        bits = rng.integers(0, 2, (50, P), dtype=np.uint8)
        qint = rng.integers(-128, 128, (1, P)).astype(np.int32)
        qint[0, :3] = [-128, 127, 0]
        words = orc.bits_to_words_msb(bits)
        planes = orc.query_planes_msb(qint)[0]
        assert np.array_equal(orc.ip_int_planes(words, planes), orc.ip_int_direct(bits, qint[0]))


def test_pair_order_comparator_cases():
    probe_idx = np.array([[5, 1, 3], [1, 5, 2], [3, 2, 1]], dtype=np.int32)
    rows = orc.pair_order(probe_idx, vanguard=1)
    # vanguard pairs (probe 0) first, by cluster then query
    assert [tuple(r) for r in rows[:3]] == [(1, 1, 0), (3, 2, 0), (5, 0, 0)]
    far = [tuple(r) for r in rows[3:]]
    assert far == sorted(far, key=lambda r: (r[0], r[2], r[1]))
    assert len(rows) == 9


def test_hybrid_search_all_probes_matches_brute_force(fx):
    name, ref, ivf, sd, q = fx
    base = read_fbin(GOLDEN / name / "base.fbin")
    res = orc.hybrid_search(sd, q, 10, ivf.nlist, ivf.metric, ivf.ex_bits)
    gt = orc.brute_force_gt(base, q, 10, ivf.metric)
    assert orc.recall_at_k(res.ids, gt, 10) >= 0.95
    # the reference CPU path's top-k at full nprobe agrees as closely
    ref_ids = ref["search_ids"][-1]
    assert orc.recall_at_k(res.ids, ref_ids.astype(np.uint32), 10) >= 0.95
    # every vector of every probed cluster was a candidate with infinite thresholds
    assert all(len(c) == ivf.num for c in res.candidates)


def test_vanguard_seed_selection_brute_force():
    rng = np.random.default_rng(21)
    for n, keep in ((50, 20), (300, 20), (10, 20), (1000, 100)):
        low = rng.integers(0, 40, n).astype(np.float32)  # many ties
        cutoff = np.float32(30)
        got = orc.vanguard_seeds(low, keep, cutoff)
        valid = [i for i in range(n) if low[i] < cutoff]
        want = sorted(valid, key=lambda i: (low[i], i))[:keep]
        assert got.tolist() == want


def test_refine_error_bound_covers_f32_evaluation(fx):
    """The refined distance's rounding bound (refine_error_scale(P) times the magnitude of
    its terms) against FP32 evaluations in two different orders: each lies within half the
    bound of the FP64 value (the gamma_{P+8} half of the derivation), so the two differ by
    less than the bound; the same with adversarial terms (all of one sign, the worst case of
    sequential summation) at P = 1,024."""
    name, ref, ivf, sd, q = fx
    P = ivf.padded_dim
    qr = orc.rotate(q, sd.rotator)
    _, kb = orc.query_factors(qr, ivf.ex_bits)
    rng = np.random.default_rng(22)
    for i in range(min(8, q.shape[0])):
        gids = rng.integers(0, ivf.num, 64)
        ex = rng.normal(0, 1, 64).astype(np.float32)
        g = np.float32(abs(rng.normal(0, 5)))
        fa, fr = sd.ex_factors[gids, 0], sd.ex_factors[gids, 1]
        codes = orc.unpack_excode7(sd.long_codes[gids], P).astype(np.float32)
        ip64 = codes.astype(np.float64) @ qr[i].astype(np.float64)
        d64 = fa.astype(np.float64) + g + fr.astype(np.float64) * (128.0 * ex + ip64 + kb[i])
        # order 1: sequential accumulation of the ex-code dot; order 2: eight-wide chunks
        dot_seq = np.zeros(64, np.float32)
        for d in range(P):
            dot_seq = (dot_seq + codes[:, d] * qr[i, d]).astype(np.float32)
        dot_chunk = np.zeros(64, np.float32)
        for c in range(P // 8):
            part = np.zeros(64, np.float32)
            for d in range(8 * c, 8 * c + 8):
                part = (part + codes[:, d] * qr[i, d]).astype(np.float32)
            dot_chunk = (dot_chunk + part).astype(np.float32)
        outs = [(fa + g + fr * ((np.float32(128) * ex + dot).astype(np.float32) + kb[i])).astype(np.float32)
                for dot in (dot_seq, dot_chunk)]
        bound = orc.refine_error_bound(fa, fr, g, ex, np.abs(qr[i]).sum(), kb[i], 7, P).astype(np.float64)
        for d32 in outs:
            assert np.all(np.abs(d32 - d64) <= 0.5 * bound), name
        assert np.all(np.abs(outs[0].astype(np.float64) - outs[1]) <= bound), name
    # worst case of sequential summation: 1,024 positive terms of one size
    P = 1024
    qv = np.full(P, np.float32(0.7), np.float32)
    code = np.full(P, np.float32(127), np.float32)
    acc = np.float32(0)
    for d in range(P):
        acc = np.float32(acc + code[d] * qv[d])
    exact = 127.0 * 0.699999988079071 * P
    b = orc.refine_error_bound(np.float32(0), np.float32(1), np.float32(0), np.float32(0), float(qv.sum()), 0.0, 7, P)
    assert abs(float(acc) - exact) <= 0.5 * float(b)
    assert orc.refine_error_scale(128) < 2e-5 and orc.refine_error_scale(768) < 1e-4


def test_seed_threshold_properties():
    rng = np.random.default_rng(23)
    for topk in (1, 10, 100):
        n = 5 * max(topk, 20)
        d = rng.normal(0, 3, n).astype(np.float32)
        d[rng.random(n) < 0.2] = np.inf  # unused slots
        lows = (d - np.abs(rng.normal(0, 1, n))).astype(np.float32)
        errs = np.abs(rng.normal(0, 1e-3, n)).astype(np.float32)
        thr = orc.seed_threshold(d, lows, errs, topk)
        fin = np.isfinite(d)
        if fin.sum() < topk:
            assert thr is None
            continue
        best = np.argsort(np.where(fin, d, np.inf), kind="stable")[:topk]
        # the topk best seeds stay strictly below it, with their rounding and their lows
        assert np.all(d[best] + errs[best] < thr) and np.all(lows[best] < thr)
        assert thr >= np.sort(d[fin])[topk - 1]
    # a low above every distance lifts the threshold above it
    d = np.arange(20, dtype=np.float32)
    lows = d.copy()
    lows[3] = 50.0
    assert orc.seed_threshold(d, lows, np.zeros(20, np.float32), 10) > 50.0
    assert orc.seed_threshold(d[:5], lows[:5], np.zeros(5, np.float32), 10) is None


def test_quantize_excode_reproduces_reference_builder(golden):
    """The oracle's restatement of the rescale search reproduces the reference builder's
    ex-codes (rows 1.. against row 0 as centroid, L2)."""
    g = golden("quant_d128")
    rows = np.fromfile(GOLDEN / "quant_d128" / "rows.f32", dtype=np.float32).reshape(-1, 128)
    codes = np.stack([orc.quantize_excode(r, rows[0], 7) for r in rows[1:]])
    mism = (codes != g["excode_l2"]).mean()
    assert mism <= 0.002, mism


def test_best_rescale_factor_brute_force():
    """The priority-queue sweep equals a brute force that evaluates the ratio after every
    increment point in (t, coordinate) order."""
    import math
    rng = np.random.default_rng(31)
    for dim, ex in ((8, 7), (16, 3), (12, 5)):
        for _ in range(20):
            oa = np.abs(rng.normal(size=dim)).astype(np.float32)
            oa /= np.float32(np.linalg.norm(oa))
            cap = (1 << ex) - 1
            t_end = (cap + 10) / float(oa.max())
            t_start = t_end * orc._TIGHT_START[ex]
            c0 = [int(t_start * float(v) + 1e-5) for v in oa]
            pts = []
            for i, v in enumerate(oa.tolist()):
                k, c = 1, c0[i]
                pts.append(((c + 1) / v, i))
                while c + k < cap and (c + k + 1) / v < t_end:
                    pts.append(((c + k + 1) / v, i))
                    k += 1
            pts.sort()
            cur = list(c0)
            num = sum((c + 0.5) * v for c, v in zip(c0, oa.tolist()))
            den = dim * 0.25 + sum(c * c + c for c in c0)
            best, bt = 0.0, 0.0
            for t, i in pts:
                cur[i] += 1
                den += 2 * cur[i]
                num += float(oa[i])
                r = num / math.sqrt(den)
                if r > best:
                    best, bt = r, t
            assert orc.best_rescale_factor(oa, ex) == bt


# --------------------------------------------------------------------------------------
# Exact single-precision arithmetic from rationals (independent of numpy's float32 ops):
# the correctly rounded (nearest, ties to even) float32 of a Fraction.
# --------------------------------------------------------------------------------------
from fractions import Fraction  # noqa: E402


def f32_round(x: Fraction) -> np.float32:
    d = np.float32(float(x))  # within one float32 ulp of x
    best = None
    for c in (np.nextafter(d, np.float32(-np.inf)), d, np.nextafter(d, np.float32(np.inf))):
        err = abs(Fraction(float(c)) - x)
        key = (err, int(np.array(c).view(np.uint32)) & 1)  # ties: even mantissa
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def rint_even(x: Fraction) -> int:
    f = x.numerator // x.denominator
    r = x - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2 == 1):
        f += 1
    return f


def bq8_expected(row):
    """qint of one row by exact rational arithmetic: width = f32(amax / 127),
    inv = f32(1 / width), qint = clamp(rint_even(f32(q * inv)), -128, 127)
    (query_kernels.cuh:158-176)."""
    amax = max(abs(Fraction(float(v))) for v in row)
    width = max(f32_round(amax / 127), np.float32(1e-30))
    inv = f32_round(1 / Fraction(float(width)))
    out = [min(127, max(-128, rint_even(Fraction(float(f32_round(Fraction(float(v)) * Fraction(float(inv))))))))
           for v in row]
    return np.array(out, np.int32), width, inv


def test_quantize_query_reciprocal_product_boundaries():
    """Rows whose components sit next to a rounding boundary of q * (1/width): for each,
    q * f32(1/width) and q / width round to different integers, and the oracle must give
    the former (the reference multiplies by the reciprocal, query_kernels.cuh:158-176)."""
    rng = np.random.default_rng(21)
    found = 0
    for _ in range(400):
        amax = np.float32(rng.uniform(0.1, 50.0))
        row = np.zeros(64, np.float32)
        row[0] = amax
        _, width, inv = bq8_expected(row[:1])
        cases = []
        for k in range(-120, 121, 7):
            c = np.float32((k + 0.5) * float(width))
            for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
                by_inv = rint_even(Fraction(float(f32_round(Fraction(float(cand)) * Fraction(float(inv))))))
                by_div = rint_even(Fraction(float(f32_round(Fraction(float(cand)) / Fraction(float(width))))))
                if by_inv != by_div:
                    cases.append(cand)
        if not cases:
            continue
        row[1:1 + min(63, len(cases))] = cases[:63]
        want, w, _ = bq8_expected(row)
        qint, wo = orc.quantize_query_bitwise(row[None])
        assert wo[0] == w
        assert np.array_equal(qint[0], want)
        found += len(cases)
    assert found >= 20, found


def test_quantize_query_half_even_ties_with_width_not_one():
    """width = 2^-3 (amax = 127/8): 1/width = 8 exactly, so q = (k + 1/2)/8 gives an exact
    tie q * inv = k + 1/2, which rounds to the even neighbour."""
    row = np.zeros(64, np.float32)
    row[0] = np.float32(127.0 / 8.0)
    ties = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]
    row[1:1 + len(ties)] = np.array(ties, np.float32) / np.float32(8.0)
    qint, w = orc.quantize_query_bitwise(row[None])
    assert w[0] == np.float32(0.125)
    assert list(qint[0, :1 + len(ties)]) == [127, 0, 2, 2, 0, -2, -2, 126, -126]


def words_of_bits(bits):
    return orc.bits_to_words_msb(np.asarray(bits, np.uint8))


def test_lut4_table_closed_forms():
    P = 64
    q = np.zeros((1, P), np.float32)
    q[0, :4] = [3.0, -5.0, 0.25, 1024.0]
    # group 1: 1 + 2^-11 rounds to even (1.0) in FP16; 1 + 2^-10 is representable
    q[0, 4:8] = [1.0, 2.0 ** -11, 2.0 ** -11, 0.0]
    # group 2: FP16 overflow (65504 is the largest finite value)
    q[0, 8:12] = [60000.0, 10000.0, 0.0, 0.0]
    t = orc.lut4_table(q)[0].astype(np.float64)
    assert t.shape == (P // 4, 16)
    # single bits: bit 3 of the pattern is the group's first dimension
    assert [t[0, 8], t[0, 4], t[0, 2], t[0, 1]] == [3.0, -5.0, 0.25, 1024.0]
    # all four: 1022.25 is halfway between the FP16 neighbours 1022.0 (even) and 1022.5
    assert t[0, 0] == 0.0 and t[0, 15] == 1022.0
    assert t[1, 0b1100] == 1.0 and t[1, 0b1110] == 1.0 + 2.0 ** -10
    assert np.isinf(t[2, 0b1100]) and t[2, 0b1000] == 60000.0


def test_lut4_ip_accumulation_order_and_nibble_layout():
    """a0 gathers the even nibbles, a1 the odd ones, each in FP32 in nibble order; the
    estimate is a0 + a1. With nibble 0's entry 1.0 and every other nibble's 2^-24, a0 stays
    1.0 (1 + 2^-24 rounds back to 1), a1 sums the odd nibbles exactly, so the result is
    1 + n_odd * 2^-24 rounded once; one accumulator would return 1.0."""
    P = 128  # 32 nibbles: 16 odd ones
    q = np.zeros((1, P), np.float32)
    q[0, 0] = 1.0
    for g in range(1, P // 4):
        q[0, 4 * g] = 2.0 ** -24  # FP16's smallest subnormal
    lut = orc.lut4_table(q)[0]
    bits = np.zeros((1, P), np.uint8)
    bits[0, ::4] = 1  # the first dimension of every group: pattern 8 in every nibble
    got = orc.lut4_ip(words_of_bits(bits), lut)[0]
    assert got == np.float32(1.0 + 16 * 2.0 ** -24)
    # bit layout: a single set dimension d selects the entry of its own nibble
    rng = np.random.default_rng(4)
    qr = rng.normal(0, 1, (1, P)).astype(np.float32)
    t = orc.lut4_table(qr)[0]
    for d in (0, 1, 2, 3, 31, 32, 77, 127):
        b = np.zeros((1, P), np.uint8)
        b[0, d] = 1
        assert orc.lut4_ip(words_of_bits(b), t)[0] == np.float32(np.float16(qr[0, d]))


def test_lut4_ip_equals_exact_sum_for_representable_values():
    """Small integers: every table entry and partial sum is exact in FP16 and FP32, so the
    estimate equals the integer inner product <b, q>."""
    rng = np.random.default_rng(5)
    for P in (64, 128, 768):
        q = rng.integers(-20, 21, (3, P)).astype(np.float32)
        bits = rng.integers(0, 2, (40, P), dtype=np.uint8)
        w = words_of_bits(bits)
        for i in range(3):
            got = orc.lut4_ip(w, orc.lut4_table(q[i:i + 1])[0])
            assert np.array_equal(got, (bits.astype(np.int64) @ q[i].astype(np.int64)).astype(np.float32))
