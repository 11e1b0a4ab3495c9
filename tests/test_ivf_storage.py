"""Index storage forms and the streaming loader (CPU only).

The reference's IVF::load (ivf.hpp:447-539) accepts two files: centroids embedded in the
index, or no centroids there and an hnswlib graph "<index>.hnsw" holding them (written for
nlist >= 20000, initializer.hpp:23,255-279). Both the C++ reader (cora_ivf_load) and the
oracle's read_ivf must give the arrays the reference's IVF::load + SearchData give.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

import cora_oracle as orc
import coraanns_amd as ca
from conftest import GOLDEN, REPO

REF_BIN = REPO / "oracle" / "_ref"
HNSW_HDR = struct.Struct("<6QiI3QdQ")


def _arrays(ivf):
    return {k: np.array(getattr(ivf, k)) for k in
            ("centroids", "rotator", "short_data", "short_factors", "long_codes", "ex_factors", "ids",
             "cluster_sizes")}


def _same(a, b):
    assert a.keys() == b.keys()
    for k in a:
        assert a[k].shape == b[k].shape, k
        assert np.array_equal(a[k].view(np.uint8), b[k].view(np.uint8)), k


def write_sidecar(src, dst, perm, maxm0=6, upper=None, label_of=None, vec_floats=None):
    """Rewrite the embedded-centroid index `src` as `dst` (no centroids) plus `dst`.hnsw in
    hnswlib's saveIndex layout. Internal element i holds centroid perm[i] with label
    label_of(i) (default perm[i]); level-0 link bytes are filler (the loader does not read
    the graph); upper[i] is element i's upper-level link byte count."""
    f = orc.read_ivf(src)
    raw = np.fromfile(src, dtype=np.uint8)
    off = 34 + 8 * f.nlist + 4 * f.dim * f.padded_dim
    cent_bytes = 4 * f.padded_dim * f.nlist
    with open(dst, "wb") as fh:
        fh.write(raw[:off].tobytes())
        fh.write(raw[off + cent_bytes:].tobytes())
    P = f.padded_dim
    nv = P if vec_floats is None else vec_floats
    links0 = 4 + 4 * maxm0
    per = links0 + 4 * nv + 8
    n = f.nlist
    hdr = HNSW_HDR.pack(0, n, n, per, links0 + 4 * nv, links0, 1, 0, maxm0 // 2, maxm0, maxm0 // 2,
                        1.0 / np.log(maxm0 // 2), 200)
    rng = np.random.default_rng(5)
    el = np.zeros((n, per), np.uint8)
    el[:, :links0] = rng.integers(0, 256, (n, links0), dtype=np.uint8)
    for i in range(n):
        v = np.zeros(nv, np.float32)
        v[:min(nv, P)] = f.centroids[perm[i]][:min(nv, P)]
        el[i, links0:links0 + 4 * nv] = v.view(np.uint8)
        lab = perm[i] if label_of is None else label_of(i)
        el[i, links0 + 4 * nv:] = np.frombuffer(struct.pack("<Q", lab), np.uint8)
    upper = [0] * n if upper is None else upper
    with open(str(dst) + ".hnsw", "wb") as fh:
        fh.write(hdr)
        fh.write(el.tobytes())
        for u in upper:
            fh.write(struct.pack("<I", u))
            fh.write(bytes(u))
    return f


@pytest.mark.parametrize("name", ["l2_d96", "ip_d64"])
def test_sidecar_index_equals_embedded(tmp_path, name):
    src = GOLDEN / name / "ivf.index"
    f = orc.read_ivf(src)
    perm = np.random.default_rng(1).permutation(f.nlist)
    dst = tmp_path / "side.index"
    write_sidecar(src, dst, perm, upper=[(i % 3) * 20 for i in range(f.nlist)])
    emb, side = ca.IvfIndex(src), ca.IvfIndex(dst)
    assert emb.centroid_storage == "embedded" and side.centroid_storage == "hnsw_sidecar"
    _same(_arrays(emb), _arrays(side))
    o = orc.read_ivf(dst)
    assert np.array_equal(o.centroids.view(np.uint32), f.centroids.view(np.uint32))
    lazy = orc.open_ivf_lazy(dst)
    assert np.array_equal(lazy.centroids.view(np.uint32), f.centroids.view(np.uint32))


@pytest.mark.parametrize("chunk", ["1", "700", "5000"])
@pytest.mark.parametrize("sidecar", [False, True])
def test_streaming_chunks_give_the_same_arrays(tmp_path, monkeypatch, chunk, sidecar):
    src = GOLDEN / "l2_d96" / "ivf.index"
    path = src
    if sidecar:
        f = orc.read_ivf(src)
        path = tmp_path / "side.index"
        write_sidecar(src, path, np.arange(f.nlist)[::-1].copy())
    want = _arrays(ca.IvfIndex(path))
    monkeypatch.setenv("CORA_IVF_CHUNK_BYTES", chunk)
    _same(want, _arrays(ca.IvfIndex(path)))
    # short codes only (exact-refine mode) reads no ex data
    short = ca.IvfIndex(path, include_extended=False)
    assert short.long_codes is None
    assert np.array_equal(short.short_data, want["short_data"])


def _expect_reject(dst):
    with pytest.raises(ca.EngineError):
        ca.IvfIndex(dst)
    with pytest.raises((ValueError, FileNotFoundError)):
        orc.read_ivf(dst)


def test_sidecar_rejections(tmp_path):
    src = GOLDEN / "ip_d64" / "ivf.index"
    f = orc.read_ivf(src)
    n = f.nlist
    ident = np.arange(n)
    cases = {
        "duplicate_label": dict(label_of=lambda i: 0 if i == 1 else i),
        "label_out_of_range": dict(label_of=lambda i: n if i == n - 1 else i),
        "other_dimension": dict(vec_floats=f.padded_dim - 32),
    }
    for tag, kw in cases.items():
        dst = tmp_path / f"{tag}.index"
        write_sidecar(src, dst, ident, **kw)
        _expect_reject(dst)
    # missing sidecar
    dst = tmp_path / "missing.index"
    write_sidecar(src, dst, ident)
    os.remove(str(dst) + ".hnsw")
    _expect_reject(dst)
    # element count other than nlist, link lists cut short, trailing bytes
    for tag in ("count", "cut", "trailing"):
        dst = tmp_path / f"{tag}.index"
        write_sidecar(src, dst, ident, upper=[8] * n)
        side = str(dst) + ".hnsw"
        raw = bytearray(open(side, "rb").read())
        if tag == "count":
            raw[16:24] = struct.pack("<Q", n - 1)
        elif tag == "cut":
            raw = raw[:-5]
        else:
            raw += b"\0\0\0"
        open(side, "wb").write(bytes(raw))
        _expect_reject(dst)
    # a main file that matches neither layout
    dst = tmp_path / "odd.index"
    dst.write_bytes(src.read_bytes() + b"\0" * 4)
    _expect_reject(dst)


@pytest.mark.skipif(not ((REF_BIN / "coraanns_build_index").exists() and (REF_BIN / "ref_dump").exists()),
                    reason="reference CPU path not built (make -C oracle ref)")
def test_reference_built_sidecar_index(tmp_path):
    """An index the reference's own builder writes with an HNSW sidecar (nlist 20,000 >=
    kHnswInitializerThreshold) reads into the arrays the reference's IVF::load + SearchData
    dump, through the C++ loader and through the oracle."""
    rng = np.random.default_rng(0)
    n, d, nl = 6000, 32, 20000
    c = rng.normal(0, 1, (nl, d)).astype(np.float32)
    x = (c[rng.integers(0, nl, n)] + 0.1 * rng.normal(0, 1, (n, d))).astype(np.float32)
    assign = ((c * c).sum(1)[None, :] - 2.0 * (x @ c.T)).argmin(1).astype(np.uint32)

    def fvecs(path, a):
        rows = np.empty((a.shape[0], a.shape[1] + 1), np.uint32)
        rows[:, 0] = a.shape[1]
        rows[:, 1:] = a.view(np.uint32)
        rows.tofile(path)

    fvecs(tmp_path / "x.fvecs", x)
    fvecs(tmp_path / "c.fvecs", c)
    fvecs(tmp_path / "ids.ivecs", assign[:, None])
    idx = tmp_path / "side.index"
    subprocess.run([str(REF_BIN / "coraanns_build_index"), str(tmp_path / "x.fvecs"), str(tmp_path / "c.fvecs"),
                    str(tmp_path / "ids.ivecs"), "8", str(idx), "l2"], check=True, capture_output=True)
    assert (tmp_path / "side.index.hnsw").exists()
    q = x[:4]
    qf = tmp_path / "q.fbin"
    with open(qf, "wb") as fh:
        fh.write(np.array(q.shape, np.uint32).tobytes())
        fh.write(q.tobytes())
    out = tmp_path / "dump"
    out.mkdir()
    subprocess.run([str(REF_BIN / "ref_dump"), "index", str(idx), str(qf), str(out), "5", "4"], check=True,
                   capture_output=True)
    import conftest
    old = conftest.GOLDEN
    try:
        conftest.GOLDEN = tmp_path
        ref = conftest.load_golden("dump")
    finally:
        conftest.GOLDEN = old
    ivf = ca.IvfIndex(idx)
    assert ivf.centroid_storage == "hnsw_sidecar"
    got = _arrays(ivf)
    for k in got:
        assert np.array_equal(got[k].reshape(-1).view(np.uint8), ref[k].reshape(-1).view(np.uint8)), k
    o = orc.read_ivf(idx)
    assert np.array_equal(o.centroids.view(np.uint32), ref["centroids"].view(np.uint32))
    assert np.array_equal(o.ids, ref["ids"])
