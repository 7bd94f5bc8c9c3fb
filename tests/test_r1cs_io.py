"""CPU tests of the iden3 .r1cs / .wtns codecs and the config-5 synthetic R1CS
of the product library (cuda-zkml_amd/csrc/r1cs_io.cpp).

Pins:
  export       byte-identical to the reference's own writers
               (export_r1cs_iden3 / export_wtns_iden3, src/prover/
               r1cs_export.cuh, compiled in oracle/_ref) for the same R1CS and
               witness, including rows given out of order;
  format       an independent reader written here from the iden3 format
               description (magic, version, sections; header fields; per row
               three linear combinations of (wire u32, coefficient 32 B));
  round trip   read(write(x)) == x for matrices (per row, term order kept)
               and witnesses; malformed files are rejected;
  synthetic    the generated witness satisfies the R1CS under the oracle's
               checker and the reference's R1CS::verify_witness; determinism
               by seed; sizes as documented.
The oracle/_ref comparisons run the reference's host code compiled in place
with the reference's own CUDA-runtime test shim (tests/host/shim).  They are
cross-checks and pin nothing by themselves: the codecs are pinned by the
independent reader and the round trips.
"""
import os
import struct

import numpy as np
import pytest

import zkml_amd
from bindings import OracleR1CS, ptr, ref, ref_available
from r1cs_gen import random_r1cs
from zkpy import R as ORDER

MONT = 1 << 256
needs_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs /root/reference)")


def mont_to_std(w):
    return sum(int(w[k]) << (64 * k) for k in range(4)) * pow(MONT, -1, ORDER) % ORDER


def circuit_mats(circ, shuffle_seed=None):
    A, B, C = (zkml_amd.sparse_entries(*m) for m in circ.mats())
    if shuffle_seed is not None:
        rng = np.random.default_rng(shuffle_seed)
        A, B, C = (M[rng.permutation(len(M))] for M in (A, B, C))
    return A, B, C


def parse_r1cs(path):
    """Independent reader of the iden3 .r1cs layout."""
    d = open(path, "rb").read()
    assert d[:4] == b"r1cs"
    ver, nsec = struct.unpack_from("<II", d, 4)
    assert ver == 1
    off, secs = 12, {}
    for _ in range(nsec):
        t, ln = struct.unpack_from("<IQ", d, off)
        secs[t] = d[off + 12: off + 12 + ln]
        off += 12 + ln
    assert off == len(d)
    h = secs[1]
    n8 = struct.unpack_from("<I", h, 0)[0]
    prime = int.from_bytes(h[4:36], "little")
    nw, npo, npi, npr = struct.unpack_from("<IIII", h, 36)
    nlab, m = struct.unpack_from("<QI", h, 52)
    rows, o, c = [], 0, secs[2]
    for _ in range(m):
        lcs = []
        for _k in range(3):
            (nt,) = struct.unpack_from("<I", c, o)
            o += 4
            lc = []
            for _t in range(nt):
                (wire,) = struct.unpack_from("<I", c, o)
                lc.append((wire, int.from_bytes(c[o + 4:o + 36], "little")))
                o += 36
            lcs.append(lc)
        rows.append(lcs)
    assert o == len(c)
    labels = struct.unpack_from(f"<{nw}Q", secs[3], 0)
    return dict(n8=n8, prime=prime, nwires=nw, npubout=npo, npubin=npi, nprvin=npr, nlabels=nlab, m=m,
                rows=rows, labels=labels)


def by_row(M, m):
    out = [[] for _ in range(m)]
    for e in M:
        out[int(e["row"])].append((int(e["col"]), mont_to_std(e["value"])))
    return out


@needs_ref
@pytest.mark.parametrize("shuffle", [None, 3])
def test_r1cs_export_matches_reference_bytes(tmp_path, shuffle):
    circ = random_r1cs(60, npub=4, seed=21)
    A, B, C = circuit_mats(circ, shuffle)
    ours, theirs = str(tmp_path / "ours.r1cs"), str(tmp_path / "ref.r1cs")
    zkml_amd.iden3_r1cs_write(ours, circ.nc, circ.nv, circ.npub, circ.npriv, A, B, C)
    rows = np.concatenate([M["row"] for M in (A, B, C)]).astype(np.int32)
    cols = np.concatenate([M["col"] for M in (A, B, C)]).astype(np.int32)
    vals = np.ascontiguousarray(np.concatenate([M["value"] for M in (A, B, C)]), dtype=np.uint64)
    counts = np.array([len(A), len(B), len(C)], dtype=np.uint64)
    assert ref().ref_export_r1cs(circ.nc, circ.nv, circ.npub, circ.npriv, ptr(rows), ptr(cols), ptr(vals),
                                 ptr(counts), theirs.encode()) == 1
    assert open(ours, "rb").read() == open(theirs, "rb").read()


@needs_ref
def test_wtns_export_matches_reference_bytes(tmp_path):
    circ = random_r1cs(40, npub=2, seed=22)
    w = np.ascontiguousarray(circ.witness_words(), dtype=np.uint64)
    ours, theirs = str(tmp_path / "ours.wtns"), str(tmp_path / "ref.wtns")
    zkml_amd.wtns_write(ours, w)
    assert ref().ref_export_wtns(ptr(w), w.shape[0], theirs.encode()) == 1
    assert open(ours, "rb").read() == open(theirs, "rb").read()


def test_r1cs_format_and_round_trip(tmp_path):
    circ = random_r1cs(50, npub=3, seed=23)
    A, B, C = circuit_mats(circ, 5)
    path = str(tmp_path / "c.r1cs")
    zkml_amd.iden3_r1cs_write(path, circ.nc, circ.nv, circ.npub, circ.npriv, A, B, C)
    f = parse_r1cs(path)
    assert f["n8"] == 32 and f["prime"] == ORDER
    assert (f["nwires"], f["npubout"], f["npubin"], f["nprvin"], f["nlabels"], f["m"]) == \
        (circ.nv, circ.npub, 0, circ.npriv, circ.nv, circ.nc)
    assert list(f["labels"]) == list(range(circ.nv))
    for k, M in enumerate((A, B, C)):
        assert [r[k] for r in f["rows"]] == by_row(M, circ.nc)
    nc, nv, npub, npriv, A2, B2, C2 = zkml_amd.iden3_r1cs_read(path)
    assert (nc, nv, npub, npriv) == (circ.nc, circ.nv, circ.npub, circ.npriv)
    for M, M2 in ((A, A2), (B, B2), (C, C2)):
        assert by_row(M, nc) == by_row(M2, nc)


def test_wtns_round_trip_and_rejects(tmp_path):
    circ = random_r1cs(30, npub=2, seed=24)
    w = circ.witness_words()
    path = str(tmp_path / "w.wtns")
    zkml_amd.wtns_write(path, w)
    assert np.array_equal(zkml_amd.wtns_read(path), w)
    d = bytearray(open(path, "rb").read())
    bad = tmp_path / "bad.wtns"
    bad.write_bytes(bytes(d[:-1]))  # truncated
    with pytest.raises(zkml_amd.ZkError):
        zkml_amd.wtns_read(str(bad))
    d2 = bytearray(d)
    d2[24] ^= 1  # prime field changed
    bad.write_bytes(bytes(d2))
    with pytest.raises(zkml_amd.ZkError):
        zkml_amd.wtns_read(str(bad))


def test_r1cs_rejects_malformed(tmp_path):
    circ = random_r1cs(10, npub=1, seed=25)
    A, B, C = circuit_mats(circ)
    path = tmp_path / "c.r1cs"
    zkml_amd.iden3_r1cs_write(str(path), circ.nc, circ.nv, circ.npub, circ.npriv, A, B, C)
    d = open(path, "rb").read()
    for bad in (d[:-5], b"r1cx" + d[4:], d[:4] + struct.pack("<I", 2) + d[8:]):
        path.write_bytes(bad)
        with pytest.raises(zkml_amd.ZkError):
            zkml_amd.iden3_r1cs_read(str(path))


def test_synthetic_r1cs_satisfied_and_deterministic():
    nc, npub, ninp = 3000, 4, 16
    A, B, C, w = zkml_amd.synthetic_r1cs(nc, npub, ninp, 7)
    nv = 1 + npub + ninp + nc
    assert w.shape == (nv, 4)
    assert len(C) == nc and nc <= len(A) <= 3 * nc and nc <= len(B) <= 3 * nc
    assert (A["col"] < nv).all() and (C["col"] == np.arange(1 + npub + ninp, nv)).all()
    mats = [(M["row"], M["col"], M["value"].reshape(-1, 4)) for M in (A, B, C)]
    oc = OracleR1CS(nc, nv, npub, ninp, mats)
    assert oc.verify(w)
    w_bad = w.copy()
    w_bad[-1, 0] ^= 1
    assert not oc.verify(w_bad)
    if ref_available():
        rows = np.concatenate([M["row"] for M in (A, B, C)]).astype(np.int32)
        cols = np.concatenate([M["col"] for M in (A, B, C)]).astype(np.int32)
        vals = np.ascontiguousarray(np.concatenate([M["value"] for M in (A, B, C)]), dtype=np.uint64)
        counts = np.array([len(A), len(B), len(C)], dtype=np.uint64)
        assert ref().ref_verify_witness(nc, nv, ptr(rows), ptr(cols), ptr(vals), ptr(counts),
                                        ptr(np.ascontiguousarray(w))) == 1
    A2, B2, C2, w2 = zkml_amd.synthetic_r1cs(nc, npub, ninp, 7)
    assert np.array_equal(w, w2) and np.array_equal(A, A2) and np.array_equal(B, B2)
    assert not np.array_equal(zkml_amd.synthetic_r1cs(nc, npub, ninp, 8)[3], w)
