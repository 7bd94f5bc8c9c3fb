"""CPU checks of the committed BASELINE config 1 / config 4 statements
(tests/golden/statements): they load through the product's iden3 readers
with the recorded hashes and sizes, and the witnesses satisfy the R1CS under
the oracle's checker and the reference's own R1CS::verify_witness."""
import numpy as np
import pytest

from bindings import OracleR1CS, ptr, ref, ref_available
from statements import load, meta


@pytest.mark.parametrize("name", ["config1", "config4"])
def test_statement_fixture(name):
    m = meta()[name]
    nc, nv, npub, npriv, A, B, C, w = load(name)
    assert (nc, nv, npub) == (m["constraints"], m["variables"], m["public"])
    assert w.shape == (nv, 4)
    mats = [(M["row"], M["col"], M["value"].reshape(-1, 4)) for M in (A, B, C)]
    oc = OracleR1CS(nc, nv, npub, npriv, mats)
    assert oc.verify(w)
    if ref_available():
        rows = np.concatenate([M["row"] for M in (A, B, C)]).astype(np.int32)
        cols = np.concatenate([M["col"] for M in (A, B, C)]).astype(np.int32)
        vals = np.ascontiguousarray(np.concatenate([M["value"] for M in (A, B, C)]), dtype=np.uint64)
        counts = np.array([len(A), len(B), len(C)], dtype=np.uint64)
        assert ref().ref_verify_witness(nc, nv, ptr(rows), ptr(cols), ptr(vals), ptr(counts),
                                        ptr(np.ascontiguousarray(w))) == 1
