"""Loader of the committed BASELINE config 1 / config 4 statement fixtures
(tests/golden/statements/*.xz, written by make_statements.py there)."""
import hashlib
import json
import lzma
import os
import tempfile

import zkml_amd

DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "statements")


def meta():
    return json.load(open(os.path.join(DIR, "statements.json")))


def load(name, check_hash=True):
    """(nc, nv, npub, npriv, A, B, C, w) of a fixture, through the product's
    iden3 readers."""
    m = meta()[name]
    with tempfile.TemporaryDirectory() as td:
        paths = {}
        for ext in ("r1cs", "wtns"):
            data = lzma.decompress(open(os.path.join(DIR, f"{name}.{ext}.xz"), "rb").read())
            if check_hash:
                assert hashlib.sha256(data).hexdigest() == m[ext + "_sha256"], (name, ext)
            paths[ext] = os.path.join(td, f"{name}.{ext}")
            open(paths[ext], "wb").write(data)
        nc, nv, npub, npriv, A, B, C = zkml_amd.iden3_r1cs_read(paths["r1cs"])
        w = zkml_amd.wtns_read(paths["wtns"])
    return nc, nv, npub, npriv, A, B, C, w
