"""Write the BASELINE config 1 and config 4 statements as iden3 fixtures.

Both are built by the reference's own statement builder (build_statement_v2,
src/prover/statement_v2.cuh, compiled from the reference sources into
oracle/_ref/libzkref.so by `make -C oracle ref`) and written with its own
exporters (export_r1cs_iden3 / export_wtns_iden3), then xz-compressed:

  config1  quantized MLP 64 -> 32 -> 10, int8 weights U[-127, 127], int32
           biases, uint8 inputs U[0, 16], RELU_EXACT(34 bits, shift 8),
           public model / inputs / outputs, 3 samples, std::mt19937_64(42)
  config4  the reference's tiny CNN as statement variant B (private model and
           inputs under Poseidon commitments, private outputs, in-circuit
           routing), tests/host/test_statement_v2.cpp:28-43 and :129-137

    python tests/golden/statements/make_statements.py      (this container only)
"""
import hashlib
import json
import lzma
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from bindings import ref  # noqa: E402


def main():
    lib = ref()
    meta = {}
    with tempfile.TemporaryDirectory() as td:
        jobs = {
            "config1": lambda r, w, info: lib.ref_statement_mlp(42, 3, 64, 32, 10, 34, 8, r, w, info),
            "config4": lambda r, w, info: lib.ref_statement_tiny_cnn_b(r, w, info),
        }
        for name, fn in jobs.items():
            r1cs, wtns = os.path.join(td, name + ".r1cs"), os.path.join(td, name + ".wtns")
            info = np.zeros(3, dtype=np.int32)
            rc = fn(r1cs.encode(), wtns.encode(), info.ctypes.data)
            assert rc == 0, (name, rc)
            entry = {"constraints": int(info[0]), "variables": int(info[1]), "public": int(info[2])}
            for src, ext in ((r1cs, "r1cs"), (wtns, "wtns")):
                data = open(src, "rb").read()
                entry[ext + "_sha256"] = hashlib.sha256(data).hexdigest()
                with open(os.path.join(HERE, f"{name}.{ext}.xz"), "wb") as f:
                    f.write(lzma.compress(data, preset=9))
            meta[name] = entry
            print(name, entry)
    with open(os.path.join(HERE, "statements.json"), "w") as f:
        json.dump(meta, f, indent=1)


if __name__ == "__main__":
    main()
