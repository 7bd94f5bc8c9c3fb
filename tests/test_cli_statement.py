"""CPU tests of zkml-prove's statement-v2 front end (cuda-zkml_amd/cli/prove.cpp,
model_files.hpp) against the reference's own front end (src/cli/prove.cu,
compiled in oracle/_ref/libzkref_cli.so).

zkml-prove runs with --device 99 (no such GPU): it parses the model and
inputs, builds the statement, checks the witness and writes --export-r1cs /
--export-wtns before it opens a device, then stops with exit status 1.  The
exported files carry the quantized-model tag as a public input, so equal
bytes pin the architecture parser, the int32 loader, the .npy / .bin input
loaders, the hex parser and the tag together with the statement builder.
The oracle/_ref comparisons run the reference's host code compiled in place
with the reference's own CUDA-runtime test shim (tests/host/shim).  They are
cross-checks and pin nothing by themselves: these tests skip without it, and the
statement builder behind the front end is pinned without it in
tests/test_statement_pins.py.
"""
import os
import re
import subprocess

import numpy as np
import pytest

from cli_models import (PROVE, digits_cnn, ref_cli_available, ref_statement, small_mlp, write_model,
                        write_sample)

needs_ref_cli = pytest.mark.skipif(not ref_cli_available(), reason="oracle/_ref not built (needs /root/reference)")


def run_prove(args, tmp):
    r1cs, wtns = os.path.join(tmp, "ours.r1cs"), os.path.join(tmp, "ours.wtns")
    p = subprocess.run([PROVE, "--statement-v2", "--integer-model", "--integer-input", "--device", "99",
                        "--export-r1cs", r1cs, "--export-wtns", wtns] + args, capture_output=True, text=True,
                       timeout=120)
    return p, r1cs, wtns


def tag_of(stdout):
    m = re.search(r"Quantized model tag: (0x[0-9a-f]+)", stdout)
    return int(m.group(1), 16) if m else None


CASES = {
    "cnn_public": dict(),
    "cnn_context_route": dict(context="0x1234abcd", route_threshold=3),
    "cnn_private_all": dict(private_input=True, blinding=["0x5eed1"], private_model=True, private_outputs=True,
                            route_threshold=2),
}


@needs_ref_cli
@pytest.mark.parametrize("case", sorted(CASES))
def test_cnn_statement_matches_reference_front_end(case, tmp_path):
    opt = CASES[case]
    layers, params = digits_cnn()
    arch, model = write_model(str(tmp_path), layers, params)
    rng = np.random.default_rng(7)
    x = write_sample(str(tmp_path / "x.npy"), rng.integers(0, 17, 64))
    rc, info, tag, meta = ref_statement(arch, model, [x], str(tmp_path / "ref.r1cs"), str(tmp_path / "ref.wtns"),
                                        **opt)
    assert rc == 0 and info[3] == 1
    args = ["--model", model, "--arch", arch, "--input", x]
    if "context" in opt:
        args += ["--context", opt["context"]]
    if opt.get("private_input"):
        args += ["--private-input", "--input-blinding", ",".join(opt["blinding"])]
    if opt.get("private_model"):
        args += ["--private-model"]
    if opt.get("private_outputs"):
        args += ["--private-outputs"]
    if "route_threshold" in opt:
        args += ["--route-threshold", str(opt["route_threshold"])]
    p, r1cs, wtns = run_prove(args, str(tmp_path))
    assert tag_of(p.stdout) == tag, p.stdout + p.stderr
    assert f"R1CS: {info[0]} constraints, {info[1]} variables, {info[2]} public" in p.stdout
    assert open(r1cs, "rb").read() == open(tmp_path / "ref.r1cs", "rb").read()
    assert open(wtns, "rb").read() == open(tmp_path / "ref.wtns", "rb").read()
    assert p.returncode == 1  # no device 99


@needs_ref_cli
@pytest.mark.parametrize("relu", ["relu_exact", "relu_approx"])
def test_mlp_batch_statement_matches_reference_front_end(relu, tmp_path):
    layers, params = small_mlp(relu=relu)
    arch, model = write_model(str(tmp_path), layers, params, name="mlp")
    rng = np.random.default_rng(11)
    xs = [write_sample(str(tmp_path / f"x{i}.bin"), rng.integers(-5, 9, 5)) for i in range(3)]
    rc, info, tag, meta = ref_statement(arch, model, xs, str(tmp_path / "ref.r1cs"), str(tmp_path / "ref.wtns"),
                                        private_input=True, blinding=["0xa", "0xb", "0xc"], route_threshold=-1)
    assert rc == 0
    # architecture found next to the model (MODEL.int32.bin.arch.json is the reference's fallback name)
    os.rename(arch, model + ".arch.json")
    p, r1cs, wtns = run_prove(["--model", model, "--batch-inputs", ",".join(xs), "--private-input",
                               "--input-blinding", "0xa,0xb,0xc", "--route-threshold", "-1"], str(tmp_path))
    assert tag_of(p.stdout) == tag, p.stdout + p.stderr
    assert open(r1cs, "rb").read() == open(tmp_path / "ref.r1cs", "rb").read()
    assert open(wtns, "rb").read() == open(tmp_path / "ref.wtns", "rb").read()


def test_front_end_rejections(tmp_path):
    layers, params = small_mlp()
    arch, model = write_model(str(tmp_path), layers, params, name="mlp")
    x = write_sample(str(tmp_path / "x.npy"), [1, 2, 3, 4, 5])
    base = ["--model", model, "--arch", arch, "--input", x]

    def fails(args, text, v2=True):
        cmd = [PROVE] + (["--statement-v2", "--integer-model", "--integer-input"] if v2 else []) + args
        p = subprocess.run(cmd + ["--device", "99"], capture_output=True, text=True, timeout=60)
        assert p.returncode == 1 and text in p.stderr, (args, p.stdout, p.stderr)

    fails(base + ["--context", "xyz"], "--context expects a hex value")
    fails(["--model", model, "--context", "0x1"], "require --statement-v2", v2=False)
    fails(base + ["--private-outputs"], "private_outputs requires route")
    fails(base + ["--private-input"], "one blinding value per sample")
    fails(base + ["--private-input", "--input-blinding", "0xq"], "bad --input-blinding value")
    bad = write_sample(str(tmp_path / "bad.npy"), [1.5, 2, 3, 4, 5])
    fails(["--model", model, "--arch", arch, "--input", bad], "Cannot load batch input")
    short = write_sample(str(tmp_path / "short.npy"), [1, 2])
    fails(["--model", model, "--arch", arch, "--input", short], "Cannot load batch input")
    np.asarray(list(params) + [7], dtype=np.int32).tofile(str(tmp_path / "long.int32.bin"))
    fails(["--model", str(tmp_path / "long.int32.bin"), "--arch", arch, "--input", x], "1 trailing values")
    p = subprocess.run([PROVE, "--statement-v2", "--model", model, "--arch", arch, "--input", x, "--device", "99"],
                       capture_output=True, text=True, timeout=60)
    assert p.returncode == 1 and "--integer-model" in p.stderr
    with open(tmp_path / "bad.arch.json", "w") as f:
        f.write('{"layers": [{"type": "relu_exact", "in_features": 4, "out_features": 4, "bits": 70}]}')
    fails(["--model", model, "--arch", str(tmp_path / "bad.arch.json"), "--input", x], "relu_exact needs")
