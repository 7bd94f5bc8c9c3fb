"""Model / input files for zkml-prove's statement-v2 path (architecture
sidecar, int32 parameters, float32 .npy / .bin samples) and the bindings of
the reference front end compiled in oracle/_ref/libzkref_cli.so."""
import ctypes
import json
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_CLI_SO = os.path.join(ROOT, "oracle", "_ref", "libzkref_cli.so")
PROVE = os.path.join(ROOT, "cuda-zkml_amd", "zkml-prove")
VERIFY = os.path.join(ROOT, "cuda-zkml_amd", "zkml-verify")

_lib = None


def ref_cli_available():
    return os.path.exists(REF_CLI_SO)


def ref_cli():
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(REF_CLI_SO, mode=os.RTLD_LAZY)
        vp = ctypes.c_void_p
        lib.ref_cli_statement_v2.argtypes = [ctypes.c_char_p] * 4 + [ctypes.c_int, ctypes.c_char_p] + \
            [ctypes.c_int] * 3 + [ctypes.c_longlong, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                                  ctypes.c_size_t, vp, vp]
        _lib = lib
    return _lib


def ref_statement(arch, model, inputs, r1cs, wtns, context=None, private_input=False, blinding=None,
                  private_model=False, private_outputs=False, route_threshold=None):
    info = np.zeros(4, dtype=np.int32)
    tag = np.zeros(1, dtype=np.uint64)
    meta = ctypes.create_string_buffer(8192)
    enc = lambda s: s.encode() if s is not None else None  # noqa: E731
    rc = ref_cli().ref_cli_statement_v2(enc(arch), enc(model), enc(",".join(inputs)), enc(context),
                                        int(private_input), enc(",".join(blinding) if blinding else None),
                                        int(private_model), int(private_outputs), int(route_threshold is not None),
                                        int(route_threshold or 0), r1cs.encode(), wtns.encode(), meta, 8192,
                                        info.ctypes.data, tag.ctypes.data)
    return rc, info, int(tag[0]), meta.value.decode()


def write_model(d, layers, params, name="model"):
    """layers: architecture dicts; params: int32 values in load_integer_weights order."""
    os.makedirs(d, exist_ok=True)
    mp = os.path.join(d, f"{name}.int32.bin")
    ap = os.path.join(d, f"{name}.arch.json")
    np.asarray(params, dtype=np.int32).tofile(mp)
    with open(ap, "w") as f:
        json.dump({"name": name, "layers": layers}, f, indent=2)
    return ap, mp


def write_sample(path, values):
    a = np.asarray(values, dtype=np.float32)
    if path.endswith(".npy"):
        np.save(path, a)
    else:
        a.tofile(path)
    return path


def digits_cnn(seed=1):
    """BASELINE config 4's shape (8x8 input, four 3x3 filters, exact ReLU,
    256 -> 10), as the reference's run_phase12_e2e.py write_cnn."""
    rng = np.random.default_rng(seed)
    layers = [
        {"type": "conv2d", "in_features": 64, "out_features": 4 * 64, "in_channels": 1, "in_height": 8,
         "in_width": 8, "out_channels": 4, "kernel_size": 3, "stride": 1, "padding": 1},
        {"type": "relu_exact", "in_features": 256, "out_features": 256, "bits": 16, "shift": 3},
        {"type": "linear", "in_features": 256, "out_features": 10},
        {"type": "softmax", "in_features": 10, "out_features": 10},
    ]
    params = np.concatenate([rng.integers(-4, 5, 36), rng.integers(-8, 9, 4),
                             rng.integers(-3, 4, 2560), rng.integers(-16, 17, 10)]).astype(np.int32)
    return layers, params


def small_mlp(seed=2, relu="relu_exact"):
    rng = np.random.default_rng(seed)
    hidden = 6
    layers = [{"type": "linear", "in_features": 5, "out_features": hidden}]
    if relu == "relu_exact":
        layers.append({"type": "relu_exact", "in_features": hidden, "out_features": hidden, "bits": 20,
                       "shift": 2})
    else:
        layers.append({"type": "RELU", "in_features": hidden, "out_features": hidden})
    layers += [{"type": "linear", "in_features": hidden, "out_features": 3},
               {"type": "softmax_approx", "in_features": 3, "out_features": 3}]
    params = np.concatenate([rng.integers(-20, 21, 5 * hidden), rng.integers(-100, 101, hidden),
                             rng.integers(-9, 10, hidden * 3), rng.integers(-50, 51, 3)]).astype(np.int32)
    return layers, params
