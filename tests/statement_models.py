"""The models of the committed statement fixtures, rebuilt in Python for the
product's statement builder (zkml_amd.statement_v2).

  config1  tests/golden/statements/make_statements.py: quantized MLP
           64 -> 32 -> 10 drawn from std::mt19937_64(42) in the order of the
           fixture generator (weights rng() % 255 - 127, biases
           (int32)(uint32) rng() per linear layer, then inputs rng() % 17),
           RELU_EXACT(34, 8), 3 samples, statement v2 defaults.
  config4  the reference's tiny CNN (tests/host/test_statement_v2.cpp:28-43)
           as statement variant B (:129-137): the published 62,692-constraint
           private statement, the bench's 2^16 proof.
  config4_named  BASELINE config 4's network as written: a 1x8x8 uint8
           input, CONV2D with four 3x3 int8 filters (stride 1, no padding ->
           4x6x6 = 144), RELU_EXACT, LINEAR 144 -> 32, RELU_EXACT, LINEAR
           32 -> 10; private model and input under Poseidon commitments,
           private outputs, in-circuit top-1/top-2 routing; one sample.
"""
import numpy as np

import zkml_amd as z
from mt64 import MT19937_64


def mlp(seed=42, batch=3, n_in=64, hidden=32, n_out=10, bits=34, shift=8):
    rng = MT19937_64(seed)
    dims = [(n_in, hidden), (hidden, n_out)]
    params = []
    for i, o in dims:
        w = [int(rng() % 255) - 127 for _ in range(i * o)]
        b = [int(np.uint32(rng() & 0xFFFFFFFF).astype(np.int32)) for _ in range(o)]
        params.append((w, b))
    xs = [[int(rng() % 17) for _ in range(n_in)] for _ in range(batch)]
    layers = [z.layer_linear(n_in, hidden, *params[0]), z.layer_relu_exact(hidden, bits, shift),
              z.layer_linear(hidden, n_out, *params[1]), z.layer_softmax(n_out)]
    return layers, xs


def tiny_cnn():
    cw = [((i * 5) % 7) - 3 for i in range(2 * 1 * 3 * 3)]
    lw = [((i * 3) % 9) - 4 for i in range(72 * 4)]
    layers = [z.layer_conv2d(1, 6, 6, 2, 3, 3, 1, 1, cw, [4, -2]), z.layer_relu_exact(72, 24, 2),
              z.layer_linear(72, 4, lw, [i - 1 for i in range(4)]), z.layer_softmax(4)]
    xs = [[(i * 7) % 13 - 4 for i in range(36)], [(i * 11) % 17 - 8 for i in range(36)]]
    return layers, xs


def config1():
    layers, xs = mlp()
    return z.statement_v2(layers, xs)


def config4():
    layers, xs = tiny_cnn()
    return z.statement_v2(layers, xs, model_tag=0xC0FFEE, private_input=True, input_blinding=[0x5EED1, 0x5EED2],
                          private_model=True, private_outputs=True, route_threshold=5)


def cnn_private(seed=44):
    """BASELINE config 4's network, drawn from std::mt19937_64(seed) in layer
    order: weights rng() % 255 - 127 (int8), biases (int32)(uint32) rng(),
    then the input rng() % 256 (uint8).  RELU_EXACT(34, 8) after the
    convolution (|z| < 9 * 127 * 255 + 2^31 < 2^33) and RELU_EXACT(42, 8)
    after the first linear layer (|z| < 144 * 127 * 2^25 + 2^31 < 2^41)."""
    rng = MT19937_64(seed)
    def draw(count):
        return [int(rng() % 255) - 127 for _ in range(count)]
    def bias(count):
        return [int(np.uint32(rng() & 0xFFFFFFFF).astype(np.int32)) for _ in range(count)]
    cw, cb = draw(4 * 1 * 3 * 3), bias(4)
    w1, b1 = draw(144 * 32), bias(32)
    w2, b2 = draw(32 * 10), bias(10)
    x = [int(rng() % 256) for _ in range(64)]
    layers = [z.layer_conv2d(1, 8, 8, 4, 3, 3, 1, 0, cw, cb), z.layer_relu_exact(144, 34, 8),
              z.layer_linear(144, 32, w1, b1), z.layer_relu_exact(32, 42, 8),
              z.layer_linear(32, 10, w2, b2), z.layer_softmax(10)]
    return layers, [x]


CONFIG4_NAMED_OPTS = dict(model_tag=0xC0FFEE, private_input=True, input_blinding=[0x5EED1], private_model=True,
                          private_outputs=True, route_threshold=5)


def config4_named():
    layers, xs = cnn_private()
    return z.statement_v2(layers, xs, **CONFIG4_NAMED_OPTS)
