"""Seeded synthetic workloads for the BASELINE.json configs.

Every tensor is drawn from a portable generator so any machine reproduces the
same bytes: tensor t uses SplitMix64 seeded with 0x4E455254 + t; element i
takes the (i+1)-th output; a uniform is the top 24 bits / 2^24; a normal is
Box-Muller over two uniforms (cos branch), computed in float64 and rounded
once to float32. std::normal_distribution is implementation-defined, hence
this explicit recipe.

Builders return a `Graph` (nert_amd.graph) whose tensor table carries every
shape, so the gfx950 runner needs no shape inference, and whose ONNX encoding
loads in the reference (tests check the reference's InferShapes agrees).
"""

from __future__ import annotations

import numpy as np

from .graph import Graph

BASE_SEED = 0x4E455254
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
F32 = np.float32


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of SplitMix64 started at `seed` (uint64 array)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + (np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform01(seed: int, n: int) -> np.ndarray:
    """n float64 uniforms in [0, 1) with 24-bit resolution."""
    return (splitmix64(seed, n) >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))


class Rng:
    """Hands out one SplitMix64 stream per tensor, in creation order."""

    def __init__(self, base: int = BASE_SEED):
        self.base = base
        self.index = 0

    def _seed(self) -> int:
        s = self.base + self.index
        self.index += 1
        return s

    def uniform(self, shape, lo: float, hi: float) -> np.ndarray:
        n = int(np.prod(shape))
        u = uniform01(self._seed(), n)
        return (lo + (hi - lo) * u).reshape(shape)

    def normal(self, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        n = int(np.prod(shape))
        u = uniform01(self._seed(), 2 * n)
        u1 = u[0::2] + (1.0 / (1 << 25))  # keep log() finite
        u2 = u[1::2]
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        return (mean + std * z).reshape(shape)


def _conv_out(n, k, s, p, d=1):
    return (n + 2 * p - (d * (k - 1) + 1)) // s + 1


class _Builder:
    def __init__(self, rng: Rng):
        self.g = Graph()
        self.rng = rng
        self.count = 0

    def name(self, prefix: str) -> str:
        self.count += 1
        return f"{prefix}{self.count}"

    def shape(self, t: str) -> tuple[int, ...]:
        return self.g.tensors[t][1]

    def conv(self, x: str, m: int, k: int, s: int, p: int, bn: bool = True, bias_std: float = 0.01) -> str:
        n, c, h, w = self.shape(x)
        fan_in = c * k * k
        wt = self.rng.normal((m, c, k, k), 0.0, np.sqrt(2.0 / fan_in))
        if bn:
            # BatchNormalization folded into the convolution in float64, rounded
            # once (there is no BatchNormalization row in NERT,
            # src/kernels/cpu_kernels.cpp:16-90).
            gamma = self.rng.uniform((m,), 0.8, 1.2)
            beta = self.rng.normal((m,), 0.0, 0.1)
            mean = self.rng.normal((m,), 0.0, 0.1)
            var = self.rng.uniform((m,), 0.5, 1.5)
            scale = gamma / np.sqrt(var + 1e-5)
            wt = wt * scale[:, None, None, None]
            bias = beta - mean * scale
        else:
            bias = self.rng.normal((m,), 0.0, bias_std)
        wn = self.g.add_initializer(self.name("W"), wt.astype(F32))
        bn_ = self.g.add_initializer(self.name("B"), bias.astype(F32))
        oh, ow = _conv_out(h, k, s, p), _conv_out(w, k, s, p)
        attrs = {"kernel_shape": [k, k], "strides": [s, s], "pads": [p, p, p, p]}
        return self.g.add_node("Conv", [x, wn, bn_], [(self.name("conv"), F32, (n, m, oh, ow))], attrs)[0]

    def unary(self, op: str, x: str) -> str:
        return self.g.add_node(op, [x], [(self.name(op.lower()), F32, self.shape(x))])[0]

    def add(self, a: str, b: str) -> str:
        return self.g.add_node("Add", [a, b], [(self.name("add"), F32, self.shape(a))])[0]


def resnet18(batch: int = 32, num_classes: int = 1000, seed: int = BASE_SEED) -> tuple[Graph, dict[str, np.ndarray]]:
    """ResNet-18 (BN folded) at [batch,3,224,224] -> [batch,1000].

    Stem Conv7x7/2+Relu, MaxPool3x3/2; four stages of two BasicBlocks
    (64/128/256/512, stride-2 1x1 downsample); GlobalAveragePool, Flatten,
    Gemm 512->1000. 49 nodes. Returns (graph, {input name: seeded input})."""
    rng = Rng(seed)
    b = _Builder(rng)
    g = b.g
    x = g.add_input("input", F32, (batch, 3, 224, 224))
    xval = rng.normal((batch, 3, 224, 224)).astype(F32)
    y = b.unary("Relu", b.conv(x, 64, 7, 2, 3))
    n, c, h, w = b.shape(y)
    oh, ow = _conv_out(h, 3, 2, 1), _conv_out(w, 3, 2, 1)
    y = g.add_node("MaxPool", [y], [(b.name("pool"), F32, (n, c, oh, ow))],
                   {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]})[0]
    in_c = 64
    for stage, width in enumerate([64, 128, 256, 512]):
        for block in range(2):
            stride = 2 if (stage > 0 and block == 0) else 1
            identity = y
            out = b.unary("Relu", b.conv(y, width, 3, stride, 1))
            out = b.conv(out, width, 3, 1, 1)
            if stride != 1 or in_c != width:
                identity = b.conv(y, width, 1, stride, 0)
            y = b.unary("Relu", b.add(out, identity))
            in_c = width
    n, c = b.shape(y)[:2]
    y = g.add_node("GlobalAveragePool", [y], [(b.name("gap"), F32, (n, c, 1, 1))])[0]
    y = g.add_node("Flatten", [y], [(b.name("flat"), F32, (n, c))], {"axis": 1})[0]
    bound = 1.0 / np.sqrt(c)
    fw = g.add_initializer("fc_W", rng.uniform((num_classes, c), -bound, bound).astype(F32))
    fb = g.add_initializer("fc_B", rng.uniform((num_classes,), -bound, bound).astype(F32))
    y = g.add_node("Gemm", [y, fw, fb], [("logits", F32, (n, num_classes))],
                   {"transB": 1, "alpha": 1.0, "beta": 1.0})[0]
    g.outputs.append(y)
    return g, {x: xval}


def resnet18_input(batch: int, seed: int = BASE_SEED) -> np.ndarray:
    """The seeded input resnet18() draws, without building the weights again."""
    rng = Rng(seed)
    return rng.normal((batch, 3, 224, 224)).astype(F32)
