"""Op-level measurement cases: all 49 of the reference's op-bench fixtures
(olibartfast/nert bench/runtime/main.cpp:331-674; twelve of them quoted with
MI300X figures), BASELINE.json configs[0] and configs[1](a)(b)(c), and the
bandwidth-bound rows at the shapes configs[2] and configs[3] run them.

Each case is one node with the fixture's shapes, attributes and value ranges
(values drawn from this package's seeded generator; the reference draws from
std::mt19937_64(0xC0FFEE), whose values do not change the work). `work` is
the algorithmic amount the roofline uses: 2*M*N*K (or the conv's
2*N*M*(C/g)*kh*kw*OH*OW) flops for MFMA-bound cases, input + output bytes
for bandwidth-bound ones. `mi300x_ms` is the reference HIP layer's published
dev_ms on MI300X (specs/2026-10-23-amd-devcloud/bench-results.txt; it
includes a host-to-device zero fill of the output inside the timed loop).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable

import numpy as np

from .graph import Graph
from .workloads import Rng

F32, I64, BOOL = np.float32, np.int64, np.bool_


@dataclass
class OpCase:
    name: str
    op: str
    inputs_spec: list[tuple[str, tuple[int, ...], Any, Callable[[Rng, tuple[int, ...]], np.ndarray]]]
    outputs_spec: list[tuple[str, tuple[int, ...], Any]]
    bound: str            # "mfma" or "hbm"
    work: float           # flops (mfma) or bytes (hbm) per launch
    attrs: dict = field(default_factory=dict)
    initializers: dict = field(default_factory=dict)
    mi300x_ms: float | None = None
    source: str = ""
    order: list[str] | None = None  # node input order, when inputs and initializers interleave

    def graph(self) -> Graph:
        g = Graph()
        for n, shape, dtype, _ in self.inputs_spec:
            g.add_input(n, dtype, shape)
        for n, v in self.initializers.items():
            g.add_initializer(n, v)
        names = self.order or [s[0] for s in self.inputs_spec] + list(self.initializers)
        outs = g.add_node(self.op, names, [(n, d, s) for n, s, d in self.outputs_spec], self.attrs, name=self.name)
        g.outputs.extend(outs)
        return g

    def inputs(self, seed: int = 0xC0FFEE) -> dict[str, np.ndarray]:
        rng = Rng(seed)
        return {n: make(rng, shape).astype(dtype) for n, shape, dtype, make in self.inputs_spec}


def _u(lo, hi):
    return lambda rng, shape: rng.uniform(shape, lo, hi)


def _nrm(std):
    return lambda rng, shape: rng.normal(shape, 0.0, std)


def _signed(lo, hi):
    """|v| ~ U(lo, hi) with a random sign (the Div fixture's divisor)."""
    def make(rng, shape):
        mag = rng.uniform(shape, lo, hi)
        return np.where(rng.uniform(shape, 0.0, 1.0) < 0.5, -mag, mag)
    return make


def _bool(rng, shape):
    return rng.uniform(shape, 0.0, 1.0) < 0.5


def _with_nans(lo, hi):
    """U(lo, hi) with a NaN at element 17 and a negative NaN at 9001 (the
    IsNaN fixture)."""
    def make(rng, shape):
        x = rng.uniform(shape, lo, hi).astype(F32)
        x.reshape(-1)[17] = np.nan
        x.reshape(-1)[9001] = -np.float32(np.nan)
        return x
    return make


def _bytes(*shapes_dtypes) -> float:
    return float(sum(int(np.prod(s)) * np.dtype(d).itemsize for s, d in shapes_dtypes))


K_BIG, K_NEW = 4 * 1024 * 1024, 1024 * 1024


def _cases() -> list[OpCase]:
    c: list[OpCase] = []
    src = "bench/runtime/main.cpp"
    # --- the reference's fixtures that have a published MI300X figure ---
    c.append(OpCase("gemm_512", "Gemm", [("a", (512, 512), F32, _u(-1, 1)), ("b", (512, 512), F32, _u(-1, 1))],
                    [("y", (512, 512), F32)], "mfma", 2.0 * 512 ** 3, mi300x_ms=0.15, source=f"{src}:337-346"))
    c.append(OpCase("conv_8x16x64x64", "Conv",
                    [("x", (8, 16, 64, 64), F32, _u(-1, 1)), ("w", (32, 16, 3, 3), F32, _u(-1, 1)),
                     ("b", (32,), F32, _u(-1, 1))],
                    [("y", (8, 32, 62, 62), F32)], "mfma", 2.0 * 8 * 32 * 62 * 62 * 16 * 9,
                    mi300x_ms=0.21, source=f"{src}:409-419"))
    c.append(OpCase("softmax_256x4096", "Softmax", [("x", (256, 4096), F32, _u(-3, 3))], [("y", (256, 4096), F32)],
                    "hbm", _bytes(((256, 4096), F32), ((256, 4096), F32)), {"axis": -1}, mi300x_ms=5.38,
                    source=f"{src}:388-396"))
    c.append(OpCase("layernorm_1024x1024", "LayerNormalization", [("x", (1024, 1024), F32, _u(-3, 3))],
                    [("y", (1024, 1024), F32)], "hbm", _bytes(((1024, 1024), F32), ((1024,), F32), ((1024, 1024), F32)),
                    {"axis": 1}, {"scale": np.ones(1024, F32)}, mi300x_ms=1.45, source=f"{src}:614-623"))
    c.append(OpCase("reducemean_1024x1024", "ReduceMean", [("x", (1024, 1024), F32, _u(-3, 3))],
                    [("y", (1024, 1), F32)], "hbm", _bytes(((1024, 1024), F32), ((1024, 1), F32)), {},
                    {"axes": np.array([1], I64)}, mi300x_ms=0.59, source=f"{src}:568-577"))
    c.append(OpCase("gap_8x64x112x112", "GlobalAveragePool", [("x", (8, 64, 112, 112), F32, _u(-3, 3))],
                    [("y", (8, 64, 1, 1), F32)], "hbm", _bytes(((8, 64, 112, 112), F32), ((8, 64, 1, 1), F32)),
                    mi300x_ms=3.35, source=f"{src}:624-632"))
    c.append(OpCase("maxpool_8x64x112x112", "MaxPool", [("x", (8, 64, 112, 112), F32, _u(-3, 3))],
                    [("y", (8, 64, 55, 55), F32)], "hbm", _bytes(((8, 64, 112, 112), F32), ((8, 64, 55, 55), F32)),
                    {"kernel_shape": [3, 3], "strides": [2, 2]}, mi300x_ms=0.16, source=f"{src}:376-387"))
    c.append(OpCase("relu_4m", "Relu", [("x", (K_BIG,), F32, _u(-6, 6))], [("y", (K_BIG,), F32)], "hbm",
                    _bytes(((K_BIG,), F32), ((K_BIG,), F32)), mi300x_ms=0.35, source=f"{src}:347-355"))
    c.append(OpCase("add_2048x2048", "Add", [("a", (2048, 2048), F32, _u(-3, 3)), ("b", (2048,), F32, _u(-3, 3))],
                    [("y", (2048, 2048), F32)], "hbm",
                    _bytes(((2048, 2048), F32), ((2048,), F32), ((2048, 2048), F32)), mi300x_ms=0.37,
                    source=f"{src}:356-364"))
    c.append(OpCase("sigmoid_4m", "Sigmoid", [("x", (K_BIG,), F32, _u(-6, 6))], [("y", (K_BIG,), F32)], "hbm",
                    _bytes(((K_BIG,), F32), ((K_BIG,), F32)), mi300x_ms=0.35, source=f"{src}:347-355"))
    c.append(OpCase("erf_1m", "Erf", [("x", (K_NEW,), F32, _u(-4, 4))], [("y", (K_NEW,), F32)], "hbm",
                    _bytes(((K_NEW,), F32), ((K_NEW,), F32)), mi300x_ms=0.10, source=f"{src}:429-440"))
    c.append(OpCase("argmax_1024x1024", "ArgMax", [("x", (1024, 1024), F32, _u(-3, 3))], [("y", (1024, 1), I64)],
                    "hbm", _bytes(((1024, 1024), F32), ((1024, 1), I64)), {"axis": 1}, mi300x_ms=0.27,
                    source=f"{src}:578-586"))
    # --- the rest of the reference's op-bench fixtures (no published MI300X figure) ---
    c.append(OpCase("tanh_4m", "Tanh", [("x", (K_BIG,), F32, _u(-6, 6))], [("y", (K_BIG,), F32)], "hbm",
                    _bytes(((K_BIG,), F32), ((K_BIG,), F32)), source=f"{src}:347-355"))
    for op in ("Mul", "Sub"):
        c.append(OpCase(f"{op.lower()}_2048x2048", op,
                        [("a", (2048, 2048), F32, _u(-3, 3)), ("b", (2048,), F32, _u(-3, 3))],
                        [("y", (2048, 2048), F32)], "hbm",
                        _bytes(((2048, 2048), F32), ((2048,), F32), ((2048, 2048), F32)), source=f"{src}:356-365"))
    c.append(OpCase("div_4m", "Div", [("a", (K_BIG,), F32, _u(-3, 3)), ("b", (K_BIG,), F32, _signed(0.5, 2.0))],
                    [("y", (K_BIG,), F32)], "hbm", _bytes(((K_BIG,), F32), ((K_BIG,), F32), ((K_BIG,), F32)),
                    source=f"{src}:366-381"))
    c.append(OpCase("averagepool_8x64x112x112", "AveragePool", [("x", (8, 64, 112, 112), F32, _u(-3, 3))],
                    [("y", (8, 64, 55, 55), F32)], "hbm", _bytes(((8, 64, 112, 112), F32), ((8, 64, 55, 55), F32)),
                    {"kernel_shape": [3, 3], "strides": [2, 2]}, source=f"{src}:382-392"))
    c.append(OpCase("reshape_2x3x4", "Reshape", [("x", (2, 3, 4), F32, _u(-1, 1))], [("y", (6, 4), F32)], "hbm",
                    _bytes(((2, 3, 4), F32), ((6, 4), F32)), {}, {"shape": np.array([6, 4], I64)},
                    source=f"{src}:402-410"))
    for op, lo, hi in (("Sin", -6, 6), ("Cos", -6, 6), ("Exp", -6, 3), ("Elu", -6, 6), ("Log", 0.1, 6),
                       ("Floor", -6, 6), ("Abs", -6, 6), ("Neg", -6, 6), ("Sqrt", 0, 16)):
        c.append(OpCase(f"{op.lower()}_1m", op, [("x", (K_NEW,), F32, _u(lo, hi))], [("y", (K_NEW,), F32)], "hbm",
                        _bytes(((K_NEW,), F32), ((K_NEW,), F32)), source=f"{src}:429-441"))
    c.append(OpCase("isnan_1m", "IsNaN", [("x", (K_NEW,), F32, _with_nans(-3, 3))], [("y", (K_NEW,), BOOL)],
                    "hbm", _bytes(((K_NEW,), F32), ((K_NEW,), BOOL)), source=f"{src}:442-453"))
    for op in ("Greater", "Less", "GreaterOrEqual", "LessOrEqual"):
        c.append(OpCase(f"{op.lower()}_1024x1024", op,
                        [("a", (1024, 1024), F32, _u(-3, 3)), ("b", (1024,), F32, _u(-3, 3))],
                        [("y", (1024, 1024), BOOL)], "hbm",
                        _bytes(((1024, 1024), F32), ((1024,), F32), ((1024, 1024), BOOL)), source=f"{src}:454-463"))
    for op in ("And", "Or"):
        c.append(OpCase(f"{op.lower()}_1024x1024", op,
                        [("a", (1024, 1024), BOOL, _bool), ("b", (1024,), BOOL, _bool)],
                        [("y", (1024, 1024), BOOL)], "hbm",
                        _bytes(((1024, 1024), BOOL), ((1024,), BOOL), ((1024, 1024), BOOL)), source=f"{src}:464-473"))
    c.append(OpCase("not_1m", "Not", [("x", (K_NEW,), BOOL, _bool)], [("y", (K_NEW,), BOOL)], "hbm",
                    _bytes(((K_NEW,), BOOL), ((K_NEW,), BOOL)), source=f"{src}:474-482"))
    c.append(OpCase("pow_1024x1024", "Pow", [("a", (1024, 1024), F32, _u(0.5, 2)), ("b", (1024,), F32, _u(-1, 1))],
                    [("y", (1024, 1024), F32)], "hbm",
                    _bytes(((1024, 1024), F32), ((1024,), F32), ((1024, 1024), F32)), source=f"{src}:483-491"))
    for op in ("Max", "Min"):
        c.append(OpCase(f"{op.lower()}_1024x1024_fold3", op,
                        [("a", (1024, 1024), F32, _u(-3, 3)), ("b", (1024,), F32, _u(-3, 3)),
                         ("c", (1,), F32, _u(-3, 3))],
                        [("y", (1024, 1024), F32)], "hbm",
                        _bytes(((1024, 1024), F32), ((1024,), F32), ((1,), F32), ((1024, 1024), F32)),
                        source=f"{src}:493-502"))
    c.append(OpCase("clip_1m", "Clip", [("x", (K_NEW,), F32, _u(-5, 5))], [("y", (K_NEW,), F32)], "hbm",
                    _bytes(((K_NEW,), F32), ((K_NEW,), F32)), {},
                    {"min": np.array([0.0], F32), "max": np.array([1.0], F32)}, source=f"{src}:503-512"))
    c.append(OpCase("identity_1m", "Identity", [("x", (K_NEW,), F32, _u(-3, 3))], [("y", (K_NEW,), F32)], "hbm",
                    _bytes(((K_NEW,), F32), ((K_NEW,), F32)), source=f"{src}:513-520"))
    c.append(OpCase("squeeze_1x1024x1", "Squeeze", [("x", (1, 1024, 1), F32, _u(-3, 3))], [("y", (1024,), F32)],
                    "hbm", _bytes(((1, 1024, 1), F32), ((1024,), F32)), source=f"{src}:522-529"))
    c.append(OpCase("tile_1024x1", "Tile", [("x", (1024, 1), F32, _u(-3, 3))], [("y", (2048, 3), F32)], "hbm",
                    _bytes(((1024, 1), F32), ((2048, 3), F32)), {}, {"repeats": np.array([2, 3], I64)},
                    source=f"{src}:531-538"))
    c.append(OpCase("range_1m", "Range", [], [("y", (K_NEW,), F32)], "hbm", _bytes(((K_NEW,), F32)), {},
                    {"start": np.array([0.0], F32), "limit": np.array([float(K_NEW)], F32),
                     "delta": np.array([1.0], F32)}, source=f"{src}:540-547"))
    c.append(OpCase("eyelike_1024x1024", "EyeLike", [("x", (1024, 1024), F32, _u(-1, 1))],
                    [("y", (1024, 1024), F32)], "hbm", _bytes(((1024, 1024), F32)), source=f"{src}:549-556"))
    c.append(OpCase("pad_1024x1024", "Pad", [("x", (1024, 1024), F32, _u(-3, 3))], [("y", (1026, 1026), F32)],
                    "hbm", _bytes(((1024, 1024), F32), ((1026, 1026), F32)), {},
                    {"pads": np.array([1, 1, 1, 1], I64)}, source=f"{src}:558-566"))
    for op in ("ReduceSum", "ReduceL2"):
        c.append(OpCase(f"{op.lower()}_1024x1024", op, [("x", (1024, 1024), F32, _u(-3, 3))],
                        [("y", (1024, 1), F32)], "hbm", _bytes(((1024, 1024), F32), ((1024, 1), F32)), {},
                        {"axes": np.array([1], I64)}, source=f"{src}:568-577"))
    c.append(OpCase("cumsum_1024x1024", "CumSum", [("x", (1024, 1024), F32, _u(-3, 3))],
                    [("y", (1024, 1024), F32)], "hbm", _bytes(((1024, 1024), F32), ((1024, 1024), F32)), {},
                    {"axis": np.array([1], I64)}, source=f"{src}:588-597"))
    c.append(OpCase("scatternd_1024x1024", "ScatterND",
                    [("x", (1024, 1024), F32, _u(-3, 3)), ("updates", (1024, 1024), F32, _u(-3, 3))],
                    [("y", (1024, 1024), F32)], "hbm",
                    _bytes(((1024, 1024), F32), ((1024, 1), I64), ((1024, 1024), F32), ((1024, 1024), F32)), {},
                    {"indices": np.arange(1024, dtype=I64).reshape(1024, 1)}, source=f"{src}:598-612",
                    order=["x", "indices", "updates"]))
    # --- BASELINE.json configs[0] and configs[1] ---
    c.append(OpCase("cfg0_conv_1x64x56x56", "Conv",
                    [("x", (1, 64, 56, 56), F32, _nrm(1.0)), ("w", (64, 64, 3, 3), F32, _nrm(np.sqrt(2 / 576))),
                     ("b", (64,), F32, _nrm(0.01))],
                    [("y", (1, 64, 56, 56), F32)], "mfma", 2.0 * 64 * 56 * 56 * 64 * 9,
                    {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1]}, source="BASELINE.json configs[0]"))
    c.append(OpCase("cfg1a_matmul_8x1024", "MatMul",
                    [("a", (8, 1024, 1024), F32, _u(-1, 1)), ("b", (8, 1024, 1024), F32, _u(-1, 1))],
                    [("y", (8, 1024, 1024), F32)], "mfma", 2.0 * 8 * 1024 ** 3, source="BASELINE.json configs[1](a)"))
    c.append(OpCase("cfg1b_gemm_2048x1024x4096", "Gemm",
                    [("a", (2048, 4096), F32, _u(-1, 1)), ("b", (1024, 4096), F32, _u(-1, 1)),
                     ("c", (1024,), F32, _u(-1, 1))],
                    [("y", (2048, 1024), F32)], "mfma", 2.0 * 2048 * 1024 * 4096,
                    {"transB": 1, "alpha": 1.0, "beta": 1.0}, source="BASELINE.json configs[1](b)"))
    c.append(OpCase("cfg1c_gemm_32x1000x512", "Gemm",
                    [("a", (32, 512), F32, _u(-1, 1)), ("b", (1000, 512), F32, _u(-1, 1)),
                     ("c", (1000,), F32, _u(-1, 1))],
                    [("y", (32, 1000), F32)], "hbm", _bytes(((32, 512), F32), ((1000, 512), F32), ((1000,), F32),
                                                           ((32, 1000), F32)),
                    {"transB": 1, "alpha": 1.0, "beta": 1.0}, source="BASELINE.json configs[1](c)"))
    # --- the bandwidth-bound rows at the model configs' shapes ---
    c.append(OpCase("cfg2_maxpool_32x64x112x112", "MaxPool", [("x", (32, 64, 112, 112), F32, _nrm(1.0))],
                    [("y", (32, 64, 56, 56), F32)], "hbm",
                    _bytes(((32, 64, 112, 112), F32), ((32, 64, 56, 56), F32)),
                    {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]},
                    source="BASELINE.json configs[2] (ResNet-18 stem pool)"))
    c.append(OpCase("cfg3_softmax_16x12x197x197", "Softmax", [("x", (16, 12, 197, 197), F32, _nrm(3.0))],
                    [("y", (16, 12, 197, 197), F32)], "hbm",
                    _bytes(((16, 12, 197, 197), F32), ((16, 12, 197, 197), F32)), {"axis": -1},
                    source="BASELINE.json configs[3] (ViT attention)"))
    c.append(OpCase("cfg3_layernorm_16x197x768", "LayerNormalization", [("x", (16, 197, 768), F32, _nrm(1.0))],
                    [("y", (16, 197, 768), F32)], "hbm",
                    _bytes(((16, 197, 768), F32), ((768,), F32), ((768,), F32), ((16, 197, 768), F32)),
                    {"axis": -1, "epsilon": 1e-6},
                    {"scale": np.linspace(0.9, 1.1, 768, dtype=F32), "bias": np.linspace(-0.1, 0.1, 768, dtype=F32)},
                    source="BASELINE.json configs[3] (ViT pre-LN)"))
    return c


CASES: list[OpCase] = _cases()
