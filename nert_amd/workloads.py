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


def _const_i64(g: Graph, name: str, values) -> str:
    return g.add_initializer(name, np.asarray(values, dtype=np.int64))


def vit_b16(batch: int = 16, layers: int = 12, num_classes: int = 1000,
            seed: int = BASE_SEED) -> tuple[Graph, dict[str, np.ndarray]]:
    """ViT-B/16-style encoder at [batch,3,224,224] -> [batch,1000].

    Patch-embed Conv 16x16/16 to 768 channels, Reshape + Transpose to
    [batch,196,768], class token (Expand + Concat), position embedding (Add),
    `layers` pre-LN blocks (LayerNormalization eps 1e-6; fused QKV MatMul,
    Reshape/Transpose/Split/Squeeze into 12 heads of 64; MatMul QK^T scaled by
    1/8; Softmax on the last axis; MatMul V; output projection; MLP
    768->3072->768 with Gelu = 0.5*x*(1+Erf(x/sqrt(2)))), final LayerNorm,
    class-token Gather and a Gemm head. Weights ~ N(0, 0.02), biases zero
    except the drawn ones below; the input ~ N(0, 1)."""
    rng = Rng(seed)
    b = _Builder(rng)
    g = b.g
    d, heads, hd, mlp, tokens = 768, 12, 64, 3072, 197
    x = g.add_input("input", F32, (batch, 3, 224, 224))
    xval = rng.normal((batch, 3, 224, 224)).astype(F32)

    def init(shape, std=0.02):
        return g.add_initializer(b.name("p"), rng.normal(shape, 0.0, std).astype(F32))

    def node(op, inputs, shape, attrs=None, dtype=F32):
        return g.add_node(op, inputs, [(b.name(op.lower()), dtype, shape)], attrs)[0]

    def matmul_bias(h, k_in, k_out, shape_prefix):
        w = init((k_in, k_out))
        bias = init((k_out,))
        y = node("MatMul", [h, w], shape_prefix + (k_out,))
        return node("Add", [y, bias], shape_prefix + (k_out,))

    def layernorm(h):
        scale = g.add_initializer(b.name("ln_s"), (1.0 + rng.normal((d,), 0.0, 0.02)).astype(F32))
        bias = init((d,))
        return node("LayerNormalization", [h, scale, bias], (batch, tokens, d), {"axis": -1, "epsilon": 1e-6})

    w_patch = init((d, 3, 16, 16))
    b_patch = init((d,))
    y = node("Conv", [x, w_patch, b_patch], (batch, d, 14, 14), {"kernel_shape": [16, 16], "strides": [16, 16]})
    y = node("Reshape", [y, _const_i64(g, b.name("shape"), [batch, d, 196])], (batch, d, 196))
    y = node("Transpose", [y], (batch, 196, d), {"perm": [0, 2, 1]})
    cls = init((1, 1, d))
    cls = node("Expand", [cls, _const_i64(g, b.name("shape"), [batch, 1, d])], (batch, 1, d))
    y = node("Concat", [cls, y], (batch, tokens, d), {"axis": 1})
    y = node("Add", [y, init((1, tokens, d))], (batch, tokens, d))
    sqrt2 = g.add_initializer("sqrt2", np.array(np.sqrt(2.0), F32))
    one = g.add_initializer("one", np.array(1.0, F32))
    half = g.add_initializer("half", np.array(0.5, F32))
    scale = g.add_initializer("attn_scale", np.array(0.125, F32))
    split3 = _const_i64(g, "split3", [1, 1, 1])
    axis0 = _const_i64(g, "axis0", [0])
    for _ in range(layers):
        h = layernorm(y)
        qkv = matmul_bias(h, d, 3 * d, (batch, tokens))
        qkv = node("Reshape", [qkv, _const_i64(g, b.name("shape"), [batch, tokens, 3, heads, hd])],
                   (batch, tokens, 3, heads, hd))
        qkv = node("Transpose", [qkv], (3, batch, heads, tokens, hd), {"perm": [2, 0, 3, 1, 4]})
        parts = g.add_node("Split", [qkv, split3],
                           [(b.name("split"), F32, (1, batch, heads, tokens, hd)) for _ in range(3)], {"axis": 0})
        q, k, v = (node("Squeeze", [p_, axis0], (batch, heads, tokens, hd)) for p_ in parts)
        kt = node("Transpose", [k], (batch, heads, hd, tokens), {"perm": [0, 1, 3, 2]})
        s = node("MatMul", [q, kt], (batch, heads, tokens, tokens))
        s = node("Mul", [s, scale], (batch, heads, tokens, tokens))
        p = node("Softmax", [s], (batch, heads, tokens, tokens), {"axis": -1})
        o = node("MatMul", [p, v], (batch, heads, tokens, hd))
        o = node("Transpose", [o], (batch, tokens, heads, hd), {"perm": [0, 2, 1, 3]})
        o = node("Reshape", [o, _const_i64(g, b.name("shape"), [batch, tokens, d])], (batch, tokens, d))
        y = node("Add", [y, matmul_bias(o, d, d, (batch, tokens))], (batch, tokens, d))
        h = layernorm(y)
        m = matmul_bias(h, d, mlp, (batch, tokens))
        e = node("Erf", [node("Div", [m, sqrt2], (batch, tokens, mlp))], (batch, tokens, mlp))
        e = node("Add", [e, one], (batch, tokens, mlp))
        m = node("Mul", [node("Mul", [m, e], (batch, tokens, mlp)), half], (batch, tokens, mlp))
        y = node("Add", [y, matmul_bias(m, mlp, d, (batch, tokens))], (batch, tokens, d))
    y = layernorm(y)
    y = node("Gather", [y, g.add_initializer("cls_index", np.array(0, np.int64))], (batch, d), {"axis": 1})
    hw = init((num_classes, d))
    hb = init((num_classes,))
    y = g.add_node("Gemm", [y, hw, hb], [("logits", F32, (batch, num_classes))], {"transB": 1})[0]
    g.outputs.append(y)
    return g, {x: xval}


def detector(batch: int = 8, size: int = 640, k: int = 300, expose_scores: bool = False,
             seed: int = BASE_SEED) -> tuple[Graph, dict[str, np.ndarray]]:
    """a small anchor-free CSP-style detector at [batch,3,size,size].

    Backbone: five Conv 3x3/2 + SiLU (Sigmoid, Mul) stages, widths
    16/32/64/128/256 (strides 2..32). Neck: Resize nearest x2 + Concat with
    the stride-16 and stride-8 maps, each followed by a 1x1 Conv + SiLU.
    Heads: 1x1 Conv to 4 + 80 channels at strides 8/16/32 (80x80 + 40x40 +
    20x20 = 8400 anchors at 640), Reshape + Concat to [batch,84,8400],
    Transpose, Slice boxes / scores, Sigmoid scores [batch,8400,80], Reshape
    to [batch,672000], TopK k (largest, sorted). The class is index % 80 and
    the anchor index / 80 (int64 Div/Mod); boxes are gathered from
    [batch*8400, 4] with anchor + 8400 * image (Add of an int64 column).
    Outputs: scores [batch,k] f32, boxes [batch,k,4] f32, classes [batch,k]
    int64 (and the sigmoid scores when `expose_scores`). Weights
    Kaiming-normal, biases N(0, 0.01), BN-free; the input ~ U(0, 1)."""
    rng = Rng(seed)
    b = _Builder(rng)
    g = b.g
    ncls = 80
    x = g.add_input("input", F32, (batch, 3, size, size))
    xval = rng.uniform((batch, 3, size, size), 0.0, 1.0).astype(F32)

    def silu(t):
        return b.g.add_node("Mul", [t, b.unary("Sigmoid", t)], [(b.name("silu"), F32, b.shape(t))])[0]

    feats = []
    y = x
    for width in (16, 32, 64, 128, 256):
        y = silu(b.conv(y, width, 3, 2, 1, bn=False))
        feats.append(y)
    p3, p4, p5 = feats[2], feats[3], feats[4]

    def up_cat(top, lateral):
        n, c, h, w = b.shape(top)
        scales = g.add_initializer(b.name("scales"), np.array([1, 1, 2, 2], F32))
        u = g.add_node("Resize", [top, "", scales], [(b.name("resize"), F32, (n, c, 2 * h, 2 * w))],
                       {"mode": "nearest"})[0]
        lc = b.shape(lateral)[1]
        return g.add_node("Concat", [u, lateral], [(b.name("concat"), F32, (n, c + lc, 2 * h, 2 * w))],
                          {"axis": 1})[0]

    n4 = silu(b.conv(up_cat(p5, p4), 128, 1, 1, 0, bn=False))
    n3 = silu(b.conv(up_cat(n4, p3), 64, 1, 1, 0, bn=False))
    flat = []
    for f in (n3, n4, p5):
        h = b.conv(f, 4 + ncls, 1, 1, 0, bn=False)
        n, c, hh, ww = b.shape(h)
        flat.append(g.add_node("Reshape", [h, _const_i64(g, b.name("shape"), [n, c, hh * ww])],
                               [(b.name("reshape"), F32, (n, c, hh * ww))])[0])
    anchors = sum(b.shape(f)[2] for f in flat)
    y = g.add_node("Concat", flat, [(b.name("concat"), F32, (batch, 4 + ncls, anchors))], {"axis": 2})[0]
    y = g.add_node("Transpose", [y], [(b.name("transpose"), F32, (batch, anchors, 4 + ncls))], {"perm": [0, 2, 1]})[0]

    def sl(start, end, shape):
        return g.add_node("Slice", [y, _const_i64(g, b.name("starts"), [start]), _const_i64(g, b.name("ends"), [end]),
                                    _const_i64(g, b.name("axes"), [2])], [(b.name("slice"), F32, shape)])[0]

    boxes = sl(0, 4, (batch, anchors, 4))
    scores = b.unary("Sigmoid", sl(4, 4 + ncls, (batch, anchors, ncls)))
    flat_scores = g.add_node("Reshape", [scores, _const_i64(g, b.name("shape"), [batch, anchors * ncls])],
                             [("scores_flat", F32, (batch, anchors * ncls))])[0]
    top_v, top_i = g.add_node("TopK", [flat_scores, _const_i64(g, "k", [k])],
                              [("top_scores", F32, (batch, k)), (b.name("top_idx"), np.int64, (batch, k))],
                              {"axis": -1, "largest": 1, "sorted": 1})
    ncls_t = g.add_initializer("num_classes", np.array(ncls, np.int64))
    anchor = g.add_node("Div", [top_i, ncls_t], [(b.name("anchor"), np.int64, (batch, k))])[0]
    cls_id = g.add_node("Mod", [top_i, ncls_t], [("classes", np.int64, (batch, k))])[0]
    offs = g.add_initializer("image_offset", (np.arange(batch, dtype=np.int64) * anchors).reshape(batch, 1))
    flat_idx = g.add_node("Add", [anchor, offs], [(b.name("flat_idx"), np.int64, (batch, k))])[0]
    all_boxes = g.add_node("Reshape", [boxes, _const_i64(g, b.name("shape"), [batch * anchors, 4])],
                           [(b.name("reshape"), F32, (batch * anchors, 4))])[0]
    out_boxes = g.add_node("Gather", [all_boxes, flat_idx], [("boxes", F32, (batch, k, 4))], {"axis": 0})[0]
    g.outputs += [top_v, out_boxes, cls_id]
    if expose_scores:
        g.outputs.append(flat_scores)
    return g, {x: xval}
