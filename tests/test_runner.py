"""CPU: the runner's graph rewrite (Conv -> Add -> Relu fusion) and arena plan."""

import numpy as np

from nert_amd import workloads
from nert_amd.graph import Graph
from nert_amd.runner import fuse_conv_chains, pack_conv_weights, pair_downsample_convs, plan_arena

F = np.float32


def _valid_order(g):
    avail = set(g.initializers) | set(g.inputs)
    for n in g.nodes:
        for t in n.inputs:
            assert not t or t in avail, (n.op, t)
        avail.update(n.outputs)
    assert all(o in avail for o in g.outputs)


def test_resnet18_fusion():
    g, _ = workloads.resnet18(batch=2)
    f = fuse_conv_chains(g)
    ops = [n.op for n in f.nodes]
    # 20 convs: 17 end in Relu (9 plain, 8 with the residual Add); the three
    # 1x1 downsample convs feed an Add and stay plain.
    assert ops.count("FusedConv") == 17 and ops.count("Conv") == 3
    assert "Relu" not in ops and "Add" not in ops
    assert sum(1 for n in f.nodes if n.op == "FusedConv" and len(n.inputs) == 4) == 8
    assert all(n.attrs.get("activation") == "Relu" for n in f.nodes if n.op == "FusedConv")
    _valid_order(f)
    assert f.outputs == g.outputs


def test_resnet18_downsample_pairs():
    """Each stage's first 3x3/2 conv and its 1x1/2 shortcut become one
    six-input, two-output FusedConv at the later node's position."""
    g, _ = workloads.resnet18(batch=2)
    f = pair_downsample_convs(fuse_conv_chains(g))
    pairs = [n for n in f.nodes if n.op == "FusedConv" and len(n.outputs) == 2]
    assert len(pairs) == 3 and sum(1 for n in f.nodes if n.op == "Conv") == 0
    for n in pairs:
        x, w, b, z, w2, b2 = n.inputs
        assert z == "" and g.initializers[w].shape[2:] == (3, 3) and g.initializers[w2].shape[2:] == (1, 1)
        assert g.initializers[w2].shape[:2] == g.initializers[w].shape[:2] and b2 in g.initializers
        assert n.attrs["strides"] == [2, 2] and n.attrs["pads"] == [1, 1, 1, 1] and n.attrs["activation"] == "Relu"
        assert g.tensors[n.outputs[0]][1] == g.tensors[n.outputs[1]][1]
    _valid_order(f)
    assert len(f.nodes) == len(fuse_conv_chains(g).nodes) - 3


def test_pack_conv_weights():
    """3x3 convs with C/group a multiple of 8 get W in the packed order as a
    seventh input: packed[m][b][t][j] = W[m][8 b + j][t]; pairs keep their
    six inputs before it; other convs are left as they are."""
    g, _ = workloads.resnet18(batch=2)
    f = pack_conv_weights(pair_downsample_convs(fuse_conv_chains(g)))
    packed = [n for n in f.nodes if n.op == "FusedConv" and len(n.inputs) == 7]
    # 17 3x3 convs of the 20 (the stem is 7x7 with C = 3; the pairs' 1x1s ride along)
    assert len(packed) == 16 and sum(1 for n in packed if n.inputs[4]) == 3
    for n in packed:
        w = g.initializers[n.inputs[1]]
        p = f.initializers[n.inputs[6]]
        assert p.shape == w.shape and p.dtype == w.dtype and f.tensors[n.inputs[6]] == (p.dtype, p.shape)
        m, cg = w.shape[:2]
        # brute force over every element, against the formula
        flat = p.reshape(m, -1)
        for b in range(cg // 8):
            for t in range(9):
                for j in range(8):
                    assert np.array_equal(flat[:, (b * 9 + t) * 8 + j], w[:, 8 * b + j, t // 3, t % 3])
        if not n.inputs[4]:
            assert n.inputs[4:6] == ["", ""] and len(n.outputs) == 1
    assert [n.outputs for n in f.nodes] == [n.outputs for n in pair_downsample_convs(fuse_conv_chains(g)).nodes]
    stem = f.nodes[0]
    assert stem.op == "FusedConv" and len(stem.inputs) < 7
    _valid_order(f)
    # a grouped 3x3 conv with 4 channels per group and a plain Conv with 8
    h = Graph()
    x = h.add_input("x", F, (1, 16, 6, 6))
    wa = h.add_initializer("wa", np.arange(16 * 4 * 9, dtype=F).reshape(16, 4, 3, 3))
    wb = h.add_initializer("wb", np.arange(8 * 16 * 9, dtype=F).reshape(8, 16, 3, 3))
    (a,) = h.add_node("Conv", [x, wa], [("a", F, (1, 16, 6, 6))], {"pads": [1, 1, 1, 1], "group": 4})
    (b,) = h.add_node("Conv", [a, wb], [("b", F, (1, 8, 6, 6))], {"pads": [1, 1, 1, 1]})
    h.outputs = [b]
    k = pack_conv_weights(h)
    assert k.nodes[0].op == "Conv" and k.nodes[0].inputs == [x, wa]
    assert k.nodes[1].op == "FusedConv" and k.nodes[1].inputs == [a, wb, "", "", "", "", "wb:packed"]
    assert k.nodes[1].attrs == {"pads": [1, 1, 1, 1]}
    assert k.initializers["wb:packed"].reshape(8, 2, 9, 8)[5, 1, 4, 3] == h.initializers[wb][5, 11, 1, 1]


def _pair_graph(pads2=(0, 0, 0, 0), stride2=(2, 2), m2=8, between=False):
    g = Graph()
    x = g.add_input("x", F, (1, 4, 8, 8))
    w = g.add_initializer("w", np.ones((8, 4, 3, 3), F))
    w2 = g.add_initializer("w2", np.ones((m2, 4, 1, 1), F))
    oh = (8 + pads2[0] + pads2[2] - 1) // stride2[0] + 1
    (d,) = g.add_node("Conv", [x, w2], [("d", F, (1, m2, oh, oh))], {"strides": list(stride2), "pads": list(pads2)})
    if between:
        (e,) = g.add_node("Relu", [d], [("e", F, (1, m2, oh, oh))])
    (c,) = g.add_node("Conv", [x, w], [("c", F, (1, 8, 4, 4))], {"strides": [2, 2], "pads": [1, 1, 1, 1]})
    g.outputs = [c, d] + ([e] if between else [])
    return g


def test_downsample_pair_rules():
    f = pair_downsample_convs(_pair_graph())
    assert [n.op for n in f.nodes] == ["FusedConv"] and f.nodes[0].outputs == ["c", "d"]
    assert f.nodes[0].inputs == ["x", "w", "", "", "w2", ""]
    _valid_order(f)
    # a padded or differently strided 1x1, other output channels, or a reader
    # of the earlier output between the two: no pair
    for kw in ({"pads2": (1, 1, 1, 1)}, {"stride2": (1, 1)}, {"m2": 4}, {"between": True}):
        assert all(n.op != "FusedConv" for n in pair_downsample_convs(_pair_graph(**kw)).nodes), kw


def _chain(extra_consumer=False, output_mid=False, broadcast=False):
    g = Graph()
    x = g.add_input("x", F, (1, 4, 6, 6))
    w = g.add_initializer("w", np.ones((4, 4, 3, 3), F))
    zshape = (1, 4, 1, 1) if broadcast else (1, 4, 6, 6)
    z = g.add_input("z", F, zshape)
    (c,) = g.add_node("Conv", [x, w], [("c", F, (1, 4, 6, 6))], {"pads": [1, 1, 1, 1]})
    (a,) = g.add_node("Add", [c, z], [("a", F, (1, 4, 6, 6))])
    (r,) = g.add_node("Relu", [a], [("r", F, (1, 4, 6, 6))])
    g.outputs = [r]
    if extra_consumer:
        (e,) = g.add_node("Relu", [c], [("e", F, (1, 4, 6, 6))])
        g.outputs.append(e)
    if output_mid:
        g.outputs.append(a)
    return g


def test_fusion_rules():
    f = fuse_conv_chains(_chain())
    assert [n.op for n in f.nodes] == ["FusedConv"]
    assert f.nodes[0].inputs == ["x", "w", "", "z"] and f.nodes[0].outputs == ["r"]
    # the conv output has a second consumer: nothing fuses into the conv
    assert [n.op for n in fuse_conv_chains(_chain(extra_consumer=True)).nodes] == ["Conv", "Add", "Relu", "Relu"]
    # the Add output is a graph output: Conv+Add fuse, the Relu stays
    assert [n.op for n in fuse_conv_chains(_chain(output_mid=True)).nodes] == ["FusedConv", "Relu"]
    # a broadcasting Add is left alone; the Relu cannot reach the conv
    assert [n.op for n in fuse_conv_chains(_chain(broadcast=True)).nodes] == ["Conv", "Add", "Relu"]


def _silu_chain(swap=False, sig_output=False, third_consumer=False, with_add=False):
    g = Graph()
    x = g.add_input("x", F, (1, 4, 6, 6))
    w = g.add_initializer("w", np.ones((4, 4, 3, 3), F))
    (c,) = g.add_node("Conv", [x, w], [("c", F, (1, 4, 6, 6))], {"pads": [1, 1, 1, 1]})
    if with_add:
        z = g.add_input("z", F, (1, 4, 6, 6))
        (c,) = g.add_node("Add", [z, c], [("a", F, (1, 4, 6, 6))])
    (s,) = g.add_node("Sigmoid", [c], [("s", F, (1, 4, 6, 6))])
    (m,) = g.add_node("Mul", [s, c] if swap else [c, s], [("m", F, (1, 4, 6, 6))])
    g.outputs = [m]
    if sig_output:
        g.outputs.append(s)
    if third_consumer:
        (e,) = g.add_node("Relu", [c], [("e", F, (1, 4, 6, 6))])
        g.outputs.append(e)
    return g


def test_silu_fusion_rules():
    for swap in (False, True):
        f = fuse_conv_chains(_silu_chain(swap=swap))
        assert [n.op for n in f.nodes] == ["FusedConv"]
        assert f.nodes[0].attrs["activation"] == "Silu" and f.nodes[0].outputs == ["m"]
        assert f.nodes[0].inputs == ["x", "w"]
    f = fuse_conv_chains(_silu_chain(with_add=True))
    assert [n.op for n in f.nodes] == ["FusedConv"] and f.nodes[0].inputs == ["x", "w", "", "z"]
    _valid_order(f)
    # the Sigmoid output is also a graph output, or the conv output has a
    # third consumer: the pair stays separate rows
    assert [n.op for n in fuse_conv_chains(_silu_chain(sig_output=True)).nodes] == ["Conv", "Sigmoid", "Mul"]
    assert [n.op for n in fuse_conv_chains(_silu_chain(third_consumer=True)).nodes] == \
        ["Conv", "Sigmoid", "Mul", "Relu"]


def test_detector_fusion():
    g, _ = workloads.detector(batch=1, size=128, k=50)
    f = fuse_conv_chains(g)
    silu = [n for n in f.nodes if n.op == "FusedConv" and n.attrs.get("activation") == "Silu"]
    # five backbone stages and the two neck convolutions end in SiLU
    assert len(silu) == 7
    assert sum(1 for n in f.nodes if n.op == "Sigmoid") == 1  # the score head's
    _valid_order(f)


def test_arena_plan_reuses_memory():
    g, _ = workloads.resnet18(batch=2)
    offsets, size = plan_arena(fuse_conv_chains(g))
    total = sum(int(np.prod(g.tensors[t][1])) * 4 for t in offsets)
    assert size < total / 2
    assert all(o % 256 == 0 for o in offsets.values())
    # fusion removes the chain intermediates from the plan altogether
    assert size < plan_arena(g)[1]


def _intervals(g, offsets, alias):
    """(offset, size, first, last, name) per owned buffer, with views folded in."""
    first, last = {}, {}
    for idx, n in enumerate(g.nodes):
        for t in n.outputs:
            first.setdefault(t, idx)
            last.setdefault(t, idx)
        for t in n.inputs:
            if t:
                last[alias.get(t, (t, 0))[0]] = idx
    for t in g.outputs:
        last[alias.get(t, (t, 0))[0]] = len(g.nodes)
    out = []
    for t, start in first.items():
        size = int(np.prod(g.tensors[t][1])) * np.dtype(g.tensors[t][0]).itemsize
        out.append((offsets[t], max(size, 1), start, last[t], t))
    return out


def test_view_rows_alias_their_input():
    from nert_amd.runner import alias_views

    g, _ = workloads.vit_b16(batch=2, layers=2)
    f, alias = alias_views(fuse_conv_chains(g))
    assert not any(n.op in ("Squeeze", "Reshape", "Split") for n in f.nodes)
    assert len(f.nodes) < len(g.nodes)
    _valid_order_with(f, alias)
    offsets, size = plan_arena(f, alias)
    nbytes = lambda t: int(np.prod(g.tensors[t][1])) * np.dtype(g.tensors[t][0]).itemsize
    for view, (owner, off) in alias.items():
        assert offsets[view] == offsets[owner] + off
        assert 0 <= off and off + nbytes(view) <= nbytes(owner)
    # the three Split parts of one layer tile their owner exactly
    parts = sorted(off for v, (o, off) in alias.items() if v.startswith("split"))
    assert parts and parts[0] == 0
    # no two buffers that are live at the same time overlap
    iv = _intervals(f, offsets, alias)
    for i, (o1, s1, a1, b1, t1) in enumerate(iv):
        for o2, s2, a2, b2, t2 in iv[i + 1:]:
            if a1 <= b2 and a2 <= b1:
                assert o1 + s1 <= o2 or o2 + s2 <= o1, (t1, t2)


def _valid_order_with(g, alias):
    avail = set(g.initializers) | set(g.inputs)
    for n in g.nodes:
        for t in n.inputs:
            assert not t or alias.get(t, (t, 0))[0] in avail or t in avail, (n.op, t)
        avail.update(n.outputs)
        avail.update(v for v, (o, _) in alias.items() if o in avail)


def test_vit_matmul_fusion():
    from nert_amd.runner import fuse_matmul_chains

    g, _ = workloads.vit_b16(batch=2, layers=2)
    f = fuse_matmul_chains(g)
    fused = [n for n in f.nodes if n.op == "FusedMatMul"]
    # per layer: QKV + bias, QK^T * 1/8, projection + bias, fc1 + bias + Gelu, fc2 + bias
    assert len(fused) == 10
    assert sum(1 for n in fused if n.attrs.get("activation") == "Gelu") == 2
    assert sum(1 for n in fused if n.attrs.get("alpha") == 0.125) == 2
    assert not any(n.op in ("Erf", "Div") for n in f.nodes)
    assert [n.op for n in f.nodes].count("MatMul") == 2  # A.V stays plain
    _valid_order(f)


def test_matmul_fusion_rules():
    from nert_amd.runner import fuse_matmul_chains

    def chain(extra=False, bias_shape=(6,)):
        g = Graph()
        a = g.add_input("a", F, (4, 8))
        w = g.add_initializer("w", np.ones((8, 6), F))
        b = g.add_initializer("b", np.ones(bias_shape, F))
        y = g.add_node("MatMul", [a, w], [("y", F, (4, 6))])[0]
        z = g.add_node("Add", [y, b], [("z", F, (4, 6))])[0]
        g.outputs = [z]
        if extra:
            g.add_node("Relu", [y], [("r", F, (4, 6))])
            g.outputs.append("r")
        return g

    assert [n.op for n in fuse_matmul_chains(chain()).nodes] == ["FusedMatMul"]
    # the MatMul output has a second consumer: nothing fuses
    assert [n.op for n in fuse_matmul_chains(chain(extra=True)).nodes] == ["MatMul", "Add", "Relu"]
    # a bias that is not [N] stays a separate Add
    assert [n.op for n in fuse_matmul_chains(chain(bias_shape=(4, 6))).nodes] == ["MatMul", "Add"]


def test_add_layernorm_fusion_rules():
    """A same-shape float Add feeding a LayerNormalization with per-element
    initializer Scale/B fuses (at the Add's place, keeping the sum as an
    output); a broadcasting Add, a norm with Mean output, or a non-initializer
    Scale do not."""
    from nert_amd.graph import Graph
    from nert_amd.runner import fuse_add_layernorm

    F = np.float32

    def build(b_shape=(2, 3, 8), extra_out=False, scale_init=True):
        g = Graph()
        a = g.add_input("a", F, (2, 3, 8))
        b = g.add_input("b", F, b_shape)
        sc = g.add_initializer("sc", np.ones(8, F)) if scale_init else g.add_input("sc", F, (8,))
        bi = g.add_initializer("bi", np.zeros(8, F))
        s_ = g.add_node("Add", [a, b], [("s", F, (2, 3, 8))], name="add")[0]
        outs = [("y", F, (2, 3, 8))] + ([("mean", F, (2, 3, 1))] if extra_out else [])
        y = g.add_node("LayerNormalization", [s_, sc, bi], outs, {"axis": -1, "epsilon": 1e-6}, name="ln")[0]
        z = g.add_node("Add", [s_, y], [("z", F, (2, 3, 8))], name="res")[0]
        g.outputs.append(z)
        return g

    f = fuse_add_layernorm(build())
    assert [n.op for n in f.nodes] == ["FusedAddLayerNorm", "Add"]
    assert f.nodes[0].outputs == ["s", "y"] and f.nodes[0].inputs == ["a", "b", "sc", "bi"]
    assert f.nodes[0].attrs == {"axis": -1, "epsilon": 1e-6}
    for g in (build(b_shape=(8,)), build(extra_out=True), build(scale_init=False)):
        assert [n.op for n in fuse_add_layernorm(g).nodes] == ["Add", "LayerNormalization", "Add"]


def test_fuse_attention_rules():
    """The attention block becomes one FusedAttention(qkv) node carrying heads
    and scale; it stays unfused when an intermediate is also a graph output
    or when the head dimension is not 64."""
    from attn_graph import attention_block
    from nert_amd.runner import fuse_attention

    f = fuse_attention(attention_block(2, 197, 12, scale=0.125))
    assert [n.op for n in f.nodes] == ["FusedAttention"]
    n = f.nodes[0]
    assert n.inputs == ["qkv"] and n.outputs == ["attn_out"]
    assert n.attrs == {"heads": 12, "scale": 0.125}
    assert len(fuse_attention(attention_block(1, 1000, 2)).nodes) == 1
    for g in (attention_block(2, 50, 3, scores_output=True), attention_block(2, 50, 3, head_dim=32)):
        assert "FusedAttention" not in [n.op for n in fuse_attention(g).nodes]
        assert len(fuse_attention(g).nodes) == len(g.nodes)


def test_fuse_rows_on_vit():
    """Two encoder layers: two attention blocks, eight MatMul chains (QKV,
    projection and the two MLP products per layer) and four residual
    Add + LayerNorm pairs fuse; without the attention fusion the QK^T chains
    fuse as MatMul chains instead."""
    from collections import Counter

    from nert_amd import workloads
    from nert_amd.runner import fuse_rows

    g, _ = workloads.vit_b16(batch=2, layers=2)
    ops = Counter(n.op for n in fuse_rows(g).nodes)
    assert (ops["FusedAttention"], ops["FusedMatMul"], ops["FusedAddLayerNorm"], ops["Softmax"]) == (2, 8, 4, 0)
    ops = Counter(n.op for n in fuse_rows(g, attention=False).nodes)
    assert (ops["FusedAttention"], ops["FusedMatMul"], ops["Softmax"]) == (0, 10, 2)
