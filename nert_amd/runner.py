"""Runs a Graph on the gfx950 layer with every tensor resident in HBM.

Plays the role the reference executor plays for a device
(src/executor.cpp:202-225 construct, :422-560 Execute): plan one arena for the
intermediates, upload initializers once, then call each node's row through the
seam's C form (nert_hip_run_node) in graph order. Two things differ, both
MI355X-side choices: graph inputs are bound once and stay in HBM (the timed
region never stages host data), and the whole node sequence can be captured
into one HIP graph and replayed, which removes per-row host overhead.

The arena plan is a first-fit over definition/last-use intervals with 256-byte
alignment, so intermediates whose lifetimes do not overlap share memory and
the working set stays small enough to live in the 256 MB Infinity Cache where
possible. Rows that only reinterpret a dense buffer's shape (Reshape, Flatten,
Squeeze, Unsqueeze, Identity) become views: their output shares the input's
arena block for the union of both lifetimes, and no copy is queued. So do the
outputs of a Split whose parts are contiguous slabs of its input (every axis
before the split axis has extent 1): each part is the input at a byte offset.
"""

from __future__ import annotations

import ctypes as C
from typing import Any, Iterable

import numpy as np

from . import abi
from .device import ERROR_FLAG_TEXT, DeviceArray, Event, NertError, check, lib, take_error_flags
from .graph import Graph, Node

ALIGN = 256


VIEW_OPS = {"Reshape", "Flatten", "Squeeze", "Unsqueeze", "Identity"}


def alias_views(g: Graph) -> tuple[Graph, dict[str, tuple[str, int]]]:
    """Drops view rows whose outputs can share the input's buffer.

    A row qualifies when its first input is an intermediate (produced by a
    node, not a graph input or initializer) and none of the tensors involved
    is a graph output: a shape-only row whose dtype and element count agree
    (a dense row-major buffer reads the same under either shape), or a Split
    along an axis preceded only by unit axes (each part is a contiguous slab).
    Returns the graph without those rows and a map from each aliased output
    to (the tensor that owns the storage, byte offset into it).
    """
    produced = {t for n in g.nodes for t in n.outputs}
    outputs = set(g.outputs)
    alias: dict[str, tuple[str, int]] = {}
    kept: list[Node] = []

    def owner_of(x: str) -> tuple[str, int]:
        return alias.get(x, (x, 0))

    for n in g.nodes:
        x = n.inputs[0] if n.inputs else ""
        ok_input = bool(x) and x in produced and x not in g.initializers and x not in g.inputs and x not in outputs
        if ok_input and n.op in VIEW_OPS and len(n.outputs) == 1:
            y = n.outputs[0]
            (xd, xs), (yd, ys) = g.tensors[x], g.tensors[y]
            if y not in outputs and np.dtype(xd) == np.dtype(yd) and int(np.prod(xs)) == int(np.prod(ys)):
                alias[y] = owner_of(x)
                continue
        if ok_input and n.op == "Split" and not any(o in outputs for o in n.outputs):
            xd, xs = g.tensors[x]
            axis = int(n.attrs.get("axis", 0)) % max(len(xs), 1)
            parts = [g.tensors[o][1] for o in n.outputs]
            contiguous = int(np.prod(xs[:axis])) == 1 and all(
                np.dtype(g.tensors[o][0]) == np.dtype(xd) and len(sh) == len(xs) for o, sh in zip(n.outputs, parts))
            if contiguous and sum(sh[axis] for sh in parts) == xs[axis]:
                inner = int(np.prod(xs[axis + 1:])) * np.dtype(xd).itemsize
                owner, base = owner_of(x)
                pos = 0
                for o, sh in zip(n.outputs, parts):
                    alias[o] = (owner, base + pos * inner)
                    pos += sh[axis]
                continue
        kept.append(n)
    return (Graph(nodes=kept, initializers=g.initializers, inputs=g.inputs, outputs=g.outputs, tensors=g.tensors),
            alias)


def plan_arena(g: Graph, alias: dict[str, tuple[str, int]] | None = None) -> tuple[dict[str, int], int]:
    """Offsets for every node output that is not a graph input/initializer;
    an aliased tensor gets its owner's offset plus its byte offset, and the
    owner stays live until the last use of any of its views."""
    alias = alias or {}
    produced: dict[str, int] = {}
    last_use: dict[str, int] = {}
    for idx, n in enumerate(g.nodes):
        for t in n.inputs:
            if t:
                last_use[alias.get(t, (t, 0))[0]] = idx
        for t in n.outputs:
            produced.setdefault(t, idx)
            last_use.setdefault(t, idx)
    end = len(g.nodes)
    for t in g.outputs:
        last_use[alias.get(t, (t, 0))[0]] = end
    live: list[tuple[int, int, int]] = []  # (offset, size, last_use)
    offsets: dict[str, int] = {}
    arena = 0
    for t, start in sorted(produced.items(), key=lambda kv: kv[1]):
        dtype, shape = g.tensors[t]
        size = max(1, int(np.prod(shape)) * np.dtype(dtype).itemsize)
        size = (size + ALIGN - 1) // ALIGN * ALIGN
        # Only tensors still live at this node's definition block memory; a
        # node's inputs stay live through the node (inclusive intervals).
        live = [e for e in live if e[2] >= start]
        cursor = 0
        for off, sz, _ in sorted(live):
            if cursor + size <= off:
                break
            cursor = max(cursor, off + sz)
        offsets[t] = cursor
        live.append((cursor, size, last_use[t]))
        arena = max(arena, cursor + size)
    for view, (owner, byte_offset) in alias.items():
        if owner in offsets:
            offsets[view] = offsets[owner] + byte_offset
    return offsets, arena


def fuse_conv_chains(g: Graph) -> Graph:
    """Rewrites Conv -> [Add] -> [Relu | SiLU] chains into single FusedConv nodes.

    A chain fuses when each intermediate tensor has exactly one consumer and is
    not a graph output, and the Add sums the conv output with a tensor of the
    same shape (no broadcasting). SiLU is the pair Sigmoid(t) -> Mul(t, s) (in
    either operand order): t's only consumers are that Sigmoid and that Mul,
    and s's only consumer is the Mul. The fused node takes the place of the
    chain's last node, where every operand (including the Add's other input)
    already exists. The FusedConv row applies bias, summand and activation in
    the kernel epilogue in the unfused order, so the outputs are bit-identical;
    the chain's intermediates are never written to memory.
    """
    consumers: dict[str, list[int]] = {}
    for idx, n in enumerate(g.nodes):
        for t in n.inputs:
            if t:
                consumers.setdefault(t, []).append(idx)
    outputs = set(g.outputs)

    def sole(t: str, op: str) -> int | None:
        if t in outputs:
            return None
        c = consumers.get(t, [])
        if len(c) == 1 and g.nodes[c[0]].op == op:
            return c[0]
        return None

    def silu(t: str) -> tuple[int, int] | None:
        """(Sigmoid index, Mul index) when t feeds exactly a SiLU pair."""
        if t in outputs:
            return None
        c = consumers.get(t, [])
        if len(c) != 2:
            return None
        ops = {g.nodes[i].op: i for i in c}
        if set(ops) != {"Sigmoid", "Mul"}:
            return None
        sig, mul = ops["Sigmoid"], ops["Mul"]
        s_node, m_node = g.nodes[sig], g.nodes[mul]
        if len(s_node.inputs) != 1 or len(s_node.outputs) != 1:
            return None
        s_out = s_node.outputs[0]
        if sole(s_out, "Mul") != mul or sorted(m_node.inputs) != sorted([t, s_out]) or t == s_out:
            return None
        return sig, mul

    replace: dict[int, Node] = {}
    dropped: set[int] = set()
    for idx, n in enumerate(g.nodes):
        if n.op != "Conv" or idx in dropped:
            continue
        out = n.outputs[0]
        z = ""
        last = idx
        a = sole(out, "Add")
        if a is not None and a not in dropped:
            add = g.nodes[a]
            others = [t for t in add.inputs if t != out]
            if len(add.inputs) == 2 and len(others) == 1 and others[0] and \
                    tuple(g.tensors[others[0]][1]) == tuple(g.tensors[out][1]):
                z = others[0]
                dropped.add(a)
                out = add.outputs[0]
                last = a
        activation = None
        r = sole(out, "Relu")
        pair = silu(out)
        if r is not None and r not in dropped:
            activation = "Relu"
            dropped.add(r)
            out = g.nodes[r].outputs[0]
            last = r
        elif pair is not None and not dropped.intersection(pair):
            activation = "Silu"
            dropped.update(pair)
            out = g.nodes[pair[1]].outputs[0]
            last = pair[1]
        if last == idx:
            continue
        inputs = [n.inputs[0], n.inputs[1], n.inputs[2] if len(n.inputs) > 2 else "", z]
        while inputs and not inputs[-1]:
            inputs.pop()
        attrs = dict(n.attrs)
        if activation:
            attrs["activation"] = activation
        dropped.add(idx)
        dropped.discard(last)
        replace[last] = Node("FusedConv", inputs, [out], attrs, n.name)
    nodes = [replace.get(i, nd) for i, nd in enumerate(g.nodes) if i not in dropped or i in replace]
    return Graph(nodes=nodes, initializers=g.initializers, inputs=g.inputs, outputs=g.outputs, tensors=g.tensors)


def _conv_geometry(g: Graph, n: Node) -> tuple[tuple[int, ...], list[int], list[int], list[int], int] | None:
    """(weight shape, strides, pads, dilations, group) of a 2-D Conv or
    FusedConv node with an initializer weight and explicit padding."""
    if n.op not in ("Conv", "FusedConv") or len(n.inputs) < 2 or n.inputs[1] not in g.initializers:
        return None
    w = g.initializers[n.inputs[1]]
    if w.ndim != 4 or w.dtype != np.float32 or n.attrs.get("auto_pad", "NOTSET") != "NOTSET":
        return None
    strides = [int(v) for v in n.attrs.get("strides", [1, 1])]
    pads = [int(v) for v in n.attrs.get("pads", [0, 0, 0, 0])]
    dilations = [int(v) for v in n.attrs.get("dilations", [1, 1])]
    return tuple(w.shape), strides, pads, dilations, int(n.attrs.get("group", 1))


def pair_downsample_convs(g: Graph) -> Graph:
    """Pairs a 3x3 convolution (pad 1, dilation 1, group 1; a Conv or a
    FusedConv) with a 1x1 Conv (pad 0, bias optional) of the same input,
    stride and output channels -- a ResNet block's first conv and its
    downsampling shortcut -- into one FusedConv node with six inputs
    (X, W, B, Z, W2, B2) and two outputs, which nert_hip_conv_pair_f32 runs in
    one launch (the 1x1 reads the 3x3's centre-tap inputs). The 3x3 output
    keeps its bits; the 1x1 output differs from the separate Conv row only in
    the order of its fp32 additions. The pair sits at the later of the two
    nodes' positions, which is taken only when no node in between reads the
    earlier node's output.
    """
    consumers: dict[str, list[int]] = {}
    for idx, n in enumerate(g.nodes):
        for t in n.inputs:
            if t:
                consumers.setdefault(t, []).append(idx)
    replace: dict[int, Node] = {}
    dropped: set[int] = set()
    for idx, n in enumerate(g.nodes):
        geo = _conv_geometry(g, n)
        if idx in dropped or idx in replace or geo is None or len(n.outputs) != 1 or len(n.inputs) > 4:
            continue
        ws, strides, pads, dil, group = geo
        if ws[2:] != (3, 3) or pads != [1, 1, 1, 1] or dil != [1, 1] or group != 1:
            continue
        for c in consumers.get(n.inputs[0], []):
            d = g.nodes[c]
            if c == idx or c in dropped or c in replace or d.op != "Conv" or len(d.outputs) != 1:
                continue
            dgeo = _conv_geometry(g, d)
            if dgeo is None or dgeo[0] != (ws[0], ws[1], 1, 1) or dgeo[1] != strides or any(dgeo[2]) or \
                    dgeo[3] != [1, 1] or dgeo[4] != 1:
                continue
            b2 = d.inputs[2] if len(d.inputs) > 2 else ""
            if b2 and b2 not in g.initializers:
                continue
            lo, hi = sorted((idx, c))
            early_out = g.nodes[lo].outputs[0]
            if any(lo < k < hi for k in consumers.get(early_out, [])):
                continue
            if g.tensors[d.outputs[0]][1] != g.tensors[n.outputs[0]][1]:
                continue
            ins = list(n.inputs) + [""] * (4 - len(n.inputs))
            attrs = {k: v for k, v in n.attrs.items() if k in ("strides", "pads", "dilations", "group", "activation")}
            replace[hi] = Node("FusedConv", ins + [d.inputs[1], b2], [n.outputs[0], d.outputs[0]], attrs, n.name)
            dropped.add(lo)
            break
    nodes = [replace.get(i, nd) for i, nd in enumerate(g.nodes) if i not in dropped]
    return Graph(nodes=nodes, initializers=g.initializers, inputs=g.inputs, outputs=g.outputs, tensors=g.tensors)


def pack_conv_weights(g: Graph) -> Graph:
    """Gives every 3x3 Conv or FusedConv whose weight is a float32
    initializer with C/group a multiple of 8 a second copy of that weight in
    the order the 3x3 LDS-patch kernel stores it -- per output channel,
    blocks of 8 input channels, in a block the 9 taps, in a tap the 8
    channels: packed[m][b][t][j] = W[m][8 b + j][t] -- as the FusedConv row's
    seventh input (X, W, B, Z, W2, B2, W packed; the omitted ones empty),
    which runs nert_hip_conv_packed_f32. The kernel then copies the weights
    to LDS with 16-byte stores instead of transposing 4-byte ones. The copy
    is made once, here; the results are bit-identical."""
    initializers = dict(g.initializers)
    tensors = dict(g.tensors)
    nodes = []
    for n in g.nodes:
        w_name = n.inputs[1] if len(n.inputs) > 1 else ""
        w = g.initializers.get(w_name)
        fits = n.op in ("Conv", "FusedConv") and len(n.inputs) <= 6 and w is not None and w.dtype == np.float32 and \
            w.ndim == 4 and w.shape[2:] == (3, 3) and w.shape[1] % 8 == 0
        if not fits:
            nodes.append(n)
            continue
        name = w_name + ":packed"
        if name not in initializers:
            m, cg = w.shape[0], w.shape[1]
            packed = np.ascontiguousarray(w.reshape(m, cg // 8, 8, 9).transpose(0, 1, 3, 2)).reshape(w.shape)
            initializers[name] = packed
            tensors[name] = (packed.dtype, tuple(packed.shape))
        ins = list(n.inputs) + [""] * (6 - len(n.inputs)) + [name]
        nodes.append(Node("FusedConv", ins, list(n.outputs), dict(n.attrs), n.name))
    return Graph(nodes=nodes, initializers=initializers, inputs=g.inputs, outputs=g.outputs, tensors=tensors)


def _scalar(g: Graph, name: str) -> float | None:
    """The value of a float32 scalar initializer (shape () or (1,)), else None."""
    v = g.initializers.get(name)
    if v is None or v.dtype != np.float32 or v.size != 1 or v.ndim > 1:
        return None
    return float(v.reshape(()))


def fuse_matmul_chains(g: Graph) -> Graph:
    """Rewrites MatMul -> [Mul by a scalar] -> [Add of a [N] bias] -> [erf
    Gelu: Div by c1, Erf, Add c2, Mul by the pre-Gelu value, Mul by c3] into
    one FusedMatMul node (alpha, bias and the Gelu constants in its epilogue).

    Every intermediate must have exactly the consumers the pattern names and
    not be a graph output; scalars and the bias must be float32 initializers.
    The fused node sits where the chain's last node was. Its epilogue rounds
    each step like the separate rows, so the outputs are bit-identical.
    """
    consumers: dict[str, list[int]] = {}
    for idx, n in enumerate(g.nodes):
        for t in n.inputs:
            if t:
                consumers.setdefault(t, []).append(idx)
    outputs = set(g.outputs)

    def sole(t: str) -> int | None:
        c = consumers.get(t, [])
        return c[0] if len(c) == 1 and t not in outputs else None

    def other(n: Node, t: str) -> str | None:
        if len(n.inputs) != 2:
            return None
        if n.inputs[0] == t:
            return n.inputs[1]
        return n.inputs[0] if n.inputs[1] == t else None

    dropped: set[int] = set()
    replace: dict[int, Node] = {}
    for idx, n in enumerate(g.nodes):
        if n.op != "MatMul" or idx in dropped or len(n.inputs) != 2:
            continue
        chain = [idx]
        cur = n.outputs[0]
        shape = g.tensors[cur][1]
        attrs: dict[str, Any] = {}
        bias = ""
        nxt = sole(cur)
        if nxt is not None and g.nodes[nxt].op == "Mul":
            c = other(g.nodes[nxt], cur)
            v = _scalar(g, c) if c else None
            if v is not None and g.tensors[g.nodes[nxt].outputs[0]][1] == shape:
                attrs["alpha"] = v
                chain.append(nxt)
                cur = g.nodes[nxt].outputs[0]
                nxt = sole(cur)
        if nxt is not None and g.nodes[nxt].op == "Add":
            c = other(g.nodes[nxt], cur)
            init = g.initializers.get(c) if c else None
            if (init is not None and init.dtype == np.float32 and init.shape == (shape[-1],)
                    and g.tensors[g.nodes[nxt].outputs[0]][1] == shape):
                bias = c
                chain.append(nxt)
                cur = g.nodes[nxt].outputs[0]
        gelu = _match_gelu(g, cur, consumers, outputs, other)
        if gelu is not None:
            nodes, consts = gelu
            attrs.update({"activation": "Gelu", "gelu_div": consts[0], "gelu_add": consts[1], "gelu_mul": consts[2]})
            chain.extend(nodes)
            cur = g.nodes[nodes[-1]].outputs[0]
        if len(chain) == 1:
            continue
        last = max(chain)
        for i in chain:
            dropped.add(i)
        dropped.discard(last)
        replace[last] = Node("FusedMatMul", [n.inputs[0], n.inputs[1]] + ([bias] if bias else []), [cur], attrs,
                             n.name)
    nodes = [replace.get(i, nd) for i, nd in enumerate(g.nodes) if i not in dropped or i in replace]
    return Graph(nodes=nodes, initializers=g.initializers, inputs=g.inputs, outputs=g.outputs, tensors=g.tensors)


def _match_gelu(g: Graph, v: str, consumers, outputs, other):
    """Div(v, c1) -> Erf -> Add(., c2) -> Mul(v, .) -> Mul(., c3) with v
    consumed only by the Div and the first Mul; returns (node indices,
    (c1, c2, c3)) or None."""
    cons = consumers.get(v, [])
    if v in outputs or len(cons) != 2:
        return None
    div = next((i for i in cons if g.nodes[i].op == "Div" and g.nodes[i].inputs[0] == v), None)
    if div is None:
        return None
    c1 = _scalar(g, g.nodes[div].inputs[1])

    def only(t):
        c = consumers.get(t, [])
        return c[0] if len(c) == 1 and t not in outputs else None

    erf = only(g.nodes[div].outputs[0])
    if c1 is None or erf is None or g.nodes[erf].op != "Erf":
        return None
    add = only(g.nodes[erf].outputs[0])
    if add is None or g.nodes[add].op != "Add":
        return None
    c2n = other(g.nodes[add], g.nodes[erf].outputs[0])
    c2 = _scalar(g, c2n) if c2n else None
    mul1 = only(g.nodes[add].outputs[0])
    if c2 is None or mul1 is None or g.nodes[mul1].op != "Mul" or mul1 not in cons:
        return None
    if other(g.nodes[mul1], g.nodes[add].outputs[0]) != v:
        return None
    mul2 = only(g.nodes[mul1].outputs[0])
    if mul2 is None or g.nodes[mul2].op != "Mul":
        return None
    c3n = other(g.nodes[mul2], g.nodes[mul1].outputs[0])
    c3 = _scalar(g, c3n) if c3n else None
    if c3 is None:
        return None
    return [div, erf, add, mul1, mul2], (c1, c2, c3)


def fuse_add_layernorm(g: Graph) -> Graph:
    """Rewrites a residual Add whose output feeds a LayerNormalization into
    one FusedAddLayerNorm node (outputs: the sum, which later rows still
    read, and the normalised tensor).

    The Add must sum two float32 tensors of its output's shape (no
    broadcasting); the LayerNormalization must take that sum as X, have only
    the Y output, and per-element float32 initializers for Scale (and B).
    The fused node sits where the Add was (the norm's other operands are
    initializers). The row adds in float32 like the Add row and normalises
    with the LayerNormalization row's kernel, so the outputs are
    bit-identical; the sum is read once instead of written and read back.
    """
    consumers: dict[str, list[int]] = {}
    for idx, n in enumerate(g.nodes):
        for t in n.inputs:
            if t:
                consumers.setdefault(t, []).append(idx)
    replace: dict[int, Node] = {}
    dropped: set[int] = set()
    for idx, n in enumerate(g.nodes):
        if n.op != "Add" or len(n.inputs) != 2 or len(n.outputs) != 1 or idx in dropped:
            continue
        out = n.outputs[0]
        dtype, shape = g.tensors[out]
        if np.dtype(dtype) != np.float32 or not shape or any(
                g.tensors[t][1] != shape or np.dtype(g.tensors[t][0]) != np.float32 for t in n.inputs):
            continue
        for c in consumers.get(out, []):
            ln = g.nodes[c]
            if ln.op != "LayerNormalization" or c in dropped or ln.inputs[0] != out or len(ln.outputs) != 1:
                continue
            axis = int(ln.attrs.get("axis", -1)) % len(shape)
            inner = int(np.prod(shape[axis:]))
            params = [t for t in ln.inputs[1:] if t]
            if not params or len(ln.inputs) > 3 or any(
                    t not in g.initializers or g.initializers[t].dtype != np.float32 or g.initializers[t].size != inner
                    or g.initializers[t].ndim != 1 for t in params):
                continue
            attrs = {"axis": int(ln.attrs.get("axis", -1))}
            if "epsilon" in ln.attrs:
                attrs["epsilon"] = ln.attrs["epsilon"]
            replace[idx] = Node("FusedAddLayerNorm", [n.inputs[0], n.inputs[1]] + list(ln.inputs[1:]),
                                [out, ln.outputs[0]], attrs, ln.name)
            dropped.add(c)
            break
    nodes = [replace.get(i, nd) for i, nd in enumerate(g.nodes) if i not in dropped]
    return Graph(nodes=nodes, initializers=g.initializers, inputs=g.inputs, outputs=g.outputs, tensors=g.tensors)


ATTENTION_HEAD_DIM = 64   # what nert_hip_attention_f32 computes


def _ints(g: Graph, name: str) -> list[int] | None:
    v = g.initializers.get(name)
    if v is None or v.dtype != np.int64:
        return None
    return [int(x) for x in v.reshape(-1)]


def fuse_attention(g: Graph) -> Graph:
    """Rewrites a transformer encoder's attention block into one
    FusedAttention node:

        qkv [B,S,3*H*D] -Reshape-> [B,S,3,H,D] -Transpose(2,0,3,1,4)-> Split
        (axis 0, three parts) -> Squeeze(axis 0) -> q, k, v [B,H,S,D];
        MatMul(q, Transpose(k, 0,1,3,2)) -> Mul by a float32 scalar ->
        Softmax(last axis) -> MatMul(., v) -> Transpose(0,2,1,3) ->
        Reshape [B,S,H*D]

    becomes FusedAttention(qkv) -> [B,S,H*D] with attributes heads and
    scale, placed where the final Reshape was. Every intermediate must have
    exactly the consumer the pattern names and not be a graph output; D must
    be 64 (what the kernel computes). The fused row keeps Q,
    K and V where the projection wrote them and never materialises the
    scores in HBM; its values agree with the separate rows within the fp32
    parity bar (not bit for bit: the products accumulate in another order).
    """
    consumers: dict[str, list[int]] = {}
    producer: dict[str, int] = {}
    for idx, n in enumerate(g.nodes):
        for t in n.inputs:
            if t:
                consumers.setdefault(t, []).append(idx)
        for t in n.outputs:
            producer[t] = idx
    outputs = set(g.outputs)

    def sole(t: str) -> int | None:
        c = consumers.get(t, [])
        return c[0] if len(c) == 1 and t not in outputs else None

    def made_by(t: str, op: str, consumer: int) -> int | None:
        """Index of t's producer if it is an `op` node whose only output t
        feeds only `consumer`."""
        i = producer.get(t)
        if i is None or g.nodes[i].op != op or sole(t) != consumer:
            return None
        return i

    def perm(i: int) -> list[int] | None:
        p = g.nodes[i].attrs.get("perm")
        return [int(x) for x in p] if p is not None else None

    replace: dict[int, Node] = {}
    dropped: set[int] = set()
    for si, sm in enumerate(g.nodes):
        if sm.op != "Softmax" or si in dropped or len(sm.inputs) != 1 or len(sm.outputs) != 1:
            continue
        p = sm.outputs[0]
        dt, pshape = g.tensors[p]
        if np.dtype(dt) != np.float32 or len(pshape) != 4 or int(sm.attrs.get("axis", -1)) not in (-1, 3):
            continue
        mul = made_by(sm.inputs[0], "Mul", si)
        if mul is None or len(g.nodes[mul].inputs) != 2:
            continue
        a0, a1 = g.nodes[mul].inputs
        scale, s = (_scalar(g, a1), a0) if _scalar(g, a1) is not None else (_scalar(g, a0), a1)
        if scale is None:
            continue
        mm1 = made_by(s, "MatMul", mul)
        if mm1 is None:
            continue
        q, kt = g.nodes[mm1].inputs
        tk = made_by(kt, "Transpose", mm1)
        if tk is None or perm(tk) != [0, 1, 3, 2]:
            continue
        k = g.nodes[tk].inputs[0]
        mm2 = sole(p)
        if mm2 is None or g.nodes[mm2].op != "MatMul" or g.nodes[mm2].inputs[0] != p:
            continue
        v = g.nodes[mm2].inputs[1]
        to = sole(g.nodes[mm2].outputs[0])
        if to is None or g.nodes[to].op != "Transpose" or perm(to) != [0, 2, 1, 3]:
            continue
        rs = sole(g.nodes[to].outputs[0])
        if rs is None or g.nodes[rs].op != "Reshape":
            continue
        out = g.nodes[rs].outputs[0]
        # q, k, v: the three parts of one Split, each through Squeeze(axis 0).
        sq = [made_by(t, "Squeeze", c) for t, c in ((q, mm1), (k, tk), (v, mm2))]
        if any(i is None for i in sq):
            continue
        parts = [g.nodes[i].inputs[0] for i in sq]
        if any(_ints(g, g.nodes[i].inputs[1]) != [0] if len(g.nodes[i].inputs) > 1 and g.nodes[i].inputs[1]
               else [int(x) for x in g.nodes[i].attrs.get("axes", [])] != [0] for i in sq):
            continue
        sp = producer.get(parts[0])
        if sp is None or g.nodes[sp].op != "Split" or g.nodes[sp].outputs != parts or any(
                sole(t) != i for t, i in zip(parts, sq)) or int(g.nodes[sp].attrs.get("axis", 0)) != 0:
            continue
        split_sizes = (_ints(g, g.nodes[sp].inputs[1]) if len(g.nodes[sp].inputs) > 1 and g.nodes[sp].inputs[1]
                       else g.nodes[sp].attrs.get("split"))
        if split_sizes is not None and [int(x) for x in split_sizes] != [1, 1, 1]:
            continue
        t5 = made_by(g.nodes[sp].inputs[0], "Transpose", sp)
        if t5 is None or perm(t5) != [2, 0, 3, 1, 4]:
            continue
        r5 = made_by(g.nodes[t5].inputs[0], "Reshape", t5)
        if r5 is None:
            continue
        qkv = g.nodes[r5].inputs[0]
        qdt, qkv_shape = g.tensors[qkv]
        _, shape5 = g.tensors[g.nodes[r5].outputs[0]]
        if np.dtype(qdt) != np.float32 or len(qkv_shape) != 3 or len(shape5) != 5:
            continue
        b_, s_, three, h_, d_ = shape5
        if (three != 3 or tuple(qkv_shape) != (b_, s_, 3 * h_ * d_) or d_ != ATTENTION_HEAD_DIM
                or s_ <= 0 or tuple(g.tensors[out][1]) != (b_, s_, h_ * d_)
                or tuple(pshape) != (b_, h_, s_, s_)):
            continue
        replace[rs] = Node("FusedAttention", [qkv], [out], {"heads": int(h_), "scale": float(scale)}, sm.name)
        dropped.update([r5, t5, sp, *sq, tk, mm1, mul, si, mm2, to])
    nodes = [replace.get(i, nd) for i, nd in enumerate(g.nodes) if i not in dropped]
    return Graph(nodes=nodes, initializers=g.initializers, inputs=g.inputs, outputs=g.outputs, tensors=g.tensors)


class _PackedNode:
    __slots__ = ("op", "name", "attrs", "ins", "outs", "err")

    def __init__(self, op: str, name: str, attrs: abi.AttrPack, ins: abi.TensorPack, outs: abi.TensorPack):
        self.op = op.encode()
        self.name = name.encode()
        self.attrs = attrs
        self.ins = ins
        self.outs = outs
        self.err = C.create_string_buffer(1024)


def fuse_rows(g: Graph, attention: bool = True, pairs: bool = True, packed: bool = True) -> Graph:
    """The runner's fusions in order: Conv chains, 3x3 convs paired with
    their 1x1 downsampling shortcuts (when `pairs`), packed 3x3 weights (when
    `packed`), attention blocks (when `attention`), MatMul chains, residual
    Add + LayerNorm. All but the pairs' 1x1 outputs and the attention blocks
    are bit-identical to the separate rows; those two sum in another order,
    within the rows' tolerance."""
    g = fuse_conv_chains(g)
    if pairs:
        g = pair_downsample_convs(g)
    if packed:
        g = pack_conv_weights(g)
    if attention:
        g = fuse_attention(g)
    return fuse_add_layernorm(fuse_matmul_chains(g))


class Program:
    def __init__(self, g: Graph, fuse: bool = True, views: bool = True, attention: bool = True, pairs: bool = True,
                 packed: bool = True):
        if fuse:
            g = fuse_rows(g, attention, pairs, packed)
        self.alias: dict[str, tuple[str, int]] = {}
        if views:
            g, self.alias = alias_views(g)
        self.graph = g
        self.offsets, self.arena_bytes = plan_arena(g, self.alias)
        self.arena = DeviceArray((max(self.arena_bytes, 1),), np.uint8)
        self.resident: dict[str, DeviceArray] = {}
        for name, value in g.initializers.items():
            self.resident[name] = DeviceArray.from_host(value)
        for name in g.inputs:
            dtype, shape = g.tensors[name]
            self.resident[name] = DeviceArray(shape, dtype)
        self.nodes = [self._pack(n) for n in g.nodes]
        self.exec_graph = None
        self._events: list[Event] = []
        self._control: dict[str, np.ndarray] = {}

    def ptr(self, name: str) -> int:
        if name in self.resident:
            return self.resident[name].ptr or 0
        return (self.arena.ptr or 0) + self.offsets[name]

    def _entry(self, name: str):
        if not name:
            return None
        dtype, shape = self.graph.tensors[name]
        return (self.ptr(name), abi.dtype_code(dtype), shape)

    def _pack(self, n) -> _PackedNode:
        return _PackedNode(n.op, n.name, abi.AttrPack(n.attrs), abi.TensorPack([self._entry(t) for t in n.inputs]),
                           abi.TensorPack([self._entry(t) for t in n.outputs]))

    def set_input(self, name: str, value: np.ndarray) -> None:
        """Uploads a graph input. Rows read small integer operands (indices,
        shapes, divisors) on the host when they launch, so once the program
        is captured, a new value for an int64 or bool input re-captures it:
        the graph then carries launches checked against the new values."""
        d = self.resident[name]
        a = np.asarray(value, dtype=d.dtype, order="C")
        if a.shape != d.shape:
            raise ValueError(f"input {name}: shape {a.shape} != {d.shape}")
        control = d.dtype in (np.dtype(np.int64), np.dtype(np.bool_))
        changed = control and not np.array_equal(self._control.get(name), a)
        check(lib().nert_hip_memcpy_h2d(d.ptr, a.ctypes.data, d.nbytes), "h2d")
        if control:
            self._control[name] = a.copy()
        if changed and self.exec_graph is not None:
            self.close()
            self.capture()

    def check_errors(self) -> None:
        """Raises NertError when rows run since the last check (a replayed
        graph's deferred checks included) raised the device error word: an
        out-of-range Gather/GatherElements/ScatterND index or an int64
        division by zero. Synchronises the layer stream."""
        flags = take_error_flags()
        if flags:
            what = ", ".join(t for bit, t in ERROR_FLAG_TEXT.items() if flags & bit) or f"flags {flags:#x}"
            raise NertError(abi.INFERENCE_ERROR, f"device error raised by the replayed rows: {what}")

    def output(self, name: str) -> np.ndarray:
        dtype, shape = self.graph.tensors[name]
        out = np.empty(shape, dtype)
        if out.nbytes:
            check(lib().nert_hip_memcpy_d2h(out.ctypes.data, self.ptr(name), out.nbytes), "d2h")
        return out

    def _call(self, p: _PackedNode) -> None:
        rc = lib().nert_hip_run_node(p.op, p.name, 0, p.attrs.array, p.attrs.count, p.ins.array, p.ins.count,
                                     p.outs.array, p.outs.count, p.err, len(p.err))
        if rc != abi.OK:
            raise NertError(rc, p.err.value.decode())

    def run(self) -> None:
        """Queues every node once (asynchronous; the layer stream orders it)."""
        for p in self.nodes:
            self._call(p)

    def run_timed(self, ops: Iterable[str]) -> dict[int, float]:
        """Runs once with HIP events around each node whose op is in `ops`;
        returns {node index: milliseconds} measured on the layer stream."""
        wanted = {o.encode() for o in ops}
        marks: list[tuple[int, Event, Event]] = []
        need = sum(1 for p in self.nodes if p.op in wanted)
        while len(self._events) < 2 * need:
            self._events.append(Event())
        k = 0
        for idx, p in enumerate(self.nodes):
            if p.op in wanted:
                e0, e1 = self._events[k], self._events[k + 1]
                k += 2
                e0.record()
                self._call(p)
                e1.record()
                marks.append((idx, e0, e1))
            else:
                self._call(p)
        return {idx: e0.elapsed_ms(e1) for idx, e0, e1 in marks}

    def time_rows(self, indices: Iterable[int], reps: int = 20) -> dict[int, float]:
        """Per-row device time as the replayed step sees it: for each node
        index, `reps` back-to-back launches of that row alone are captured
        into one HIP graph, which is replayed twice (warm) and then once
        between HIP events on the layer stream. Returns {index: ms per
        launch}. Rows run on the operands the last full run left in place, so
        call it after run() or replay(); the output buffers are rewritten
        with the same values."""
        result: dict[int, float] = {}
        e0, e1 = Event(), Event()
        for idx in indices:
            p = self.nodes[idx]
            check(lib().nert_hip_stream_sync(None), "sync")
            check(lib().nert_hip_capture_begin(), "capture begin")
            try:
                for _ in range(reps):
                    self._call(p)
            finally:
                handle = C.c_void_p()
                rc = lib().nert_hip_capture_end(C.byref(handle))
            check(rc, "capture end")
            try:
                for _ in range(2):
                    check(lib().nert_hip_graph_launch(handle, None), "graph launch")
                e0.record()
                check(lib().nert_hip_graph_launch(handle, None), "graph launch")
                e1.record()
                result[idx] = e0.elapsed_ms(e1) / reps
            finally:
                lib().nert_hip_graph_destroy(handle)
        return result

    def capture(self) -> None:
        """Captures the node sequence into one HIP graph (after a warm run so
        every workspace has reached its size)."""
        self.run()
        check(lib().nert_hip_stream_sync(None), "sync")
        check(lib().nert_hip_capture_begin(), "capture begin")
        try:
            self.run()
        finally:
            handle = C.c_void_p()
            rc = lib().nert_hip_capture_end(C.byref(handle))
        check(rc, "capture end")
        self.exec_graph = handle

    def replay(self) -> None:
        if self.exec_graph is None:
            raise NertError(abi.OTHER_ERROR, "replay before capture")
        check(lib().nert_hip_graph_launch(self.exec_graph, None), "graph launch")

    def close(self) -> None:
        if self.exec_graph is not None:
            lib().nert_hip_graph_destroy(self.exec_graph)
            self.exec_graph = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
