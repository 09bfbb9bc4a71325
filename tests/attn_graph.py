"""A transformer encoder's attention block as separate reference rows, the form
the runner's fuse_attention pass rewrites (nert_amd/workloads.py builds the same
block inside vit_b16):

    qkv [B,S,3*H*D] -Reshape-> [B,S,3,H,D] -Transpose(2,0,3,1,4)-> Split(axis 0)
    -> Squeeze(axis 0) -> q, k, v; MatMul(q, Transpose(k, 0,1,3,2)) -> Mul(scale)
    -> Softmax(-1) -> MatMul(., v) -> Transpose(0,2,1,3) -> Reshape [B,S,H*D]
"""

from __future__ import annotations

import numpy as np

from nert_amd.graph import Graph

F32 = np.float32


def attention_block(batch: int, seq: int, heads: int, head_dim: int = 64, scale: float = 0.125,
                    scores_output: bool = False) -> Graph:
    g = Graph()
    qkv = g.add_input("qkv", F32, (batch, seq, 3 * heads * head_dim))
    i64 = lambda name, v: g.add_initializer(name, np.asarray(v, np.int64))  # noqa: E731
    g.add_initializer("scale", np.array(scale, F32))

    def node(op, ins, shape, attrs=None, name=None):
        return g.add_node(op, ins, [(name or f"t{len(g.nodes)}", F32, shape)], attrs)[0]

    x5 = node("Reshape", [qkv, i64("shape5", [batch, seq, 3, heads, head_dim])], (batch, seq, 3, heads, head_dim))
    xt = node("Transpose", [x5], (3, batch, heads, seq, head_dim), {"perm": [2, 0, 3, 1, 4]})
    parts = g.add_node("Split", [xt, i64("split3", [1, 1, 1])],
                       [(f"part{i}", F32, (1, batch, heads, seq, head_dim)) for i in range(3)], {"axis": 0})
    axis0 = i64("axis0", [0])
    q, k, v = (node("Squeeze", [p, axis0], (batch, heads, seq, head_dim)) for p in parts)
    kt = node("Transpose", [k], (batch, heads, head_dim, seq), {"perm": [0, 1, 3, 2]})
    s = node("MatMul", [q, kt], (batch, heads, seq, seq))
    s = node("Mul", [s, "scale"], (batch, heads, seq, seq))
    p = node("Softmax", [s], (batch, heads, seq, seq), {"axis": -1}, name="probs")
    o = node("MatMul", [p, v], (batch, heads, seq, head_dim))
    o = node("Transpose", [o], (batch, seq, heads, head_dim), {"perm": [0, 2, 1, 3]})
    y = node("Reshape", [o, i64("shape3", [batch, seq, heads * head_dim])], (batch, seq, heads * head_dim),
             name="attn_out")
    g.outputs.append(y)
    if scores_output:
        g.outputs.append(p)
    return g
