"""GPU parity of the fused attention row (FusedAttention, through
nert_hip_attention_f32) against the reference executor running the separate
rows it replaces (MatMul, Mul, Softmax, MatMul and the Reshape / Transpose /
Split / Squeeze copies around them: src/kernels/mat_mul.cpp, mul.cpp,
softmax.cpp, transpose.cpp, split.cpp), on the same seeded inputs. Float
outputs within 1e-4 + 1e-4|ref|. Cases: the ViT-B/16 shape, one token, a
ragged sequence, long sequences (512, 1000), batch x heads not a multiple
of 8 (the plain workgroup order), steep scores, non-power-of-two scales. (With
inputs of std 6 the scores reach +-100 and the fp32 rounding of the 64-term
dot products alone moves the outputs by about the 1e-4 bar, for any fp32
evaluation of the rows; the steep cases here stay at std 3.)"""

import ctypes as C
import os
import tempfile
from pathlib import Path

import numpy as np
import pytest

from attn_graph import attention_block
from nert_amd import graph
from nert_amd.device import DeviceArray, check, lib, synchronize
from nert_amd.runner import Program
from oracle import ref
from rowcheck import compare

pytestmark = pytest.mark.gpu


def _reference(g, feeds: list[np.ndarray], out_shapes) -> list[np.ndarray]:
    path = os.path.join(tempfile.mkdtemp(), "attn.onnx")
    Path(path).write_bytes(graph.to_onnx(g))
    lg = ref.LoadedGraph(path)
    try:
        outs = [np.zeros(s, np.float32) for s in out_shapes]
        ref.model_run(lg.handle, feeds, outs)
        return outs
    finally:
        lg.close()


@pytest.mark.parametrize("batch,seq,heads,scale,std", [
    (2, 197, 12, 0.125, 1.0),   # ViT-B/16
    (1, 1, 1, 0.125, 1.0),      # one token
    (3, 33, 5, 0.1, 1.0),       # ragged, B*H = 15
    (1, 1000, 2, 0.125, 1.0),   # long: 32 key blocks, the last partial
    (2, 512, 4, 0.125, 1.0),    # whole key blocks only, B*H = 8
    (2, 64, 4, 0.125, 3.0),     # steep scores: std 9, softmax peaks near e^27
    (1, 95, 8, 0.3, 3.0),       # std 22
])
def test_fused_attention_matches_reference_rows(gpu, batch, seq, heads, scale, std):
    print(f"case batch={batch} seq={seq} heads={heads}", flush=True)
    g = attention_block(batch, seq, heads, scale=scale)
    rng = np.random.default_rng(seq * 1000 + heads)
    qkv = (rng.standard_normal((batch, seq, 3 * heads * 64)) * std).astype(np.float32)
    prog = Program(g)
    try:
        assert [n.op for n in prog.graph.nodes] == ["FusedAttention"]
        prog.set_input("qkv", qkv)
        prog.run()
        prog.check_errors()
        eager = prog.output("attn_out")
        prog.capture()
        prog.replay()
        prog.replay()
        prog.check_errors()
        assert np.array_equal(prog.output("attn_out"), eager), "replay differs from the eager run"
    finally:
        prog.close()
    (want,) = _reference(g, [qkv], [(batch, seq, heads * 64)])
    compare(eager, want, what=f"attention {batch}x{seq}x{heads}")


def _head_major_reference(q, k, v, scale: float) -> np.ndarray:
    """MatMul(Q, K^T), Mul, Softmax, MatMul(P, V) on the reference executor
    for [B, H, S, D] tensors."""
    b, h, s, d = q.shape
    g = graph.Graph()
    for n in ("q", "k", "v"):
        g.add_input(n, np.float32, (b, h, s, d))
    g.add_initializer("scale", np.array(scale, np.float32))
    kt = g.add_node("Transpose", ["k"], [("kt", np.float32, (b, h, d, s))], {"perm": [0, 1, 3, 2]})[0]
    sc = g.add_node("MatMul", ["q", kt], [("s", np.float32, (b, h, s, s))])[0]
    sc = g.add_node("Mul", [sc, "scale"], [("ss", np.float32, (b, h, s, s))])[0]
    p = g.add_node("Softmax", [sc], [("p", np.float32, (b, h, s, s))], {"axis": -1})[0]
    o = g.add_node("MatMul", [p, "v"], [("o", np.float32, (b, h, s, d))])[0]
    g.outputs.append(o)
    (want,) = _reference(g, [q, k, v], [(b, h, s, d)])
    return want


def test_attention_entry_point_with_head_major_strides(gpu):
    """nert_hip_attention_f32 on separate Q, K, V tensors in [B, H, S, D]
    layout, written to a [B, H, S, D] output (strides other than the packed
    projection's), against MatMul / Mul / Softmax / MatMul on the reference."""
    b, h, s, d = 3, 3, 70, 64
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((b, h, s, d)).astype(np.float32) for _ in range(3))
    want = _head_major_reference(q, k, v, 0.2)
    dq, dk, dv = (DeviceArray.from_host(t) for t in (q, k, v))
    out = DeviceArray.from_host(np.zeros((b, h, s, d), np.float32))
    strides = (C.c_int64 * 3)(h * s * d, d, s * d)
    check(lib().nert_hip_attention_f32(dq.ptr, dk.ptr, dv.ptr, out.ptr, b, h, s, d, strides, strides, 0.2, None),
          "attention")
    synchronize()
    compare(out.to_host(), want, what="head-major attention")
    for t in (dq, dk, dv, out):
        t.close()


@pytest.mark.parametrize("seq", [1, 33, 197])
def test_attention_reads_no_key_past_the_sequence(gpu, seq):
    """Each (batch, head) slice of K and V sits in a larger buffer whose rows
    after the sequence hold NaN, +inf and -inf (inside the allocation, so a
    read of them cannot fault). The last key block's rows past the sequence
    must not be read: the output stays finite and matches the reference rows
    on the unpadded tensors."""
    b, h, d, spare = 2, 3, 64, 40
    print(f"case seq={seq}", flush=True)
    rng = np.random.default_rng(seq + 17)
    q, k, v = (rng.standard_normal((b, h, seq, d)).astype(np.float32) for _ in range(3))
    want = _head_major_reference(q, k, v, 0.125)

    def poisoned(t: np.ndarray) -> np.ndarray:
        full = np.empty((b, h, seq + spare, d), np.float32)
        full[:, :, :seq] = t
        full[:, :, seq::3] = np.nan
        full[:, :, seq + 1::3] = np.inf
        full[:, :, seq + 2::3] = -np.inf
        return full

    # One stride set serves Q, K and V, so Q sits in the same padded layout
    # (its rows past the sequence are never read either).
    dq, dk, dv = (DeviceArray.from_host(poisoned(t)) for t in (q, k, v))
    out = DeviceArray.from_host(np.zeros((b, h, seq, d), np.float32))
    in_strides = (C.c_int64 * 3)(h * (seq + spare) * d, d, (seq + spare) * d)
    out_strides = (C.c_int64 * 3)(h * seq * d, d, seq * d)
    check(lib().nert_hip_attention_f32(dq.ptr, dk.ptr, dv.ptr, out.ptr, b, h, seq, d, in_strides, out_strides,
                                       0.125, None), "attention")
    synchronize()
    got = out.to_host()
    assert np.isfinite(got).all(), "a key row past the sequence reached the output"
    compare(got, want, what=f"attention over poisoned padding, seq {seq}")
    for t in (dq, dk, dv, out):
        t.close()


def test_attention_entry_point_rejects_unsupported_shapes(gpu):
    """head_dim other than 64, a token stride shorter than the head and
    misaligned rows are refused with a message, before any launch."""
    buf = DeviceArray.from_host(np.zeros(3 * 64 * 64 + 4, np.float32))
    packed = (C.c_int64 * 3)(0, 3 * 64, 64)
    L = lib()
    assert L.nert_hip_attention_f32(buf.ptr, buf.ptr, buf.ptr, buf.ptr, 1, 1, 8, 32, packed, packed, 1.0, None) != 0
    assert "head_dim" in L.nert_hip_last_error().decode()
    short = (C.c_int64 * 3)(0, 32, 64)
    assert L.nert_hip_attention_f32(buf.ptr, buf.ptr, buf.ptr, buf.ptr, 1, 1, 8, 64, short, packed, 1.0, None) != 0
    assert "token stride" in L.nert_hip_last_error().decode()
    odd = buf.ptr + 4
    assert L.nert_hip_attention_f32(odd, odd, odd, buf.ptr, 1, 1, 8, 64, packed, packed, 1.0, None) != 0
    assert "aligned" in L.nert_hip_last_error().decode()
    buf.close()
