"""Writes tests/golden/known_answers.json: the hand-computed input/output values
that the reference's own tests assert, transcribed as data.

Each case cites the reference test it comes from (olibartfast/nert
test/kernels_test.cpp or test/hip_kernels_test.cpp). The values are the
tests' literals; nothing here runs or imports the reference.

    python tests/golden/make_known_answers.py
"""

import json
from pathlib import Path


def t(shape, data, dtype="f32"):
    return {"shape": list(shape), "dtype": dtype, "data": list(data)}


CASES = [
    # --- Gemm: test/kernels_test.cpp:370-441, test/hip_kernels_test.cpp:99-128
    dict(id="GemmPlainProduct", src="test/kernels_test.cpp:370", op="Gemm",
         inputs=[t([2, 3], [1, 2, 3, 4, 5, 6]), t([3, 2], [7, 8, 9, 10, 11, 12])],
         outputs=[t([2, 2], [58, 64, 139, 154])]),
    dict(id="GemmTransA", src="test/kernels_test.cpp:383", op="Gemm", attrs={"transA": 1},
         inputs=[t([3, 2], [1, 2, 3, 4, 5, 6]), t([3, 2], [7, 8, 9, 10, 11, 12])],
         outputs=[t([2, 2], [89, 98, 116, 128])]),
    dict(id="GemmTransB", src="test/kernels_test.cpp:397", op="Gemm", attrs={"transB": 1},
         inputs=[t([2, 3], [1, 2, 3, 4, 5, 6]), t([2, 3], [7, 9, 11, 8, 10, 12])],
         outputs=[t([2, 2], [58, 64, 139, 154])]),
    dict(id="GemmAlphaBetaRankOneBias", src="test/kernels_test.cpp:411", op="Gemm",
         attrs={"alpha": 2.0, "beta": 0.5},
         inputs=[t([2, 2], [1, 2, 3, 4]), t([2, 2], [5, 6, 7, 8]), t([2], [10, 20])],
         outputs=[t([2, 2], [43, 54, 91, 110])]),
    # --- MatMul: test/kernels_test.cpp:443-510, test/hip_kernels_test.cpp:199-260
    dict(id="MatMulTwoDimensional", src="test/kernels_test.cpp:443", op="MatMul",
         inputs=[t([2, 3], [1, 2, 3, 4, 5, 6]), t([3, 2], [7, 8, 9, 10, 11, 12])],
         outputs=[t([2, 2], [58, 64, 139, 154])]),
    dict(id="MatMulBatchedThreeDimensional", src="test/kernels_test.cpp:456", op="MatMul",
         inputs=[t([2, 2, 3], [1, 2, 3, 4, 5, 6, 1, 0, 1, 0, 1, 0]),
                 t([2, 3, 2], [1, 0, 0, 1, 1, 1, 2, 0, 0, 2, 0, 0])],
         outputs=[t([2, 2, 2], [4, 5, 10, 11, 2, 0, 0, 2])]),
    dict(id="MatMulPromotesOneDimensionalLhs", src="test/kernels_test.cpp:469", op="MatMul",
         inputs=[t([3], [1, 2, 3]), t([3, 2], [1, 0, 0, 1, 1, 1])], outputs=[t([2], [4, 5])]),
    dict(id="MatMulPromotesOneDimensionalRhs", src="test/kernels_test.cpp:482", op="MatMul",
         inputs=[t([2, 3], [1, 2, 3, 4, 5, 6]), t([3], [1, 0, 1])], outputs=[t([2], [4, 10])]),
    dict(id="HipMatMulBatchedBroadcast", src="test/hip_kernels_test.cpp:199", op="MatMul",
         inputs=[t([2, 3], [1, 2, 3, 4, 5, 6]), t([2, 3, 2], [1, 0, 0, 1, 1, 1, 2, 0, 0, 2, 1, 0])],
         outputs=[t([2, 2, 2], [4, 5, 10, 11, 5, 4, 14, 10])]),
    dict(id="HipMatMulPromotedVector", src="test/hip_kernels_test.cpp:232", op="MatMul",
         inputs=[t([3], [1, 2, 3]), t([3, 2], [1, 2, 3, 4, 5, 6])], outputs=[t([2], [22, 28])]),
    # --- Conv: test/kernels_test.cpp:511-602, test/hip_kernels_test.cpp:603-700
    dict(id="ConvIdentityOneByOne", src="test/kernels_test.cpp:511", op="Conv",
         inputs=[t([1, 1, 3, 3], range(1, 10)), t([1, 1, 1, 1], [1])],
         outputs=[t([1, 1, 3, 3], range(1, 10))]),
    dict(id="ConvKnownTwoByTwoKernel", src="test/kernels_test.cpp:524", op="Conv",
         inputs=[t([1, 1, 3, 3], range(1, 10)), t([1, 1, 2, 2], [1, 1, 1, 1])],
         outputs=[t([1, 1, 2, 2], [12, 16, 24, 28])]),
    dict(id="ConvWithBias", src="test/kernels_test.cpp:537", op="Conv",
         inputs=[t([1, 1, 3, 3], range(1, 10)), t([1, 1, 2, 2], [1, 1, 1, 1]), t([1], [0.5])],
         outputs=[t([1, 1, 2, 2], [12.5, 16.5, 24.5, 28.5])]),
    dict(id="ConvDepthwiseGroupEqualsChannels", src="test/kernels_test.cpp:552", op="Conv", attrs={"group": 2},
         inputs=[t([1, 2, 2, 2], [1, 2, 3, 4, 10, 20, 30, 40]), t([2, 1, 2, 2], [1, 0, 0, 1, 0, 1, 1, 0])],
         outputs=[t([1, 2, 1, 1], [5, 50])]),
    dict(id="ConvStrideAndPadding", src="test/kernels_test.cpp:568", op="Conv",
         attrs={"strides": [2, 2], "pads": [1, 1, 1, 1]},
         inputs=[t([1, 1, 4, 4], range(1, 17)), t([1, 1, 3, 3], [1] * 9)],
         outputs=[t([1, 1, 2, 2], [14, 30, 57, 99])]),
    dict(id="HipConvPointwiseNoBias", src="test/hip_kernels_test.cpp:603", op="Conv",
         inputs=[t([1, 2, 2, 2], range(1, 9)), t([3, 2, 1, 1], [1, 0, 0, 1, 1, 1])],
         outputs=[t([1, 3, 2, 2], [1, 2, 3, 4, 5, 6, 7, 8, 6, 8, 10, 12])]),
    dict(id="HipConvPadded3x3WithBias", src="test/hip_kernels_test.cpp:634", op="Conv",
         attrs={"pads": [1, 1, 1, 1]},
         inputs=[t([1, 1, 3, 3], range(1, 10)), t([1, 1, 3, 3], [1] * 9), t([1], [10])],
         outputs=[t([1, 1, 3, 3], [22, 31, 26, 37, 55, 43, 34, 49, 38])]),
    dict(id="HipConvDepthwiseWithBias", src="test/hip_kernels_test.cpp:668", op="Conv", attrs={"group": 2},
         inputs=[t([1, 2, 2, 2], range(1, 9)), t([2, 1, 1, 1], [2, 3]), t([2], [1, -1])],
         outputs=[t([1, 2, 2, 2], [3, 5, 7, 9, 14, 17, 20, 23])]),
]


def main() -> None:
    out = Path(__file__).resolve().parent / "known_answers.json"
    out.write_text(json.dumps({"source": "olibartfast/nert test literals", "cases": CASES}, indent=1) + "\n")
    print(f"wrote {len(CASES)} cases to {out}")


if __name__ == "__main__":
    main()
