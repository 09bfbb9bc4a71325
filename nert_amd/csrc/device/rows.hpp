#pragma once
// Row declarations of the gfx950 kernel table. Every row has the reference
// KernelFn signature (include/nert/device.hpp:30-31).

#include "seam.hpp"

namespace nert_hip {
namespace rows {

using seam::Views;
using nert::Node;

#define NERT_HIP_ROW(name) void name(const Node& node, const Views& inputs, const Views& outputs)

// rows_gemm.cpp
NERT_HIP_ROW(Gemm);
NERT_HIP_ROW(MatMul);
NERT_HIP_ROW(Conv);
NERT_HIP_ROW(FusedConv); // not a reference row: the runner's Conv+Add+Relu fusion
NERT_HIP_ROW(FusedMatMul); // not a reference row: the runner's MatMul+scale+bias+Gelu fusion
NERT_HIP_ROW(FusedAddLayerNorm); // not a reference row: the runner's residual Add + LayerNormalization fusion
NERT_HIP_ROW(FusedAttention); // not a reference row: the runner's MatMul/Mul/Softmax/MatMul attention fusion

// Window helpers shared by Conv, ConvTranspose and the pools
// (src/kernels/conv.cpp:78-134, src/kernels/max_pool.cpp).
void ResolveWindowPads(const std::string& context, const std::string& auto_pad, const std::vector<int64_t>& in_spatial,
                       const std::vector<int64_t>& kernel, const std::vector<int64_t>& dilations,
                       const std::vector<int64_t>& strides, const std::vector<int64_t>& pads_attr,
                       std::vector<int64_t>& pad_begin, std::vector<int64_t>& pad_end);
int64_t WindowOutput(const std::string& context, int64_t in, int64_t kernel, int64_t dilation, int64_t pad_begin,
                     int64_t pad_end, int64_t stride, bool ceil_mode);

// rows_elementwise.cpp
NERT_HIP_ROW(Relu);
NERT_HIP_ROW(Sigmoid);
NERT_HIP_ROW(Tanh);
NERT_HIP_ROW(Exp);
NERT_HIP_ROW(Log);
NERT_HIP_ROW(Sqrt);
NERT_HIP_ROW(Sin);
NERT_HIP_ROW(Cos);
NERT_HIP_ROW(Floor);
NERT_HIP_ROW(Erf);
NERT_HIP_ROW(Abs);
NERT_HIP_ROW(Neg);
NERT_HIP_ROW(Sign);
NERT_HIP_ROW(Elu);
NERT_HIP_ROW(Clip);
NERT_HIP_ROW(IsNaN);
NERT_HIP_ROW(Not);
NERT_HIP_ROW(Add);
NERT_HIP_ROW(Sub);
NERT_HIP_ROW(Mul);
NERT_HIP_ROW(Div);
NERT_HIP_ROW(Pow);
NERT_HIP_ROW(Mod);
NERT_HIP_ROW(Max);
NERT_HIP_ROW(Min);
NERT_HIP_ROW(Equal);
NERT_HIP_ROW(Greater);
NERT_HIP_ROW(Less);
NERT_HIP_ROW(GreaterOrEqual);
NERT_HIP_ROW(LessOrEqual);
NERT_HIP_ROW(And);
NERT_HIP_ROW(Or);
NERT_HIP_ROW(Where);
NERT_HIP_ROW(Cast);

// rows_pool.cpp
NERT_HIP_ROW(MaxPool);
NERT_HIP_ROW(AveragePool);
NERT_HIP_ROW(GlobalAveragePool);

// rows_reduce.cpp
NERT_HIP_ROW(ReduceMean);
NERT_HIP_ROW(ReduceMax);
NERT_HIP_ROW(ReduceSum);
NERT_HIP_ROW(ReduceL2);
NERT_HIP_ROW(Softmax);
NERT_HIP_ROW(LayerNormalization);
NERT_HIP_ROW(InstanceNormalization);
NERT_HIP_ROW(ArgMax);
NERT_HIP_ROW(CumSum);

// rows_shape.cpp
NERT_HIP_ROW(Identity);
NERT_HIP_ROW(Flatten);
NERT_HIP_ROW(Reshape);

// rows_move.cpp
NERT_HIP_ROW(Transpose);
NERT_HIP_ROW(Concat);
NERT_HIP_ROW(Split);
NERT_HIP_ROW(Slice);
NERT_HIP_ROW(Expand);
NERT_HIP_ROW(Tile);
NERT_HIP_ROW(Squeeze);
NERT_HIP_ROW(Unsqueeze);
NERT_HIP_ROW(Pad);

// rows_index.cpp
NERT_HIP_ROW(Gather);
NERT_HIP_ROW(GatherElements);
NERT_HIP_ROW(ScatterND);
NERT_HIP_ROW(TopK);
NERT_HIP_ROW(Shape);
NERT_HIP_ROW(ConstantOfShape);
NERT_HIP_ROW(Range);
NERT_HIP_ROW(EyeLike);

// rows_contract.cpp
NERT_HIP_ROW(Resize);
NERT_HIP_ROW(GridSample);
NERT_HIP_ROW(Einsum);
NERT_HIP_ROW(ConvTranspose);

} // namespace rows
} // namespace nert_hip
