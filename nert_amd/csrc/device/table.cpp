// The gfx950 kernel table and the node-level C entry points.
//
// Exact op-type strings map to rows; unknown types resolve to null so the
// executor rejects the node naming op and node (src/executor.cpp:485-488), as
// with the CPU table (src/kernels/cpu_kernels.cpp:15-93). The seam's
// KernelTable::find answers for exactly the reference's 73 op types
// (src/hip/table.cpp:95-173); the fused rows that this library's own runner
// emits (FusedConv, FusedMatMul, FusedAddLayerNorm, FusedAttention) are
// reachable only through the node-level C entry points.

#include "rows.hpp"
#include "../../../include/nert_abi_node.hpp"

#include <unordered_map>

namespace nert_hip {

nert::KernelFn FindRow(const std::string& op_type) {
    using namespace rows;
    static const std::unordered_map<std::string, nert::KernelFn> table = {
        {"Gemm", &Gemm},
        {"MatMul", &MatMul},
        {"Conv", &Conv},
        {"Relu", &Relu},
        {"Sigmoid", &Sigmoid},
        {"Tanh", &Tanh},
        {"Exp", &Exp},
        {"Log", &Log},
        {"Sqrt", &Sqrt},
        {"Sin", &Sin},
        {"Cos", &Cos},
        {"Floor", &Floor},
        {"Erf", &Erf},
        {"Abs", &Abs},
        {"Neg", &Neg},
        {"Sign", &Sign},
        {"Elu", &Elu},
        {"Clip", &Clip},
        {"IsNaN", &IsNaN},
        {"Not", &Not},
        {"Add", &Add},
        {"Sub", &Sub},
        {"Mul", &Mul},
        {"Div", &Div},
        {"Pow", &Pow},
        {"Mod", &Mod},
        {"Max", &Max},
        {"Min", &Min},
        {"Equal", &Equal},
        {"Greater", &Greater},
        {"Less", &Less},
        {"GreaterOrEqual", &GreaterOrEqual},
        {"LessOrEqual", &LessOrEqual},
        {"And", &And},
        {"Or", &Or},
        {"Where", &Where},
        {"Cast", &Cast},
        {"MaxPool", &MaxPool},
        {"AveragePool", &AveragePool},
        {"GlobalAveragePool", &GlobalAveragePool},
        {"ReduceMean", &ReduceMean},
        {"ReduceMax", &ReduceMax},
        {"ReduceSum", &ReduceSum},
        {"ReduceL2", &ReduceL2},
        {"Softmax", &Softmax},
        {"LayerNormalization", &LayerNormalization},
        {"InstanceNormalization", &InstanceNormalization},
        {"ArgMax", &ArgMax},
        {"CumSum", &CumSum},
        {"Identity", &Identity},
        {"Flatten", &Flatten},
        {"Reshape", &Reshape},
        {"Transpose", &Transpose},
        {"Concat", &Concat},
        {"Split", &Split},
        {"Slice", &Slice},
        {"Expand", &Expand},
        {"Tile", &Tile},
        {"Squeeze", &Squeeze},
        {"Unsqueeze", &Unsqueeze},
        {"Pad", &Pad},
        {"Gather", &Gather},
        {"GatherElements", &GatherElements},
        {"ScatterND", &ScatterND},
        {"TopK", &TopK},
        {"Shape", &Shape},
        {"ConstantOfShape", &ConstantOfShape},
        {"Range", &Range},
        {"EyeLike", &EyeLike},
        {"Resize", &Resize},
        {"GridSample", &GridSample},
        {"Einsum", &Einsum},
        {"ConvTranspose", &ConvTranspose},
    };
    const auto it = table.find(op_type);
    return it == table.end() ? nullptr : it->second;
}

nert::KernelFn FindRunnerRow(const std::string& op_type) {
    using namespace rows;
    static const std::unordered_map<std::string, nert::KernelFn> fused = {
        {"FusedConv", &FusedConv},
        {"FusedMatMul", &FusedMatMul},
        {"FusedAddLayerNorm", &FusedAddLayerNorm},
        {"FusedAttention", &FusedAttention},
    };
    const auto it = fused.find(op_type);
    return it == fused.end() ? FindRow(op_type) : it->second;
}

} // namespace nert_hip

extern "C" {

int nert_hip_run_node(const char* op_type, const char* node_name, int64_t schema_version, const nert_attr_desc* attrs,
                      int n_attrs, const nert_tensor_desc* inputs, int n_inputs, const nert_tensor_desc* outputs,
                      int n_outputs, char* err, int err_len) {
    try {
        (void)nert::HipDevice(); // device set-up; throws when no GPU is usable
        return nert_abi::RunFoundRow(&nert_hip::FindRunnerRow, op_type, node_name, schema_version, attrs, n_attrs,
                                     inputs, n_inputs, outputs, n_outputs, err, err_len);
    } catch (const std::exception& e) {
        nert_abi::CopyMessage(e.what(), err, err_len);
        return NERT_OTHER_ERROR;
    }
}

int nert_hip_has_row(const char* op_type) {
    return nert_hip::FindRunnerRow(op_type != nullptr ? op_type : "") != nullptr ? 1 : 0;
}

} // extern "C"
