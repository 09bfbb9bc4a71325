// MaxPool, AveragePool and GlobalAveragePool rows; validation mirrors
// src/kernels/max_pool.cpp:138-205, average_pool.cpp:136-190 and
// global_average_pool.cpp:32-60.

#include "rows.hpp"

namespace nert_hip {
namespace rows {

using namespace seam;

NERT_HIP_ROW(MaxPool) {
    const std::string context = "MaxPool (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.empty()) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& x = inputs[0];
    const TensorView& out = outputs[0];
    if (x.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (x.dims.size() != 4) {
        throw InferenceException(context + ": input must be rank 4 (NCHW)");
    }
    (void)ElementCount(x.dims, context);
    (void)ElementCount(out.dims, context);
    const std::vector<int64_t> kernel = IntsAttr(node, "kernel_shape", "MaxPool");
    if (kernel.empty()) {
        throw InferenceException(context + ": kernel_shape is required");
    }
    if (kernel.size() != 2) {
        throw InferenceException(context + ": kernel_shape must have two spatial entries");
    }
    std::vector<int64_t> strides = IntsAttr(node, "strides", "MaxPool");
    std::vector<int64_t> dilations = IntsAttr(node, "dilations", "MaxPool");
    if (strides.empty()) {
        strides = {1, 1};
    }
    if (dilations.empty()) {
        dilations = {1, 1};
    }
    if (strides.size() != 2 || dilations.size() != 2) {
        throw InferenceException(context + ": stride and dilation must each have two spatial entries");
    }
    for (size_t i = 0; i < 2; ++i) {
        if (kernel[i] <= 0) {
            throw InferenceException(context + ": kernel dimensions must be positive");
        }
        if (strides[i] <= 0 || dilations[i] <= 0) {
            throw InferenceException(context + ": stride and dilation must be positive");
        }
    }
    const bool ceil_mode = IntAttr(node, "ceil_mode", 0, "MaxPool") != 0;
    const std::vector<int64_t> in_spatial = {x.dims[2], x.dims[3]};
    std::vector<int64_t> pad_begin;
    std::vector<int64_t> pad_end;
    ResolveWindowPads(context, StringAttr(node, "auto_pad", "NOTSET", "MaxPool"), in_spatial, kernel, dilations,
                      strides, IntsAttr(node, "pads", "MaxPool"), pad_begin, pad_end);
    const int64_t oh =
        WindowOutput(context, x.dims[2], kernel[0], dilations[0], pad_begin[0], pad_end[0], strides[0], ceil_mode);
    const int64_t ow =
        WindowOutput(context, x.dims[3], kernel[1], dilations[1], pad_begin[1], pad_end[1], strides[1], ceil_mode);
    if (out.dims != std::vector<int64_t>{x.dims[0], x.dims[1], oh, ow}) {
        throw InferenceException(context + ": output shape does not match the pooling window");
    }
    if (x.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    nert_pool_desc d{};
    d.batch = x.dims[0];
    d.channels = x.dims[1];
    d.in[0] = x.dims[2];
    d.in[1] = x.dims[3];
    d.out[0] = oh;
    d.out[1] = ow;
    for (int i = 0; i < 2; ++i) {
        d.kernel[i] = kernel[i];
        d.stride[i] = strides[i];
        d.dilation[i] = dilations[i];
        d.pad_begin[i] = pad_begin[i];
        d.pad_end[i] = pad_end[i];
    }
    CheckStatus(nert_hip_maxpool2d_f32(static_cast<const float*>(x.data), static_cast<float*>(out.data), &d, Stream()),
                context);
    AfterRow(Views{out}, context);
}

NERT_HIP_ROW(AveragePool) {
    const std::string context = "AveragePool (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& x = inputs[0];
    const TensorView& out = outputs[0];
    if (x.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (x.dims.size() != 4) {
        throw InferenceException(context + ": input must be rank 4 (NCHW)");
    }
    (void)ElementCount(x.dims, context);
    (void)ElementCount(out.dims, context);
    const std::vector<int64_t> kernel = IntsAttr(node, "kernel_shape", "AveragePool");
    if (kernel.size() != 2) {
        throw InferenceException(context + ": kernel_shape must have two spatial entries");
    }
    std::vector<int64_t> strides = IntsAttr(node, "strides", "AveragePool");
    if (strides.empty()) {
        strides = {1, 1};
    }
    if (strides.size() != 2) {
        throw InferenceException(context + ": strides must have two spatial entries");
    }
    for (size_t i = 0; i < 2; ++i) {
        if (kernel[i] <= 0 || strides[i] <= 0) {
            throw InferenceException(context + ": kernel and stride must be positive");
        }
    }
    const std::vector<int64_t> dilations = {1, 1};
    const bool ceil_mode = IntAttr(node, "ceil_mode", 0, "AveragePool") != 0;
    const bool include_pad = IntAttr(node, "count_include_pad", 0, "AveragePool") != 0;
    const std::vector<int64_t> in_spatial = {x.dims[2], x.dims[3]};
    std::vector<int64_t> pad_begin;
    std::vector<int64_t> pad_end;
    ResolveWindowPads(context, StringAttr(node, "auto_pad", "NOTSET", "AveragePool"), in_spatial, kernel, dilations,
                      strides, IntsAttr(node, "pads", "AveragePool"), pad_begin, pad_end);
    const int64_t oh = WindowOutput(context, x.dims[2], kernel[0], 1, pad_begin[0], pad_end[0], strides[0], ceil_mode);
    const int64_t ow = WindowOutput(context, x.dims[3], kernel[1], 1, pad_begin[1], pad_end[1], strides[1], ceil_mode);
    if (out.dims != std::vector<int64_t>{x.dims[0], x.dims[1], oh, ow}) {
        throw InferenceException(context + ": output shape does not match the pooling window");
    }
    if (x.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    nert_pool_desc d{};
    d.batch = x.dims[0];
    d.channels = x.dims[1];
    d.in[0] = x.dims[2];
    d.in[1] = x.dims[3];
    d.out[0] = oh;
    d.out[1] = ow;
    for (int i = 0; i < 2; ++i) {
        d.kernel[i] = kernel[i];
        d.stride[i] = strides[i];
        d.dilation[i] = 1;
        d.pad_begin[i] = pad_begin[i];
        d.pad_end[i] = pad_end[i];
    }
    d.count_include_pad = include_pad ? 1 : 0;
    CheckStatus(nert_hip_avgpool2d_f32(static_cast<const float*>(x.data), static_cast<float*>(out.data), &d, Stream()),
                context);
    AfterRow(outputs, context);
}

NERT_HIP_ROW(GlobalAveragePool) {
    const std::string context = "GlobalAveragePool (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& x = inputs[0];
    const TensorView& out = outputs[0];
    if (x.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (x.dims.size() < 2) {
        throw InferenceException(context + ": input must have batch and channel axes (rank at least 2)");
    }
    (void)ElementCount(x.dims, context);
    (void)ElementCount(out.dims, context);
    std::vector<int64_t> expected = {x.dims[0], x.dims[1]};
    expected.insert(expected.end(), x.dims.size() - 2, 1);
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape must be the input shape with all spatial axes at 1");
    }
    // The reference reads the buffers without a null check; a null view here
    // would fault on the device, so it is rejected instead.
    if (x.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    int64_t spatial = 1;
    for (size_t i = 2; i < x.dims.size(); ++i) {
        spatial *= x.dims[i];
    }
    CheckStatus(nert_hip_global_avgpool_f32(static_cast<const float*>(x.data), static_cast<float*>(out.data),
                                            x.dims[0] * x.dims[1], spatial, Stream()),
                context);
    AfterRow(outputs, context);
}

} // namespace rows
} // namespace nert_hip
