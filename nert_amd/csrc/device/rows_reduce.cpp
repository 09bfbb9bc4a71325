// Reduction rows: ReduceMean/ReduceMax/ReduceSum/ReduceL2, Softmax,
// LayerNormalization, InstanceNormalization, ArgMax, CumSum.
//
// The schema-dependent forms come from the reference's own header-only
// resolvers (src/reduce_axes.hpp, src/axes_form.hpp, src/softmax_form.hpp),
// so an opset-17 ReduceMean reads its `axes` attribute and an opset-18 one its
// input exactly as the CPU rows do. Validation order and messages follow
// src/kernels/{reduce_mean,reduce_max,reduce_sum,reduce_l2,softmax,
// layer_normalization,instance_normalization,arg_max,cum_sum}.cpp.

#include "rows.hpp"

#include "axes_form.hpp"
#include "reduce_axes.hpp"
#include "softmax_form.hpp"

namespace nert_hip {
namespace rows {

using namespace seam;

namespace {

int64_t CtxInt(const Node& node, const std::string& name, int64_t fallback, const std::string& context) {
    const Attribute* attr = FindAttr(node, name);
    if (attr == nullptr) {
        return fallback;
    }
    const int64_t* v = std::get_if<int64_t>(&attr->value);
    if (v == nullptr) {
        throw InferenceException(context + ": attribute '" + name + "' must be an integer");
    }
    return *v;
}

// Marks the reduced axes; returns the expected output dims.
std::vector<int64_t> MarkAxes(const std::vector<int64_t>& axes, const std::vector<int64_t>& in_dims, bool keepdims,
                              std::vector<uint8_t>& reduced, const std::string& context) {
    const int64_t rank = static_cast<int64_t>(in_dims.size());
    reduced.assign(static_cast<size_t>(rank), 0);
    for (int64_t axis : axes) {
        if (axis < -rank || axis >= rank) {
            throw InferenceException(context + ": axis out of range");
        }
        const int64_t normalized = axis < 0 ? axis + rank : axis;
        if (reduced[static_cast<size_t>(normalized)]) {
            throw InferenceException(context + ": duplicate axis");
        }
        reduced[static_cast<size_t>(normalized)] = 1;
    }
    std::vector<int64_t> expected;
    for (int64_t i = 0; i < rank; ++i) {
        if (reduced[static_cast<size_t>(i)]) {
            if (keepdims) {
                expected.push_back(1);
            }
        } else {
            expected.push_back(in_dims[static_cast<size_t>(i)]);
        }
    }
    return expected;
}

std::vector<int64_t> AllAxes(int64_t rank) {
    std::vector<int64_t> axes;
    for (int64_t i = 0; i < rank; ++i) {
        axes.push_back(i);
    }
    return axes;
}

// Axes of the ReduceMean/ReduceL2/ReduceMax family (src/reduce_axes.hpp).
// Returns true for the noop identity (only when `allow_noop`).
bool ReduceAxesOf(const Node& node, const Views& inputs, int64_t rank, bool allow_noop, std::vector<int64_t>& axes,
                  const std::string& context) {
    const nert::ReduceAxes resolved = nert::ResolveReduceAxes(node);
    if (resolved.form == nert::ReduceAxesForm::Attribute) {
        if (resolved.axes_attribute != nullptr) {
            const std::vector<int64_t>* values = nert::ReduceAttributeIntList(resolved.axes_attribute);
            if (values == nullptr) {
                throw InferenceException(context + ": attribute 'axes' must be an integer list");
            }
            axes = *values;
        }
        if (axes.empty()) {
            axes = AllAxes(rank);
        }
        return false;
    }
    bool supplied = false;
    if (inputs.size() == 2 && inputs[1].dtype != DataType::Unknown) {
        supplied = true;
        const TensorView& av = inputs[1];
        if (av.dtype != DataType::Int64) {
            throw InferenceException(context + ": axes tensor must be int64");
        }
        const int64_t count = nert::ReduceAxesElementCount(av.dims, context);
        if (count > 0 && av.data == nullptr) {
            throw InferenceException(context + ": null axes buffer");
        }
        if (count > 0) {
            axes = ReadInt64(av, count, context);
        }
    }
    if (axes.empty()) {
        if (allow_noop && supplied && resolved.noop_with_empty_axes) {
            return true;
        }
        axes = AllAxes(rank);
    }
    return false;
}

void Launch(int op, int dtype, const TensorView& in, const TensorView& out, const std::vector<uint8_t>& reduced,
            const std::string& context) {
    CheckStatus(nert_hip_reduce(op, dtype, in.data, out.data, static_cast<int>(in.dims.size()), in.dims.data(),
                                reduced.data(), Stream()),
                context);
}

void Copy(const TensorView& in, const TensorView& out, const std::string& context) {
    const int64_t bytes = Count(in.dims) * ElementSize(in.dtype);
    if (bytes > 0 && in.data != out.data) {
        CheckStatus(nert_hip_memcpy_d2d(out.data, in.data, bytes, Stream()), context);
    }
}

} // namespace

// src/kernels/reduce_mean.cpp:44-195
NERT_HIP_ROW(ReduceMean) {
    const std::string context = "ReduceMean (node '" + node.name + "')";
    if (inputs.empty() || inputs.size() > 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one or two inputs and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": data tensors must be float32");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    (void)ElementCount(in.dims, context);
    if (in.data == nullptr) {
        throw InferenceException(context + ": null input buffer");
    }
    const int64_t keepdims = IntAttr(node, "keepdims", 1, "ReduceMean");
    std::vector<int64_t> axes;
    const bool identity = ReduceAxesOf(node, inputs, rank, true, axes, context);
    if (out.data == nullptr) {
        throw InferenceException(context + ": null output buffer");
    }
    if (identity) {
        if (out.dims != in.dims) {
            throw InferenceException(context + ": output shape does not match the input");
        }
        (void)ElementCount(out.dims, context);
        Copy(in, out, context);
        AfterRow(outputs, context);
        return;
    }
    std::vector<uint8_t> reduced;
    if (out.dims != MarkAxes(axes, in.dims, keepdims != 0, reduced, context)) {
        throw InferenceException(context + ": output shape does not match the reduced axes");
    }
    (void)ElementCount(out.dims, context);
    Launch(NERT_RED_MEAN, NERT_F32, in, out, reduced, context);
    AfterRow(outputs, context);
}

// src/kernels/reduce_max.cpp:46-166
NERT_HIP_ROW(ReduceMax) {
    const std::string context = "ReduceMax (node '" + node.name + "')";
    if (inputs.empty() || inputs.size() > 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one or two inputs and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": data tensors must be float32");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    (void)ElementCount(in.dims, context);
    if (in.data == nullptr) {
        throw InferenceException(context + ": null input buffer");
    }
    const int64_t keepdims = CtxInt(node, "keepdims", 1, context);
    std::vector<int64_t> axes;
    (void)ReduceAxesOf(node, inputs, rank, false, axes, context);
    std::vector<uint8_t> reduced;
    if (out.dims != MarkAxes(axes, in.dims, keepdims != 0, reduced, context)) {
        throw InferenceException(context + ": output shape does not match the reduced axes");
    }
    (void)ElementCount(out.dims, context);
    if (out.data == nullptr) {
        throw InferenceException(context + ": null output buffer");
    }
    Launch(NERT_RED_MAX, NERT_F32, in, out, reduced, context);
    AfterRow(outputs, context);
}

// src/kernels/reduce_l2.cpp:84-195
NERT_HIP_ROW(ReduceL2) {
    const std::string context = "ReduceL2 (node '" + node.name + "')";
    if (inputs.empty() || inputs.size() > 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one or two inputs and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": data tensors must be float32");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    (void)ElementCount(in.dims, context);
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    const bool keepdims = IntAttr(node, "keepdims", 1, "ReduceL2") != 0;
    std::vector<int64_t> axes;
    const bool identity = ReduceAxesOf(node, inputs, rank, true, axes, context);
    if (identity) {
        if (out.dims != in.dims) {
            throw InferenceException(context + ": output shape does not match the input");
        }
        Copy(in, out, context);
        AfterRow(outputs, context);
        return;
    }
    std::vector<uint8_t> reduced;
    if (out.dims != MarkAxes(axes, in.dims, keepdims, reduced, context)) {
        throw InferenceException(context + ": output shape does not match the reduced axes");
    }
    Launch(NERT_RED_L2, NERT_F32, in, out, reduced, context);
    AfterRow(outputs, context);
}

// src/kernels/reduce_sum.cpp:74-184 (axes from src/axes_form.hpp)
NERT_HIP_ROW(ReduceSum) {
    const std::string context = "ReduceSum (node '" + node.name + "')";
    if (inputs.empty() || inputs.size() > 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one or two inputs and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if ((in.dtype != DataType::Float32 && in.dtype != DataType::Int64) || out.dtype != in.dtype) {
        throw InferenceException(context + ": data tensors must share dtype float32 or int64");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    (void)ElementCount(in.dims, context);
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    const bool keepdims = CtxInt(node, "keepdims", 1, context) != 0;
    const bool noop_empty = CtxInt(node, "noop_with_empty_axes", 0, context) != 0;
    const nert::AxesForm form = nert::ResolveAxesForm(node);
    std::vector<int64_t> axes;
    if (form.source == nert::AxesSource::Attribute) {
        if (form.axes_attribute != nullptr) {
            const std::vector<int64_t>* values = nert::NodeAttributeIntList(form.axes_attribute);
            if (values == nullptr) {
                throw InferenceException(context + ": attribute 'axes' must be an integer list");
            }
            axes = *values;
        }
    } else if (inputs.size() == 2 && inputs[1].dtype != DataType::Unknown) {
        const TensorView& av = inputs[1];
        if (av.dtype != DataType::Int64) {
            throw InferenceException(context + ": axes tensor must be int64");
        }
        const int64_t count = nert::AxesElementCount(av.dims, context);
        if (count > 0) {
            if (av.data == nullptr) {
                throw InferenceException(context + ": null axes buffer");
            }
            axes = ReadInt64(av, count, context);
        }
    }
    if (axes.empty()) {
        if (noop_empty) {
            if (out.dims != in.dims) {
                throw InferenceException(context + ": output shape does not match the input");
            }
            Copy(in, out, context);
            AfterRow(outputs, context);
            return;
        }
        axes = AllAxes(rank);
    }
    std::vector<uint8_t> reduced;
    if (out.dims != MarkAxes(axes, in.dims, keepdims, reduced, context)) {
        throw InferenceException(context + ": output shape does not match the reduced axes");
    }
    (void)ElementCount(out.dims, context);
    Launch(NERT_RED_SUM, DtypeCode(in.dtype), in, out, reduced, context);
    AfterRow(outputs, context);
}

// src/kernels/softmax.cpp:47-96 with src/softmax_form.hpp
NERT_HIP_ROW(Softmax) {
    const std::string context = "Softmax (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (in.dims != out.dims) {
        throw InferenceException(context + ": output shape must match the input shape");
    }
    (void)ElementCount(out.dims, context);
    (void)ElementCount(in.dims, context);
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    const nert::SoftmaxForm form = nert::ResolveSoftmaxForm(node);
    int64_t axis = nert::SoftmaxAxis(node, form, context);
    if (axis < -rank || axis >= rank) {
        throw InferenceException(context + ": axis out of range");
    }
    if (axis < 0) {
        axis += rank;
    }
    int64_t outer = 1;
    for (int64_t i = 0; i < axis; ++i) {
        outer *= in.dims[static_cast<size_t>(i)];
    }
    int64_t dim = rank == 0 ? 1 : in.dims[static_cast<size_t>(axis)];
    int64_t inner = 1;
    if (form == nert::SoftmaxForm::LegacyCoerce2D) {
        dim = 1;
        for (int64_t i = axis; i < rank; ++i) {
            dim *= in.dims[static_cast<size_t>(i)];
        }
    } else {
        for (int64_t i = axis + 1; i < rank; ++i) {
            inner *= in.dims[static_cast<size_t>(i)];
        }
    }
    CheckStatus(nert_hip_softmax_f32(static_cast<const float*>(in.data), static_cast<float*>(out.data), outer, dim,
                                     inner, Stream()),
                context);
    AfterRow(outputs, context);
}

namespace {
const float* NormParam(const TensorView& view, int64_t inner, int& scalar, const std::string& context,
                       const char* what) {
    if (view.dtype != DataType::Float32 || view.data == nullptr) {
        throw InferenceException(context + ": " + what + " must be a float32 tensor");
    }
    const int64_t count = ElementCount(view.dims, context);
    if (count != inner && count != 1) {
        throw InferenceException(context + ": " + what + " must have one value per normalized element");
    }
    scalar = count == 1 ? 1 : 0;
    return static_cast<const float*>(view.data);
}
} // namespace

// src/kernels/layer_normalization.cpp:77-131
NERT_HIP_ROW(LayerNormalization) {
    const std::string context = "LayerNormalization (node '" + node.name + "')";
    if (inputs.size() < 2 || inputs.size() > 3 || outputs.empty() || outputs.size() > 3) {
        throw InferenceException(context + ": expected X, Scale, optional B, and one to three outputs");
    }
    const TensorView& x = inputs[0];
    const TensorView& y = outputs[0];
    if (x.dtype != DataType::Float32 || y.dtype != DataType::Float32) {
        throw InferenceException(context + ": X and Y must be float32");
    }
    if (x.dims.empty() || x.dims != y.dims) {
        throw InferenceException(context + ": Y must have the shape of a non-scalar X");
    }
    const int64_t rank = static_cast<int64_t>(x.dims.size());
    int64_t axis = IntAttr(node, "axis", -1, "LayerNormalization");
    if (axis < 0) {
        axis += rank;
    }
    if (axis < 0 || axis >= rank) {
        throw InferenceException(context + ": axis is out of range");
    }
    const float epsilon = FloatAttr(node, "epsilon", 1e-5f, "LayerNormalization");
    int64_t outer = 1;
    int64_t inner = 1;
    for (int64_t i = 0; i < rank; ++i) {
        (i < axis ? outer : inner) *= x.dims[static_cast<size_t>(i)];
    }
    (void)ElementCount(x.dims, context);
    if (x.data == nullptr || y.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    int scale_scalar = 0;
    const float* scale = NormParam(inputs[1], inner, scale_scalar, context, "Scale");
    int bias_scalar = 0;
    const float* bias = nullptr;
    if (inputs.size() == 3 && inputs[2].dtype != DataType::Unknown) {
        bias = NormParam(inputs[2], inner, bias_scalar, context, "B");
    }
    float* mean_out = nullptr;
    float* invstd_out = nullptr;
    for (size_t o = 1; o < outputs.size(); ++o) {
        if (outputs[o].dtype == DataType::Unknown) {
            continue;
        }
        if (outputs[o].dtype != DataType::Float32 || outputs[o].data == nullptr ||
            ElementCount(outputs[o].dims, context) != outer) {
            throw InferenceException(context + ": Mean and InvStdDev must be float32 with one value per row");
        }
        (o == 1 ? mean_out : invstd_out) = static_cast<float*>(outputs[o].data);
    }
    CheckStatus(nert_hip_layernorm_f32(static_cast<const float*>(x.data), scale, scale_scalar, bias, bias_scalar,
                                       static_cast<float*>(y.data), mean_out, invstd_out, outer, inner,
                                       static_cast<double>(epsilon), Stream()),
                context);
    AfterRow(outputs, context);
}

// Not a reference row: the runner's fusion of a residual Add whose output
// feeds a LayerNormalization over its trailing axes (pre-LN transformer
// blocks). Inputs A, B (same shape), Scale, optional B of the norm; outputs
// the sum (still read by later rows) and the normalised tensor. Equal bit for
// bit to the Add row followed by the LayerNormalization row.
NERT_HIP_ROW(FusedAddLayerNorm) {
    const std::string context = "FusedAddLayerNorm (node '" + node.name + "')";
    if (inputs.size() < 3 || inputs.size() > 4 || outputs.size() != 2) {
        throw InferenceException(context + ": expected A, B, Scale, optional bias, and two outputs");
    }
    const TensorView& a = inputs[0];
    const TensorView& b = inputs[1];
    const TensorView& sum = outputs[0];
    const TensorView& y = outputs[1];
    for (const TensorView* t : {&a, &b, &sum, &y}) {
        if (t->dtype != DataType::Float32) {
            throw InferenceException(context + ": tensors must be float32");
        }
        if (t->dims != a.dims) {
            throw InferenceException(context + ": A, B and both outputs must share one shape");
        }
    }
    if (a.dims.empty()) {
        throw InferenceException(context + ": tensors must not be scalars");
    }
    const int64_t rank = static_cast<int64_t>(a.dims.size());
    int64_t axis = IntAttr(node, "axis", -1, "FusedAddLayerNorm");
    if (axis < 0) {
        axis += rank;
    }
    if (axis < 0 || axis >= rank) {
        throw InferenceException(context + ": axis is out of range");
    }
    const float epsilon = FloatAttr(node, "epsilon", 1e-5f, "FusedAddLayerNorm");
    int64_t outer = 1;
    int64_t inner = 1;
    for (int64_t i = 0; i < rank; ++i) {
        (i < axis ? outer : inner) *= a.dims[static_cast<size_t>(i)];
    }
    (void)ElementCount(a.dims, context);
    if (a.data == nullptr || b.data == nullptr || sum.data == nullptr || y.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    int scale_scalar = 0;
    const float* scale = NormParam(inputs[2], inner, scale_scalar, context, "Scale");
    int bias_scalar = 0;
    const float* bias = nullptr;
    if (inputs.size() == 4 && inputs[3].dtype != DataType::Unknown) {
        bias = NormParam(inputs[3], inner, bias_scalar, context, "B");
    }
    if (scale_scalar || bias_scalar) {
        throw InferenceException(context + ": Scale and B must have one value per normalised element");
    }
    CheckStatus(nert_hip_add_layernorm_f32(static_cast<const float*>(a.data), static_cast<const float*>(b.data), scale,
                                           bias, static_cast<float*>(sum.data), static_cast<float*>(y.data), outer,
                                           inner, static_cast<double>(epsilon), Stream()),
                context);
    AfterRow(outputs, context);
}

// src/kernels/instance_normalization.cpp:44-80
NERT_HIP_ROW(InstanceNormalization) {
    const std::string context = "InstanceNormalization (node '" + node.name + "')";
    if (inputs.size() != 3 || outputs.size() != 1) {
        throw InferenceException(context + ": expected input, scale, B, and one output");
    }
    const TensorView& x = inputs[0];
    const TensorView& y = outputs[0];
    if (x.dtype != DataType::Float32 || y.dtype != DataType::Float32) {
        throw InferenceException(context + ": input and output must be float32");
    }
    if (x.dims.size() < 2 || x.dims != y.dims) {
        throw InferenceException(context + ": output must have the shape of an input of rank >= 2");
    }
    for (int64_t dim : x.dims) {
        if (dim <= 0) {
            throw InferenceException(context + ": non-positive dimension");
        }
    }
    if (x.data == nullptr || y.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    const int64_t batch = x.dims[0];
    const int64_t channels = x.dims[1];
    int64_t spatial = 1;
    for (size_t i = 2; i < x.dims.size(); ++i) {
        spatial *= x.dims[i];
    }
    auto channel_param = [&](const TensorView& view, const char* what) {
        if (view.dtype != DataType::Float32 || view.data == nullptr) {
            throw InferenceException(context + ": " + what + " must be a float32 tensor");
        }
        if (view.dims.size() != 1 || view.dims[0] != channels) {
            throw InferenceException(context + ": " + what + " must be rank-1 with one value per channel");
        }
        return static_cast<const float*>(view.data);
    };
    const float* scale = channel_param(inputs[1], "scale");
    const float* bias = channel_param(inputs[2], "B");
    const float epsilon = FloatAttr(node, "epsilon", 1e-5f, "InstanceNormalization");
    CheckStatus(nert_hip_instancenorm_f32(static_cast<const float*>(x.data), scale, bias, static_cast<float*>(y.data),
                                          batch, channels, spatial, static_cast<double>(epsilon), Stream()),
                context);
    AfterRow(outputs, context);
}

// src/kernels/arg_max.cpp:58-123
NERT_HIP_ROW(ArgMax) {
    const std::string context = "ArgMax (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 && in.dtype != DataType::Int64) {
        throw InferenceException(context + ": input must be float32 or int64");
    }
    if (out.dtype != DataType::Int64) {
        throw InferenceException(context + ": output must be int64");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    if (rank == 0) {
        throw InferenceException(context + ": input must have rank >= 1");
    }
    int64_t axis = CtxInt(node, "axis", 0, context);
    if (axis < -rank || axis >= rank) {
        throw InferenceException(context + ": axis out of range");
    }
    if (axis < 0) {
        axis += rank;
    }
    const int64_t keepdims = CtxInt(node, "keepdims", 1, context);
    if (keepdims != 0 && keepdims != 1) {
        throw InferenceException(context + ": keepdims must be 0 or 1 here");
    }
    const int64_t last = CtxInt(node, "select_last_index", 0, context);
    if (last != 0 && last != 1) {
        throw InferenceException(context + ": select_last_index must be 0 or 1 here");
    }
    const int64_t dim = in.dims[static_cast<size_t>(axis)];
    std::vector<int64_t> expected = in.dims;
    if (keepdims != 0) {
        expected[static_cast<size_t>(axis)] = 1;
    } else {
        expected.erase(expected.begin() + axis);
    }
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the reduced axis");
    }
    (void)ElementCount(in.dims, context);
    const int64_t out_count = ElementCount(out.dims, context);
    if (out_count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    int64_t outer = 1;
    for (int64_t i = 0; i < axis; ++i) {
        outer *= in.dims[static_cast<size_t>(i)];
    }
    int64_t inner = 1;
    for (int64_t i = axis + 1; i < rank; ++i) {
        inner *= in.dims[static_cast<size_t>(i)];
    }
    CheckStatus(nert_hip_argmax(DtypeCode(in.dtype), in.data, static_cast<int64_t*>(out.data), outer, dim, inner,
                                static_cast<int>(last), Stream()),
                context);
    AfterRow(outputs, context);
}

// src/kernels/cum_sum.cpp:75-145
NERT_HIP_ROW(CumSum) {
    const std::string context = "CumSum (node '" + node.name + "')";
    if (inputs.size() != 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected a data input, an axis input, and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& axis_view = inputs[1];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 && in.dtype != DataType::Int64) {
        throw InferenceException(context + ": input must be float32 or int64");
    }
    if (out.dtype != in.dtype) {
        throw InferenceException(context + ": output must share the input dtype");
    }
    if (axis_view.dtype != DataType::Int64) {
        throw InferenceException(context + ": axis input must be int64");
    }
    if (ElementCount(axis_view.dims, context) != 1) {
        throw InferenceException(context + ": axis input must be a scalar");
    }
    if (axis_view.data == nullptr) {
        throw InferenceException(context + ": null axis buffer");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    if (rank == 0) {
        throw InferenceException(context + ": input must have rank >= 1");
    }
    int64_t axis = ReadInt64(axis_view, 1, context)[0];
    if (axis < -rank || axis >= rank) {
        throw InferenceException(context + ": axis out of range");
    }
    if (axis < 0) {
        axis += rank;
    }
    const int64_t exclusive = CtxInt(node, "exclusive", 0, context);
    if (exclusive != 0 && exclusive != 1) {
        throw InferenceException(context + ": exclusive must be 0 or 1 here");
    }
    const int64_t reverse = CtxInt(node, "reverse", 0, context);
    if (reverse != 0 && reverse != 1) {
        throw InferenceException(context + ": reverse must be 0 or 1 here");
    }
    if (out.dims != in.dims) {
        throw InferenceException(context + ": output shape must match the input");
    }
    const int64_t out_count = ElementCount(out.dims, context);
    if (out_count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    int64_t outer = 1;
    for (int64_t i = 0; i < axis; ++i) {
        outer *= in.dims[static_cast<size_t>(i)];
    }
    int64_t inner = 1;
    for (int64_t i = axis + 1; i < rank; ++i) {
        inner *= in.dims[static_cast<size_t>(i)];
    }
    CheckStatus(nert_hip_cumsum(DtypeCode(in.dtype), in.data, out.data, outer, in.dims[static_cast<size_t>(axis)],
                                inner, static_cast<int>(exclusive), static_cast<int>(reverse), Stream()),
                context);
    AfterRow(outputs, context);
}

} // namespace rows
} // namespace nert_hip
