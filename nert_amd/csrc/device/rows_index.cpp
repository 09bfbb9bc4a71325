// Index and generator rows: Gather, GatherElements, ScatterND, TopK, Shape,
// ConstantOfShape, Range, EyeLike. Validation mirrors
// src/kernels/{gather,gather_elements,scatter_nd,top_k,shape,
// constant_of_shape,range,eye_like}.cpp.
//
// Out-of-range indices throw like the reference. When the indices are in the
// host shadow (initializers, small uploads) they are checked on the host
// before launch; otherwise the kernel raises the device index flag and the
// row waits for it (deferred while the stream is being captured).

#include "rows.hpp"

#include <algorithm>
#include <cmath>

namespace nert_hip {
namespace rows {

using namespace seam;

namespace {

const char* kMovable = ": tensors must be float32, int64, or bool";

int64_t Wrap(int64_t k, int64_t dim) { return k < 0 ? k + dim : k; }

} // namespace

// src/kernels/gather.cpp:49-129
NERT_HIP_ROW(Gather) {
    const std::string context = "Gather (node '" + node.name + "')";
    if (inputs.size() != 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected data and indices inputs and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& indices = inputs[1];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 && in.dtype != DataType::Int64 && in.dtype != DataType::Bool) {
        throw InferenceException(context + kMovable);
    }
    if (out.dtype != in.dtype) {
        throw InferenceException(context + ": output dtype must match the input dtype");
    }
    if (indices.dtype != DataType::Int64) {
        throw InferenceException(context + ": Gather indices must be int64");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    if (rank == 0) {
        throw InferenceException(context + ": Gather axis is out of range");
    }
    int64_t axis = IntAttrC(node, "axis", 0, context);
    if (axis < -rank || axis >= rank) {
        throw InferenceException(context + ": Gather axis is out of range");
    }
    if (axis < 0) {
        axis += rank;
    }
    std::vector<int64_t> expected(in.dims.begin(), in.dims.begin() + axis);
    expected.insert(expected.end(), indices.dims.begin(), indices.dims.end());
    expected.insert(expected.end(), in.dims.begin() + axis + 1, in.dims.end());
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the gathered indices");
    }
    const int64_t index_count = CountNonNeg(indices.dims, context);
    const int64_t out_count = CountNonNeg(out.dims, context);
    (void)CountNonNeg(in.dims, context);
    if (index_count > 0 && indices.data == nullptr) {
        throw InferenceException(context + ": null indices buffer");
    }
    if (out_count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    int64_t outer = 1;
    for (int64_t i = 0; i < axis; ++i) {
        outer *= in.dims[static_cast<size_t>(i)];
    }
    const int64_t dim = in.dims[static_cast<size_t>(axis)];
    int64_t inner = 1;
    for (int64_t i = axis + 1; i < rank; ++i) {
        inner *= in.dims[static_cast<size_t>(i)];
    }
    // The reference checks each index once per outer slice, so nothing is
    // checked when outer == 0.
    const bool checked = outer > 0 && index_count > 0;
    std::vector<int64_t> host;
    const bool on_host = checked && (out_count == 0 || HostShadowInt64(indices, index_count, host));
    if (on_host) {
        if (host.empty()) {
            host = ReadInt64(indices, index_count, context);
        }
        for (const int64_t k : host) {
            const int64_t w = Wrap(k, dim);
            if (w < 0 || w >= dim) {
                throw InferenceException(context + ": Gather index is out of range");
            }
        }
    }
    if (out_count > 0) {
        CheckStatus(nert_hip_gather(static_cast<int>(ElementSize(in.dtype)), in.data,
                                    static_cast<const int64_t*>(indices.data), out.data, outer, dim, index_count,
                                    inner, Stream()),
                    context);
    }
    AfterRow(outputs, context);
    if (checked && !on_host) {
        ThrowOnDeviceFlag(context, "Gather index is out of range");
    }
}

// src/kernels/gather_elements.cpp:73-131
NERT_HIP_ROW(GatherElements) {
    const std::string context = "GatherElements (node '" + node.name + "')";
    if (inputs.size() != 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected data and indices inputs and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& indices = inputs[1];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 && in.dtype != DataType::Int64) {
        throw InferenceException(context + ": tensors must be float32 or int64");
    }
    if (out.dtype != in.dtype) {
        throw InferenceException(context + ": output dtype must match the input dtype");
    }
    if (indices.dtype != DataType::Int64) {
        throw InferenceException(context + ": GatherElements indices must be int64");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    if (static_cast<int64_t>(indices.dims.size()) != rank) {
        throw InferenceException(context + ": GatherElements data and indices must share rank");
    }
    int64_t axis = IntAttrC(node, "axis", 1, context);
    if (rank == 0 || axis < -rank || axis >= rank) {
        throw InferenceException(context + ": GatherElements axis is out of range");
    }
    if (axis < 0) {
        axis += rank;
    }
    if (out.dims != indices.dims) {
        throw InferenceException(context + ": output shape must match the indices shape");
    }
    const int64_t count = CountNonNeg(indices.dims, context);
    (void)CountNonNeg(in.dims, context);
    (void)CountNonNeg(out.dims, context);
    if (count > 0 && indices.data == nullptr) {
        throw InferenceException(context + ": null indices buffer");
    }
    if (count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    if (count == 0) {
        AfterRow(outputs, context);
        return;
    }
    // An off-axis index coordinate beyond the data extent is out of range for
    // every element on it (src/kernels/gather_elements.cpp:47-50).
    for (int64_t j = 0; j < rank; ++j) {
        if (j != axis && indices.dims[static_cast<size_t>(j)] > in.dims[static_cast<size_t>(j)]) {
            throw InferenceException(context + ": GatherElements index is out of range");
        }
    }
    const int64_t dim = in.dims[static_cast<size_t>(axis)];
    std::vector<int64_t> host;
    const bool on_host = HostShadowInt64(indices, count, host);
    if (on_host) {
        for (const int64_t k : host) {
            const int64_t w = Wrap(k, dim);
            if (w < 0 || w >= dim) {
                throw InferenceException(context + ": GatherElements index is out of range");
            }
        }
    }
    CheckStatus(nert_hip_gather_elements(static_cast<int>(ElementSize(in.dtype)), in.data,
                                         static_cast<const int64_t*>(indices.data), out.data, static_cast<int>(rank),
                                         in.dims.data(), indices.dims.data(), static_cast<int>(axis), Stream()),
                context);
    AfterRow(outputs, context);
    if (!on_host) {
        ThrowOnDeviceFlag(context, "GatherElements index is out of range");
    }
}

// src/kernels/scatter_nd.cpp:31-118
NERT_HIP_ROW(ScatterND) {
    const std::string context = "ScatterND (node '" + node.name + "')";
    if (inputs.size() != 3 || outputs.size() != 1) {
        throw InferenceException(context + ": expected data, indices, updates, and one output");
    }
    const TensorView& data = inputs[0];
    const TensorView& indices = inputs[1];
    const TensorView& updates = inputs[2];
    const TensorView& out = outputs[0];
    if (data.dtype != DataType::Float32 && data.dtype != DataType::Int64 && data.dtype != DataType::Bool) {
        throw InferenceException(context + ": data must be float32, int64, or bool");
    }
    if (updates.dtype != data.dtype || out.dtype != data.dtype) {
        throw InferenceException(context + ": data, updates, and output must share dtype");
    }
    if (indices.dtype != DataType::Int64) {
        throw InferenceException(context + ": indices must be int64");
    }
    if (indices.dims.empty()) {
        throw InferenceException(context + ": indices must have rank >= 1");
    }
    const int64_t data_rank = static_cast<int64_t>(data.dims.size());
    const int64_t k = indices.dims.back();
    if (k < 1 || k > data_rank) {
        throw InferenceException(context + ": indices last dim must be within the data rank");
    }
    if (out.dims != data.dims) {
        throw InferenceException(context + ": output shape must match the data shape");
    }
    std::vector<int64_t> expected_updates(indices.dims.begin(), indices.dims.end() - 1);
    expected_updates.insert(expected_updates.end(), data.dims.begin() + k, data.dims.end());
    if (updates.dims != expected_updates) {
        throw InferenceException(context + ": updates shape does not match indices and data");
    }
    (void)ElementCount(data.dims, context);
    const int64_t index_count = ElementCount(indices.dims, context);
    (void)ElementCount(updates.dims, context);
    if (data.data == nullptr || indices.data == nullptr || updates.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    const int64_t slices = index_count / k;
    std::vector<int64_t> host;
    const bool on_host = HostShadowInt64(indices, index_count, host);
    if (on_host) {
        for (int64_t s = 0; s < slices; ++s) {
            for (int64_t j = 0; j < k; ++j) {
                const int64_t c = host[static_cast<size_t>(s * k + j)];
                const int64_t dim = data.dims[static_cast<size_t>(j)];
                if (c < -dim || c >= dim) {
                    throw InferenceException(context + ": index out of range");
                }
            }
        }
    }
    CheckStatus(nert_hip_scatter_nd(static_cast<int>(ElementSize(data.dtype)), data.data,
                                    static_cast<const int64_t*>(indices.data), updates.data, out.data,
                                    static_cast<int>(data_rank), data.dims.data(), slices, static_cast<int>(k),
                                    Stream()),
                context);
    AfterRow(outputs, context);
    if (!on_host) {
        ThrowOnDeviceFlag(context, "index out of range");
    }
}

// src/kernels/top_k.cpp:38-142
NERT_HIP_ROW(TopK) {
    const std::string context = "TopK (node '" + node.name + "')";
    if (inputs.size() != 2 || outputs.size() != 2) {
        throw InferenceException(context + ": expected an input, a K input, and values/indices outputs");
    }
    const TensorView& in = inputs[0];
    const TensorView& k_view = inputs[1];
    const TensorView& values = outputs[0];
    const TensorView& indices = outputs[1];
    if (in.dtype != DataType::Float32) {
        throw InferenceException(context + ": TopK input must be float32");
    }
    if (values.dtype != DataType::Float32) {
        throw InferenceException(context + ": TopK values must be float32");
    }
    if (indices.dtype != DataType::Int64) {
        throw InferenceException(context + ": TopK indices must be int64");
    }
    if (k_view.dtype != DataType::Int64) {
        throw InferenceException(context + ": TopK requires a K input");
    }
    if (IntAttrC(node, "largest", 1, context) != 1) {
        throw InferenceException(context + ": TopK 'largest' must be 1 here");
    }
    if (IntAttrC(node, "sorted", 1, context) != 1) {
        throw InferenceException(context + ": TopK 'sorted' must be 1 here");
    }
    if (CountNonNeg(k_view.dims, context) != 1) {
        throw InferenceException(context + ": TopK K input must be a scalar Int64 constant");
    }
    if (k_view.data == nullptr) {
        throw InferenceException(context + ": null K buffer");
    }
    const int64_t k = ReadInt64(k_view, 1, context)[0];
    if (k <= 0) {
        throw InferenceException(context + ": TopK K must be positive");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    int64_t axis = IntAttrC(node, "axis", -1, context);
    if (rank == 0 || axis < -rank || axis >= rank) {
        throw InferenceException(context + ": TopK axis is out of range");
    }
    if (axis < 0) {
        axis += rank;
    }
    const int64_t dim = in.dims[static_cast<size_t>(axis)];
    if (k > dim) {
        throw InferenceException(context + ": TopK K exceeds the axis dim");
    }
    std::vector<int64_t> expected = in.dims;
    expected[static_cast<size_t>(axis)] = k;
    if (values.dims != expected || indices.dims != expected) {
        throw InferenceException(context + ": output shapes do not match the selected K");
    }
    const int64_t values_count = CountNonNeg(values.dims, context);
    (void)CountNonNeg(in.dims, context);
    if (values_count > 0 && (in.data == nullptr || values.data == nullptr || indices.data == nullptr)) {
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
    if (values_count > 0) {
        CheckStatus(nert_hip_topk_f32(static_cast<const float*>(in.data), static_cast<float*>(values.data),
                                      static_cast<int64_t*>(indices.data), outer, dim, inner, k, Stream()),
                    context);
    }
    AfterRow(outputs, context);
}

// src/kernels/shape.cpp:40-72
NERT_HIP_ROW(Shape) {
    const std::string context = "Shape (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 && in.dtype != DataType::Int64 && in.dtype != DataType::Bool) {
        throw InferenceException(context + ": Shape input must be float32, int64, or bool");
    }
    if (out.dtype != DataType::Int64) {
        throw InferenceException(context + ": Shape output must be int64");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    int64_t start = IntAttr(node, "start", 0, "Shape");
    int64_t end = IntAttr(node, "end", rank, "Shape");
    start = std::min(std::max(start < 0 ? start + rank : start, int64_t{0}), rank);
    end = std::min(std::max(end < 0 ? end + rank : end, int64_t{0}), rank);
    if (end < start) {
        end = start;
    }
    if (out.dims != std::vector<int64_t>{end - start}) {
        throw InferenceException(context + ": Shape output shape must be the selected dim count");
    }
    if (end > start && out.data == nullptr) {
        throw InferenceException(context + ": null output buffer");
    }
    const std::vector<int64_t> values(in.dims.begin() + start, in.dims.begin() + end);
    if (!values.empty()) {
        CheckStatus(nert_hip_store_i64(static_cast<int64_t*>(out.data), values.data(),
                                       static_cast<int>(values.size()), Stream()),
                    context);
    }
    AfterRow(outputs, context);
    // Shape feeds shape arithmetic: keep the values readable on the host.
    PutHostShadow(out.data, values.data(), static_cast<int64_t>(values.size() * sizeof(int64_t)));
}

// src/kernels/constant_of_shape.cpp:26-99
NERT_HIP_ROW(ConstantOfShape) {
    const std::string context = "ConstantOfShape (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected a shape input and one output");
    }
    const TensorView& shape_view = inputs[0];
    const TensorView& out = outputs[0];
    if (shape_view.dtype != DataType::Int64) {
        throw InferenceException(context + ": ConstantOfShape requires a shape input");
    }
    if (shape_view.dims.size() != 1) {
        throw InferenceException(context + ": ConstantOfShape shape input must be rank 1");
    }
    const int64_t extent = CountNonNeg(shape_view.dims, context);
    if (extent > 0 && shape_view.data == nullptr) {
        throw InferenceException(context + ": null shape buffer");
    }
    const std::vector<int64_t> shape = ReadInt64(shape_view, extent, context);
    for (const int64_t v : shape) {
        if (v < 0) {
            throw InferenceException(context + ": ConstantOfShape shape values must be non-negative");
        }
    }
    const Attribute* value = nullptr;
    for (const Attribute& attr : node.attributes) {
        if (attr.name == "value") {
            value = &attr;
        }
    }
    if (out.dims != shape) {
        throw InferenceException(context + ": output shape does not match the shape input");
    }
    const int64_t out_count = Count(out.dims);
    if (out_count > 0 && out.data == nullptr) {
        throw InferenceException(context + ": null output buffer");
    }
    int code = 0;
    double fvalue = 0.0;
    int64_t ivalue = 0;
    if (value == nullptr || std::holds_alternative<float>(value->value)) {
        if (out.dtype != DataType::Float32) {
            throw InferenceException(context + ": ConstantOfShape output must be float32 for a float value");
        }
        code = NERT_F32;
        fvalue = value == nullptr ? 0.0 : static_cast<double>(std::get<float>(value->value));
    } else if (const int64_t* iv = std::get_if<int64_t>(&value->value)) {
        if (out.dtype != DataType::Int64) {
            throw InferenceException(context + ": ConstantOfShape output must be int64 for an int64 value");
        }
        code = NERT_I64;
        ivalue = *iv;
    } else if (const bool* bv = std::get_if<bool>(&value->value)) {
        if (out.dtype != DataType::Bool) {
            throw InferenceException(context + ": ConstantOfShape output must be bool for a bool value");
        }
        code = NERT_BOOL;
        ivalue = *bv ? 1 : 0;
    } else {
        throw InferenceException(context + ": ConstantOfShape 'value' must be an int64, float, or bool scalar");
    }
    CheckStatus(nert_hip_fill(code, out.data, out_count, fvalue, ivalue, Stream()), context);
    AfterRow(outputs, context);
}

// src/kernels/range.cpp:35-100
NERT_HIP_ROW(Range) {
    const std::string context = "Range (node '" + node.name + "')";
    if (inputs.size() != 3 || outputs.size() != 1) {
        throw InferenceException(context + ": expected start, limit, delta and one output");
    }
    const TensorView& out = outputs[0];
    const DataType dtype = inputs[0].dtype;
    if ((dtype != DataType::Float32 && dtype != DataType::Int64) || out.dtype != dtype) {
        throw InferenceException(context + ": tensors must share dtype float32 or int64");
    }
    if (out.dims.size() != 1 || out.dims[0] < 0) {
        throw InferenceException(context + ": output must be rank 1");
    }
    const int64_t out_count = out.dims[0];
    auto scalar_view = [&](const TensorView& view, const char* what) {
        if (view.dtype != dtype) {
            throw InferenceException(context + ": " + what + " dtype must match the other operands");
        }
        if (Count(view.dims) != 1) {
            throw InferenceException(context + ": " + what + " must be a scalar");
        }
        if (view.data == nullptr) {
            throw InferenceException(context + ": null " + std::string(what) + " buffer");
        }
    };
    if (dtype == DataType::Float32) {
        scalar_view(inputs[0], "start");
        const float start = ReadFloat(inputs[0], 1, context)[0];
        scalar_view(inputs[1], "limit");
        const float limit = ReadFloat(inputs[1], 1, context)[0];
        scalar_view(inputs[2], "delta");
        const float delta = ReadFloat(inputs[2], 1, context)[0];
        if (delta == 0.0f) {
            throw InferenceException(context + ": delta must be non-zero");
        }
        const double span =
            std::ceil((static_cast<double>(limit) - static_cast<double>(start)) / static_cast<double>(delta));
        const int64_t expected = span > 0.0 ? static_cast<int64_t>(span) : 0;
        if (out_count != expected) {
            throw InferenceException(context + ": output length does not match the range");
        }
        if (out_count > 0 && out.data == nullptr) {
            throw InferenceException(context + ": null output buffer");
        }
        CheckStatus(nert_hip_range(NERT_F32, start, delta, 0, 0, out.data, out_count, Stream()), context);
        AfterRow(outputs, context);
        return;
    }
    scalar_view(inputs[0], "start");
    const int64_t start = ReadInt64(inputs[0], 1, context)[0];
    scalar_view(inputs[1], "limit");
    const int64_t limit = ReadInt64(inputs[1], 1, context)[0];
    scalar_view(inputs[2], "delta");
    const int64_t delta = ReadInt64(inputs[2], 1, context)[0];
    if (delta == 0) {
        throw InferenceException(context + ": delta must be non-zero");
    }
    int64_t expected = 0;
    if (delta > 0 && limit > start) {
        expected = (limit - start + delta - 1) / delta;
    } else if (delta < 0 && limit < start) {
        expected = (start - limit + (-delta) - 1) / (-delta);
    }
    if (out_count != expected) {
        throw InferenceException(context + ": output length does not match the range");
    }
    if (out_count > 0 && out.data == nullptr) {
        throw InferenceException(context + ": null output buffer");
    }
    CheckStatus(nert_hip_range(NERT_I64, 0.0, 0.0, start, delta, out.data, out_count, Stream()), context);
    AfterRow(outputs, context);
}

// src/kernels/eye_like.cpp:42-84
NERT_HIP_ROW(EyeLike) {
    const std::string context = "EyeLike (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dims.size() != 2 || out.dims != in.dims) {
        throw InferenceException(context + ": input and output must share a rank-2 shape");
    }
    if (out.dtype != DataType::Float32 && out.dtype != DataType::Int64 && out.dtype != DataType::Bool) {
        throw InferenceException(context + ": output must be float32, int64, or bool");
    }
    const int64_t k = IntAttrC(node, "k", 0, context);
    (void)ElementCount(out.dims, context);
    if (out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    CheckStatus(nert_hip_eye_like(DtypeCode(out.dtype), out.data, in.dims[0], in.dims[1], k, Stream()), context);
    AfterRow(outputs, context);
}

} // namespace rows
} // namespace nert_hip
