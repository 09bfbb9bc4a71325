// Pure data-movement rows whose output is a byte copy of the input:
// Identity, Flatten, Reshape (src/kernels/{identity,flatten,reshape}.cpp).
// The copy is an asynchronous device-to-device transfer on the layer stream.

#include "rows.hpp"

namespace nert_hip {
namespace rows {

using namespace seam;

namespace {

void CopyBytes(const TensorView& in, const TensorView& out, int64_t bytes, const std::string& context) {
    if (bytes > 0 && in.data != out.data) {
        CheckStatus(nert_hip_memcpy_d2d(out.data, in.data, bytes, Stream()), context);
    }
}

} // namespace

NERT_HIP_ROW(Identity) {
    const std::string context = "Identity (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != out.dtype) {
        throw InferenceException(context + ": input and output dtypes differ");
    }
    const int64_t element = ElementSize(in.dtype);
    if (element == 0) {
        throw InferenceException(context + ": tensors must be float32, int64, or bool");
    }
    if (in.dims != out.dims) {
        throw InferenceException(context + ": input and output shapes differ");
    }
    const int64_t count = ElementCount(out.dims, context);
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    CopyBytes(in, out, count * element, context);
    AfterRow(outputs, context);
}

NERT_HIP_ROW(Flatten) {
    const std::string context = "Flatten (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 && in.dtype != DataType::Int64 && in.dtype != DataType::Bool) {
        throw InferenceException(context + ": tensors must be float32, int64, or bool");
    }
    if (out.dtype != in.dtype) {
        throw InferenceException(context + ": output dtype must match the input dtype");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    int64_t axis = 1;
    for (const Attribute& attr : node.attributes) {
        if (attr.name == "axis") {
            const int64_t* value = std::get_if<int64_t>(&attr.value);
            if (value == nullptr) {
                throw InferenceException(context + ": attribute 'axis' must be an integer");
            }
            axis = *value;
        }
    }
    if (axis < 0) {
        axis += rank + 1;
    }
    if (axis < 0 || axis > rank) {
        throw InferenceException(context + ": Flatten axis is out of range");
    }
    int64_t first = 1;
    for (int64_t i = 0; i < axis; ++i) {
        first *= in.dims[static_cast<size_t>(i)];
    }
    int64_t second = 1;
    for (size_t i = static_cast<size_t>(axis); i < in.dims.size(); ++i) {
        second *= in.dims[i];
    }
    if (out.dims != std::vector<int64_t>{first, second}) {
        throw InferenceException(context + ": output shape does not match the flattened input");
    }
    const int64_t in_count = ElementCount(in.dims, context);
    const int64_t out_count = ElementCount(out.dims, context);
    if (in_count != out_count) {
        throw InferenceException(context + ": element-count mismatch");
    }
    if (in_count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    CopyBytes(in, out, in_count * ElementSize(in.dtype), context);
    AfterRow(outputs, context);
}

NERT_HIP_ROW(Reshape) {
    const std::string context = "Reshape (node '" + node.name + "')";
    if (inputs.empty() || inputs.size() > 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one or two inputs and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != out.dtype ||
        (in.dtype != DataType::Float32 && in.dtype != DataType::Int64 && in.dtype != DataType::Bool)) {
        throw InferenceException(context + ": data tensors must share one float32, int64, or bool dtype");
    }
    bool allowzero = false;
    for (const Attribute& attr : node.attributes) {
        if (attr.name == "allowzero") {
            const int64_t* value = std::get_if<int64_t>(&attr.value);
            if (value == nullptr) {
                throw InferenceException(context + ": attribute 'allowzero' must be an integer");
            }
            allowzero = (*value != 0);
        }
    }
    const int64_t in_count = ElementCount(in.dims, context);
    if (inputs.size() == 2) {
        const TensorView& shape = inputs[1];
        if (shape.dtype != DataType::Int64) {
            throw InferenceException(context + ": shape operand must be int64");
        }
        const int64_t shape_count = ElementCount(shape.dims, context);
        if (shape_count > 0 && shape.data == nullptr) {
            throw InferenceException(context + ": null shape buffer");
        }
        const std::vector<int64_t> target = ReadInt64(shape, shape_count, context);
        // src/kernels/reshape.cpp:75-122 (the shape-inference resolution).
        std::vector<int64_t> effective(target.size(), 0);
        int64_t inferred = -1;
        for (size_t i = 0; i < target.size(); ++i) {
            const int64_t v = target[i];
            if (v == 0 && !allowzero) {
                if (i >= in.dims.size()) {
                    throw InferenceException(context + ": Reshape 0 has no matching input dimension");
                }
                effective[i] = in.dims[i];
            } else if (v == -1) {
                if (inferred >= 0) {
                    throw InferenceException(context + ": Reshape allows at most one -1");
                }
                inferred = static_cast<int64_t>(i);
            } else if (v < 0) {
                throw InferenceException(context + ": Reshape target dimensions must be positive");
            } else {
                effective[i] = v;
            }
        }
        int64_t known = 1;
        for (size_t i = 0; i < effective.size(); ++i) {
            if (static_cast<int64_t>(i) != inferred) {
                known *= effective[i];
            }
        }
        if (inferred >= 0) {
            if (known == 0 || in_count % known != 0) {
                throw InferenceException(context + ": Reshape target product does not match input elements");
            }
            effective[static_cast<size_t>(inferred)] = in_count / known;
        }
        int64_t product = 1;
        for (int64_t dim : effective) {
            product *= dim;
        }
        if (product != in_count) {
            throw InferenceException(context + ": Reshape target product does not match input elements");
        }
        if (out.dims != effective) {
            throw InferenceException(context + ": output shape does not match the resolved shape operand");
        }
    }
    const int64_t out_count = ElementCount(out.dims, context);
    if (in_count != out_count) {
        throw InferenceException(context + ": element-count mismatch");
    }
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    CopyBytes(in, out, in_count * ElementSize(in.dtype), context);
    AfterRow(outputs, context);
}

} // namespace rows
} // namespace nert_hip
