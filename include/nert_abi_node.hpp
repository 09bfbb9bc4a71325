#pragma once
// C++ side of nert_abi.h: converts the plain-C node and tensor descriptions
// into the seam's own types (nert::Node, nert::TensorView) so any device's
// kernel table can run them. Needs the NERT public headers on the include
// path (include/nert/graph.hpp and include/nert/device.hpp of olibartfast/nert).

#include "nert_abi.h"
#include "nert/device.hpp"
#include "nert/graph.hpp"

#include <cstring>
#include <string>
#include <vector>

namespace nert_abi {

inline nert::DataType ToDataType(int32_t code) {
    switch (code) {
    case NERT_F32:
        return nert::DataType::Float32;
    case NERT_I64:
        return nert::DataType::Int64;
    case NERT_BOOL:
        return nert::DataType::Bool;
    default:
        return nert::DataType::Unknown;
    }
}

inline int32_t FromDataType(nert::DataType dtype) {
    switch (dtype) {
    case nert::DataType::Float32:
        return NERT_F32;
    case nert::DataType::Int64:
        return NERT_I64;
    case nert::DataType::Bool:
        return NERT_BOOL;
    default:
        return NERT_UNKNOWN;
    }
}

// rank < 0 is the omitted-operand marker: an empty view, as the executor
// passes for a blank input name.
inline nert::TensorView ToView(const nert_tensor_desc& desc) {
    nert::TensorView view;
    if (desc.rank < 0) {
        return view;
    }
    view.data = desc.data;
    view.dtype = ToDataType(desc.dtype);
    view.dims.assign(desc.dims, desc.dims + desc.rank);
    return view;
}

inline std::vector<nert::TensorView> ToViews(const nert_tensor_desc* descs, int count) {
    std::vector<nert::TensorView> views;
    views.reserve(count > 0 ? static_cast<size_t>(count) : 0U);
    for (int i = 0; i < count; ++i) {
        views.push_back(ToView(descs[i]));
    }
    return views;
}

inline nert::Attribute ToAttribute(const nert_attr_desc& desc) {
    const std::string name = desc.name != nullptr ? desc.name : "";
    switch (desc.kind) {
    case NERT_ATTR_INT:
        return nert::Attribute(name, desc.i);
    case NERT_ATTR_FLOAT:
        return nert::Attribute(name, desc.f);
    case NERT_ATTR_STRING:
        return nert::Attribute(name, std::string(desc.s != nullptr ? desc.s : ""));
    case NERT_ATTR_INTS:
        return nert::Attribute(name, std::vector<int64_t>(desc.ints, desc.ints + desc.count));
    case NERT_ATTR_FLOATS:
        return nert::Attribute(name, std::vector<float>(desc.floats, desc.floats + desc.count));
    case NERT_ATTR_BOOL:
        return nert::Attribute(name, desc.i != 0);
    default:
        return nert::Attribute(name, int64_t{0});
    }
}

// Builds the node. Input/output names are synthesised ("in0", "out0", ...)
// with an empty name for omitted operands, which is what the form helpers
// (AxesInputPresent and friends) inspect.
inline nert::Node ToNode(const char* op_type, const char* name, int64_t schema_version, const nert_attr_desc* attrs,
                         int n_attrs, const nert_tensor_desc* inputs, int n_inputs, int n_outputs) {
    nert::Node node;
    node.op_type = op_type != nullptr ? op_type : "";
    node.name = name != nullptr ? name : "";
    node.schema_version = schema_version;
    for (int i = 0; i < n_attrs; ++i) {
        node.attributes.push_back(ToAttribute(attrs[i]));
    }
    for (int i = 0; i < n_inputs; ++i) {
        node.inputs.push_back(inputs[i].rank < 0 ? std::string() : "in" + std::to_string(i));
    }
    for (int i = 0; i < n_outputs; ++i) {
        node.outputs.push_back("out" + std::to_string(i));
    }
    return node;
}

inline void CopyMessage(const std::string& message, char* err, int err_len) {
    if (err == nullptr || err_len <= 0) {
        return;
    }
    const size_t n = message.size() < static_cast<size_t>(err_len - 1) ? message.size() : static_cast<size_t>(err_len - 1);
    std::memcpy(err, message.data(), n);
    err[n] = '\0';
}

// Runs one row found by `find` (op type -> row, null when none) and maps the
// outcome to nert_status.
template <typename Find>
inline int RunFoundRow(Find&& find, const char* op_type, const char* name, int64_t schema_version,
                       const nert_attr_desc* attrs, int n_attrs, const nert_tensor_desc* inputs, int n_inputs,
                       const nert_tensor_desc* outputs, int n_outputs, char* err, int err_len) {
    try {
        const nert::Node node = ToNode(op_type, name, schema_version, attrs, n_attrs, inputs, n_inputs, n_outputs);
        const nert::KernelFn fn = find(node.op_type);
        if (fn == nullptr) {
            CopyMessage("no kernel for op '" + node.op_type + "'", err, err_len);
            return NERT_NO_KERNEL;
        }
        fn(node, ToViews(inputs, n_inputs), ToViews(outputs, n_outputs));
        CopyMessage("", err, err_len);
        return NERT_OK;
    } catch (const nert::InferenceException& e) {
        CopyMessage(e.what(), err, err_len);
        return NERT_INFERENCE_ERROR;
    } catch (const std::exception& e) {
        CopyMessage(e.what(), err, err_len);
        return NERT_OTHER_ERROR;
    }
}

// Runs one row from `device`'s table (`device.kernels().find`).
inline int RunNode(const nert::Device& device, const char* op_type, const char* name, int64_t schema_version,
                   const nert_attr_desc* attrs, int n_attrs, const nert_tensor_desc* inputs, int n_inputs,
                   const nert_tensor_desc* outputs, int n_outputs, char* err, int err_len) {
    return RunFoundRow([&](const std::string& op) { return device.kernels().find(op); }, op_type, name,
                       schema_version, attrs, n_attrs, inputs, n_inputs, outputs, n_outputs, err, err_len);
}

} // namespace nert_abi
