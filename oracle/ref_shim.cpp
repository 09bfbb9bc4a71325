// C-ABI shim over the reference CPU library (oracle/_ref/libnert_ref.so).
//
// Test infrastructure only. It lets the Python tests and bench.py's
// cpu_baseline leg drive the reference's own CpuDevice rows
// (src/cpu_device.cpp:88, table src/kernels/cpu_kernels.cpp:15-93) and its
// executor (src/executor.cpp:202-369) with plain pointers, so every parity
// check compares against the real reference code, compiled unmodified.

#include "../include/nert_abi_node.hpp"

#include "nert/device.hpp"
#include "nert/executor.hpp"
#include "nert/graph.hpp"
#include "nert/model_loader.hpp"
#include "nert/shapes.hpp"

#include <chrono>
#include <map>
#include <string>
#include <vector>

extern "C" {

// One row of CpuDevice's table on host buffers.
int nert_ref_run_node(const char* op_type, const char* name, int64_t schema_version, const nert_attr_desc* attrs,
                      int n_attrs, const nert_tensor_desc* inputs, int n_inputs, const nert_tensor_desc* outputs,
                      int n_outputs, char* err, int err_len) {
    return nert_abi::RunNode(nert::CpuDevice(), op_type, name, schema_version, attrs, n_attrs, inputs, n_inputs,
                             outputs, n_outputs, err, err_len);
}

// Loads an ONNX file with the reference loader (src/model_loader.cpp:2278);
// returns an owned nert::Graph* or null with the message in `err`.
void* nert_ref_load_graph(const char* path, char* err, int err_len) {
    try {
        return new nert::Graph(nert::LoadGraphFromFile(path != nullptr ? path : ""));
    } catch (const std::exception& e) {
        nert_abi::CopyMessage(e.what(), err, err_len);
        return nullptr;
    }
}

void nert_ref_free_graph(void* graph) { delete static_cast<nert::Graph*>(graph); }

// True (1) when the CPU table has a row for `op_type`.
int nert_ref_has_row(const char* op_type) {
    return nert::CpuDevice().kernels().find(op_type != nullptr ? op_type : "") != nullptr ? 1 : 0;
}

// Runs `graph` (a nert::Graph* built by the caller) through the reference
// executor on CpuDevice: Model(graph, dims, CpuDevice()).RunTyped(inputs).
// Inputs and outputs are host buffers named in the same order as the graph's
// declared inputs/outputs; each output buffer must hold the output's bytes.
// `seconds` receives the wall time of RunTyped alone.
int nert_ref_model_run(const void* graph_handle, int n_inputs, const nert_tensor_desc* inputs, int n_outputs,
                       const nert_tensor_desc* outputs, double* seconds, char* err, int err_len) {
    try {
        const nert::Graph& graph = *static_cast<const nert::Graph*>(graph_handle);
        if (n_inputs != static_cast<int>(graph.inputs.size()) || n_outputs != static_cast<int>(graph.outputs.size())) {
            nert_abi::CopyMessage("input/output count does not match the graph", err, err_len);
            return NERT_OTHER_ERROR;
        }
        nert::ShapeMap dims;
        nert::HostTensorMap host_inputs;
        for (int i = 0; i < n_inputs; ++i) {
            const std::string& name = graph.inputs[static_cast<size_t>(i)].first;
            const nert::TensorView view = nert_abi::ToView(inputs[i]);
            dims[name] = view.dims;
            nert::HostTensor tensor;
            tensor.dtype = view.dtype;
            tensor.dims = view.dims;
            int64_t count = 1;
            for (int64_t d : view.dims) {
                count *= d;
            }
            const size_t bytes = static_cast<size_t>(count) * nert::HostElementSize(view.dtype);
            const auto* src = static_cast<const uint8_t*>(view.data);
            tensor.bytes.assign(src, src + bytes);
            host_inputs.emplace(name, std::move(tensor));
        }
        nert::Model model(graph, dims, nert::CpuDevice());
        const auto start = std::chrono::steady_clock::now();
        nert::HostTensorMap result = model.RunTyped(host_inputs);
        const auto stop = std::chrono::steady_clock::now();
        if (seconds != nullptr) {
            *seconds = std::chrono::duration<double>(stop - start).count();
        }
        for (int i = 0; i < n_outputs; ++i) {
            const std::string& name = graph.outputs[static_cast<size_t>(i)].first;
            const auto it = result.find(name);
            if (it == result.end()) {
                nert_abi::CopyMessage("missing output " + name, err, err_len);
                return NERT_OTHER_ERROR;
            }
            const nert::TensorView view = nert_abi::ToView(outputs[i]);
            std::memcpy(view.data, it->second.bytes.data(), it->second.bytes.size());
        }
        nert_abi::CopyMessage("", err, err_len);
        return NERT_OK;
    } catch (const nert::InferenceException& e) {
        nert_abi::CopyMessage(e.what(), err, err_len);
        return NERT_INFERENCE_ERROR;
    } catch (const std::exception& e) {
        nert_abi::CopyMessage(e.what(), err, err_len);
        return NERT_OTHER_ERROR;
    }
}

// Shapes the reference's own InferShapes derives for `graph` at the given
// input dims; writes the rank and dims of tensor `name` (up to 8 dims).
// Used to pin the synthetic graph builders' shape tables.
int nert_ref_infer_shape(const void* graph_handle, int n_inputs, const nert_tensor_desc* inputs, const char* name,
                         int64_t* dims_out, int* rank_out, char* err, int err_len) {
    try {
        const nert::Graph& graph = *static_cast<const nert::Graph*>(graph_handle);
        nert::ShapeMap dims;
        for (int i = 0; i < n_inputs; ++i) {
            const nert::TensorView view = nert_abi::ToView(inputs[i]);
            dims[graph.inputs[static_cast<size_t>(i)].first] = view.dims;
        }
        const nert::InferredShapes shapes = nert::InferShapes(graph, dims);
        const auto it = shapes.tensors.find(name != nullptr ? name : "");
        if (it == shapes.tensors.end()) {
            nert_abi::CopyMessage("no shape for tensor", err, err_len);
            return NERT_OTHER_ERROR;
        }
        *rank_out = static_cast<int>(it->second.dims.size());
        for (size_t d = 0; d < it->second.dims.size() && d < 8; ++d) {
            dims_out[d] = it->second.dims[d];
        }
        return NERT_OK;
    } catch (const std::exception& e) {
        nert_abi::CopyMessage(e.what(), err, err_len);
        return NERT_OTHER_ERROR;
    }
}

} // extern "C"
