// Drop-in check: the reference executor (nert::Model, src/executor.cpp:202-369,
// from oracle/_ref/libnert_ref.so) running a graph on the gfx950
// nert::HipDevice() from nert_amd/lib/libnert_hip.so -- exactly how a NERT
// user would swap the device. Test infrastructure: loaded by tests/ only.

#include "../../include/nert_abi_node.hpp"

#include "nert/device.hpp"
#include "nert/executor.hpp"
#include "nert/graph.hpp"

#include <chrono>
#include <cstring>

extern "C" int dropin_model_run(const void* graph_handle, int n_inputs, const nert_tensor_desc* inputs,
                                int n_outputs, const nert_tensor_desc* outputs, int runs, double* seconds,
                                int64_t* arena_bytes, char* err, int err_len) {
    try {
        const nert::Graph& graph = *static_cast<const nert::Graph*>(graph_handle);
        nert::ShapeMap dims;
        nert::HostTensorMap host_inputs;
        for (int i = 0; i < n_inputs; ++i) {
            const std::string& name = graph.inputs[static_cast<size_t>(i)].first;
            const nert::TensorView view = nert_abi::ToView(inputs[i]);
            dims[name] = view.dims;
            nert::HostTensor t;
            t.dtype = view.dtype;
            t.dims = view.dims;
            int64_t count = 1;
            for (int64_t d : view.dims) {
                count *= d;
            }
            const auto* src = static_cast<const uint8_t*>(view.data);
            t.bytes.assign(src, src + count * static_cast<int64_t>(nert::HostElementSize(view.dtype)));
            host_inputs.emplace(name, std::move(t));
        }
        nert::Model model(graph, dims, nert::HipDevice());
        *arena_bytes = model.plan().arena_size;
        nert::HostTensorMap result;
        double total = 0.0;
        for (int r = 0; r < runs; ++r) {
            const auto start = std::chrono::steady_clock::now();
            result = model.RunTyped(host_inputs);
            total += std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
        }
        *seconds = total / (runs > 0 ? runs : 1);
        for (int i = 0; i < n_outputs; ++i) {
            const std::string& name = graph.outputs[static_cast<size_t>(i)].first;
            const nert::TensorView view = nert_abi::ToView(outputs[i]);
            const auto& bytes = result.at(name).bytes;
            std::memcpy(view.data, bytes.data(), bytes.size());
        }
        return NERT_OK;
    } catch (const nert::InferenceException& e) {
        nert_abi::CopyMessage(e.what(), err, err_len);
        return NERT_INFERENCE_ERROR;
    } catch (const std::exception& e) {
        nert_abi::CopyMessage(e.what(), err, err_len);
        return NERT_OTHER_ERROR;
    }
}
