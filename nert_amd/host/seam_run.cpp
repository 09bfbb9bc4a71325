// C-ABI over the unchanged NERT host side driving the gfx950 device:
// nert::LoadGraphFromFile (src/model_loader.cpp:2278), optionally
// nert::FoldConstants(graph, CpuDevice()) (src/constant_folding.cpp:108-143),
// then nert::Model(graph, dims, nert::HipDevice()) (src/executor.cpp:202-369)
// and Model::RunTyped (include/nert/executor.hpp:71-76), exactly the calls a
// NERT user makes to swap the device. Used by bench.py's drop-in leg.

#include "../../include/nert_abi_node.hpp"

#include "nert/constant_folding.hpp"
#include "nert/device.hpp"
#include "nert/executor.hpp"
#include "nert/graph.hpp"
#include "nert/model_loader.hpp"

#include <chrono>
#include <cstring>
#include <memory>
#include <string>

namespace {

struct Session {
    nert::Graph graph;
    std::unique_ptr<nert::Model> model;
    nert::HostTensorMap inputs;
};

} // namespace

extern "C" {

// Loads `path`, folds constants on CpuDevice when fold != 0, and builds the
// Model on HipDevice() for the given inputs (graph input order), which are
// copied and reused by every nert_seam_run. Returns a session or null with
// the message in `err`.
void* nert_seam_open(const char* path, int fold, int n_inputs, const nert_tensor_desc* inputs, int64_t* arena_bytes,
                     char* err, int err_len) {
    try {
        auto s = std::make_unique<Session>();
        s->graph = nert::LoadGraphFromFile(path != nullptr ? path : "");
        if (fold != 0) {
            (void)nert::FoldConstants(s->graph, nert::CpuDevice());
        }
        nert::ShapeMap dims;
        for (int i = 0; i < n_inputs; ++i) {
            const std::string& name = s->graph.inputs.at(static_cast<size_t>(i)).first;
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
            s->inputs.emplace(name, std::move(t));
        }
        s->model = std::make_unique<nert::Model>(s->graph, dims, nert::HipDevice());
        *arena_bytes = s->model->plan().arena_size;
        return s.release();
    } catch (const std::exception& e) {
        nert_abi::CopyMessage(e.what(), err, err_len);
        return nullptr;
    }
}

// `runs` RunTyped calls on the session's inputs; *seconds = mean wall time
// per call (host inputs in, host outputs out). The last call's outputs are
// copied into `outputs` (graph output order).
int nert_seam_run(void* session, int runs, int n_outputs, const nert_tensor_desc* outputs, double* seconds, char* err,
                  int err_len) {
    try {
        auto* s = static_cast<Session*>(session);
        nert::HostTensorMap result;
        const auto start = std::chrono::steady_clock::now();
        for (int r = 0; r < runs; ++r) {
            result = s->model->RunTyped(s->inputs);
        }
        *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count() /
                   (runs > 0 ? runs : 1);
        for (int i = 0; i < n_outputs && runs > 0; ++i) {
            const auto& bytes = result.at(s->graph.outputs.at(static_cast<size_t>(i)).first).bytes;
            std::memcpy(nert_abi::ToView(outputs[i]).data, bytes.data(), bytes.size());
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

void nert_seam_close(void* session) { delete static_cast<Session*>(session); }

} // extern "C"
