// C-ABI over the unchanged NERT host side driving the gfx950 device:
// nert::LoadGraphFromFile (src/model_loader.cpp:2278), optionally
// nert::FoldConstants(graph, CpuDevice()) (src/constant_folding.cpp:108-143),
// then nert::Model(graph, dims, nert::HipDevice()) (src/executor.cpp:202-369)
// and Model::RunTyped (include/nert/executor.hpp:71-76), exactly the calls a
// NERT user makes to swap the device; and the reference's full-model gate
// (tools/hip_model_check.cpp) on that device. Used by bench.py's drop-in legs.

#include "../../include/nert_abi_node.hpp"

#include "nert/constant_folding.hpp"
#include "nert/device.hpp"
#include "nert/executor.hpp"
#include "nert/graph.hpp"
#include "nert/model_loader.hpp"

#include <chrono>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

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

// The reference's full-model HIP gate (tools/hip_model_check.cpp:36-88) on a
// graph with one float32 input and one float32 output: load `path` (not
// timed), construct nert::Model(graph, {{input, dims}}, nert::HipDevice())
// (timed: shapes, plan, arena, resident uploads), then two Model::Run calls
// on the same host input (each timed, host input in, host output out).
// `output` receives run 2's output; times in milliseconds.
int nert_seam_gate(const char* path, const float* input, int64_t input_count, float* output, int64_t output_count,
                   double* construct_ms, double* run1_ms, double* run2_ms, char* err, int err_len) {
    try {
        using Clock = std::chrono::steady_clock;
        const nert::Graph graph = nert::LoadGraphFromFile(path != nullptr ? path : "");
        if (graph.inputs.size() != 1 || graph.outputs.size() != 1 ||
            graph.inputs[0].second.dtype != nert::DataType::Float32 ||
            graph.outputs[0].second.dtype != nert::DataType::Float32) {
            throw std::runtime_error("gate requires one float32 input and one float32 output");
        }
        const auto& dims = graph.inputs[0].second.dims;
        int64_t count = 1;
        for (int64_t d : dims) {
            count *= d;
        }
        if (count != input_count) {
            throw std::runtime_error("input element-count mismatch");
        }
        const std::vector<float> x(input, input + input_count);
        const auto t0 = Clock::now();
        nert::Model model(graph, {{graph.inputs[0].first, dims}}, nert::HipDevice());
        const auto t1 = Clock::now();
        *construct_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
        double* run_ms[2] = {run1_ms, run2_ms};
        for (int run = 0; run < 2; ++run) {
            const auto r0 = Clock::now();
            const auto result = model.Run({{graph.inputs[0].first, x}});
            const auto r1 = Clock::now();
            *run_ms[run] = std::chrono::duration<double, std::milli>(r1 - r0).count();
            const auto& got = result.outputs.at(graph.outputs[0].first);
            if (static_cast<int64_t>(got.size()) != output_count) {
                throw std::runtime_error("output element-count mismatch");
            }
            std::memcpy(output, got.data(), got.size() * sizeof(float));
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

} // extern "C"
