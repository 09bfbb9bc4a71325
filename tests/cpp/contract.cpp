// Seam contract checks for the gfx950 nert::HipDevice(), as the reference's
// own suites state them for any device:
//   test/hip_device_test.cpp:23-148  names itself "hip", not a host device,
//                                    every first-party row resolves, no
//                                    allocation for sizes <= 0, 1 KiB round trip;
//   include/nert/device.hpp:33-76    aligned buffers, release(nullptr),
//                                    zero-byte transfers, arena offsets;
//   test/executor_test.cpp:375-479   residents upload once across runs, a
//                                    throwing row releases the staged inputs
//                                    and the model runs again afterwards;
//   src/constant_folding.cpp:108-143 FoldConstants(g, CpuDevice()) before the
//                                    drop-in.
// Test infrastructure: loaded by tests/ only. Links the reference library
// (oracle/_ref) for the executor, CpuDevice and FoldConstants, and the gfx950
// layer (nert_amd/lib) for HipDevice().

#include "../../include/nert_abi_node.hpp"

#include "nert/constant_folding.hpp"
#include "nert/device.hpp"
#include "nert/executor.hpp"
#include "nert/graph.hpp"

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

namespace {

void Fail(const std::string& what, char* err, int err_len) { nert_abi::CopyMessage(what.c_str(), err, err_len); }

// Forwards to HipDevice() and counts allocator and transfer calls; while
// g_throw_op is set, that op's row is replaced by one that throws.
std::string g_throw_op;

void ThrowingRow(const nert::Node& node, const std::vector<nert::TensorView>&, const std::vector<nert::TensorView>&) {
    throw nert::InferenceException(node.op_type + " (node '" + node.name + "'): boom");
}

struct Counts {
    int64_t allocate_calls = 0, release_calls = 0, live = 0, h2d_calls = 0, h2d_bytes = 0, d2h_calls = 0;
};

class CountingAllocator : public nert::Allocator {
  public:
    CountingAllocator(nert::Allocator& inner, Counts& c) : inner_(inner), c_(c) {}
    void* allocate(int64_t bytes) override {
        ++c_.allocate_calls;
        void* p = inner_.allocate(bytes);
        c_.live += p != nullptr ? 1 : 0;
        return p;
    }
    void release(void* buffer) override {
        ++c_.release_calls;
        c_.live -= buffer != nullptr ? 1 : 0;
        inner_.release(buffer);
    }

  private:
    nert::Allocator& inner_;
    Counts& c_;
};

class CountingTransfer : public nert::Transfer {
  public:
    CountingTransfer(nert::Transfer& inner, Counts& c) : inner_(inner), c_(c) {}
    void host_to_device(void* dst, const void* src, int64_t bytes) override {
        ++c_.h2d_calls;
        c_.h2d_bytes += bytes;
        inner_.host_to_device(dst, src, bytes);
    }
    void device_to_host(void* dst, const void* src, int64_t bytes) override {
        ++c_.d2h_calls;
        inner_.device_to_host(dst, src, bytes);
    }

  private:
    nert::Transfer& inner_;
    Counts& c_;
};

class ProbeTable : public nert::KernelTable {
  public:
    explicit ProbeTable(const nert::KernelTable& inner) : inner_(inner) {}
    nert::KernelFn find(const std::string& op_type) const override {
        if (!g_throw_op.empty() && op_type == g_throw_op) {
            return &ThrowingRow;
        }
        return inner_.find(op_type);
    }

  private:
    const nert::KernelTable& inner_;
};

class ProbeDevice : public nert::Device {
  public:
    ProbeDevice()
        : hip_(const_cast<nert::Device&>(nert::HipDevice())), alloc_(hip_.allocator(), counts),
          transfer_(hip_.transfer(), counts), table_(hip_.kernels()) {}
    const char* name() const override { return "hip-probe"; }
    nert::Allocator& allocator() override { return alloc_; }
    nert::Transfer& transfer() override { return transfer_; }
    const nert::KernelTable& kernels() const override { return table_; }
    bool is_host() const override { return hip_.is_host(); }
    bool supports_arena_offsets() const override { return hip_.supports_arena_offsets(); }
    Counts counts;

  private:
    nert::Device& hip_;
    CountingAllocator alloc_;
    CountingTransfer transfer_;
    ProbeTable table_;
};

nert::HostTensorMap HostInputs(const nert::Graph& graph, int n, const nert_tensor_desc* inputs,
                               nert::ShapeMap* dims) {
    nert::HostTensorMap host;
    for (int i = 0; i < n; ++i) {
        const std::string& name = graph.inputs[static_cast<size_t>(i)].first;
        const nert::TensorView view = nert_abi::ToView(inputs[i]);
        if (dims != nullptr) {
            (*dims)[name] = view.dims;
        }
        nert::HostTensor t;
        t.dtype = view.dtype;
        t.dims = view.dims;
        int64_t count = 1;
        for (int64_t d : view.dims) {
            count *= d;
        }
        const auto* src = static_cast<const uint8_t*>(view.data);
        t.bytes.assign(src, src + count * static_cast<int64_t>(nert::HostElementSize(view.dtype)));
        host.emplace(name, std::move(t));
    }
    return host;
}

void CopyOutputs(const nert::Graph& graph, const nert::HostTensorMap& result, int n, const nert_tensor_desc* outputs) {
    for (int i = 0; i < n; ++i) {
        const std::string& name = graph.outputs[static_cast<size_t>(i)].first;
        const nert::TensorView view = nert_abi::ToView(outputs[i]);
        const auto& bytes = result.at(name).bytes;
        std::memcpy(view.data, bytes.data(), bytes.size());
    }
}

} // namespace

extern "C" {

// Constructs HipDevice(); 0 and its facts, or the InferenceException text
// (no usable GPU) with NERT_INFERENCE_ERROR.
int contract_device_facts(char* name, int name_len, int* is_host, int* arena_offsets, char* err, int err_len) {
    try {
        const nert::Device& hip = nert::HipDevice();
        nert_abi::CopyMessage(hip.name(), name, name_len);
        *is_host = hip.is_host() ? 1 : 0;
        *arena_offsets = hip.supports_arena_offsets() ? 1 : 0;
        return NERT_OK;
    } catch (const nert::InferenceException& e) {
        Fail(e.what(), err, err_len);
        return NERT_INFERENCE_ERROR;
    } catch (const std::exception& e) {
        Fail(e.what(), err, err_len);
        return NERT_OTHER_ERROR;
    }
}

// For each op: found[i] = 1 when HipDevice().kernels().find(op) is non-null,
// cpu_found[i] likewise for CpuDevice().
int contract_find_rows(const char* const* ops, int n, int* found, int* cpu_found) {
    const nert::KernelTable& hip = nert::HipDevice().kernels();
    const nert::KernelTable& cpu = nert::CpuDevice().kernels();
    for (int i = 0; i < n; ++i) {
        found[i] = hip.find(ops[i]) != nullptr ? 1 : 0;
        cpu_found[i] = cpu.find(ops[i]) != nullptr ? 1 : 0;
    }
    return NERT_OK;
}

// Allocator and transfer contract; 0 when every check holds, else the first
// failed check in `err`.
int contract_allocator_transfer(char* err, int err_len) {
    try {
        nert::Device& hip = const_cast<nert::Device&>(nert::HipDevice());
        nert::Allocator& a = hip.allocator();
        nert::Transfer& t = hip.transfer();
        if (a.allocate(0) != nullptr || a.allocate(-1) != nullptr || a.allocate(-8) != nullptr) {
            Fail("allocate(bytes <= 0) must return null", err, err_len);
            return 1;
        }
        a.release(nullptr);
        // Alignment at sizes the planner and the executor's staging use,
        // including ones the block cache rounds, and after reuse.
        const int64_t sizes[] = {1, 3, 63, 64, 65, 1000, 4096, 65537, 1 << 20, (1 << 20) + 17, 7 << 20};
        std::vector<void*> held;
        for (int round = 0; round < 2; ++round) {
            for (int64_t s : sizes) {
                void* p = a.allocate(s);
                if (p == nullptr) {
                    Fail("allocate(" + std::to_string(s) + ") returned null", err, err_len);
                    return 1;
                }
                if (reinterpret_cast<uintptr_t>(p) % 64 != 0) {
                    Fail("allocate(" + std::to_string(s) + ") is not 64-byte aligned", err, err_len);
                    return 1;
                }
                held.push_back(p);
            }
            for (void* p : held) {
                a.release(p);
            }
            held.clear();
        }
        // Zero-byte transfers are no-ops, even with null pointers.
        t.host_to_device(nullptr, nullptr, 0);
        t.device_to_host(nullptr, nullptr, 0);
        // 1 KiB round trip of patterned bytes (hip_device_test.cpp:131-148),
        // and a ragged 3 MiB + 5 one that takes the staged path.
        for (int64_t bytes : {int64_t{1024}, int64_t{(3 << 20) + 5}}) {
            std::vector<uint8_t> host(static_cast<size_t>(bytes));
            for (size_t i = 0; i < host.size(); ++i) {
                host[i] = static_cast<uint8_t>((i * 31 + 7) & 0xFF);
            }
            void* dev = a.allocate(bytes);
            if (dev == nullptr) {
                Fail("round-trip allocation failed", err, err_len);
                return 1;
            }
            t.host_to_device(dev, host.data(), bytes);
            std::vector<uint8_t> back(host.size(), 0);
            t.device_to_host(back.data(), dev, bytes);
            a.release(dev);
            if (back != host) {
                Fail("round trip of " + std::to_string(bytes) + " bytes changed the data", err, err_len);
                return 1;
            }
        }
        return NERT_OK;
    } catch (const std::exception& e) {
        Fail(e.what(), err, err_len);
        return NERT_OTHER_ERROR;
    }
}

// One Model on a counting HipDevice wrapper: construction, a Run in which
// `throw_op`'s row throws, then `good_runs` normal Runs. counts receives, in
// order: after construction {allocate, release, live, h2d_calls, h2d_bytes},
// after the failed Run the same five, after the last good Run the same five,
// after destruction the same five (20 values). The good Runs' outputs go to
// `outputs`; the failed Run's message to `err` (NERT_OK overall when the
// failed Run threw and the good ones did not).
int contract_throw_then_run(const void* graph_handle, int n_inputs, const nert_tensor_desc* inputs, int n_outputs,
                            const nert_tensor_desc* outputs, const char* throw_op, int good_runs, int64_t* counts,
                            char* err, int err_len) {
    try {
        const nert::Graph& graph = *static_cast<const nert::Graph*>(graph_handle);
        nert::ShapeMap dims;
        const nert::HostTensorMap host = HostInputs(graph, n_inputs, inputs, &dims);
        ProbeDevice probe;
        auto snap = [&](int at) {
            const Counts& c = probe.counts;
            const int64_t v[5] = {c.allocate_calls, c.release_calls, c.live, c.h2d_calls, c.h2d_bytes};
            std::memcpy(counts + 5 * at, v, sizeof(v));
        };
        std::string thrown;
        {
            nert::Model model(graph, dims, probe);
            snap(0);
            g_throw_op = throw_op != nullptr ? throw_op : "";
            try {
                (void)model.RunTyped(host);
            } catch (const nert::InferenceException& e) {
                thrown = e.what();
            }
            g_throw_op.clear();
            snap(1);
            nert::HostTensorMap result;
            for (int r = 0; r < good_runs; ++r) {
                result = model.RunTyped(host);
            }
            snap(2);
            if (good_runs > 0) {
                CopyOutputs(graph, result, n_outputs, outputs);
            }
        }
        snap(3);
        Fail(thrown, err, err_len);
        return thrown.empty() ? NERT_OTHER_ERROR : NERT_OK;
    } catch (const std::exception& e) {
        g_throw_op.clear();
        Fail(e.what(), err, err_len);
        return NERT_OTHER_ERROR;
    }
}

// One Model on HipDevice() run twice: first on `bad` inputs (expected to be
// rejected by a row with a data-dependent check), then on `good` inputs,
// whose outputs are returned. The first Run's message goes to `err`;
// returns NERT_OK when the first Run threw and the second did not.
int contract_reject_then_run(const void* graph_handle, int n_inputs, const nert_tensor_desc* bad,
                             const nert_tensor_desc* good, int n_outputs, const nert_tensor_desc* outputs, char* err,
                             int err_len) {
    try {
        const nert::Graph& graph = *static_cast<const nert::Graph*>(graph_handle);
        nert::ShapeMap dims;
        const nert::HostTensorMap bad_host = HostInputs(graph, n_inputs, bad, &dims);
        const nert::HostTensorMap good_host = HostInputs(graph, n_inputs, good, nullptr);
        nert::Model model(graph, dims, nert::HipDevice());
        std::string thrown;
        try {
            (void)model.RunTyped(bad_host);
        } catch (const nert::InferenceException& e) {
            thrown = e.what();
        }
        CopyOutputs(graph, model.RunTyped(good_host), n_outputs, outputs);
        Fail(thrown, err, err_len);
        return thrown.empty() ? NERT_OTHER_ERROR : NERT_OK;
    } catch (const std::exception& e) {
        Fail(e.what(), err, err_len);
        return NERT_OTHER_ERROR;
    }
}

// FoldConstants(graph, CpuDevice()) on a copy of the graph, then
// Model(folded, dims, HipDevice()).RunTyped. *folded receives the count of
// folded nodes and *nodes_left the node count the drop-in ran.
int contract_fold_then_run(const void* graph_handle, int n_inputs, const nert_tensor_desc* inputs, int n_outputs,
                           const nert_tensor_desc* outputs, int* folded, int* nodes_left, char* err, int err_len) {
    try {
        nert::Graph graph = *static_cast<const nert::Graph*>(graph_handle);
        *folded = nert::FoldConstants(graph, nert::CpuDevice());
        *nodes_left = static_cast<int>(graph.nodes.size());
        nert::ShapeMap dims;
        const nert::HostTensorMap host = HostInputs(graph, n_inputs, inputs, &dims);
        nert::Model model(graph, dims, nert::HipDevice());
        CopyOutputs(graph, model.RunTyped(host), n_outputs, outputs);
        return NERT_OK;
    } catch (const nert::InferenceException& e) {
        Fail(e.what(), err, err_len);
        return NERT_INFERENCE_ERROR;
    } catch (const std::exception& e) {
        Fail(e.what(), err, err_len);
        return NERT_OTHER_ERROR;
    }
}

} // extern "C"
