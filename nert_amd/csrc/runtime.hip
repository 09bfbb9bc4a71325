// Device runtime behind the C-ABI: device selection, the launch stream,
// memory, transfers, events, workspace and the last-error string.
//
// One process-lifetime context on device 0, as NERT's seam expects
// (src/hip_device.cpp:33-44 pins ordinal 0). All kernels and transfers are
// ordered on one stream, created at default priority, so the only host/device
// synchronisation points are blocking transfers and explicit syncs.

#include "common.hpp"
#include "workspace_book.hpp"
#include "../../include/nert_hip.h"

#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace nert_hip {
namespace {

thread_local std::string g_last_error;

struct Context {
    bool ready = false;
    hipStream_t stream = nullptr;
    void* workspace[kWorkspaceSlots] = {};
    int64_t workspace_bytes[kWorkspaceSlots] = {};
    WorkspaceBook book;  // replaced workspaces stay alive while graph execs may use them
    int32_t* flags = nullptr;
    uint32_t* tile_counters = nullptr;
};

Context& Ctx() {
    static Context ctx;
    return ctx;
}

std::mutex& Mutex() {
    static std::mutex m;
    return m;
}

void EnsureReady() {
    Context& ctx = Ctx();
    if (ctx.ready) {
        return;
    }
    std::lock_guard<std::mutex> lock(Mutex());
    if (ctx.ready) {
        return;
    }
    int count = 0;
    Check(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (count <= 0) {
        throw Error("no HIP device found");
    }
    Check(hipSetDevice(0), "hipSetDevice");
    Check(hipStreamCreateWithFlags(&ctx.stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    Check(hipMalloc(reinterpret_cast<void**>(&ctx.flags), 64), "hipMalloc(flags)");
    Check(hipMemsetAsync(ctx.flags, 0, 64, ctx.stream), "hipMemsetAsync(flags)");
    Check(hipMalloc(reinterpret_cast<void**>(&ctx.tile_counters), kTileCounters * sizeof(uint32_t)),
          "hipMalloc(tile counters)");
    Check(hipMemsetAsync(ctx.tile_counters, 0, kTileCounters * sizeof(uint32_t), ctx.stream),
          "hipMemsetAsync(tile counters)");
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    TopkScratchSetup();
    ctx.ready = true;
}

} // namespace

bool RuntimeReady() { return Ctx().ready; }

void SetLastError(const std::string& message) { g_last_error = message; }

hipStream_t DefaultStream() {
    EnsureReady();
    return Ctx().stream;
}

void* Workspace(int64_t bytes, hipStream_t stream, int slot) {
    EnsureReady();
    if (slot < 0 || slot >= kWorkspaceSlots) {
        throw Error("workspace slot out of range");
    }
    Context& ctx = Ctx();
    if (bytes <= ctx.workspace_bytes[slot]) {
        return ctx.workspace[slot];
    }
    // Grow geometrically; the old buffer may still be read by queued work.
    int64_t want = ctx.workspace_bytes[slot] * 2;
    if (want < bytes) {
        want = bytes;
    }
    want = (want + 0xFFFFF) & ~static_cast<int64_t>(0xFFFFF);
    void* grown = nullptr;
    Check(hipMalloc(&grown, static_cast<size_t>(want)), "hipMalloc(workspace)");
    std::lock_guard<std::mutex> lock(Mutex());
    const std::vector<void*> free_now = ctx.book.Replaced(ctx.workspace[slot]);
    if (!free_now.empty()) {
        Check(hipStreamSynchronize(stream), "hipStreamSynchronize(workspace)");
        Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize(workspace)");
        for (void* p : free_now) {
            Check(hipFree(p), "hipFree(workspace)");
        }
    }
    ctx.workspace[slot] = grown;
    ctx.workspace_bytes[slot] = want;
    return grown;
}

int32_t* ErrorFlags() {
    EnsureReady();
    return Ctx().flags;
}

int32_t& PendingErrorFlags() {
    static int32_t pending = 0;
    return pending;
}

uint32_t* TileCounters(int64_t count) {
    EnsureReady();
    static const bool enabled = [] {
        const char* v = std::getenv("NERT_HIP_SPLIT_FIXUP");
        return v == nullptr || std::strcmp(v, "0") != 0;
    }();
    return enabled && count >= 0 && count <= kTileCounters ? Ctx().tile_counters : nullptr;
}

void GraphCreated() {
    std::lock_guard<std::mutex> lock(Mutex());
    Ctx().book.GraphCreated();
}

void GraphDestroyed() {
    std::vector<void*> free_now;
    {
        std::lock_guard<std::mutex> lock(Mutex());
        free_now = Ctx().book.GraphDestroyed();
    }
    if (!free_now.empty()) {
        Check(hipStreamSynchronize(Ctx().stream), "hipStreamSynchronize(workspace)");
        for (void* p : free_now) {
            Check(hipFree(p), "hipFree(workspace)");
        }
    }
}

namespace {

constexpr int64_t kShadowMaxBytes = 64 * 1024;

struct ShadowStore {
    std::mutex mutex;
    std::map<uintptr_t, std::vector<uint8_t>> entries;

    // Removes every entry overlapping [addr, addr + bytes). Caller holds mutex.
    void DropLocked(uintptr_t addr, int64_t bytes) {
        if (entries.empty() || bytes <= 0) {
            return;
        }
        auto it = entries.upper_bound(addr);
        if (it != entries.begin()) {
            auto prev = std::prev(it);
            if (prev->first + prev->second.size() > addr) {
                it = prev;
            }
        }
        while (it != entries.end() && it->first < addr + static_cast<uintptr_t>(bytes)) {
            it = entries.erase(it);
        }
    }
};

ShadowStore& Shadows() {
    static ShadowStore store;
    return store;
}

} // namespace

void ShadowPut(const void* dst, const void* src, int64_t bytes) {
    ShadowStore& s = Shadows();
    std::lock_guard<std::mutex> lock(s.mutex);
    s.DropLocked(reinterpret_cast<uintptr_t>(dst), bytes);
    if (bytes <= 0 || bytes > kShadowMaxBytes) {
        return;
    }
    const auto* p = static_cast<const uint8_t*>(src);
    s.entries[reinterpret_cast<uintptr_t>(dst)] = std::vector<uint8_t>(p, p + bytes);
}

void ShadowDrop(const void* dst, int64_t bytes) {
    ShadowStore& s = Shadows();
    std::lock_guard<std::mutex> lock(s.mutex);
    s.DropLocked(reinterpret_cast<uintptr_t>(dst), bytes);
}

bool ShadowGet(const void* src, int64_t bytes, void* out) {
    ShadowStore& s = Shadows();
    std::lock_guard<std::mutex> lock(s.mutex);
    const auto it = s.entries.find(reinterpret_cast<uintptr_t>(src));
    if (it == s.entries.end() || static_cast<int64_t>(it->second.size()) < bytes) {
        return false;
    }
    std::memcpy(out, it->second.data(), static_cast<size_t>(bytes));
    return true;
}

namespace {

// Pinned bounce buffers for transfers from and to pageable host memory.
//
// A pageable copy cannot be DMA'd directly; the runtime stages it through its
// own buffers one piece at a time. Here the copy is cut into pieces (the
// first kStageFirst bytes, doubling up to kStageChunk) dealt round-robin to
// kStageLanes host threads. Each lane owns two pinned slots (hipHostMalloc,
// allocated once, kept until the process ends): H2D, the lane memcpy's a
// piece into a free slot and queues the slot's DMA, then fills its other slot
// while that DMA runs; D2H, the lane queues the next piece's DMA before
// copying the finished one out. Host memcpy and PCIe DMA overlap, and the
// lanes' memcpy's run in parallel. Measured on MI355X for 18-38 MiB copies:
// H2D 37-41 GB/s (the runtime's own pageable path 30-36), D2H 34-40 GB/s
// (17.7), pinned-to-device 56 GB/s. Copies whose host side is already pinned
// (or below kStageMin) go straight to hipMemcpyAsync. NERT_HIP_STAGING=0
// turns staging off (every copy a plain hipMemcpyAsync).
constexpr int64_t kStageChunk = 4 << 20;
constexpr int64_t kStageFirst = 1 << 20;
constexpr int kStageLanes = 2;
constexpr int64_t kStageMin = 1 << 20;

struct Staging {
    std::mutex mutex;  // one staged transfer at a time
    bool ready = false;
    void* slot[2 * kStageLanes] = {};
    hipEvent_t done[2 * kStageLanes] = {};
};

Staging& Stage() {
    static Staging st;
    return st;
}

bool StagingEnabled() {
    const char* v = std::getenv("NERT_HIP_STAGING");
    return v == nullptr || std::strcmp(v, "0") != 0;
}

bool HostIsPinned(const void* p) {
    hipPointerAttribute_t attr{};
    const hipError_t rc = hipPointerGetAttributes(&attr, p);
    if (rc != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeHost;
}

void EnsureStaging(Staging& st) {
    if (st.ready) {
        return;
    }
    for (int i = 0; i < 2 * kStageLanes; ++i) {
        Check(hipHostMalloc(&st.slot[i], static_cast<size_t>(kStageChunk), hipHostMallocDefault),
              "hipHostMalloc(staging)");
        Check(hipEventCreateWithFlags(&st.done[i], hipEventDisableTiming), "hipEventCreate(staging)");
    }
    st.ready = true;
}

// Piece boundaries of a staged copy: sizes double from kStageFirst up to
// kStageChunk, so the first DMA starts after a short memcpy and the steady
// state moves large pieces (each DMA carries a fixed submission cost).
std::vector<int64_t> StagePieces(int64_t bytes) {
    std::vector<int64_t> starts;
    int64_t piece = kStageFirst < kStageChunk ? kStageFirst : kStageChunk;
    for (int64_t off = 0; off < bytes; off += piece, piece = piece * 2 < kStageChunk ? piece * 2 : kStageChunk) {
        starts.push_back(off);
    }
    starts.push_back(bytes);
    return starts;
}

// Runs lane(0..lanes-1) on the calling thread and lanes-1 helper threads;
// rethrows the first lane error after all lanes have stopped.
template <class Lane>
void RunLanes(int lanes, Lane lane) {
    std::vector<std::string> errors(static_cast<size_t>(lanes));
    auto guarded = [&](int t) {
        try {
            lane(t);
        } catch (const std::exception& e) {
            errors[static_cast<size_t>(t)] = e.what();
        }
    };
    std::vector<std::thread> helpers;
    for (int t = 1; t < lanes; ++t) {
        helpers.emplace_back(guarded, t);
    }
    guarded(0);
    for (auto& h : helpers) {
        h.join();
    }
    for (const auto& e : errors) {
        if (!e.empty()) {
            throw Error(e);
        }
    }
}

void StagedH2D(char* dst, const char* src, int64_t bytes, hipStream_t s) {
    Staging& st = Stage();
    std::lock_guard<std::mutex> lock(st.mutex);
    EnsureStaging(st);
    const std::vector<int64_t> at = StagePieces(bytes);
    const int64_t pieces = static_cast<int64_t>(at.size()) - 1;
    const int lanes = static_cast<int>(pieces < kStageLanes ? pieces : kStageLanes);
    RunLanes(lanes, [&](int t) {
        int k = 0;
        for (int64_t c = t; c < pieces; c += lanes, ++k) {
            const int slot = 2 * t + (k & 1);
            const int64_t off = at[static_cast<size_t>(c)];
            const int64_t n = at[static_cast<size_t>(c) + 1] - off;
            if (k >= 2) {
                Check(hipEventSynchronize(st.done[slot]), "hipEventSynchronize(staging)");
            }
            std::memcpy(st.slot[slot], src + off, static_cast<size_t>(n));
            Check(hipMemcpyAsync(dst + off, st.slot[slot], static_cast<size_t>(n), hipMemcpyHostToDevice, s),
                  "hipMemcpyAsync(H2D)");
            Check(hipEventRecord(st.done[slot], s), "hipEventRecord(staging)");
        }
    });
    Check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

void StagedD2H(char* dst, const char* src, int64_t bytes, hipStream_t s) {
    Staging& st = Stage();
    std::lock_guard<std::mutex> lock(st.mutex);
    EnsureStaging(st);
    const std::vector<int64_t> at = StagePieces(bytes);
    const int64_t pieces = static_cast<int64_t>(at.size()) - 1;
    const int lanes = static_cast<int>(pieces < kStageLanes ? pieces : kStageLanes);
    RunLanes(lanes, [&](int t) {
        auto issue = [&](int64_t c, int slot) {
            const int64_t off = at[static_cast<size_t>(c)];
            const int64_t n = at[static_cast<size_t>(c) + 1] - off;
            Check(hipMemcpyAsync(st.slot[slot], src + off, static_cast<size_t>(n), hipMemcpyDeviceToHost, s),
                  "hipMemcpyAsync(D2H)");
            Check(hipEventRecord(st.done[slot], s), "hipEventRecord(staging)");
        };
        int k = 0;
        issue(t, 2 * t);
        for (int64_t c = t; c < pieces; c += lanes, ++k) {
            const int slot = 2 * t + (k & 1);
            if (c + lanes < pieces) {
                issue(c + lanes, 2 * t + ((k + 1) & 1));
            }
            Check(hipEventSynchronize(st.done[slot]), "hipEventSynchronize(staging)");
            const int64_t off = at[static_cast<size_t>(c)];
            std::memcpy(dst + off, st.slot[slot], static_cast<size_t>(at[static_cast<size_t>(c) + 1] - off));
        }
    });
}

bool UseStaging(const void* host, int64_t bytes) {
    return bytes >= kStageMin && StagingEnabled() && !HostIsPinned(host);
}

} // namespace

} // namespace nert_hip

using nert_hip::Guard;

extern "C" {

const char* nert_hip_last_error(void) { return nert_hip::g_last_error.c_str(); }

int nert_hip_init(void) {
    return Guard([] { nert_hip::EnsureReady(); });
}

int nert_hip_device_count(int* count) {
    return Guard([&] {
        int n = 0;
        const hipError_t status = hipGetDeviceCount(&n);
        *count = status == hipSuccess ? n : 0;
    });
}

void* nert_hip_malloc(int64_t bytes) {
    if (bytes <= 0) {
        return nullptr;
    }
    void* ptr = nullptr;
    const int rc = Guard([&] {
        nert_hip::EnsureReady();
        nert_hip::Check(hipMalloc(&ptr, static_cast<size_t>(bytes)), "hipMalloc");
    });
    return rc == 0 ? ptr : nullptr;
}

int nert_hip_free(void* ptr) {
    if (ptr == nullptr) {
        return 0;
    }
    return Guard([&] {
        nert_hip::Check(hipStreamSynchronize(nert_hip::DefaultStream()), "hipStreamSynchronize");
        hipDeviceptr_t base = nullptr;
        size_t size = 0;
        if (hipMemGetAddressRange(&base, &size, ptr) == hipSuccess) {
            nert_hip::ShadowDrop(ptr, static_cast<int64_t>(size));
        } else {
            (void)hipGetLastError();
        }
        nert_hip::Check(hipFree(ptr), "hipFree");
    });
}

void* nert_hip_host_alloc(int64_t bytes) {
    if (bytes <= 0) {
        return nullptr;
    }
    void* ptr = nullptr;
    const int rc = Guard([&] {
        nert_hip::EnsureReady();
        nert_hip::Check(hipHostMalloc(&ptr, static_cast<size_t>(bytes), hipHostMallocDefault), "hipHostMalloc");
    });
    return rc == 0 ? ptr : nullptr;
}

int nert_hip_host_free(void* ptr) {
    if (ptr == nullptr) {
        return 0;
    }
    return Guard([&] {
        nert_hip::Check(hipStreamSynchronize(nert_hip::DefaultStream()), "hipStreamSynchronize");
        nert_hip::Check(hipHostFree(ptr), "hipHostFree");
    });
}

int nert_hip_memcpy_h2d(void* dst, const void* src, int64_t bytes) {
    if (bytes == 0) {
        return 0;
    }
    return Guard([&] {
        hipStream_t s = nert_hip::DefaultStream();
        if (nert_hip::UseStaging(src, bytes)) {
            nert_hip::StagedH2D(static_cast<char*>(dst), static_cast<const char*>(src), bytes, s);
        } else {
            nert_hip::Check(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyHostToDevice, s),
                            "hipMemcpyAsync(H2D)");
            nert_hip::Check(hipStreamSynchronize(s), "hipStreamSynchronize");
        }
        nert_hip::ShadowPut(dst, src, bytes);
    });
}

int nert_hip_memcpy_d2h(void* dst, const void* src, int64_t bytes) {
    if (bytes == 0) {
        return 0;
    }
    return Guard([&] {
        hipStream_t s = nert_hip::DefaultStream();
        if (nert_hip::UseStaging(dst, bytes)) {
            nert_hip::StagedD2H(static_cast<char*>(dst), static_cast<const char*>(src), bytes, s);
        } else {
            nert_hip::Check(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyDeviceToHost, s),
                            "hipMemcpyAsync(D2H)");
            nert_hip::Check(hipStreamSynchronize(s), "hipStreamSynchronize");
        }
    });
}

int nert_hip_forget_host_shadow(const void* ptr, int64_t bytes) {
    return Guard([&] { nert_hip::ShadowDrop(ptr, bytes); });
}

int nert_hip_memcpy_d2d(void* dst, const void* src, int64_t bytes, void* stream) {
    if (bytes == 0) {
        return 0;
    }
    return Guard([&] {
        nert_hip::ShadowDrop(dst, bytes);
        nert_hip::Check(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyDeviceToDevice,
                                       nert_hip::StreamOr(stream)),
                        "hipMemcpyAsync(D2D)");
    });
}

void* nert_hip_default_stream(void) {
    void* s = nullptr;
    (void)Guard([&] { s = nert_hip::DefaultStream(); });
    return s;
}

int nert_hip_stream_sync(void* stream) {
    return Guard([&] { nert_hip::Check(hipStreamSynchronize(nert_hip::StreamOr(stream)), "hipStreamSynchronize"); });
}

void* nert_hip_event_create(void) {
    hipEvent_t e = nullptr;
    const int rc = Guard([&] {
        nert_hip::EnsureReady();
        nert_hip::Check(hipEventCreate(&e), "hipEventCreate");
    });
    return rc == 0 ? static_cast<void*>(e) : nullptr;
}

int nert_hip_event_record(void* event, void* stream) {
    return Guard([&] {
        nert_hip::Check(hipEventRecord(static_cast<hipEvent_t>(event), nert_hip::StreamOr(stream)), "hipEventRecord");
    });
}

int nert_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
    return Guard([&] {
        nert_hip::Check(hipEventSynchronize(static_cast<hipEvent_t>(stop)), "hipEventSynchronize");
        nert_hip::Check(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
                        "hipEventElapsedTime");
    });
}

int nert_hip_event_destroy(void* event) {
    return Guard([&] { nert_hip::Check(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy"); });
}

int nert_hip_capture_begin(void) {
    return Guard([&] {
        // The graph's deferred checks report through the error word: start
        // it cleared (eagerly, before the capture; no memset node is
        // recorded into the graph). Bits that eager rows raised before the
        // capture are kept in the host-side pending mask, so the next
        // nert_hip_take_error_flags still reports them.
        hipStream_t s = nert_hip::DefaultStream();
        int32_t raised = 0;
        nert_hip::Check(hipMemcpyAsync(&raised, nert_hip::ErrorFlags(), sizeof(raised), hipMemcpyDeviceToHost, s),
                        "hipMemcpyAsync(flags)");
        nert_hip::Check(hipStreamSynchronize(s), "hipStreamSynchronize");
        nert_hip::PendingErrorFlags() |= raised;
        const int32_t zero = 0;
        nert_hip::Check(hipMemcpyAsync(nert_hip::ErrorFlags(), &zero, sizeof(zero), hipMemcpyHostToDevice, s),
                        "hipMemcpyAsync(flags)");
        nert_hip::Check(hipStreamSynchronize(s), "hipStreamSynchronize");
        nert_hip::Check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    });
}

int nert_hip_capture_end(void** graph_exec) {
    return Guard([&] {
        *graph_exec = nullptr;
        hipGraph_t graph = nullptr;
        nert_hip::Check(hipStreamEndCapture(nert_hip::DefaultStream(), &graph), "hipStreamEndCapture");
        hipGraphExec_t exec = nullptr;
        const hipError_t status = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        nert_hip::Check(status, "hipGraphInstantiate");
        nert_hip::GraphCreated();
        *graph_exec = exec;
    });
}

int nert_hip_graph_launch(void* graph_exec, void* stream) {
    return Guard([&] {
        nert_hip::Check(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), nert_hip::StreamOr(stream)),
                        "hipGraphLaunch");
    });
}

int nert_hip_graph_destroy(void* graph_exec) {
    if (graph_exec == nullptr) {
        return 0;
    }
    return Guard([&] {
        nert_hip::Check(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)), "hipGraphExecDestroy");
        nert_hip::GraphDestroyed();
    });
}

} // extern "C"
