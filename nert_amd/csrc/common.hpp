#pragma once
// Shared helpers for the gfx950 kernels and the C-ABI wrappers.
//
// Every C-ABI entry point returns 0 on success or a non-zero status with a
// message retrievable through nert_hip_last_error(); internal code reports
// failures by throwing nert_hip::Error, which the wrappers convert.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace nert_hip {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void SetLastError(const std::string& message);

inline void Check(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        throw Error(std::string(what) + " failed: " + hipGetErrorString(status));
    }
}

// The launch stream every entry point uses when the caller passes null.
hipStream_t DefaultStream();

inline hipStream_t StreamOr(void* stream) {
    return stream != nullptr ? static_cast<hipStream_t>(stream) : DefaultStream();
}

// Reusable device workspaces on the default device: each slot grows on
// demand (a stream-synchronised reallocation), never shrinks. Kernels that
// need scratch (split-K partials, TopK candidates, error flags) take slot 0;
// a row that keeps an intermediate alive across a GEMM launch (which may take
// slot 0 for its partials) holds it in slot 1.
constexpr int kWorkspaceSlots = 2;
void* Workspace(int64_t bytes, hipStream_t stream, int slot = 0);

// A 64-byte device flag block (zeroed at creation) used by rows that must
// report data-dependent errors (out-of-range indices, integer division by
// zero) back to the host.
int32_t* ErrorFlags();
// Bits read off the device word when a capture began (raised by eager rows
// before it); the next nert_hip_take_error_flags reports and clears them.
int32_t& PendingErrorFlags();
// Tile counters for kernels whose workgroups finish a tile's split sum among
// themselves (the last one to arrive reduces; FinishSplitTile in
// mfma_tile.hpp, used by the conv and GEMM kernels): kTileCounters words,
// zeroed once at set-up, and every launch that uses them leaves them zero.
// Null when `count` exceeds the capacity or NERT_HIP_SPLIT_FIXUP=0 (the
// caller then runs its separate reduce kernel). Launches on one stream never
// overlap; kernels on different streams that both use them race, as they do
// on the workspaces.
constexpr int64_t kTileCounters = 1 << 16;
uint32_t* TileCounters(int64_t count);
// True once the device, stream and error word are set up (nert_hip_init).
bool RuntimeReady();
// Set-up of the fixed scratch of nert_hip_topk_f32_noalloc (topk.hip), run by
// the runtime's initialisation with the device current.
void TopkScratchSetup();
// Live graph execs keep replaced workspaces alive (workspace_book.hpp).
void GraphCreated();
void GraphDestroyed();

// Host shadows of small host-to-device uploads (<= 64 KiB), keyed by device
// address. nert_hip_memcpy_h2d records them; device-side writes that go
// through the runtime (d2d copies, frees, seam row outputs) drop overlapping
// entries. Rows use them to read control operands without a D2H round trip.
void ShadowPut(const void* dst, const void* src, int64_t bytes);
void ShadowDrop(const void* dst, int64_t bytes);
bool ShadowGet(const void* src, int64_t bytes, void* out);

// Unsigned division by a runtime divisor via multiply-high and shift
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994): q = (umulhi(n, m) + n) >> s, exact for all
// 32-bit n when evaluated in 64 bits. Kernels whose index space fits 32 bits
// decode multi-dimensional indices with it instead of 64-bit division.
struct FastDiv {
    uint32_t d;
    uint32_t m;
    uint32_t s;
    static FastDiv Make(uint32_t d) {
        FastDiv f{d, 0, 0};
        if (d > 1) {
            uint32_t l = 0;
            while ((uint64_t{1} << l) < d) {
                ++l;
            }
            f.s = l;
            f.m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1);
        }
        return f;
    }
    __device__ __forceinline__ uint32_t Div(uint32_t n) const {
        return static_cast<uint32_t>((static_cast<uint64_t>(__umulhi(n, m)) + n) >> s);
    }
};

// Quotient and remainder of a 32-bit index by FastDiv `f`.
__device__ __forceinline__ uint32_t DivMod(const FastDiv& f, uint32_t n, uint32_t& rem) {
    const uint32_t q = f.Div(n);
    rem = n - q * f.d;
    return q;
}

inline unsigned GridFor(int64_t work, int per_block, int64_t cap = 1 << 20) {
    int64_t blocks = (work + per_block - 1) / per_block;
    if (blocks < 1) {
        blocks = 1;
    }
    if (blocks > cap) {
        blocks = cap;
    }
    return static_cast<unsigned>(blocks);
}

// Number of K splits for a tiled GEMM-shaped launch. The grid should fill
// the blocks the chip holds at once (`resident`, e.g. 256 CUs x 2) without
// spilling into a second, partly empty round; each split keeps at least
// `min_k_tiles` K tiles so the pipeline prologue stays amortised.
inline int PlanSplits(int64_t tiles, int64_t k_tiles, int64_t resident, int64_t min_k_tiles, int max_splits = 16) {
    int splits = 1;
    while (splits < max_splits && tiles * splits * 2 <= resident && k_tiles >= min_k_tiles * splits * 2) {
        splits *= 2;
    }
    return splits;
}

// Blocks of one 256-thread MFMA tile kernel the chip keeps resident
// (256 CUs, two such blocks per CU at the engine's register use).
constexpr int64_t kResidentBlocks = 512;

// Runs `body` and converts exceptions into a C status code.
template <typename F>
int Guard(F&& body) {
    try {
        body();
        return 0;
    } catch (const std::exception& e) {
        SetLastError(e.what());
        return 1;
    }
}

inline void CheckLaunch(const char* what) { Check(hipGetLastError(), what); }

} // namespace nert_hip

// Sigmoid as the Sigmoid row and the fused SiLU epilogue both compute it:
// 1 / (1 + exp(-x)) (src/kernels/sigmoid.cpp:52) with the hardware
// reciprocal (v_rcp_f32, within 1 ulp) in place of an IEEE division, which
// costs ten instructions; one definition, so the fused and separate rows
// agree bit for bit.
__device__ __forceinline__ float SigmoidF32(float x) { return __builtin_amdgcn_rcpf(__fadd_rn(1.0f, expf(-x))); }

// Device-side vector types for the MFMA builtins.
typedef float nert_floatx2 __attribute__((ext_vector_type(2)));
typedef float nert_floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int nert_uintx4 __attribute__((ext_vector_type(4)));
typedef float nert_floatx16 __attribute__((ext_vector_type(16)));
