// TopK (largest = 1, sorted = 1) along an axis of a float32 tensor.
//
// Order (src/kernels/top_k.cpp:125-134): value descending, equal values by
// ascending index (-0.0 and +0.0 compare equal). Every element gets a unique
// 64-bit key
//     key = orderable(value) << 32 | (0xFFFFFFFF - index)
// where orderable() maps float bits to an unsigned integer with the float
// order (-0.0 folded onto +0.0, NaN above +inf), so "descending key" is
// exactly the reference's order and there are no ties left.
//
// Rows of up to kSmallRow elements sort in one workgroup's LDS. Longer rows
// (the detector's [8, 672000], K = 300) run a radix select over the key,
// 8 bits per pass from the top, with many workgroups per row: each pass builds
// a 256-bin histogram of the keys that still match the chosen prefix (one LDS
// histogram per wave, so the waves do not contend for the same bins), and
// every workgroup of the next pass (or of the collection) scans the previous
// pass's histogram itself and picks the bin holding the K-th largest key, so
// a pass is one launch. When that bin is needed whole the threshold is final
// and later passes return at once. Keys >= threshold (exactly K per row) are
// collected and ordered -- by rank (the count of larger keys, spread over
// several workgroups per row) when K <= 1024, else in 4096-key LDS runs
// merged by per-key binary search -- and written out.

#include "common.hpp"
#include "../../include/nert_hip.h"

namespace nert_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kSmallRow = 4096;
constexpr int kRun = 4096;

struct RowGeom {
    int64_t dim;
    int64_t inner;
    int64_t k;
    int32_t vec; // rows contiguous, 16-byte aligned, chunks of whole quads: 16-byte loads
};

// Calls visit(i, x[base + i * inner]) for i in [begin, end) of a row, one
// element per thread per step, or (vec) one 16-byte quad per thread per step.
template <class Visit>
__device__ __forceinline__ void ForRowRange(const float* __restrict__ x, const RowGeom& g, int64_t base, int64_t begin,
                                            int64_t end, Visit visit) {
    if (g.vec) {
        const nert_floatx4* q = reinterpret_cast<const nert_floatx4*>(x + base);
        for (int64_t i = begin + 4 * threadIdx.x; i < end; i += 4 * blockDim.x) {
            const nert_floatx4 v = q[i / 4];
            visit(i, v[0]);
            visit(i + 1, v[1]);
            visit(i + 2, v[2]);
            visit(i + 3, v[3]);
        }
    } else {
        for (int64_t i = begin + threadIdx.x; i < end; i += blockDim.x) {
            visit(i, x[base + i * g.inner]);
        }
    }
}

__device__ __forceinline__ int64_t RowBase(int64_t row, const RowGeom& g) {
    const int64_t o = row / g.inner;
    const int64_t n = row - o * g.inner;
    return o * g.dim * g.inner + n;
}

__device__ __forceinline__ uint64_t KeyOf(float v, int64_t index) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7FFFFFFFu) == 0) {
        b = 0; // -0.0 == +0.0
    }
    uint32_t ord;
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) {
        ord = 0xFFFFFFFFu; // NaN: above +inf
    } else {
        ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    }
    return (static_cast<uint64_t>(ord) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(index));
}

__device__ __forceinline__ int64_t IndexOf(uint64_t key) {
    return static_cast<int64_t>(0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFu));
}

// Descending bitonic sort of n (a power of two) keys in LDS.
__device__ void BitonicDesc(uint64_t* s, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < n / 2; i += blockDim.x) {
                const int lo = 2 * stride * (i / stride) + (i % stride);
                const int hi = lo + stride;
                const bool up = (lo & size) == 0;
                const uint64_t a = s[lo];
                const uint64_t b = s[hi];
                if ((a < b) == up) {
                    s[lo] = b;
                    s[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ void WriteOut(const float* x, float* values, int64_t* indices, int64_t row, int64_t t,
                                         uint64_t key, const RowGeom& g) {
    const int64_t idx = IndexOf(key);
    const int64_t o = row / g.inner;
    const int64_t n = row - o * g.inner;
    const int64_t dst = (o * g.k + t) * g.inner + n;
    values[dst] = x[RowBase(row, g) + idx * g.inner];
    indices[dst] = idx;
}

// One workgroup per row: the whole row sorts in LDS.
__global__ void __launch_bounds__(kThreads) SmallRowKernel(const float* __restrict__ x, float* __restrict__ values,
                                                           int64_t* __restrict__ indices, RowGeom g, int n_pow2) {
    __shared__ uint64_t s[kSmallRow];
    const int64_t row = blockIdx.x;
    const int64_t base = RowBase(row, g);
    for (int i = threadIdx.x; i < n_pow2; i += blockDim.x) {
        s[i] = i < g.dim ? KeyOf(x[base + i * g.inner], i) : 0;
    }
    __syncthreads();
    BitonicDesc(s, n_pow2);
    for (int t = threadIdx.x; t < g.k; t += blockDim.x) {
        WriteOut(x, values, indices, row, t, s[t], g);
    }
}

// ---- long rows: radix select ----------------------------------------------

struct SelectState {
    uint64_t prefix; // chosen high bits of the threshold key
    int64_t remaining; // keys still to take from inside the prefix
    int32_t done;
    int32_t count; // collected keys
};

// Select state and histograms of the passes, per row: the state a pass
// selects with goes to st[pass & 1] (written by the row's first workgroup of
// the next pass), and pass p counts into hist[p % 3] while hist[(p + 1) % 3]
// is cleared for pass p + 1 (nobody reads it during pass p).
struct SelectBuffers {
    SelectState* st[2];
    uint32_t* hist[3];
};

__global__ void InitSelectKernel(SelectBuffers b, int64_t rows, int64_t k) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < rows * 256; i += stride) {
        b.hist[0][i] = 0;
        b.hist[1][i] = 0;
        b.hist[2][i] = 0;
        if (i < rows) {
            b.st[0][i].prefix = 0;
            b.st[0][i].remaining = k;
            b.st[0][i].done = 0;
            b.st[0][i].count = 0;
        }
    }
}

// The state after a pass: its histogram (256 digits) scanned from the top
// digit down, the chosen digit the one whose inclusive count first reaches
// `remaining`; when that digit's keys are all needed the threshold is final
// (done). Run by all 256 threads of a workgroup (one digit each: in-wave
// shuffles, then the four wave totals); every workgroup of the row gets the
// same state from the same counts. The result is in `out` (LDS) after the
// final barrier.
__device__ void NextState(const SelectState& s, const uint32_t* rh, int pass, SelectState* out) {
    __shared__ uint32_t totals[kThreads / 64];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const uint32_t count = rh[255 - t];
    uint32_t incl = count;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off, 64);
        if (lane >= off) {
            incl += y;
        }
    }
    if (lane == 63) {
        totals[wave] = incl;
    }
    if (t == 0) {
        *out = s;
    }
    __syncthreads();
    for (int w = 0; w < wave; ++w) {
        incl += totals[w];
    }
    const int64_t excl = static_cast<int64_t>(incl) - count;
    if (!s.done && excl < s.remaining && static_cast<int64_t>(incl) >= s.remaining) {
        SelectState ns = s;
        ns.prefix |= static_cast<uint64_t>(255 - t) << (56 - 8 * pass);
        ns.remaining = s.remaining - excl;
        if (static_cast<int64_t>(count) == ns.remaining) {
            ns.done = 1;
        }
        *out = ns;
    }
    __syncthreads();
}

// Pass `pass` over a chunk of a row: first the state to select with (pass
// 0: the initial one; later passes: the previous pass's state advanced by
// its histogram, NextState), then a 256-bin histogram of the keys that still
// match the chosen prefix (one LDS histogram per wave, so the waves do not
// contend for the same bins), added to the row's histogram for this pass.
// The row's first workgroup also records the state and clears the next
// pass's histogram. Once the threshold is final the pass returns at once.
__global__ void __launch_bounds__(kThreads) HistKernel(const float* __restrict__ x, RowGeom g, int64_t chunk,
                                                       int chunks, SelectBuffers sb, int pass) {
    const int64_t row = blockIdx.x / chunks;
    const int c = blockIdx.x - static_cast<int>(row * chunks);
    __shared__ SelectState cur;
    if (pass == 0) {
        if (threadIdx.x == 0) {
            cur = sb.st[0][row];
        }
        __syncthreads();
    } else {
        const SelectState prev = sb.st[(pass - 1) & 1][row];
        NextState(prev, sb.hist[(pass - 1) % 3] + row * 256, pass - 1, &cur);
        if (c == 0) {
            if (threadIdx.x == 0) {
                sb.st[pass & 1][row] = cur;
            }
            sb.hist[(pass + 1) % 3][row * 256 + threadIdx.x] = 0;
        }
    }
    const SelectState s = cur;
    if (s.done) {
        return;
    }
    __shared__ uint32_t h[kThreads / 64][256];
    const int wave = threadIdx.x >> 6;
    for (int w = 0; w < kThreads / 64; ++w) {
        h[w][threadIdx.x] = 0;
    }
    __syncthreads();
    const int shift = 56 - 8 * pass;
    const int64_t begin = c * chunk;
    int64_t end = begin + chunk;
    if (end > g.dim) {
        end = g.dim;
    }
    const int64_t base = RowBase(row, g);
    ForRowRange(x, g, base, begin, end, [&](int64_t i, float v) {
        const uint64_t key = KeyOf(v, i);
        // pass 0 has no prefix to match (a 64-bit shift would be undefined)
        const bool match = pass == 0 || (key >> (shift + 8)) == (s.prefix >> (shift + 8));
        if (match) {
            atomicAdd(&h[wave][(key >> shift) & 0xFF], 1u);
        }
    });
    __syncthreads();
    uint32_t v = 0;
    for (int w = 0; w < kThreads / 64; ++w) {
        v += h[w][threadIdx.x];
    }
    if (v != 0) {
        atomicAdd(&sb.hist[pass % 3][row * 256 + threadIdx.x], v);
    }
}

// Keys >= the final threshold (the state after the last pass, advanced by
// that pass's histogram here in every workgroup): exactly K per row.
__global__ void __launch_bounds__(kThreads) CollectKernel(const float* __restrict__ x, RowGeom g, int64_t chunk,
                                                          int chunks, SelectBuffers sb, int last_pass,
                                                          uint64_t* __restrict__ cand) {
    const int64_t row = blockIdx.x / chunks;
    const int c = blockIdx.x - static_cast<int>(row * chunks);
    __shared__ SelectState fin;
    NextState(sb.st[last_pass & 1][row], sb.hist[last_pass % 3] + row * 256, last_pass, &fin);
    const uint64_t threshold = fin.prefix;
    // The collected-key counter: st[0]'s count, zero since initialisation.
    int32_t* count = &sb.st[0][row].count;
    const int64_t begin = c * chunk;
    int64_t end = begin + chunk;
    if (end > g.dim) {
        end = g.dim;
    }
    const int64_t base = RowBase(row, g);
    ForRowRange(x, g, base, begin, end, [&](int64_t i, float v) {
        const uint64_t key = KeyOf(v, i);
        if (key >= threshold) {
            const int pos = atomicAdd(count, 1);
            if (pos < g.k) {
                cand[row * g.k + pos] = key;
            }
        }
    });
}

// Sorts runs of kRun candidates (descending) in LDS, in place.
__global__ void __launch_bounds__(kThreads) SortRunsKernel(uint64_t* cand, int64_t k, int runs_per_row, int n_pow2) {
    __shared__ uint64_t s[kRun];
    const int64_t row = blockIdx.x / runs_per_row;
    const int r = blockIdx.x - static_cast<int>(row * runs_per_row);
    uint64_t* p = cand + row * k + static_cast<int64_t>(r) * kRun;
    int64_t len = k - static_cast<int64_t>(r) * kRun;
    if (len > kRun) {
        len = kRun;
    }
    for (int i = threadIdx.x; i < n_pow2; i += blockDim.x) {
        s[i] = i < len ? p[i] : 0;
    }
    __syncthreads();
    BitonicDesc(s, n_pow2);
    for (int i = threadIdx.x; i < len; i += blockDim.x) {
        p[i] = s[i];
    }
}

// Merges pairs of sorted runs of `width`: a key's new place is its place in
// its run plus the number of keys of the partner run greater than it.
__global__ void MergeKernel(const uint64_t* __restrict__ src, uint64_t* __restrict__ dst, int64_t rows, int64_t k,
                            int64_t width) {
    const int64_t total = rows * k;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < total; e += stride) {
        const int64_t row = e / k;
        const int64_t i = e - row * k;
        const int64_t run = i / width;
        const int64_t pair_base = (run & ~int64_t{1}) * width;
        const int64_t pos = i - run * width;
        const int64_t partner = run ^ 1;
        int64_t p_begin = partner * width;
        int64_t p_end = p_begin + width;
        if (p_end > k) {
            p_end = k;
        }
        const uint64_t key = src[e];
        int64_t greater = 0;
        if (p_begin < k) {
            // partner is descending: count of keys > key
            int64_t lo = p_begin;
            int64_t hi = p_end;
            const uint64_t* q = src + row * k;
            while (lo < hi) {
                const int64_t mid = (lo + hi) >> 1;
                if (q[mid] > key) {
                    lo = mid + 1;
                } else {
                    hi = mid;
                }
            }
            greater = lo - p_begin;
        }
        dst[row * k + pair_base + pos + greater] = key;
    }
}

// K <= kRankMax: a key's place is the number of larger keys (all keys are
// unique). Workgroup (row, part) places keys part * 64 .. part * 64 + 63 of
// the row, four threads per key each counting a quarter of the row's keys
// out of an LDS copy.
constexpr int kRankMax = 1024;

__global__ void __launch_bounds__(256) RankSortKernel(const uint64_t* __restrict__ cand,
                                                      uint64_t* __restrict__ sorted, int64_t k, int parts) {
    __shared__ uint64_t s[kRankMax];
    const int64_t row = blockIdx.x / parts;
    const int part = blockIdx.x - static_cast<int>(row * parts);
    const uint64_t* p = cand + row * k;
    for (int i = threadIdx.x; i < k; i += blockDim.x) {
        s[i] = p[i];
    }
    __syncthreads();
    const int i = part * 64 + (threadIdx.x >> 2);
    const int q = threadIdx.x & 3;
    const uint64_t key = i < k ? s[i] : 0;
    int larger = 0;
    for (int j = q; j < k; j += 4) {
        larger += s[j] > key ? 1 : 0;
    }
    larger += __shfl_xor(larger, 1, 64);
    larger += __shfl_xor(larger, 2, 64);
    if (q == 0 && i < k) {
        sorted[row * k + larger] = key;
    }
}

__global__ void EmitKernel(const float* __restrict__ x, const uint64_t* __restrict__ sorted, float* values,
                           int64_t* indices, int64_t rows, RowGeom g) {
    const int64_t total = rows * g.k;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < total; e += stride) {
        const int64_t row = e / g.k;
        WriteOut(x, values, indices, row, e - row * g.k, sorted[e], g);
    }
}

int PowTwoAtLeast(int64_t n) {
    int p = 1;
    while (p < n) {
        p <<= 1;
    }
    return p;
}

// Scratch of the allocation-free entry point (nert_hip_topk_f32_noalloc):
// one array per GPU, held until the process ends. In host code `scratch`
// names a host-side stand-in, never the device memory: the device address
// comes from hipGetSymbolAddress (TopkScratchSetup), once per device.
constexpr int64_t kNoAllocScratchBytes = 4 << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
uint8_t* g_scratch_ptr[kMaxDevices] = {};

// The workspace a long-row TopK needs: select state | histograms | two
// candidate buffers (256-byte aligned pieces).
struct TopkLayout {
    int64_t st_bytes, hist_bytes, cand_bytes;
    int64_t total() const { return st_bytes + hist_bytes + 2 * cand_bytes; }
};

TopkLayout LayoutFor(int64_t rows, int64_t k) {
    TopkLayout l{};
    l.st_bytes = 2 * ((rows * static_cast<int64_t>(sizeof(SelectState)) + 255) / 256 * 256);
    l.hist_bytes = 3 * ((rows * 256 * 4 + 255) / 256 * 256);
    l.cand_bytes = (rows * k * 8 + 255) / 256 * 256;
    return l;
}

// The TopK launch sequence. `fixed` is the caller's scratch (fixed_bytes
// long) or null, in which case the layer's grow-only workspace is used.
void TopkImpl(const float* x, float* values, int64_t* indices, int64_t outer, int64_t dim, int64_t inner, int64_t k,
              void* stream, uint8_t* fixed, int64_t fixed_bytes) {
    if (k <= 0 || k > dim || dim > 0xFFFFFFFFll) {
        throw Error("topk: need 0 < k <= dim < 2^32");
    }
    const int64_t rows = outer * inner;
    if (rows <= 0) {
        return;
    }
    hipStream_t s = StreamOr(stream);
    RowGeom g{dim, inner, k, 0};
    if (dim <= kSmallRow) {
        if (rows > 0x7FFFFFFF) {
            throw Error("topk: too many rows");
        }
        SmallRowKernel<<<static_cast<unsigned>(rows), kThreads, 0, s>>>(x, values, indices, g, PowTwoAtLeast(dim));
        CheckLaunch("topk small-row launch");
        return;
    }
    // Long rows: about 2048 workgroups over all rows, >= 4096 keys each.
    int64_t chunks = (2048 + rows - 1) / rows;
    const int64_t max_chunks = (dim + 4095) / 4096;
    if (chunks > max_chunks) {
        chunks = max_chunks;
    }
    if (chunks < 1) {
        chunks = 1;
    }
    int64_t chunk = (dim + chunks - 1) / chunks;
    // Contiguous, aligned rows of whole quads: chunks of whole quads too.
    g.vec = inner == 1 && dim % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    if (g.vec) {
        chunk = (chunk + 3) / 4 * 4;
    }
    if (rows * chunks > 0x7FFFFFFF) {
        throw Error("topk: too many rows");
    }
    const TopkLayout lay = LayoutFor(rows, k);
    const int64_t st_bytes = lay.st_bytes;
    const int64_t hist_bytes = lay.hist_bytes;
    const int64_t cand_bytes = lay.cand_bytes;
    uint8_t* ws = fixed;
    if (fixed == nullptr) {
        ws = static_cast<uint8_t*>(Workspace(lay.total(), s));
    } else if (lay.total() > fixed_bytes) {
        throw Error("topk_noalloc: " + std::to_string(rows) + " rows x k = " + std::to_string(k) + " need " +
                    std::to_string(lay.total()) + " bytes of scratch; the fixed scratch holds " +
                    std::to_string(fixed_bytes));
    }
    SelectBuffers sb{};
    sb.st[0] = reinterpret_cast<SelectState*>(ws);
    sb.st[1] = reinterpret_cast<SelectState*>(ws + st_bytes / 2);
    for (int i = 0; i < 3; ++i) {
        sb.hist[i] = reinterpret_cast<uint32_t*>(ws + st_bytes + i * (hist_bytes / 3));
    }
    auto* cand = reinterpret_cast<uint64_t*>(ws + st_bytes + hist_bytes);
    auto* cand2 = reinterpret_cast<uint64_t*>(ws + st_bytes + hist_bytes + cand_bytes);

    InitSelectKernel<<<GridFor(rows * 256, 256, 4096), 256, 0, s>>>(sb, rows, k);
    const unsigned blocks = static_cast<unsigned>(rows * chunks);
    constexpr int kPasses = 8;
    for (int pass = 0; pass < kPasses; ++pass) {
        HistKernel<<<blocks, kThreads, 0, s>>>(x, g, chunk, static_cast<int>(chunks), sb, pass);
    }
    CollectKernel<<<blocks, kThreads, 0, s>>>(x, g, chunk, static_cast<int>(chunks), sb, kPasses - 1, cand);
    if (k <= kRankMax) {
        const int parts = static_cast<int>((k + 63) / 64);
        RankSortKernel<<<static_cast<unsigned>(rows * parts), 256, 0, s>>>(cand, cand2, k, parts);
        EmitKernel<<<GridFor(rows * k, 256, 16384), 256, 0, s>>>(x, cand2, values, indices, rows, g);
        CheckLaunch("topk launch");
        return;
    }
    const int64_t runs = (k + kRun - 1) / kRun;
    const int run_pow2 = PowTwoAtLeast(k < kRun ? k : kRun);
    SortRunsKernel<<<static_cast<unsigned>(rows * runs), kThreads, 0, s>>>(cand, k, static_cast<int>(runs),
                                                                         run_pow2);
    uint64_t* src = cand;
    uint64_t* dst = cand2;
    for (int64_t width = kRun; width < k; width *= 2) {
        MergeKernel<<<GridFor(rows * k, 256, 16384), 256, 0, s>>>(src, dst, rows, k, width);
        uint64_t* t = src;
        src = dst;
        dst = t;
    }
    EmitKernel<<<GridFor(rows * k, 256, 16384), 256, 0, s>>>(x, src, values, indices, rows, g);
    CheckLaunch("topk launch");
}

} // namespace

// Resolves this device's copy of `scratch` (called by the runtime's set-up
// with the device current, before any TopK call).
void TopkScratchSetup() {
    int dev = 0;
    Check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) {
        throw Error("topk scratch: device ordinal out of range");
    }
    void* ptr = nullptr;
    Check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(topk scratch)");
    g_scratch_ptr[dev] = static_cast<uint8_t*>(ptr);
}

} // namespace nert_hip

using namespace nert_hip;

extern "C" {

int nert_hip_topk_f32(const float* x, float* values, int64_t* indices, int64_t outer, int64_t dim, int64_t inner,
                      int64_t k, void* stream) {
    return Guard([&] { TopkImpl(x, values, indices, outer, dim, inner, k, stream, nullptr, 0); });
}

int nert_hip_topk_f32_noalloc(const float* x, float* values, int64_t* indices, int64_t outer, int64_t dim,
                              int64_t inner, int64_t k, void* stream) {
    return Guard([&] {
        if (!RuntimeReady()) {
            throw Error("topk_noalloc: call nert_hip_init() first (it sets up the fixed scratch)");
        }
        int dev = 0;
        Check(hipGetDevice(&dev), "hipGetDevice");
        uint8_t* ptr = dev >= 0 && dev < kMaxDevices ? g_scratch_ptr[dev] : nullptr;
        if (ptr == nullptr) {
            throw Error("topk_noalloc: no fixed scratch on the current device");
        }
        TopkImpl(x, values, indices, outer, dim, inner, k, stream, ptr, kNoAllocScratchBytes);
    });
}

} // extern "C"
