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
// with K <= 1024 (the detector's [8, 672000], K = 300) read the row once, in
// chunks of up to 24576 keys, one workgroup each (ChunkTop): a chunk keeps
// every key at or above its own threshold for rank K (a 24-bit window fitted
// to the chunk's value range), which holds the chunk's K largest, so the
// row's K largest are among the chunks' candidates. The row's last chunk
// workgroup to finish (a zero-kept counter per row) then merges them
// (MergeTop): the candidates' own threshold for rank K splits them into keys
// in the result and keys tied on the threshold's bits, ranked among
// themselves in LDS (or radix-selected past an LDS capacity); the K keys are
// ranked (all keys are unique; by a counting sort on the threshold's bins
// when it stopped at 12 bits) and written out. When a chunk had more
// candidates than its slots hold, the merge reads the row again. Without the
// counters (NERT_HIP_SPLIT_FIXUP=0) the merge is a second launch, one
// workgroup per row.
// Longer rows with K > 1024 run a radix select over the whole key, 8 bits per
// pass, then sort the K collected keys in 4096-key LDS runs merged by per-key
// binary search.

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

// Float bits -> unsigned integer with the float order: -0.0 folded onto
// +0.0, every NaN above +inf.
__device__ __forceinline__ uint32_t OrdOf(float v) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7FFFFFFFu) == 0) {
        b = 0; // -0.0 == +0.0
    }
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) {
        return 0xFFFFFFFFu; // NaN: above +inf
    }
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint64_t MakeKey(uint32_t ord, int64_t index) {
    return (static_cast<uint64_t>(ord) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(index));
}

__device__ __forceinline__ uint64_t KeyOf(float v, int64_t index) { return MakeKey(OrdOf(v), index); }

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

// ---- long rows, K <= kFastMaxK: one read of the row -----------------------

constexpr int kFastMaxK = 1024;
constexpr int kFT = 1024;            // threads per workgroup of the two kernels
constexpr int kBins = 4096;          // 12-bit digits
constexpr int kWgCand = 1024;        // candidate keys a chunk workgroup keeps
constexpr int kBatch = 16;           // candidate keys per merging thread held in registers
constexpr int kTieCap = 2048;        // keys tied on 24 bits that the merge ranks in LDS
constexpr uint32_t kMergeTieBin = 256; // the merge's threshold stops at 12 bits when its bin holds this many
constexpr int kChunkQuads = 6;       // 16-byte loads per thread and chunk (all issued up front)
constexpr int kChunkMax = kFT * 4 * kChunkQuads;
constexpr int kMergeKeys = kFT * kBatch; // candidates per row the merge aims for
constexpr int64_t kFastMaxRows = 4096;

// A chunk of a row, loaded up front: up to kChunkQuads 16-byte loads per
// thread (contiguous aligned rows) or 4 * kChunkQuads scalar loads (strided
// rows); element e of the thread has row index Index(e), valid while < end.
struct ChunkRegs {
    float v[4 * kChunkQuads];
    int64_t begin;
    int64_t end;
    int32_t vec;
    __device__ __forceinline__ int64_t Index(int e) const {
        return vec ? begin + 4 * (threadIdx.x + (e >> 2) * kFT) + (e & 3)
                   : begin + threadIdx.x + static_cast<int64_t>(e) * kFT;
    }
    __device__ __forceinline__ void Load(const float* __restrict__ x, const RowGeom& g, int64_t base, int64_t b,
                                         int64_t e) {
        begin = b;
        end = e;
        vec = g.vec;
        if (vec) {
            const nert_floatx4* q = reinterpret_cast<const nert_floatx4*>(x + base);
#pragma unroll
            for (int j = 0; j < kChunkQuads; ++j) {
                const int64_t i = begin + 4 * (threadIdx.x + j * kFT);
                const nert_floatx4 t = i < end ? q[i / 4] : nert_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                v[4 * j] = t[0];
                v[4 * j + 1] = t[1];
                v[4 * j + 2] = t[2];
                v[4 * j + 3] = t[3];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4 * kChunkQuads; ++j) {
                const int64_t i = begin + threadIdx.x + static_cast<int64_t>(j) * kFT;
                v[j] = i < end ? x[base + i * g.inner] : 0.0f;
            }
        }
    }
};

// The bin holding the `need`-th largest key among `nbins` LDS counts (bin
// nbins - 1 highest), counting from the top; *above = keys in higher bins.
// Run by a whole workgroup of kFT threads; contains barriers. The counts
// must reach `need`.
__device__ __forceinline__ uint32_t BlockTopSelect(const uint32_t* h, int nbins, uint32_t need, uint32_t* above) {
    __shared__ uint32_t wave_sum[kFT / 64];
    __shared__ uint32_t res_bin;
    __shared__ uint32_t res_above;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int per = nbins >= kFT ? nbins / kFT : 1;
    const bool active = per * t < nbins;
    uint32_t local = 0;
    if (active) {
        for (int j = 0; j < per; ++j) {
            local += h[nbins - 1 - per * t - j];
        }
    }
    uint32_t incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off, 64);
        if (lane >= off) {
            incl += y;
        }
    }
    if (lane == 63) {
        wave_sum[wave] = incl;
    }
    if (t == 0) {
        res_bin = 0;
        res_above = 0;
    }
    __syncthreads();
    for (int w = 0; w < wave; ++w) {
        incl += wave_sum[w];
    }
    const uint32_t excl = incl - local;
    if (active && excl < need && incl >= need) {
        uint32_t cum = excl;
        for (int j = 0; j < per; ++j) {
            const int b = nbins - 1 - per * t - j;
            const uint32_t c = h[b];
            if (cum + c >= need) {
                res_bin = static_cast<uint32_t>(b);
                res_above = cum;
                break;
            }
            cum += c;
        }
    }
    __syncthreads();
    const uint32_t bin = res_bin;
    *above = res_above;
    __syncthreads(); // the next call may overwrite the results
    return bin;
}

// Block-wide maximum of `hi` and minimum of `lo` (kFT threads; barriers).
__device__ __forceinline__ void BlockRange(uint32_t hi, uint32_t lo, uint32_t* top, uint32_t* bottom) {
    __shared__ uint32_t range[2];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t h2 = __shfl_xor(hi, off, 64);
        const uint32_t l2 = __shfl_xor(lo, off, 64);
        hi = h2 > hi ? h2 : hi;
        lo = l2 < lo ? l2 : lo;
    }
    if (threadIdx.x == 0) {
        range[0] = 0;
        range[1] = 0xFFFFFFFFu;
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        atomicMax(&range[0], hi);
        atomicMin(&range[1], lo);
    }
    __syncthreads();
    *top = range[0];
    *bottom = range[1];
    __syncthreads(); // the next call may overwrite the results
}

// h[b] := the number of keys in the bins above b, for kBins LDS counts
// (kFT threads, kBins / kFT bins each from the top down; barriers).
__device__ __forceinline__ void SuffixAbove(uint32_t* h) {
    constexpr int kPer = kBins / kFT;
    __shared__ uint32_t wave_sum[kFT / 64];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    uint32_t c[kPer];
    uint32_t local = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        c[j] = h[kBins - 1 - kPer * t - j];
        local += c[j];
    }
    uint32_t incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off, 64);
        if (lane >= off) {
            incl += y;
        }
    }
    if (lane == 63) {
        wave_sum[wave] = incl;
    }
    __syncthreads();
    for (int w = 0; w < wave; ++w) {
        incl += wave_sum[w];
    }
    uint32_t run = incl - local;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        h[kBins - 1 - kPer * t - j] = run;
        run += c[j];
    }
    __syncthreads();
}

// The threshold of a set of keys for rank `need`, on a window of 24 key
// bits fitted to the set's orderable values, which lie in [bottom, top]:
// every key shares the key bits above bit L + 24, where L = 20 + s and s is
// how far the highest bit in which top and bottom differ lies above bit 11
// (0 if it does not). The top 12 window bits of the keys give bin t1 (with
// `above1` keys above it), the next 12 bits of the keys in t1 give bin t2;
// returns L and sets *floor = (top's bits above the window) << 24 | t1 << 12
// | t2, so that (key >> L) > *floor holds for fewer than `need` keys and
// (key >> L) >= *floor for at least `need`. When bin t1 holds at most
// `max_in_bin` keys and the keys from t1 up at most `max_total`, the second
// level is skipped: then it returns L + 12 and *floor = (top's bits above
// the window) << 12 | t1, with the same two properties, sets *coarse, and
// leaves the first level's counts in `h`. A window fitted to
// the values spreads them over the bins (few LDS adds to one address),
// however narrow their range. `visit(f)` calls f(key, valid) for each
// thread's share of the set, the same in every call; `h` is kBins words of
// LDS. Run by the whole workgroup; contains barriers.
template <typename Visit>
__device__ __forceinline__ int ThresholdInRange(uint32_t* h, uint32_t need, Visit visit, uint32_t top, uint32_t bottom,
                                                uint64_t* floor, uint32_t max_in_bin, uint32_t max_total,
                                                bool* coarse = nullptr) {
    const uint32_t diff = top ^ bottom;
    const int width = diff == 0 ? 0 : 32 - __clz(static_cast<int>(diff));
    const int L = 20 + (width > 12 ? width - 12 : 0);
    for (int b = threadIdx.x; b < kBins; b += kFT) {
        h[b] = 0;
    }
    __syncthreads();
    visit([&](uint64_t key, bool valid) {
        if (valid) {
            atomicAdd(&h[static_cast<uint32_t>(key >> (L + 12)) & 0xFFF], 1u);
        }
    });
    __syncthreads();
    uint32_t above1 = 0;
    const uint32_t t1 = BlockTopSelect(h, kBins, need, &above1);
    // top's bits above the window (none when the window reaches the top bit;
    // a 64-bit shift would be undefined).
    const uint64_t common = L + 24 < 64 ? (static_cast<uint64_t>(top) << 32) >> (L + 24) : 0;
    const uint32_t in_bin = h[t1];
    __syncthreads(); // every thread has read h[t1] before the clear below
    if (coarse != nullptr) {
        *coarse = false;
    }
    if (in_bin <= max_in_bin && above1 + in_bin <= max_total) {
        *floor = (common << 12) | t1;
        if (coarse != nullptr) {
            *coarse = true;
        }
        return L + 12;
    }
    for (int b = threadIdx.x; b < kBins; b += kFT) {
        h[b] = 0;
    }
    __syncthreads();
    visit([&](uint64_t key, bool valid) {
        if (valid && (static_cast<uint32_t>(key >> (L + 12)) & 0xFFF) == t1) {
            atomicAdd(&h[static_cast<uint32_t>(key >> L) & 0xFFF], 1u);
        }
    });
    __syncthreads();
    uint32_t above2 = 0;
    const uint32_t t2 = BlockTopSelect(h, kBins, need - above1, &above2);
    *floor = (common << 24) | (static_cast<uint64_t>(t1) << 12) | t2;
    return L;
}

// The range of the orderable values a visit covers, block-wide.
template <typename Visit>
__device__ __forceinline__ void VisitRange(Visit visit, uint32_t* top, uint32_t* bottom) {
    uint32_t hi = 0;
    uint32_t lo = 0xFFFFFFFFu;
    visit([&](uint64_t key, bool valid) {
        const uint32_t ord = static_cast<uint32_t>(key >> 32);
        hi = valid && ord > hi ? ord : hi;
        lo = valid && ord < lo ? ord : lo;
    });
    BlockRange(hi, lo, top, bottom);
}

// Per chunk workgroup: how many candidates it found (may exceed kWgCand)
// and bounds on their orderable values: the chunk's largest, and a value no
// larger than the smallest candidate's.
struct ChunkStats {
    uint32_t count;
    uint32_t top;
    uint32_t bottom;
    uint32_t pad;
};

// Candidates and stats are written and read at device scope (sc1): the
// workgroup that merges a row may run on another XCD, with its own L2, in
// the same launch as the workgroups that wrote them.
__device__ __forceinline__ void StoreShared(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t LoadShared(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void StoreStats(ChunkStats* p, const ChunkStats& v) {
    uint32_t* w = &p->count;
    __hip_atomic_store(w, v.count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(w + 1, v.top, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(w + 2, v.bottom, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ ChunkStats LoadStats(const ChunkStats* p) {
    uint32_t* w = const_cast<uint32_t*>(&p->count);
    return ChunkStats{__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                      __hip_atomic_load(w + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                      __hip_atomic_load(w + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), 0};
}

// Read of the row, one workgroup per chunk (workgroup wg = row * chunks +
// c): the chunk's candidates for the row's K largest -- every key at or
// above the chunk's own threshold for rank K (all of them when the chunk has
// at most K keys), which holds the chunk's K largest -- written in thread
// order to the workgroup's slots (the first kWgCand), with the chunk's
// stats.
__device__ __forceinline__ void ChunkTop(const float* __restrict__ x, const RowGeom& g, int64_t chunk, int chunks,
                                         uint64_t* cand, ChunkStats* stats, int wg) {
    const int64_t row = wg / chunks;
    const int c = wg - static_cast<int>(row * chunks);
    const uint32_t k = static_cast<uint32_t>(g.k);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    ChunkRegs r;
    const int64_t begin = c * chunk;
    const int64_t end = begin + chunk < g.dim ? begin + chunk : g.dim;
    r.Load(x, g, RowBase(row, g), begin, end);
    __shared__ uint32_t h[kBins];
    __shared__ uint32_t wave_sum[kFT / 64];
    // The elements' orderable values, formed once (0 past the chunk's end:
    // no value maps to 0, -inf maps to 0x007FFFFF), and the low key word of
    // element e, (0xFFFFFFFF - index), as the thread's first element's minus
    // a constant: every visit then costs 32-bit operations only.
    uint32_t ord[4 * kChunkQuads];
#pragma unroll
    for (int e = 0; e < 4 * kChunkQuads; ++e) {
        ord[e] = r.Index(e) < r.end ? OrdOf(r.v[e]) : 0u;
    }
    const uint32_t low0 = 0xFFFFFFFFu - static_cast<uint32_t>(r.Index(0));
    const auto low = [&](int e) {
        return low0 - static_cast<uint32_t>(r.vec ? 4 * (e >> 2) * kFT + (e & 3) : e * kFT);
    };
    const auto visit = [&](auto f) {
#pragma unroll
        for (int e = 0; e < 4 * kChunkQuads; ++e) {
            f((static_cast<uint64_t>(ord[e]) << 32) | low(e), ord[e] != 0u);
        }
    };
    // Bounds of the chunk's K-th largest value: at most the chunk's largest;
    // at least the smallest of the threads' own largest values when at
    // least K threads hold keys (those are that many distinct keys), else
    // at least the chunk's smallest. The threshold histograms count only
    // the keys within the bounds, so their window is fitted to the top of
    // the chunk rather than to its whole range.
    uint32_t hi = 0;
    uint32_t lo = 0xFFFFFFFFu;
    visit([&](uint64_t key, bool valid) {
        const uint32_t ord = static_cast<uint32_t>(key >> 32);
        hi = valid && ord > hi ? ord : hi;
        lo = valid && ord < lo ? ord : lo;
    });
    const int64_t n = end - begin;
    const int64_t holders = g.vec ? (n + 3) / 4 : n; // threads with a key: this many, up to kFT
    if (holders >= static_cast<int64_t>(k)) {
        lo = r.Index(0) < r.end ? hi : 0xFFFFFFFFu;
    }
    uint32_t top = 0;
    uint32_t bottom = 0;
    BlockRange(hi, lo, &top, &bottom);
    // A chunk of at most K keys passes them all (floor 0 at L = 0). Every
    // candidate's orderable value is at least the floor's.
    uint64_t floor = 0;
    int L = 0;
    if (n > static_cast<int64_t>(k)) {
        const uint32_t low = bottom;
        L = ThresholdInRange(
            h, k,
            [&](auto f) {
                visit([&](uint64_t key, bool valid) { f(key, valid && static_cast<uint32_t>(key >> 32) >= low); });
            },
            top, bottom, &floor, 0xFFFFFFFFu, static_cast<uint32_t>(kWgCand));
        bottom = static_cast<uint32_t>((floor << L) >> 32);
    }
    // Candidates of this thread (bit e of `pass` for element e), then their
    // places: a block-wide exclusive sum over threads.
    uint32_t pass = 0;
#pragma unroll
    for (int e = 0; e < 4 * kChunkQuads; ++e) {
        const uint64_t key = (static_cast<uint64_t>(ord[e]) << 32) | low(e);
        if (ord[e] != 0u && (key >> L) >= floor) {
            pass |= 1u << e;
        }
    }
    const uint32_t mine = static_cast<uint32_t>(__popc(pass));
    uint32_t incl = mine;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off, 64);
        if (lane >= off) {
            incl += y;
        }
    }
    if (lane == 63) {
        wave_sum[wave] = incl;
    }
    __syncthreads();
    uint32_t at = incl - mine;
    uint32_t total = 0;
    for (int w = 0; w < kFT / 64; ++w) {
        at += w < wave ? wave_sum[w] : 0;
        total += wave_sum[w];
    }
    uint64_t* slots = cand + static_cast<int64_t>(wg) * kWgCand;
#pragma unroll
    for (int e = 0; e < 4 * kChunkQuads; ++e) {
        if ((pass >> e) & 1u) {
            if (at < kWgCand) {
                StoreShared(slots + at, (static_cast<uint64_t>(ord[e]) << 32) | low(e));
            }
            ++at;
        }
    }
    if (tid == 0) {
        StoreStats(stats + wg, ChunkStats{total, top, bottom, 0});
    }
}

// The value of a result key: rebuilt from its orderable bits, except for
// zeros (-0.0 was folded onto +0.0) and NaNs, which are read back.
__device__ __forceinline__ float ValueOf(const float* x, const RowGeom& g, int64_t row, uint64_t key) {
    const uint32_t ord = static_cast<uint32_t>(key >> 32);
    if (ord == 0x80000000u || ord == 0xFFFFFFFFu) {
        return x[RowBase(row, g) + IndexOf(key) * g.inner];
    }
    return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord);
}

// One workgroup per row: the row's K largest among its chunks' candidates
// (or, when a chunk had more candidates than slots, among all of the row's
// keys, read again). The 24-bit threshold of the candidates for rank K
// splits them: keys above it are in the result, keys on it (tied on 24 bits)
// are ranked among themselves in LDS, or radix-selected over their remaining
// 40 key bits past kTieCap. The K keys are then ranked (all keys are unique)
// and written out.
__device__ __forceinline__ void MergeTop(const float* __restrict__ x, float* values, int64_t* indices,
                                         const RowGeom& g, int chunks, const uint64_t* cand, const ChunkStats* stats,
                                         int64_t row) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const uint32_t k = static_cast<uint32_t>(g.k);
    const int64_t wg0 = row * chunks;
    __shared__ uint32_t h[kBins];
    __shared__ __attribute__((aligned(16))) uint64_t fin[kFastMaxK];
    __shared__ uint64_t ties[kTieCap];
    __shared__ uint32_t rank_s[kFastMaxK];
    __shared__ uint32_t off_s[kFT];
    __shared__ uint32_t wave_sum[kFT / 64];
    __shared__ uint32_t total_s;
    __shared__ uint32_t fits_s;
    __shared__ uint32_t overflow_s;
    __shared__ uint32_t top_s;
    __shared__ uint32_t bottom_s;
    __shared__ uint32_t n_fin;
    __shared__ uint32_t n_ties;
    // Chunk c's candidates go to threads c * T .. c * T + T - 1, kBatch
    // slots each: the chunk's stats and every slot are loaded at once (slots
    // past the chunk's count are read but not used).
    const int T = kFT / chunks;
    const int group = tid / T;
    const int member_slot = tid - group * T;
    const bool member = group < chunks;
    ChunkStats cs{0, 0, 0xFFFFFFFFu, 0};
    if (member) {
        cs = LoadStats(stats + wg0 + group);
    }
    uint64_t kv[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
        const int slot = member_slot + T * j;
        kv[j] = member && slot < kWgCand ? LoadShared(cand + (wg0 + group) * kWgCand + slot) : 0;
    }
    // Wave 0 reads every chunk's stats and reduces them (whether the
    // candidates fit the groups' registers, whether a chunk overflowed its
    // slots, their value range) for one barrier.
    if (wave == 0) {
        bool fits = true;
        bool overflow = false;
        uint32_t hi = 0;
        uint32_t lo = 0xFFFFFFFFu;
        for (int c = lane; c < chunks; c += 64) {
            const ChunkStats st = LoadStats(stats + wg0 + c);
            fits = fits && st.count <= static_cast<uint32_t>(kWgCand) && st.count <= static_cast<uint32_t>(T * kBatch);
            overflow = overflow || st.count > static_cast<uint32_t>(kWgCand);
            hi = st.top > hi ? st.top : hi;
            lo = st.bottom < lo ? st.bottom : lo;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const uint32_t h2 = __shfl_xor(hi, off, 64);
            const uint32_t l2 = __shfl_xor(lo, off, 64);
            hi = h2 > hi ? h2 : hi;
            lo = l2 < lo ? l2 : lo;
        }
        const bool all_fit = __all(fits);
        const bool any_overflow = __any(overflow);
        if (lane == 0) {
            fits_s = all_fit ? 1u : 0u;
            overflow_s = any_overflow ? 1u : 0u;
            top_s = hi;
            bottom_s = lo;
            n_fin = 0;
            n_ties = 0;
        }
    }
    for (uint32_t i = tid; i < k; i += kFT) {
        fin[i] = uint64_t{0xFFFFFFFFu}; // a key of index 0: every index read back stays in the row
        rank_s[i] = 0;
    }
    __syncthreads();
    const bool in_regs = fits_s != 0;
    const bool from_cand = overflow_s == 0;
    uint32_t total = 0;
    if (!in_regs && from_cand) {
        // More candidates than the groups' registers hold: offsets of the
        // chunks' candidates in chunk order, for streaming them in batches.
        const uint32_t nc = tid < chunks ? LoadStats(stats + wg0 + tid).count : 0;
        uint32_t incl = nc;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t y = __shfl_up(incl, off, 64);
            if (lane >= off) {
                incl += y;
            }
        }
        if (lane == 63) {
            wave_sum[wave] = incl;
        }
        __syncthreads();
        uint32_t before = 0;
        uint32_t all = 0;
        for (int w = 0; w < kFT / 64; ++w) {
            before += w < wave ? wave_sum[w] : 0;
            all += wave_sum[w];
        }
        off_s[tid] = before + incl - nc;
        if (tid == 0) {
            total_s = all;
        }
        __syncthreads();
        total = total_s;
    }
    // Candidate i (in chunk order) sits in the slots of the last chunk whose
    // offset is <= i.
    const auto owner = [&](uint32_t i) {
        int lo = 0;
        int hi = chunks - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (off_s[mid] <= i) {
                lo = mid;
            } else {
                hi = mid - 1;
            }
        }
        return lo;
    };
    const uint32_t held = member ? (cs.count < static_cast<uint32_t>(kWgCand) ? cs.count : kWgCand) : 0;
    const int64_t base = RowBase(row, g);
    // The candidates: in the groups' registers; else streamed in batches;
    // or the whole row when a chunk had more than its slots hold.
    const auto source = [&](auto f) {
        if (in_regs) {
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                f(kv[j], static_cast<uint32_t>(member_slot + T * j) < held);
            }
        } else if (from_cand) {
            // (kv is free here: the registers path is not taken.)
            for (uint32_t b0 = 0; b0 < total; b0 += kMergeKeys) {
#pragma unroll
                for (int j = 0; j < kBatch; ++j) {
                    const uint32_t i = b0 + tid + j * kFT;
                    kv[j] = 0;
                    if (i < total) {
                        const int w = owner(i);
                        kv[j] = LoadShared(cand + (wg0 + w) * kWgCand + (i - off_s[w]));
                    }
                }
#pragma unroll
                for (int j = 0; j < kBatch; ++j) {
                    f(kv[j], b0 + tid + j * kFT < total);
                }
            }
        } else {
            for (int64_t i0 = 0; i0 < g.dim; i0 += kFT) {
                const int64_t i = i0 + tid;
                const bool ok = i < g.dim;
                f(ok ? KeyOf(x[base + i * g.inner], i) : 0, ok);
            }
        }
    };
    uint32_t range_top = 0;
    uint32_t range_bottom = 0;
    if (in_regs) {
        range_top = top_s;
        range_bottom = bottom_s;
    } else {
        VisitRange(source, &range_top, &range_bottom);
    }
    uint64_t top = 0;
    bool coarse = false;
    const int L = ThresholdInRange(h, k, source, range_top, range_bottom, &top, kMergeTieBin, 0xFFFFFFFFu, &coarse);
    if (coarse) {
        // A counting sort on the threshold's bins: keys above the threshold
        // bin t1 go straight to the slots of their bin, bins in descending
        // order (h[b] becomes the count above b, then each key takes the
        // next slot of its bin), so a key's rank is its bin's first slot
        // plus the count of larger keys in its bin; the keys in t1 (at most
        // kMergeTieBin) are ranked among themselves after them.
        const uint32_t t1 = static_cast<uint32_t>(top & 0xFFF);
        SuffixAbove(h);
        const uint32_t fin0 = h[t1]; // keys above the threshold, fewer than K
        source([&](uint64_t key, bool valid) {
            if (!valid) {
                return;
            }
            if ((key >> L) > top) {
                fin[atomicAdd(&h[static_cast<uint32_t>(key >> L) & 0xFFF], 1u)] = key;
            } else if ((key >> L) == top) {
                ties[atomicAdd(&n_ties, 1u)] = key;
            }
        });
        __syncthreads();
        const uint32_t need = k - fin0;
        const uint32_t nt = n_ties;
        for (uint32_t i = tid; i < nt; i += kFT) {
            const uint64_t key = ties[i];
            uint32_t rank = 0;
            for (uint32_t j = 0; j < nt; ++j) {
                rank += ties[j] > key ? 1u : 0u;
            }
            if (rank < need) {
                fin[fin0 + rank] = key;
            }
        }
        __syncthreads();
        const int64_t o = row / g.inner;
        const int64_t n = row - o * g.inner;
        for (uint32_t i = tid; i < k; i += kFT) {
            const uint64_t key = fin[i];
            uint32_t rank = i;
            if (i < fin0) {
                // The bin's slots: [h[b + 1] (0 for the top bin), h[b]).
                const uint32_t b = static_cast<uint32_t>(key >> L) & 0xFFF;
                const uint32_t first = b + 1 < static_cast<uint32_t>(kBins) ? h[b + 1] : 0u;
                const uint32_t end = h[b];
                rank = first;
                for (uint32_t q = first; q < end; ++q) {
                    rank += fin[q] > key ? 1u : 0u;
                }
            }
            const int64_t dst = (o * g.k + rank) * g.inner + n;
            values[dst] = ValueOf(x, g, row, key);
            indices[dst] = IndexOf(key);
        }
        return;
    }
    source([&](uint64_t key, bool valid) {
        if (!valid) {
            return;
        }
        if ((key >> L) > top) {
            const uint32_t p = atomicAdd(&n_fin, 1u);
            if (p < k) {
                fin[p] = key;
            }
        } else if ((key >> L) == top) {
            const uint32_t p = atomicAdd(&n_ties, 1u);
            if (p < kTieCap) {
                ties[p] = key;
            }
        }
    });
    __syncthreads();
    const uint32_t fin0 = n_fin < k ? n_fin : k; // keys above the floor
    const uint32_t need = k - fin0;
    const uint32_t nt = n_ties;
    if (nt <= static_cast<uint32_t>(kTieCap)) {
        // A tied key's place among the ties is the count of larger ones
        // (keys are unique); the `need` largest join the result.
        for (uint32_t i = tid; i < nt; i += kFT) {
            const uint64_t key = ties[i];
            uint32_t rank = 0;
            for (uint32_t j = 0; j < nt; ++j) {
                rank += ties[j] > key ? 1u : 0u;
            }
            if (rank < need) {
                fin[fin0 + rank] = key;
            }
        }
    } else {
        // Radix select over the tied keys' remaining L bits, 8 per pass from
        // the top (the last pass's digit may also hold bits fixed already,
        // equal in every key it counts), then take the tied keys at or above
        // the result.
        uint64_t prefix = top << L;
        uint64_t mask = ~((uint64_t{1} << L) - 1);
        uint32_t remaining = need;
        for (int shift = L - 8;; shift -= 8) {
            const int sh = shift > 0 ? shift : 0;
            for (int b = tid; b < 256; b += kFT) {
                h[b] = 0;
            }
            __syncthreads();
            source([&](uint64_t key, bool valid) {
                if (valid && (key & mask) == prefix) {
                    atomicAdd(&h[static_cast<uint32_t>(key >> sh) & 0xFF], 1u);
                }
            });
            __syncthreads();
            uint32_t ab = 0;
            const uint32_t d = BlockTopSelect(h, 256, remaining, &ab);
            remaining -= ab;
            prefix = (prefix & ~(0xFFull << sh)) | (static_cast<uint64_t>(d) << sh);
            mask |= 0xFFull << sh;
            if (sh == 0) {
                break;
            }
        }
        source([&](uint64_t key, bool valid) {
            if (valid && (key >> L) == top && key >= prefix) {
                const uint32_t p = atomicAdd(&n_fin, 1u);
                if (p < k) {
                    fin[p] = key;
                }
            }
        });
    }
    __syncthreads();
    // Ranks: `per` threads count the larger keys of one result key each,
    // over slices of four-key (two 16-byte LDS reads) steps; slots past K
    // hold the smallest key, never larger.
    for (uint32_t i = k + tid; i < (k + 3) / 4 * 4; i += kFT) {
        fin[i] = 0;
    }
    __syncthreads();
    const uint32_t quads = (k + 3) / 4;
    const uint32_t per = k < static_cast<uint32_t>(kFT) ? static_cast<uint32_t>(kFT) / k : 1u;
    const uint32_t slice = (quads + per - 1) / per;
    const ulonglong2* fin2 = reinterpret_cast<const ulonglong2*>(fin);
    for (uint32_t t = tid; t < k * per; t += kFT) {
        const uint32_t i = t / per;
        const uint32_t part = t - i * per;
        const uint64_t key = fin[i];
        const uint32_t q1 = (part + 1) * slice < quads ? (part + 1) * slice : quads;
        uint32_t larger = 0;
#pragma unroll 4
        for (uint32_t q = part * slice; q < q1; ++q) {
            const ulonglong2 a = fin2[2 * q];
            const ulonglong2 b = fin2[2 * q + 1];
            larger += (a.x > key ? 1u : 0u) + (a.y > key ? 1u : 0u) + (b.x > key ? 1u : 0u) + (b.y > key ? 1u : 0u);
        }
        if (larger != 0) {
            atomicAdd(&rank_s[i], larger);
        }
    }
    __syncthreads();
    const int64_t o = row / g.inner;
    const int64_t n = row - o * g.inner;
    for (uint32_t i = tid; i < k; i += kFT) {
        const uint64_t key = fin[i];
        const int64_t dst = (o * g.k + rank_s[i]) * g.inner + n;
        values[dst] = ValueOf(x, g, row, key);
        indices[dst] = IndexOf(key);
    }
}

// After a chunk's candidate and stats stores: waits for them, counts the
// workgroup in on its row's counter, and returns (to every thread) whether
// it was the row's last chunk; the last one leaves the counter zero.
__device__ __forceinline__ bool ArriveLastChunk(uint32_t* counter, int chunks, int* flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = before + 1 == static_cast<uint32_t>(chunks);
        if (last) {
            __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        *flag = last ? 1 : 0;
    }
    __syncthreads();
    return *flag != 0;
}

// One launch: every chunk workgroup finds its candidates; the row's last to
// finish merges the row (counters[row] zero before and after).
__global__ void __launch_bounds__(kFT) ChunkMergeTopKernel(const float* __restrict__ x, float* values,
                                                           int64_t* indices, RowGeom g, int64_t chunk, int chunks,
                                                           uint64_t* cand, ChunkStats* stats, uint32_t* counters) {
    ChunkTop(x, g, chunk, chunks, cand, stats, static_cast<int>(blockIdx.x));
    __shared__ int last;
    const int64_t row = blockIdx.x / chunks;
    if (ArriveLastChunk(counters + row, chunks, &last)) {
        MergeTop(x, values, indices, g, chunks, cand, stats, row);
    }
}

// The same as two launches (no counters): chunks, then one workgroup per row.
__global__ void __launch_bounds__(kFT) ChunkTopKernel(const float* __restrict__ x, RowGeom g, int64_t chunk,
                                                      int chunks, uint64_t* cand, ChunkStats* stats) {
    ChunkTop(x, g, chunk, chunks, cand, stats, static_cast<int>(blockIdx.x));
}

__global__ void __launch_bounds__(kFT) MergeTopKernel(const float* __restrict__ x, float* values, int64_t* indices,
                                                      RowGeom g, int chunks, const uint64_t* cand,
                                                      const ChunkStats* stats) {
    MergeTop(x, values, indices, g, chunks, cand, stats, blockIdx.x);
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
constexpr int64_t kRowCounterBytes = kFastMaxRows * 4; // zero-kept, at the start of the scratch
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

// Long rows with K <= kFastMaxK: chunk candidates and the per-row merge,
// one read of the row. `counters` (one zero-kept word per row) or null for
// two launches.
void FastTopk(const float* x, float* values, int64_t* indices, int64_t rows, RowGeom g, hipStream_t s, uint8_t* fixed,
              int64_t fixed_bytes, uint32_t* counters) {
    // About 256 workgroups over all rows; chunks of at most kChunkMax keys
    // and at least 4096, and (where the chunk limit allows) few enough per
    // row that their candidates, about K each, fit the merge's registers.
    int64_t chunks = (256 + rows - 1) / rows;
    const int64_t min_chunks = (g.dim + kChunkMax - 1) / kChunkMax;
    const int64_t max_chunks = (g.dim + 4095) / 4096;
    const int64_t merge_chunks = kMergeKeys / (g.k + 16);
    chunks = chunks > merge_chunks ? merge_chunks : chunks;
    chunks = chunks > max_chunks ? max_chunks : chunks;
    chunks = chunks < min_chunks ? min_chunks : chunks;
    chunks = chunks < 1 ? 1 : chunks;
    int64_t chunk = (g.dim + chunks - 1) / chunks;
    g.vec = g.inner == 1 && g.dim % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    if (g.vec) {
        chunk = (chunk + 3) / 4 * 4;
    }
    chunks = (g.dim + chunk - 1) / chunk; // every chunk non-empty
    if (chunk > kChunkMax || chunks > kFT || rows * chunks > 0x7FFFFFFF) {
        throw Error("topk: chunking out of range");
    }
    const auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    const int64_t cand_bytes = up(rows * chunks * kWgCand * 8);
    const int64_t need = cand_bytes + up(rows * chunks * static_cast<int64_t>(sizeof(ChunkStats)));
    uint8_t* ws = fixed;
    if (fixed == nullptr) {
        ws = static_cast<uint8_t*>(Workspace(need, s));
    } else if (need > fixed_bytes) {
        throw Error("topk_noalloc: " + std::to_string(rows) + " rows x k = " + std::to_string(g.k) + " need " +
                    std::to_string(need) + " bytes of scratch; the fixed scratch holds " +
                    std::to_string(fixed_bytes));
    }
    auto* cand = reinterpret_cast<uint64_t*>(ws);
    auto* stats = reinterpret_cast<ChunkStats*>(ws + cand_bytes);
    if (counters != nullptr) {
        ChunkMergeTopKernel<<<static_cast<unsigned>(rows * chunks), kFT, 0, s>>>(
            x, values, indices, g, chunk, static_cast<int>(chunks), cand, stats, counters);
    } else {
        ChunkTopKernel<<<static_cast<unsigned>(rows * chunks), kFT, 0, s>>>(x, g, chunk, static_cast<int>(chunks),
                                                                              cand, stats);
        MergeTopKernel<<<static_cast<unsigned>(rows), kFT, 0, s>>>(x, values, indices, g, static_cast<int>(chunks),
                                                                   cand, stats);
    }
    CheckLaunch("topk launch");
}

// The TopK launch sequence. `fixed` is the caller's scratch (fixed_bytes
// long, its first kRowCounterBytes the zero-kept row counters) or null, in
// which case the layer's grow-only workspace and tile counters are used.
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
    uint32_t* counters = nullptr;
    if (fixed != nullptr) {
        counters = reinterpret_cast<uint32_t*>(fixed);
        fixed += kRowCounterBytes;
        fixed_bytes -= kRowCounterBytes;
    }
    if (k <= kFastMaxK && rows <= kFastMaxRows) {
        if (counters == nullptr) {
            counters = TileCounters(rows);
        }
        FastTopk(x, values, indices, rows, g, s, fixed, fixed_bytes, counters);
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
    // The row counters start at zero; every launch that uses them leaves
    // them zero.
    Check(hipMemset(ptr, 0, kRowCounterBytes), "hipMemset(topk scratch counters)");
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
