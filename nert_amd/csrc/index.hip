// Index rows: Gather, GatherElements, ScatterND, plus the generators Range
// and EyeLike.
//
// Out-of-range indices are data-dependent failures: the kernels skip the
// element and raise bit kIndexFlag in the device error-flag block, which the
// row reads back (or the host validates the indices first when it holds
// them). ScatterND applies duplicate indices in order, like the reference's
// sequential loop: every destination slot takes the update of the LAST slice
// that addresses it, found with an atomicMax over slice numbers, so the
// result does not depend on scheduling.

#include "common.hpp"
#include "../../include/nert_hip.h"

namespace nert_hip {
namespace {

constexpr int32_t kIndexFlag = 2;
constexpr int kMaxRank = 10;

__device__ __forceinline__ void RaiseFlag(int32_t* flags, int32_t bit) { atomicOr(flags, bit); }

// Divisors of the [outer, index_count, inner] decomposition; the 32-bit
// path is taken when the output has < 2^31 elements.
struct GatherDivs {
    FastDiv inner, count;
    int32_t small;
};

__device__ __forceinline__ void GatherDecode(int64_t i, int64_t inner, int64_t index_count, const GatherDivs& g,
                                             int64_t& o, int64_t& j, int64_t& e) {
    if (g.small) {
        uint32_t r;
        const uint32_t q = DivMod(g.inner, static_cast<uint32_t>(i), r);
        e = r;
        o = DivMod(g.count, q, r);
        j = r;
    } else {
        e = i % inner;
        const int64_t q = i / inner;
        j = q % index_count;
        o = q / index_count;
    }
}

// y[o, j, n] = x[o, wrap(idx[j]), n] over [outer, index_count, inner]
// (src/kernels/gather.cpp:29-46).
template <typename T>
__global__ void GatherKernel(const T* __restrict__ x, const int64_t* __restrict__ idx, T* __restrict__ y, int64_t outer,
                             int64_t dim, int64_t index_count, int64_t inner, GatherDivs g, int32_t* flags) {
    const int64_t n = outer * index_count * inner;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t o, j, e;
        GatherDecode(i, inner, index_count, g, o, j, e);
        int64_t k = idx[j];
        if (k < 0) {
            k += dim;
        }
        if (k < 0 || k >= dim) {
            RaiseFlag(flags, kIndexFlag);
            continue;
        }
        y[i] = x[(o * dim + k) * inner + e];
    }
}

// Rows of 16-byte vectors when inner is a multiple of the vector width.
template <typename V>
__global__ void GatherRowsKernel(const V* __restrict__ x, const int64_t* __restrict__ idx, V* __restrict__ y,
                                 int64_t outer, int64_t dim, int64_t index_count, int64_t inner_v, GatherDivs g,
                                 int32_t* flags) {
    const int64_t n = outer * index_count * inner_v;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t o, j, e;
        GatherDecode(i, inner_v, index_count, g, o, j, e);
        int64_t k = idx[j];
        if (k < 0) {
            k += dim;
        }
        if (k < 0 || k >= dim) {
            RaiseFlag(flags, kIndexFlag);
            continue;
        }
        y[i] = x[(o * dim + k) * inner_v + e];
    }
}

struct ElemArgs {
    int rank;
    int axis;
    int64_t idx_dims[kMaxRank];
    int64_t in_strides[kMaxRank];
    int64_t dim;
};

// y[i] = x[coords(i) with coords[axis] = wrap(idx[i])]
// (src/kernels/gather_elements.cpp:43-71).
template <typename T>
__global__ void GatherElementsKernel(const T* __restrict__ x, const int64_t* __restrict__ idx, T* __restrict__ y,
                                     ElemArgs a, int64_t n, int32_t* flags) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t rem = i;
        int64_t off = 0;
        for (int d = a.rank - 1; d >= 0; --d) {
            const int64_t c = rem % a.idx_dims[d];
            rem /= a.idx_dims[d];
            if (d != a.axis) {
                off += c * a.in_strides[d];
            }
        }
        int64_t k = idx[i];
        if (k < 0) {
            k += a.dim;
        }
        if (k < 0 || k >= a.dim) {
            RaiseFlag(flags, kIndexFlag);
            continue;
        }
        y[i] = x[off + k * a.in_strides[a.axis]];
    }
}

struct ScatterArgs {
    int k;
    int64_t dims[kMaxRank];
    int64_t slot_strides[kMaxRank]; // strides of data.dims[:k] counted in slices
};

// Pass 1: owner[slot] = 1 + the highest slice number addressing the slot
// (0, the cleared value, when none does).
__global__ void ScatterOwnerKernel(const int64_t* __restrict__ idx, ScatterArgs a, int64_t slices,
                                   unsigned long long* owner, int32_t* flags) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t s = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; s < slices; s += stride) {
        int64_t slot = 0;
        bool ok = true;
        for (int j = 0; j < a.k; ++j) {
            int64_t c = idx[s * a.k + j];
            const int64_t dim = a.dims[j];
            if (c < -dim || c >= dim) {
                ok = false;
                break;
            }
            if (c < 0) {
                c += dim;
            }
            slot += c * a.slot_strides[j];
        }
        if (!ok) {
            RaiseFlag(flags, kIndexFlag);
            continue;
        }
        atomicMax(owner + slot, static_cast<unsigned long long>(s + 1));
    }
}

// Pass 2: each destination element of an owned slot takes its update.
template <typename T>
__global__ void ScatterApplyKernel(const T* __restrict__ updates, T* __restrict__ out,
                                   const unsigned long long* __restrict__ owner, int64_t slots, int64_t slice_size) {
    const int64_t n = slots * slice_size;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        const int64_t slot = i / slice_size;
        const unsigned long long w = owner[slot];
        if (w != 0) {
            out[i] = updates[static_cast<int64_t>(w - 1) * slice_size + (i - slot * slice_size)];
        }
    }
}

__global__ void ZeroU64Kernel(unsigned long long* p, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        p[i] = 0;
    }
}

// src/kernels/range.cpp:62-64: start + float(i) * delta, two roundings.
// Contraction into an fma (one rounding) is switched off for this body.
__global__ void RangeF32Kernel(float* y, float start, float delta, int64_t n) {
#pragma clang fp contract(off)
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        const float step = static_cast<float>(i) * delta;
        y[i] = start + step;
    }
}

__global__ void RangeI64Kernel(int64_t* y, int64_t start, int64_t delta, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        y[i] = static_cast<int64_t>(static_cast<uint64_t>(start) + static_cast<uint64_t>(i) * static_cast<uint64_t>(delta));
    }
}

template <typename T>
__global__ void EyeKernel(T* y, int64_t rows, int64_t cols, int64_t k, T one) {
    const int64_t n = rows * cols;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / cols;
        const int64_t c = i - r * cols;
        y[i] = c - r == k ? one : T(0);
    }
}

struct SmallI64 {
    int64_t v[16];
};

__global__ void StoreI64Kernel(int64_t* y, SmallI64 values, int count) {
    const int i = static_cast<int>(threadIdx.x);
    if (i < count) {
        y[i] = values.v[i];
    }
}

template <typename T>
void LaunchGather(const void* x, const int64_t* idx, void* y, int64_t outer, int64_t dim, int64_t index_count,
                  int64_t inner, hipStream_t s) {
    const int64_t bytes_inner = inner * static_cast<int64_t>(sizeof(T));
    const bool vec = bytes_inner % 16 == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0 &&
                     (reinterpret_cast<uintptr_t>(y) % 16) == 0;
    const int64_t unit = vec ? bytes_inner / 16 : inner;
    const int64_t n = outer * index_count * unit;
    GatherDivs g{};
    g.small = n < (int64_t{1} << 31) ? 1 : 0;
    if (g.small) {
        g.inner = FastDiv::Make(static_cast<uint32_t>(unit));
        g.count = FastDiv::Make(static_cast<uint32_t>(index_count));
    }
    if (vec) {
        GatherRowsKernel<uint4><<<GridFor(n, 256, 16384), 256, 0, s>>>(
            static_cast<const uint4*>(x), idx, static_cast<uint4*>(y), outer, dim, index_count, unit, g, ErrorFlags());
    } else {
        GatherKernel<T><<<GridFor(n, 256, 16384), 256, 0, s>>>(static_cast<const T*>(x), idx, static_cast<T*>(y),
                                                               outer, dim, index_count, unit, g, ErrorFlags());
    }
}

} // namespace
} // namespace nert_hip

using namespace nert_hip;

extern "C" {

int nert_hip_gather(int elem_size, const void* x, const int64_t* indices, void* y, int64_t outer, int64_t dim,
                    int64_t index_count, int64_t inner, void* stream) {
    return Guard([&] {
        if (outer * index_count * inner <= 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        switch (elem_size) {
        case 1:
            LaunchGather<uint8_t>(x, indices, y, outer, dim, index_count, inner, s);
            break;
        case 4:
            LaunchGather<uint32_t>(x, indices, y, outer, dim, index_count, inner, s);
            break;
        case 8:
            LaunchGather<uint64_t>(x, indices, y, outer, dim, index_count, inner, s);
            break;
        default:
            throw Error("gather: unsupported element size");
        }
        CheckLaunch("gather launch");
    });
}

int nert_hip_gather_elements(int elem_size, const void* x, const int64_t* indices, void* y, int rank,
                             const int64_t* in_dims, const int64_t* idx_dims, int axis, void* stream) {
    return Guard([&] {
        if (rank < 1 || rank > kMaxRank || axis < 0 || axis >= rank) {
            throw Error("gather_elements: rank must be 1..10 and axis inside it");
        }
        ElemArgs a{};
        a.rank = rank;
        a.axis = axis;
        a.dim = in_dims[axis];
        int64_t n = 1;
        int64_t st = 1;
        for (int d = rank - 1; d >= 0; --d) {
            a.idx_dims[d] = idx_dims[d];
            a.in_strides[d] = st;
            st *= in_dims[d];
            n *= idx_dims[d];
        }
        if (n <= 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        const unsigned grid = GridFor(n, 256, 16384);
        if (elem_size == 4) {
            GatherElementsKernel<uint32_t><<<grid, 256, 0, s>>>(static_cast<const uint32_t*>(x), indices,
                                                                static_cast<uint32_t*>(y), a, n, ErrorFlags());
        } else if (elem_size == 8) {
            GatherElementsKernel<uint64_t><<<grid, 256, 0, s>>>(static_cast<const uint64_t*>(x), indices,
                                                                static_cast<uint64_t*>(y), a, n, ErrorFlags());
        } else {
            throw Error("gather_elements: unsupported element size");
        }
        CheckLaunch("gather_elements launch");
    });
}

int nert_hip_scatter_nd(int elem_size, const void* data, const int64_t* indices, const void* updates, void* out,
                        int data_rank, const int64_t* data_dims, int64_t slice_count, int k, void* stream) {
    return Guard([&] {
        if (data_rank < 1 || data_rank > kMaxRank || k < 1 || k > data_rank) {
            throw Error("scatter_nd: rank must be 1..10 with 1 <= k <= rank");
        }
        hipStream_t s = StreamOr(stream);
        int64_t count = 1;
        for (int d = 0; d < data_rank; ++d) {
            count *= data_dims[d];
        }
        if (count <= 0) {
            return;
        }
        if (out != data) {
            Check(hipMemcpyAsync(out, data, static_cast<size_t>(count) * elem_size, hipMemcpyDeviceToDevice, s),
                  "hipMemcpyAsync(scatter_nd)");
        }
        if (slice_count <= 0) {
            return;
        }
        ScatterArgs a{};
        a.k = k;
        int64_t slots = 1;
        for (int d = k - 1; d >= 0; --d) {
            a.dims[d] = data_dims[d];
            a.slot_strides[d] = slots;
            slots *= data_dims[d];
        }
        const int64_t slice_size = count / slots;
        auto* owner = static_cast<unsigned long long*>(Workspace(slots * 8, s));
        ZeroU64Kernel<<<GridFor(slots, 256, 4096), 256, 0, s>>>(owner, slots);
        ScatterOwnerKernel<<<GridFor(slice_count, 256, 4096), 256, 0, s>>>(indices, a, slice_count, owner,
                                                                           ErrorFlags());
        const unsigned grid = GridFor(slots * slice_size, 256, 16384);
        switch (elem_size) {
        case 1:
            ScatterApplyKernel<uint8_t><<<grid, 256, 0, s>>>(static_cast<const uint8_t*>(updates),
                                                            static_cast<uint8_t*>(out), owner, slots, slice_size);
            break;
        case 4:
            ScatterApplyKernel<uint32_t><<<grid, 256, 0, s>>>(static_cast<const uint32_t*>(updates),
                                                             static_cast<uint32_t*>(out), owner, slots, slice_size);
            break;
        case 8:
            ScatterApplyKernel<uint64_t><<<grid, 256, 0, s>>>(static_cast<const uint64_t*>(updates),
                                                             static_cast<uint64_t*>(out), owner, slots, slice_size);
            break;
        default:
            throw Error("scatter_nd: unsupported element size");
        }
        CheckLaunch("scatter_nd launch");
    });
}

int nert_hip_range(int dtype, double fstart, double fdelta, int64_t istart, int64_t idelta, void* y, int64_t count,
                   void* stream) {
    return Guard([&] {
        if (count <= 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        const unsigned grid = GridFor(count, 256, 4096);
        if (dtype == NERT_F32) {
            RangeF32Kernel<<<grid, 256, 0, s>>>(static_cast<float*>(y), static_cast<float>(fstart),
                                                static_cast<float>(fdelta), count);
        } else if (dtype == NERT_I64) {
            RangeI64Kernel<<<grid, 256, 0, s>>>(static_cast<int64_t*>(y), istart, idelta, count);
        } else {
            throw Error("range: dtype must be float32 or int64");
        }
        CheckLaunch("range launch");
    });
}

int nert_hip_store_i64(int64_t* y, const int64_t* values, int count, void* stream) {
    return Guard([&] {
        if (count < 0 || count > 16) {
            throw Error("store_i64: count must be 0..16");
        }
        if (count == 0) {
            return;
        }
        SmallI64 v{};
        for (int i = 0; i < count; ++i) {
            v.v[i] = values[i];
        }
        StoreI64Kernel<<<1, 64, 0, StreamOr(stream)>>>(y, v, count);
        CheckLaunch("store_i64 launch");
    });
}

int nert_hip_eye_like(int dtype, void* y, int64_t rows, int64_t cols, int64_t k, void* stream) {
    return Guard([&] {
        if (rows * cols <= 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        const unsigned grid = GridFor(rows * cols, 256, 16384);
        if (dtype == NERT_F32) {
            EyeKernel<float><<<grid, 256, 0, s>>>(static_cast<float*>(y), rows, cols, k, 1.0f);
        } else if (dtype == NERT_I64) {
            EyeKernel<int64_t><<<grid, 256, 0, s>>>(static_cast<int64_t*>(y), rows, cols, k, int64_t{1});
        } else if (dtype == NERT_BOOL) {
            EyeKernel<uint8_t><<<grid, 256, 0, s>>>(static_cast<uint8_t*>(y), rows, cols, k, uint8_t{1});
        } else {
            throw Error("eye_like: unsupported dtype");
        }
        CheckLaunch("eye_like launch");
    });
}

} // extern "C"
