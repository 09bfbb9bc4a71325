// Data movement: one strided-copy kernel serves Transpose, Slice, Expand,
// Tile, Concat and Split; Pad has its own mapping (constant/edge/reflect).
//
// A strided copy walks the destination box in row-major order and reads the
// source through per-axis strides (0 broadcasts for Expand, negative steps
// for Slice, an optional per-axis modulus for Tile). The host drops unit axes
// and merges axes both sides walk contiguously, so most ViT/detector
// reshuffles become rank-2 or rank-3 walks. When the innermost run is
// contiguous on both sides, it moves as 16-, 8- or 4-byte units (whatever
// the run length, the other strides and both base addresses allow). When the
// destination's contiguous axis is not the source's, the copy is a batched
// 2-D transpose between those two axes and goes through 32x32 LDS tiles, so
// reads and writes are both coalesced.

#include "common.hpp"
#include "../../include/nert_hip.h"

#include <algorithm>
#include <vector>

namespace nert_hip {
namespace {

constexpr int kMaxRank = 10;

struct CopyArgs {
    const uint8_t* src;
    uint8_t* dst;
    int rank;
    int64_t dims[kMaxRank];
    int64_t src_strides[kMaxRank]; // elements
    int64_t dst_strides[kMaxRank];
    int64_t src_mods[kMaxRank]; // 0 = no modulus
    FastDiv div[kMaxRank];      // by dims (32-bit index path)
    FastDiv mod_div[kMaxRank];  // by src_mods
};

// Index spaces below 2^31 elements (all but giant tensors): the same walk
// with 32-bit multiply-shift division instead of 64-bit division.
template <typename T>
__global__ void StridedCopy32Kernel(CopyArgs a, uint32_t n) {
    const T* src = reinterpret_cast<const T*>(a.src);
    T* dst = reinterpret_cast<T*>(a.dst);
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint32_t rem = i;
        int64_t so = 0;
        int64_t d_o = 0;
        for (int d = a.rank - 1; d >= 0; --d) {
            uint32_t c;
            rem = DivMod(a.div[d], rem, c);
            uint32_t sc = c;
            if (a.src_mods[d] > 0) {
                DivMod(a.mod_div[d], c, sc);
            }
            so += static_cast<int64_t>(sc) * a.src_strides[d];
            d_o += static_cast<int64_t>(c) * a.dst_strides[d];
        }
        dst[d_o] = src[so];
    }
}

template <typename T>
__global__ void StridedCopyKernel(CopyArgs a, int64_t n) {
    const T* src = reinterpret_cast<const T*>(a.src);
    T* dst = reinterpret_cast<T*>(a.dst);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t rem = i;
        int64_t so = 0;
        int64_t d_o = 0;
        for (int d = a.rank - 1; d >= 0; --d) {
            const int64_t c = rem % a.dims[d];
            rem /= a.dims[d];
            const int64_t sc = a.src_mods[d] > 0 ? c % a.src_mods[d] : c;
            so += sc * a.src_strides[d];
            d_o += c * a.dst_strides[d];
        }
        dst[d_o] = src[so];
    }
}

// Batched transpose: axis `ai` is contiguous in the destination, axis `aj`
// in the source; the remaining axes (batch) are decoded from the tile index.
struct TransposeArgs {
    const uint8_t* src;
    uint8_t* dst;
    int64_t di, dj;               // extents of the two axes
    int64_t si, dj_stride;        // source stride of axis i, destination stride of axis j
    int nb;                       // batch axes
    int64_t bdims[kMaxRank];
    int64_t bsrc[kMaxRank];
    int64_t bdst[kMaxRank];
    FastDiv bdiv[kMaxRank];
    FastDiv tiles_i_div;          // by ceil(di / 32)
    FastDiv tiles_ij_div;         // by tiles along i x tiles along j
    uint32_t tiles;               // total tiles, under 2^31
};

template <typename T>
__global__ __launch_bounds__(256) void TransposeTileKernel(TransposeArgs a) {
    __shared__ T tile[32][33];
    const T* src = reinterpret_cast<const T*>(a.src);
    T* dst = reinterpret_cast<T*>(a.dst);
    const int tx = threadIdx.x & 31;
    const int ty = threadIdx.x >> 5;
    for (uint32_t t = blockIdx.x; t < a.tiles; t += gridDim.x) {
        uint32_t ij;
        uint32_t b = DivMod(a.tiles_ij_div, t, ij);
        uint32_t ti;
        const uint32_t tj = DivMod(a.tiles_i_div, ij, ti);
        int64_t so = 0, d_o = 0;
        for (int d = a.nb - 1; d >= 0; --d) {
            uint32_t c;
            b = DivMod(a.bdiv[d], b, c);
            so += static_cast<int64_t>(c) * a.bsrc[d];
            d_o += static_cast<int64_t>(c) * a.bdst[d];
        }
        const int64_t i0 = static_cast<int64_t>(ti) * 32;
        const int64_t j0 = static_cast<int64_t>(tj) * 32;
        // Read along j (source-contiguous): row r = i offset.
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int r = ty + 8 * k;
            if (i0 + r < a.di && j0 + tx < a.dj) {
                tile[r][tx] = src[so + (i0 + r) * a.si + j0 + tx];
            }
        }
        __syncthreads();
        // Write along i (destination-contiguous): row r = j offset.
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int r = ty + 8 * k;
            if (j0 + r < a.dj && i0 + tx < a.di) {
                dst[d_o + (j0 + r) * a.dj_stride + i0 + tx] = tile[tx][r];
            }
        }
        __syncthreads();
    }
}

int64_t Collapse(int rank, const int64_t* dims, const int64_t* ss, const int64_t* ds, const int64_t* mods,
                 CopyArgs& a) {
    std::vector<int64_t> cd, cs, cdst, cm;
    int64_t n = 1;
    for (int d = 0; d < rank; ++d) {
        n *= dims[d];
        if (dims[d] == 1) {
            continue;
        }
        const int64_t m = mods != nullptr ? mods[d] : 0;
        const bool mod_here = m > 0 && m != dims[d];
        if (!cd.empty() && !mod_here && cm.back() == 0 && cs.back() == ss[d] * dims[d] &&
            cdst.back() == ds[d] * dims[d]) {
            cd.back() *= dims[d];
            cs.back() = ss[d];
            cdst.back() = ds[d];
            continue;
        }
        cd.push_back(dims[d]);
        cs.push_back(ss[d]);
        cdst.push_back(ds[d]);
        cm.push_back(mod_here ? m : 0);
    }
    if (cd.empty()) {
        cd.push_back(1);
        cs.push_back(0);
        cdst.push_back(0);
        cm.push_back(0);
    }
    if (static_cast<int>(cd.size()) > kMaxRank) {
        throw Error("copy: more than 10 non-mergeable axes");
    }
    a.rank = static_cast<int>(cd.size());
    for (int d = 0; d < a.rank; ++d) {
        a.dims[d] = cd[d];
        a.src_strides[d] = cs[d];
        a.dst_strides[d] = cdst[d];
        a.src_mods[d] = cm[d];
        if (n < (int64_t{1} << 31)) {
            a.div[d] = FastDiv::Make(static_cast<uint32_t>(cd[d]));
            a.mod_div[d] = FastDiv::Make(static_cast<uint32_t>(cm[d] > 0 ? cm[d] : 1));
        }
    }
    return n;
}

// ---- Pad -----------------------------------------------------------------
struct PadArgs {
    int rank;
    int mode; // 0 constant, 1 reflect, 2 edge
    int64_t in_dims[kMaxRank];
    int64_t out_dims[kMaxRank];
    int64_t begins[kMaxRank];
    int64_t in_strides[kMaxRank];
    FastDiv div[kMaxRank]; // by out_dims (32-bit index path)
    int32_t small;         // output has < 2^31 elements
};

// src/kernels/pad.cpp MapPosition: -1 means "use the fill value".
__device__ __forceinline__ int64_t MapPos(int64_t pos, int64_t dim, int mode) {
    if (pos >= 0 && pos < dim) {
        return pos;
    }
    if (mode == 0) {
        return -1;
    }
    if (mode == 2) {
        return pos < 0 ? 0 : dim - 1;
    }
    if (dim == 1) {
        return 0;
    }
    const int64_t period = 2 * (dim - 1);
    int64_t m = pos % period;
    if (m < 0) {
        m += period;
    }
    return m < dim ? m : period - m;
}

template <typename T>
__global__ void PadKernel(const T* __restrict__ x, T* __restrict__ y, PadArgs a, T fill, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t rem = i;
        uint32_t rem32 = static_cast<uint32_t>(i);
        int64_t off = 0;
        bool filled = false;
        for (int d = a.rank - 1; d >= 0; --d) {
            int64_t c;
            if (a.small) {
                uint32_t c32;
                rem32 = DivMod(a.div[d], rem32, c32);
                c = c32;
            } else {
                c = rem % a.out_dims[d];
                rem /= a.out_dims[d];
            }
            const int64_t s = MapPos(c - a.begins[d], a.in_dims[d], a.mode);
            filled = filled || s < 0;
            off += (s < 0 ? 0 : s) * a.in_strides[d];
        }
        y[i] = filled ? fill : x[off];
    }
}

// The destination's contiguous axis (the last) is not contiguous in the
// source but another axis is: a batched 2-D transpose. Needs non-negative
// strides, no modulus, and fewer than 2^31 tiles.
bool TryTranspose(const CopyArgs& a, int elem_size, int64_t n, hipStream_t s) {
    const int last = a.rank - 1;
    if (a.rank < 2 || a.dst_strides[last] != 1 || a.src_strides[last] == 1 || n < 1024 ||
        (elem_size != 1 && elem_size != 4 && elem_size != 8)) {
        return false;
    }
    int j = -1;
    for (int d = 0; d < a.rank; ++d) {
        if (a.src_mods[d] != 0 || a.src_strides[d] < 0) {
            return false;
        }
        if (d != last && a.src_strides[d] == 1) {
            j = d;
        }
    }
    if (j < 0 || a.dims[last] < 8 || a.dims[j] < 8) {
        return false;
    }
    TransposeArgs t{};
    t.src = a.src;
    t.dst = a.dst;
    t.di = a.dims[last];
    t.dj = a.dims[j];
    t.si = a.src_strides[last];
    t.dj_stride = a.dst_strides[j];
    int64_t batch = 1;
    for (int d = 0; d < a.rank; ++d) {
        if (d == last || d == j) {
            continue;
        }
        t.bdims[t.nb] = a.dims[d];
        t.bsrc[t.nb] = a.src_strides[d];
        t.bdst[t.nb] = a.dst_strides[d];
        t.bdiv[t.nb] = FastDiv::Make(static_cast<uint32_t>(a.dims[d]));
        ++t.nb;
        batch *= a.dims[d];
    }
    const int64_t ti = (t.di + 31) / 32;
    const int64_t tj = (t.dj + 31) / 32;
    const int64_t tiles = ti * tj * batch;
    if (tiles >= (int64_t{1} << 31) || ti * tj >= (int64_t{1} << 31)) {
        return false;
    }
    t.tiles = static_cast<uint32_t>(tiles);
    t.tiles_i_div = FastDiv::Make(static_cast<uint32_t>(ti));
    t.tiles_ij_div = FastDiv::Make(static_cast<uint32_t>(ti * tj));
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(tiles, 16384));
    switch (elem_size) {
    case 1:
        TransposeTileKernel<uint8_t><<<grid, 256, 0, s>>>(t);
        break;
    case 4:
        TransposeTileKernel<uint32_t><<<grid, 256, 0, s>>>(t);
        break;
    default:
        TransposeTileKernel<uint64_t><<<grid, 256, 0, s>>>(t);
        break;
    }
    CheckLaunch("transpose launch");
    return true;
}

// Concat in one launch: output row r is the inputs' rows r side by side.
// blockIdx.y walks the rows, x the units (16, 4 or 1 bytes) of a row; a unit
// finds its input by a scan over the (at most kConcatMax) input starts.
constexpr int kConcatMax = 8;

struct ConcatArgs {
    const uint8_t* src[kConcatMax];
    int64_t start[kConcatMax + 1]; // units of a row before input i; start[n] = row length
    int32_t n;
    int64_t outer;
    uint8_t* dst;
};

template <typename T>
__global__ __launch_bounds__(256) void ConcatRowsKernel(ConcatArgs a) {
    const int64_t row_units = a.start[a.n];
    for (int64_t row = blockIdx.y; row < a.outer; row += gridDim.y) {
        T* d = reinterpret_cast<T*>(a.dst) + row * row_units;
        for (int64_t j = blockIdx.x * 256 + threadIdx.x; j < row_units; j += static_cast<int64_t>(gridDim.x) * 256) {
            int i = 0;
            while (i + 1 < a.n && j >= a.start[i + 1]) {
                ++i;
            }
            const int64_t len = a.start[i + 1] - a.start[i];
            d[j] = reinterpret_cast<const T*>(a.src[i])[row * len + (j - a.start[i])];
        }
    }
}

} // namespace
} // namespace nert_hip

using namespace nert_hip;

extern "C" {

int nert_hip_concat_rows(int n_inputs, const void* const* srcs, const int64_t* row_bytes, void* dst, int64_t outer,
                         void* stream) {
    return Guard([&] {
        if (n_inputs < 1 || n_inputs > kConcatMax) {
            throw Error("concat_rows: 1 to " + std::to_string(kConcatMax) + " inputs");
        }
        int64_t total = 0;
        uintptr_t align = reinterpret_cast<uintptr_t>(dst);
        for (int i = 0; i < n_inputs; ++i) {
            if (row_bytes[i] < 0) {
                throw Error("concat_rows: negative row length");
            }
            total += row_bytes[i];
            align |= static_cast<uintptr_t>(row_bytes[i]);
            if (row_bytes[i] > 0) {
                align |= reinterpret_cast<uintptr_t>(srcs[i]);
            }
        }
        if (outer <= 0 || total == 0) {
            return;
        }
        const int unit = (align & 15) == 0 ? 16 : ((align & 3) == 0 ? 4 : 1);
        ConcatArgs a{};
        a.n = n_inputs;
        a.outer = outer;
        a.dst = static_cast<uint8_t*>(dst);
        for (int i = 0; i < n_inputs; ++i) {
            a.src[i] = static_cast<const uint8_t*>(srcs[i]);
            a.start[i + 1] = a.start[i] + row_bytes[i] / unit;
        }
        const int64_t row_units = total / unit;
        const unsigned gy = static_cast<unsigned>(std::min<int64_t>(outer, 65535));
        const int64_t want_x = (row_units + 255) / 256;
        const unsigned gx = static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(want_x, 16384 / gy)));
        hipStream_t s = StreamOr(stream);
        const dim3 grid(gx, gy);
        if (unit == 16) {
            ConcatRowsKernel<uint4><<<grid, 256, 0, s>>>(a);
        } else if (unit == 4) {
            ConcatRowsKernel<uint32_t><<<grid, 256, 0, s>>>(a);
        } else {
            ConcatRowsKernel<uint8_t><<<grid, 256, 0, s>>>(a);
        }
        CheckLaunch("concat launch");
    });
}

int nert_hip_copy_strided(int elem_size, const void* src, void* dst, int rank, const int64_t* dims,
                          const int64_t* src_strides, const int64_t* dst_strides, const int64_t* src_mods,
                          void* stream) {
    return Guard([&] {
        CopyArgs a{};
        a.src = static_cast<const uint8_t*>(src);
        a.dst = static_cast<uint8_t*>(dst);
        const int64_t n = Collapse(rank, dims, src_strides, dst_strides, src_mods, a);
        if (n <= 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        // Fully contiguous on both sides: a plain copy.
        if (a.rank == 1 && a.src_strides[0] == 1 && a.dst_strides[0] == 1 && a.src_mods[0] == 0) {
            Check(hipMemcpyAsync(dst, src, static_cast<size_t>(n) * elem_size, hipMemcpyDeviceToDevice, s),
                  "hipMemcpyAsync(copy)");
            return;
        }
        if (TryTranspose(a, elem_size, n, s)) {
            return;
        }
        // Innermost run contiguous on both sides: move it in wider units.
        const int last = a.rank - 1;
        if (a.src_strides[last] == 1 && a.dst_strides[last] == 1 && a.src_mods[last] == 0) {
            for (int unit : {16, 8}) {
                if (unit <= elem_size || unit % elem_size != 0) {
                    continue;
                }
                const int64_t per = unit / elem_size;
                bool ok = a.dims[last] % per == 0 && reinterpret_cast<uintptr_t>(src) % unit == 0 &&
                          reinterpret_cast<uintptr_t>(dst) % unit == 0;
                for (int d = 0; d < last && ok; ++d) {
                    ok = a.src_strides[d] % per == 0 && a.dst_strides[d] % per == 0 && a.src_mods[d] == 0;
                }
                if (!ok) {
                    continue;
                }
                int64_t dims[kMaxRank], ss[kMaxRank], ds[kMaxRank];
                for (int d = 0; d < a.rank; ++d) {
                    dims[d] = d == last ? a.dims[d] / per : a.dims[d];
                    ss[d] = d == last ? 1 : a.src_strides[d] / per;
                    ds[d] = d == last ? 1 : a.dst_strides[d] / per;
                }
                CopyArgs v{};
                v.src = a.src;
                v.dst = a.dst;
                const int64_t nv = Collapse(a.rank, dims, ss, ds, nullptr, v);
                const unsigned vgrid = GridFor(nv, 256, 16384);
                if (nv >= (int64_t{1} << 31)) {
                    if (unit == 16) {
                        StridedCopyKernel<uint4><<<vgrid, 256, 0, s>>>(v, nv);
                    } else {
                        StridedCopyKernel<uint2><<<vgrid, 256, 0, s>>>(v, nv);
                    }
                } else if (unit == 16) {
                    StridedCopy32Kernel<uint4><<<vgrid, 256, 0, s>>>(v, static_cast<uint32_t>(nv));
                } else {
                    StridedCopy32Kernel<uint2><<<vgrid, 256, 0, s>>>(v, static_cast<uint32_t>(nv));
                }
                CheckLaunch("strided copy launch");
                return;
            }
        }
        const unsigned grid = GridFor(n, 256, 16384);
        const bool small = n < (int64_t{1} << 31);
        const uint32_t n32 = static_cast<uint32_t>(small ? n : 0);
        switch (elem_size) {
        case 1:
            small ? StridedCopy32Kernel<uint8_t><<<grid, 256, 0, s>>>(a, n32)
                  : StridedCopyKernel<uint8_t><<<grid, 256, 0, s>>>(a, n);
            break;
        case 4:
            small ? StridedCopy32Kernel<uint32_t><<<grid, 256, 0, s>>>(a, n32)
                  : StridedCopyKernel<uint32_t><<<grid, 256, 0, s>>>(a, n);
            break;
        case 8:
            small ? StridedCopy32Kernel<uint64_t><<<grid, 256, 0, s>>>(a, n32)
                  : StridedCopyKernel<uint64_t><<<grid, 256, 0, s>>>(a, n);
            break;
        default:
            throw Error("copy: unsupported element size");
        }
        CheckLaunch("strided copy launch");
    });
}

int nert_hip_pad(int dtype, const void* x, void* y, int rank, const int64_t* in_dims, const int64_t* out_dims,
                 const int64_t* begins, int mode, double fvalue, int64_t ivalue, void* stream) {
    return Guard([&] {
        if (rank > kMaxRank) {
            throw Error("pad: rank above 10");
        }
        PadArgs a{};
        a.rank = rank;
        a.mode = mode;
        int64_t n = 1;
        int64_t st = 1;
        for (int d = rank - 1; d >= 0; --d) {
            a.in_dims[d] = in_dims[d];
            a.out_dims[d] = out_dims[d];
            a.begins[d] = begins[d];
            a.div[d] = FastDiv::Make(static_cast<uint32_t>(out_dims[d] > 0 && out_dims[d] < (int64_t{1} << 32)
                                                                ? out_dims[d] : 1));
            a.in_strides[d] = st;
            st *= in_dims[d];
            n *= out_dims[d];
        }
        if (n <= 0) {
            return;
        }
        a.small = n < (int64_t{1} << 31) ? 1 : 0;
        hipStream_t s = StreamOr(stream);
        const unsigned grid = GridFor(n, 256, 16384);
        if (dtype == NERT_F32) {
            PadKernel<float><<<grid, 256, 0, s>>>(static_cast<const float*>(x), static_cast<float*>(y), a,
                                                  static_cast<float>(fvalue), n);
        } else {
            PadKernel<int64_t><<<grid, 256, 0, s>>>(static_cast<const int64_t*>(x), static_cast<int64_t*>(y), a,
                                                    ivalue, n);
        }
        CheckLaunch("pad launch");
    });
}

} // extern "C"
