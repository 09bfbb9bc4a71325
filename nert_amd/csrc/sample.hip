// Resampling: Resize (nearest / linear with the ONNX coordinate transforms)
// and GridSample (bilinear / nearest, zeros / border / reflection padding).
//
// Both follow the reference's double-precision coordinate math step for step
// (src/kernels/resize.cpp:48-123, src/kernels/grid_sample.cpp:41-71,132-157).
// Resize evaluates it once per output coordinate of each axis, in a small
// kernel that writes per-axis tables (lower and upper source index, weight)
// to the workspace; the main kernel then only gathers. Nothing is uploaded
// per call, so the row stays capturable. Contraction
// of a*b+c into fma is off in these kernels: every product and sum rounds
// where the reference's does.

#include "common.hpp"
#include "../../include/nert_hip.h"

#pragma clang fp contract(off)

namespace nert_hip {
namespace {

constexpr int kMaxRank = 8;

struct ResizeArgs {
    int rank;
    int linear;
    int transform; // NERT_RESIZE_* transform codes
    int nearest;   // NERT_RESIZE_* nearest codes
    int64_t in_dims[kMaxRank];
    int64_t out_dims[kMaxRank];
    int64_t in_strides[kMaxRank];
    double scales[kMaxRank];
    FastDiv div[kMaxRank]; // by out_dims (32-bit index path)
    int32_t small;         // output has < 2^31 elements
};

// src/kernels/resize.cpp:48-63
__device__ double SourceCoord(int transform, int64_t o, int64_t in_len, int64_t out_len, double scale) {
    const double x = static_cast<double>(o);
    switch (transform) {
    case NERT_RESIZE_HALF_PIXEL:
        return (x + 0.5) / scale - 0.5;
    case NERT_RESIZE_PYTORCH_HALF_PIXEL:
        return out_len > 1 ? (x + 0.5) / scale - 0.5 : 0.0;
    case NERT_RESIZE_ALIGN_CORNERS:
        return out_len == 1 ? 0.0 : x * static_cast<double>(in_len - 1) / static_cast<double>(out_len - 1);
    default: // NERT_RESIZE_ASYMMETRIC
        return x / scale;
    }
}

// static_cast<int64_t>(double) as x86-64 does it: NaN and out-of-range give
// INT64_MIN.
__device__ __forceinline__ int64_t ToI64(double v) {
    if (!(v >= -9223372036854775808.0 && v < 9223372036854775808.0)) {
        return static_cast<int64_t>(0x8000000000000000ULL);
    }
    return static_cast<int64_t>(v);
}

// std::min(std::max(x, lo), hi), NaN passing through as x.
__device__ __forceinline__ double ClampRef(double x, double lo, double hi) {
    const double a = x < lo ? lo : x;
    return hi < a ? hi : a;
}

// src/kernels/resize.cpp:65-82
__device__ int64_t NearestIndex(int mode, double x, int64_t in_len) {
    int64_t index;
    if (mode == NERT_RESIZE_ROUND_PREFER_FLOOR) {
        const double f = floor(x);
        index = ToI64(x - f == 0.5 ? f : round(x));
    } else if (mode == NERT_RESIZE_ROUND_PREFER_CEIL) {
        index = ToI64(round(x));
    } else if (mode == NERT_RESIZE_FLOOR) {
        index = ToI64(floor(x));
    } else {
        index = ToI64(ceil(x));
    }
    return index < 0 ? 0 : (index > in_len - 1 ? in_len - 1 : index);
}

// Per-axis tables: entry base[d] + o holds the source taps of output
// coordinate o along axis d.
struct ResizeTables {
    int64_t* lower;
    int64_t* upper;
    double* weight;
    int64_t base[kMaxRank];
    int64_t total;
};

__global__ void ResizeTableKernel(ResizeArgs a, ResizeTables t) {
    for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < t.total;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int d = 0;
        while (d + 1 < a.rank && e >= t.base[d + 1]) {
            ++d;
        }
        const int64_t o = e - t.base[d];
        const double src = SourceCoord(a.transform, o, a.in_dims[d], a.out_dims[d], a.scales[d]);
        if (!a.linear) {
            t.lower[e] = t.upper[e] = NearestIndex(a.nearest, src, a.in_dims[d]);
            t.weight[e] = 0.0;
            continue;
        }
        const double clamped = ClampRef(src, 0.0, static_cast<double>(a.in_dims[d] - 1));
        const int64_t lo = ToI64(floor(clamped));
        const int64_t up = lo + 1 < a.in_dims[d] - 1 ? lo + 1 : a.in_dims[d] - 1;
        t.lower[e] = lo;
        t.upper[e] = up;
        t.weight[e] = up == lo ? 0.0 : clamped - static_cast<double>(lo);
    }
}

// Nearest: one gather per output element through the tables.
template <typename T>
__global__ void ResizeNearestKernel(const T* __restrict__ x, T* __restrict__ y, ResizeArgs a, ResizeTables t,
                                    int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t rem = i;
        uint32_t rem32 = static_cast<uint32_t>(i);
        int64_t off = 0;
        for (int d = a.rank - 1; d >= 0; --d) {
            int64_t o;
            if (a.small) {
                uint32_t c;
                rem32 = DivMod(a.div[d], rem32, c);
                o = c;
            } else {
                o = rem % a.out_dims[d];
                rem /= a.out_dims[d];
            }
            off += t.lower[t.base[d] + o] * a.in_strides[d];
        }
        y[i] = x[off];
    }
}

// Nearest, four consecutive outputs of the last axis per thread (its output
// length a multiple of 4, fewer than 2^31 outputs, y 16-byte aligned): the
// index decode and the outer axes' table lookups once per four outputs, one
// 16-byte store. The same gathers as ResizeNearestKernel.
__global__ void ResizeNearestQuadKernel(const float* __restrict__ x, float* __restrict__ y, ResizeArgs a,
                                        ResizeTables t, uint32_t quads) {
    const int last = a.rank - 1;
    for (uint32_t q = blockIdx.x * blockDim.x + threadIdx.x; q < quads; q += gridDim.x * blockDim.x) {
        uint32_t c_last;
        uint32_t rem32 = DivMod(a.div[last], 4 * q, c_last);
        int64_t off = 0;
        for (int d = last - 1; d >= 0; --d) {
            uint32_t c;
            rem32 = DivMod(a.div[d], rem32, c);
            off += t.lower[t.base[d] + c] * a.in_strides[d];
        }
        const int64_t* row = t.lower + t.base[last] + c_last;
        nert_floatx4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = x[off + row[e]];
        }
        *reinterpret_cast<nert_floatx4*>(y + 4 * static_cast<int64_t>(q)) = v;
    }
}

// The same for a resize of the last two axes only (every outer axis keeps
// its length at scale 1, where each coordinate transform and nearest mode
// maps o to o): an output row's source row once, the plane offset from the
// flattened outer index, four column lookups per thread.
__global__ void ResizeNearestRowsQuadKernel(const float* __restrict__ x, float* __restrict__ y, ResizeArgs a,
                                            ResizeTables t, uint32_t quads, FastDiv div_row_quads, FastDiv div_out_h,
                                            int64_t in_plane, int64_t in_w) {
    const int hd = a.rank - 2;
    for (uint32_t q = blockIdx.x * blockDim.x + threadIdx.x; q < quads; q += gridDim.x * blockDim.x) {
        uint32_t cq, oy;
        const uint32_t row = DivMod(div_row_quads, q, cq);
        const uint32_t plane = DivMod(div_out_h, row, oy);
        const float* src = x + plane * in_plane + t.lower[t.base[hd] + oy] * in_w;
        const int64_t* cols = t.lower + t.base[hd + 1] + 4 * cq;
        nert_floatx4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = src[cols[e]];
        }
        *reinterpret_cast<nert_floatx4*>(y + 4 * static_cast<int64_t>(q)) = v;
    }
}

// Linear: the taps of every interpolating axis, in the reference's order
// (each interpolating axis doubles the list, lower before upper,
// src/kernels/resize.cpp:102-122), weights from the tables.
template <typename T>
__global__ void ResizeLinearKernel(const T* __restrict__ x, T* __restrict__ y, ResizeArgs a, ResizeTables t,
                                   int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t lower[kMaxRank];
        int64_t upper[kMaxRank];
        double weight[kMaxRank];
        int64_t rem = i;
        uint32_t rem32 = static_cast<uint32_t>(i);
        for (int d = a.rank - 1; d >= 0; --d) {
            int64_t o;
            if (a.small) {
                uint32_t c;
                rem32 = DivMod(a.div[d], rem32, c);
                o = c;
            } else {
                o = rem % a.out_dims[d];
                rem /= a.out_dims[d];
            }
            lower[d] = t.lower[t.base[d] + o];
            upper[d] = t.upper[t.base[d] + o];
            weight[d] = t.weight[t.base[d] + o];
        }
        int interp[kMaxRank];
        int m = 0;
        int64_t base = 0;
        for (int d = 0; d < a.rank; ++d) {
            if (weight[d] == 0.0) {
                base += lower[d] * a.in_strides[d];
            } else {
                interp[m++] = d;
            }
        }
        if (m == 0) {
            y[i] = x[base];
            continue;
        }
        double value = 0.0;
        for (int q = 0; q < (1 << m); ++q) {
            int64_t off = base;
            double w = 1.0;
            for (int j = 0; j < m; ++j) {
                const int d = interp[j];
                const bool up = (q >> (m - 1 - j)) & 1;
                off += (up ? upper[d] : lower[d]) * a.in_strides[d];
                w = w * (up ? weight[d] : 1.0 - weight[d]);
            }
            value += w * static_cast<double>(x[off]);
        }
        y[i] = static_cast<T>(value);
    }
}

// ---- GridSample -------------------------------------------------------------

// src/kernels/grid_sample.cpp:41-51
__device__ double Reflect(double x, double lo, double hi) {
    if (hi == lo) {
        return lo;
    }
    const double range = hi - lo;
    const double d = fabs(x - lo);
    const double flips = floor(d / range);
    const double extra = d - flips * range;
    return fmod(flips, 2.0) == 0.0 ? lo + extra : hi - extra;
}

// src/kernels/grid_sample.cpp:54-65
__device__ double GridCoord(double g, int64_t len, bool align, int padding) {
    const double size = static_cast<double>(len);
    double x = align ? (g + 1.0) / 2.0 * (size - 1.0) : ((g + 1.0) * size - 1.0) / 2.0;
    if (padding == NERT_GRID_REFLECTION) {
        x = align ? Reflect(x, 0.0, size - 1.0) : Reflect(x, -0.5, size - 0.5);
        x = ClampRef(x, 0.0, size - 1.0);
    } else if (padding == NERT_GRID_BORDER) {
        x = ClampRef(x, 0.0, size - 1.0);
    }
    return x;
}

// One thread per output pixel (b, i, j); the channel loop reuses the
// coordinates, as the reference does.
__global__ void GridSampleKernel(const float* __restrict__ x, const float* __restrict__ grid, float* __restrict__ y,
                                 int64_t n, int64_t c, int64_t h, int64_t w, int64_t ho, int64_t wo, int nearest,
                                 int padding, int align) {
    const int64_t pixels = n * ho * wo;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; p < pixels; p += stride) {
        const int64_t j = p % wo;
        const int64_t i = (p / wo) % ho;
        const int64_t b = p / (wo * ho);
        const float* g = grid + p * 2;
        const double px = GridCoord(static_cast<double>(g[0]), w, align != 0, padding);
        const double py = GridCoord(static_cast<double>(g[1]), h, align != 0, padding);
        int64_t x0, y0;
        double wx = 0.0, wy = 0.0;
        if (nearest) {
            x0 = ToI64(rint(px));
            y0 = ToI64(rint(py));
        } else {
            const double fx = floor(px);
            const double fy = floor(py);
            x0 = ToI64(fx);
            y0 = ToI64(fy);
            wx = px - fx;
            wy = py - fy;
        }
        const bool in00 = y0 >= 0 && y0 < h && x0 >= 0 && x0 < w;
        const bool in01 = y0 >= 0 && y0 < h && x0 + 1 >= 0 && x0 + 1 < w;
        const bool in10 = y0 + 1 >= 0 && y0 + 1 < h && x0 >= 0 && x0 < w;
        const bool in11 = y0 + 1 >= 0 && y0 + 1 < h && x0 + 1 >= 0 && x0 + 1 < w;
        for (int64_t ch = 0; ch < c; ++ch) {
            const float* plane = x + (b * c + ch) * h * w;
            double value;
            const double v00 = in00 ? static_cast<double>(plane[y0 * w + x0]) : 0.0;
            if (nearest) {
                value = v00;
            } else {
                const double v01 = in01 ? static_cast<double>(plane[y0 * w + x0 + 1]) : 0.0;
                const double v10 = in10 ? static_cast<double>(plane[(y0 + 1) * w + x0]) : 0.0;
                const double v11 = in11 ? static_cast<double>(plane[(y0 + 1) * w + x0 + 1]) : 0.0;
                value = v00 * (1.0 - wx) * (1.0 - wy) + v01 * wx * (1.0 - wy) + v10 * (1.0 - wx) * wy + v11 * wx * wy;
            }
            y[((b * c + ch) * ho + i) * wo + j] = static_cast<float>(value);
        }
    }
}

// GridSample with the channels spread over blockIdx.y in groups of
// kGsChannels: thread = output pixel, as in GridSampleKernel, with the same
// double coordinate and weight arithmetic in the same order (so the results
// are identical), but the four taps of every channel of the group are loaded
// up front from clamped, always-valid offsets and masked afterwards, so the
// loads overlap instead of each waiting on a branch.
constexpr int kGsChannels = 4;

__global__ __launch_bounds__(256) void GridSampleGroupKernel(const float* __restrict__ x,
                                                             const float* __restrict__ grid, float* __restrict__ y,
                                                             int64_t c, int64_t h, int64_t w, int64_t ho, int64_t wo,
                                                             int nearest, int padding, int align, FastDiv fwo,
                                                             FastDiv fho, uint32_t pixels) {
    const uint32_t p = blockIdx.x * 256u + threadIdx.x;
    if (p >= pixels) {
        return;
    }
    uint32_t j, i;
    const uint32_t b = DivMod(fho, DivMod(fwo, p, j), i);
    const float* g = grid + static_cast<int64_t>(p) * 2;
    const double px = GridCoord(static_cast<double>(g[0]), w, align != 0, padding);
    const double py = GridCoord(static_cast<double>(g[1]), h, align != 0, padding);
    int64_t x0, y0;
    double wx = 0.0, wy = 0.0;
    if (nearest) {
        x0 = ToI64(rint(px));
        y0 = ToI64(rint(py));
    } else {
        const double fx = floor(px);
        const double fy = floor(py);
        x0 = ToI64(fx);
        y0 = ToI64(fy);
        wx = px - fx;
        wy = py - fy;
    }
    const bool inx0 = x0 >= 0 && x0 < w, inx1 = x0 + 1 >= 0 && x0 + 1 < w;
    const bool iny0 = y0 >= 0 && y0 < h, iny1 = y0 + 1 >= 0 && y0 + 1 < h;
    const int64_t cx0 = x0 < 0 ? 0 : (x0 >= w ? w - 1 : x0);
    const int64_t cx1 = x0 + 1 < 0 ? 0 : (x0 + 1 >= w ? w - 1 : x0 + 1);
    const int64_t cy0 = y0 < 0 ? 0 : (y0 >= h ? h - 1 : y0);
    const int64_t cy1 = y0 + 1 < 0 ? 0 : (y0 + 1 >= h ? h - 1 : y0 + 1);
    const int64_t o00 = cy0 * w + cx0, o01 = cy0 * w + cx1, o10 = cy1 * w + cx0, o11 = cy1 * w + cx1;
    const int64_t ch0 = static_cast<int64_t>(blockIdx.y) * kGsChannels;
    float a[kGsChannels][4];
#pragma unroll
    for (int k = 0; k < kGsChannels; ++k) {
        const int64_t ch = ch0 + k < c ? ch0 + k : c - 1;
        const float* plane = x + (static_cast<int64_t>(b) * c + ch) * h * w;
        a[k][0] = plane[o00];
        a[k][1] = plane[o01];
        a[k][2] = plane[o10];
        a[k][3] = plane[o11];
    }
    const int64_t out_plane = ho * wo;
    float* out = y + (static_cast<int64_t>(b) * c + ch0) * out_plane + static_cast<int64_t>(i) * wo + j;
#pragma unroll
    for (int k = 0; k < kGsChannels; ++k) {
        if (ch0 + k >= c) {
            break;
        }
        const double v00 = iny0 && inx0 ? static_cast<double>(a[k][0]) : 0.0;
        double value;
        if (nearest) {
            value = v00;
        } else {
            const double v01 = iny0 && inx1 ? static_cast<double>(a[k][1]) : 0.0;
            const double v10 = iny1 && inx0 ? static_cast<double>(a[k][2]) : 0.0;
            const double v11 = iny1 && inx1 ? static_cast<double>(a[k][3]) : 0.0;
            value = v00 * (1.0 - wx) * (1.0 - wy) + v01 * wx * (1.0 - wy) + v10 * (1.0 - wx) * wy + v11 * wx * wy;
        }
        out[k * out_plane] = static_cast<float>(value);
    }
}

} // namespace
} // namespace nert_hip

using namespace nert_hip;

extern "C" {

int nert_hip_resize(int dtype, const void* x, void* y, int rank, const int64_t* in_dims, const int64_t* out_dims,
                    const double* scales, int linear, int transform, int nearest, void* stream) {
    return Guard([&] {
        if (rank < 1 || rank > kMaxRank) {
            throw Error("resize: rank must be 1..8");
        }
        ResizeArgs a{};
        a.rank = rank;
        a.linear = linear;
        a.transform = transform;
        a.nearest = nearest;
        int64_t n = 1;
        int64_t st = 1;
        for (int d = rank - 1; d >= 0; --d) {
            a.in_dims[d] = in_dims[d];
            a.out_dims[d] = out_dims[d];
            a.scales[d] = scales[d];
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
        if (!(dtype == NERT_F32 || (dtype == NERT_I64 && !linear))) {
            throw Error("resize: float32, or int64 for nearest");
        }
        hipStream_t s = StreamOr(stream);
        ResizeTables t{};
        for (int d = 0; d < rank; ++d) {
            t.base[d] = t.total;
            t.total += out_dims[d];
        }
        char* ws = static_cast<char*>(Workspace(t.total * 24, s));
        t.lower = reinterpret_cast<int64_t*>(ws);
        t.upper = t.lower + t.total;
        t.weight = reinterpret_cast<double*>(t.upper + t.total);
        ResizeTableKernel<<<GridFor(t.total, 256, 1024), 256, 0, s>>>(a, t);
        CheckLaunch("resize table launch");
        const unsigned grid = GridFor(n, 256, 16384);
        if (dtype == NERT_F32 && linear) {
            ResizeLinearKernel<float><<<grid, 256, 0, s>>>(static_cast<const float*>(x), static_cast<float*>(y), a,
                                                           t, n);
        } else if (dtype == NERT_F32 && a.small && rank >= 2 && out_dims[rank - 1] % 4 == 0 &&
                   reinterpret_cast<uintptr_t>(y) % 16 == 0 && [&] {
                       for (int d = 0; d + 2 < rank; ++d) {
                           if (in_dims[d] != out_dims[d] || scales[d] != 1.0) {
                               return false;
                           }
                       }
                       return true;
                   }()) {
            const auto quads = static_cast<uint32_t>(n / 4);
            ResizeNearestRowsQuadKernel<<<GridFor(quads, 256, 16384), 256, 0, s>>>(
                static_cast<const float*>(x), static_cast<float*>(y), a, t, quads,
                FastDiv::Make(static_cast<uint32_t>(out_dims[rank - 1] / 4)),
                FastDiv::Make(static_cast<uint32_t>(out_dims[rank - 2])), in_dims[rank - 2] * in_dims[rank - 1],
                in_dims[rank - 1]);
        } else if (dtype == NERT_F32 && a.small && out_dims[rank - 1] % 4 == 0 &&
                   reinterpret_cast<uintptr_t>(y) % 16 == 0) {
            const auto quads = static_cast<uint32_t>(n / 4);
            ResizeNearestQuadKernel<<<GridFor(quads, 256, 16384), 256, 0, s>>>(static_cast<const float*>(x),
                                                                               static_cast<float*>(y), a, t, quads);
        } else if (dtype == NERT_F32) {
            ResizeNearestKernel<float><<<grid, 256, 0, s>>>(static_cast<const float*>(x), static_cast<float*>(y), a,
                                                            t, n);
        } else {
            ResizeNearestKernel<int64_t><<<grid, 256, 0, s>>>(static_cast<const int64_t*>(x),
                                                              static_cast<int64_t*>(y), a, t, n);
        }
        CheckLaunch("resize launch");
    });
}

int nert_hip_grid_sample_f32(const float* x, const float* grid, float* y, int64_t n, int64_t c, int64_t h, int64_t w,
                             int64_t ho, int64_t wo, int nearest, int padding, int align_corners, void* stream) {
    return Guard([&] {
        const int64_t pixels = n * ho * wo;
        if (pixels <= 0 || c <= 0) {
            return;
        }
        const int64_t groups = (c + kGsChannels - 1) / kGsChannels;
        if (pixels < (int64_t{1} << 31) && groups <= 65535 && h > 0 && w > 0) {
            const dim3 blocks(static_cast<unsigned>((pixels + 255) / 256), static_cast<unsigned>(groups));
            GridSampleGroupKernel<<<blocks, 256, 0, StreamOr(stream)>>>(
                x, grid, y, c, h, w, ho, wo, nearest, padding, align_corners,
                FastDiv::Make(static_cast<uint32_t>(wo)), FastDiv::Make(static_cast<uint32_t>(ho)),
                static_cast<uint32_t>(pixels));
        } else {
            GridSampleKernel<<<GridFor(pixels, 256, 16384), 256, 0, StreamOr(stream)>>>(
                x, grid, y, n, c, h, w, ho, wo, nearest, padding, align_corners);
        }
        CheckLaunch("grid_sample launch");
    });
}

} // extern "C"
