// Pooling rows: MaxPool (2-D), AveragePool (2-D) and GlobalAveragePool.
//
// MaxPool keeps the reference's comparison exactly: a tap replaces the
// running best only when `x > best`, starting from -inf and skipping padded
// taps (src/kernels/max_pool.cpp:210-238), so NaN inputs never win.
// GlobalAveragePool gives each (n, c) plane to one wave: lanes stride the
// plane with coalesced loads, accumulate in double like the reference
// (src/kernels/global_average_pool.cpp:62-68) and combine with a shuffle tree.

#include "common.hpp"
#include "../../include/nert_hip.h"

#include <algorithm>

namespace nert_hip {
namespace {

struct PoolArgs {
    const float* x;
    float* y;
    int64_t planes; // N*C
    int32_t in_h, in_w, out_h, out_w;
    int32_t k_h, k_w, s_h, s_w, d_h, d_w, p_h, p_w;
    int32_t pad_end_h, pad_end_w;
    int32_t count_include_pad;
    FastDiv div_w, div_h; // by out_w, out_h (32-bit index path)
};

// Output index -> (plane, oh, ow); SMALL when the output has < 2^31 elements.
template <bool SMALL>
__device__ __forceinline__ void PoolDecode(const PoolArgs& p, int64_t i, int64_t& plane, int32_t& oh, int32_t& ow) {
    if constexpr (SMALL) {
        uint32_t r;
        const uint32_t t = DivMod(p.div_w, static_cast<uint32_t>(i), r);
        ow = static_cast<int32_t>(r);
        plane = DivMod(p.div_h, t, r);
        oh = static_cast<int32_t>(r);
    } else {
        ow = static_cast<int32_t>(i % p.out_w);
        const int64_t t = i / p.out_w;
        oh = static_cast<int32_t>(t % p.out_h);
        plane = t / p.out_h;
    }
}

template <bool SMALL>
__global__ void MaxPool2dKernel(PoolArgs p) {
    const int64_t total = p.planes * p.out_h * p.out_w;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total; i += stride) {
        int64_t plane;
        int32_t oh, ow;
        PoolDecode<SMALL>(p, i, plane, oh, ow);
        const float* xp = p.x + plane * p.in_h * p.in_w;
        const int32_t h0 = oh * p.s_h - p.p_h;
        const int32_t w0 = ow * p.s_w - p.p_w;
        float best = -__builtin_huge_valf();
        for (int32_t kh = 0; kh < p.k_h; ++kh) {
            const int32_t ih = h0 + kh * p.d_h;
            if (static_cast<uint32_t>(ih) >= static_cast<uint32_t>(p.in_h)) {
                continue;
            }
            const float* row = xp + static_cast<int64_t>(ih) * p.in_w;
            for (int32_t kw = 0; kw < p.k_w; ++kw) {
                const int32_t iw = w0 + kw * p.d_w;
                if (static_cast<uint32_t>(iw) >= static_cast<uint32_t>(p.in_w)) {
                    continue;
                }
                const float v = row[iw];
                if (v > best) {
                    best = v;
                }
            }
        }
        p.y[i] = best;
    }
}

// MaxPool through LDS: a workgroup owns `rows` output rows of one plane. It
// copies the input rows they read (full width; rows outside the image as
// -inf, which never wins the `x > best` test, so they act as skipped taps)
// into LDS with 16-byte loads where the row length allows, then takes every
// window max from LDS: each input element leaves HBM once instead of once
// per window that covers it. Columns outside the image are skipped by the
// bounds test, as the reference skips padded taps.
struct PoolTile {
    int32_t rows;      // output rows per workgroup
    int32_t rows_in;   // input rows they read
    int32_t row_blocks;
    int32_t vec;       // 16-byte loads (in_w % 4 == 0, aligned input)
    FastDiv div_blocks; // by row_blocks
    FastDiv div_in_w;   // by in_w (or in_w / 4 with vec)
    FastDiv div_out_w;  // by out_w
};

__global__ __launch_bounds__(256) void MaxPoolTileKernel(PoolArgs p, PoolTile t) {
    extern __shared__ float tile[]; // [rows_in][in_w]
    uint32_t rb;
    const int64_t plane = DivMod(t.div_blocks, blockIdx.x, rb);
    const int oh0 = static_cast<int>(rb) * t.rows;
    const int ih0 = oh0 * p.s_h - p.p_h;
    const float* xp = p.x + plane * p.in_h * p.in_w;
    const float ninf = -__builtin_huge_valf();
    if (t.vec) {
        // Every 16-byte load of the tile is issued before the first LDS
        // store (batches of kBatch per thread), so a thread waits for one
        // memory round trip per batch rather than one per quad.
        constexpr int kBatch = 4;
        const int quads_row = p.in_w / 4;
        const int quads = t.rows_in * quads_row;
        for (int e0 = 0; e0 < quads; e0 += kBatch * 256) {
            nert_floatx4 v[kBatch];
            int dst[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int e = e0 + j * 256 + threadIdx.x;
                uint32_t c4;
                const int r = static_cast<int>(DivMod(t.div_in_w, static_cast<uint32_t>(e < quads ? e : 0), c4));
                const int ih = ih0 + r;
                const bool in = e < quads && static_cast<unsigned>(ih) < static_cast<unsigned>(p.in_h);
                const nert_floatx4 w = *reinterpret_cast<const nert_floatx4*>(
                    xp + static_cast<int64_t>(in ? ih : 0) * p.in_w + 4 * c4);
                v[j] = in ? w : nert_floatx4{ninf, ninf, ninf, ninf};
                dst[j] = e < quads ? r * p.in_w + 4 * static_cast<int>(c4) : -1;
            }
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                if (dst[j] >= 0) {
                    *reinterpret_cast<nert_floatx4*>(tile + dst[j]) = v[j];
                }
            }
        }
    } else {
        const int elems = t.rows_in * p.in_w;
        for (int e = threadIdx.x; e < elems; e += blockDim.x) {
            uint32_t c;
            const int r = static_cast<int>(DivMod(t.div_in_w, static_cast<uint32_t>(e), c));
            const int ih = ih0 + r;
            tile[e] = static_cast<unsigned>(ih) < static_cast<unsigned>(p.in_h)
                          ? xp[static_cast<int64_t>(ih) * p.in_w + c]
                          : ninf;
        }
    }
    __syncthreads();
    float* yp = p.y + plane * p.out_h * p.out_w;
    const int outs = t.rows * p.out_w;
    for (int o = threadIdx.x; o < outs; o += blockDim.x) {
        uint32_t ow;
        const int r = static_cast<int>(DivMod(t.div_out_w, static_cast<uint32_t>(o), ow));
        const int oh = oh0 + r;
        if (oh >= p.out_h) {
            break; // o only grows
        }
        const int w0 = static_cast<int>(ow) * p.s_w - p.p_w;
        float best = ninf;
        for (int kh = 0; kh < p.k_h; ++kh) {
            const float* row = tile + (r * p.s_h + kh * p.d_h) * p.in_w;
            for (int kw = 0; kw < p.k_w; ++kw) {
                const int iw = w0 + kw * p.d_w;
                if (static_cast<unsigned>(iw) >= static_cast<unsigned>(p.in_w)) {
                    continue;
                }
                const float v = row[iw];
                if (v > best) {
                    best = v;
                }
            }
        }
        yp[static_cast<int64_t>(oh) * p.out_w + ow] = best;
    }
}

// True when a useful tile fits in 48 KiB of LDS: at least 4 output rows, or
// the whole output height.
bool TryMaxPoolTile(const PoolArgs& p, hipStream_t s) {
    constexpr int64_t kLdsFloats = 48 * 1024 / 4;
    const int64_t halo = static_cast<int64_t>(p.k_h - 1) * p.d_h + 1;
    int64_t rows = 16;
    while (rows > 1 && ((rows - 1) * p.s_h + halo) * p.in_w > kLdsFloats) {
        rows /= 2;
    }
    rows = std::min<int64_t>(rows, p.out_h);
    const int64_t rows_in = (rows - 1) * p.s_h + halo;
    if (rows_in * p.in_w > kLdsFloats || (rows < 4 && rows < p.out_h) || rows * p.out_w > (int64_t{1} << 30)) {
        return false;
    }
    PoolTile t{};
    t.rows = static_cast<int32_t>(rows);
    t.rows_in = static_cast<int32_t>(rows_in);
    t.row_blocks = static_cast<int32_t>((p.out_h + rows - 1) / rows);
    const int64_t blocks = p.planes * t.row_blocks;
    if (blocks >= (int64_t{1} << 31)) {
        return false;
    }
    t.vec = p.in_w % 4 == 0 && (reinterpret_cast<uintptr_t>(p.x) & 15) == 0 ? 1 : 0;
    t.div_blocks = FastDiv::Make(static_cast<uint32_t>(t.row_blocks));
    t.div_in_w = FastDiv::Make(static_cast<uint32_t>(t.vec ? p.in_w / 4 : p.in_w));
    t.div_out_w = FastDiv::Make(static_cast<uint32_t>(p.out_w));
    const size_t lds = static_cast<size_t>(rows_in * p.in_w) * sizeof(float);
    MaxPoolTileKernel<<<static_cast<unsigned>(blocks), 256, lds, s>>>(p, t);
    return true;
}

// ---- 3x3 / stride 2 max pooling straight from registers ------------------------
//
// The ResNet stem pool (pad 1) and the unpadded 3x3/2 pool. A lane owns one
// 16-byte column quad (input columns 4k .. 4k+3, output columns 2k and 2k+1)
// of R consecutive output rows of one plane: it loads its 2R+1 input rows'
// quads at once (all loads in flight together, each input byte read once but
// for one shared row per R), takes column 4k-1 (pad 1) or 4k+4 (pad 0) from
// the neighbouring lane, reduces each input row to the two outputs' 3-wide
// row maxima, then each output to the maximum of three row maxima, and
// stores the two outputs as one 8-byte store (4-byte stores where the row
// length is odd or the second output is past the row). A wave holds
// 64 / (W/4) planes' row runs side by side. Max semantics are those of the
// tap loop above (start at -inf, take a tap only if it is strictly greater,
// taps in row-major order, out-of-range taps skipped): the first maximal
// tap in row-major order wins, which the row-then-column reduction keeps,
// so the result is bit-identical, signed zeros and NaNs included.
template <int R, int PAD>
__global__ __launch_bounds__(256) void MaxPool3x3S2Kernel(PoolArgs p, int32_t quads_row, int32_t groups_per_wave,
                                                          int32_t chunks, int64_t groups) {
    const float ninf = -__builtin_huge_valf();
    const int lane = threadIdx.x & 63;
    const int64_t wave = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
    const int gl = lane / quads_row;
    const int k = lane - gl * quads_row;
    const int64_t group = wave * groups_per_wave + gl;
    const bool active = gl < groups_per_wave && group < groups;
    const int64_t plane = active ? group / chunks : 0;
    const int oh0 = static_cast<int>(group - plane * chunks) * R;
    const float* xp = p.x + plane * p.in_h * p.in_w + 4 * k;
    nert_floatx4 v[2 * R + 1];
#pragma unroll
    for (int j = 0; j < 2 * R + 1; ++j) {
        const int ih = 2 * oh0 - PAD + j;
        const bool in = active && static_cast<unsigned>(ih) < static_cast<unsigned>(p.in_h);
        v[j] = in ? *reinterpret_cast<const nert_floatx4*>(xp + static_cast<int64_t>(ih) * p.in_w)
                  : nert_floatx4{ninf, ninf, ninf, ninf};
    }
    auto max3 = [&](float a, float b, float c) {
        float m = ninf;
        m = a > m ? a : m;
        m = b > m ? b : m;
        m = c > m ? c : m;
        return m;
    };
    float h0[2 * R + 1];
    float h1[2 * R + 1];
#pragma unroll
    for (int j = 0; j < 2 * R + 1; ++j) {
        if constexpr (PAD == 1) {
            const float up = __shfl_up(v[j][3], 1);
            const float left = k == 0 ? ninf : up;
            h0[j] = max3(left, v[j][0], v[j][1]);
            h1[j] = max3(v[j][1], v[j][2], v[j][3]);
        } else {
            const float down = __shfl_down(v[j][0], 1);
            const float right = k == quads_row - 1 ? ninf : down;
            h0[j] = max3(v[j][0], v[j][1], v[j][2]);
            h1[j] = max3(v[j][2], v[j][3], right);
        }
    }
    if (!active) {
        return;
    }
    float* yp = p.y + plane * p.out_h * p.out_w + 2 * k;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int oh = oh0 + r;
        if (oh < p.out_h) {
            const float o0 = max3(h0[2 * r], h0[2 * r + 1], h0[2 * r + 2]);
            const float o1 = max3(h1[2 * r], h1[2 * r + 1], h1[2 * r + 2]);
            float* dst = yp + static_cast<int64_t>(oh) * p.out_w;
            if (2 * k + 1 < p.out_w && p.out_w % 2 == 0) {
                *reinterpret_cast<nert_floatx2*>(dst) = nert_floatx2{o0, o1};
            } else {
                if (2 * k < p.out_w) {
                    dst[0] = o0;
                }
                if (2 * k + 1 < p.out_w) {
                    dst[1] = o1;
                }
            }
        }
    }
}

bool TryMaxPool3x3S2(const PoolArgs& p, hipStream_t s) {
    constexpr int kRows = 8;
    // Pad 1 on both axes: W = 2 OW (columns up to 2 OW read). Pad 0: OW =
    // W / 2 - 1, or W / 2 with a right pad (whose tap is skipped). Odd OW
    // stores its outputs one float at a time.
    const bool pad1 = p.p_h == 1 && p.p_w == 1 && p.out_w * 2 == p.in_w;
    const bool pad0 = p.p_h == 0 && p.p_w == 0 && (p.out_w == p.in_w / 2 - 1 || p.out_w == p.in_w / 2);
    if (p.k_h != 3 || p.k_w != 3 || p.s_h != 2 || p.s_w != 2 || p.d_h != 1 || p.d_w != 1 || !(pad1 || pad0) ||
        p.in_w % 4 != 0 || p.in_w > 256 || p.out_h < 1 || p.out_w < 1 ||
        (reinterpret_cast<uintptr_t>(p.x) & 15) != 0 || (reinterpret_cast<uintptr_t>(p.y) & 7) != 0) {
        return false;
    }
    const int32_t quads_row = p.in_w / 4;
    const int32_t groups_per_wave = 64 / quads_row;
    const int32_t chunks = (p.out_h + kRows - 1) / kRows;
    const int64_t groups = p.planes * chunks;
    const int64_t waves = (groups + groups_per_wave - 1) / groups_per_wave;
    const int64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7FFFFFFF) {
        return false;
    }
    if (pad1) {
        MaxPool3x3S2Kernel<kRows, 1><<<static_cast<unsigned>(blocks), 256, 0, s>>>(p, quads_row, groups_per_wave,
                                                                                   chunks, groups);
    } else {
        MaxPool3x3S2Kernel<kRows, 0><<<static_cast<unsigned>(blocks), 256, 0, s>>>(p, quads_row, groups_per_wave,
                                                                                   chunks, groups);
    }
    return true;
}

// AveragePool, exactly as src/kernels/average_pool.cpp:196-223: a float sum
// over the window clipped to the input, in row-major tap order, divided once
// by either the clipped tap count or (count_include_pad) the window clipped to
// the padded extent. Same operations in the same order, so the result is
// bit-identical to the reference.
template <bool SMALL>
__global__ void AvgPool2dKernel(PoolArgs p) {
    const int64_t total = p.planes * p.out_h * p.out_w;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total; i += stride) {
        int64_t plane;
        int32_t oh, ow;
        PoolDecode<SMALL>(p, i, plane, oh, ow);
        const float* xp = p.x + plane * p.in_h * p.in_w;
        const int32_t h_start = oh * p.s_h - p.p_h;
        const int32_t h_end = min(h_start + p.k_h, p.in_h + p.pad_end_h);
        const int32_t h0 = max(h_start, 0);
        const int32_t h1 = min(h_end, p.in_h);
        const int32_t w_start = ow * p.s_w - p.p_w;
        const int32_t w_end = min(w_start + p.k_w, p.in_w + p.pad_end_w);
        const int32_t w0 = max(w_start, 0);
        const int32_t w1 = min(w_end, p.in_w);
        float sum = 0.0f;
        for (int32_t ih = h0; ih < h1; ++ih) {
            const float* row = xp + static_cast<int64_t>(ih) * p.in_w;
            for (int32_t iw = w0; iw < w1; ++iw) {
                sum = __fadd_rn(sum, row[iw]);
            }
        }
        const int64_t divisor = p.count_include_pad ? static_cast<int64_t>(h_end - h_start) * (w_end - w_start)
                                                    : static_cast<int64_t>(h1 - h0) * (w1 - w0);
        p.y[i] = divisor > 0 ? __fdiv_rn(sum, static_cast<float>(divisor)) : 0.0f;
    }
}

__device__ __forceinline__ double WaveSum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        v += __shfl_xor(v, off, 64);
    }
    return v;
}

// One wave per plane; `waves` planes per 256-thread block.
__global__ __launch_bounds__(256) void GlobalAvgPoolKernel(const float* __restrict__ x, float* __restrict__ y,
                                                           int64_t planes, int64_t spatial) {
    const int lane = threadIdx.x & 63;
    const int64_t plane = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (plane >= planes) {
        return;
    }
    const float* xp = x + plane * spatial;
    double sum = 0.0;
    for (int64_t k = lane; k < spatial; k += 64) {
        sum += static_cast<double>(xp[k]);
    }
    sum = WaveSum(sum);
    if (lane == 0) {
        y[plane] = static_cast<float>(sum / static_cast<double>(spatial));
    }
}

// Large planes (the reference bench's [8, 64, 112, 112]): one 256-thread
// workgroup per plane, 16-byte loads when the plane allows, four loads in
// flight per thread, double accumulation, then the waves' sums through LDS
// in a fixed order.
template <bool VEC>
__global__ __launch_bounds__(256) void GlobalAvgPoolBlockKernel(const float* __restrict__ x, float* __restrict__ y,
                                                                int64_t spatial) {
    __shared__ double part[4];
    const int tid = threadIdx.x;
    const float* xp = x + static_cast<int64_t>(blockIdx.x) * spatial;
    double sum = 0.0;
    if constexpr (VEC) {
        const nert_floatx4* x4 = reinterpret_cast<const nert_floatx4*>(xp);
        const int64_t quads = spatial / 4;
        int64_t i = tid;
        for (; i + 768 < quads; i += 1024) {
            const nert_floatx4 a = x4[i];
            const nert_floatx4 b = x4[i + 256];
            const nert_floatx4 c = x4[i + 512];
            const nert_floatx4 d = x4[i + 768];
            sum += ((static_cast<double>(a[0]) + a[1]) + (static_cast<double>(a[2]) + a[3])) +
                   ((static_cast<double>(b[0]) + b[1]) + (static_cast<double>(b[2]) + b[3]));
            sum += ((static_cast<double>(c[0]) + c[1]) + (static_cast<double>(c[2]) + c[3])) +
                   ((static_cast<double>(d[0]) + d[1]) + (static_cast<double>(d[2]) + d[3]));
        }
        for (; i < quads; i += 256) {
            const nert_floatx4 a = x4[i];
            sum += (static_cast<double>(a[0]) + a[1]) + (static_cast<double>(a[2]) + a[3]);
        }
    } else {
        for (int64_t i = tid; i < spatial; i += 256) {
            sum += static_cast<double>(xp[i]);
        }
    }
    sum = WaveSum(sum);
    if ((tid & 63) == 0) {
        part[tid >> 6] = sum;
    }
    __syncthreads();
    if (tid == 0) {
        const double total = (part[0] + part[1]) + (part[2] + part[3]);
        y[blockIdx.x] = static_cast<float>(total / static_cast<double>(spatial));
    }
}

PoolArgs MakeArgs(const float* x, float* y, const nert_pool_desc* d) {
    PoolArgs p{};
    p.x = x;
    p.y = y;
    p.planes = d->batch * d->channels;
    p.in_h = static_cast<int32_t>(d->in[0]);
    p.in_w = static_cast<int32_t>(d->in[1]);
    p.out_h = static_cast<int32_t>(d->out[0]);
    p.out_w = static_cast<int32_t>(d->out[1]);
    p.k_h = static_cast<int32_t>(d->kernel[0]);
    p.k_w = static_cast<int32_t>(d->kernel[1]);
    p.s_h = static_cast<int32_t>(d->stride[0]);
    p.s_w = static_cast<int32_t>(d->stride[1]);
    p.d_h = static_cast<int32_t>(d->dilation[0]);
    p.d_w = static_cast<int32_t>(d->dilation[1]);
    p.p_h = static_cast<int32_t>(d->pad_begin[0]);
    p.p_w = static_cast<int32_t>(d->pad_begin[1]);
    p.pad_end_h = static_cast<int32_t>(d->pad_end[0]);
    p.pad_end_w = static_cast<int32_t>(d->pad_end[1]);
    p.count_include_pad = static_cast<int32_t>(d->count_include_pad);
    p.div_w = FastDiv::Make(static_cast<uint32_t>(p.out_w > 0 ? p.out_w : 1));
    p.div_h = FastDiv::Make(static_cast<uint32_t>(p.out_h > 0 ? p.out_h : 1));
    return p;
}

} // namespace
} // namespace nert_hip

using namespace nert_hip;

extern "C" {

int nert_hip_maxpool2d_f32(const float* x, float* y, const nert_pool_desc* d, void* stream) {
    return Guard([&] {
        PoolArgs p = MakeArgs(x, y, d);
        const int64_t total = p.planes * p.out_h * p.out_w;
        if (total <= 0) {
            return;
        }
        if (TryMaxPool3x3S2(p, StreamOr(stream)) || TryMaxPoolTile(p, StreamOr(stream))) {
            // done
        } else if (total < (int64_t{1} << 31)) {
            MaxPool2dKernel<true><<<GridFor(total, 256, 16384), 256, 0, StreamOr(stream)>>>(p);
        } else {
            MaxPool2dKernel<false><<<GridFor(total, 256, 16384), 256, 0, StreamOr(stream)>>>(p);
        }
        CheckLaunch("MaxPool2dKernel launch");
    });
}

int nert_hip_avgpool2d_f32(const float* x, float* y, const nert_pool_desc* d, void* stream) {
    return Guard([&] {
        PoolArgs p = MakeArgs(x, y, d);
        const int64_t total = p.planes * p.out_h * p.out_w;
        if (total <= 0) {
            return;
        }
        if (total < (int64_t{1} << 31)) {
            AvgPool2dKernel<true><<<GridFor(total, 256, 16384), 256, 0, StreamOr(stream)>>>(p);
        } else {
            AvgPool2dKernel<false><<<GridFor(total, 256, 16384), 256, 0, StreamOr(stream)>>>(p);
        }
        CheckLaunch("AvgPool2dKernel launch");
    });
}

int nert_hip_global_avgpool_f32(const float* x, float* y, int64_t planes, int64_t spatial, void* stream) {
    return Guard([&] {
        if (planes <= 0 || spatial <= 0) {
            return;
        }
        if (spatial >= 2048 && planes <= 0x7FFFFFFF) {
            const bool vec = spatial % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
            if (vec) {
                GlobalAvgPoolBlockKernel<true><<<static_cast<unsigned>(planes), 256, 0, StreamOr(stream)>>>(x, y,
                                                                                                           spatial);
            } else {
                GlobalAvgPoolBlockKernel<false><<<static_cast<unsigned>(planes), 256, 0, StreamOr(stream)>>>(x, y,
                                                                                                            spatial);
            }
            CheckLaunch("GlobalAvgPoolBlockKernel launch");
            return;
        }
        const int64_t blocks = (planes + 3) / 4;
        if (blocks > 0x7FFFFFFF) {
            throw Error("global_avgpool: too many planes");
        }
        GlobalAvgPoolKernel<<<static_cast<unsigned>(blocks), 256, 0, StreamOr(stream)>>>(x, y, planes, spatial);
        CheckLaunch("GlobalAvgPoolKernel launch");
    });
}

} // extern "C"
