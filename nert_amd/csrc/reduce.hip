// Reductions: ReduceSum/Mean/Max/L2, Softmax, LayerNormalization,
// InstanceNormalization, ArgMax and CumSum.
//
// Layout: a contiguous reduction (the reduced axes are the trailing ones, or
// the normalised axis is last) gives each output row to one wave: lanes read
// consecutive elements (coalesced), accumulate in double like the reference
// rows do, and combine with a __shfl_xor butterfly. A reduction over a middle
// block of axes, [A, R, B] with B > 1, gives each (a, b) pair to one lane and
// walks R with stride B, so neighbouring lanes still read neighbouring
// addresses. Anything else falls back to a per-output walk over the reduced
// index space.
//
// Semantics follow the reference rows: sums of float32 in double rounded once
// (src/kernels/reduce_sum.cpp:33-70, reduce_mean.cpp:180-197), ReduceMax
// starting from the lowest float with std::max so NaN never wins
// (reduce_max.cpp:152-165), ReduceL2 as sqrt of a double sum of squares
// (reduce_l2.cpp:63-80), Softmax with the reference's float peak rule
// (softmax.cpp:98-119; its exponentials are double, ours fp32 with a double
// sum: within 1e-6 relative, far inside the 1e-4 bar, and the rows stay
// memory-bound), LayerNorm/InstanceNorm two-pass double statistics
// (layer_normalization.cpp:134-159, instance_normalization.cpp:80-103),
// ArgMax's sequential first/last-maximum rule (arg_max.cpp:41-57) and
// CumSum's sequential scan (cum_sum.cpp:40-70), and a block scan per row
// when the scan axis is contiguous.

#include "common.hpp"
#include "../../include/nert_hip.h"

#include <vector>

namespace nert_hip {
namespace {

constexpr int kMaxRank = 8;

template <typename T>
__device__ __forceinline__ T WaveAllSum(T v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        v += __shfl_xor(v, off, 64);
    }
    return v;
}

__device__ __forceinline__ float RefMax(float a, float b) { return (a < b) ? b : a; } // std::max(a, b)

struct ReduceShape {
    int kept_rank;
    int red_rank;
    int64_t kept_dims[kMaxRank];
    int64_t kept_strides[kMaxRank];
    int64_t red_dims[kMaxRank];
    int64_t red_strides[kMaxRank];
    int64_t red_count;
};

template <typename Acc>
struct OpState {
    Acc v;
};

// ---- contiguous rows: one wave per output ----------------------------------
template <int OP, typename T>
__global__ __launch_bounds__(256) void ReduceRowsKernel(const T* __restrict__ x, T* __restrict__ y, int64_t rows,
                                                        int64_t len) {
    const int lane = threadIdx.x & 63;
    const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) {
        return;
    }
    const T* p = x + row * len;
    if constexpr (OP == NERT_RED_MAX) {
        float best = -3.402823466e+38f;
        for (int64_t i = lane; i < len; i += 64) {
            best = RefMax(best, p[i]);
        }
        // NaN never wins std::max against a number, so the order of the
        // combination does not matter.
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            best = RefMax(best, __shfl_xor(best, off, 64));
        }
        if (lane == 0) {
            y[row] = best;
        }
    } else if constexpr (sizeof(T) == 8) { // int64 ReduceSum: exact wrap-around sum
        uint64_t sum = 0;
        for (int64_t i = lane; i < len; i += 64) {
            sum += static_cast<uint64_t>(p[i]);
        }
        sum = WaveAllSum(sum);
        if (lane == 0) {
            y[row] = static_cast<T>(sum);
        }
    } else {
        double sum = 0.0;
        for (int64_t i = lane; i < len; i += 64) {
            const double v = static_cast<double>(p[i]);
            sum += OP == NERT_RED_L2 ? v * v : v;
        }
        sum = WaveAllSum(sum);
        if (lane == 0) {
            double r = sum;
            if (OP == NERT_RED_MEAN) {
                r = sum / static_cast<double>(len);
            } else if (OP == NERT_RED_L2) {
                r = sqrt(sum);
            }
            y[row] = static_cast<T>(r);
        }
    }
}

// ---- [A, R, B]: one lane per (a, b) -----------------------------------------
template <int OP, typename T>
__global__ void ReduceColsKernel(const T* __restrict__ x, T* __restrict__ y, int64_t A, int64_t R, int64_t B) {
    const int64_t total = A * B;
    for (int64_t o = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; o < total;
         o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t a = o / B;
        const int64_t b = o - a * B;
        const T* p = x + a * R * B + b;
        if constexpr (OP == NERT_RED_MAX) {
            float best = -3.402823466e+38f;
            for (int64_t r = 0; r < R; ++r) {
                best = RefMax(best, p[r * B]);
            }
            y[o] = best;
        } else if constexpr (sizeof(T) == 8) {
            uint64_t sum = 0;
            for (int64_t r = 0; r < R; ++r) {
                sum += static_cast<uint64_t>(p[r * B]);
            }
            y[o] = static_cast<T>(sum);
        } else {
            double sum = 0.0;
            for (int64_t r = 0; r < R; ++r) {
                const double v = static_cast<double>(p[r * B]);
                sum += OP == NERT_RED_L2 ? v * v : v;
            }
            if (OP == NERT_RED_MEAN) {
                sum /= static_cast<double>(R);
            } else if (OP == NERT_RED_L2) {
                sum = sqrt(sum);
            }
            y[o] = static_cast<T>(sum);
        }
    }
}

// ---- general: one lane per output, decoded reduced index ----------------------
template <int OP, typename T>
__global__ void ReduceGeneralKernel(const T* __restrict__ x, T* __restrict__ y, ReduceShape s, int64_t outputs) {
    for (int64_t o = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; o < outputs;
         o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t base = 0;
        int64_t rem = o;
        for (int d = s.kept_rank - 1; d >= 0; --d) {
            const int64_t c = rem % s.kept_dims[d];
            rem /= s.kept_dims[d];
            base += c * s.kept_strides[d];
        }
        float best = -3.402823466e+38f;
        double sum = 0.0;
        uint64_t isum = 0;
        for (int64_t r = 0; r < s.red_count; ++r) {
            int64_t off = base;
            int64_t rr = r;
            for (int d = s.red_rank - 1; d >= 0; --d) {
                const int64_t c = rr % s.red_dims[d];
                rr /= s.red_dims[d];
                off += c * s.red_strides[d];
            }
            if constexpr (OP == NERT_RED_MAX) {
                best = RefMax(best, static_cast<float>(x[off]));
            } else if constexpr (sizeof(T) == 8) {
                isum += static_cast<uint64_t>(x[off]);
            } else {
                const double v = static_cast<double>(x[off]);
                sum += OP == NERT_RED_L2 ? v * v : v;
            }
        }
        if constexpr (OP == NERT_RED_MAX) {
            y[o] = static_cast<T>(best);
        } else if constexpr (sizeof(T) == 8) {
            y[o] = static_cast<T>(isum);
        } else {
            if (OP == NERT_RED_MEAN) {
                sum /= static_cast<double>(s.red_count);
            } else if (OP == NERT_RED_L2) {
                sum = sqrt(sum);
            }
            y[o] = static_cast<T>(sum);
        }
    }
}

template <int OP, typename T>
void LaunchReduce(const T* x, T* y, int rank, const int64_t* dims, const uint8_t* reduced, hipStream_t s) {
    // Collapse neighbouring axes with the same reduced flag.
    std::vector<int64_t> cd;
    std::vector<bool> cr;
    for (int d = 0; d < rank; ++d) {
        if (dims[d] == 1) {
            continue;
        }
        const bool r = reduced[d] != 0;
        if (!cd.empty() && cr.back() == r) {
            cd.back() *= dims[d];
        } else {
            cd.push_back(dims[d]);
            cr.push_back(r);
        }
    }
    int64_t outputs = 1;
    int64_t red = 1;
    for (size_t i = 0; i < cd.size(); ++i) {
        (cr[i] ? red : outputs) *= cd[i];
    }
    if (outputs == 0 || red == 0) {
        return;
    }
    const size_t n = cd.size();
    if (n == 0 || (n == 1 && cr[0]) || (n == 2 && !cr[0] && cr[1]) || (n == 1 && !cr[0])) {
        // [outputs, red] with red contiguous (red may be 1: a copy).
        const int64_t blocks = (outputs + 3) / 4;
        ReduceRowsKernel<OP, T><<<static_cast<unsigned>(blocks), 256, 0, s>>>(x, y, outputs, red);
    } else if ((n == 2 && cr[0] && !cr[1]) || (n == 3 && !cr[0] && cr[1] && !cr[2])) {
        const int64_t A = n == 3 ? cd[0] : 1;
        const int64_t R = n == 3 ? cd[1] : cd[0];
        const int64_t B = n == 3 ? cd[2] : cd[1];
        ReduceColsKernel<OP, T><<<GridFor(A * B, 256, 8192), 256, 0, s>>>(x, y, A, R, B);
    } else {
        ReduceShape sh{};
        std::vector<int64_t> strides(n, 1);
        for (size_t i = n; i-- > 1;) {
            strides[i - 1] = strides[i] * cd[i];
        }
        for (size_t i = 0; i < n; ++i) {
            if (cr[i]) {
                if (sh.red_rank >= kMaxRank) {
                    throw Error("reduce: too many reduced axis groups");
                }
                sh.red_dims[sh.red_rank] = cd[i];
                sh.red_strides[sh.red_rank++] = strides[i];
            } else {
                if (sh.kept_rank >= kMaxRank) {
                    throw Error("reduce: too many kept axis groups");
                }
                sh.kept_dims[sh.kept_rank] = cd[i];
                sh.kept_strides[sh.kept_rank++] = strides[i];
            }
        }
        sh.red_count = red;
        ReduceGeneralKernel<OP, T><<<GridFor(outputs, 256, 8192), 256, 0, s>>>(x, y, sh, outputs);
    }
    CheckLaunch("reduce launch");
}

// ---- Softmax ---------------------------------------------------------------
// Rows along the last axis: one wave per row.
__global__ __launch_bounds__(256) void SoftmaxRowsKernel(const float* __restrict__ x, float* __restrict__ y,
                                                         int64_t rows, int64_t dim) {
    const int lane = threadIdx.x & 63;
    const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) {
        return;
    }
    const float* p = x + row * dim;
    float* q = y + row * dim;
    // Peak with the reference's rule (value > peak, starting at element 0):
    // NaN elements after the first never raise it, so a parallel max over the
    // non-NaN elements seeded with element 0 is the same value.
    const float first = p[0];
    float peak = first;
    for (int64_t i = lane; i < dim; i += 64) {
        const float v = p[i];
        peak = v > peak ? v : peak;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(peak, off, 64);
        peak = o > peak ? o : peak;
    }
    if (first != first) {
        peak = first;
    }
    double total = 0.0;
    for (int64_t i = lane; i < dim; i += 64) {
        total += static_cast<double>(expf(p[i] - peak));
    }
    total = WaveAllSum(total);
    const float inv = static_cast<float>(1.0 / total);
    for (int64_t i = lane; i < dim; i += 64) {
        q[i] = expf(p[i] - peak) * inv;
    }
}

// Rows of at most LANES * PER elements: the row is read once into registers
// and each exponential is computed once (the reference evaluates the same exp
// twice, so reusing it gives the same values). LANES = 32 puts two rows on
// each wave (shuffles of width 32 stay within a row's half): short rows then
// run on half as many waves, with twice the independent work per wave.
template <int PER, int LANES = 64>
__global__ __launch_bounds__(256) void SoftmaxRowsRegKernel(const float* __restrict__ x, float* __restrict__ y,
                                                            int64_t rows, int dim) {
    static_assert(LANES == 32 || LANES == 64, "a row takes a whole wave or half of one");
    const int lane = threadIdx.x & (LANES - 1);
    const int64_t row = blockIdx.x * static_cast<int64_t>(256 / LANES) + (threadIdx.x / LANES);
    if (row >= rows) {
        return;
    }
    const float* p = x + row * dim;
    float* q = y + row * dim;
    // Loads from clamped (always valid) addresses, then a select: every
    // load of the row is in flight at once instead of one guarded load
    // (and one memory round trip) after another.
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = lane + LANES * k;
        v[k] = p[i < dim ? i : dim - 1];
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        v[k] = lane + LANES * k < dim ? v[k] : -__builtin_huge_valf();
    }
    // Peak rule of the reference (value > peak from element 0): see
    // SoftmaxRowsKernel.
    const float first = __shfl(v[0], 0, LANES);
    float peak = first;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        peak = v[k] > peak ? v[k] : peak;
    }
#pragma unroll
    for (int off = LANES / 2; off > 0; off >>= 1) {
        const float o = __shfl_xor(peak, off, LANES);
        peak = o > peak ? o : peak;
    }
    if (first != first) {
        peak = first;
    }
    float e[PER];
    double total = 0.0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        e[k] = lane + LANES * k < dim ? expf(v[k] - peak) : 0.0f;
        total += static_cast<double>(e[k]);
    }
#pragma unroll
    for (int off = LANES / 2; off > 0; off >>= 1) {
        total += __shfl_xor(total, off, LANES);
    }
    const float inv = static_cast<float>(1.0 / total);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = lane + LANES * k;
        if (i < dim) {
            q[i] = e[k] * inv;
        }
    }
}

// Rows of up to 256 * PER elements, one 256-thread workgroup per row, held in
// registers (one read of the row; 16-byte loads and stores when VEC): peak and
// sum through the waves' shuffles and LDS, fp32 exponentials, double sum.
template <int PER, bool VEC>
__global__ __launch_bounds__(256) void SoftmaxRowsBlockKernel(const float* __restrict__ x, float* __restrict__ y,
                                                              int dim) {
    __shared__ float peaks[4];
    __shared__ double sums[4];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const float* p = x + static_cast<int64_t>(blockIdx.x) * dim;
    float* q = y + static_cast<int64_t>(blockIdx.x) * dim;
    float v[PER];
    // Element j of this thread: 4 * (tid + 256 * (j / 4)) + j % 4 (VEC) or
    // tid + 256 * j; clamped loads, then a select.
    auto index = [&](int j) { return VEC ? 4 * (tid + 256 * (j / 4)) + (j & 3) : tid + 256 * j; };
    if constexpr (VEC) {
#pragma unroll
        for (int j = 0; j < PER; j += 4) {
            const int i = 4 * (tid + 256 * (j / 4));
            const nert_floatx4 w = *reinterpret_cast<const nert_floatx4*>(p + (i < dim ? i : 0));
            v[j] = w[0];
            v[j + 1] = w[1];
            v[j + 2] = w[2];
            v[j + 3] = w[3];
        }
    } else {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = index(j);
            v[j] = p[i < dim ? i : dim - 1];
        }
    }
    const float first = p[0];
    float peak = first;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const float w = index(j) < dim ? v[j] : -__builtin_huge_valf();
        peak = w > peak ? w : peak;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(peak, off, 64);
        peak = o > peak ? o : peak;
    }
    if ((tid & 63) == 0) {
        peaks[wave] = peak;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        peak = peaks[w] > peak ? peaks[w] : peak;
    }
    if (first != first) {
        peak = first; // the reference's peak rule: see SoftmaxRowsKernel
    }
    double total = 0.0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        v[j] = index(j) < dim ? expf(v[j] - peak) : 0.0f;
        total += static_cast<double>(v[j]);
    }
    total = WaveAllSum(total);
    if ((tid & 63) == 0) {
        sums[wave] = total;
    }
    __syncthreads();
    total = (sums[0] + sums[1]) + (sums[2] + sums[3]);
    const float inv = static_cast<float>(1.0 / total);
    if constexpr (VEC) {
#pragma unroll
        for (int j = 0; j < PER; j += 4) {
            const int i = 4 * (tid + 256 * (j / 4));
            if (i < dim) {
                *reinterpret_cast<nert_floatx4*>(q + i) =
                    nert_floatx4{v[j] * inv, v[j + 1] * inv, v[j + 2] * inv, v[j + 3] * inv};
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = index(j);
            if (i < dim) {
                q[i] = v[j] * inv;
            }
        }
    }
}

// Normalised axis with inner > 1: one lane per (outer, inner) column.
__global__ void SoftmaxColsKernel(const float* __restrict__ x, float* __restrict__ y, int64_t outer, int64_t dim,
                                  int64_t inner) {
    const int64_t total_cols = outer * inner;
    for (int64_t c = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; c < total_cols;
         c += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t o = c / inner;
        const int64_t n = c - o * inner;
        const float* p = x + o * dim * inner + n;
        float* q = y + o * dim * inner + n;
        float peak = p[0];
        for (int64_t k = 1; k < dim; ++k) {
            const float v = p[k * inner];
            if (v > peak) {
                peak = v;
            }
        }
        double total = 0.0;
        for (int64_t k = 0; k < dim; ++k) {
            total += static_cast<double>(expf(p[k * inner] - peak));
        }
        const float inv = static_cast<float>(1.0 / total);
        for (int64_t k = 0; k < dim; ++k) {
            q[k * inner] = expf(p[k * inner] - peak) * inv;
        }
    }
}

// ---- LayerNorm / InstanceNorm ------------------------------------------------
// One wave per row: mean, then centred sum of squares, in double.
__global__ __launch_bounds__(256) void LayerNormKernel(const float* __restrict__ x, const float* __restrict__ scale,
                                                       int scale_scalar, const float* __restrict__ bias,
                                                       int bias_scalar, float* __restrict__ y, float* mean_out,
                                                       float* invstd_out, int64_t rows, int64_t inner, double eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) {
        return;
    }
    const float* p = x + row * inner;
    float* q = y + row * inner;
    double sum = 0.0;
    for (int64_t i = lane; i < inner; i += 64) {
        sum += static_cast<double>(p[i]);
    }
    const double mean = WaveAllSum(sum) / static_cast<double>(inner);
    double sq = 0.0;
    for (int64_t i = lane; i < inner; i += 64) {
        const double c = static_cast<double>(p[i]) - mean;
        sq += c * c;
    }
    const double inv = 1.0 / sqrt(WaveAllSum(sq) / static_cast<double>(inner) + eps);
    for (int64_t i = lane; i < inner; i += 64) {
        const double scaled = (static_cast<double>(p[i]) - mean) * inv * static_cast<double>(scale[scale_scalar ? 0 : i]);
        q[i] = static_cast<float>(bias != nullptr ? scaled + static_cast<double>(bias[bias_scalar ? 0 : i]) : scaled);
    }
    if (lane == 0) {
        if (mean_out != nullptr) {
            mean_out[row] = static_cast<float>(mean);
        }
        if (invstd_out != nullptr) {
            invstd_out[row] = static_cast<float>(inv);
        }
    }
}

// Rows of at most 64 * PER elements held in registers: one read of the row.
template <int PER>
__global__ __launch_bounds__(256) void LayerNormRegKernel(const float* __restrict__ x, const float* __restrict__ scale,
                                                          int scale_scalar, const float* __restrict__ bias,
                                                          int bias_scalar, float* __restrict__ y, float* mean_out,
                                                          float* invstd_out, int64_t rows, int inner, double eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) {
        return;
    }
    const float* p = x + row * inner;
    float* q = y + row * inner;
    // Clamped-address loads, then a select (see SoftmaxRowsRegKernel). Scale
    // and bias are read in the same batch as the row, unconditionally (a
    // scalar or absent operand reads element 0 of a valid array), so the three
    // streams of loads share one round trip to memory.
    const float* bsrc = bias != nullptr ? bias : scale;
    const int sstep = scale_scalar ? 0 : 1;
    const int bstep = bias == nullptr || bias_scalar ? 0 : 1;
    float v[PER];
    float sc[PER];
    float bi[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = lane + 64 * k;
        const int ic = i < inner ? i : inner - 1;
        v[k] = p[ic];
        sc[k] = scale[ic * sstep];
        bi[k] = bsrc[ic * bstep];
    }
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        v[k] = lane + 64 * k < inner ? v[k] : 0.0f;
        sum += static_cast<double>(v[k]);
    }
    const double mean = WaveAllSum(sum) / static_cast<double>(inner);
    double sq = 0.0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        if (lane + 64 * k < inner) {
            const double c = static_cast<double>(v[k]) - mean;
            sq += c * c;
        }
    }
    const double inv = 1.0 / sqrt(WaveAllSum(sq) / static_cast<double>(inner) + eps);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = lane + 64 * k;
        if (i < inner) {
            const double scaled = (static_cast<double>(v[k]) - mean) * inv * static_cast<double>(sc[k]);
            q[i] = static_cast<float>(bias != nullptr ? scaled + static_cast<double>(bi[k]) : scaled);
        }
    }
    if (lane == 0) {
        if (mean_out != nullptr) {
            mean_out[row] = static_cast<float>(mean);
        }
        if (invstd_out != nullptr) {
            invstd_out[row] = static_cast<float>(inv);
        }
    }
}

// Rows of at most 256 * Q elements (inner % 4 == 0, 16-byte aligned
// tensors, per-element or absent Scale and B): lane l holds the quads
// l, l + 64, ... of its row in registers, read and written with 16-byte
// accesses; the statistics are the two-pass double ones of
// LayerNormRegKernel. LayerNormQuadRow is the part after the row is in
// registers, shared by the plain kernel and the one that first adds two
// rows (FusedAddLayerNorm), so both normalise bit-identically.
template <int Q>
__device__ __forceinline__ void LayerNormQuadRow(const nert_floatx4 (&v)[Q], const nert_floatx4 (&sc)[Q],
                                                 const nert_floatx4 (&bi)[Q], bool has_bias, nert_floatx4* q,
                                                 float* mean_out, float* invstd_out, int64_t row, int inner,
                                                 double eps) {
    const int lane = threadIdx.x & 63;
    const int quads = inner / 4;
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < Q; ++k) {
        if (lane + 64 * k < quads) {
            sum += (static_cast<double>(v[k][0]) + static_cast<double>(v[k][1])) +
                   (static_cast<double>(v[k][2]) + static_cast<double>(v[k][3]));
        }
    }
    const double mean = WaveAllSum(sum) / static_cast<double>(inner);
    double sq = 0.0;
#pragma unroll
    for (int k = 0; k < Q; ++k) {
        if (lane + 64 * k < quads) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double c = static_cast<double>(v[k][e]) - mean;
                sq += c * c;
            }
        }
    }
    const double inv = 1.0 / sqrt(WaveAllSum(sq) / static_cast<double>(inner) + eps);
#pragma unroll
    for (int k = 0; k < Q; ++k) {
        const int i = lane + 64 * k;
        if (i < quads) {
            nert_floatx4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double scaled = (static_cast<double>(v[k][e]) - mean) * inv * static_cast<double>(sc[k][e]);
                o[e] = static_cast<float>(has_bias ? scaled + static_cast<double>(bi[k][e]) : scaled);
            }
            q[i] = o;
        }
    }
    if (lane == 0) {
        if (mean_out != nullptr) {
            mean_out[row] = static_cast<float>(mean);
        }
        if (invstd_out != nullptr) {
            invstd_out[row] = static_cast<float>(inv);
        }
    }
}

// Loads the quads of row `row` this lane owns from `src` (clamped addresses,
// always valid) into `out`.
template <int Q>
__device__ __forceinline__ void LoadQuads(const float* src, int quads, nert_floatx4 (&out)[Q]) {
    const int lane = threadIdx.x & 63;
    const nert_floatx4* p = reinterpret_cast<const nert_floatx4*>(src);
#pragma unroll
    for (int k = 0; k < Q; ++k) {
        const int i = lane + 64 * k;
        out[k] = p[i < quads ? i : quads - 1];
    }
}

template <int Q>
__global__ __launch_bounds__(256) void LayerNormQuadKernel(const float* __restrict__ x,
                                                           const float* __restrict__ scale,
                                                           const float* __restrict__ bias, float* __restrict__ y,
                                                           float* mean_out, float* invstd_out, int64_t rows,
                                                           int inner, double eps) {
    const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) {
        return;
    }
    const int quads = inner / 4;
    nert_floatx4 v[Q];
    nert_floatx4 sc[Q];
    nert_floatx4 bi[Q];
    LoadQuads<Q>(x + row * inner, quads, v);
    LoadQuads<Q>(scale, quads, sc);
    LoadQuads<Q>(bias != nullptr ? bias : scale, quads, bi);
    LayerNormQuadRow<Q>(v, sc, bi, bias != nullptr, reinterpret_cast<nert_floatx4*>(y + row * inner), mean_out,
                        invstd_out, row, inner, eps);
}

// FusedAddLayerNorm: s = a + b (float, as the Add row rounds it), written to
// `sum`, then LayerNorm of s into y -- one read of each operand instead of
// writing s and reading it back.
template <int Q>
__global__ __launch_bounds__(256) void AddLayerNormQuadKernel(const float* __restrict__ a,
                                                              const float* __restrict__ b,
                                                              const float* __restrict__ scale,
                                                              const float* __restrict__ bias,
                                                              float* __restrict__ sum, float* __restrict__ y,
                                                              int64_t rows, int inner, double eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) {
        return;
    }
    const int quads = inner / 4;
    nert_floatx4 v[Q];
    nert_floatx4 w[Q];
    nert_floatx4 sc[Q];
    nert_floatx4 bi[Q];
    LoadQuads<Q>(a + row * inner, quads, v);
    LoadQuads<Q>(b + row * inner, quads, w);
    LoadQuads<Q>(scale, quads, sc);
    LoadQuads<Q>(bias != nullptr ? bias : scale, quads, bi);
    nert_floatx4* s4 = reinterpret_cast<nert_floatx4*>(sum + row * inner);
#pragma unroll
    for (int k = 0; k < Q; ++k) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[k][e] = __fadd_rn(v[k][e], w[k][e]);
        }
        if (lane + 64 * k < quads) {
            s4[lane + 64 * k] = v[k];
        }
    }
    LayerNormQuadRow<Q>(v, sc, bi, bias != nullptr, reinterpret_cast<nert_floatx4*>(y + row * inner), nullptr,
                        nullptr, row, inner, eps);
}

__global__ void AddFlatKernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ s,
                              int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        s[i] = __fadd_rn(a[i], b[i]);
    }
}

template <typename T>
__device__ __forceinline__ T BlockSum(T v, T* smem) {
    v = WaveAllSum(v);
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) {
        smem[wave] = v;
    }
    __syncthreads();
    T total = 0;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) {
        total += smem[w];
    }
    return total;
}

// One 256-thread block per (n, c) plane.
__global__ __launch_bounds__(256) void InstanceNormKernel(const float* __restrict__ x, const float* __restrict__ scale,
                                                          const float* __restrict__ bias, float* __restrict__ y,
                                                          int64_t channels, int64_t spatial, double eps) {
    __shared__ double smem[4];
    const int64_t plane = blockIdx.x;
    const int64_t c = plane % channels;
    const float* p = x + plane * spatial;
    float* q = y + plane * spatial;
    double sum = 0.0;
    for (int64_t i = threadIdx.x; i < spatial; i += blockDim.x) {
        sum += static_cast<double>(p[i]);
    }
    const double mean = BlockSum(sum, smem) / static_cast<double>(spatial);
    double sq = 0.0;
    for (int64_t i = threadIdx.x; i < spatial; i += blockDim.x) {
        const double d = static_cast<double>(p[i]) - mean;
        sq += d * d;
    }
    const double inv = 1.0 / sqrt(BlockSum(sq, smem) / static_cast<double>(spatial) + eps);
    const double s = static_cast<double>(scale[c]);
    const double b = static_cast<double>(bias[c]);
    for (int64_t i = threadIdx.x; i < spatial; i += blockDim.x) {
        q[i] = static_cast<float>((static_cast<double>(p[i]) - mean) * inv * s + b);
    }
}

// Register-resident InstanceNorm: a group of GROUP threads (one wave, or the
// whole 256-thread block) owns a plane of at most GROUP * PER elements, reads
// it once into registers (clamped loads, masked afterwards), and forms the
// double mean, then the double sum of squared deviations, from the registers:
// one HBM read and one write per element.
template <int GROUP, int PER>
__global__ __launch_bounds__(256) void InstanceNormResidentKernel(const float* __restrict__ x,
                                                                  const float* __restrict__ scale,
                                                                  const float* __restrict__ bias,
                                                                  float* __restrict__ y, int64_t channels,
                                                                  int64_t spatial, int64_t planes, double eps) {
    __shared__ double smem[4];
    constexpr int kPlanesPerBlock = 256 / GROUP;
    const int t = static_cast<int>(threadIdx.x) % GROUP;
    const int64_t plane = static_cast<int64_t>(blockIdx.x) * kPlanesPerBlock + threadIdx.x / GROUP;
    if (GROUP == 64 && plane >= planes) {
        return; // whole waves leave; the wave kernel has no block barrier
    }
    const int64_t c = plane % channels;
    const float* p = x + plane * spatial;
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int64_t i = t + static_cast<int64_t>(k) * GROUP;
        v[k] = p[i < spatial ? i : spatial - 1];
    }
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        if (t + static_cast<int64_t>(k) * GROUP < spatial) {
            sum += static_cast<double>(v[k]);
        }
    }
    sum = GROUP == 64 ? WaveAllSum(sum) : BlockSum(sum, smem);
    const double mean = sum / static_cast<double>(spatial);
    double sq = 0.0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        if (t + static_cast<int64_t>(k) * GROUP < spatial) {
            const double d = static_cast<double>(v[k]) - mean;
            sq += d * d;
        }
    }
    sq = GROUP == 64 ? WaveAllSum(sq) : BlockSum(sq, smem);
    const double inv = 1.0 / sqrt(sq / static_cast<double>(spatial) + eps);
    const double sc = static_cast<double>(scale[c]);
    const double bi = static_cast<double>(bias[c]);
    float* q = y + plane * spatial;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int64_t i = t + static_cast<int64_t>(k) * GROUP;
        if (i < spatial) {
            q[i] = static_cast<float>((static_cast<double>(v[k]) - mean) * inv * sc + bi);
        }
    }
}

// Split-plane InstanceNorm for planes larger than one block holds: blockIdx.y
// is the plane, blockIdx.x a chunk of kInChunk elements. PASS 0 writes each
// chunk's double sum; PASS 1 forms the mean from those (in chunk order) and
// writes each chunk's sum of squared deviations; PASS 2 forms mean and
// inverse deviation the same way and normalises the chunk.
constexpr int kInPer = 16;
constexpr int kInChunk = 256 * kInPer;

template <int PASS>
__global__ __launch_bounds__(256) void InstanceNormSplitKernel(const float* __restrict__ x,
                                                               const float* __restrict__ scale,
                                                               const float* __restrict__ bias, float* __restrict__ y,
                                                               double* __restrict__ partial, int64_t channels,
                                                               int64_t spatial, int chunks, double eps) {
    __shared__ double smem[4];
    __shared__ double stats[2];
    const int64_t plane = blockIdx.y;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kInChunk;
    const float* p = x + plane * spatial;
    double* sums = partial + plane * chunks;
    double* sqs = partial + (static_cast<int64_t>(gridDim.y) + plane) * chunks;
    float v[kInPer];
#pragma unroll
    for (int k = 0; k < kInPer; ++k) {
        const int64_t i = base + threadIdx.x + k * 256;
        v[k] = p[i < spatial ? i : spatial - 1];
    }
    if (PASS > 0) {
        // Every block of the plane folds the chunk partials the same way
        // (strided per thread, then the block tree), so all agree bit for bit.
        double total = 0.0;
        double sq = 0.0;
        for (int j = threadIdx.x; j < chunks; j += 256) {
            total += sums[j];
            if (PASS == 2) {
                sq += sqs[j];
            }
        }
        total = BlockSum(total, smem);
        if (PASS == 2) {
            sq = BlockSum(sq, smem);
        }
        if (threadIdx.x == 0) {
            stats[0] = total / static_cast<double>(spatial);
            stats[1] = PASS == 2 ? 1.0 / sqrt(sq / static_cast<double>(spatial) + eps) : 0.0;
        }
        __syncthreads();
    }
    const double mean = PASS > 0 ? stats[0] : 0.0;
    if (PASS < 2) {
        double acc = 0.0;
#pragma unroll
        for (int k = 0; k < kInPer; ++k) {
            if (base + threadIdx.x + k * 256 < spatial) {
                const double d = static_cast<double>(v[k]) - mean;
                acc += PASS == 0 ? static_cast<double>(v[k]) : d * d;
            }
        }
        acc = BlockSum(acc, smem);
        if (threadIdx.x == 0) {
            (PASS == 0 ? sums : sqs)[blockIdx.x] = acc;
        }
        return;
    }
    const int64_t c = plane % channels;
    const double inv = stats[1];
    const double sc = static_cast<double>(scale[c]);
    const double bi = static_cast<double>(bias[c]);
    float* q = y + plane * spatial;
#pragma unroll
    for (int k = 0; k < kInPer; ++k) {
        const int64_t i = base + threadIdx.x + k * 256;
        if (i < spatial) {
            q[i] = static_cast<float>((static_cast<double>(v[k]) - mean) * inv * sc + bi);
        }
    }
}

// ---- ArgMax ----------------------------------------------------------------
// Sequential rule: index i replaces the best when v > best, or (last) when
// v == best; so NaN never wins after index 0 and a NaN at index 0 wins.
template <typename T>
__device__ __forceinline__ bool Beats(T v, int64_t i, T bv, int64_t bi, bool last) {
    // Combination of two candidates where bi < i in scan order.
    return v > bv || (last && v == bv);
}

template <typename T>
__global__ void ArgMaxKernel(const T* __restrict__ x, int64_t* __restrict__ y, int64_t outer, int64_t dim,
                             int64_t inner, int last) {
    const int64_t total = outer * inner;
    for (int64_t c = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; c < total;
         c += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t o = c / inner;
        const int64_t n = c - o * inner;
        const T* p = x + o * dim * inner + n;
        int64_t best = 0;
        T bv = p[0];
        for (int64_t i = 1; i < dim; ++i) {
            const T v = p[i * inner];
            if (v > bv || (last && v == bv)) {
                bv = v;
                best = i;
            }
        }
        y[c] = best;
    }
}

// inner == 1 and long rows: one wave per row. Each lane scans a strided
// subsequence in order, then candidates are merged in index order with the
// same rule; a NaN at index 0 short-circuits to 0.
template <typename T>
__global__ __launch_bounds__(256) void ArgMaxRowsKernel(const T* __restrict__ x, int64_t* __restrict__ y,
                                                        int64_t rows, int64_t dim, int last) {
    const int lane = threadIdx.x & 63;
    const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) {
        return;
    }
    const T* p = x + row * dim;
    const T first = p[0];
    int64_t bi = -1;
    T bv = first;
    for (int64_t i = lane; i < dim; i += 64) {
        const T v = p[i];
        if (v == v && (bi < 0 || v > bv || (last && v == bv))) {
            bv = v;
            bi = i;
        }
    }
    // Merge: prefer the larger value; on ties the smaller index (first) or
    // the larger index (last). Lanes without a non-NaN candidate lose.
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const T ov = __shfl_xor(bv, off, 64);
        const int64_t oi = __shfl_xor(bi, off, 64);
        bool take;
        if (oi < 0) {
            take = false;
        } else if (bi < 0) {
            take = true;
        } else if (ov != bv) {
            take = ov > bv;
        } else {
            take = last ? oi > bi : oi < bi;
        }
        if (take) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        y[row] = (first != first || bi < 0) ? 0 : bi;
    }
}

// ---- CumSum ----------------------------------------------------------------
template <typename T, typename Acc>
__global__ void CumSumKernel(const T* __restrict__ x, T* __restrict__ y, int64_t outer, int64_t dim, int64_t inner,
                             int exclusive, int reverse) {
    const int64_t total = outer * inner;
    for (int64_t c = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; c < total;
         c += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t o = c / inner;
        const int64_t n = c - o * inner;
        Acc run = Acc{};
        for (int64_t s = 0; s < dim; ++s) {
            const int64_t i = reverse ? dim - 1 - s : s;
            const int64_t idx = (o * dim + i) * inner + n;
            if (exclusive) {
                y[idx] = static_cast<T>(run);
                run += static_cast<Acc>(x[idx]);
            } else {
                run += static_cast<Acc>(x[idx]);
                y[idx] = static_cast<T>(run);
            }
        }
    }
}

// Contiguous scan axis (inner == 1): one workgroup per row scans it in
// chunks of 1024 positions, four consecutive positions per thread: each
// thread's running sum over its four, a block-wide exclusive scan of the
// thread totals (wave shuffles, then the four wave totals), plus the carry of
// the chunks before. Sums in Acc (double for float rows, like the sequential
// kernel; the association differs only inside double precision).
template <typename T, typename Acc>
__global__ __launch_bounds__(256) void CumSumRowsKernel(const T* __restrict__ x, T* __restrict__ y, int64_t dim,
                                                        int exclusive, int reverse) {
    constexpr int kPer = 4;
    __shared__ Acc wave_total[4];
    const int64_t row = blockIdx.x;
    const T* xr = x + row * dim;
    T* yr = y + row * dim;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    Acc carry = Acc{};
    for (int64_t base = 0; base < dim; base += 256 * kPer) {
        Acc v[kPer];
        Acc total = Acc{};
#pragma unroll
        for (int e = 0; e < kPer; ++e) {
            const int64_t pos = base + threadIdx.x * kPer + e; // position in scan order
            v[e] = pos < dim ? static_cast<Acc>(xr[reverse ? dim - 1 - pos : pos]) : Acc{};
            total += v[e];
        }
        Acc incl = total;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const Acc up = __shfl_up(incl, off, 64);
            if (lane >= off) {
                incl += up;
            }
        }
        if (lane == 63) {
            wave_total[wave] = incl;
        }
        __syncthreads();
        Acc before = carry + (incl - total);
        Acc block_total = Acc{};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            before += w < wave ? wave_total[w] : Acc{};
            block_total += wave_total[w];
        }
        __syncthreads(); // wave_total is rewritten by the next chunk
        Acc run = before;
#pragma unroll
        for (int e = 0; e < kPer; ++e) {
            const int64_t pos = base + threadIdx.x * kPer + e;
            const Acc out = exclusive ? run : run + v[e];
            run += v[e];
            if (pos < dim) {
                yr[reverse ? dim - 1 - pos : pos] = static_cast<T>(out);
            }
        }
        carry += block_total;
    }
}

unsigned RowBlocks(int64_t rows) {
    const int64_t b = (rows + 3) / 4;
    if (b > 0x7FFFFFFF) {
        throw Error("too many rows");
    }
    return static_cast<unsigned>(b < 1 ? 1 : b);
}

// Blocks of 256 threads for two rows per wave (eight rows per block).
unsigned PairRowBlocks(int64_t rows) {
    const int64_t b = (rows + 7) / 8;
    if (b > 0x7FFFFFFF) {
        throw Error("too many rows");
    }
    return static_cast<unsigned>(b < 1 ? 1 : b);
}

} // namespace
} // namespace nert_hip

using namespace nert_hip;

extern "C" {

int nert_hip_reduce(int op, int dtype, const void* x, void* y, int rank, const int64_t* dims, const uint8_t* reduced,
                    void* stream) {
    return Guard([&] {
        hipStream_t s = StreamOr(stream);
        if (dtype == NERT_I64) {
            if (op != NERT_RED_SUM) {
                throw Error("reduce: int64 supports sum only");
            }
            LaunchReduce<NERT_RED_SUM, int64_t>(static_cast<const int64_t*>(x), static_cast<int64_t*>(y), rank, dims,
                                                reduced, s);
            return;
        }
        const float* xf = static_cast<const float*>(x);
        float* yf = static_cast<float*>(y);
        switch (op) {
        case NERT_RED_SUM:
            LaunchReduce<NERT_RED_SUM, float>(xf, yf, rank, dims, reduced, s);
            break;
        case NERT_RED_MEAN:
            LaunchReduce<NERT_RED_MEAN, float>(xf, yf, rank, dims, reduced, s);
            break;
        case NERT_RED_MAX:
            LaunchReduce<NERT_RED_MAX, float>(xf, yf, rank, dims, reduced, s);
            break;
        case NERT_RED_L2:
            LaunchReduce<NERT_RED_L2, float>(xf, yf, rank, dims, reduced, s);
            break;
        default:
            throw Error("reduce: unknown op");
        }
    });
}

int nert_hip_softmax_f32(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner, void* stream) {
    return Guard([&] {
        if (outer * dim * inner == 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        if (inner == 1 && dim <= 224) {
            SoftmaxRowsRegKernel<7, 32><<<PairRowBlocks(outer), 256, 0, s>>>(x, y, outer, static_cast<int>(dim));
        } else if (inner == 1 && dim <= 256) {
            SoftmaxRowsRegKernel<4><<<RowBlocks(outer), 256, 0, s>>>(x, y, outer, static_cast<int>(dim));
        } else if (inner == 1 && dim <= 1024) {
            SoftmaxRowsRegKernel<16><<<RowBlocks(outer), 256, 0, s>>>(x, y, outer, static_cast<int>(dim));
        } else if (inner == 1 && dim <= 4096 && outer <= 0x7FFFFFFF) {
            const bool vec = dim % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                             (reinterpret_cast<uintptr_t>(y) & 15) == 0;
            if (vec) {
                SoftmaxRowsBlockKernel<16, true><<<static_cast<unsigned>(outer), 256, 0, s>>>(x, y,
                                                                                             static_cast<int>(dim));
            } else {
                SoftmaxRowsBlockKernel<16, false><<<static_cast<unsigned>(outer), 256, 0, s>>>(x, y,
                                                                                              static_cast<int>(dim));
            }
        } else if (inner == 1) {
            SoftmaxRowsKernel<<<RowBlocks(outer), 256, 0, s>>>(x, y, outer, dim);
        } else {
            SoftmaxColsKernel<<<GridFor(outer * inner, 256, 8192), 256, 0, s>>>(x, y, outer, dim, inner);
        }
        CheckLaunch("softmax launch");
    });
}

int nert_hip_layernorm_f32(const float* x, const float* scale, int scale_scalar, const float* bias, int bias_scalar,
                           float* y, float* mean_out, float* invstd_out, int64_t rows, int64_t inner, double epsilon,
                           void* stream) {
    return Guard([&] {
        if (rows * inner == 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        const auto aligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
        const bool quad = inner % 4 == 0 && inner <= 1024 && !scale_scalar && (bias == nullptr || !bias_scalar) &&
                          aligned(x) && aligned(y) && aligned(scale) && (bias == nullptr || aligned(bias));
        if (quad) {
            // Q = quads per lane, exactly what the row needs (no idle loads).
            const int q = static_cast<int>((inner / 4 + 63) / 64);
            const int n = static_cast<int>(inner);
            const unsigned blocks = RowBlocks(rows);
            if (q == 1) {
                LayerNormQuadKernel<1><<<blocks, 256, 0, s>>>(x, scale, bias, y, mean_out, invstd_out, rows, n, epsilon);
            } else if (q == 2) {
                LayerNormQuadKernel<2><<<blocks, 256, 0, s>>>(x, scale, bias, y, mean_out, invstd_out, rows, n, epsilon);
            } else if (q == 3) {
                LayerNormQuadKernel<3><<<blocks, 256, 0, s>>>(x, scale, bias, y, mean_out, invstd_out, rows, n, epsilon);
            } else {
                LayerNormQuadKernel<4><<<blocks, 256, 0, s>>>(x, scale, bias, y, mean_out, invstd_out, rows, n, epsilon);
            }
        } else if (inner <= 256) {
            LayerNormRegKernel<4><<<RowBlocks(rows), 256, 0, s>>>(x, scale, scale_scalar, bias, bias_scalar, y,
                                                                  mean_out, invstd_out, rows, static_cast<int>(inner),
                                                                  epsilon);
        } else if (inner <= 1024) {
            LayerNormRegKernel<16><<<RowBlocks(rows), 256, 0, s>>>(x, scale, scale_scalar, bias, bias_scalar, y,
                                                                   mean_out, invstd_out, rows, static_cast<int>(inner),
                                                                   epsilon);
        } else {
            LayerNormKernel<<<RowBlocks(rows), 256, 0, s>>>(x, scale, scale_scalar, bias, bias_scalar, y, mean_out,
                                                            invstd_out, rows, inner, epsilon);
        }
        CheckLaunch("layernorm launch");
    });
}

int nert_hip_add_layernorm_f32(const float* a, const float* b, const float* scale, const float* bias, float* sum,
                               float* y, int64_t rows, int64_t inner, double epsilon, void* stream) {
    return Guard([&] {
        if (rows * inner == 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        const auto aligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
        const bool quad = inner % 4 == 0 && inner <= 1024 && aligned(a) && aligned(b) && aligned(scale) &&
                          (bias == nullptr || aligned(bias)) && aligned(sum) && aligned(y);
        if (!quad) {
            // The separate Add and LayerNormalization launches, as the rows run them.
            AddFlatKernel<<<GridFor(rows * inner, 256, 16384), 256, 0, s>>>(a, b, sum, rows * inner);
            CheckLaunch("add launch");
            if (nert_hip_layernorm_f32(sum, scale, 0, bias, 0, y, nullptr, nullptr, rows, inner, epsilon, stream) != 0) {
                throw Error(std::string(nert_hip_last_error()));
            }
            return;
        }
        const int q = static_cast<int>((inner / 4 + 63) / 64);
        const int n = static_cast<int>(inner);
        const unsigned blocks = RowBlocks(rows);
        if (q == 1) {
            AddLayerNormQuadKernel<1><<<blocks, 256, 0, s>>>(a, b, scale, bias, sum, y, rows, n, epsilon);
        } else if (q == 2) {
            AddLayerNormQuadKernel<2><<<blocks, 256, 0, s>>>(a, b, scale, bias, sum, y, rows, n, epsilon);
        } else if (q == 3) {
            AddLayerNormQuadKernel<3><<<blocks, 256, 0, s>>>(a, b, scale, bias, sum, y, rows, n, epsilon);
        } else {
            AddLayerNormQuadKernel<4><<<blocks, 256, 0, s>>>(a, b, scale, bias, sum, y, rows, n, epsilon);
        }
        CheckLaunch("add-layernorm launch");
    });
}

int nert_hip_instancenorm_f32(const float* x, const float* scale, const float* bias, float* y, int64_t batch,
                              int64_t channels, int64_t spatial, double epsilon, void* stream) {
    return Guard([&] {
        const int64_t planes = batch * channels;
        if (planes * spatial == 0) {
            return;
        }
        if (planes > 0x7FFFFFFF) {
            throw Error("instancenorm: too many planes");
        }
        hipStream_t s = StreamOr(stream);
        const unsigned wave_blocks = static_cast<unsigned>((planes + 3) / 4);
        const unsigned plane_blocks = static_cast<unsigned>(planes);
        if (spatial <= 256) {
            InstanceNormResidentKernel<64, 4><<<wave_blocks, 256, 0, s>>>(x, scale, bias, y, channels, spatial,
                                                                          planes, epsilon);
        } else if (spatial <= 1024) {
            InstanceNormResidentKernel<64, 16><<<wave_blocks, 256, 0, s>>>(x, scale, bias, y, channels, spatial,
                                                                           planes, epsilon);
        } else if (spatial <= 4096) {
            InstanceNormResidentKernel<256, 16><<<plane_blocks, 256, 0, s>>>(x, scale, bias, y, channels, spatial,
                                                                             planes, epsilon);
        } else if (spatial <= 8192) {
            InstanceNormResidentKernel<256, 32><<<plane_blocks, 256, 0, s>>>(x, scale, bias, y, channels, spatial,
                                                                             planes, epsilon);
        } else if (planes <= 65535 && (spatial + kInChunk - 1) / kInChunk <= 0x7FFFFFFF) {
            const int chunks = static_cast<int>((spatial + kInChunk - 1) / kInChunk);
            auto* partial = static_cast<double*>(Workspace(2 * planes * chunks * 8, s));
            const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(planes));
            InstanceNormSplitKernel<0><<<grid, 256, 0, s>>>(x, scale, bias, y, partial, channels, spatial, chunks,
                                                            epsilon);
            InstanceNormSplitKernel<1><<<grid, 256, 0, s>>>(x, scale, bias, y, partial, channels, spatial, chunks,
                                                            epsilon);
            InstanceNormSplitKernel<2><<<grid, 256, 0, s>>>(x, scale, bias, y, partial, channels, spatial, chunks,
                                                            epsilon);
        } else {
            InstanceNormKernel<<<plane_blocks, 256, 0, s>>>(x, scale, bias, y, channels, spatial, epsilon);
        }
        CheckLaunch("instancenorm launch");
    });
}

int nert_hip_argmax(int dtype, const void* x, int64_t* y, int64_t outer, int64_t dim, int64_t inner, int select_last,
                    void* stream) {
    return Guard([&] {
        if (outer * dim * inner == 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        if (inner == 1 && dim >= 256) {
            if (dtype == NERT_F32) {
                ArgMaxRowsKernel<float><<<RowBlocks(outer), 256, 0, s>>>(static_cast<const float*>(x), y, outer, dim,
                                                                          select_last);
            } else {
                ArgMaxRowsKernel<int64_t><<<RowBlocks(outer), 256, 0, s>>>(static_cast<const int64_t*>(x), y, outer,
                                                                            dim, select_last);
            }
        } else if (dtype == NERT_F32) {
            ArgMaxKernel<float><<<GridFor(outer * inner, 256, 8192), 256, 0, s>>>(static_cast<const float*>(x), y,
                                                                                   outer, dim, inner, select_last);
        } else {
            ArgMaxKernel<int64_t><<<GridFor(outer * inner, 256, 8192), 256, 0, s>>>(static_cast<const int64_t*>(x), y,
                                                                                     outer, dim, inner, select_last);
        }
        CheckLaunch("argmax launch");
    });
}

int nert_hip_cumsum(int dtype, const void* x, void* y, int64_t outer, int64_t dim, int64_t inner, int exclusive,
                    int reverse, void* stream) {
    return Guard([&] {
        if (outer * dim * inner == 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        if (inner == 1 && dim >= 64 && outer <= 0x7FFFFFFF) {
            if (dtype == NERT_F32) {
                CumSumRowsKernel<float, double><<<static_cast<unsigned>(outer), 256, 0, s>>>(
                    static_cast<const float*>(x), static_cast<float*>(y), dim, exclusive, reverse);
            } else {
                CumSumRowsKernel<int64_t, int64_t><<<static_cast<unsigned>(outer), 256, 0, s>>>(
                    static_cast<const int64_t*>(x), static_cast<int64_t*>(y), dim, exclusive, reverse);
            }
            CheckLaunch("cumsum launch");
            return;
        }
        if (dtype == NERT_F32) {
            CumSumKernel<float, double><<<GridFor(outer * inner, 256, 8192), 256, 0, s>>>(
                static_cast<const float*>(x), static_cast<float*>(y), outer, dim, inner, exclusive, reverse);
        } else {
            CumSumKernel<int64_t, int64_t><<<GridFor(outer * inner, 256, 8192), 256, 0, s>>>(
                static_cast<const int64_t*>(x), static_cast<int64_t*>(y), outer, dim, inner, exclusive, reverse);
        }
        CheckLaunch("cumsum launch");
    });
}

} // extern "C"
