// Bandwidth-bound elementwise rows: unary math, n-ary broadcast arithmetic,
// comparisons and logic, Where, Cast and fills.
//
// Contiguous unary maps move 16 bytes per lane per access (float4 / 2 x
// int64). Broadcasts are collapsed on the host (adjacent axes that every
// operand walks contiguously, or that every operand broadcasts, merge), so a
// typical residual Add or per-channel bias becomes a rank-1 or rank-2 index
// walk. Per-element semantics follow the reference rows exactly where they
// are observable: std::max/std::min NaN ordering (Relu(NaN) = 0, Max keeps the
// first operand's NaN), truncating int64 division and remainder, and the
// x86 result of an out-of-range float -> int64 conversion.

#include "common.hpp"
#include "../../include/nert_hip.h"

#include <cmath>
#include <vector>

namespace nert_hip {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxRank = 12;

// ---------------------------------------------------------------- unary ---

__device__ __forceinline__ float RefMax(float a, float b) { return (a < b) ? b : a; } // std::max(a, b)
__device__ __forceinline__ float RefMin(float a, float b) { return (b < a) ? b : a; } // std::min(a, b)

struct UnaryParams {
    int op;
    float f0, f1;
    int64_t i0, i1;
};

__device__ __forceinline__ float UnaryF32(int op, float x, const UnaryParams& p) {
    switch (op) {
    case NERT_UN_RELU:
        return RefMax(0.0f, x);
    case NERT_UN_SIGMOID:
        return SigmoidF32(x);
    case NERT_UN_TANH:
        return tanhf(x);
    case NERT_UN_EXP:
        return expf(x);
    case NERT_UN_LOG:
        return logf(x);
    case NERT_UN_SQRT:
        return sqrtf(x);
    case NERT_UN_SIN:
        return sinf(x);
    case NERT_UN_COS:
        return cosf(x);
    case NERT_UN_FLOOR:
        return floorf(x);
    case NERT_UN_ABS:
        return fabsf(x);
    case NERT_UN_NEG:
        return -x;
    case NERT_UN_SIGN:
        return x != x ? x : static_cast<float>((0.0f < x) - (x < 0.0f));
    case NERT_UN_ERF:
        return erff(x);
    case NERT_UN_ELU: {
        // The reference evaluates the negative branch in double.
        const double v = static_cast<double>(x);
        return v >= 0.0 ? x : static_cast<float>(static_cast<double>(p.f0) * (exp(v) - 1.0));
    }
    case NERT_UN_CLIP:
        return RefMin(RefMax(x, p.f0), p.f1);
    default:
        return x;
    }
}

__device__ __forceinline__ int64_t UnaryI64(int op, int64_t x, const UnaryParams& p) {
    switch (op) {
    case NERT_UN_ABS:
        return x < 0 ? static_cast<int64_t>(0ULL - static_cast<uint64_t>(x)) : x;
    case NERT_UN_NEG:
        return static_cast<int64_t>(0ULL - static_cast<uint64_t>(x));
    case NERT_UN_SIGN:
        return (0 < x) - (x < 0);
    case NERT_UN_CLIP: {
        const int64_t lo = x < p.i0 ? p.i0 : x;
        return p.i1 < lo ? p.i1 : lo;
    }
    default:
        return x;
    }
}

__global__ void UnaryF32Kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n, UnaryParams p,
                               bool vec) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (vec) {
        const int64_t n4 = n / 4;
        const float4* x4 = reinterpret_cast<const float4*>(x);
        float4* y4 = reinterpret_cast<float4*>(y);
        for (int64_t j = i; j < n4; j += stride) {
            float4 v = x4[j];
            v.x = UnaryF32(p.op, v.x, p);
            v.y = UnaryF32(p.op, v.y, p);
            v.z = UnaryF32(p.op, v.z, p);
            v.w = UnaryF32(p.op, v.w, p);
            y4[j] = v;
        }
        for (int64_t j = n4 * 4 + i; j < n; j += stride) {
            y[j] = UnaryF32(p.op, x[j], p);
        }
        return;
    }
    for (; i < n; i += stride) {
        y[i] = UnaryF32(p.op, x[i], p);
    }
}

__global__ void UnaryI64Kernel(const int64_t* __restrict__ x, int64_t* __restrict__ y, int64_t n, UnaryParams p) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        y[i] = UnaryI64(p.op, x[i], p);
    }
}

__global__ void IsNanKernel(const float* __restrict__ x, uint8_t* __restrict__ y, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        const float v = x[i];
        y[i] = v != v ? 1 : 0;
    }
}

__global__ void NotKernel(const uint8_t* __restrict__ x, uint8_t* __restrict__ y, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        y[i] = x[i] != 0 ? 0 : 1;
    }
}

unsigned ElementGrid(int64_t n) { return GridFor(n, kBlock, 8192); }

// ------------------------------------------------------------ broadcast ---

struct BcastArgs {
    const void* in[3];
    void* out;
    int rank;
    int nin;
    int64_t dims[kMaxRank];
    int64_t strides[3][kMaxRank];
    int32_t* flags;
};

__device__ __forceinline__ void Offsets(const BcastArgs& a, int64_t i, int64_t off[3]) {
    off[0] = off[1] = off[2] = 0;
    for (int d = a.rank - 1; d >= 0; --d) {
        const int64_t dim = a.dims[d];
        const int64_t c = i % dim;
        i /= dim;
        off[0] += c * a.strides[0][d];
        off[1] += c * a.strides[1][d];
        off[2] += c * a.strides[2][d];
    }
}

template <typename T>
__device__ __forceinline__ T Arith(int op, T x, T z, int32_t* flags);

template <>
__device__ __forceinline__ float Arith<float>(int op, float x, float z, int32_t*) {
    switch (op) {
    case NERT_BIN_ADD:
        return x + z;
    case NERT_BIN_SUB:
        return x - z;
    case NERT_BIN_MUL:
        return x * z;
    case NERT_BIN_DIV:
        return x / z;
    case NERT_BIN_POW:
        return z == 2.0f ? x * x : powf(x, z);
    case NERT_BIN_MAX:
        return RefMax(x, z);
    case NERT_BIN_MIN:
        return RefMin(x, z);
    default:
        return 0.f;
    }
}

template <>
__device__ __forceinline__ int64_t Arith<int64_t>(int op, int64_t x, int64_t z, int32_t* flags) {
    switch (op) {
    case NERT_BIN_ADD:
        return static_cast<int64_t>(static_cast<uint64_t>(x) + static_cast<uint64_t>(z));
    case NERT_BIN_SUB:
        return static_cast<int64_t>(static_cast<uint64_t>(x) - static_cast<uint64_t>(z));
    case NERT_BIN_MUL:
        return static_cast<int64_t>(static_cast<uint64_t>(x) * static_cast<uint64_t>(z));
    case NERT_BIN_DIV:
    case NERT_BIN_MOD:
        if (z == 0) {
            atomicOr(flags, 1);
            return 0;
        }
        if (z == -1) { // avoid the INT64_MIN / -1 trap; wraps like two's complement
            return op == NERT_BIN_DIV ? static_cast<int64_t>(0ULL - static_cast<uint64_t>(x)) : 0;
        }
        return op == NERT_BIN_DIV ? x / z : x % z;
    case NERT_BIN_MAX:
        return x < z ? z : x;
    case NERT_BIN_MIN:
        return z < x ? z : x;
    default:
        return 0;
    }
}

template <typename T>
__device__ __forceinline__ bool Compare(int op, T x, T z) {
    switch (op) {
    case NERT_BIN_EQUAL:
        return x == z;
    case NERT_BIN_GREATER:
        return x > z;
    case NERT_BIN_LESS:
        return x < z;
    case NERT_BIN_GREATER_EQUAL:
        return x >= z;
    case NERT_BIN_LESS_EQUAL:
        return x <= z;
    default:
        return false;
    }
}

// Arithmetic: out has T; inputs 2 (or 3 for three-input Max/Min chains).
template <typename T>
__global__ void ArithKernel(BcastArgs a, int op, int64_t n) {
    const T* x = static_cast<const T*>(a.in[0]);
    const T* z = static_cast<const T*>(a.in[1]);
    T* y = static_cast<T*>(a.out);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t off[3];
        Offsets(a, i, off);
        y[i] = Arith<T>(op, x[off[0]], z[off[1]], a.flags);
    }
}

// Same-shape float fast path (both operands contiguous, no broadcast).
__global__ void ArithF32FlatKernel(const float* __restrict__ x, const float* __restrict__ z, float* __restrict__ y,
                                   int op, int64_t n, bool vec) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (vec) {
        const int64_t n4 = n / 4;
        for (int64_t j = i; j < n4; j += stride) {
            const float4 u = reinterpret_cast<const float4*>(x)[j];
            const float4 v = reinterpret_cast<const float4*>(z)[j];
            float4 r;
            r.x = Arith<float>(op, u.x, v.x, nullptr);
            r.y = Arith<float>(op, u.y, v.y, nullptr);
            r.z = Arith<float>(op, u.z, v.z, nullptr);
            r.w = Arith<float>(op, u.w, v.w, nullptr);
            reinterpret_cast<float4*>(y)[j] = r;
        }
        i += n4 * 4;
    }
    for (; i < n; i += stride) {
        y[i] = Arith<float>(op, x[i], z[i], nullptr);
    }
}

// Rank-2 float broadcast y[r, c] = x[r*xs0 + c*xs1] (op) z[r*zs0 + c*zs1]
// with the inner axis walked four at a time when every operand allows it.
// SMALL: fewer than 2^31 quads, row index by 32-bit multiply-shift.
template <bool SMALL>
__global__ void ArithF32Rank2Kernel(BcastArgs a, int op, int64_t rows, int64_t cols, FastDiv div_cols4) {
    const float* x = static_cast<const float*>(a.in[0]);
    const float* z = static_cast<const float*>(a.in[1]);
    float* y = static_cast<float*>(a.out);
    const int64_t xs0 = a.strides[0][0], xs1 = a.strides[0][1];
    const int64_t zs0 = a.strides[1][0], zs1 = a.strides[1][1];
    const int64_t cols4 = cols / 4;
    const int64_t total = rows * cols4;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total; i += stride) {
        int64_t r, c;
        if constexpr (SMALL) {
            uint32_t rem;
            r = DivMod(div_cols4, static_cast<uint32_t>(i), rem);
            c = static_cast<int64_t>(rem) * 4;
        } else {
            r = i / cols4;
            c = (i - r * cols4) * 4;
        }
        const float* xp = x + r * xs0 + c * xs1;
        const float* zp = z + r * zs0 + c * zs1;
        float4 u, v;
        if (xs1 == 1) {
            u = *reinterpret_cast<const float4*>(xp);
        } else {
            u = make_float4(xp[0], xp[0], xp[0], xp[0]);
        }
        if (zs1 == 1) {
            v = *reinterpret_cast<const float4*>(zp);
        } else {
            v = make_float4(zp[0], zp[0], zp[0], zp[0]);
        }
        float4 out;
        out.x = Arith<float>(op, u.x, v.x, nullptr);
        out.y = Arith<float>(op, u.y, v.y, nullptr);
        out.z = Arith<float>(op, u.z, v.z, nullptr);
        out.w = Arith<float>(op, u.w, v.w, nullptr);
        *reinterpret_cast<float4*>(y + r * cols + c) = out;
    }
}

template <typename T>
__global__ void CompareKernel(BcastArgs a, int op, int64_t n) {
    const T* x = static_cast<const T*>(a.in[0]);
    const T* z = static_cast<const T*>(a.in[1]);
    uint8_t* y = static_cast<uint8_t*>(a.out);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t off[3];
        Offsets(a, i, off);
        y[i] = Compare<T>(op, x[off[0]], z[off[1]]) ? 1 : 0;
    }
}

__global__ void LogicKernel(BcastArgs a, int op, int64_t n) {
    const uint8_t* x = static_cast<const uint8_t*>(a.in[0]);
    const uint8_t* z = static_cast<const uint8_t*>(a.in[1]);
    uint8_t* y = static_cast<uint8_t*>(a.out);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t off[3];
        Offsets(a, i, off);
        const bool u = x[off[0]] != 0;
        const bool v = z[off[1]] != 0;
        y[i] = (op == NERT_BIN_AND ? (u && v) : (u || v)) ? 1 : 0;
    }
}

template <typename T>
__global__ void WhereKernel(BcastArgs a, int64_t n) {
    const uint8_t* c = static_cast<const uint8_t*>(a.in[0]);
    const T* x = static_cast<const T*>(a.in[1]);
    const T* z = static_cast<const T*>(a.in[2]);
    T* y = static_cast<T*>(a.out);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t off[3];
        Offsets(a, i, off);
        y[i] = c[off[0]] != 0 ? x[off[1]] : z[off[2]];
    }
}

// Builds collapsed broadcast arguments. in_dims[k] are each operand's dims
// (any rank <= out rank, right-aligned), out_dims the broadcast shape.
BcastArgs Collapse(int nin, const void* const* ins, const int64_t* const* in_dims, const int* in_ranks, void* out,
                   int out_rank, const int64_t* out_dims) {
    // Aligned element strides per operand (0 = broadcast axis).
    std::vector<int64_t> dims(out_dims, out_dims + out_rank);
    std::vector<std::vector<int64_t>> st(nin, std::vector<int64_t>(out_rank, 0));
    for (int k = 0; k < nin; ++k) {
        int64_t s = 1;
        for (int j = out_rank - 1; j >= 0; --j) {
            const int src = j - (out_rank - in_ranks[k]);
            if (src < 0) {
                continue;
            }
            const int64_t d = in_dims[k][src];
            st[k][j] = (d == out_dims[j] && d != 1) ? s : 0;
            s *= d;
        }
    }
    // Drop unit output axes, then merge mergeable neighbours.
    std::vector<int64_t> cd;
    std::vector<std::vector<int64_t>> cs(nin);
    for (int j = 0; j < out_rank; ++j) {
        if (dims[j] == 1) {
            continue;
        }
        if (!cd.empty()) {
            bool merge = true;
            for (int k = 0; k < nin; ++k) {
                const int64_t prev = cs[k].back();
                const int64_t cur = st[k][j];
                if (!((prev == 0 && cur == 0) || (prev == cur * dims[j] && cur != 0))) {
                    merge = false;
                    break;
                }
            }
            if (merge) {
                cd.back() *= dims[j];
                for (int k = 0; k < nin; ++k) {
                    cs[k].back() = st[k][j];
                }
                continue;
            }
        }
        cd.push_back(dims[j]);
        for (int k = 0; k < nin; ++k) {
            cs[k].push_back(st[k][j]);
        }
    }
    if (cd.empty()) {
        cd.push_back(1);
        for (int k = 0; k < nin; ++k) {
            cs[k].push_back(0);
        }
    }
    if (static_cast<int>(cd.size()) > kMaxRank) {
        throw Error("broadcast: more than 12 non-mergeable axes");
    }
    BcastArgs a{};
    a.nin = nin;
    a.rank = static_cast<int>(cd.size());
    for (int d = 0; d < a.rank; ++d) {
        a.dims[d] = cd[d];
        for (int k = 0; k < nin; ++k) {
            a.strides[k][d] = cs[k][d];
        }
    }
    for (int k = 0; k < nin; ++k) {
        a.in[k] = ins[k];
    }
    a.out = out;
    return a;
}

bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Operand k of a rank-2 walk can be read four columns at a time: either it is
// constant along the columns, or contiguous with 16-byte aligned rows.
bool Rank2Vectorizable(const BcastArgs& a, int k) {
    const int64_t s0 = a.strides[k][0];
    const int64_t s1 = a.strides[k][1];
    return s1 == 0 || (s1 == 1 && s0 % 4 == 0 && Aligned16(a.in[k]));
}

void LaunchRank2(const BcastArgs& a, int op, hipStream_t s) {
    const int64_t quads = a.dims[0] * (a.dims[1] / 4);
    if (quads < (int64_t{1} << 31)) {
        ArithF32Rank2Kernel<true><<<ElementGrid(quads), kBlock, 0, s>>>(
            a, op, a.dims[0], a.dims[1], FastDiv::Make(static_cast<uint32_t>(a.dims[1] / 4)));
    } else {
        ArithF32Rank2Kernel<false><<<ElementGrid(quads), kBlock, 0, s>>>(a, op, a.dims[0], a.dims[1], FastDiv{});
    }
}

} // namespace
} // namespace nert_hip

using namespace nert_hip;

extern "C" {

int nert_hip_unary(int op, int dtype, const void* x, void* y, int64_t count, double p0, double p1, void* stream) {
    return Guard([&] {
        if (count <= 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        UnaryParams p{};
        p.op = op;
        if (op == NERT_UN_ISNAN) {
            IsNanKernel<<<ElementGrid(count), kBlock, 0, s>>>(static_cast<const float*>(x), static_cast<uint8_t*>(y),
                                                              count);
        } else if (op == NERT_UN_NOT) {
            NotKernel<<<ElementGrid(count), kBlock, 0, s>>>(static_cast<const uint8_t*>(x), static_cast<uint8_t*>(y),
                                                            count);
        } else if (dtype == NERT_F32) {
            p.f0 = static_cast<float>(p0);
            p.f1 = static_cast<float>(p1);
            const bool vec = Aligned16(x) && Aligned16(y);
            UnaryF32Kernel<<<ElementGrid(vec ? count / 4 + 1 : count), kBlock, 0, s>>>(
                static_cast<const float*>(x), static_cast<float*>(y), count, p, vec);
        } else if (dtype == NERT_I64) {
            p.i0 = static_cast<int64_t>(p0);
            p.i1 = static_cast<int64_t>(p1);
            UnaryI64Kernel<<<ElementGrid(count), kBlock, 0, s>>>(static_cast<const int64_t*>(x),
                                                                 static_cast<int64_t*>(y), count, p);
        } else {
            throw Error("unary: unsupported dtype");
        }
        CheckLaunch("unary launch");
    });
}

// int64 Clip needs exact 64-bit bounds, which a double cannot carry.
int nert_hip_clip_i64(const int64_t* x, int64_t* y, int64_t count, int64_t lo, int64_t hi, void* stream) {
    return Guard([&] {
        if (count <= 0) {
            return;
        }
        UnaryParams p{};
        p.op = NERT_UN_CLIP;
        p.i0 = lo;
        p.i1 = hi;
        UnaryI64Kernel<<<ElementGrid(count), kBlock, 0, StreamOr(stream)>>>(x, y, count, p);
        CheckLaunch("clip launch");
    });
}

int nert_hip_broadcast(int op, int dtype, int n_inputs, const void* const* inputs, const int64_t* const* input_dims,
                       const int* input_ranks, void* out, int out_rank, const int64_t* out_dims, void* stream) {
    return Guard([&] {
        if (n_inputs < 2 || n_inputs > 3) {
            throw Error("broadcast: two or three operands");
        }
        int64_t n = 1;
        for (int d = 0; d < out_rank; ++d) {
            n *= out_dims[d];
        }
        if (n <= 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        BcastArgs a = Collapse(n_inputs, inputs, input_dims, input_ranks, out, out_rank, out_dims);
        a.flags = ErrorFlags();
        const unsigned grid = ElementGrid(n);
        if (op == NERT_BIN_WHERE) {
            if (dtype == NERT_F32) {
                WhereKernel<float><<<grid, kBlock, 0, s>>>(a, n);
            } else {
                WhereKernel<int64_t><<<grid, kBlock, 0, s>>>(a, n);
            }
        } else if (op == NERT_BIN_AND || op == NERT_BIN_OR) {
            LogicKernel<<<grid, kBlock, 0, s>>>(a, op, n);
        } else if (op >= NERT_BIN_EQUAL && op <= NERT_BIN_LESS_EQUAL) {
            if (dtype == NERT_F32) {
                CompareKernel<float><<<grid, kBlock, 0, s>>>(a, op, n);
            } else {
                CompareKernel<int64_t><<<grid, kBlock, 0, s>>>(a, op, n);
            }
        } else if (dtype == NERT_F32) {
            const bool flat = a.rank == 1 && a.strides[0][0] == 1 && a.strides[1][0] == 1;
            if (flat) {
                const bool vec = Aligned16(inputs[0]) && Aligned16(inputs[1]) && Aligned16(out);
                ArithF32FlatKernel<<<ElementGrid(vec ? n / 4 + 1 : n), kBlock, 0, s>>>(
                    static_cast<const float*>(inputs[0]), static_cast<const float*>(inputs[1]),
                    static_cast<float*>(out), op, n, vec);
            } else if (a.rank == 2 && a.dims[1] % 4 == 0 && Aligned16(out) && Rank2Vectorizable(a, 0) &&
                       Rank2Vectorizable(a, 1)) {
                LaunchRank2(a, op, s);
            } else if (a.rank == 1 && a.dims[0] % 4 == 0 && Aligned16(out)) {
                // One operand a scalar: the rank-2 walk over a single row.
                BcastArgs r = a;
                r.rank = 2;
                r.dims[1] = a.dims[0];
                r.dims[0] = 1;
                for (int k = 0; k < 2; ++k) {
                    r.strides[k][1] = a.strides[k][0];
                    r.strides[k][0] = 0;
                }
                if (Rank2Vectorizable(r, 0) && Rank2Vectorizable(r, 1)) {
                    LaunchRank2(r, op, s);
                } else {
                    ArithKernel<float><<<grid, kBlock, 0, s>>>(a, op, n);
                }
            } else {
                ArithKernel<float><<<grid, kBlock, 0, s>>>(a, op, n);
            }
        } else if (dtype == NERT_I64) {
            ArithKernel<int64_t><<<grid, kBlock, 0, s>>>(a, op, n);
        } else {
            throw Error("broadcast: unsupported dtype");
        }
        CheckLaunch("broadcast launch");
    });
}

// Reads and clears the device error flags (synchronises the stream).
int nert_hip_take_error_flags(int32_t* flags_out, void* stream) {
    return Guard([&] {
        hipStream_t s = StreamOr(stream);
        int32_t* flags = ErrorFlags();
        // Under stream capture the check is deferred: the flag stays raised
        // and the first call after the captured work ran reports it.
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        Check(hipStreamIsCapturing(s, &capture), "hipStreamIsCapturing");
        if (capture != hipStreamCaptureStatusNone) {
            *flags_out = 0;
            return;
        }
        int32_t raised = 0;
        Check(hipMemcpyAsync(&raised, flags, sizeof(int32_t), hipMemcpyDeviceToHost, s), "hipMemcpyAsync(flags)");
        Check(hipStreamSynchronize(s), "hipStreamSynchronize");
        if (raised != 0) {
            const int32_t zero = 0;
            Check(hipMemcpyAsync(flags, &zero, sizeof(int32_t), hipMemcpyHostToDevice, s), "hipMemcpyAsync(flags)");
            Check(hipStreamSynchronize(s), "hipStreamSynchronize");
        }
        *flags_out = raised | PendingErrorFlags();
        PendingErrorFlags() = 0;
    });
}

} // extern "C"

// ----------------------------------------------------------------- cast ---

namespace nert_hip {
namespace {

__device__ __forceinline__ int64_t F32ToI64(float v) {
    // x86 cvttss2si semantics for static_cast<int64_t>(float): NaN and
    // out-of-range values give INT64_MIN.
    if (!(v >= -9223372036854775808.0f && v < 9223372036854775808.0f)) {
        return static_cast<int64_t>(0x8000000000000000ULL);
    }
    return static_cast<int64_t>(v);
}

__device__ __forceinline__ int64_t SaturateI32(float v) {
    const double d = static_cast<double>(v);
    if (d != d) {
        return 0;
    }
    if (d >= 2147483647.0) {
        return 2147483647LL;
    }
    if (d <= -2147483648.0) {
        return -2147483648LL;
    }
    return static_cast<int64_t>(d);
}

__global__ void CastKernel(const void* __restrict__ x, void* __restrict__ y, int64_t n, int src, int dst,
                           int to_int32) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        if (dst == NERT_F32) {
            float v;
            if (src == NERT_F32) {
                v = static_cast<const float*>(x)[i];
            } else if (src == NERT_I64) {
                v = static_cast<float>(static_cast<const int64_t*>(x)[i]);
            } else {
                v = static_cast<const uint8_t*>(x)[i] != 0 ? 1.0f : 0.0f;
            }
            static_cast<float*>(y)[i] = v;
        } else if (dst == NERT_I64) {
            int64_t v;
            if (src == NERT_F32) {
                const float f = static_cast<const float*>(x)[i];
                v = to_int32 ? SaturateI32(f) : F32ToI64(f);
            } else if (src == NERT_I64) {
                v = static_cast<const int64_t*>(x)[i];
                if (to_int32) {
                    v = v > 2147483647LL ? 2147483647LL : (v < -2147483648LL ? -2147483648LL : v);
                }
            } else {
                v = static_cast<const uint8_t*>(x)[i] != 0 ? 1 : 0;
            }
            static_cast<int64_t*>(y)[i] = v;
        } else {
            bool v;
            if (src == NERT_F32) {
                v = static_cast<const float*>(x)[i] != 0.0f;
            } else if (src == NERT_I64) {
                v = static_cast<const int64_t*>(x)[i] != 0;
            } else {
                v = static_cast<const uint8_t*>(x)[i] != 0;
            }
            static_cast<uint8_t*>(y)[i] = v ? 1 : 0;
        }
    }
}

template <typename T>
__global__ void FillKernel(T* __restrict__ y, int64_t n, T value) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        y[i] = value;
    }
}

} // namespace
} // namespace nert_hip

extern "C" {

int nert_hip_cast(int src_dtype, int dst_dtype, int to_int32, const void* x, void* y, int64_t count, void* stream) {
    return Guard([&] {
        if (count <= 0) {
            return;
        }
        CastKernel<<<ElementGrid(count), kBlock, 0, StreamOr(stream)>>>(x, y, count, src_dtype, dst_dtype, to_int32);
        CheckLaunch("cast launch");
    });
}

int nert_hip_fill(int dtype, void* y, int64_t count, double fvalue, int64_t ivalue, void* stream) {
    return Guard([&] {
        if (count <= 0) {
            return;
        }
        hipStream_t s = StreamOr(stream);
        if (dtype == NERT_F32) {
            FillKernel<float><<<ElementGrid(count), kBlock, 0, s>>>(static_cast<float*>(y), count,
                                                                    static_cast<float>(fvalue));
        } else if (dtype == NERT_I64) {
            FillKernel<int64_t><<<ElementGrid(count), kBlock, 0, s>>>(static_cast<int64_t*>(y), count, ivalue);
        } else {
            FillKernel<uint8_t><<<ElementGrid(count), kBlock, 0, s>>>(static_cast<uint8_t*>(y), count,
                                                                      static_cast<uint8_t>(ivalue != 0 ? 1 : 0));
        }
        CheckLaunch("fill launch");
    });
}

} // extern "C"
