// Conv as an implicit GEMM on fp32 MFMA.
//
// Per group g:  Y_g[m, n] = sum_k W_g[m, k] * X_col[k, n] + bias[m]
//   m = output channel within the group        (M_g = M / group)
//   k = (c, kd, kh, kw), c within the group     (K_g = C/group * kD*kH*kW)
//   n = (b, od, oh, ow)                         (N = batch * OD*OH*OW)
// W is already [M, K_g] row-major (ONNX OIHW), so it loads like a row-major
// GEMM operand. X_col is never materialised: the B loader gathers each
// element from NCHW X with the stride/dilation/pad arithmetic and writes zero
// for padding taps, exactly the taps the reference skips
// (src/kernels/conv.cpp:267-285). 1-D and 2-D convolutions arrive lifted to
// three spatial axes with unit leading extents, as the reference lifts them
// (src/kernels/conv.cpp:233-249).
//
// The gather is arranged so almost all index arithmetic is scalar: every
// lane of a wave loads the same k row of the B tile (consecutive n across the
// lanes), so the (c, kd, kh, kw) decode of k is wave-uniform and runs on the
// SALU, with compile-time divisors for 1x1, 3x3 and 7x7 kernels and
// multiply-shift division otherwise. Per gathered element a lane does two
// adds, a bounds test and one load. Pointwise stride-1 unpadded convolutions
// skip the gather and run as a batched GEMM on the same engine.

#include <array>
#include <cmath>
#include <cstdlib>
#include <map>
#include <mutex>
#include <type_traits>

#include "gemm_engine.hpp"
#include "tune.hpp"
#include "mfma_tile.hpp"
#include "../../include/nert_hip.h"

namespace nert_hip {
namespace {

struct ConvArgs {
    const float* x;
    const float* w;
    // W again in the order the 3x3 LDS-patch kernel stores it, or null: per
    // output channel, blocks of 8 input channels, in a block the taps, in a
    // tap the 8 channels ([M][C_g / 8][KH * KW][8]); that kernel then copies
    // it to LDS with 16-byte stores instead of transposing 4-byte ones.
    // Every other kernel reads `w`.
    const float* w_packed;
    const float* bias;
    float* y;
    int64_t batch, c, m, group;
    int64_t cg, mg, kg; // channels per group, outputs per group, K per group
    int32_t in_d, in_h, in_w;
    int32_t k_d, k_h, k_w;
    int32_t out_d, out_h, out_w;
    int32_t s_d, s_h, s_w;
    int32_t d_d, d_h, d_w;
    int32_t p_d, p_h, p_w;
    int64_t plane_out; // OD*OH*OW
    int64_t plane_in;  // ID*IH*IW
    int64_t n_total;   // batch * plane_out
    FastDiv div_kvol, div_khw, div_kw;
    int64_t k_per_split;
    float* partial; // [splits][group][M_g][N] when split
    // Optional epilogue (fused rows): y = act(acc + bias + residual), in that
    // order, so the result equals Conv, then Add, then the activation rows
    // bit for bit.
    const float* residual; // same layout as y, or null
    int32_t act;           // 0 none, 1 Relu, 2 SiLU (x * Sigmoid(x))
    // Split tiles of the gather kernels finished inside the kernel
    // (FinishSplitTile) instead of through `partial`: counters per
    // [group][tile], slots [group * tiles + tile][split][BM * BN].
    uint32_t* split_counters;
    float* split_slots;
};

// The fused activation, each step rounded as the separate rows round it:
// Relu is std::max(0.0f, v) (NaN maps to 0 like the reference Relu); SiLU is
// the Sigmoid row's SigmoidF32(v) followed by the Mul row's product.
__device__ __forceinline__ float Activate(int act, float v) {
    if (act == 1) {
        return (0.0f < v) ? v : 0.0f;
    }
    if (act == 2) {
        return __fmul_rn(v, SigmoidF32(v));
    }
    return v;
}

__device__ __forceinline__ float Finish(const ConvArgs& p, float v, int64_t y_index) {
    if (p.residual != nullptr) {
        v = v + p.residual[y_index];
    }
    return Activate(p.act, v);
}

// Gathers B(k, n) = X_col for one K tile. Thread t owns column nn = t % BN for
// every pass (the column decode happens once per block); rows are assigned
// so that each wave's lanes share one k.
template <int BN, int BK, int THREADS, int PITCH, int KH, int KW, bool CHECKED>
struct ConvBLoader {
    static_assert(THREADS % BN == 0 && BN % 64 == 0, "a wave must cover part of one B row");
    static constexpr int kRowsPerPass = THREADS / BN;
    static constexpr int kPer = BK / kRowsPerPass;
    struct Stage {
        float v[kPer];
    };
    const ConvArgs* p;
    const float* xb;       // X at (b, g*C_g, 0, 0, 0) for this thread's column
    int64_t col_off;       // (id0*IH + ih0)*IW + iw0, may be negative
    int32_t id0, ih0, iw0; // window origin of this thread's output position
    bool col_ok;
    int32_t kk0; // this wave's first row within a tile (wave-uniform)
    int64_t k_total;

    __device__ __forceinline__ void init(const ConvArgs& args, int64_t col0, int g) {
        p = &args;
        const int nn = threadIdx.x % BN;
        kk0 = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(threadIdx.x / BN));
        const int64_t n = col0 + nn;
        col_ok = n < args.n_total;
        const int64_t nc = col_ok ? n : 0;
        const int64_t b = nc / args.plane_out;
        int64_t rem = nc - b * args.plane_out;
        const int32_t hw = args.out_h * args.out_w;
        const int32_t od = static_cast<int32_t>(rem / hw);
        rem -= static_cast<int64_t>(od) * hw;
        const int32_t oh = static_cast<int32_t>(rem / args.out_w);
        const int32_t ow = static_cast<int32_t>(rem - static_cast<int64_t>(oh) * args.out_w);
        id0 = od * args.s_d - args.p_d;
        ih0 = oh * args.s_h - args.p_h;
        iw0 = ow * args.s_w - args.p_w;
        col_off = (static_cast<int64_t>(id0) * args.in_h + ih0) * args.in_w + iw0;
        xb = args.x + (b * args.c + static_cast<int64_t>(g) * args.cg) * args.plane_in;
    }

    // Wave-uniform decode of k into the channel and the tap displacement.
    __device__ __forceinline__ void Decode(int32_t k, int32_t& c, int32_t& dd, int32_t& dh, int32_t& dw) const {
        int32_t kd = 0, kh, kw;
        if constexpr (KH > 0) {
            c = k / (KH * KW);
            const int32_t r = k - c * (KH * KW);
            kh = r / KW;
            kw = r - kh * KW;
        } else {
            c = static_cast<int32_t>(p->div_kvol.Div(static_cast<uint32_t>(k)));
            int32_t r = k - c * static_cast<int32_t>(p->div_kvol.d);
            kd = static_cast<int32_t>(p->div_khw.Div(static_cast<uint32_t>(r)));
            r -= kd * static_cast<int32_t>(p->div_khw.d);
            kh = static_cast<int32_t>(p->div_kw.Div(static_cast<uint32_t>(r)));
            kw = r - kh * static_cast<int32_t>(p->div_kw.d);
        }
        dd = kd * p->d_d;
        dh = kh * p->d_h;
        dw = kw * p->d_w;
    }

    // Padding taps read a clamped in-bounds address and select zero, so the
    // gather has no branches and all of a thread's loads stay in flight.
    __device__ __forceinline__ void load(int64_t k0, Stage& s) const {
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            int64_t k = k0 + kk0 + q * kRowsPerPass; // wave-uniform
            const bool k_ok = !CHECKED || k < k_total;
            k = k_ok ? k : 0;
            int32_t c, dd, dh, dw;
            Decode(static_cast<int32_t>(k), c, dd, dh, dw);
            const int64_t koff =
                static_cast<int64_t>(c) * p->plane_in + (static_cast<int64_t>(dd) * p->in_h + dh) * p->in_w + dw;
            const bool in = k_ok && (!CHECKED || col_ok) &&
                            static_cast<uint32_t>(ih0 + dh) < static_cast<uint32_t>(p->in_h) &&
                            static_cast<uint32_t>(iw0 + dw) < static_cast<uint32_t>(p->in_w) &&
                            (KH > 0 || static_cast<uint32_t>(id0 + dd) < static_cast<uint32_t>(p->in_d));
            const float v = xb[in ? col_off + koff : 0];
            s.v[q] = in ? v : 0.f;
        }
    }
    __device__ __forceinline__ void store(const Stage& s, float* lds) const {
        const int nn = threadIdx.x % BN;
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            lds[(kk0 + q * kRowsPerPass) * PITCH + nn] = s.v[q];
        }
    }
};

// ---- Tap-major implicit GEMM (C_g a multiple of BK) ---------------------------
//
// K is walked in tiles of BK channels at a single filter tap (kh, kw): the
// weight view is A[m][k'] with k' = tap * C_g + c, and the tiles are visited
// channel block by channel block, all taps of a block in a row. For a given column the padding test and the
// input address then hold for the whole tile: each thread computes its
// pixel's byte offset once per tile and reads the tile's channels at
// wave-uniform plane strides. Operands are read with buffer loads: the
// per-lane offset is a VGPR, the channel / tap displacement an SGPR, and a
// padding tap or an out-of-range row or column gets an offset beyond the
// buffer, which the hardware range check turns into 0.0 -- no selects, no
// clamped addresses, and no separate edge path. Requires both tensors under
// 2 GiB (32-bit buffer offsets); the host checks.

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup i on XCD
// i % 8), each with its own L2. Workgroup i of the first `count` rounded down
// to a multiple of 8 takes tile (i % 8) * (whole / 8) + i / 8, so each XCD
// works through one contiguous run of tiles, whose neighbours share operand
// rows or columns in that XCD's L2; the rest keep their index.
__device__ __forceinline__ int64_t XcdTile(int64_t i, int64_t count) {
    const int64_t whole = count / 8 * 8;
    return i < whole ? (i % 8) * (whole / 8) + i / 8 : i;
}

// For `count` = tiles_m * tiles_n tiles numbered row tile fastest, with
// tiles_m a multiple of 8: workgroup i (on XCD i % 8) takes row tile
// (i % 8) * (tiles_m / 8) + j % (tiles_m / 8) of column tile j / (tiles_m / 8),
// j = i / 8, so each XCD covers one eighth of the row tiles (of the weights)
// and every column tile.
__device__ __forceinline__ int64_t XcdTileByRow(int64_t i, int64_t count, int64_t tiles_m) {
    const int64_t per = tiles_m / 8;
    const int64_t j = i / 8;
    (void)count;
    return (i % 8) * per + j % per + tiles_m * (j / per);
}

constexpr uint32_t kBufferWord3 = 0x00020000; // raw 32-bit dword buffer (gfx9 family)
constexpr uint32_t kOutOfRange = 0x80000000u; // >= every num_records used here

__device__ __forceinline__ __amdgpu_buffer_rsrc_t MakeRsrc(const float* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), static_cast<int>(kBufferWord3));
}

__device__ __forceinline__ float BufferLoad(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voffset),
                                                                          static_cast<int>(soffset), 0));
}

// A tile (BM x BK, k-major in LDS) of the tap-major weight view:
// A[m][tap * C_g + c] = W[g*M_g + m][c][tap]. Thread t holds k = t % BK and
// rows t / BK + j * (THREADS / BK); its byte offsets are fixed for the whole
// K walk, only the wave-uniform (c0, tap) displacement changes per tile.
template <int BM, int BK, int THREADS, int PITCH>
struct TapALoader {
    static constexpr int kRowsPerPass = THREADS / BK;
    static constexpr int kPer = BM / kRowsPerPass;
    static_assert(THREADS % BK == 0 && BM % kRowsPerPass == 0, "A tile must split evenly");
    struct Stage {
        float v[kPer];
    };
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t voff[kPer];
    int32_t cg, taps;

    __device__ __forceinline__ void init(const ConvArgs& p, int64_t row0, int g, int32_t t) {
        rsrc = MakeRsrc(p.w, static_cast<uint32_t>(p.m * p.kg * 4));
        cg = static_cast<int32_t>(p.cg);
        taps = t;
        const int kk = threadIdx.x % BK;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int64_t m = row0 + threadIdx.x / BK + j * kRowsPerPass;
            voff[j] = m < p.mg ? static_cast<uint32_t>(((g * p.mg + m) * p.kg + kk * t) * 4) : kOutOfRange;
        }
    }
    __device__ __forceinline__ void load(int64_t k0, Stage& s) const {
        // K tiles run channel-block-major, taps inside: tile kt covers
        // channels (kt / taps) * BK .. + BK at tap kt % taps, so the KH*KW
        // taps of one channel block reuse the same X rows from L2.
        const int32_t kt = static_cast<int32_t>(k0) / BK;
        const int32_t tap = kt % taps;
        const int32_t c0 = (kt / taps) * BK;
        const uint32_t soff = static_cast<uint32_t>((c0 * taps + tap) * 4);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            s.v[j] = BufferLoad(rsrc, voff[j], soff);
        }
    }
    __device__ __forceinline__ void store(const Stage& s, float* lds) const {
        const int kk = threadIdx.x % BK;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            lds[kk * PITCH + threadIdx.x / BK + j * kRowsPerPass] = s.v[j];
        }
    }
};

// B tile (BK x BN) of the tap-major im2col view. Thread t owns column
// t % BN and rows kk0 + q * (THREADS / BN), kk0 wave-uniform.
template <int BN, int BK, int THREADS, int PITCH, int KH, int KW>
struct TapBLoader {
    static_assert(THREADS % BN == 0 && BN % 64 == 0, "a wave must cover part of one B row");
    static constexpr int kRowsPerPass = THREADS / BN;
    static constexpr int kPer = BK / kRowsPerPass;
    struct Stage {
        float v[kPer];
    };
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t pix;  // byte offset of (b, g*C_g, 0, 0) + window origin, or kOutOfRange
    int32_t ih0, iw0;
    int32_t in_h, in_w, d_h, d_w, k_w;
    int32_t cg, taps;
    uint32_t plane_bytes;
    int32_t kk0;

    __device__ __forceinline__ void init(const ConvArgs& p, int64_t col0, int g) {
        rsrc = MakeRsrc(p.x, static_cast<uint32_t>(p.batch * p.c * p.plane_in * 4));
        const int64_t n = col0 + threadIdx.x % BN;
        kk0 = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(threadIdx.x / BN));
        in_h = p.in_h;
        in_w = p.in_w;
        d_h = p.d_h;
        d_w = p.d_w;
        k_w = p.k_w;
        cg = static_cast<int32_t>(p.cg);
        taps = KH > 0 ? KH * KW : p.k_h * p.k_w;
        plane_bytes = static_cast<uint32_t>(p.plane_in * 4);
        if (n < p.n_total) {
            const int64_t b = n / p.plane_out;
            const int32_t rem = static_cast<int32_t>(n - b * p.plane_out);
            const int32_t oh = rem / p.out_w;
            const int32_t ow = rem - oh * p.out_w;
            ih0 = oh * p.s_h - p.p_h;
            iw0 = ow * p.s_w - p.p_w;
            pix = static_cast<uint32_t>((b * p.c + static_cast<int64_t>(g) * p.cg) * p.plane_in * 4);
        } else {
            ih0 = -(1 << 28); // every tap out of range
            iw0 = 0;
            pix = 0;
        }
    }
    __device__ __forceinline__ void load(int64_t k0, Stage& s) const {
        const int32_t kt = static_cast<int32_t>(k0) / BK; // same tile order as TapALoader
        const int32_t tap = kt % taps;
        const int32_t c0 = (kt / taps) * BK;
        int32_t kh, kw;
        if constexpr (KH > 0) {
            kh = tap / KW;
            kw = tap - kh * KW;
        } else {
            kh = tap / k_w;
            kw = tap - kh * k_w;
        }
        const int32_t ih = ih0 + kh * d_h;
        const int32_t iw = iw0 + kw * d_w;
        const bool in = static_cast<uint32_t>(ih) < static_cast<uint32_t>(in_h) &&
                        static_cast<uint32_t>(iw) < static_cast<uint32_t>(in_w);
        const uint32_t voff = in ? pix + static_cast<uint32_t>((ih * in_w + iw) * 4) : kOutOfRange;
        const uint32_t soff0 = static_cast<uint32_t>(c0 + kk0) * plane_bytes;
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            s.v[q] = BufferLoad(rsrc, voff, soff0 + static_cast<uint32_t>(q * kRowsPerPass) * plane_bytes);
        }
    }
    __device__ __forceinline__ void store(const Stage& s, float* lds) const {
        const int nn = threadIdx.x % BN;
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            lds[(kk0 + q * kRowsPerPass) * PITCH + nn] = s.v[q];
        }
    }
};

template <class Shape>
__device__ __forceinline__ void ConvEpilogue(const ConvArgs& p, const Accum<Shape>& acc, int64_t row0, int64_t col0,
                                             int g, int split) {
    if (p.partial != nullptr) {
        float* out = p.partial + (static_cast<int64_t>(split) * p.group + g) * p.mg * p.n_total;
        ForEachAccum<Shape>(acc, [&](int r, int c, float v) {
            const int64_t gr = row0 + r;
            const int64_t gc = col0 + c;
            if (gr < p.mg && gc < p.n_total) {
                out[gr * p.n_total + gc] = v;
            }
        });
        return;
    }
    // Column (pixel) decode once per 32-column block; bias and residual
    // operands are loaded from clamped, always-valid addresses before any
    // store, so the loads of a lane are all in flight together instead of
    // one per guarded branch.
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wave_m = wave % Shape::kWavesM;
    const int wave_n = wave / Shape::kWavesM;
    const int half = lane >> 5;
#pragma unroll
    for (int j = 0; j < Shape::kSubN; ++j) {
        const int64_t gc = col0 + wave_n * Shape::kWaveN + 32 * j + (lane & 31);
        const bool col_ok = gc < p.n_total;
        const int64_t gcc = col_ok ? gc : 0;
        const int64_t b = gcc / p.plane_out;
        const int64_t ybase = b * p.m * p.plane_out + (gcc - b * p.plane_out);
#pragma unroll
        for (int i = 0; i < Shape::kSubM; ++i) {
            float value[16];
            int64_t yi[16];
            bool ok[16];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t gr = row0 + wave_m * Shape::kWaveM + 32 * i + 8 * (v >> 2) + 4 * half + (v & 3);
                ok[v] = col_ok && gr < p.mg;
                const int64_t oc = static_cast<int64_t>(g) * p.mg + (ok[v] ? gr : 0);
                yi[v] = ybase + oc * p.plane_out;
                value[v] = p.bias != nullptr ? acc.c[i][j][v] + p.bias[oc] : acc.c[i][j][v];
            }
            if (p.residual != nullptr) {
                float res[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    res[v] = p.residual[ok[v] ? yi[v] : 0];
                }
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    value[v] = value[v] + res[v];
                }
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                float out = value[v];
                out = Activate(p.act, out);
                if (ok[v]) {
                    p.y[yi[v]] = out;
                }
            }
        }
    }
}

template <class Shape, int KH, int KW>
__global__ __launch_bounds__(Shape::kThreads) void ConvTapKernel(ConvArgs p) {
    __shared__ __attribute__((aligned(16))) float lds[2 * (Shape::kLdsA + Shape::kLdsB)];
    const int64_t tiles_m = (p.mg + Shape::kBM - 1) / Shape::kBM;
    const int64_t tile = XcdTile(blockIdx.x, gridDim.x);
    const int64_t row0 = (tile % tiles_m) * Shape::kBM;
    const int64_t col0 = (tile / tiles_m) * Shape::kBN;
    const int g = blockIdx.y;
    const int split = blockIdx.z;
    const int64_t k_begin = static_cast<int64_t>(split) * p.k_per_split;
    int64_t k_end = k_begin + p.k_per_split;
    if (k_end > p.kg) {
        k_end = p.kg;
    }
    Accum<Shape> acc;
    acc.zero();
    TapALoader<Shape::kBM, Shape::kBK, Shape::kThreads, Shape::kPitchA> aload;
    aload.init(p, row0, g, KH > 0 ? KH * KW : p.k_h * p.k_w);
    TapBLoader<Shape::kBN, Shape::kBK, Shape::kThreads, Shape::kPitchB, KH, KW> bload;
    bload.init(p, col0, g);
    MainLoop<Shape>(aload, bload, k_begin, k_end, lds, acc);
    if (p.split_counters != nullptr) {
        const int64_t t = static_cast<int64_t>(g) * gridDim.x + tile;
        if (!FinishSplitTile<Shape, float>(acc, p.split_slots + t * gridDim.z * Shape::kBM * Shape::kBN,
                                           p.split_counters + t, split, static_cast<int>(gridDim.z),
                                           reinterpret_cast<int*>(lds))) {
            return;
        }
    }
    ConvEpilogue<Shape>(p, acc, row0, col0, g, split);
}

template <class Shape, int KH, int KW>
__global__ __launch_bounds__(Shape::kThreads) void ConvKernel(ConvArgs p) {
    __shared__ __attribute__((aligned(16))) float lds[2 * (Shape::kLdsA + Shape::kLdsB)];
    const int64_t tiles_m = (p.mg + Shape::kBM - 1) / Shape::kBM;
    const int64_t tile = XcdTile(blockIdx.x, gridDim.x);
    const int64_t tm = tile % tiles_m;
    const int64_t tn = tile / tiles_m;
    const int64_t row0 = tm * Shape::kBM;
    const int64_t col0 = tn * Shape::kBN;
    const int g = blockIdx.y;
    const int split = blockIdx.z;

    const int64_t k_begin = static_cast<int64_t>(split) * p.k_per_split;
    int64_t k_end = k_begin + p.k_per_split;
    if (k_end > p.kg) {
        k_end = p.kg;
    }

    Accum<Shape> acc;
    acc.zero();
    const float* wg = p.w + (static_cast<int64_t>(g) * p.mg + row0) * p.kg;
    // Interior tiles (full rows and columns, 16-byte aligned weight rows) run
    // every full K tile unchecked; the rest, and the K remainder, run checked.
    const bool interior = p.kg % 4 == 0 && ((reinterpret_cast<uintptr_t>(p.w) & 15) == 0) &&
                          row0 + Shape::kBM <= p.mg && col0 + Shape::kBN <= p.n_total;
    const int64_t k_full = interior ? k_begin + (k_end - k_begin) / Shape::kBK * Shape::kBK : k_begin;
    if (k_full > k_begin) {
        KContigLoader<Shape::kBM, Shape::kBK, Shape::kThreads, Shape::kPitchA, false> aload;
        aload.base = wg;
        aload.row_stride = p.kg;
        aload.rows_left = p.mg - row0;
        aload.k_total = k_full;
        ConvBLoader<Shape::kBN, Shape::kBK, Shape::kThreads, Shape::kPitchB, KH, KW, false> bload;
        bload.init(p, col0, g);
        bload.k_total = k_full;
        MainLoop<Shape>(aload, bload, k_begin, k_full, lds, acc);
    }
    if (k_full < k_end) {
        KContigLoader<Shape::kBM, Shape::kBK, Shape::kThreads, Shape::kPitchA, true> aload;
        aload.base = wg;
        aload.row_stride = p.kg;
        aload.rows_left = p.mg - row0;
        aload.k_total = k_end;
        ConvBLoader<Shape::kBN, Shape::kBK, Shape::kThreads, Shape::kPitchB, KH, KW, true> bload;
        bload.init(p, col0, g);
        bload.k_total = k_end;
        MainLoop<Shape>(aload, bload, k_full, k_end, lds, acc);
    }

    if (p.split_counters != nullptr) {
        const int64_t t = static_cast<int64_t>(g) * gridDim.x + tile;
        if (!FinishSplitTile<Shape, float>(acc, p.split_slots + t * gridDim.z * Shape::kBM * Shape::kBN,
                                           p.split_counters + t, split, static_cast<int>(gridDim.z),
                                           reinterpret_cast<int*>(lds))) {
            return;
        }
    } else if (p.partial != nullptr) {
        float* out = p.partial + (static_cast<int64_t>(split) * p.group + g) * p.mg * p.n_total;
        ForEachAccum<Shape>(acc, [&](int r, int c, float v) {
            const int64_t gr = row0 + r;
            const int64_t gc = col0 + c;
            if (gr < p.mg && gc < p.n_total) {
                out[gr * p.n_total + gc] = v;
            }
        });
        return;
    }
    ForEachAccum<Shape>(acc, [&](int r, int c, float v) {
        const int64_t gr = row0 + r;
        const int64_t gc = col0 + c;
        if (gr < p.mg && gc < p.n_total) {
            const int64_t oc = static_cast<int64_t>(g) * p.mg + gr;
            const int64_t b = gc / p.plane_out;
            const int64_t pix = gc - b * p.plane_out;
            const float value = p.bias != nullptr ? v + p.bias[oc] : v;
            const int64_t yi = (b * p.m + oc) * p.plane_out + pix;
            p.y[yi] = Finish(p, value, yi);
        }
    });
}

// Sums the split-K partials in split order (deterministic) and applies the
// bias, four outputs per thread when an image plane holds whole quads.
__global__ void ConvSplitReduceKernel(ConvArgs p, int splits, int vec) {
    const int64_t per_split = p.group * p.mg * p.n_total;
    const int64_t quads = per_split / vec;
    for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < quads;
         q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t i = q * vec;
        const int64_t gc = i % p.n_total;
        const int64_t oc = i / p.n_total; // g * mg + m
        const int64_t b = gc / p.plane_out;
        const int64_t pix = gc - b * p.plane_out;
        const float bias = p.bias != nullptr ? p.bias[oc] : 0.f;
        const int64_t yi = (b * p.m + oc) * p.plane_out + pix;
        float* out = p.y + yi;
        if (vec == 4) {
            nert_floatx4 sum = *reinterpret_cast<const nert_floatx4*>(p.partial + i);
            for (int s = 1; s < splits; ++s) {
                sum += *reinterpret_cast<const nert_floatx4*>(p.partial + s * per_split + i);
            }
            sum += bias;
            if (p.residual != nullptr || p.act != 0) {
                for (int e = 0; e < 4; ++e) {
                    sum[e] = Finish(p, sum[e], yi + e);
                }
            }
            *reinterpret_cast<nert_floatx4*>(out) = sum;
        } else {
            float sum = p.partial[i];
            for (int s = 1; s < splits; ++s) {
                sum += p.partial[s * per_split + i];
            }
            *out = Finish(p, sum + bias, yi);
        }
    }
}

// The sum of `count` >= 1 float4 slices `stride` floats apart, added in slice
// order. The loads of up to eight slices are issued before the first addition
// (slots past the last slice re-read its address and are not added), so a
// thread waits for memory once per eight slices instead of once per slice.
__device__ __forceinline__ nert_floatx4 SumSlicesQuad(const float* src, int64_t stride, int count) {
    nert_floatx4 sum = *reinterpret_cast<const nert_floatx4*>(src);
    for (int s0 = 0; s0 < count; s0 += 8) {
        nert_floatx4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[j] = *reinterpret_cast<const nert_floatx4*>(src + static_cast<int64_t>(min(s0 + j, count - 1)) * stride);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (s0 + j > 0 && s0 + j < count) {
                sum += v[j];
            }
        }
    }
    return sum;
}

// The same sums for partial planes whose element count is a multiple of 4 and
// under 2^31: four consecutive elements per thread, 16-byte partial loads,
// 32-bit index decoding; the output index is decoded per element, so the four
// may straddle an image boundary (planes of 49 pixels). Same order of
// additions as ConvSplitReduceKernel, so the results are identical.
__global__ __launch_bounds__(256) void ConvSplitReduceQuadKernel(ConvArgs p, int splits, FastDiv div_n,
                                                                 FastDiv div_plane) {
    const uint32_t per_split = static_cast<uint32_t>(p.group * p.mg * p.n_total);
    const uint32_t quads = per_split / 4;
    const int plane_out = static_cast<int>(p.plane_out);
    for (uint32_t q = blockIdx.x * 256u + threadIdx.x; q < quads; q += gridDim.x * 256u) {
        const uint32_t i = q * 4u;
        // Output indices, bias and residual first, so their loads are in
        // flight with the partials' loads.
        int64_t yi[4];
        float bias[4];
        float res[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t gc, pix;
            const uint32_t oc = DivMod(div_n, i + e, gc); // g * mg + m
            const uint32_t b = DivMod(div_plane, gc, pix);
            yi[e] = (static_cast<int64_t>(b) * p.m + oc) * plane_out + pix;
            bias[e] = p.bias != nullptr ? p.bias[oc] : 0.f;
            res[e] = p.residual != nullptr ? p.residual[yi[e]] : 0.0f;
        }
        const nert_floatx4 sum = SumSlicesQuad(p.partial + i, per_split, splits);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float out = sum[e] + bias[e];
            if (p.residual != nullptr) {
                out = out + res[e];
            }
            out = Activate(p.act, out);
            p.y[yi[e]] = out;
        }
    }
}

void LaunchSplitReduce(const ConvArgs& p, int splits, hipStream_t stream) {
    const int64_t per_split = p.group * p.mg * p.n_total;
    const int vec = (p.plane_out % 4 == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0) ? 4 : 1;
    if (vec == 1 && per_split % 4 == 0 && per_split < (int64_t{1} << 31)) {
        ConvSplitReduceQuadKernel<<<GridFor(per_split / 4, 256, 8192), 256, 0, stream>>>(
            p, splits, FastDiv::Make(static_cast<uint32_t>(p.n_total)),
            FastDiv::Make(static_cast<uint32_t>(p.plane_out)));
    } else {
        ConvSplitReduceKernel<<<GridFor(per_split / vec, 256, 8192), 256, 0, stream>>>(p, splits, vec);
    }
    CheckLaunch("ConvSplitReduceKernel launch");
}

// Eight waves per workgroup, 64x32 or 32x64 each: measured on the ResNet-18
// bs32 layers, two waves per SIMD from one workgroup hide the gather latency
// better than four waves with 64x64 tiles (1.3-1.5x faster per layer).
using ConvShapeL = TileShape<128, 128, 16, 2, 4>; // 8 waves, 64x32 each
using ConvShapeW = TileShape<64, 256, 16, 2, 4>;  // 8 waves, 32x64 each, for M_g <= 64
using ConvShapeS = TileShape<32, 128, 16, 1, 4>;  // 4 waves, 32x32 each, for M_g <= 32
// Small tiles for short K (the 1x1 stride-2 downsampling convs, K = C_g =
// 64..256): a few K steps per tile, so the load latency is hidden by more
// resident workgroups rather than by the pipeline; 4 x 392 .. 8 x 49 tiles
// on the ResNet-18 bs32 shapes instead of 196 .. 208.
using ConvShapeQ = TileShape<64, 64, 16, 2, 2>;  // 4 waves, 32x32 each
using ConvShapeT = TileShape<32, 64, 32, 1, 2>;  // 2 waves, 32x32 each
using ConvShapeQK = TileShape<64, 64, 32, 2, 2>; // ConvShapeQ with 32-deep K steps
using ConvShapeMK = TileShape<64, 128, 32, 2, 2>; // 4 waves, 32x64 each, 32-deep K steps

template <class Shape>
int64_t ConvTiles(const ConvArgs& p) {
    return ((p.mg + Shape::kBM - 1) / Shape::kBM) * ((p.n_total + Shape::kBN - 1) / Shape::kBN) * p.group;
}

template <class Shape>
void LaunchConv(ConvArgs p, hipStream_t stream) {
    const int64_t k_tiles = (p.kg + Shape::kBK - 1) / Shape::kBK;
    const int64_t tiles = ConvTiles<Shape>(p);
    const int splits = PlanSplits(tiles, k_tiles, kResidentBlocks, 8);
    p.k_per_split = ((k_tiles + splits - 1) / splits) * Shape::kBK;
    const int64_t tiles_mn = ((p.mg + Shape::kBM - 1) / Shape::kBM) * ((p.n_total + Shape::kBN - 1) / Shape::kBN);
    p.partial = nullptr;
    p.split_counters = nullptr;
    p.split_slots = nullptr;
    if (splits > 1) {
        p.split_counters = TileCounters(tiles_mn * p.group);
        if (p.split_counters != nullptr) {
            p.split_slots = static_cast<float*>(Workspace(
                tiles_mn * p.group * splits * Shape::kBM * Shape::kBN * static_cast<int64_t>(sizeof(float)), stream));
        } else {
            p.partial = static_cast<float*>(
                Workspace(static_cast<int64_t>(splits) * p.group * p.mg * p.n_total * 4, stream));
        }
    }
    dim3 grid(static_cast<unsigned>(tiles_mn), static_cast<unsigned>(p.group), static_cast<unsigned>(splits));
    const bool tap_major = p.k_d == 1 && p.in_d == 1 && p.out_d == 1 && p.cg % Shape::kBK == 0 &&
                           p.batch * p.c * p.plane_in * 4 < (int64_t{1} << 31) &&
                           p.m * p.kg * 4 < (int64_t{1} << 31);
    if (tap_major) {
        if (p.k_h == 3 && p.k_w == 3) {
            ConvTapKernel<Shape, 3, 3><<<grid, Shape::kThreads, 0, stream>>>(p);
        } else if (p.k_h == 1 && p.k_w == 1) {
            ConvTapKernel<Shape, 1, 1><<<grid, Shape::kThreads, 0, stream>>>(p);
        } else {
            ConvTapKernel<Shape, 0, 0><<<grid, Shape::kThreads, 0, stream>>>(p);
        }
    } else if (p.k_d == 1 && p.k_h == 3 && p.k_w == 3) {
        ConvKernel<Shape, 3, 3><<<grid, Shape::kThreads, 0, stream>>>(p);
    } else if (p.k_d == 1 && p.k_h == 1 && p.k_w == 1) {
        ConvKernel<Shape, 1, 1><<<grid, Shape::kThreads, 0, stream>>>(p);
    } else if (p.k_d == 1 && p.k_h == 7 && p.k_w == 7) {
        ConvKernel<Shape, 7, 7><<<grid, Shape::kThreads, 0, stream>>>(p);
    } else {
        ConvKernel<Shape, 0, 0><<<grid, Shape::kThreads, 0, stream>>>(p);
    }
    CheckLaunch("ConvKernel launch");
    if (splits > 1 && p.split_counters == nullptr) {
        LaunchSplitReduce(p, splits, stream);
    }
}

// ---- 3x3 convolution from an LDS input patch shared by all taps -------------
//
// The tap-major kernel above stages a fresh B tile for every (channel block,
// tap) pair, although the nine taps of a 3x3 filter read shifted windows of
// the same input rows. Here a workgroup owns BM output channels x BN
// consecutive output pixels (flattened over batch, rows and columns) and
// walks the channels in blocks of kHaloBK. Per block it copies into LDS
//   - the input patch those pixels read: every input row any of them touches,
//     full padded width, zero outside the image, all kHaloBK channels of a
//     position side by side (kHaloCS floats per position), and
//   - the weights of its BM channels for the block, [m][tap][c],
// then runs all nine taps out of LDS: the B fragment of tap (kh, kw) for a
// pixel is the patch position of its window origin shifted by
// kh * d_h * PW + kw * d_w, a wave-uniform offset. Pixels of one tile may
// belong to several images: the patch then holds one run of rows per image
// (the first and last run partial) and a pixel's origin row counts from the
// start of its image's run.
//
// Each lane's half of an MFMA's K = 2 pair is a channel: lanes 0-31 take
// channel kk and lanes 32-63 channel 4 + kk of the block (kk = 0..3), so one
// 16-byte LDS read returns a lane's operand for four consecutive MFMAs; A and
// B use the same pairing, so the sum over the block's eight channels is the
// same convolution. Two barriers per block; the next block's global loads are
// in flight during the current block's 9 x 4 MFMA steps.
constexpr int kHaloBK = 8;               // channels per K step
constexpr int kHaloCS = kHaloBK + 4;     // LDS floats per patch position (16-byte aligned rows)
constexpr int kHaloMaxLds = 64 * 1024;   // dynamic LDS budget per workgroup

struct HaloGeom {
    int32_t pw;            // patch row length: (OW - 1) * s_w + (KW - 1) * d_w + 1
    int32_t positions;     // patch positions (rows * pw) the LDS holds
    int32_t blocks;        // channel blocks per group: C_g / kHaloBK
    int32_t blocks_per_split;
    FastDiv div_plane_out; // by OH * OW
    FastDiv div_out_w;     // by OW
    FastDiv div_pw;        // by pw
    FastDiv div_rows_full; // by the patch rows of a whole image
    int32_t rows_full;
    // Tail split (group 1 only): workgroups 0 .. n_full-1 take tiles whole;
    // the remaining tiles are cut into tail_pieces channel ranges of
    // tail_bps blocks, one workgroup each, whose partial sums go to
    // tail_partial[piece][BM][BN] for ConvTailReduceKernel.
    int32_t n_full;
    int32_t tail_pieces;
    int32_t tail_bps;
    float* tail_partial;
    // Channel-major XCD order (no tail split, tiles_m % 8 == 0): each XCD
    // takes tiles_m / 8 channel tiles and every pixel tile, so it reads only
    // its eighth of the weights; set where the weights outweigh the input.
    int32_t xcd_by_channel;
    // In-kernel finish of split tiles (FinishSplitTile), when non-null:
    // counters[t] for tail tile t, or for tile g * tiles + tile under split-K,
    // whose parts go to split_slots[g * tiles + tile][split][BM * BN]; tail
    // pieces use tail_partial the same way. Null: the parts go to
    // tail_partial / ConvArgs::partial for a separate reduce kernel.
    uint32_t* counters;
    float* split_slots;
    int32_t tiles;
    // Paired 1x1 convolution (HaloConvKernel<..., true>): Y2 = X (*) W2 + B2
    // at the same stride, pad 0, which reads exactly the centre tap's inputs
    // (the 3x3 conv has pad 1 and dilation 1). W2 is [M][C]; each lane loads
    // its own MFMA operands of a channel block straight into registers (no
    // LDS, so the paired launch keeps the plain launch's occupancy). Split
    // parts of Y2 go to split_slots2 / tail_partial2 the way the main
    // output's go to the fields above, under the same tile counter
    // (FinishSplitTilePair).
    const float* w2;
    const float* bias2;
    float* y2;
    float* split_slots2;
    float* tail_partial2;
};

// The epilogue arguments of a paired 1x1 output: its own output and bias,
// no summand, no activation.
__device__ __forceinline__ ConvArgs PairArgs(const ConvArgs& p, const HaloGeom& h) {
    ConvArgs q = p;
    q.y = h.y2;
    q.bias = h.bias2;
    q.residual = nullptr;
    q.act = 0;
    q.partial = nullptr;
    return q;
}

// Register budget: 128 VGPRs (four waves per SIMD, two workgroups per CU),
// except with four patch positions per thread, where that would spill.
// PACKED: the weights come from p.w_packed (ConvArgs), copied to LDS with
// 16-byte stores.
template <class Shape, int KH, int KW, int NPOS, bool PAIR = false, bool PACKED = false>
__global__ __launch_bounds__(Shape::kThreads, NPOS >= 4 ? 2 : 4) void HaloConvKernel(ConvArgs p, HaloGeom h) {
    constexpr int BM = Shape::kBM;
    constexpr int BN = Shape::kBN;
    constexpr int BK = Shape::kBK;      // channels per K step: 8 or 16
    constexpr int CS = BK + 4;          // LDS floats per patch position
    constexpr int KG = BK / 8;          // groups of 8 channels (one k-quad pair each)
    constexpr int THREADS = Shape::kThreads;
    constexpr int kTaps = KH * KW;
    constexpr int kAPitch = kTaps * BK + 4;                        // [m][tap][c] rows, 16-byte aligned
    constexpr int kQuadsRow = kTaps * BK / 4;                      // 16-byte weight loads per row and block
    constexpr int kAQuads = (BM * kQuadsRow + THREADS - 1) / THREADS; // weight loads per thread
    static_assert(BK % 8 == 0 && (kTaps * BK) % 4 == 0, "weight rows must split into 16-byte loads");
    constexpr int kCentre = (KH / 2) * KW + KW / 2; // the tap a paired 1x1 shares
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* const as = smem;
    float* const bs = smem + BM * kAPitch;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave % Shape::kWavesM;
    const int wave_n = wave / Shape::kWavesM;
    const int half = lane >> 5;
    const int64_t tiles_m = (p.mg + BM - 1) / BM;
    // Workgroups are dispatched round-robin over the 8 XCDs (workgroup i on
    // XCD i % 8), each with its own L2. Remap so that each XCD takes one
    // contiguous run of tiles: neighbouring tiles share their input patch
    // (the next channel tile) or its halo rows (the next pixel tile).
    const int g = blockIdx.y;
    const int split = blockIdx.z;
    int cb_begin = split * h.blocks_per_split;
    int cb_end = min(cb_begin + h.blocks_per_split, h.blocks);
    int piece = -1; // >= 0: this workgroup computes a tail piece
    int64_t tile = h.xcd_by_channel ? XcdTileByRow(blockIdx.x, gridDim.x, tiles_m)
                                    : XcdTile(blockIdx.x, h.tail_pieces > 0 ? h.n_full : static_cast<int64_t>(gridDim.x));
    if (h.tail_pieces > 0 && tile >= h.n_full) {
        piece = static_cast<int>(tile - h.n_full);
        tile = h.n_full + piece / h.tail_pieces;
        cb_begin = (piece % h.tail_pieces) * h.tail_bps;
        cb_end = min(cb_begin + h.tail_bps, h.blocks);
    }
    const int64_t row0 = (tile % tiles_m) * BM;
    const int64_t col0 = (tile / tiles_m) * BN;

    // The tile's first and last pixels: image and output row of each.
    uint32_t rem;
    const uint32_t n_first = static_cast<uint32_t>(col0);
    const uint32_t n_last = static_cast<uint32_t>(min(col0 + BN, p.n_total) - 1);
    const int32_t b_first = static_cast<int32_t>(DivMod(h.div_plane_out, n_first, rem));
    const int32_t oh_first = static_cast<int32_t>(h.div_out_w.Div(rem));
    const int32_t b_last = static_cast<int32_t>(DivMod(h.div_plane_out, n_last, rem));
    const int32_t oh_last = static_cast<int32_t>(h.div_out_w.Div(rem));
    const int32_t halo = (KH - 1) * p.d_h + 1;
    const int32_t run0_end = b_last == b_first ? oh_last : p.out_h - 1;
    const int32_t rows0 = (run0_end - oh_first) * p.s_h + halo; // patch rows of the first image

    // Patch positions this thread copies: q = tid + i * THREADS. Their byte
    // offsets at channel 0 of the group are fixed for the whole K walk.
    const __amdgpu_buffer_rsrc_t xr = MakeRsrc(p.x, static_cast<uint32_t>(p.batch * p.c * p.plane_in * 4));
    uint32_t bvoff[NPOS];
#pragma unroll
    for (int i = 0; i < NPOS; ++i) {
        const uint32_t q = static_cast<uint32_t>(tid + i * THREADS);
        uint32_t off = kOutOfRange;
        if (q < static_cast<uint32_t>(h.positions)) {
            uint32_t x;
            const int32_t r = static_cast<int32_t>(DivMod(h.div_pw, q, x));
            int32_t seg = 0;
            int32_t local = r;
            if (r >= rows0) {
                uint32_t lr;
                seg = 1 + static_cast<int32_t>(DivMod(h.div_rows_full, static_cast<uint32_t>(r - rows0), lr));
                local = static_cast<int32_t>(lr);
            }
            const int32_t b = b_first + seg;
            const int32_t ih = (seg == 0 ? oh_first : 0) * p.s_h - p.p_h + local;
            const int32_t iw = static_cast<int32_t>(x) - p.p_w;
            if (b <= b_last && ih >= 0 && ih < p.in_h && iw >= 0 && iw < p.in_w) {
                off = static_cast<uint32_t>(((static_cast<int64_t>(b) * p.c + static_cast<int64_t>(g) * p.cg) *
                                                 p.plane_in +
                                             ih * p.in_w + iw) *
                                            4);
            }
        }
        bvoff[i] = off;
    }
    const uint32_t plane_bytes = static_cast<uint32_t>(p.plane_in * 4);

    // Weights: a block's slice of a row is kTaps * BK consecutive floats
    // (channel-major, taps inside), copied as 16-byte loads; quad
    // e = tid + j * THREADS is row e / kQuadsRow, floats 4 * (e % kQuadsRow)...
    // The host guarantees 16-byte alignment (C_g a multiple of 4).
    const __amdgpu_buffer_rsrc_t wr = MakeRsrc(PACKED ? p.w_packed : p.w, static_cast<uint32_t>(p.m * p.kg * 4));
    uint32_t avoff[kAQuads];
#pragma unroll
    for (int j = 0; j < kAQuads; ++j) {
        const int e = tid + j * THREADS;
        const int64_t m = row0 + e / kQuadsRow;
        const int k0 = (e % kQuadsRow) * 4;
        avoff[j] = e < BM * kQuadsRow && m < p.mg ? static_cast<uint32_t>(((g * p.mg + m) * p.kg + k0) * 4)
                                                  : kOutOfRange;
    }
    const __amdgpu_buffer_rsrc_t w2r = MakeRsrc(PAIR ? h.w2 : p.w, static_cast<uint32_t>(p.m * p.cg * 4));
    // Paired 1x1 operands: lane l of sub-block i takes row l % 32 and, for
    // channel group g of a block, channels 8 g + 4 (l / 32) .. + 3 -- the
    // A-fragment layout of the main weights, read from W2 [m][c] directly.
    uint32_t a2off[PAIR ? Shape::kSubM : 1];
#pragma unroll
    for (int i = 0; i < (PAIR ? Shape::kSubM : 0); ++i) {
        const int64_t m = row0 + wave_m * Shape::kWaveM + 32 * i + (lane & 31);
        a2off[i] = m < p.mg ? static_cast<uint32_t>((m * p.cg + half * 4) * 4) : kOutOfRange;
    }

    // MFMA operand bases: A row of this lane, B patch position of the window
    // origin of each of the wave's pixel columns.
    const int a_lane = (wave_m * Shape::kWaveM + (lane & 31)) * kAPitch + half * 4;
    int b_lane[Shape::kSubN];
#pragma unroll
    for (int j = 0; j < Shape::kSubN; ++j) {
        const int64_t n = col0 + wave_n * Shape::kWaveN + 32 * j + (lane & 31);
        int32_t pos = 0; // columns past the end read position 0; their results are never stored
        if (n < p.n_total) {
            const int32_t b = static_cast<int32_t>(DivMod(h.div_plane_out, static_cast<uint32_t>(n), rem));
            uint32_t ow;
            const int32_t oh = static_cast<int32_t>(DivMod(h.div_out_w, rem, ow));
            const int32_t seg = b - b_first;
            const int32_t start = seg == 0 ? 0 : rows0 + (seg - 1) * h.rows_full;
            const int32_t first = seg == 0 ? oh_first : 0;
            pos = (start + (oh - first) * p.s_h) * h.pw + static_cast<int32_t>(ow) * p.s_w;
        }
        b_lane[j] = pos * CS + half * 4;
    }
    const int row_step = p.d_h * h.pw * CS;
    const int col_step = p.d_w * CS;

    float bv[NPOS][BK];
    nert_floatx4 av[kAQuads];
    nert_floatx4 a2n[PAIR ? Shape::kSubM : 1][KG];
    nert_floatx4 a2v[PAIR ? Shape::kSubM : 1][KG];
    auto load = [&](int cb) {
        const uint32_t c_off = static_cast<uint32_t>(cb * BK) * plane_bytes;
#pragma unroll
        for (int i = 0; i < NPOS; ++i) {
#pragma unroll
            for (int c = 0; c < BK; ++c) {
                bv[i][c] = BufferLoad(xr, bvoff[i], c_off + static_cast<uint32_t>(c) * plane_bytes);
            }
        }
        const uint32_t w_off = static_cast<uint32_t>(cb * BK * kTaps * 4);
#pragma unroll
        for (int j = 0; j < kAQuads; ++j) {
            av[j] = __builtin_bit_cast(nert_floatx4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         wr, static_cast<int>(avoff[j]), static_cast<int>(w_off), 0));
        }
#pragma unroll
        for (int i = 0; i < (PAIR ? Shape::kSubM : 0); ++i) {
#pragma unroll
            for (int g = 0; g < KG; ++g) {
                a2n[i][g] = __builtin_bit_cast(nert_floatx4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                 w2r, static_cast<int>(a2off[i]),
                                                                 static_cast<int>((cb * BK + 8 * g) * 4), 0));
            }
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int i = 0; i < NPOS; ++i) {
            const int q = tid + i * THREADS;
            if (q < h.positions) {
                float* dst = bs + q * CS;
#pragma unroll
                for (int c4 = 0; c4 < BK / 4; ++c4) {
                    *reinterpret_cast<nert_floatx4*>(dst + 4 * c4) =
                        nert_floatx4{bv[i][4 * c4], bv[i][4 * c4 + 1], bv[i][4 * c4 + 2], bv[i][4 * c4 + 3]};
                }
            }
        }
        // Weight float k of a row slice is channel k / kTaps, tap k % kTaps;
        // packed, it is 8-channel group k / (8 kTaps), tap k % (8 kTaps) / 8,
        // channel k % 8 of the group, so a quad is 4 channels of one tap.
#pragma unroll
        for (int j = 0; j < kAQuads; ++j) {
            const int e = tid + j * THREADS;
            if (e < BM * kQuadsRow) {
                float* row = as + (e / kQuadsRow) * kAPitch;
                const int k0 = (e % kQuadsRow) * 4;
                if constexpr (PACKED) {
                    const int in8 = k0 % (8 * kTaps);
                    *reinterpret_cast<nert_floatx4*>(row + (in8 / 8) * BK + (k0 / (8 * kTaps)) * 8 + in8 % 8) = av[j];
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int k = k0 + q;
                        row[(k % kTaps) * BK + k / kTaps] = av[j][q];
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < (PAIR ? Shape::kSubM : 0); ++i) {
#pragma unroll
            for (int g = 0; g < KG; ++g) {
                a2v[i][g] = a2n[i][g];
            }
        }
    };

    Accum<Shape> acc;
    acc.zero();
    Accum<Shape> acc2;
    if constexpr (PAIR) {
        acc2.zero();
    }
    if (cb_begin < cb_end) {
        load(cb_begin);
    }
    for (int cb = cb_begin; cb < cb_end; ++cb) {
        store();
        __syncthreads();
        if (cb + 1 < cb_end) {
            load(cb + 1);
        }
        // Operands of tap t + 1 are read while the MFMAs of tap t run; the
        // scheduling barriers keep the compiler from sinking the reads back
        // behind the MFMAs.
        nert_floatx4 a_next[Shape::kSubM][KG];
        nert_floatx4 b_next[Shape::kSubN][KG];
#pragma unroll
        for (int g = 0; g < KG; ++g) {
#pragma unroll
            for (int i = 0; i < Shape::kSubM; ++i) {
                a_next[i][g] = *reinterpret_cast<const nert_floatx4*>(as + a_lane + i * 32 * kAPitch + 8 * g);
            }
#pragma unroll
            for (int j = 0; j < Shape::kSubN; ++j) {
                b_next[j][g] = *reinterpret_cast<const nert_floatx4*>(bs + b_lane[j] + 8 * g);
            }
        }
#pragma unroll
        for (int t = 0; t < kTaps; ++t) {
            nert_floatx4 a[Shape::kSubM][KG];
            nert_floatx4 b[Shape::kSubN][KG];
#pragma unroll
            for (int g = 0; g < KG; ++g) {
#pragma unroll
                for (int i = 0; i < Shape::kSubM; ++i) {
                    a[i][g] = a_next[i][g];
                }
#pragma unroll
                for (int j = 0; j < Shape::kSubN; ++j) {
                    b[j][g] = b_next[j][g];
                }
            }
            if (t + 1 < kTaps) {
                const int toff = ((t + 1) / KW) * row_step + ((t + 1) % KW) * col_step;
#pragma unroll
                for (int g = 0; g < KG; ++g) {
#pragma unroll
                    for (int i = 0; i < Shape::kSubM; ++i) {
                        a_next[i][g] = *reinterpret_cast<const nert_floatx4*>(as + a_lane + i * 32 * kAPitch +
                                                                              (t + 1) * BK + 8 * g);
                    }
#pragma unroll
                    for (int j = 0; j < Shape::kSubN; ++j) {
                        b_next[j][g] = *reinterpret_cast<const nert_floatx4*>(bs + b_lane[j] + toff + 8 * g);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int g = 0; g < KG; ++g) {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
                    for (int i = 0; i < Shape::kSubM; ++i) {
#pragma unroll
                        for (int j = 0; j < Shape::kSubN; ++j) {
                            acc.c[i][j] =
                                __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][g][kk], b[j][g][kk], acc.c[i][j], 0, 0, 0);
                        }
                    }
                }
            }
            if constexpr (PAIR) {
                if (t == kCentre) {
                    // The paired 1x1 conv reads the centre tap's inputs.
#pragma unroll
                    for (int g = 0; g < KG; ++g) {
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
                            for (int i = 0; i < Shape::kSubM; ++i) {
#pragma unroll
                                for (int j = 0; j < Shape::kSubN; ++j) {
                                    acc2.c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a2v[i][g][kk], b[j][g][kk],
                                                                                         acc2.c[i][j], 0, 0, 0);
                                }
                            }
                        }
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
    }
    if (h.counters != nullptr && (piece >= 0 || h.split_slots != nullptr)) {
        int64_t t;
        float* slots;
        int part, parts;
        if (piece >= 0) {
            t = piece / h.tail_pieces;
            part = piece % h.tail_pieces;
            parts = h.tail_pieces;
            slots = h.tail_partial + t * parts * BM * BN;
        } else {
            t = static_cast<int64_t>(g) * h.tiles + tile;
            part = split;
            parts = static_cast<int>(gridDim.z);
            slots = h.split_slots + t * parts * BM * BN;
        }
        if constexpr (PAIR) {
            float* slots2 = piece >= 0 ? h.tail_partial2 + t * parts * BM * BN : h.split_slots2 + t * parts * BM * BN;
            if (FinishSplitTilePair<Shape, float>(acc, slots, acc2, slots2, h.counters + t, part, parts,
                                                  reinterpret_cast<int*>(smem))) {
                ConvEpilogue<Shape>(p, acc, row0, col0, g, 0);
                ConvEpilogue<Shape>(PairArgs(p, h), acc2, row0, col0, g, 0);
            }
        } else if (FinishSplitTile<Shape, float>(acc, slots, h.counters + t, part, parts,
                                                 reinterpret_cast<int*>(smem))) {
            ConvEpilogue<Shape>(p, acc, row0, col0, g, 0);
        }
        return;
    }
    if (piece >= 0) {
        float* out = h.tail_partial + static_cast<int64_t>(piece) * BM * BN;
        ForEachAccum<Shape>(acc, [&](int r, int c, float v) { out[r * BN + c] = v; });
        return;
    }
    ConvEpilogue<Shape>(p, acc, row0, col0, g, split);
    if constexpr (PAIR) {
        // Paired launches are never split without the in-kernel finish.
        ConvEpilogue<Shape>(PairArgs(p, h), acc2, row0, col0, g, 0);
    }
}

// Sums each tail tile's pieces in piece order (deterministic) and applies the
// epilogue the other workgroups apply (group 1). Four consecutive columns of
// a tile row per thread (16-byte loads of every piece, issued together),
// 32-bit index decoding; the same additions in the same order as
// ConvTailReduceKernel below, so the results are identical.
__global__ __launch_bounds__(256) void ConvTailReduceQuadKernel(ConvArgs p, int n_full, int pieces, int bm, int bn,
                                                                const float* partial, uint32_t quads,
                                                                FastDiv div_tile_quads, FastDiv div_row_quads,
                                                                FastDiv div_tiles_m, FastDiv div_plane) {
    const uint32_t per_tile = static_cast<uint32_t>(bm * bn);
    const int plane_out = static_cast<int>(p.plane_out);
    for (uint32_t q = blockIdx.x * 256u + threadIdx.x; q < quads; q += gridDim.x * 256u) {
        uint32_t rc4, c4, tm;
        const uint32_t t = DivMod(div_tile_quads, q, rc4);
        const uint32_t r = DivMod(div_row_quads, rc4, c4);
        const uint32_t tn = DivMod(div_tiles_m, static_cast<uint32_t>(n_full) + t, tm);
        const uint32_t gr = tm * bm + r;
        if (gr >= p.mg) {
            continue;
        }
        const uint32_t gc0 = tn * bn + 4 * c4;
        // Output indices, bias and residual first (clamped, always-valid
        // addresses), so their loads are in flight with the pieces' loads.
        int64_t yi[4];
        bool ok[4];
        float res[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t gc = gc0 + e;
            ok[e] = gc < p.n_total;
            uint32_t pix;
            const uint32_t b = DivMod(div_plane, ok[e] ? gc : 0u, pix);
            yi[e] = (static_cast<int64_t>(b) * p.m + gr) * plane_out + pix;
            res[e] = p.residual != nullptr ? p.residual[yi[e]] : 0.0f;
        }
        const float bias = p.bias != nullptr ? p.bias[gr] : 0.0f;
        const float* src = partial + static_cast<int64_t>(t) * pieces * per_tile + r * bn + 4 * c4;
        const nert_floatx4 v = SumSlicesQuad(src, per_tile, pieces);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (!ok[e]) {
                break;
            }
            float out = v[e];
            if (p.bias != nullptr) {
                out = out + bias;
            }
            if (p.residual != nullptr) {
                out = out + res[e];
            }
            out = Activate(p.act, out);
            p.y[yi[e]] = out;
        }
    }
}

__global__ void ConvTailReduceKernel(ConvArgs p, int n_full, int pieces, int bm, int bn, const float* partial,
                                     int64_t tail_tiles) {
    const int64_t tiles_m = (p.mg + bm - 1) / bm;
    const int64_t per_tile = static_cast<int64_t>(bm) * bn;
    const int64_t total = tail_tiles * per_tile;
    for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t t = e / per_tile;
        const int64_t rc = e - t * per_tile;
        const int64_t r = rc / bn;
        const int64_t c = rc - r * bn;
        const int64_t tile = n_full + t;
        const int64_t gr = (tile % tiles_m) * bm + r;
        const int64_t gc = (tile / tiles_m) * bn + c;
        if (gr >= p.mg || gc >= p.n_total) {
            continue;
        }
        const float* src = partial + t * pieces * per_tile + rc;
        float v = src[0];
        for (int q = 1; q < pieces; ++q) {
            v += src[q * per_tile];
        }
        const int64_t b = gc / p.plane_out;
        const int64_t yi = (b * p.m + gr) * p.plane_out + (gc - b * p.plane_out);
        if (p.bias != nullptr) {
            v = v + p.bias[gr];
        }
        p.y[yi] = Finish(p, v, yi);
    }
}

// Tile shapes. Which one (and which split-K count) is fastest depends on how
// the tile count falls against the CUs: measured on the ResNet-18 bs32 3x3
// layers the best of these is 3-6% ahead of a fixed choice, so the first call
// of each geometry times them (below).
using HaloShapeW = TileShape<64, 256, kHaloBK, 2, 4>; // 8 waves, 32x64 each (M_g <= 64)
using HaloShapeM = TileShape<64, 128, kHaloBK, 2, 4>; // 8 waves, 32x32 each
using HaloShapeQ = TileShape<64, 64, kHaloBK, 2, 2>;  // 4 waves, 32x32 each
using HaloShapeN = TileShape<32, 128, kHaloBK, 1, 4>; // 4 waves, 32x32 each
// The same 32x32-per-wave shapes with 16 channels per K step: twice the MFMAs
// per LDS-store/barrier phase, twice the LDS.
using HaloShapeM16 = TileShape<64, 128, 16, 2, 4>;
using HaloShapeQ16 = TileShape<64, 64, 16, 2, 2>;
using HaloShapeN16 = TileShape<32, 128, 16, 1, 4>;

template <class Shape, int NPOS, bool PACKED>
void LaunchHaloPacked(const ConvArgs& p, const HaloGeom& h, dim3 grid, size_t lds, hipStream_t stream) {
    if (h.w2 != nullptr) {
        HaloConvKernel<Shape, 3, 3, NPOS, true, PACKED><<<grid, Shape::kThreads, lds, stream>>>(p, h);
    } else {
        HaloConvKernel<Shape, 3, 3, NPOS, false, PACKED><<<grid, Shape::kThreads, lds, stream>>>(p, h);
    }
}

template <class Shape, int NPOS>
void LaunchHaloPos(const ConvArgs& p, const HaloGeom& h, dim3 grid, size_t lds, hipStream_t stream) {
    if (p.w_packed != nullptr) {
        LaunchHaloPacked<Shape, NPOS, true>(p, h, grid, lds, stream);
    } else {
        LaunchHaloPacked<Shape, NPOS, false>(p, h, grid, lds, stream);
    }
}

template <class Shape>
void LaunchHalo(const ConvArgs& p, const HaloGeom& h, dim3 grid, size_t lds, int64_t per_thread,
                hipStream_t stream) {
    if (per_thread == 1) {
        LaunchHaloPos<Shape, 1>(p, h, grid, lds, stream);
    } else if (per_thread == 2) {
        LaunchHaloPos<Shape, 2>(p, h, grid, lds, stream);
    } else {
        LaunchHaloPos<Shape, 4>(p, h, grid, lds, stream);
    }
}

// Shapes with 16-channel K steps need more than the 64 KiB default of
// dynamic LDS (up to kHaloMaxLds16, two workgroups per CU): raised once per
// process for the shape's kernels; false when the runtime refuses.
constexpr int kHaloMaxLds16 = 80 * 1024;

template <class Shape, bool PAIR, bool PACKED>
bool AllowHaloLdsFor() {
    const auto raise = [](const void* kernel) {
        return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kHaloMaxLds16) == hipSuccess;
    };
    return raise(reinterpret_cast<const void*>(&HaloConvKernel<Shape, 3, 3, 1, PAIR, PACKED>)) &&
           raise(reinterpret_cast<const void*>(&HaloConvKernel<Shape, 3, 3, 2, PAIR, PACKED>)) &&
           raise(reinterpret_cast<const void*>(&HaloConvKernel<Shape, 3, 3, 4, PAIR, PACKED>));
}

template <class Shape>
bool AllowHaloLds() {
    static const bool allowed = [] {
        const bool ok = AllowHaloLdsFor<Shape, false, false>() && AllowHaloLdsFor<Shape, true, false>() &&
                        AllowHaloLdsFor<Shape, false, true>() && AllowHaloLdsFor<Shape, true, true>();
        if (!ok) {
            (void)hipGetLastError();
        }
        return ok;
    }();
    return allowed;
}

// 3x3, 2-D, C_g a multiple of kHaloBK, stride no larger than the filter's
// extent, everything addressable with 32-bit offsets, and one workgroup's
// patch and weights within kHaloMaxLds.
// A split-K count (up to 8) under which the workgroup count fills whole
// rounds of 256 CUs best: the smallest s minimising ceil(T*s/256)/(T*s/256).
inline int BalancedSplits(int64_t tiles, int blocks) {
    int best = 1;
    double best_loss = 1e30;
    for (int s = 1; s <= std::min(8, blocks); ++s) {
        const double units = static_cast<double>(tiles * s) / 256.0;
        const double loss = std::ceil(units) / units;
        if (loss < best_loss - 1e-9) {
            best_loss = loss;
            best = s;
        }
    }
    return best;
}

// The paired 1x1 output of a launch (HaloGeom::w2): null for a plain conv.
struct HaloPair {
    const float* w2;
    const float* bias2;
    float* y2;
};

template <class Shape>
bool TryHaloShape(ConvArgs p, hipStream_t stream, int force_splits, bool tail = false,
                  const HaloPair* pair = nullptr) {
    constexpr int kTaps = 9;
    HaloGeom h{};
    h.pw = (p.out_w - 1) * p.s_w + 2 * p.d_w + 1;
    h.rows_full = (p.out_h - 1) * p.s_h + 2 * p.d_h + 1;
    // A tile's pixels touch at most r_max output rows in at most s_max
    // images; its patch has rows * s_h + images * (2 * d_h + 1 - s_h) rows.
    const int64_t r_max = (Shape::kBN - 1 + p.out_w - 1) / p.out_w + 1;
    const int64_t s_max = std::min<int64_t>((r_max - 1 + p.out_h - 1) / p.out_h + 1, p.batch);
    const int64_t rows = r_max * p.s_h + s_max * (2 * p.d_h + 1 - p.s_h);
    const int64_t positions = rows * h.pw;
    constexpr int BK = Shape::kBK;
    if (p.cg % BK != 0) {
        return false;
    }
    const int64_t lds = (static_cast<int64_t>(Shape::kBM) * (kTaps * BK + 4) + positions * (BK + 4)) * 4;
    if (pair != nullptr) {
        if (p.group != 1) {
            return false;
        }
        h.w2 = pair->w2;
        h.bias2 = pair->bias2;
        h.y2 = pair->y2;
    }
    if (lds > (BK > 8 ? kHaloMaxLds16 : kHaloMaxLds) || (lds > kHaloMaxLds && !AllowHaloLds<Shape>())) {
        return false;
    }
    const int64_t per_thread = (positions + Shape::kThreads - 1) / Shape::kThreads;
    if (per_thread > 4) {
        return false;
    }
    h.positions = static_cast<int32_t>(positions);
    h.blocks = static_cast<int32_t>(p.cg / BK);
    h.div_plane_out = FastDiv::Make(static_cast<uint32_t>(p.plane_out));
    h.div_out_w = FastDiv::Make(static_cast<uint32_t>(p.out_w));
    h.div_pw = FastDiv::Make(static_cast<uint32_t>(h.pw));
    h.div_rows_full = FastDiv::Make(static_cast<uint32_t>(h.rows_full));
    const int64_t tiles = ((p.mg + Shape::kBM - 1) / Shape::kBM) * ((p.n_total + Shape::kBN - 1) / Shape::kBN);
    if (tail) {
        // Whole rounds of one tile per CU run whole; the rest is cut along
        // the channel blocks into about one piece per CU.
        constexpr int64_t kCUs = 256;
        const int64_t rest = tiles % kCUs;
        const int64_t n_full = tiles - rest;
        if (p.group != 1 || n_full == 0 || rest == 0) {
            return false;
        }
        // Piece count: the CUs' last partial round, ceil(rest * P / 256)
        // pieces of 1/P tile each, as short as possible.
        int pieces = 2;
        double best = 1e30;
        for (int q = 2; q <= std::min(h.blocks, 16); ++q) {
            const double round = std::ceil(static_cast<double>(rest * q) / kCUs) / q;
            if (round < best - 1e-9) {
                best = round;
                pieces = q;
            }
        }
        h.tail_bps = (h.blocks + pieces - 1) / pieces;
        h.tail_pieces = (h.blocks + h.tail_bps - 1) / h.tail_bps;
        h.n_full = static_cast<int32_t>(n_full);
        h.blocks_per_split = h.blocks;
        const int64_t per_tile = static_cast<int64_t>(Shape::kBM) * Shape::kBN;
        const int64_t outputs = pair != nullptr ? 2 : 1;
        h.counters = TileCounters(rest);
        if (pair != nullptr && h.counters == nullptr) {
            return false;
        }
        h.tail_partial = static_cast<float*>(
            Workspace(outputs * rest * h.tail_pieces * per_tile * static_cast<int64_t>(sizeof(float)), stream));
        if (pair != nullptr) {
            h.tail_partial2 = h.tail_partial + rest * h.tail_pieces * per_tile;
        }
        p.k_per_split = 0;
        p.partial = nullptr;
        const dim3 grid(static_cast<unsigned>(n_full + rest * h.tail_pieces), 1, 1);
        LaunchHalo<Shape>(p, h, grid, static_cast<size_t>(lds), per_thread, stream);
        CheckLaunch("HaloConvKernel launch");
        if (h.counters != nullptr) {
            return true;
        }
        const int64_t tiles_m = (p.mg + Shape::kBM - 1) / Shape::kBM;
        if (rest * per_tile < (int64_t{1} << 31) && p.n_total < (int64_t{1} << 31) && Shape::kBN % 4 == 0) {
            const auto quads = static_cast<uint32_t>(rest * per_tile / 4);
            ConvTailReduceQuadKernel<<<GridFor(quads, 256, 8192), 256, 0, stream>>>(
                p, h.n_full, h.tail_pieces, Shape::kBM, Shape::kBN, h.tail_partial, quads,
                FastDiv::Make(static_cast<uint32_t>(per_tile / 4)), FastDiv::Make(Shape::kBN / 4),
                FastDiv::Make(static_cast<uint32_t>(tiles_m)), FastDiv::Make(static_cast<uint32_t>(p.plane_out)));
        } else {
            ConvTailReduceKernel<<<GridFor(rest * per_tile, 256, 4096), 256, 0, stream>>>(
                p, h.n_full, h.tail_pieces, Shape::kBM, Shape::kBN, h.tail_partial, rest);
        }
        CheckLaunch("ConvTailReduceKernel launch");
        return true;
    }
    // force_splits: > 0 a count, 0 PlanSplits' choice, -1 the balanced count.
    const int splits = force_splits > 0    ? std::min(force_splits, static_cast<int>(h.blocks))
                       : force_splits == 0 ? PlanSplits(tiles * p.group, h.blocks, kResidentBlocks, 4)
                                           : BalancedSplits(tiles * p.group, h.blocks);
    h.blocks_per_split = (h.blocks + splits - 1) / splits;
    p.k_per_split = 0;
    p.partial = nullptr;
    if (splits > 1) {
        const int64_t outputs = pair != nullptr ? 2 : 1;
        h.counters = TileCounters(tiles * p.group);
        if (pair != nullptr && h.counters == nullptr) {
            return false;
        }
        if (h.counters != nullptr) {
            h.tiles = static_cast<int32_t>(tiles);
            const int64_t slot_floats = tiles * p.group * splits * Shape::kBM * Shape::kBN;
            h.split_slots = static_cast<float*>(
                Workspace(outputs * slot_floats * static_cast<int64_t>(sizeof(float)), stream));
            if (pair != nullptr) {
                h.split_slots2 = h.split_slots + slot_floats;
            }
        } else {
            p.partial = static_cast<float*>(
                Workspace(static_cast<int64_t>(splits) * p.group * p.mg * p.n_total * 4, stream));
        }
    }
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(p.group), static_cast<unsigned>(splits));
    h.xcd_by_channel = ((p.mg + Shape::kBM - 1) / Shape::kBM) % 8 == 0 && p.m * p.kg > p.batch * p.c * p.plane_in;
    LaunchHalo<Shape>(p, h, grid, static_cast<size_t>(lds), per_thread, stream);
    CheckLaunch("HaloConvKernel launch");
    if (splits > 1 && h.counters == nullptr) {
        LaunchSplitReduce(p, splits, stream);
    }
    return true;
}

bool HaloApplies(const ConvArgs& p) {
    return p.k_d == 1 && p.in_d == 1 && p.out_d == 1 && p.k_h == 3 && p.k_w == 3 && p.cg % kHaloBK == 0 &&
           reinterpret_cast<uintptr_t>(p.w) % 16 == 0 && p.s_h >= 1 && p.s_w >= 1 && p.d_h >= 1 && p.d_w >= 1 &&
           p.s_h <= 2 * p.d_h + 1 && p.n_total < (int64_t{1} << 31) &&
           p.batch * p.c * p.plane_in * 4 < (int64_t{1} << 31) && p.m * p.kg * 4 < (int64_t{1} << 31) &&
           p.out_w < (1 << 16) && p.out_h < (1 << 16);
}

// ---- Per-geometry choice of a kernel configuration ----------------------------
// (tune.hpp). Measured on ResNet-18 bs32: the best candidate is 3-6% ahead of
// any fixed rule on the 3x3 layers, and the 1x1 stride-2 layers want small
// tiles. The cache key is the geometry alone, so a Conv row and a FusedConv
// row of the same geometry compute their sums the same way.
using ConvKey = std::array<int64_t, 22>;

ConvKey KeyOf(const ConvArgs& p) {
    return ConvKey{p.batch, p.c,     p.m,     p.group, p.in_d, p.in_h, p.in_w, p.k_d, p.k_h, p.k_w, p.out_d,
                   p.out_h, p.out_w, p.s_d,   p.s_h,   p.s_w,  p.d_d,  p.d_h,  p.d_w, p.p_d, p.p_h, p.p_w};
}

template <class Launch>
int ChooseConvConfig(const char* family, std::map<ConvKey, int>& cache, const ConvArgs& p, hipStream_t stream,
                     int count, int fallback, Launch launch) {
    static std::mutex mu;
    const size_t y_bytes = static_cast<size_t>(p.batch * p.m * p.plane_out) * sizeof(float);
    return ChooseConfig(family, cache, mu, KeyOf(p), y_bytes, stream, count, fallback, [&](int i, float* scratch) {
        ConvArgs q = p;
        q.y = scratch;
        return launch(i, q, stream);
    });
}

// 3x3 candidates: tile shape i / 4 (0 W, 1 M, 2 Q, 3 N) with split-K count
// {PlanSplits' choice, 1, 2, 4}[i % 4]; 16 + s: shape s with the tail split;
// 20 + s: shape s with the balanced split count; 24 + 3 s + v: the
// 16-channel shape s (0 M16, 1 Q16, 2 N16) with v = 0 PlanSplits' choice,
// 1 the tail split, 2 the balanced split count.
constexpr int kHaloCandidates = 33;

template <class Shape>
bool TryHalo16(const ConvArgs& p, hipStream_t stream, int v, const HaloPair* pair) {
    return v == 0   ? TryHaloShape<Shape>(p, stream, 0, false, pair)
           : v == 1 ? TryHaloShape<Shape>(p, stream, 0, true, pair)
                    : TryHaloShape<Shape>(p, stream, -1, false, pair);
}

bool LaunchHaloCandidate(int i, const ConvArgs& p, hipStream_t stream, const HaloPair* pair = nullptr) {
    static constexpr int kSplits[4] = {0, 1, 2, 4};
    if (i >= 24) {
        const int s16 = (i - 24) / 3;
        const int v = (i - 24) % 3;
        return s16 == 0   ? TryHalo16<HaloShapeM16>(p, stream, v, pair)
               : s16 == 1 ? TryHalo16<HaloShapeQ16>(p, stream, v, pair)
                          : TryHalo16<HaloShapeN16>(p, stream, v, pair);
    }
    if (i >= 20) {
        switch (i - 20) {
        case 0:
            return p.mg <= 64 && TryHaloShape<HaloShapeW>(p, stream, -1, false, pair);
        case 1:
            return TryHaloShape<HaloShapeM>(p, stream, -1, false, pair);
        case 2:
            return TryHaloShape<HaloShapeQ>(p, stream, -1, false, pair);
        default:
            return TryHaloShape<HaloShapeN>(p, stream, -1, false, pair);
        }
    }
    if (i >= 16) {
        switch (i - 16) {
        case 0:
            return p.mg <= 64 && TryHaloShape<HaloShapeW>(p, stream, 0, true, pair);
        case 1:
            return TryHaloShape<HaloShapeM>(p, stream, 0, true, pair);
        case 2:
            return TryHaloShape<HaloShapeQ>(p, stream, 0, true, pair);
        default:
            return TryHaloShape<HaloShapeN>(p, stream, 0, true, pair);
        }
    }
    const int splits = kSplits[i % 4];
    switch (i / 4) {
    case 0:
        return p.mg <= 64 && TryHaloShape<HaloShapeW>(p, stream, splits, false, pair);
    case 1:
        return TryHaloShape<HaloShapeM>(p, stream, splits, false, pair);
    case 2:
        return TryHaloShape<HaloShapeQ>(p, stream, splits, false, pair);
    default:
        return TryHaloShape<HaloShapeN>(p, stream, splits, false, pair);
    }
}

bool TryHaloConv(const ConvArgs& p, hipStream_t stream) {
    if (!HaloApplies(p)) {
        return false;
    }
    static std::map<ConvKey, int> chosen;
    const int fallback = p.mg <= 64 ? 0 : 4; // 64x256 tiles for M_g <= 64, else 64x128
    // NERT_HIP_CONV_CANDIDATE=i forces candidate i wherever it fits (tests
    // of every configuration use it; 100 + i names the other kernels'
    // candidate i); otherwise the per-geometry choice.
    if (const char* forced = std::getenv("NERT_HIP_CONV_CANDIDATE")) {
        const int i = std::atoi(forced);
        if (i >= 0 && i < kHaloCandidates && LaunchHaloCandidate(i, p, stream)) {
            return true;
        }
    }
    const int c = ChooseConvConfig("conv3x3", chosen, p, stream, kHaloCandidates, fallback,
                                   [](int i, const ConvArgs& q, hipStream_t st) { return LaunchHaloCandidate(i, q, st); });
    // Whether a candidate fits depends on the geometry alone, so a cached
    // choice fits; the default is tried next only as a safeguard.
    return LaunchHaloCandidate(c, p, stream) || LaunchHaloCandidate(fallback, p, stream);
}

// A 3x3 convolution (pad 1, dilation 1, group 1) and the 1x1 convolution of
// the same input at the same stride with pad 0 -- a ResNet block's first conv
// and its downsampling shortcut -- in one launch of the halo kernel: the 1x1
// reads exactly the inputs of the 3x3's centre tap, so it adds one tap's
// MFMAs per channel block to the 3x3 and no loads beyond its weights. The
// 1x1 output has the 3x3's M and output shape, its own bias, no summand and
// no activation. Its sums run over the same channel blocks and split parts
// as the 3x3's, so they differ from a separate 1x1 launch only in the order
// of the additions. Per-geometry choice under its own family ("conv3x3pair",
// keyed by the 3x3 geometry). False when the pair does not fit the halo
// kernel; the caller then runs the two convolutions separately.
bool TryHaloPair(const ConvArgs& p, const HaloPair& pair, hipStream_t stream) {
    if (!HaloApplies(p) || p.group != 1 || p.d_h != 1 || p.d_w != 1 || p.p_h != 1 || p.p_w != 1 ||
        reinterpret_cast<uintptr_t>(pair.w2) % 16 != 0) {
        return false;
    }
    static std::map<ConvKey, int> chosen;
    auto launch = [&pair](int i, const ConvArgs& q, hipStream_t st) { return LaunchHaloCandidate(i, q, st, &pair); };
    if (const char* forced = std::getenv("NERT_HIP_CONV_CANDIDATE")) {
        const int i = std::atoi(forced);
        if (i >= 0 && i < kHaloCandidates && launch(i, p, stream)) {
            return true;
        }
    }
    const int fallback = p.mg <= 64 ? 0 : 4;
    const int c = ChooseConvConfig("conv3x3pair", chosen, p, stream, kHaloCandidates, fallback, launch);
    return launch(c, p, stream) || launch(fallback, p, stream);
}

// ---- 1x1 convolutions with a short K, straight from memory --------------------
//
// A 1x1 convolution with few input channels (the ResNet downsampling convs:
// 64-256 channels, stride 2) has too few K steps for an LDS pipeline to get
// going. Here every wave owns a 32x32 output block (32 channels x 32 pixels)
// and runs its whole K with MFMAs fed directly from memory: lane half h
// takes channels 8j + 4h .. 8j + 4h + 3, so one 16-byte weight load and four
// input loads (one per channel plane) feed four MFMA steps; nothing waits on
// a barrier. The four waves of a workgroup cover four channel blocks of the
// same pixels, so the input columns they share come from L1/L2.
__global__ __launch_bounds__(256) void PointwiseDirectKernel(ConvArgs p) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int half = lane >> 5;
    const int64_t m_blocks = (p.mg + 31) / 32;
    const int64_t groups_m = (m_blocks + 3) / 4;
    const int64_t mb = (blockIdx.x % groups_m) * 4 + wave;
    const int64_t n0 = (blockIdx.x / groups_m) * 32;
    const int g = blockIdx.y;
    if (mb >= m_blocks) {
        return;
    }
    const int64_t m0 = mb * 32;
    // This lane's pixel (column) and weight row.
    const int64_t n = n0 + (lane & 31);
    const bool n_ok = n < p.n_total;
    const int64_t nc = n_ok ? n : 0;
    const int64_t b = nc / p.plane_out;
    const int64_t opix = nc - b * p.plane_out;
    const int64_t oh = opix / p.out_w;
    const int64_t ow = opix - oh * p.out_w;
    const int64_t ih = oh * p.s_h - p.p_h;
    const int64_t iw = ow * p.s_w - p.p_w;
    const bool in = n_ok && ih >= 0 && ih < p.in_h && iw >= 0 && iw < p.in_w;
    const float* xp = p.x + (b * p.c + static_cast<int64_t>(g) * p.cg) * p.plane_in + (in ? ih * p.in_w + iw : 0) +
                      4 * half * p.plane_in;
    const int64_t m = m0 + (lane & 31);
    const bool m_ok = m < p.mg;
    const float* wp = p.w + (static_cast<int64_t>(g) * p.mg + (m_ok ? m : 0)) * p.cg + 4 * half;
    nert_floatx16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        acc[v] = 0.0f;
    }
#pragma unroll 4
    for (int64_t k = 0; k < p.cg; k += 8) {
        nert_floatx4 a = *reinterpret_cast<const nert_floatx4*>(wp + k);
        float bv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            bv[q] = xp[(k + q) * p.plane_in];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(m_ok ? a[q] : 0.0f, in ? bv[q] : 0.0f, acc, 0, 0, 0);
        }
    }
    // Epilogue as in ConvEpilogue: bias, then residual, then the activation.
    const int64_t ybase = b * p.m * p.plane_out + opix;
    float value[16];
    int64_t yi[16];
    bool ok[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int64_t r = m0 + 8 * (v >> 2) + 4 * half + (v & 3);
        ok[v] = n_ok && r < p.mg;
        const int64_t oc = static_cast<int64_t>(g) * p.mg + (ok[v] ? r : 0);
        yi[v] = ybase + oc * p.plane_out;
        value[v] = p.bias != nullptr ? acc[v] + p.bias[oc] : acc[v];
    }
    if (p.residual != nullptr) {
        float res[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            res[v] = p.residual[ok[v] ? yi[v] : 0];
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            value[v] = value[v] + res[v];
        }
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        float out = value[v];
        out = Activate(p.act, out);
        if (ok[v]) {
            p.y[yi[v]] = out;
        }
    }
}

bool TryPointwiseDirect(const ConvArgs& p, hipStream_t stream) {
    if (p.k_d != 1 || p.k_h != 1 || p.k_w != 1 || p.in_d != 1 || p.out_d != 1 || p.cg % 8 != 0 ||
        (reinterpret_cast<uintptr_t>(p.w) & 15) != 0 || p.group > 65535) {
        return false;
    }
    const int64_t m_blocks = (p.mg + 31) / 32;
    const int64_t blocks = ((m_blocks + 3) / 4) * ((p.n_total + 31) / 32);
    if (blocks >= (int64_t{1} << 31)) {
        return false;
    }
    PointwiseDirectKernel<<<dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(p.group)), 256, 0, stream>>>(p);
    CheckLaunch("PointwiseDirectKernel launch");
    return true;
}

// Tap-major and gather kernels: 0-2 ConvShapeL, ConvShapeW, ConvShapeS;
// 3: the direct 1x1 kernel; 4-7: ConvShapeQ, ConvShapeT, ConvShapeQK,
// ConvShapeMK.
constexpr int kGatherCandidates = 8;

bool LaunchGatherCandidate(int i, const ConvArgs& p, hipStream_t stream) {
    switch (i) {
    case 0:
        LaunchConv<ConvShapeL>(p, stream);
        return true;
    case 1:
        LaunchConv<ConvShapeW>(p, stream);
        return true;
    case 2:
        LaunchConv<ConvShapeS>(p, stream);
        return true;
    case 4:
        LaunchConv<ConvShapeQ>(p, stream);
        return true;
    case 5:
        LaunchConv<ConvShapeT>(p, stream);
        return true;
    case 6:
        LaunchConv<ConvShapeQK>(p, stream);
        return true;
    case 7:
        LaunchConv<ConvShapeMK>(p, stream);
        return true;
    default:
        return TryPointwiseDirect(p, stream);
    }
}

void LaunchGatherConv(const ConvArgs& p, hipStream_t stream) {
    static std::map<ConvKey, int> chosen;
    const int fallback = p.mg <= 32 ? 2 : (p.mg <= 64 ? 1 : 0);
    if (const char* forced = std::getenv("NERT_HIP_CONV_CANDIDATE")) {
        const int i = std::atoi(forced) - 100; // 100 + i: gather candidate i
        if (i >= 0 && i < kGatherCandidates && LaunchGatherCandidate(i, p, stream)) {
            return;
        }
    }
    const int c = ChooseConvConfig("conv", chosen, p, stream, kGatherCandidates, fallback, LaunchGatherCandidate);
    if (!LaunchGatherCandidate(c, p, stream)) {
        LaunchGatherCandidate(fallback, p, stream);
    }
}

// ---- Small-channel convolution from an LDS input patch -------------------------
//
// For C_g <= 4 (image stems: 3 input channels) the K dimension is only C*KH*KW
// and a K tile would hold a few channels of many taps, so the gather loaders
// spend their time on index arithmetic. Instead a workgroup keeps the weights
// of its 64 output channels in LDS ([m][c][kh][kw] rows, as stored) and walks
// 16x16 blocks of output pixels: for each it copies the input patch the block
// reads (C x PH x PW, zero outside the image) into LDS and runs every MFMA out
// of LDS. The workgroups are persistent (about two per CU, each taking every
// gridDim.x-th block), so the weights are read once per workgroup, and the
// patch is double buffered: the next block's patch is loaded into registers
// while the current block's MFMAs run, one barrier per block. An MFMA step
// covers two neighbouring taps of one filter row (kw = 2q and 2q + 1); for an
// odd KW the last step's second tap does not exist, and its lanes read the
// zero slot.
constexpr int kPatchTile = 16;    // output block is kPatchTile x kPatchTile pixels
constexpr int kPatchM = 64;       // output channels per workgroup
constexpr int kPatchMaxIn = 8192; // patch floats

struct PatchGeom {
    int32_t knat;      // C_g * KH * KW, the weight row length
    int32_t wpitch;    // LDS weight row pitch (odd: conflict-free column reads)
    int32_t ph, pw;    // patch rows / row pitch
    int32_t tiles_w, tiles_h;
    int32_t patch_floats;  // C_g * ph * pw
    int32_t patch_stride;  // LDS floats between the two patch buffers
    int32_t blocks;        // batch * tiles_h * tiles_w
    FastDiv div_plane;     // by ph * pw
    FastDiv div_pw;        // by pw
};

template <int PAIRS>
__global__ __launch_bounds__(512, 4) void PatchConvKernel(ConvArgs p, PatchGeom pg) {
    // Dynamic LDS: weights [kPatchM][wpitch], bias [kPatchM], the zero slot
    // (4 floats), then two patch buffers.
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* const ws = smem;
    float* const bias_s = ws + kPatchM * pg.wpitch;
    float* const zero_s = bias_s + kPatchM;
    float* const patches = zero_s + 4;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = blockIdx.z;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kPatchM;
    const int cg = static_cast<int>(p.cg);
    const int kh_n = p.k_h, kw_n = p.k_w;

    // Weights: one wave per row, lanes along the row (zero rows past M_g).
    const float* wg = p.w + (static_cast<int64_t>(g) * p.mg + m0) * pg.knat;
    for (int m = wave; m < kPatchM; m += 8) {
        const bool ok = m0 + m < p.mg;
        for (int k = lane; k < pg.knat; k += 64) {
            ws[m * pg.wpitch + k] = ok ? wg[static_cast<int64_t>(m) * pg.knat + k] : 0.0f;
        }
    }
    if (tid < kPatchM) {
        const int64_t m = m0 + tid;
        bias_s[tid] = p.bias != nullptr && m < p.mg ? p.bias[static_cast<int64_t>(g) * p.mg + m] : 0.0f;
    }
    if (tid == 0) {
        zero_s[0] = 0.0f;
    }

    // Patch element e = tid + i * 512 is channel e / (ph * pw), row, column.
    // The copy goes straight from memory into LDS (buffer loads with the LDS
    // flag: no registers, zero for the padding taps via the range check); a
    // wave's 64 lanes fill 64 consecutive floats.
    auto load_patch = [&](int blk, float* dst) {
        const int tx0 = (blk % pg.tiles_w) * kPatchTile;
        const int rest = blk / pg.tiles_w;
        const int ty0 = (rest % pg.tiles_h) * kPatchTile;
        const int64_t b = rest / pg.tiles_h;
        const int ih0 = ty0 * p.s_h - p.p_h;
        const int iw0 = tx0 * p.s_w - p.p_w;
        // One image's channels of group g: under 2 GiB (host check).
        const __amdgpu_buffer_rsrc_t xr = MakeRsrc(p.x + (b * p.c + static_cast<int64_t>(g) * cg) * p.plane_in,
                                                   static_cast<uint32_t>(cg * p.plane_in * 4));
        const int plane_in = static_cast<int>(p.plane_in);
        for (int w0 = wave * 64; w0 < pg.patch_floats; w0 += 512) {
            const int e = w0 + lane;
            if (e < pg.patch_floats) {
                uint32_t rem, x;
                const uint32_t c = DivMod(pg.div_plane, static_cast<uint32_t>(e), rem);
                const int ih = ih0 + static_cast<int>(DivMod(pg.div_pw, rem, x));
                const int iw = iw0 + static_cast<int>(x);
                const bool in = static_cast<unsigned>(ih) < static_cast<unsigned>(p.in_h) &&
                                static_cast<unsigned>(iw) < static_cast<unsigned>(p.in_w);
                const uint32_t off =
                    in ? static_cast<uint32_t>((static_cast<int>(c) * plane_in + ih * p.in_w + iw) * 4) : kOutOfRange;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)(dst + w0), 4,
                                                         static_cast<int>(off), 0, 0, 0);
            }
        }
    };

    // 8 waves: 2 along M (32 rows each) x 4 along N (64 pixels = 4 block rows).
    const int wave_m = wave & 1;
    const int wave_n = wave >> 1;
    const int half = lane >> 5;
    const int col = lane & 31;
    int poff[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = wave_n * 64 + j * 32 + col;
        poff[j] = (n / kPatchTile) * p.s_h * pg.pw + (n % kPatchTile) * p.s_w + half * p.d_w;
    }
    const bool odd = kw_n != 2 * PAIRS;
    const float* wrow = ws + (wave_m * 32 + col) * pg.wpitch + half;
    const int plane_patch = pg.ph * pg.pw;

    int blk = blockIdx.x;
    if (blk < pg.blocks) {
        load_patch(blk, patches);
    }
    for (int buf = 0; blk < pg.blocks; blk += gridDim.x, buf ^= 1) {
        float* const patch = patches + buf * pg.patch_stride;
        // This wave's copies of the current patch are complete; after the
        // barrier everyone's are, and nobody still reads the other buffer.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        const int next = blk + static_cast<int>(gridDim.x);
        if (next < pg.blocks) {
            load_patch(next, patches + (buf ^ 1) * pg.patch_stride);
        }
        nert_floatx16 acc[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                acc[j][v] = 0.0f;
            }
        }
        for (int row = 0; row < cg * kh_n; ++row) {
            const int c = row / kh_n;
            const int kh = row - c * kh_n;
            const int rbase = c * plane_patch + kh * p.d_h * pg.pw;
            const float* wr = wrow + row * kw_n;
#pragma unroll
            for (int q = 0; q < PAIRS; ++q) {
                // Lanes of the missing tap read a real (finite) weight and a zero input.
                const bool zero = odd && half == 1 && q == PAIRS - 1;
                const float a = wr[zero ? -1 : 2 * q];
                const int off = rbase + 2 * q * p.d_w;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float bv = *(zero ? zero_s : patch + off + poff[j]);
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bv, acc[j], 0, 0, 0);
                }
            }
        }

        // Epilogue: D row = output channel, column = pixel of the 16x16 block;
        // four channels (one accumulator row group) at a time, with 32-bit
        // offsets into this image's output (under 2^31 elements, host check).
        const int tx0 = (blk % pg.tiles_w) * kPatchTile;
        const int rest = blk / pg.tiles_w;
        const int ty0 = (rest % pg.tiles_h) * kPatchTile;
        const int64_t b = rest / pg.tiles_h;
        float* const yb = p.y + b * p.m * p.plane_out;
        const float* const zb = p.residual != nullptr ? p.residual + b * p.m * p.plane_out : nullptr;
        const int plane_out = static_cast<int>(p.plane_out);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = wave_n * 64 + j * 32 + col;
            const int oy = ty0 + n / kPatchTile;
            const int ox = tx0 + n % kPatchTile;
            const bool pix_ok = oy < p.out_h && ox < p.out_w;
            const int pix = pix_ok ? oy * p.out_w + ox : 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int ml0 = wave_m * 32 + 8 * r + 4 * half;
                float value[4];
                int yi[4];
                bool ok[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int ml = ml0 + v;
                    ok[v] = pix_ok && m0 + ml < p.mg;
                    const int oc = g * static_cast<int>(p.mg) + (ok[v] ? static_cast<int>(m0) + ml : 0);
                    yi[v] = oc * plane_out + pix;
                    value[v] = p.bias != nullptr ? acc[j][4 * r + v] + bias_s[ml] : acc[j][4 * r + v];
                }
                if (zb != nullptr) {
                    float res[4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        res[v] = zb[ok[v] ? yi[v] : 0];
                    }
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        value[v] = value[v] + res[v];
                    }
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float out = value[v];
                    out = Activate(p.act, out);
                    if (ok[v]) {
                        yb[yi[v]] = out;
                    }
                }
            }
        }
    }
}

// Raises PatchConvKernel<PAIRS>'s dynamic LDS limit above the 64 KiB default
// once per process; false when the runtime refuses.
template <int PAIRS>
bool AllowPatchLds(size_t bytes) {
    static const bool allowed =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&PatchConvKernel<PAIRS>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    if (!allowed) {
        (void)hipGetLastError();
    }
    return bytes <= 64 * 1024 || allowed;
}

template <int PAIRS>
bool LaunchPatch(const ConvArgs& p, const PatchGeom& pg, dim3 grid, size_t lds, hipStream_t stream) {
    if (!AllowPatchLds<PAIRS>(lds)) {
        return false;
    }
    PatchConvKernel<PAIRS><<<grid, 512, lds, stream>>>(p, pg);
    return true;
}

// ---- Stride-2 image stems: four taps per lane per operand read ---------------
//
// The patch kernel above feeds every MFMA with two 4-byte LDS reads. For the
// stride-2 stems with filter rows of 5 to 8 taps (the 7x7 ResNet stem) the
// rows are padded to 8 taps and split the way the 3x3 kernel splits its
// channels: MFMA step kk of a filter row takes tap kk in lanes 0-31 and tap
// 4 + kk in lanes 32-63. A lane's four taps are then consecutive input
// columns 2 * ox + 4 * half + kk, 8-byte aligned because the stride is 2, so
// two 8-byte reads per pixel column and one 16-byte weight read feed the
// row's eight MFMAs. Taps past the filter's width have zero weights and their
// input values are replaced by zero in registers (a 0 * inf would be NaN).
constexpr int kStemTaps = 8;

// Seven-tap filter rows (P7): padding each row to eight taps wastes one MFMA
// step in eight. Instead filter rows r0 = 2q and r1 = 2q + 1 take seven
// steps: r0's taps (0 | 4), (1 | 5), (2 | 6) (lanes 0-31 | lanes 32-63),
// then (r0 tap 3 | r1 tap 3), then r1's three pairs; an odd last row takes
// its three pairs and (tap 3 | zero). The weights are stored in that step
// order, [pair][lane half][8 steps] per output channel, so a lane reads a
// pair's steps as two 16-byte loads; the inputs come as an 8-byte read
// (taps 0, 1 | 4, 5) and a 4-byte read (tap 2 | 6) per row and pixel column,
// and one 4-byte read (tap 3 of r0 | of r1) per pair: 74 MFMA steps per
// pixel column for the 3-channel 7x7 stem instead of 84.
constexpr int kStemPairFloats = 16;

struct StemGeom {
    int32_t rows;          // C_g * KH filter rows
    int32_t wpitch;        // LDS weight row pitch (rows * 8 + 4 floats)
    int32_t ph, pitch;     // patch rows, LDS patch row pitch (a multiple of 4)
    int32_t pw;            // patch columns read from the input
    int32_t tiles_w, tiles_h;
    int32_t patch_floats;  // C_g * ph * pitch
    int32_t blocks;        // batch * tiles_h * tiles_w
    int32_t whole;         // blocks taken whole; the rest in `pieces` row strips each
    int32_t pieces;        // 2 (rows 0-7, 8-15) or 4 (rows 4i .. 4i+3; seven-tap stems)
    int32_t units;         // whole + pieces * (blocks - whole)
    FastDiv div_plane;     // by ph * pitch
    FastDiv div_pitch;     // by pitch
};

// Work units: blocks below sg.whole are taken whole; each later block is
// sg.pieces units, strips of its output rows. A half (rows 0-7 or 8-15) is
// computed by the four waves that own those rows; a quarter (4 rows, two
// 32-pixel columns) by waves 0-3, one 32x32 output block each, so the four
// SIMDs share it. The host sets whole to the blocks of the full rounds of
// workgroups when the rest, cut, fits one round, so the last partial round
// costs a half or a quarter of a block instead of a whole one.
__device__ __forceinline__ int StemUnitBlock(const StemGeom& sg, int u, int& piece) {
    if (u < sg.whole) {
        piece = -1;
        return u;
    }
    piece = (u - sg.whole) % sg.pieces;
    return sg.whole + (u - sg.whole) / sg.pieces;
}

template <bool P7>
__global__ __launch_bounds__(512, 4) void StemQuadKernel(ConvArgs p, StemGeom sg) {
    // Dynamic LDS: weights [kPatchM][wpitch], bias [kPatchM], two patches.
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* const ws = smem;
    float* const bias_s = ws + kPatchM * sg.wpitch;
    float* const patches = bias_s + kPatchM;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = blockIdx.z;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kPatchM;
    const int cg = static_cast<int>(p.cg);
    const int kh_n = p.k_h, kw_n = p.k_w;
    const int knat = cg * kh_n * kw_n;

    // Weights, rows padded to 8 taps with zeros (zero rows past M_g), or in
    // the seven-tap pair order.
    const float* wg = p.w + (static_cast<int64_t>(g) * p.mg + m0) * knat;
    const int pairs = (sg.rows + 1) / 2;
    for (int m = wave; m < kPatchM; m += 8) {
        const bool ok = m0 + m < p.mg;
        if constexpr (P7) {
            for (int k = lane; k < pairs * kStemPairFloats; k += 64) {
                const int q = k >> 4;
                const int hf = (k >> 3) & 1;
                const int st = k & 7;
                int row = 2 * q;
                int t = -1;
                if (st < 3) {
                    t = st + 4 * hf;
                } else if (st == 3) {
                    row += hf;
                    t = 3;
                } else if (st < 7) {
                    row += 1;
                    t = st - 4 + 4 * hf;
                }
                ws[m * sg.wpitch + k] =
                    ok && t >= 0 && row < sg.rows ? wg[static_cast<int64_t>(m) * knat + row * 7 + t] : 0.0f;
            }
        } else {
            for (int k = lane; k < sg.rows * kStemTaps; k += 64) {
                const int row = k >> 3;
                const int t = k & 7;
                ws[m * sg.wpitch + k] = ok && t < kw_n ? wg[static_cast<int64_t>(m) * knat + row * kw_n + t] : 0.0f;
            }
        }
    }
    if (tid < kPatchM) {
        const int64_t m = m0 + tid;
        bias_s[tid] = p.bias != nullptr && m < p.mg ? p.bias[static_cast<int64_t>(g) * p.mg + m] : 0.0f;
    }

    // Patch element e = tid + i * 512 is channel, row, column of the padded
    // [C][ph][pitch] layout; columns past pw and positions outside the image
    // load zero. Straight from memory into LDS, 64 consecutive floats a wave.
    auto load_patch = [&](int blk, float* dst) {
        const int tx0 = (blk % sg.tiles_w) * kPatchTile;
        const int rest = blk / sg.tiles_w;
        const int ty0 = (rest % sg.tiles_h) * kPatchTile;
        const int64_t b = rest / sg.tiles_h;
        const int ih0 = ty0 * p.s_h - p.p_h;
        const int iw0 = tx0 * p.s_w - p.p_w;
        const __amdgpu_buffer_rsrc_t xr = MakeRsrc(p.x + (b * p.c + static_cast<int64_t>(g) * cg) * p.plane_in,
                                                   static_cast<uint32_t>(cg * p.plane_in * 4));
        const int plane_in = static_cast<int>(p.plane_in);
        for (int w0 = wave * 64; w0 < sg.patch_floats; w0 += 512) {
            const int e = w0 + lane;
            if (e < sg.patch_floats) {
                uint32_t rem, x;
                const uint32_t c = DivMod(sg.div_plane, static_cast<uint32_t>(e), rem);
                const int ih = ih0 + static_cast<int>(DivMod(sg.div_pitch, rem, x));
                const int iw = iw0 + static_cast<int>(x);
                const bool in = static_cast<int>(x) < sg.pw &&
                                static_cast<unsigned>(ih) < static_cast<unsigned>(p.in_h) &&
                                static_cast<unsigned>(iw) < static_cast<unsigned>(p.in_w);
                const uint32_t off =
                    in ? static_cast<uint32_t>((static_cast<int>(c) * plane_in + ih * p.in_w + iw) * 4) : kOutOfRange;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)(dst + w0), 4,
                                                         static_cast<int>(off), 0, 0, 0);
            }
        }
    };

    // 8 waves: 2 along M (32 rows each) x 4 along N (64 pixels = 4 block rows).
    const int wave_m = wave & 1;
    const int wave_n = wave >> 1;
    const int half = lane >> 5;
    const int col = lane & 31;
    bool zero_tap[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        zero_tap[kk] = 4 * half + kk >= kw_n;
    }
    const float* const wrow = ws + (wave_m * 32 + col) * sg.wpitch + 4 * half;
    const int plane_patch = sg.ph * sg.pitch;
    const int row_step = p.d_h * sg.pitch;

    float bias_r[16];
    bool bias_read = false;
    int unit = blockIdx.x;
    int row_half = -1;
    if (unit < sg.units) {
        load_patch(StemUnitBlock(sg, unit, row_half), patches);
    }
    for (int buf = 0; unit < sg.units; unit += gridDim.x, buf ^= 1) {
        const int blk = StemUnitBlock(sg, unit, row_half);
        float* const patch = patches + buf * sg.patch_floats;
        // This wave's copies of the current patch are complete; after the
        // barrier everyone's are, and nobody still reads the other buffer.
        // After the first block the copies are followed by the previous
        // block's 32 output stores, of which the newest 16 may still be in
        // flight: vector memory operations complete in issue order, so
        // vmcnt <= 16 already implies the copies are done (simm16 0x4070:
        // vmcnt 16, expcnt untouched, lgkmcnt 0). The stores then drain
        // under this block's MFMAs.
        // A plain s_barrier: the waits above already cover the LDS writes
        // (the copies through vmcnt, ordinary LDS stores through lgkmcnt),
        // and __syncthreads' release fence would wait for every store.
        if (bias_read) {
            __builtin_amdgcn_s_waitcnt(0x4070);
        } else {
            __builtin_amdgcn_s_waitcnt(0);
        }
        __builtin_amdgcn_s_barrier();
        if (!bias_read) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    bias_r[4 * r + v] = bias_s[wave_m * 32 + 8 * r + 4 * half + v];
                }
            }
            bias_read = true;
        }
        const int next = unit + static_cast<int>(gridDim.x);
        if (next < sg.units) {
            int next_half;
            load_patch(StemUnitBlock(sg, next, next_half), patches + (buf ^ 1) * sg.patch_floats);
        }
        // A half or quarter unit: only the waves with a share of its rows
        // work. Such units come only in a workgroup's last round, so the
        // skipped waves' missing stores never meet the store-count wait above.
        // wn: the 64-pixel strip (4 block rows) of this wave; j0, jn: its
        // 32-pixel columns.
        int wn = wave_n, j0 = 0, jn = 2;
        if (row_half >= 0) {
            if (sg.pieces == 2) {
                if ((wave_n >> 1) != row_half) {
                    continue;
                }
            } else {
                if (wave >= 4) {
                    continue;
                }
                wn = row_half;
                j0 = wave >> 1;
                jn = 1;
            }
        }
        int boff[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = wn * 64 + (j0 + j) * 32 + col;
            boff[j] = (n / kPatchTile) * p.s_h * sg.pitch + (n % kPatchTile) * 2 + 4 * half;
        }
        nert_floatx16 acc[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                acc[j][v] = 0.0f;
            }
        }
        if constexpr (P7) {
            // Patch offset of filter row r (channel r / KH, row r % KH).
            auto row_off = [&](int r) { return (r / kh_n) * plane_patch + (r % kh_n) * row_step; };
            const float* wp = ws + (wave_m * 32 + col) * sg.wpitch + 8 * half;
            auto pair_rows = [&](auto jn_c) {
            constexpr int JN = decltype(jn_c)::value;
            for (int q = 0; q < pairs; ++q) {
                const int r0 = 2 * q;
                const bool two = r0 + 1 < sg.rows;
                const int o0 = row_off(r0);
                const int o1 = two ? row_off(r0 + 1) : o0;
                const nert_floatx4 alo = *reinterpret_cast<const nert_floatx4*>(wp + q * kStemPairFloats);
                const nert_floatx4 ahi = *reinterpret_cast<const nert_floatx4*>(wp + q * kStemPairFloats + 4);
                float b[JN][7];
#pragma unroll
                for (int j = 0; j < JN; ++j) {
                    const float* s0 = patch + o0 + boff[j];
                    const float* s1 = patch + o1 + boff[j];
                    const nert_floatx2 x01 = *reinterpret_cast<const nert_floatx2*>(s0);
                    const float x2 = s0[2];
                    // Tap 3 (column 2 ox + 3): row r0 in lanes 0-31, r1 in
                    // lanes 32-63 (whose boff is 4 columns further on).
                    const float x3 = patch[(half != 0 ? o1 : o0) + boff[j] - 4 * half + 3];
                    const nert_floatx2 y01 = *reinterpret_cast<const nert_floatx2*>(s1);
                    const float y2 = s1[2];
                    b[j][0] = x01[0];
                    b[j][1] = x01[1];
                    b[j][2] = x2;
                    b[j][3] = two || half == 0 ? x3 : 0.0f;
                    b[j][4] = y01[0];
                    b[j][5] = y01[1];
                    b[j][6] = y2;
                }
#pragma unroll
                for (int st = 0; st < 4; ++st) {
#pragma unroll
                    for (int j = 0; j < JN; ++j) {
                        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(alo[st], b[j][st], acc[j], 0, 0, 0);
                    }
                }
                if (two) {
#pragma unroll
                    for (int st = 0; st < 3; ++st) {
#pragma unroll
                        for (int j = 0; j < JN; ++j) {
                            acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ahi[st], b[j][4 + st], acc[j], 0, 0, 0);
                        }
                    }
                }
            }
            };
            if (jn == 2) {
                pair_rows(std::integral_constant<int, 2>{});
            } else {
                pair_rows(std::integral_constant<int, 1>{});
            }
        } else {
            for (int c = 0; c < cg; ++c) {
                const float* prow = patch + c * plane_patch;
                const float* wr = wrow + c * kh_n * kStemTaps;
                for (int kh = 0; kh < kh_n; ++kh) {
                    const nert_floatx4 a = *reinterpret_cast<const nert_floatx4*>(wr + kh * kStemTaps);
                    float bq[2][4];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float* src = prow + kh * row_step + boff[j];
                        const nert_floatx2 lo = *reinterpret_cast<const nert_floatx2*>(src);
                        const nert_floatx2 hi = *reinterpret_cast<const nert_floatx2*>(src + 2);
                        bq[j][0] = zero_tap[0] ? 0.0f : lo[0];
                        bq[j][1] = zero_tap[1] ? 0.0f : lo[1];
                        bq[j][2] = zero_tap[2] ? 0.0f : hi[0];
                        bq[j][3] = zero_tap[3] ? 0.0f : hi[1];
                    }
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kk], bq[j][kk], acc[j], 0, 0, 0);
                        }
                    }
                }
            }
        }

        // Epilogue, as in the patch kernel, but every lane issues all 32 of
        // its stores (buffer stores; a lane without an output element stores
        // to an out-of-range offset, which the hardware drops), so the store
        // count behind the next block's copies is fixed.
        const int tx0 = (blk % sg.tiles_w) * kPatchTile;
        const int rest = blk / sg.tiles_w;
        const int ty0 = (rest % sg.tiles_h) * kPatchTile;
        const int64_t b = rest / sg.tiles_h;
        const uint32_t image_bytes = static_cast<uint32_t>(p.m * p.plane_out * 4);
        const __amdgpu_buffer_rsrc_t yr = MakeRsrc(p.y + b * p.m * p.plane_out, image_bytes);
        const bool has_residual = p.residual != nullptr;
        const __amdgpu_buffer_rsrc_t zr =
            MakeRsrc(has_residual ? p.residual + b * p.m * p.plane_out : p.y, has_residual ? image_bytes : 0u);
        const int plane_out = static_cast<int>(p.plane_out);
        const bool has_bias = p.bias != nullptr;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (j >= jn) {
                break;
            }
            const int n = wn * 64 + (j0 + j) * 32 + col;
            const int oy = ty0 + n / kPatchTile;
            const int ox = tx0 + n % kPatchTile;
            const bool pix_ok = oy < p.out_h && ox < p.out_w;
            const int pix = pix_ok ? oy * p.out_w + ox : 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int ml0 = wave_m * 32 + 8 * r + 4 * half;
                float value[4];
                int yi[4];
                bool ok[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int ml = ml0 + v;
                    ok[v] = pix_ok && m0 + ml < p.mg;
                    const int oc = g * static_cast<int>(p.mg) + (ok[v] ? static_cast<int>(m0) + ml : 0);
                    yi[v] = oc * plane_out + pix;
                    value[v] = has_bias ? acc[j][4 * r + v] + bias_r[4 * r + v] : acc[j][4 * r + v];
                }
                if (has_residual) {
                    float res[4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        res[v] = BufferLoad(zr, ok[v] ? static_cast<uint32_t>(yi[v]) * 4u : kOutOfRange, 0);
                    }
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        value[v] = value[v] + res[v];
                    }
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float out = value[v];
                    out = Activate(p.act, out);
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, out), yr,
                                                          static_cast<int>(ok[v] ? static_cast<uint32_t>(yi[v]) * 4u
                                                                                 : kOutOfRange),
                                                          0, 0);
                }
            }
        }
    }
}

// Stride-2, undilated-along-W stems with 5..8 taps per filter row whose
// weights and two padded patches fit in 160 KiB of LDS.
bool TryStemQuad(const ConvArgs& p, hipStream_t stream) {
    if (p.k_d != 1 || p.in_d != 1 || p.out_d != 1 || p.cg > 4 || p.s_w != 2 || p.d_w != 1 || p.k_w < 5 ||
        p.k_w > kStemTaps) {
        return false;
    }
    StemGeom sg{};
    const bool p7 = p.k_w == 7;
    sg.rows = static_cast<int32_t>(p.cg) * p.k_h;
    sg.wpitch = p7 ? (sg.rows + 1) / 2 * kStemPairFloats + 4 : sg.rows * kStemTaps + 4;
    sg.ph = (kPatchTile - 1) * p.s_h + (p.k_h - 1) * p.d_h + 1;
    sg.pw = (kPatchTile - 1) * 2 + kStemTaps;
    sg.pitch = (sg.pw + 3) / 4 * 4;
    const int64_t patch_floats = p.cg * sg.ph * sg.pitch;
    const size_t lds_bytes =
        (static_cast<size_t>(kPatchM) * sg.wpitch + kPatchM + 2 * static_cast<size_t>(patch_floats)) * sizeof(float);
    if (lds_bytes > 160 * 1024) {
        return false;
    }
    sg.patch_floats = static_cast<int32_t>(patch_floats);
    sg.tiles_w = (p.out_w + kPatchTile - 1) / kPatchTile;
    sg.tiles_h = (p.out_h + kPatchTile - 1) / kPatchTile;
    const int64_t blocks = p.batch * sg.tiles_w * sg.tiles_h;
    const int64_t m_blocks = (p.mg + kPatchM - 1) / kPatchM;
    if (blocks > 0x7FFFFFFF || m_blocks > 65535 || p.group > 65535 || p.cg * p.plane_in * 4 >= (int64_t{1} << 31) ||
        p.m * p.plane_out * 4 >= (int64_t{1} << 31)) {
        return false;
    }
    sg.blocks = static_cast<int32_t>(blocks);
    const int64_t per_slot = std::max<int64_t>(1, kResidentBlocks / (m_blocks * p.group));
    const int64_t slots = std::min(blocks, per_slot);
    const int64_t rest = blocks % slots;
    // Quarters (seven-tap kernel only) when they fit the last round, else halves.
    sg.pieces = p7 && 4 * rest <= slots ? 4 : 2;
    sg.whole = static_cast<int32_t>(rest > 0 && sg.pieces * rest <= slots ? blocks - rest : blocks);
    sg.units = static_cast<int32_t>(sg.whole + sg.pieces * (blocks - sg.whole));
    sg.div_plane = FastDiv::Make(static_cast<uint32_t>(sg.ph * sg.pitch));
    sg.div_pitch = FastDiv::Make(static_cast<uint32_t>(sg.pitch));
    auto* kernel = p7 ? &StemQuadKernel<true> : &StemQuadKernel<false>;
    static const bool allowed7 = hipFuncSetAttribute(reinterpret_cast<const void*>(&StemQuadKernel<true>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     160 * 1024) == hipSuccess;
    static const bool allowed8 = hipFuncSetAttribute(reinterpret_cast<const void*>(&StemQuadKernel<false>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     160 * 1024) == hipSuccess;
    if (!(p7 ? allowed7 : allowed8)) {
        (void)hipGetLastError();
        if (lds_bytes > 64 * 1024) {
            return false;
        }
    }
    const dim3 grid(static_cast<unsigned>(slots), static_cast<unsigned>(m_blocks), static_cast<unsigned>(p.group));
    kernel<<<grid, 512, lds_bytes, stream>>>(p, sg);
    CheckLaunch("StemQuadKernel launch");
    return true;
}

// ---- Tiny convolutions on the vector ALUs ------------------------------------
//
// A 2-D convolution with at most kDirectK taps x channels per group and at
// most kDirectM output channels per group (the detector's stem: 3 channels,
// 3x3, 16 outputs) does a few hundred multiply-adds per output pixel against
// tens of bytes moved: HBM work, which the MFMA patch kernel (64 output
// channels per tile) spends mostly on empty rows. Here one thread owns one
// output pixel: it loads the pixel's K inputs once (buffer loads; padding
// taps get an out-of-range offset and read 0) and runs M dot products of
// length K in K order against weights every lane shares (wave-uniform
// addresses, so scalar loads), then applies bias, residual and activation
// as the other kernels do.
constexpr int kDirectK = 32;
constexpr int kDirectM = 32;

struct DirectGeom {
    FastDiv div_plane_out; // by OH * OW
    FastDiv div_out_w;     // by OW
};

// KH, KW > 0: that filter size at compile time (the taps' offsets and
// bounds checks unrolled); 0: any size up to kDirectK taps x channels.
template <int KH, int KW>
__global__ __launch_bounds__(256) void DirectSmallConvKernel(ConvArgs p, DirectGeom dg) {
    // The group's weights, [m][k] rows padded to kDirectK floats, in LDS:
    // every lane reads the same address (a broadcast), 16 bytes at a time.
    __shared__ __attribute__((aligned(16))) float ws[kDirectM * kDirectK];
    const int g = blockIdx.y;
    const int kg = static_cast<int>(p.kg);
    const int mg = static_cast<int>(p.mg);
    const float* wg = p.w + static_cast<int64_t>(g) * mg * kg;
    for (int e = threadIdx.x; e < kDirectM * kDirectK; e += 256) {
        const int m = e / kDirectK;
        const int k = e - m * kDirectK;
        ws[e] = m < mg && k < kg ? wg[m * kg + k] : 0.0f;
    }
    __syncthreads();
    const uint32_t n = blockIdx.x * 256u + threadIdx.x;
    if (n >= static_cast<uint32_t>(p.n_total)) {
        return;
    }
    uint32_t pix, ox;
    const uint32_t b = DivMod(dg.div_plane_out, n, pix);
    const int oy = static_cast<int>(DivMod(dg.div_out_w, pix, ox));
    const int iy0 = oy * p.s_h - p.p_h;
    const int ix0 = static_cast<int>(ox) * p.s_w - p.p_w;
    const int kh_n = KH > 0 ? KH : p.k_h;
    const int kw_n = KW > 0 ? KW : p.k_w;
    const int plane_in = static_cast<int>(p.plane_in);
    // Element offset of the pixel's window origin in channel 0 of its group
    // (negative when the window starts in the padding; only in-image taps
    // are loaded).
    const int base = (static_cast<int>(b) * static_cast<int>(p.c) + g * static_cast<int>(p.cg)) * plane_in +
                     iy0 * p.in_w + ix0;
    const __amdgpu_buffer_rsrc_t xr = MakeRsrc(p.x, static_cast<uint32_t>(p.batch * p.c * p.plane_in * 4));
    float x[kDirectK];
#pragma unroll
    for (int k = 0; k < kDirectK; ++k) {
        x[k] = 0.0f;
        if (k < kg) {
            const int c = k / (kh_n * kw_n);
            const int r = k - c * (kh_n * kw_n);
            const int kh = r / kw_n;
            const int kw = r - kh * kw_n;
            const int ih = iy0 + kh * p.d_h;
            const int iw = ix0 + kw * p.d_w;
            const bool in = static_cast<unsigned>(ih) < static_cast<unsigned>(p.in_h) &&
                            static_cast<unsigned>(iw) < static_cast<unsigned>(p.in_w);
            const int off = base + c * plane_in + kh * p.d_h * p.in_w + kw * p.d_w;
            x[k] = BufferLoad(xr, in ? static_cast<uint32_t>(off) * 4u : kOutOfRange, 0);
        }
    }
    // Output element offset of channel 0 of the group at this pixel; plus
    // m * OH * OW for channel m.
    const int plane_out = static_cast<int>(p.plane_out);
    const int ybase = (static_cast<int>(b) * static_cast<int>(p.m) + g * mg) * plane_out + static_cast<int>(pix);
    // Four output channels at a time: four independent multiply-add chains.
    for (int m0 = 0; m0 < mg; m0 += 4) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k4 = 0; k4 < kDirectK; k4 += 4) {
            if (k4 < kg) {
                nert_floatx4 w4[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    w4[j] = *reinterpret_cast<const nert_floatx4*>(ws + (m0 + j) * kDirectK + k4);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (k4 + e < kg) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            acc[j] = fmaf(x[k4 + e], w4[j][e], acc[j]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = m0 + j;
            if (m < mg) {
                const int yi = ybase + m * plane_out;
                const float v = p.bias != nullptr ? acc[j] + p.bias[g * mg + m] : acc[j];
                p.y[yi] = Finish(p, v, yi);
            }
        }
    }
}

// 32-bit element offsets: input and output under 2^31 bytes.
bool DirectSmallApplies(const ConvArgs& p) {
    return p.k_d == 1 && p.in_d == 1 && p.out_d == 1 && p.kg <= kDirectK && p.mg <= kDirectM &&
           p.batch * p.c * p.plane_in * 4 < (int64_t{1} << 31) && p.batch * p.m * p.plane_out * 4 < (int64_t{1} << 31) &&
           p.group <= 65535;
}

void LaunchDirectSmall(const ConvArgs& p, hipStream_t stream) {
    DirectGeom dg{};
    dg.div_plane_out = FastDiv::Make(static_cast<uint32_t>(p.plane_out));
    dg.div_out_w = FastDiv::Make(static_cast<uint32_t>(p.out_w));
    const dim3 grid(static_cast<unsigned>((p.n_total + 255) / 256), static_cast<unsigned>(p.group));
    if (p.k_h == 3 && p.k_w == 3) {
        DirectSmallConvKernel<3, 3><<<grid, 256, 0, stream>>>(p, dg);
    } else {
        DirectSmallConvKernel<0, 0><<<grid, 256, 0, stream>>>(p, dg);
    }
    CheckLaunch("DirectSmallConvKernel launch");
}

// True when the patch kernel applies: 2-D, few channels per group, filter
// rows of up to 8 taps, and a workgroup's weights and two input patches fit
// in 160 KiB of LDS.
bool TryPatchConv(const ConvArgs& p, hipStream_t stream) {
    if (TryStemQuad(p, stream)) {
        return true;
    }
    if (p.k_d != 1 || p.in_d != 1 || p.out_d != 1 || p.cg > 4 || p.k_w > 8) {
        return false;
    }
    PatchGeom pg{};
    const int pairs = (p.k_w + 1) / 2;
    pg.knat = static_cast<int32_t>(p.cg) * p.k_h * p.k_w;
    pg.wpitch = pg.knat | 1;
    pg.ph = (kPatchTile - 1) * p.s_h + (p.k_h - 1) * p.d_h + 1;
    pg.pw = (kPatchTile - 1) * p.s_w + (2 * pairs - 1) * p.d_w + 1;
    const int64_t patch_floats = p.cg * pg.ph * pg.pw;
    if (patch_floats > kPatchMaxIn) {
        return false;
    }
    pg.patch_floats = static_cast<int32_t>(patch_floats);
    pg.patch_stride = static_cast<int32_t>((patch_floats + 3) / 4 * 4);
    const size_t lds_bytes =
        (static_cast<size_t>(kPatchM) * pg.wpitch + kPatchM + 4 + 2 * static_cast<size_t>(pg.patch_stride)) *
        sizeof(float);
    if (lds_bytes > 160 * 1024) {
        return false;
    }
    pg.tiles_w = (p.out_w + kPatchTile - 1) / kPatchTile;
    pg.tiles_h = (p.out_h + kPatchTile - 1) / kPatchTile;
    const int64_t blocks = p.batch * pg.tiles_w * pg.tiles_h;
    const int64_t m_blocks = (p.mg + kPatchM - 1) / kPatchM;
    if (blocks > 0x7FFFFFFF || m_blocks > 65535 || p.group > 65535 || p.cg * p.plane_in * 4 >= (int64_t{1} << 31) ||
        p.m * p.plane_out >= (int64_t{1} << 31)) {
        return false;
    }
    pg.blocks = static_cast<int32_t>(blocks);
    pg.div_plane = FastDiv::Make(static_cast<uint32_t>(pg.ph * pg.pw));
    pg.div_pw = FastDiv::Make(static_cast<uint32_t>(pg.pw));
    // About two resident workgroups per CU in total, each walking blocks.
    const int64_t per_slot = std::max<int64_t>(1, kResidentBlocks / (m_blocks * p.group));
    const dim3 grid(static_cast<unsigned>(std::min(blocks, per_slot)), static_cast<unsigned>(m_blocks),
                    static_cast<unsigned>(p.group));
    bool launched;
    switch (pairs) {
    case 1:
        launched = LaunchPatch<1>(p, pg, grid, lds_bytes, stream);
        break;
    case 2:
        launched = LaunchPatch<2>(p, pg, grid, lds_bytes, stream);
        break;
    case 3:
        launched = LaunchPatch<3>(p, pg, grid, lds_bytes, stream);
        break;
    default:
        launched = LaunchPatch<4>(p, pg, grid, lds_bytes, stream);
        break;
    }
    if (launched) {
        CheckLaunch("PatchConvKernel launch");
    }
    return launched;
}

// Small-channel convolutions: the patch (or stem) kernel, or, where the
// filter and output-channel counts are tiny, the direct VALU kernel -- the
// per-geometry choice between the two (timed like the other families;
// NERT_HIP_CONV_CANDIDATE=300 + i forces candidate i).
bool LaunchSmallCandidate(int i, const ConvArgs& p, hipStream_t stream) {
    if (i == 1) {
        if (!DirectSmallApplies(p)) {
            return false;
        }
        LaunchDirectSmall(p, stream);
        return true;
    }
    return TryPatchConv(p, stream);
}

bool TrySmallChannelConv(const ConvArgs& p, hipStream_t stream) {
    if (!DirectSmallApplies(p) || p.cg > 4) {
        return TryPatchConv(p, stream);
    }
    if (const char* forced = std::getenv("NERT_HIP_CONV_CANDIDATE")) {
        const int i = std::atoi(forced) - 300;
        if ((i == 0 || i == 1) && LaunchSmallCandidate(i, p, stream)) {
            return true;
        }
    }
    static std::map<ConvKey, int> chosen;
    const int c = ChooseConvConfig("small", chosen, p, stream, 2, 0, LaunchSmallCandidate);
    return LaunchSmallCandidate(c, p, stream) || LaunchSmallCandidate(1, p, stream);
}

// y = act(y + residual) in place: the fused pointwise convolution's
// epilogue, run after the GEMM has written conv + bias (each step rounded
// like the Add and activation rows).
__global__ void ResidualActKernel(float* y, const float* residual, int act, int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        float v = y[i];
        if (residual != nullptr) {
            v = __fadd_rn(v, residual[i]);
        }
        y[i] = Activate(act, v);
    }
}

// A 1x1, stride-1, unpadded, ungrouped convolution is Y[b] = W[M,C] * X[b][C,P]
// with P = D*H*W: a batched GEMM whose B batches are the images. The fused
// form (residual, activation) runs the same GEMM and then ResidualActKernel, so a
// Conv and a FusedConv of one geometry sum in the same order.
// ---- Non-overlapping patches (stride = kernel, no padding): a GEMM -----------
//
// A conv whose windows tile the input exactly (the ViT patch embedding:
// 16 x 16 windows at stride 16) reads every input element once, so it is a
// plain GEMM once each image's patches are laid out as rows:
//     P[b][p][k] = X[b][c][oh * KH + kh][ow * KW + kw],
//     p = oh * OW + ow,  k = (c * KH + kh) * KW + kw,
// and Y = W (M x K, the ONNX weight as it is) * P^T + bias over all images'
// patches at once (B K-contiguous), the output written back per image in
// NCHW (the engine's grouped output layout). The GEMM's B loader reads P
// from X in place (GemmArgs::PatchB): a run of 4 k is 4 consecutive input
// columns. When the pixels per image are not whole quads, the batched form
// with W broadcast runs over P built first by PatchRowsKernel.
// PatchRowsKernel builds P: the OW patch rows of one band of KH input rows
// (b, oh) are a contiguous run of OW * K floats, written by a few
// workgroups, kPatchQuadsPerBlock floats x 4 each, one 16-byte load and
// store per thread and step; the loads are runs of KW floats of X.
constexpr int32_t kPatchQuadsPerBlock = 1024;
__global__ __launch_bounds__(256) void PatchRowsKernel(const float* __restrict__ x, float* __restrict__ out,
                                                       int32_t c, int32_t kh, int32_t kw, int32_t out_h,
                                                       int32_t out_w, int32_t in_h, int32_t in_w, int32_t parts) {
    const int64_t band = blockIdx.x / parts; // b * out_h + oh
    const int32_t part = static_cast<int32_t>(blockIdx.x - band * parts);
    const int64_t b = band / out_h;
    const int32_t oh = static_cast<int32_t>(band - b * out_h);
    const int32_t k_total = c * kh * kw;
    const int32_t quads = out_w * k_total / 4;
    const float* xb = x + (b * c * in_h + static_cast<int64_t>(oh) * kh) * in_w;
    nert_floatx4* dst = reinterpret_cast<nert_floatx4*>(out + band * out_w * static_cast<int64_t>(k_total));
    const int32_t end = min(quads, (part + 1) * kPatchQuadsPerBlock);
    for (int32_t q = part * kPatchQuadsPerBlock + threadIdx.x; q < end; q += 256) {
        const int32_t e = 4 * q;
        const int32_t ow = e / k_total;
        const int32_t k = e - ow * k_total;
        const int32_t q_kw = k % kw;
        const int32_t t = k / kw; // c * KH + kh
        const int32_t r = t % kh;
        const int32_t ch = t / kh;
        const float* src = xb + (static_cast<int64_t>(ch) * in_h + r) * in_w + ow * kw + q_kw;
        dst[q] = *reinterpret_cast<const nert_floatx4*>(src);
    }
}

bool TryPatchGemm(const ConvArgs& p, hipStream_t stream) {
    const bool tiles_exactly = p.k_d == 1 && p.in_d == 1 && p.out_d == 1 && p.group == 1 && p.s_h == p.k_h &&
                               p.s_w == p.k_w && p.d_h == 1 && p.d_w == 1 && p.p_h == 0 && p.p_w == 0 &&
                               p.in_h == p.out_h * p.k_h && p.in_w == p.out_w * p.k_w && p.k_h * p.k_w > 1;
    // Four-float moves: KW and the row length multiples of 4, X 16-byte aligned.
    const bool quads = p.k_w % 4 == 0 && p.in_w % 4 == 0 && (reinterpret_cast<uintptr_t>(p.x) & 15) == 0;
    if (!tiles_exactly || !quads || p.batch > 65535 || p.batch * p.out_h * p.out_w * p.c >= (int64_t{1} << 31) ||
        p.out_w * p.c * p.k_h * p.k_w >= (int64_t{1} << 31)) {
        return false;
    }
    const int64_t k_total = p.c * p.k_h * p.k_w;
    GemmArgs g{};
    g.a = p.w;
    g.y = p.y;
    g.m = p.m;
    g.k = k_total;
    g.a_sm = k_total;
    g.a_sk = 1;
    g.b_sk = 1;
    g.b_sn = k_total;
    g.alpha = 1.0f;
    g.beta = 1.0f;
    g.has_bias = p.bias != nullptr ? 1 : 0;
    g.bias = p.bias;
    g.bias_sm = 1;
    g.bias_sn = 0;
    if (p.plane_out % 4 == 0 && p.n_total < (int64_t{1} << 31) &&
        p.batch * p.c * p.plane_in < (int64_t{1} << 31)) {
        // One GEMM over every image's patches (N = batch x pixels, no
        // per-image column tiles half empty), B read from X in place, written
        // back per image in NCHW.
        g.b = p.x;
        g.patch = GemmArgs::PatchB{p.x,
                                   static_cast<int32_t>(p.c),
                                   p.k_h,
                                   p.k_w,
                                   p.in_h,
                                   p.in_w,
                                   p.out_h,
                                   p.out_w,
                                   FastDiv::Make(static_cast<uint32_t>(p.k_h * p.k_w)),
                                   FastDiv::Make(static_cast<uint32_t>(p.k_w)),
                                   FastDiv::Make(static_cast<uint32_t>(p.plane_out)),
                                   FastDiv::Make(static_cast<uint32_t>(p.out_w))};
        g.n = p.n_total;
        g.y_group = p.plane_out;
        LaunchGemm(g, 1, stream);
    } else {
        // Images whose pixels are not whole quads: the patch rows first
        // (workspace slot 1, alive across the GEMM, which may take slot 0 for
        // split-K partial sums), then one GEMM per image.
        auto* rows = static_cast<float*>(
            Workspace(p.batch * p.plane_out * k_total * static_cast<int64_t>(sizeof(float)), stream, 1));
        const int64_t band_quads = p.out_w * k_total / 4;
        const int64_t parts = (band_quads + kPatchQuadsPerBlock - 1) / kPatchQuadsPerBlock;
        PatchRowsKernel<<<static_cast<unsigned>(p.batch * p.out_h * parts), 256, 0, stream>>>(
            p.x, rows, static_cast<int32_t>(p.c), p.k_h, p.k_w, p.out_h, p.out_w, p.in_h, p.in_w,
            static_cast<int32_t>(parts));
        CheckLaunch("PatchRowsKernel launch");
        g.b = rows;
        g.n = p.plane_out;
        g.batch_rank = 1;
        g.bdims[0] = p.batch;
        g.a_bs[0] = 0;
        g.b_bs[0] = p.plane_out * k_total;
        LaunchGemm(g, p.batch, stream);
    }
    if (p.residual != nullptr || p.act != 0) {
        const int64_t n = p.batch * p.m * p.plane_out;
        ResidualActKernel<<<GridFor(n, 256, 16384), 256, 0, stream>>>(p.y, p.residual, p.act, n);
        CheckLaunch("ResidualActKernel launch");
    }
    return true;
}

bool TryPointwise(const ConvArgs& p, hipStream_t stream) {
    const bool unit = p.k_d == 1 && p.k_h == 1 && p.k_w == 1 && p.s_d == 1 && p.s_h == 1 && p.s_w == 1 &&
                      p.p_d == 0 && p.p_h == 0 && p.p_w == 0 && p.group == 1 && p.plane_in == p.plane_out;
    if (!unit || p.batch > 65535) {
        return false;
    }
    GemmArgs g{};
    g.a = p.w;
    g.b = p.x;
    g.y = p.y;
    g.m = p.m;
    g.n = p.plane_out;
    g.k = p.c;
    g.a_sm = p.c;
    g.a_sk = 1;
    g.b_sk = p.plane_in;
    g.b_sn = 1;
    g.alpha = 1.0f;
    g.beta = 1.0f;
    g.has_bias = p.bias != nullptr ? 1 : 0;
    g.bias = p.bias;
    g.bias_sm = 1;
    g.bias_sn = 0;
    g.batch_rank = 1;
    g.bdims[0] = p.batch;
    g.a_bs[0] = 0;
    g.b_bs[0] = p.c * p.plane_in;
    LaunchGemm(g, p.batch, stream);
    if (p.residual != nullptr || p.act != 0) {
        const int64_t n = p.batch * p.m * p.plane_out;
        ResidualActKernel<<<GridFor(n, 256, 16384), 256, 0, stream>>>(p.y, p.residual, p.act, n);
        CheckLaunch("ResidualActKernel launch");
    }
    return true;
}

} // namespace
} // namespace nert_hip

namespace nert_hip {

// The kernel arguments of one convolution from the C-ABI descriptor; throws
// on an invalid group, activation or reduction length.
ConvArgs MakeConvArgs(const float* x, const float* w, const float* bias, const float* residual, float* y,
                      const nert_conv_desc* d, int act) {
    ConvArgs p{};
    p.x = x;
    p.w = w;
    p.bias = bias;
    p.y = y;
    p.residual = residual;
    if (act < 0 || act > 2) {
        throw Error("conv: activation must be 0 (none), 1 (Relu) or 2 (SiLU)");
    }
    p.act = act;
    p.batch = d->batch;
    p.c = d->in_channels;
    p.m = d->out_channels;
    p.group = d->group;
    if (p.group <= 0 || p.c % p.group != 0 || p.m % p.group != 0) {
        throw Error("conv: invalid group");
    }
    if (p.group > 65535) {
        throw Error("conv: more than 65535 groups");
    }
    p.cg = p.c / p.group;
    p.mg = p.m / p.group;
    p.in_d = static_cast<int32_t>(d->in[0]);
    p.in_h = static_cast<int32_t>(d->in[1]);
    p.in_w = static_cast<int32_t>(d->in[2]);
    p.k_d = static_cast<int32_t>(d->kernel[0]);
    p.k_h = static_cast<int32_t>(d->kernel[1]);
    p.k_w = static_cast<int32_t>(d->kernel[2]);
    p.out_d = static_cast<int32_t>(d->out[0]);
    p.out_h = static_cast<int32_t>(d->out[1]);
    p.out_w = static_cast<int32_t>(d->out[2]);
    p.s_d = static_cast<int32_t>(d->stride[0]);
    p.s_h = static_cast<int32_t>(d->stride[1]);
    p.s_w = static_cast<int32_t>(d->stride[2]);
    p.d_d = static_cast<int32_t>(d->dilation[0]);
    p.d_h = static_cast<int32_t>(d->dilation[1]);
    p.d_w = static_cast<int32_t>(d->dilation[2]);
    p.p_d = static_cast<int32_t>(d->pad[0]);
    p.p_h = static_cast<int32_t>(d->pad[1]);
    p.p_w = static_cast<int32_t>(d->pad[2]);
    p.kg = p.cg * p.k_d * p.k_h * p.k_w;
    p.plane_out = static_cast<int64_t>(p.out_d) * p.out_h * p.out_w;
    p.plane_in = static_cast<int64_t>(p.in_d) * p.in_h * p.in_w;
    p.n_total = p.batch * p.plane_out;
    if (p.kg >= (int64_t{1} << 31) || p.plane_in * p.cg >= (int64_t{1} << 40)) {
        throw Error("conv: reduction length exceeds 2^31");
    }
    p.div_kvol = FastDiv::Make(static_cast<uint32_t>(p.k_d * p.k_h * p.k_w));
    p.div_khw = FastDiv::Make(static_cast<uint32_t>(p.k_h * p.k_w));
    p.div_kw = FastDiv::Make(static_cast<uint32_t>(p.k_w));
    return p;
}

// Runs one convolution on the fastest kernel that applies.
void RunConv(const ConvArgs& p, hipStream_t s) {
    if (p.n_total == 0 || p.mg == 0) {
        return;
    }
    if (TryPointwise(p, s) || TryPatchGemm(p, s) || TrySmallChannelConv(p, s) || TryHaloConv(p, s)) {
        return;
    }
    LaunchGatherConv(p, s);
}

} // namespace nert_hip

extern "C" int nert_hip_conv_fused_f32(const float* x, const float* w, const float* bias, const float* residual,
                                       float* y, const nert_conv_desc* d, int act, void* stream) {
    return nert_hip::Guard([&] {
        nert_hip::RunConv(nert_hip::MakeConvArgs(x, w, bias, residual, y, d, act), nert_hip::StreamOr(stream));
    });
}

namespace nert_hip {

// nert_hip_conv_pair_f32's work for the arguments of its 3x3 convolution.
void RunConvPair(const ConvArgs& p, const float* w2, const float* bias2, float* y2, const nert_conv_desc* d,
                 void* stream) {
    // The 1x1 convolution: same input, stride and output shape, kernel 1,
    // pad 0, dilation 1.
    nert_conv_desc d2 = *d;
    for (int i = 0; i < 3; ++i) {
        d2.kernel[i] = 1;
        d2.pad[i] = 0;
        d2.dilation[i] = 1;
    }
    const ConvArgs p2 = MakeConvArgs(p.x, w2, bias2, nullptr, y2, &d2, 0);
    if (p.group != 1 || p.k_d != 1 || p.k_h != 3 || p.k_w != 3 || p.p_h != 1 || p.p_w != 1 || p.d_h != 1 ||
        p.d_w != 1) {
        throw Error("conv pair: the first convolution must be 3x3 with pad 1, dilation 1, group 1");
    }
    for (int i = 0; i < 3; ++i) {
        const int64_t in = d->in[i];
        const int64_t expect = (in - 1) / d->stride[i] + 1;
        if (d->out[i] != expect) {
            throw Error("conv pair: the output shape is not that of both convolutions");
        }
    }
    if (p.n_total == 0 || p.mg == 0) {
        return;
    }
    hipStream_t s = StreamOr(stream);
    if (TryHaloPair(p, HaloPair{w2, bias2, y2}, s)) {
        return;
    }
    RunConv(p, s);
    RunConv(p2, s);
}

} // namespace nert_hip

extern "C" int nert_hip_conv_pair_f32(const float* x, const float* w, const float* bias, const float* residual,
                                      float* y, const float* w2, const float* bias2, float* y2,
                                      const nert_conv_desc* d, int act, void* stream) {
    return nert_hip::Guard([&] {
        nert_hip::RunConvPair(nert_hip::MakeConvArgs(x, w, bias, residual, y, d, act), w2, bias2, y2, d, stream);
    });
}

extern "C" int nert_hip_conv_packed_f32(const float* x, const float* w, const float* w_packed, const float* bias,
                                        const float* residual, float* y, const float* w2, const float* bias2,
                                        float* y2, const nert_conv_desc* d, int act, void* stream) {
    return nert_hip::Guard([&] {
        nert_hip::ConvArgs p = nert_hip::MakeConvArgs(x, w, bias, residual, y, d, act);
        if (w_packed == nullptr) {
            throw nert_hip::Error("conv packed: the packed weights are null");
        }
        if (p.cg % 8 != 0) {
            throw nert_hip::Error("conv packed: packed weights need C / group to be a multiple of 8");
        }
        p.w_packed = w_packed;
        if (w2 != nullptr) {
            nert_hip::RunConvPair(p, w2, bias2, y2, d, stream);
            return;
        }
        nert_hip::RunConv(p, nert_hip::StreamOr(stream));
    });
}

extern "C" int nert_hip_conv_f32(const float* x, const float* w, const float* bias, float* y, const nert_conv_desc* d,
                                 void* stream) {
    return nert_hip_conv_fused_f32(x, w, bias, nullptr, y, d, 0, stream);
}
