// Gemm and MatMul on fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
// One kernel serves both rows: Y[b] = alpha * op(A[b]) * op(B[b]) + beta * C,
// where b runs over up to four broadcast batch axes (MatMul) or is absent
// (Gemm). Transposes are expressed as operand strides, so Gemm's four
// (transA, transB) cases and MatMul's broadcast batches are the same code with
// different loaders. Small problems that cannot fill 256 CUs are split along
// K; the parts of a tile are summed in a fixed order (in double, rounded
// once) by the tile's last workgroup to finish, or by a second kernel when
// the tile counters do not suffice, so the result does not depend on
// scheduling.

#include "gemm_engine.hpp"
#include "mfma_tile.hpp"
#include "tune.hpp"
#include "../../include/nert_hip.h"

#include <algorithm>
#include <cstdlib>
#include <array>
#include <map>
#include <mutex>

namespace nert_hip {
namespace {

// Builds the loader of one operand. `row_stride`/`k_stride` are the element
// strides of the operand's non-K and K index; K_CONTIG selects which is 1.
template <int ROWS, int BK, int THREADS, int PITCH, bool K_CONTIG, bool CHECKED>
__device__ __forceinline__ auto MakeOperand(const float* base, int64_t row0, int64_t row_stride, int64_t k_stride,
                                            int64_t rows, int64_t k_total) {
    if constexpr (K_CONTIG) {
        KContigLoader<ROWS, BK, THREADS, PITCH, CHECKED> l;
        l.base = base + row0 * row_stride;
        l.row_stride = row_stride;
        l.rows_left = rows - row0;
        l.k_total = k_total;
        return l;
    } else {
        RowContigLoader<ROWS, BK, THREADS, PITCH, CHECKED> l;
        l.base = base + row0;
        l.k_stride = k_stride;
        l.rows_left = rows - row0;
        l.k_total = k_total;
        return l;
    }
}

// B of a patch convolution read in place (GemmArgs::PatchB): each thread
// loads runs of 4 consecutive k of one column n, i.e. 4 consecutive input
// columns of one input row, into the k-major LDS tile the way the
// K-contiguous loader does. The x offsets of the thread's columns at k = 0
// are fixed for the whole K walk; a k's offset is c * H * W + r * W + q.
template <int ROWS, int BK, int THREADS, int PITCH, bool CHECKED>
struct PatchLoader {
    using Rows = KContigLoader<ROWS, BK, THREADS, PITCH, CHECKED>;
    static constexpr int kQuads = Rows::kQuads;
    static constexpr int kPer = Rows::kPer;
    using Stage = typename Rows::Stage;
    const GemmArgs::PatchB* v;
    uint32_t col_off[kPer];
    bool col_ok[kPer];
    uint32_t k_total;

    __device__ __forceinline__ void init(const GemmArgs::PatchB& pv, int64_t col0, int64_t n_total, int64_t k_tot) {
        v = &pv;
        k_total = static_cast<uint32_t>(k_tot);
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int q = threadIdx.x + p * THREADS;
            const int64_t n = col0 + q / (BK / 4);
            col_ok[p] = q < kQuads && n < n_total;
            // Columns past the operand (an edge tile) read its last column:
            // they only feed outputs that are never stored.
            const uint32_t nn = static_cast<uint32_t>(n < n_total ? n : n_total - 1);
            uint32_t rem;
            const uint32_t img = DivMod(pv.div_plane, nn, rem);
            uint32_t ow;
            const uint32_t oh = DivMod(pv.div_ow, rem, ow);
            col_off[p] = ((img * static_cast<uint32_t>(pv.c) * static_cast<uint32_t>(pv.in_h) +
                           oh * static_cast<uint32_t>(pv.kh)) *
                              static_cast<uint32_t>(pv.in_w) +
                          ow * static_cast<uint32_t>(pv.kw));
        }
    }
    __device__ __forceinline__ uint32_t KOff(uint32_t k) const {
        uint32_t rem;
        const uint32_t c = DivMod(v->div_khkw, k, rem);
        uint32_t q;
        const uint32_t r = DivMod(v->div_kw, rem, q);
        return (c * static_cast<uint32_t>(v->in_h) + r) * static_cast<uint32_t>(v->in_w) + q;
    }
    __device__ __forceinline__ void load(int64_t k0, Stage& s) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int q = tid + p * THREADS;
            const uint32_t k = static_cast<uint32_t>(k0) + static_cast<uint32_t>((q % (BK / 4)) * 4);
            if constexpr (!CHECKED) {
                if (kQuads % THREADS != 0 && q >= kQuads) {
                    continue; // this thread owns no quad in this pass
                }
                const nert_floatx4 val = *reinterpret_cast<const nert_floatx4*>(v->x + col_off[p] + KOff(k));
                s.v[p][0] = val[0];
                s.v[p][1] = val[1];
                s.v[p][2] = val[2];
                s.v[p][3] = val[3];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool ok = col_ok[p] && k + e < k_total;
                    const float x = v->x[ok ? col_off[p] + KOff(k + e) : 0];
                    s.v[p][e] = ok ? x : 0.f;
                }
            }
        }
    }
    __device__ __forceinline__ void store(const Stage& s, float* lds) const { Rows{}.store(s, lds); }
};

// The epilogue of every GEMM kernel: alpha * acc, plus beta * bias, then the
// optional Gelu chain, each operation rounded on its own (no contraction),
// so a fused MatMul -> Mul -> Add -> Div/Erf/Add/Mul/Mul row reproduces the
// separate rows' float results bit for bit. The division is IEEE (HIP's
// default correctly rounded fp32 divide), as in the Div row, and erff is the
// Erf row's function.
__device__ __forceinline__ float FinishWith(const GemmArgs& p, float acc, float bias) {
    float value = __fmul_rn(p.alpha, acc);
    if (p.has_bias) {
        value = __fadd_rn(value, __fmul_rn(p.beta, bias));
    }
    if (p.act == 1) {
        const float e = __fadd_rn(erff(value / p.act_div), p.act_add);
        value = __fmul_rn(__fmul_rn(value, e), p.act_mul);
    }
    return value;
}

__device__ __forceinline__ float FinishGemm(const GemmArgs& p, float acc, int64_t r, int64_t c) {
    return FinishWith(p, acc, p.has_bias ? p.bias[r * p.bias_sm + c * p.bias_sn] : 0.0f);
}

// Writes a workgroup's accumulators: raw partial sums (finish = false) or
// finished outputs. Per 32x32 block, every bias load comes from a clamped,
// always-valid address and all sixteen addresses are formed before the first
// store, so the loads and stores of a lane are in flight together instead
// of one guarded access and one wait after another.
template <class Shape>
__device__ __forceinline__ void GemmEpilogue(const GemmArgs& p, const Accum<Shape>& acc, float* out, int64_t row0,
                                             int64_t col0, bool finish) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wave_m = wave % Shape::kWavesM;
    const int wave_n = wave / Shape::kWavesM;
    const int half = lane >> 5;
    // Finished outputs follow the output layout (GemmOutIndex); raw partial
    // sums stay dense [m][n].
    const bool grouped = finish && p.y_group > 0;
    const int64_t row_stride = grouped ? p.y_group : p.n;
#pragma unroll
    for (int j = 0; j < Shape::kSubN; ++j) {
        const int64_t gc = col0 + wave_n * Shape::kWaveN + 32 * j + (lane & 31);
        const bool col_ok = gc < p.n;
        const int64_t cc = col_ok ? gc : 0;
        const int64_t col_base = grouped ? GemmOutIndex(p, 0, cc) : cc;
#pragma unroll
        for (int i = 0; i < Shape::kSubM; ++i) {
            const int64_t r0 = row0 + wave_m * Shape::kWaveM + 32 * i + 4 * half;
            float* base = out + r0 * row_stride + col_base;
            float value[16];
            bool ok[16];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t r = r0 + 8 * (v >> 2) + (v & 3);
                ok[v] = col_ok && r < p.m;
                float bias = 0.0f;
                if (finish && p.has_bias) {
                    const int64_t rr = r < p.m ? r : p.m - 1;
                    bias = p.bias[rr * p.bias_sm + cc * p.bias_sn];
                }
                value[v] = finish ? FinishWith(p, acc.c[i][j][v], bias) : acc.c[i][j][v];
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                if (ok[v]) {
                    base[(8 * (v >> 2) + (v & 3)) * row_stride] = value[v];
                }
            }
        }
    }
}

template <class Shape, bool A_KCONTIG, bool B_NCONTIG, int FLUSH, bool B_PATCH = false>
__global__ __launch_bounds__(Shape::kThreads) void GemmKernel(GemmArgs p) {
    __shared__ __attribute__((aligned(16))) float lds[2 * (Shape::kLdsA + Shape::kLdsB)];
    const int64_t tiles_m = (p.m + Shape::kBM - 1) / Shape::kBM;
    const int64_t tile = blockIdx.x;
    const int64_t tm = tile % tiles_m;
    const int64_t tn = tile / tiles_m;
    const int64_t row0 = tm * Shape::kBM;
    const int64_t col0 = tn * Shape::kBN;
    const int64_t batch = blockIdx.y;
    const int split = blockIdx.z;

    // Batch offsets from the broadcast strides (innermost axis last).
    int64_t a_off = 0;
    int64_t b_off = 0;
    int64_t rem = batch;
    for (int d = p.batch_rank - 1; d >= 0; --d) {
        const int64_t idx = rem % p.bdims[d];
        rem /= p.bdims[d];
        a_off += idx * p.a_bs[d];
        b_off += idx * p.b_bs[d];
    }
    const float* a = p.a + a_off;
    const float* b = p.b + b_off;

    const int64_t k_begin = static_cast<int64_t>(split) * p.k_per_split;
    int64_t k_end = k_begin + p.k_per_split;
    if (k_end > p.k) {
        k_end = p.k;
    }

    Accum<Shape> acc;
    acc.zero();
    // Tiles with 16-byte aligned rows take unchecked float4 loads for every
    // full K tile; the K remainder uses the checked form. So do edge tiles
    // whose missing rows (or columns) the unchecked loaders can stand in for
    // with valid ones -- any count along a K-contiguous operand, whole quads
    // along a row-contiguous one: those rows only reach outputs that are never
    // stored, and the stored outputs sum the same products in the same order.
    const bool a_vec = (A_KCONTIG ? p.a_sm : p.a_sk) % 4 == 0 && ((reinterpret_cast<uintptr_t>(a) & 15) == 0);
    const bool b_vec =
        B_PATCH || ((B_NCONTIG ? p.b_sk : p.b_sn) % 4 == 0 && ((reinterpret_cast<uintptr_t>(b) & 15) == 0));
    const bool a_rows = row0 + Shape::kBM <= p.m || A_KCONTIG || p.m % 4 == 0;
    const bool b_cols = col0 + Shape::kBN <= p.n || !B_NCONTIG || p.n % 4 == 0;
    const bool interior = a_vec && b_vec && a_rows && b_cols;
    const int64_t k_full = interior ? k_begin + (k_end - k_begin) / Shape::kBK * Shape::kBK : k_begin;
    if (k_full > k_begin) {
        const auto aload = MakeOperand<Shape::kBM, Shape::kBK, Shape::kThreads, Shape::kPitchA, A_KCONTIG, false>(
            a, row0, p.a_sm, p.a_sk, p.m, k_full);
        if constexpr (B_PATCH) {
            PatchLoader<Shape::kBN, Shape::kBK, Shape::kThreads, Shape::kPitchB, false> bload;
            bload.init(p.patch, col0, p.n, k_full);
            MainLoop<Shape, FLUSH>(aload, bload, k_begin, k_full, lds, acc);
        } else {
            const auto bload = MakeOperand<Shape::kBN, Shape::kBK, Shape::kThreads, Shape::kPitchB, !B_NCONTIG, false>(
                b, col0, p.b_sn, p.b_sk, p.n, k_full);
            MainLoop<Shape, FLUSH>(aload, bload, k_begin, k_full, lds, acc);
        }
    }
    if (k_full < k_end) {
        const auto aload = MakeOperand<Shape::kBM, Shape::kBK, Shape::kThreads, Shape::kPitchA, A_KCONTIG, true>(
            a, row0, p.a_sm, p.a_sk, p.m, k_end);
        if constexpr (B_PATCH) {
            PatchLoader<Shape::kBN, Shape::kBK, Shape::kThreads, Shape::kPitchB, true> bload;
            bload.init(p.patch, col0, p.n, k_end);
            MainLoop<Shape, FLUSH>(aload, bload, k_full, k_end, lds, acc);
        } else {
            const auto bload = MakeOperand<Shape::kBN, Shape::kBK, Shape::kThreads, Shape::kPitchB, !B_NCONTIG, true>(
                b, col0, p.b_sn, p.b_sk, p.n, k_end);
            MainLoop<Shape, FLUSH>(aload, bload, k_full, k_end, lds, acc);
        }
    }

    const int64_t plane = p.m * p.n;
    if (p.counters != nullptr) {
        const int64_t t = batch * gridDim.x + tile;
        float* slots = p.split_slots + t * gridDim.z * Shape::kBM * Shape::kBN;
        if (FinishSplitTile<Shape, double>(acc, slots, p.counters + t, split, static_cast<int>(gridDim.z),
                                           reinterpret_cast<int*>(lds))) {
            GemmEpilogue<Shape>(p, acc, p.y + batch * plane, row0, col0, true);
        }
        return;
    }
    if (p.partial != nullptr) {
        GemmEpilogue<Shape>(p, acc, p.partial + (static_cast<int64_t>(split) * gridDim.y + batch) * plane, row0, col0,
                            false);
        return;
    }
    GemmEpilogue<Shape>(p, acc, p.y + batch * plane, row0, col0, true);
}

// Sums the split-K partials in split order (deterministic), in double with
// one rounding, and applies the epilogue, four outputs per thread when rows
// hold whole quads.
__global__ void SplitReduceKernel(GemmArgs p, int splits, int64_t batches, int vec) {
    const int64_t plane = p.m * p.n;
    const int64_t total = plane * batches;
    const int64_t quads = total / vec;
    for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < quads;
         q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t i = q * vec;
        const int64_t e = i % plane;
        const int64_t r = e / p.n;
        const int64_t c = e % p.n;
        for (int v = 0; v < vec; ++v) {
            double sum = p.partial[i + v];
            for (int s = 1; s < splits; ++s) {
                sum += p.partial[s * total + i + v];
            }
            p.y[(i - e) + GemmOutIndex(p, r, c + v)] = FinishGemm(p, static_cast<float>(sum), r, c + v);
        }
    }
}

// The same sums for rows of whole quads under 2^31 outputs: four consecutive
// outputs of one row per thread, 32-bit index decoding, and the 16-byte loads
// of up to eight splits issued before the first addition (splits past the
// last re-read the last one's address and are not added), so a thread waits
// for memory once per eight splits rather than once per split. The additions
// are SplitReduceKernel's, in the same order, so the results are identical.
__global__ __launch_bounds__(256) void SplitReduceQuadKernel(GemmArgs p, int splits, uint32_t quads, uint32_t total,
                                                             FastDiv div_row_quads, FastDiv div_m) {
    for (uint32_t q = blockIdx.x * 256u + threadIdx.x; q < quads; q += gridDim.x * 256u) {
        uint32_t cq, r;
        const uint32_t row = DivMod(div_row_quads, q, cq); // over all batches
        DivMod(div_m, row, r);
        const uint32_t i = 4 * q;
        double sum[4];
        for (int s0 = 0; s0 < splits; s0 += 8) {
            nert_floatx4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int s = min(s0 + j, splits - 1);
                v[j] = *reinterpret_cast<const nert_floatx4*>(p.partial + static_cast<int64_t>(s) * total + i);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (s0 + j == 0) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        sum[e] = v[j][e];
                    }
                } else if (s0 + j < splits) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        sum[e] += v[j][e];
                    }
                }
            }
        }
        nert_floatx4 out;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            out[e] = FinishGemm(p, static_cast<float>(sum[e]), r, 4 * cq + e);
        }
        // Four columns of one output group (groups are whole quads).
        const int64_t at = p.y_group > 0 ? GemmOutIndex(p, r, 4 * static_cast<int64_t>(cq)) : i;
        *reinterpret_cast<nert_floatx4*>(p.y + at) = out;
    }
}

// Skinny GEMM (M <= 32, K contiguous in both operands: the ResNet classifier
// and Gemm with transB): one workgroup per 32 output columns; each of its 8
// waves takes an eighth of K and runs MFMAs straight from 16-byte global
// loads -- lane half h holds k = 8j + 4h .. 8j + 4h + 3 of its A row and B
// column, so one load pair feeds four MFMA steps; with K up to 512 all of a
// wave's loads are in flight at once -- then the eight partial 32x32 blocks
// are summed through LDS in wave order (deterministic) and the epilogue is
// the engine's alpha * acc + beta * bias. One launch, no split-K partials in
// memory.
constexpr int kSkinnyWaves = 8;

__global__ __launch_bounds__(512) void SkinnyGemmKernel(GemmArgs p, int64_t k_slice) {
    __shared__ float part[kSkinnyWaves - 1][64][17];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int half = lane >> 5;
    const int64_t m = lane & 31;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * 32 + (lane & 31);
    const int64_t k_begin = wave * k_slice;
    const int64_t k_end = std::min<int64_t>(k_begin + k_slice, p.k);
    const bool m_ok = m < p.m;
    const bool n_ok = n < p.n;
    const float* ap = p.a + (m_ok ? m : 0) * p.a_sm + 4 * half;
    const float* bp = p.b + (n_ok ? n : 0) * p.b_sn + 4 * half;
    nert_floatx16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        acc[v] = 0.0f;
    }
#pragma unroll 8
    for (int64_t k = k_begin; k < k_end; k += 8) {
        nert_floatx4 a = *reinterpret_cast<const nert_floatx4*>(ap + k);
        nert_floatx4 b = *reinterpret_cast<const nert_floatx4*>(bp + k);
        if (!m_ok) {
            a = nert_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        if (!n_ok) {
            b = nert_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kk], b[kk], acc, 0, 0, 0);
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            part[wave - 1][lane][v] = acc[v];
        }
    }
    __syncthreads();
    if (wave != 0) {
        return;
    }
#pragma unroll
    for (int w = 0; w < kSkinnyWaves - 1; ++w) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            acc[v] += part[w][lane][v];
        }
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int64_t r = 8 * (v >> 2) + 4 * half + (v & 3);
        if (r < p.m && n_ok) {
            p.y[r * p.n + n] = FinishGemm(p, acc[v], r, n);
        }
    }
}

bool SkinnyApplies(const GemmArgs& p, int64_t batches) {
    return batches == 1 && p.patch.x == nullptr && p.y_group == 0 && p.m <= 32 && p.a_sk == 1 && p.b_sk == 1 && p.k % 8 == 0 && p.a_sm % 4 == 0 &&
           p.b_sn % 4 == 0 && (reinterpret_cast<uintptr_t>(p.a) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(p.b) & 15) == 0 && p.k > 0 && (p.n + 31) / 32 < (int64_t{1} << 31);
}

void LaunchSkinny(const GemmArgs& p, hipStream_t stream) {
    // A multiple of 8; kSkinnyWaves slices cover K.
    const int64_t k_slice = ((p.k + 8 * kSkinnyWaves - 1) / (8 * kSkinnyWaves)) * 8;
    SkinnyGemmKernel<<<static_cast<unsigned>((p.n + 31) / 32), 64 * kSkinnyWaves, 0, stream>>>(p, k_slice);
    CheckLaunch("SkinnyGemmKernel launch");
}

// Tile shapes, chosen from a sweep over the BASELINE GEMM/MatMul shapes and
// the ViT projections on MI355X: 8 waves of 64x32 for problems with at least
// 1024 such tiles (4096^3: 135 TFLOP/s), 4 waves of 32x64 below that (more
// workgroups in flight hide the load latency), 2 waves for M <= 32.
constexpr int64_t kTwoLevelK = 1024;
constexpr int64_t kChunkK = 512;
using ShapeL = TileShape<128, 128, 16, 2, 4>; // 8 waves, 64x32 per wave
using ShapeM = TileShape<64, 128, 16, 2, 2>;  // 4 waves, 32x64 per wave
using ShapeS = TileShape<32, 64, 32, 1, 2>;   // 2 waves, skinny M
// The M and L tiles with 32-deep K steps: half the LDS-store/barrier phases
// per K, twice the LDS.
using ShapeMK = TileShape<64, 128, 32, 2, 2>;  // 4 waves, 32x64 per wave
using ShapeLK = TileShape<128, 128, 32, 2, 4>; // 8 waves, 64x32 per wave
// 4 waves of 32x32 for products a few hundred 64x128 tiles cover unevenly
// (N = 768 next to M ~ 3000: 294 such tiles on 256 CUs, 600 of these).
using ShapeQ = TileShape<64, 64, 32, 2, 2>;

template <class Shape>
void LaunchShape(GemmArgs p, int64_t batches, int splits, hipStream_t stream) {
    const int64_t tiles = ((p.m + Shape::kBM - 1) / Shape::kBM) * ((p.n + Shape::kBN - 1) / Shape::kBN);
    dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(batches), static_cast<unsigned>(splits));
    if (p.counters != nullptr) {
        p.split_slots = static_cast<float*>(
            Workspace(tiles * batches * splits * Shape::kBM * Shape::kBN * static_cast<int64_t>(sizeof(float)), stream));
    }
    dim3 block(Shape::kThreads);
    const bool a_k = p.a_sk == 1;
    const bool b_n = p.b_sn == 1;
    // K ranges beyond kTwoLevelK accumulate in chunks of kChunkK (see
    // MainLoop); shorter ones keep one set of accumulators (the second set
    // costs occupancy).
    const bool two_level = p.k_per_split > kTwoLevelK;
    constexpr int kFlush = kChunkK / Shape::kBK;
    if (p.patch.x != nullptr) {
        // (A K-contiguous, one batch: LaunchGemm checks.)
        two_level ? GemmKernel<Shape, true, false, kFlush, true><<<grid, block, 0, stream>>>(p)
                  : GemmKernel<Shape, true, false, 0, true><<<grid, block, 0, stream>>>(p);
    } else if (a_k && b_n) {
        two_level ? GemmKernel<Shape, true, true, kFlush><<<grid, block, 0, stream>>>(p)
                  : GemmKernel<Shape, true, true, 0><<<grid, block, 0, stream>>>(p);
    } else if (a_k) {
        two_level ? GemmKernel<Shape, true, false, kFlush><<<grid, block, 0, stream>>>(p)
                  : GemmKernel<Shape, true, false, 0><<<grid, block, 0, stream>>>(p);
    } else if (b_n) {
        two_level ? GemmKernel<Shape, false, true, kFlush><<<grid, block, 0, stream>>>(p)
                  : GemmKernel<Shape, false, true, 0><<<grid, block, 0, stream>>>(p);
    } else {
        two_level ? GemmKernel<Shape, false, false, kFlush><<<grid, block, 0, stream>>>(p)
                  : GemmKernel<Shape, false, false, 0><<<grid, block, 0, stream>>>(p);
    }
    CheckLaunch("GemmKernel launch");
}

template <class Shape>
int64_t TileCount(const GemmArgs& p, int64_t batches) {
    return ((p.m + Shape::kBM - 1) / Shape::kBM) * ((p.n + Shape::kBN - 1) / Shape::kBN) * batches;
}

} // namespace

namespace {

// One configuration: tile shape (0 L, 1 M, 2 S, 3 MK, 4 LK, 5 Q) and split-K count
// (0: the PlanSplits choice for that shape).
void LaunchConfig(GemmArgs p, int64_t batches, int shape, int force_splits, hipStream_t stream) {
    int64_t tiles;
    int64_t min_k_tiles = 8;
    int bk = ShapeL::kBK;
    if (shape == 0) {
        tiles = TileCount<ShapeL>(p, batches);
    } else if (shape == 1) {
        tiles = TileCount<ShapeM>(p, batches);
    } else if (shape == 3) {
        tiles = TileCount<ShapeMK>(p, batches);
        min_k_tiles = 4;
        bk = ShapeMK::kBK;
    } else if (shape == 4) {
        tiles = TileCount<ShapeLK>(p, batches);
        min_k_tiles = 4;
        bk = ShapeLK::kBK;
    } else if (shape == 5) {
        tiles = TileCount<ShapeQ>(p, batches);
        min_k_tiles = 4;
        bk = ShapeQ::kBK;
    } else {
        tiles = TileCount<ShapeS>(p, batches);
        min_k_tiles = 2;
        bk = ShapeS::kBK;
    }
    const int64_t k_tiles = (p.k + bk - 1) / bk;
    // The 2- and 4-wave shapes keep about 1024 workgroups resident.
    const bool eight_waves = shape == 0 || shape == 4;
    int splits = force_splits > 0
                     ? static_cast<int>(std::min<int64_t>(force_splits, std::max<int64_t>(k_tiles, 1)))
                     : PlanSplits(tiles, k_tiles, eight_waves ? kResidentBlocks : 2 * kResidentBlocks, min_k_tiles, 32);
    p.k_per_split = ((k_tiles + splits - 1) / splits) * bk;
    if (p.k == 0) {
        p.k_per_split = 0;
        splits = 1;
    }
    p.partial = nullptr;
    p.counters = nullptr;
    p.split_slots = nullptr;
    if (splits > 1) {
        // Split tiles finish inside the kernel when the counters suffice,
        // else in the reduce kernels below.
        p.counters = TileCounters(tiles);
        if (p.counters == nullptr) {
            p.partial =
                static_cast<float*>(Workspace(static_cast<int64_t>(splits) * batches * p.m * p.n * 4, stream));
        }
    }
    switch (shape) {
    case 0:
        LaunchShape<ShapeL>(p, batches, splits, stream);
        break;
    case 1:
        LaunchShape<ShapeM>(p, batches, splits, stream);
        break;
    case 3:
        LaunchShape<ShapeMK>(p, batches, splits, stream);
        break;
    case 4:
        LaunchShape<ShapeLK>(p, batches, splits, stream);
        break;
    case 5:
        LaunchShape<ShapeQ>(p, batches, splits, stream);
        break;
    default:
        LaunchShape<ShapeS>(p, batches, splits, stream);
        break;
    }
    if (splits > 1 && p.counters == nullptr) {
        const int vec = p.n % 4 == 0 ? 4 : 1;
        const int64_t total = batches * p.m * p.n;
        const int64_t work = total / vec;
        if (vec == 4 && total < (int64_t{1} << 31) && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0) {
            SplitReduceQuadKernel<<<GridFor(work, 256, 8192), 256, 0, stream>>>(
                p, splits, static_cast<uint32_t>(work), static_cast<uint32_t>(total),
                FastDiv::Make(static_cast<uint32_t>(p.n / 4)), FastDiv::Make(static_cast<uint32_t>(p.m)));
        } else {
            SplitReduceKernel<<<GridFor(work, 256, 8192), 256, 0, stream>>>(p, splits, batches, vec);
        }
        CheckLaunch("SplitReduceKernel launch");
    }
}

// Candidates: 0-11 shape i / 4 (L, M, S) with split count {PlanSplits, 1,
// 2, 4}[i % 4]; 12 the skinny kernel; 13-24 shape 3 + (i - 13) / 4 (MK, LK,
// Q) with split count {...}[(i - 13) % 4].
// Fallback (capture, tuning off): 8-wave 128x128 tiles for problems with at
// least 1024 of them, 4-wave 64x128 below, 2-wave 32x64 for M <= 32.
using GemmKey = std::array<int64_t, 10>;
constexpr int kGemmSplits[4] = {0, 1, 2, 4};
constexpr int kGemmCandidates = 25;
constexpr int kSkinnyCandidate = 12;

void LaunchTiled(const GemmArgs& p, int64_t batches, int i, hipStream_t stream) {
    if (i < kSkinnyCandidate) {
        LaunchConfig(p, batches, i / 4, kGemmSplits[i % 4], stream);
    } else {
        LaunchConfig(p, batches, 3 + (i - kSkinnyCandidate - 1) / 4, kGemmSplits[(i - kSkinnyCandidate - 1) % 4],
                     stream);
    }
}

} // namespace

void LaunchGemm(GemmArgs p, int64_t batches, hipStream_t stream) {
    if (p.m == 0 || p.n == 0 || batches == 0) {
        return;
    }
    // Operand strides must make one of each pair unit (contiguous tensors).
    if (!(p.a_sk == 1 || p.a_sm == 1) || !(p.b_sn == 1 || p.b_sk == 1)) {
        throw Error("gemm: operands must be contiguous in one index");
    }
    if (p.y_group > 0 && (batches != 1 || p.y_group % 4 != 0 || p.n % p.y_group != 0)) {
        throw Error("gemm: grouped output needs one batch and groups of whole quads dividing n");
    }
    if (p.patch.x != nullptr && (batches != 1 || p.a_sk != 1 || p.patch.kw % 4 != 0 ||
                                 (reinterpret_cast<uintptr_t>(p.patch.x) & 15) != 0)) {
        throw Error("gemm: an in-place patch operand needs one batch, A K-contiguous and 16-byte runs");
    }
    const int fallback_shape = p.m <= 32 ? 2 : (TileCount<ShapeL>(p, batches) < 1024 ? 1 : 0);
    static std::mutex mu;
    static std::map<GemmKey, int> chosen;
    // The key leaves the epilogue out: a fused and an unfused call of the
    // same product sum in the same order.
    const GemmKey key{p.m, p.n, p.k, batches, p.a_sk == 1, p.b_sn == 1, p.batch_rank, p.patch.x != nullptr, 0, 0};
    const size_t y_bytes = static_cast<size_t>(batches * p.m * p.n) * sizeof(float);
    const bool skinny = SkinnyApplies(p, batches);
    // NERT_HIP_GEMM_CANDIDATE=i forces candidate i wherever it applies (tests
    // of each configuration use it).
    if (const char* forced = std::getenv("NERT_HIP_GEMM_CANDIDATE")) {
        const int i = std::atoi(forced);
        if (i == kSkinnyCandidate && skinny) {
            LaunchSkinny(p, stream);
            return;
        }
        if (i >= 0 && i < kGemmCandidates && i != kSkinnyCandidate) {
            LaunchTiled(p, batches, i, stream);
            return;
        }
    }
    const int c = ChooseConfig("gemm", chosen, mu, key, y_bytes, stream, kGemmCandidates, 4 * fallback_shape,
                               [&](int i, float* scratch) {
                                   GemmArgs q = p;
                                   q.y = scratch;
                                   if (i == kSkinnyCandidate) {
                                       if (!skinny) {
                                           return false;
                                       }
                                       LaunchSkinny(q, stream);
                                       return true;
                                   }
                                   LaunchTiled(q, batches, i, stream);
                                   return true;
                               });
    if (c == kSkinnyCandidate && skinny) {
        LaunchSkinny(p, stream);
        return;
    }
    // (A cached skinny choice with operands that lost its alignment takes
    // the fallback tiles.)
    LaunchTiled(p, batches, c == kSkinnyCandidate ? 4 * fallback_shape : c, stream);
}

} // namespace nert_hip

extern "C" {

int nert_hip_gemm_f32(const float* a, const float* b, const float* c, float* y, int64_t m, int64_t n, int64_t k,
                      int trans_a, int trans_b, float alpha, float beta, int c_rank, void* stream) {
    return nert_hip::Guard([&] {
        nert_hip::GemmArgs p{};
        p.a = a;
        p.b = b;
        p.y = y;
        p.m = m;
        p.n = n;
        p.k = k;
        // A is stored [M,K] (trans_a = 0) or [K,M]; B is [K,N] or [N,K].
        p.a_sm = trans_a ? 1 : k;
        p.a_sk = trans_a ? m : 1;
        p.b_sk = trans_b ? 1 : n;
        p.b_sn = trans_b ? k : 1;
        p.alpha = alpha;
        p.beta = beta;
        p.has_bias = (c != nullptr && c_rank > 0) ? 1 : 0;
        p.bias = c;
        p.bias_sm = c_rank == 2 ? n : 0;
        p.bias_sn = 1;
        p.batch_rank = 0;
        nert_hip::LaunchGemm(p, 1, nert_hip::StreamOr(stream));
    });
}

int nert_hip_matmul_f32(const float* a, const float* b, float* y, int64_t m, int64_t n, int64_t k, int batch_rank,
                        const int64_t* batch_dims, const int64_t* a_batch_strides, const int64_t* b_batch_strides,
                        void* stream) {
    return nert_hip_matmul_fused_f32(a, b, nullptr, y, m, n, k, batch_rank, batch_dims, a_batch_strides,
                                     b_batch_strides, 1.0f, 0, nullptr, stream);
}

int nert_hip_matmul_fused_f32(const float* a, const float* b, const float* bias, float* y, int64_t m, int64_t n,
                              int64_t k, int batch_rank, const int64_t* batch_dims, const int64_t* a_batch_strides,
                              const int64_t* b_batch_strides, float scale, int act, const float* act_params,
                              void* stream) {
    return nert_hip::Guard([&] {
        if (act != 0 && (act != 1 || act_params == nullptr)) {
            throw nert_hip::Error("matmul: unknown activation");
        }
        if (batch_rank < 0 || batch_rank > 4) {
            throw nert_hip::Error("matmul: at most four batch axes are supported");
        }
        nert_hip::GemmArgs p{};
        p.a = a;
        p.b = b;
        p.y = y;
        p.m = m;
        p.n = n;
        p.k = k;
        p.a_sm = k;
        p.a_sk = 1;
        p.b_sk = n;
        p.b_sn = 1;
        p.alpha = scale;
        p.beta = 1.0f;
        p.has_bias = bias != nullptr ? 1 : 0;
        p.bias = bias;
        p.bias_sm = 0;
        p.bias_sn = 1;
        p.act = act;
        if (act == 1) {
            p.act_div = act_params[0];
            p.act_add = act_params[1];
            p.act_mul = act_params[2];
        }
        p.batch_rank = batch_rank;
        int64_t batches = 1;
        for (int d = 0; d < batch_rank; ++d) {
            p.bdims[d] = batch_dims[d];
            p.a_bs[d] = a_batch_strides[d];
            p.b_bs[d] = b_batch_strides[d];
            batches *= batch_dims[d];
        }
        if (batches > 65535) {
            throw nert_hip::Error("matmul: more than 65535 batches");
        }
        nert_hip::LaunchGemm(p, batches, nert_hip::StreamOr(stream));
    });
}

} // extern "C"
