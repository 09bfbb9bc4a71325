#pragma once
// fp32 MFMA tile engine for gfx950 (CDNA4), shared by Gemm, MatMul and the
// implicit-GEMM Conv.
//
// One workgroup computes a BM x BN tile of Y = op(A) * op(B) over a K range.
// The operands are staged through LDS in k-major form (As[k][m], Bs[k][n]) so
// that one MFMA fragment is 32 consecutive floats of one LDS row: lanes 0-31
// read k = k0 and lanes 32-63 read k = k0+1 of the same 32 columns, which is
// bank-conflict free. Global -> register loads of tile t+1 are issued before
// the MFMAs of tile t and written to the other LDS buffer afterwards (double
// buffering, one barrier per K tile).
//
// v_mfma_f32_32x32x2_f32 lane layout (wave64, one block):
//   A fragment: lane l holds A[row = l % 32][k = l / 32]
//   B fragment: lane l holds B[k = l / 32][col = l % 32]
//   D (16 regs): lane l, reg v holds D[row = 8*(v/4) + 4*(l/32) + v%4][col = l % 32]
//
// Operand loaders are policy classes. A loader fills a register stage with
// the elements its thread owns for one K tile (zero outside the problem) and
// writes them to LDS; the engine does not know how the operands are laid out
// in memory, which is what lets Conv gather its B operand straight from NCHW.

#include "common.hpp"

namespace nert_hip {

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N>
struct TileShape {
    static constexpr int kBM = BM;
    static constexpr int kBN = BN;
    static constexpr int kBK = BK;
    static constexpr int kWavesM = WAVES_M;
    static constexpr int kWavesN = WAVES_N;
    static constexpr int kThreads = WAVES_M * WAVES_N * 64;
    static constexpr int kWaveM = BM / WAVES_M; // rows per wave
    static constexpr int kWaveN = BN / WAVES_N; // cols per wave
    static constexpr int kSubM = kWaveM / 32;   // 32x32 MFMA blocks per wave along M
    static constexpr int kSubN = kWaveN / 32;
    // Row pitch of the k-major LDS tiles. +4 floats keeps the 16-byte
    // alignment of vector stores and rotates rows across banks.
    static constexpr int kPitchA = BM + 4;
    static constexpr int kPitchB = BN + 4;
    static constexpr int kLdsA = BK * kPitchA;
    static constexpr int kLdsB = BK * kPitchB;
    static_assert(kWaveM % 32 == 0 && kWaveN % 32 == 0, "wave tile must be a multiple of 32x32");
    static_assert(BK % 2 == 0, "BK must be even (MFMA K = 2)");
};

// Accumulators of one wave: kSubM x kSubN blocks of 32x32.
template <class Shape>
struct Accum {
    nert_floatx16 c[Shape::kSubM][Shape::kSubN];
    __device__ void zero() {
#pragma unroll
        for (int i = 0; i < Shape::kSubM; ++i) {
#pragma unroll
            for (int j = 0; j < Shape::kSubN; ++j) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    c[i][j][v] = 0.0f;
                }
            }
        }
    }
};

// MFMAs over one LDS-resident K tile.
template <class Shape>
__device__ __forceinline__ void MmaTile(const float* __restrict__ as, const float* __restrict__ bs, Accum<Shape>& acc,
                                        int wave_m, int wave_n, int lane) {
    const int half = lane >> 5;
    const int col = lane & 31;
    const float* a_base = as + half * Shape::kPitchA + wave_m * Shape::kWaveM + col;
    const float* b_base = bs + half * Shape::kPitchB + wave_n * Shape::kWaveN + col;
#pragma unroll
    for (int kk = 0; kk < Shape::kBK; kk += 2) {
        float a[Shape::kSubM];
        float b[Shape::kSubN];
#pragma unroll
        for (int i = 0; i < Shape::kSubM; ++i) {
            a[i] = a_base[kk * Shape::kPitchA + 32 * i];
        }
#pragma unroll
        for (int j = 0; j < Shape::kSubN; ++j) {
            b[j] = b_base[kk * Shape::kPitchB + 32 * j];
        }
#pragma unroll
        for (int i = 0; i < Shape::kSubM; ++i) {
#pragma unroll
            for (int j = 0; j < Shape::kSubN; ++j) {
                acc.c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc.c[i][j], 0, 0, 0);
            }
        }
    }
}

// The K loop: ALoader/BLoader stage K tiles [k_begin, k_end) through LDS.
// Loader interface:
//   typename Stage;                       registers for one thread's share
//   void load(int64_t k0, Stage&)         global -> registers (zero-padded)
//   void store(const Stage&, float* lds)  registers -> k-major LDS tile
template <class Shape, class ALoader, class BLoader>
__device__ __forceinline__ void MainLoop(ALoader& aload, BLoader& bload, int64_t k_begin, int64_t k_end,
                                         float* lds, Accum<Shape>& acc) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave % Shape::kWavesM;
    const int wave_n = wave / Shape::kWavesM;
    float* as[2] = {lds, lds + Shape::kLdsA + Shape::kLdsB};
    float* bs[2] = {lds + Shape::kLdsA, lds + 2 * Shape::kLdsA + Shape::kLdsB};

    acc.zero();
    if (k_begin >= k_end) {
        return;
    }
    typename ALoader::Stage sa;
    typename BLoader::Stage sb;
    aload.load(k_begin, sa);
    bload.load(k_begin, sb);
    aload.store(sa, as[0]);
    bload.store(sb, bs[0]);
    __syncthreads();
    int cur = 0;
    for (int64_t k0 = k_begin; k0 < k_end; k0 += Shape::kBK) {
        const bool more = k0 + Shape::kBK < k_end;
        if (more) {
            aload.load(k0 + Shape::kBK, sa);
            bload.load(k0 + Shape::kBK, sb);
        }
        MmaTile<Shape>(as[cur], bs[cur], acc, wave_m, wave_n, lane);
        if (more) {
            aload.store(sa, as[cur ^ 1]);
            bload.store(sb, bs[cur ^ 1]);
        }
        __syncthreads();
        cur ^= 1;
    }
}

// Visits every accumulator element with its tile-relative (row, col).
template <class Shape, class F>
__device__ __forceinline__ void ForEachAccum(const Accum<Shape>& acc, F&& fn) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave % Shape::kWavesM;
    const int wave_n = wave / Shape::kWavesM;
    const int half = lane >> 5;
    const int col = lane & 31;
#pragma unroll
    for (int i = 0; i < Shape::kSubM; ++i) {
#pragma unroll
        for (int j = 0; j < Shape::kSubN; ++j) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = wave_m * Shape::kWaveM + 32 * i + 8 * (v >> 2) + 4 * half + (v & 3);
                const int c = wave_n * Shape::kWaveN + 32 * j + col;
                fn(r, c, acc.c[i][j][v]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Strided operand loaders (Gemm / MatMul).
//
// A(m, k) = a[m * sm + k * sk]; exactly one of sm, sk is 1 in practice
// (row-major A or transposed A). B(k, n) = b[k * sk + n * sn].
// "Row" = the operand's non-K index (m for A, n for B).
// ---------------------------------------------------------------------------

// Loader for an operand whose K index is contiguous in memory (A row-major,
// or B transposed). Each thread loads runs of 4 consecutive k for one row.
template <int ROWS, int BK, int THREADS, int PITCH>
struct KContigLoader {
    static constexpr int kQuads = ROWS * BK / 4;             // float4 groups per tile
    static constexpr int kPer = (kQuads + THREADS - 1) / THREADS;
    struct Stage {
        float v[kPer][4];
    };
    const float* base; // &op(row0, 0)
    int64_t row_stride;
    int64_t rows_left; // valid rows in this tile (<= ROWS)
    int64_t k_total;
    bool vec_ok; // row_stride % 4 == 0 and base 16-byte aligned

    __device__ void load(int64_t k0, Stage& s) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int q = tid + p * THREADS;
            const int row = q / (BK / 4);
            const int kq = (q % (BK / 4)) * 4;
            const int64_t k = k0 + kq;
            float4 val = make_float4(0.f, 0.f, 0.f, 0.f);
            if (q < kQuads && row < rows_left) {
                const float* src = base + row * row_stride + k;
                if (vec_ok && k + 3 < k_total) {
                    val = *reinterpret_cast<const float4*>(src);
                } else {
                    val.x = k + 0 < k_total ? src[0] : 0.f;
                    val.y = k + 1 < k_total ? src[1] : 0.f;
                    val.z = k + 2 < k_total ? src[2] : 0.f;
                    val.w = k + 3 < k_total ? src[3] : 0.f;
                }
            }
            s.v[p][0] = val.x;
            s.v[p][1] = val.y;
            s.v[p][2] = val.z;
            s.v[p][3] = val.w;
        }
    }
    __device__ void store(const Stage& s, float* lds) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int q = tid + p * THREADS;
            if (q < kQuads) {
                const int row = q / (BK / 4);
                const int kq = (q % (BK / 4)) * 4;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    lds[(kq + e) * PITCH + row] = s.v[p][e];
                }
            }
        }
    }
};

// Loader for an operand whose row index is contiguous (A transposed, or B
// row-major). Each thread loads runs of 4 consecutive rows at one k.
template <int ROWS, int BK, int THREADS, int PITCH>
struct RowContigLoader {
    static constexpr int kQuads = ROWS * BK / 4;
    static constexpr int kPer = (kQuads + THREADS - 1) / THREADS;
    struct Stage {
        float4 v[kPer];
    };
    const float* base; // &op(row0, 0)
    int64_t k_stride;
    int64_t rows_left;
    int64_t k_total;
    bool vec_ok; // k_stride % 4 == 0 and base 16-byte aligned

    __device__ void load(int64_t k0, Stage& s) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int q = tid + p * THREADS;
            const int kk = q / (ROWS / 4);
            const int row = (q % (ROWS / 4)) * 4;
            const int64_t k = k0 + kk;
            float4 val = make_float4(0.f, 0.f, 0.f, 0.f);
            if (q < kQuads && k < k_total) {
                const float* src = base + k * k_stride + row;
                if (vec_ok && row + 3 < rows_left) {
                    val = *reinterpret_cast<const float4*>(src);
                } else {
                    val.x = row + 0 < rows_left ? src[0] : 0.f;
                    val.y = row + 1 < rows_left ? src[1] : 0.f;
                    val.z = row + 2 < rows_left ? src[2] : 0.f;
                    val.w = row + 3 < rows_left ? src[3] : 0.f;
                }
            }
            s.v[p] = val;
        }
    }
    __device__ void store(const Stage& s, float* lds) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int q = tid + p * THREADS;
            if (q < kQuads) {
                const int kk = q / (ROWS / 4);
                const int row = (q % (ROWS / 4)) * 4;
                *reinterpret_cast<float4*>(lds + kk * PITCH + row) = s.v[p];
            }
        }
    }
};

} // namespace nert_hip
