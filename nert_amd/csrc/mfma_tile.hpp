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

// Adds `part` into `sum` element by element.
template <class Shape>
__device__ __forceinline__ void AddAccum(Accum<Shape>& sum, const Accum<Shape>& part) {
#pragma unroll
    for (int i = 0; i < Shape::kSubM; ++i) {
#pragma unroll
        for (int j = 0; j < Shape::kSubN; ++j) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                sum.c[i][j][v] += part.c[i][j][v];
            }
        }
    }
}

// The K loop: ALoader/BLoader stage K tiles [k_begin, k_end) through LDS and
// accumulate into `acc` (the caller zeroes it once, so a block may run an
// unchecked interior loop and a checked tail loop into the same registers).
// FLUSH > 0 accumulates in two levels: every FLUSH K tiles are summed in a
// fresh set of registers that is then added to `acc`, so the fp32 rounding
// error of a long dot product grows with the chunk length rather than with
// all of K (about 2.5 times smaller at K = 4096 with 512-element chunks). It
// costs a second set of accumulators, hence only for long K ranges.
// Loader interface:
//   typename Stage;                       registers for one thread's share
//   void load(int64_t k0, Stage&)         global -> registers (zero-padded)
//   void store(const Stage&, float* lds)  registers -> k-major LDS tile
template <class Shape, int FLUSH = 0, class ALoader, class BLoader>
__device__ __forceinline__ void MainLoop(const ALoader& aload, const BLoader& bload, int64_t k_begin, int64_t k_end,
                                         float* lds, Accum<Shape>& sum) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave % Shape::kWavesM;
    const int wave_n = wave / Shape::kWavesM;
    // Both LDS buffers sit at compile-time offsets from the shared array and
    // the tile loop is unrolled by two, so every LDS access keeps the LDS
    // address space (ds_read/ds_write) instead of decaying to flat accesses.
    float* const a0 = lds;
    float* const b0 = lds + Shape::kLdsA;
    float* const a1 = lds + Shape::kLdsA + Shape::kLdsB;
    float* const b1 = lds + 2 * Shape::kLdsA + Shape::kLdsB;

    if (k_begin >= k_end) {
        return;
    }
    typename ALoader::Stage sa;
    typename BLoader::Stage sb;
    aload.load(k_begin, sa);
    bload.load(k_begin, sb);
    aload.store(sa, a0);
    bload.store(sb, b0);
    __syncthreads();
    Accum<Shape> chunk_regs;
    Accum<Shape>& acc = FLUSH > 0 ? chunk_regs : sum;
    if constexpr (FLUSH > 0) {
        chunk_regs.zero();
    }
    int in_chunk = 0;
    auto after_tile = [&]() {
        if constexpr (FLUSH > 0) {
            if (++in_chunk == FLUSH) {
                AddAccum(sum, chunk_regs);
                chunk_regs.zero();
                in_chunk = 0;
            }
        }
    };
    int64_t k0 = k_begin;
    while (true) {
        bool more = k0 + Shape::kBK < k_end;
        if (more) {
            aload.load(k0 + Shape::kBK, sa);
            bload.load(k0 + Shape::kBK, sb);
        }
        MmaTile<Shape>(a0, b0, acc, wave_m, wave_n, lane);
        after_tile();
        if (more) {
            aload.store(sa, a1);
            bload.store(sb, b1);
        }
        __syncthreads();
        if (!more) {
            break;
        }
        k0 += Shape::kBK;
        more = k0 + Shape::kBK < k_end;
        if (more) {
            aload.load(k0 + Shape::kBK, sa);
            bload.load(k0 + Shape::kBK, sb);
        }
        MmaTile<Shape>(a1, b1, acc, wave_m, wave_n, lane);
        after_tile();
        if (more) {
            aload.store(sa, a0);
            bload.store(sb, b0);
        }
        __syncthreads();
        if (!more) {
            break;
        }
        k0 += Shape::kBK;
    }
    if constexpr (FLUSH > 0) {
        if (in_chunk != 0) {
            AddAccum(sum, chunk_regs);
        }
    }
}

// Split tiles finished inside the kernel. Every workgroup that computes one
// part of a tile's K sum stores its accumulators (slot `part` of the tile's
// `parts` slots of BM * BN floats, in register order: 16-byte pieces,
// consecutive threads at consecutive addresses) and counts itself in the
// tile's counter. The workgroup that brings the count to `parts` resets it
// to zero (for the next launch), adds the parts in part order (P0 + P1 + ...,
// in type Sum, rounded to float once: the order and precision of the
// separate reduce kernels, so the sum is the same whichever workgroup arrives
// last), leaves it in `acc` and returns true to run the epilogue; the others
// return false. No workgroup waits on another. `flag` is one int of LDS the
// workgroup no longer reads.
//
// The slots are stored and loaded with the sc1 cache policy, the device-scope
// coherence bit the compiler itself puts on device-scope atomic loads and
// stores: such an access is performed at a level shared by all XCDs, past
// their separate L2 caches, and a store counts as complete (vmcnt) only once
// it is. Waiting for the stores before the barrier and the counter increment
// therefore orders them without a device-scope fence, whose L2 writeback and
// invalidation would stall every workgroup of the XCD. The counter is a
// device-scope atomic.
namespace split_detail {

constexpr int kDeviceCoherent = 16; // cache policy: sc1

template <class Shape>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t SlotRsrc(float* slots, int parts) {
    return __builtin_amdgcn_make_buffer_rsrc(slots, static_cast<short>(0),
                                             parts * Shape::kBM * Shape::kBN * static_cast<int>(sizeof(float)),
                                             0x00020000);
}

// Byte offset of float4 v4 of block (i, j) in slot q, for this thread.
template <class Shape>
__device__ __forceinline__ int SlotAt(int q, int i, int j, int v4) {
    return (q * Shape::kBM * Shape::kBN + (((i * Shape::kSubN + j) * 4 + v4) * Shape::kThreads + threadIdx.x) * 4) *
           4;
}

template <class Shape>
__device__ __forceinline__ void StorePart(const Accum<Shape>& acc, __amdgpu_buffer_rsrc_t r, int part) {
#pragma unroll
    for (int i = 0; i < Shape::kSubM; ++i) {
#pragma unroll
        for (int j = 0; j < Shape::kSubN; ++j) {
#pragma unroll
            for (int v4 = 0; v4 < 4; ++v4) {
                const nert_floatx4 x{acc.c[i][j][4 * v4], acc.c[i][j][4 * v4 + 1], acc.c[i][j][4 * v4 + 2],
                                     acc.c[i][j][4 * v4 + 3]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(nert_uintx4, x), r,
                                                       SlotAt<Shape>(part, i, j, v4), 0, kDeviceCoherent);
            }
        }
    }
}

// After this workgroup's part stores: waits for them, counts the workgroup
// in, and returns (to every thread) whether it was the last of `parts`.
__device__ __forceinline__ bool ArriveLast(uint32_t* counter, int parts, int* flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = before + 1 == static_cast<uint32_t>(parts);
        if (last) {
            __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        *flag = last ? 1 : 0;
    }
    __syncthreads();
    return *flag != 0;
}

// Every part from the slots, this workgroup's own included (each thread
// reads back only what it stored), summed in part order in type Sum and
// rounded once. A float sum takes a 32x32 block at a time, the loads of four
// parts of it (64 floats) in flight together. A double sum would need twice
// the registers for that, which would set the register budget (and so the
// occupancy) of the GEMM kernels around it, so it takes four consecutive
// floats at a time (still four parts' loads in flight). Both add the parts
// of an element in the same order.
template <class Shape, class Sum>
__device__ __forceinline__ void SumParts(Accum<Shape>& acc, __amdgpu_buffer_rsrc_t r, int parts) {
    constexpr int kQuads = sizeof(Sum) > sizeof(float) ? 1 : 4; // float4 pieces per part per round
#pragma unroll
    for (int i = 0; i < Shape::kSubM; ++i) {
#pragma unroll
        for (int j = 0; j < Shape::kSubN; ++j) {
#pragma unroll
            for (int v0 = 0; v0 < 4; v0 += kQuads) {
                Sum sum[4 * kQuads];
                for (int q0 = 0; q0 < parts; q0 += 4) {
                    nert_floatx4 x[4][kQuads];
#pragma unroll
                    for (int dq = 0; dq < 4; ++dq) {
                        const int q = min(q0 + dq, parts - 1);
#pragma unroll
                        for (int v = 0; v < kQuads; ++v) {
                            x[dq][v] = __builtin_bit_cast(nert_floatx4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                            r, SlotAt<Shape>(q, i, j, v0 + v), 0,
                                                                            kDeviceCoherent));
                        }
                    }
#pragma unroll
                    for (int dq = 0; dq < 4; ++dq) {
                        if (q0 + dq < parts) {
#pragma unroll
                            for (int e = 0; e < 4 * kQuads; ++e) {
                                const Sum y = static_cast<Sum>(x[dq][e >> 2][e & 3]);
                                sum[e] = q0 + dq == 0 ? y : sum[e] + y;
                            }
                        }
                    }
                }
#pragma unroll
                for (int e = 0; e < 4 * kQuads; ++e) {
                    acc.c[i][j][4 * v0 + e] = static_cast<float>(sum[e]);
                }
            }
        }
    }
}

} // namespace split_detail

template <class Shape, class Sum>
__device__ __forceinline__ bool FinishSplitTile(Accum<Shape>& acc, float* slots, uint32_t* counter, int part,
                                                int parts, int* flag) {
    const __amdgpu_buffer_rsrc_t r = split_detail::SlotRsrc<Shape>(slots, parts);
    split_detail::StorePart<Shape>(acc, r, part);
    if (!split_detail::ArriveLast(counter, parts, flag)) {
        return false;
    }
    split_detail::SumParts<Shape, Sum>(acc, r, parts);
    return true;
}

// The same for two accumulators of one tile (a conv and its paired 1x1):
// both parts are stored before the one arrival, so a single counter serves
// both and the last workgroup sums both.
template <class Shape, class Sum>
__device__ __forceinline__ bool FinishSplitTilePair(Accum<Shape>& acc, float* slots, Accum<Shape>& acc2,
                                                    float* slots2, uint32_t* counter, int part, int parts,
                                                    int* flag) {
    const __amdgpu_buffer_rsrc_t r = split_detail::SlotRsrc<Shape>(slots, parts);
    const __amdgpu_buffer_rsrc_t r2 = split_detail::SlotRsrc<Shape>(slots2, parts);
    split_detail::StorePart<Shape>(acc, r, part);
    split_detail::StorePart<Shape>(acc2, r2, part);
    if (!split_detail::ArriveLast(counter, parts, flag)) {
        return false;
    }
    split_detail::SumParts<Shape, Sum>(acc, r, parts);
    split_detail::SumParts<Shape, Sum>(acc2, r2, parts);
    return true;
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
// Strided operand loaders (Gemm / MatMul / the weight side of Conv).
//
// A(m, k) = a[m * sm + k * sk]; exactly one of sm, sk is 1 (row-major or
// transposed A). B(k, n) = b[k * sk + n * sn]. "Row" = the operand's non-K
// index (m for A, n for B). CHECKED = false is the interior-tile form: every
// element is in range and 16-byte aligned, so loads are unconditional float4
// and the compiler can keep them all in flight. CHECKED = true guards rows and
// k with a clamped address and a select instead of a branch, so edge tiles do
// not serialise their loads either.
// ---------------------------------------------------------------------------

// Operand whose K index is contiguous in memory (A row-major, B transposed):
// each thread loads runs of 4 consecutive k of one row.
template <int ROWS, int BK, int THREADS, int PITCH, bool CHECKED>
struct KContigLoader {
    static constexpr int kQuads = ROWS * BK / 4;
    static constexpr int kPer = (kQuads + THREADS - 1) / THREADS;
    struct Stage {
        float v[kPer][4];
    };
    const float* base; // &op(row0, 0)
    int64_t row_stride;
    int64_t rows_left; // valid rows in this tile (<= ROWS)
    int64_t k_total;

    __device__ __forceinline__ void load(int64_t k0, Stage& s) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int q = tid + p * THREADS;
            const int row = q / (BK / 4);
            const int kq = (q % (BK / 4)) * 4;
            const int64_t k = k0 + kq;
            if constexpr (!CHECKED) {
                if (kQuads % THREADS != 0 && q >= kQuads) {
                    continue; // this thread owns no quad in this pass
                }
                // Rows past the operand (an edge tile) read its last row:
                // they only feed output rows that are never stored.
                const int64_t r = row < rows_left ? row : rows_left - 1;
                const nert_floatx4 val = *reinterpret_cast<const nert_floatx4*>(base + r * row_stride + k);
                s.v[p][0] = val[0];
                s.v[p][1] = val[1];
                s.v[p][2] = val[2];
                s.v[p][3] = val[3];
            } else {
                const bool row_ok = q < kQuads && row < rows_left;
                const int64_t row_off = row_ok ? row * row_stride : 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool ok = row_ok && k + e < k_total;
                    const float v = base[ok ? row_off + k + e : 0];
                    s.v[p][e] = ok ? v : 0.f;
                }
            }
        }
    }
    __device__ __forceinline__ void store(const Stage& s, float* lds) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int q = tid + p * THREADS;
            if (kQuads % THREADS == 0 || q < kQuads) {
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

// Operand whose row index is contiguous (A transposed, B row-major): each
// thread loads runs of 4 consecutive rows at one k.
template <int ROWS, int BK, int THREADS, int PITCH, bool CHECKED>
struct RowContigLoader {
    static constexpr int kQuads = ROWS * BK / 4;
    static constexpr int kPer = (kQuads + THREADS - 1) / THREADS;
    struct Stage {
        nert_floatx4 v[kPer]; // native vectors: HIP's float4 class defeats register promotion
    };
    const float* base; // &op(row0, 0)
    int64_t k_stride;
    int64_t rows_left;
    int64_t k_total;

    __device__ __forceinline__ void load(int64_t k0, Stage& s) const {
        const int tid = threadIdx.x;
        // k0 * k_stride is wave-uniform (scalar); kk * k_stride + row depends
        // on the thread only, so it stays out of the K loop.
        const float* tile = base + k0 * k_stride;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int q = tid + p * THREADS;
            const int kk = q / (ROWS / 4);
            const int row = (q % (ROWS / 4)) * 4;
            const int64_t k = k0 + kk;
            if constexpr (!CHECKED) {
                if (kQuads % THREADS != 0 && q >= kQuads) {
                    continue; // this thread owns no quad in this pass
                }
                // Quads past the operand (an edge tile whose valid rows are
                // whole quads) read quad 0: they only feed outputs that are
                // never stored.
                const int r = row < rows_left ? row : 0;
                s.v[p] = *reinterpret_cast<const nert_floatx4*>(tile + (kk * k_stride + r));
            } else {
                const bool k_ok = q < kQuads && k < k_total;
                const int64_t k_off = k_ok ? k * k_stride : 0;
                float e4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool ok = k_ok && row + e < rows_left;
                    const float v = base[ok ? k_off + row + e : 0];
                    e4[e] = ok ? v : 0.f;
                }
                s.v[p] = nert_floatx4{e4[0], e4[1], e4[2], e4[3]};
            }
        }
    }
    __device__ __forceinline__ void store(const Stage& s, float* lds) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int q = tid + p * THREADS;
            if (kQuads % THREADS == 0 || q < kQuads) {
                const int kk = q / (ROWS / 4);
                const int row = (q % (ROWS / 4)) * 4;
                *reinterpret_cast<nert_floatx4*>(lds + kk * PITCH + row) = s.v[p];
            }
        }
    }
};

} // namespace nert_hip
