// Fused scaled-dot-product attention over packed Q/K/V: the MatMul(Q, K^T),
// Mul by a scalar, Softmax(last axis) and MatMul(P, V) rows of a transformer
// encoder in one kernel, reading Q, K and V where the QKV projection left
// them and writing the heads straight into the [batch, token, heads x dim]
// layout the output projection reads. It backs the runner's FusedAttention
// row; the reference computes the same result with those four rows plus the
// Reshape/Transpose/Split/Squeeze copies around them
// (src/kernels/mat_mul.cpp, mul.cpp, softmax.cpp, transpose.cpp, split.cpp).
//
// One wave per (batch, head, block of 16 queries) streams over the keys in
// blocks of 16 with the running-maximum form of the softmax (the kernel's
// comment has the lane layout): scores, probabilities and the output block
// stay in registers, with no LDS and no barrier. Q and K fragments are
// 16-byte loads: lane group g holds dims 16 g .. 16 g + 15 of its row, so
// one load feeds four MFMA steps (the same dims for both operands, so the
// sum over the 64 dims is the dot product). 16 queries a wave instead of 32
// make twice the waves at under half the registers (four waves per SIMD
// instead of two): the ViT's 2496 waves fit the machine in one round, at
// most three per SIMD. Keys past the sequence read K and V as 0 (buffer
// range checks) and get probability 0. Workgroups of one (batch, head)
// share its K and V: the XCD-aware order puts all its query blocks on one
// XCD (one L2) when batch x heads % 8 == 0.
//
// Numerics: fp32 MFMA accumulation for both products (the reference sums in
// double and rounds once), the softmax in the running-maximum form with
// hardware exp2 (the reference takes exp against the row's final maximum);
// within the 1e-4 parity bar of the reference rows.

#include "common.hpp"
#include "../../include/nert_hip.h"

#include <string>

namespace nert_hip {
namespace {

constexpr int kHeadDim = 64;
constexpr int kQueries = 16;   // queries per workgroup: one 16x16 MFMA block

struct AttnArgs {
    const float* q;
    const float* k;
    const float* v;
    float* out;
    int32_t seq;
    int32_t heads;
    int32_t key_blocks;  // ceil(seq / 16)
    int32_t q_blocks;    // ceil(seq / 16)
    int32_t xcd;         // 1: batch * heads % 8 == 0, XCD-aware order
    int32_t in_b, in_t, in_h;    // Q/K/V strides (floats): batch, token, head
    int32_t out_b, out_t, out_h; // output strides (floats)
    float scale;
};

// Any sequence length, one wave per (batch, head, block of 16 queries),
// streaming over 16-key blocks with the running-maximum form of the softmax,
// on the 16x16x4 fp32 MFMA (lane l = 16 g + n: operand row/column n, K slice
// g; result rows 4 g .. 4 g + 3 of column n). Per key block:
//   S^T = K Q^T in 16 steps; step s takes dims 16 g + s from lane group g,
//   so lane (n, g) loads dims 16 g .. 16 g + 15 of its key row (K) and query
//   row (Q) as four 16-byte loads, and ends with the scores of query n for
//   keys 4 g .. 4 g + 3 of the block;
//   O^T += V^T P^T in 4 steps per 16-dim block; step t takes key 4 g + t
//   from lane group g, which is exactly the probability the lane already
//   holds (its score r = t), so no data moves between lanes; V rows come in
//   as 4-byte loads, dims 16 b + n.
// The block maximum of query n is its lane's 4 scores and two shuffles
// (lanes n, n + 16, n + 32, n + 48), and every output accumulator of a lane
// belongs to its query, so the rescale by exp(m_old - m_new) is lane-local.
// The next block's K and V are loaded before the current block's 32 MFMAs.
// K and V are read with buffer loads whose range check returns 0 past the
// last key (the whole byte offset in the VGPR offset); only the last,
// partial block masks scores. The exponentials are the hardware exp2 of
// scores pre-multiplied by scale * log2 e (relative error a few 1e-6 at the
// score ranges here, against the separate rows' expf of the rounded scaled
// score); the total is kept per lane in double and the four lanes of a
// query combined at the end; outputs are divided once.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t AttnRsrc(const float* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             static_cast<int>(0x00020000)); // raw dword buffer (gfx9 family)
}

__global__ __launch_bounds__(64, 4) void AttentionFlashKernel(AttnArgs a) {
    const int lane = threadIdx.x;
    const int g = lane >> 4;
    const int n = lane & 15;
    int bh;
    int qb;
    if (a.xcd) {
        const int j = static_cast<int>(blockIdx.x) / 8;
        bh = static_cast<int>(blockIdx.x) % 8 + 8 * (j / a.q_blocks);
        qb = j % a.q_blocks;
    } else {
        bh = static_cast<int>(blockIdx.x) / a.q_blocks;
        qb = static_cast<int>(blockIdx.x) % a.q_blocks;
    }
    const int b = bh / a.heads;
    const int h = bh - b * a.heads;
    const int64_t in_base = static_cast<int64_t>(b) * a.in_b + static_cast<int64_t>(h) * a.in_h;
    const int last = a.seq - 1;
    // Bytes of one (batch, head) slice up to its last key's last dim.
    const uint32_t slice = static_cast<uint32_t>((static_cast<int64_t>(last) * a.in_t + 64) * 4);
    const __amdgpu_buffer_rsrc_t kr = AttnRsrc(a.k + in_base, slice);
    const __amdgpu_buffer_rsrc_t vr = AttnRsrc(a.v + in_base, slice);
    const uint32_t row_bytes = static_cast<uint32_t>(a.in_t) * 4;

    // Q: query qb * 16 + n (the last one for queries past the sequence,
    // whose outputs are not stored), dims 16 g .. 16 g + 15.
    float qf[16];
    {
        const float* row =
            a.q + in_base + static_cast<int64_t>(min(qb * kQueries + n, last)) * a.in_t + 16 * g;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const nert_floatx4 x = *reinterpret_cast<const nert_floatx4*>(row + 4 * t);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                qf[4 * t + i] = x[i];
            }
        }
    }
    // K: row kb * 16 + n, dims 16 g ..; V: rows kb * 16 + 4 g + t, dims
    // 16 d + n. Rows past the sequence read as 0. The whole byte offset goes
    // in the VGPR offset (soffset stays 0): the range check of a raw buffer
    // load covers the VGPR offset and the instruction offset, not the scalar
    // offset.
    const uint32_t k_lane = static_cast<uint32_t>(n) * row_bytes + 64u * g;
    const uint32_t v_lane = static_cast<uint32_t>(4 * g) * row_bytes + 4u * n;
    const auto load_k = [&](int kb, float* kf) {
        const uint32_t kv = k_lane + static_cast<uint32_t>(kb) * 16u * row_bytes;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const nert_floatx4 x = __builtin_bit_cast(
                nert_floatx4, __builtin_amdgcn_raw_buffer_load_b128(kr, static_cast<int>(kv + 16u * t), 0, 0));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kf[4 * t + i] = x[i];
            }
        }
    };
    const auto load_v = [&](int kb, float* vf) {
        const uint32_t vv = v_lane + static_cast<uint32_t>(kb) * 16u * row_bytes;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                vf[4 * d + t] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(
                               vr, static_cast<int>(vv + static_cast<uint32_t>(t) * row_bytes + 64u * d), 0, 0));
            }
        }
    };
    const auto scores = [&](const float* kf) {
        nert_floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[t], qf[t], acc, 0, 0, 0);
        }
        return acc;
    };
    // Software pipeline: block kb + 1's score MFMAs are issued before block
    // kb's softmax, which they do not depend on, so the matrix pipe works
    // while the wave runs the softmax; K runs two blocks ahead, V one.
    const int blocks = a.key_blocks;
    float kf[16];
    float vf[16];
    load_k(0, kf);
    load_v(0, vf);
    nert_floatx4 s_next = scores(kf);
    load_k(min(1, blocks - 1), kf);
    nert_floatx4 o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            o[d][r] = 0.0f;
        }
    }
    constexpr float kLog2e = 1.4426950408889634f;
    const float scale2 = a.scale * kLog2e; // scores in log2 units
    float m = -__builtin_huge_valf();       // running maximum (log2 units)
    double total = 0.0;
    const int full = a.seq / 16; // blocks with no key past the sequence
    for (int kb = 0; kb < blocks; ++kb) {
        nert_floatx4 s = s_next;
        // kf holds block kb + 1's keys (loaded last iteration): its scores
        // go in now, then block kb + 2's keys and block kb + 1's values load.
        s_next = scores(kf);
        float kn[16];
        float vn[16];
        load_k(min(kb + 2, blocks - 1), kn);
        load_v(min(kb + 1, blocks - 1), vn);
        // Scores in log2 units (scale * log2 e in one multiply) for exp2.
        if (kb < full) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[r] *= scale2;
            }
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = kb * 16 + 4 * g + r;
                s[r] = key < a.seq ? s[r] * scale2 : -__builtin_huge_valf();
            }
        }
        float bm = m;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            bm = s[r] > bm ? s[r] : bm;
        }
        {
            float o2 = __shfl_xor(bm, 16, 64);
            bm = o2 > bm ? o2 : bm;
            o2 = __shfl_xor(bm, 32, 64);
            bm = o2 > bm ? o2 : bm;
        }
        // Key 0 opens the scan (block 0): a NaN there stays the maximum, as
        // the reference's peak rule keeps a NaN first element.
        if (kb == 0) {
            const float first = __shfl(s[0], n, 64);
            if (first != first) {
                bm = first;
            }
        }
        const float alpha = __builtin_amdgcn_exp2f(m - bm); // 0 on the first block (m = -inf)
        m = bm;
        float part = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s[r] = __builtin_amdgcn_exp2f(s[r] - m);
            part += s[r];
        }
        total = total * static_cast<double>(alpha) + static_cast<double>(part);
        // Once the maxima settle the factor is 1 in every lane: skip the
        // multiplies then (a wave-uniform test).
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    o[d][r] *= alpha;
                }
            }
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[4 * d + t], s[t], o[d], 0, 0, 0);
            }
        }
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            kf[t] = kn[t];
            vf[t] = vn[t];
        }
    }
    total += __shfl_xor(total, 16, 64);
    total += __shfl_xor(total, 32, 64);
    const float inv = static_cast<float>(1.0 / total);
    // o[d][r] = O[query n][dim 16 d + 4 g + r]: one 16-byte store per block.
    const int query = qb * kQueries + n;
    if (query < a.seq) {
        float* op = a.out + static_cast<int64_t>(b) * a.out_b + static_cast<int64_t>(h) * a.out_h +
                    static_cast<int64_t>(query) * a.out_t + 4 * g;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            nert_floatx4 x;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                x[r] = o[d][r] * inv;
            }
            *reinterpret_cast<nert_floatx4*>(op + 16 * d) = x;
        }
    }
}

} // namespace
} // namespace nert_hip

using namespace nert_hip;

extern "C" {

int nert_hip_attention_f32(const float* q, const float* k, const float* v, float* out, int64_t batch, int64_t heads,
                           int64_t seq, int64_t head_dim, const int64_t* in_strides, const int64_t* out_strides,
                           float scale, void* stream) {
    return Guard([&] {
        if (batch < 0 || heads < 0 || seq < 0) {
            throw Error("attention: negative extent");
        }
        if (batch * heads * seq == 0) {
            return;
        }
        if (head_dim != kHeadDim) {
            throw Error("attention: head_dim must be " + std::to_string(kHeadDim));
        }
        if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || in_strides == nullptr ||
            out_strides == nullptr) {
            throw Error("attention: null pointer");
        }
        for (int i = 0; i < 3; ++i) {
            if (in_strides[i] < 0 || out_strides[i] < 0) {
                throw Error("attention: negative stride");
            }
        }
        // 16-byte Q/K loads and output stores: 4-float aligned rows.
        const auto aligned = [](const float* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
        if (!aligned(q) || !aligned(k) || !aligned(out) || in_strides[0] % 4 != 0 || in_strides[1] % 4 != 0 ||
            in_strides[2] % 4 != 0 || out_strides[0] % 4 != 0 || out_strides[1] % 4 != 0 || out_strides[2] % 4 != 0) {
            throw Error("attention: Q, K and output rows must be 16-byte aligned");
        }
        // Keys past the sequence must fall beyond a (batch, head) slice's last
        // row (the loads' range check reads them as 0): tokens at least a
        // head's width apart, and the byte offsets of the last key block's
        // rows (up to 15 rows past the sequence) under 2^32, so no offset
        // wraps back into the slice.
        if (in_strides[1] < head_dim) {
            throw Error("attention: token stride shorter than head_dim");
        }
        if ((seq + 32) * in_strides[1] + head_dim >= (int64_t{1} << 30)) {
            throw Error("attention: a (batch, head) slice spans 2^32 bytes or more");
        }
        // Largest element offsets must fit the kernel's 32-bit strides.
        const int64_t in_last = (batch - 1) * in_strides[0] + (seq - 1) * in_strides[1] + (heads - 1) * in_strides[2] +
                                head_dim - 1;
        const int64_t out_last = (batch - 1) * out_strides[0] + (seq - 1) * out_strides[1] +
                                 (heads - 1) * out_strides[2] + head_dim - 1;
        const int64_t lim = int64_t{1} << 31;
        if (in_last >= lim || out_last >= lim || in_strides[0] >= lim || in_strides[1] >= lim ||
            in_strides[2] >= lim || out_strides[0] >= lim || out_strides[1] >= lim || out_strides[2] >= lim) {
            throw Error("attention: tensors beyond 2^31 elements");
        }
        const int64_t blocks = (seq + kQueries - 1) / kQueries;
        const int64_t groups = batch * heads * blocks;
        if (groups >= lim) {
            throw Error("attention: too many workgroups");
        }
        AttnArgs a{};
        a.q = q;
        a.k = k;
        a.v = v;
        a.out = out;
        a.seq = static_cast<int32_t>(seq);
        a.heads = static_cast<int32_t>(heads);
        a.key_blocks = static_cast<int32_t>(blocks);
        a.q_blocks = static_cast<int32_t>(blocks);
        a.xcd = (batch * heads) % 8 == 0 ? 1 : 0;
        a.in_b = static_cast<int32_t>(in_strides[0]);
        a.in_t = static_cast<int32_t>(in_strides[1]);
        a.in_h = static_cast<int32_t>(in_strides[2]);
        a.out_b = static_cast<int32_t>(out_strides[0]);
        a.out_t = static_cast<int32_t>(out_strides[1]);
        a.out_h = static_cast<int32_t>(out_strides[2]);
        a.scale = scale;
        AttentionFlashKernel<<<static_cast<unsigned>(groups), 64, 0, StreamOr(stream)>>>(a);
        CheckLaunch("attention launch");
    });
}

} // extern "C"
