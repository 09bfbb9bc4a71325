// Fused scaled-dot-product attention over packed Q/K/V: the MatMul(Q, K^T),
// Mul by a scalar, Softmax(last axis) and MatMul(P, V) rows of a transformer
// encoder in one kernel, reading Q, K and V where the QKV projection left
// them and writing the heads straight into the [batch, token, heads x dim]
// layout the output projection reads. It backs the runner's FusedAttention
// row; the reference computes the same result with those four rows plus the
// Reshape/Transpose/Split/Squeeze copies around them
// (src/kernels/mat_mul.cpp, mul.cpp, softmax.cpp, transpose.cpp, split.cpp).
//
// One wave per (batch, head, block of 32 queries) streams over the keys in
// blocks of 32 with the running-maximum form of the softmax (the kernel's
// comment has the lane layout): scores, probabilities and the output block
// stay in registers, with no LDS and no barrier. Q and K fragments are
// 16-byte loads: lane half h holds dims 8j + 4h .. 8j + 4h + 3 of its row,
// so one load feeds four MFMA steps (the same pairing for both operands, so
// the sum over the 64 dims is the dot product). Keys past the sequence read
// K and V as 0 (buffer range checks) and get probability 0. Workgroups of
// one (batch, head) share its K and V: the XCD-aware order puts all its
// query blocks on one XCD (one L2) when batch x heads % 8 == 0.
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
constexpr int kQueries = 32;   // queries per workgroup: one MFMA row block

struct AttnArgs {
    const float* q;
    const float* k;
    const float* v;
    float* out;
    int32_t seq;
    int32_t heads;
    int32_t key_blocks;  // ceil(seq / 32)
    int32_t q_blocks;    // ceil(seq / 32)
    int32_t xcd;         // 1: batch * heads % 8 == 0, XCD-aware order
    int32_t in_b, in_t, in_h;    // Q/K/V strides (floats): batch, token, head
    int32_t out_b, out_t, out_h; // output strides (floats)
    float scale;
};

// Any sequence length, one wave per (batch, head, block of 32 queries),
// streaming over 32-key blocks with the running-maximum form of the softmax:
// per block, S^T = K Q^T (A = K rows, B = Q^T), so lane (c, h) holds query
// c's scores for keys 8 (e / 4) + 4 h + e % 4 of the block; the block
// maximum is the lane's own 16 values and one shuffle with lane c + 32; the
// running output is rescaled by exp(m_old - m_new) and the block's
// probabilities accumulate into O^T = V^T P^T, whose B operand is exactly
// the probabilities the lane holds (lane half h supplies keys 8 j + 4 h + qq
// at MFMA step (j, qq)) and whose accumulators all belong to query c, so the
// rescale needs no data from other lanes. The next block's K and V are
// loaded before the current block's 64 MFMAs. K and V are read with buffer
// loads whose range check returns 0 past the last key (no clamped addresses,
// no selects); only the last, partial block masks scores. The exponentials
// are the hardware exp2 of scores pre-multiplied by scale * log2 e (relative
// error a few 1e-6 at the score ranges here, against the separate rows'
// expf of the rounded scaled score); the total is kept per lane in double
// and the halves combined at the end; outputs are divided once.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t AttnRsrc(const float* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             static_cast<int>(0x00020000)); // raw dword buffer (gfx9 family)
}

__global__ __launch_bounds__(64, 2) void AttentionFlashKernel(AttnArgs a) {
    const int lane = threadIdx.x;
    const int half = lane >> 5;
    const int c = lane & 31;
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

    nert_floatx4 qf[8];
    {
        const float* row = a.q + in_base + static_cast<int64_t>(min(qb * kQueries + c, last)) * a.in_t + 4 * half;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            qf[j] = *reinterpret_cast<const nert_floatx4*>(row + 8 * j);
        }
    }
    // K: row kb * 32 + c, dims 8 j + 4 h ..; V: rows kb * 32 + 4 h + 8 (e / 4)
    // + e % 4, dims c and 32 + c. Rows past the sequence read as 0.
    const uint32_t k_lane = static_cast<uint32_t>(c) * row_bytes + 16u * half;
    const uint32_t v_lane = static_cast<uint32_t>(4 * half) * row_bytes + 4u * c;
    // The whole byte offset goes in the VGPR offset (soffset stays 0): the
    // range check of a raw buffer load covers the VGPR offset and the
    // instruction offset, not the scalar offset.
    const auto load = [&](int kb, nert_floatx4* kf, float* v0, float* v1) {
        const uint32_t blk = static_cast<uint32_t>(kb) * 32u * row_bytes;
        const uint32_t kv = k_lane + blk;
        const uint32_t vv = v_lane + blk;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            kf[j] = __builtin_bit_cast(nert_floatx4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         kr, static_cast<int>(kv + 32u * j), 0, 0));
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t off = vv + static_cast<uint32_t>(8 * (e >> 2) + (e & 3)) * row_bytes;
            v0[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vr, static_cast<int>(off), 0, 0));
            v1[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vr, static_cast<int>(off + 128u),
                                                                                   0, 0));
        }
    };
    nert_floatx4 kf[8];
    float v0[16];
    float v1[16];
    load(0, kf, v0, v1);
    nert_floatx16 o0;
    nert_floatx16 o1;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        o0[e] = 0.0f;
        o1[e] = 0.0f;
    }
    constexpr float kLog2e = 1.4426950408889634f;
    const float scale2 = a.scale * kLog2e; // scores in log2 units
    float m = -__builtin_huge_valf();       // running maximum (log2 units)
    double total = 0.0;
    const int blocks = a.key_blocks;
    const int full = a.seq / 32; // blocks with no key past the sequence
    for (int kb = 0; kb < blocks; ++kb) {
        nert_floatx4 kn[8];
        float n0[16];
        float n1[16];
        load(min(kb + 1, blocks - 1), kn, n0, n1);
        nert_floatx16 s;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            s[e] = 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[j][qq], qf[j][qq], s, 0, 0, 0);
            }
        }
        // Scores in log2 units (scale * log2 e in one multiply) for exp2.
        if (kb < full) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                s[e] *= scale2;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int key = kb * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
                s[e] = key < a.seq ? s[e] * scale2 : -__builtin_huge_valf();
            }
        }
        float bm = m;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            bm = s[e] > bm ? s[e] : bm;
        }
        {
            const float o = __shfl_xor(bm, 32, 64);
            bm = o > bm ? o : bm;
        }
        // Key 0 opens the scan (block 0): a NaN there stays the maximum, as
        // the reference's peak rule keeps a NaN first element.
        if (kb == 0) {
            const float first = __shfl(s[0], c, 64);
            if (first != first) {
                bm = first;
            }
        }
        const float alpha = __builtin_amdgcn_exp2f(m - bm); // 0 on the first block (m = -inf)
        m = bm;
        float part = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            s[e] = __builtin_amdgcn_exp2f(s[e] - m);
            part += s[e];
        }
        total = total * static_cast<double>(alpha) + static_cast<double>(part);
        // Once the maxima settle the factor is 1 in every lane: skip the
        // multiplies then (a wave-uniform test).
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                o0[e] *= alpha;
                o1[e] *= alpha;
            }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0[e], s[e], o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1[e], s[e], o1, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            kf[j] = kn[j];
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            v0[e] = n0[e];
            v1[e] = n1[e];
        }
    }
    total += __shfl_xor(total, 32, 64);
    const float inv = static_cast<float>(1.0 / total);
    // o0[e] = O[query c][dim 8 (e / 4) + 4 h + e % 4], o1 the same + 32:
    // four runs of four consecutive dims per block, 16-byte stores.
    const int query = qb * kQueries + c;
    if (query < a.seq) {
        float* op = a.out + static_cast<int64_t>(b) * a.out_b + static_cast<int64_t>(h) * a.out_h +
                    static_cast<int64_t>(query) * a.out_t + 4 * half;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            nert_floatx4 x0;
            nert_floatx4 x1;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x0[i] = o0[4 * j + i] * inv;
                x1[i] = o1[4 * j + i] * inv;
            }
            *reinterpret_cast<nert_floatx4*>(op + 8 * j) = x0;
            *reinterpret_cast<nert_floatx4*>(op + 32 + 8 * j) = x1;
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
        // rows (up to 31 rows past the sequence) under 2^32, so no offset
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
        const int64_t blocks = (seq + 31) / 32;
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
