#pragma once
// Internal launch interface of the MFMA GEMM engine (gemm.hip), shared by the
// rows that reduce to a plain or batched GEMM (Gemm, MatMul, pointwise Conv).

#include "common.hpp"

namespace nert_hip {

// Y[b](m, n) = alpha * sum_k A[b](m, k) * B[b](k, n) + beta * bias(m, n)
struct GemmArgs {
    const float* a;
    const float* b;
    float* y;
    const float* bias;
    int64_t m, n, k;
    int64_t a_sm, a_sk; // A(m,k) = a[m*a_sm + k*a_sk]; one of the two is 1
    int64_t b_sk, b_sn; // B(k,n) = b[k*b_sk + n*b_sn]; one of the two is 1
    int64_t bias_sm, bias_sn; // bias(m,n) = bias[m*bias_sm + n*bias_sn]
    float alpha, beta;
    int has_bias;
    int batch_rank; // up to 4 broadcast batch axes; Y batches are dense (m*n apart)
    int64_t bdims[4];
    int64_t a_bs[4];
    int64_t b_bs[4];
    int64_t k_per_split; // set by LaunchGemm
    float* partial;      // set by LaunchGemm: split-K parts for the reduce kernels, or null
    // Set by LaunchGemm instead of `partial` when the split tiles are
    // finished inside the kernel (FinishSplitTile): per-tile counters and
    // slots [batch * tiles + tile][split][BM * BN].
    uint32_t* counters;
    float* split_slots;
    // Optional activation after the bias (fused MatMul rows): act 1 is the
    // erf Gelu chain y -> y * (erf(y / act_div) + act_add) * act_mul.
    int act;
    float act_div, act_add, act_mul;
    // Output layout (one batch only): 0, Y(m, n) at y[m * n_total + n]; G > 0
    // (a multiple of 4 dividing n), the columns form groups of G stored as
    // [n / G][m][n % G], e.g. a conv's NCHW output when n runs over (image,
    // pixel) and G is the pixels per image.
    int64_t y_group;
    // B read in place from the input of a convolution whose windows tile it
    // exactly (stride = kernel, no padding) when patch.x is set (one batch,
    // A K-contiguous): B(k, n) = x[img][c][oh * kh + r][ow * kw + q] for
    // n = (img * out_h + oh) * out_w + ow and k = (c * kh + r) * kw + q, with
    // kw a multiple of 4 and x 16-byte aligned (runs of 4 k are 16 bytes).
    struct PatchB {
        const float* x;
        int32_t c, kh, kw, in_h, in_w, out_h, out_w;
        FastDiv div_khkw;  // by kh * kw
        FastDiv div_kw;    // by kw
        FastDiv div_plane; // by out_h * out_w
        FastDiv div_ow;    // by out_w
    } patch;
};

// Offset of output (r, c) under the layout above.
__device__ __forceinline__ int64_t GemmOutIndex(const GemmArgs& p, int64_t r, int64_t c) {
    if (p.y_group > 0) {
        const int64_t g = c / p.y_group;
        return (g * p.m + r) * p.y_group + (c - g * p.y_group);
    }
    return r * p.n + c;
}

void LaunchGemm(GemmArgs p, int64_t batches, hipStream_t stream);

} // namespace nert_hip
