// Einsum over one or two float32 operands, and ConvTranspose.
//
// Einsum: the host resolves the equation into per-label extents and strides
// (output labels, then summed labels in alphabetical order). A two-operand
// equation whose labels fall into the batched-GEMM classes -- batch labels
// (in both operands and the output), row labels (first operand and output),
// column labels (second operand and output), contracted labels (both
// operands, not the output) -- with each class mergeable into one strided
// index, and the output ordered [batch][rows][columns] (or columns before
// rows, which swaps the operands), runs on the MFMA GEMM engine with fp32
// accumulation. Every other equation (one operand, diagonals that do not
// merge, labels summed in one operand only, broadcast output labels,
// interleaved row/column labels) takes the exact path: one thread per output
// element walks the summed labels as an odometer, last label fastest,
// multiplying the operands in double and accumulating in double, so each
// output sums its terms in the same order as the reference's odometer over
// all labels (src/kernels/einsum.cpp:205-258) and rounds once.
//
// ConvTranspose: the reference scatters every input pixel into the output
// (src/kernels/conv_transpose.cpp:160-188). Here it is a GEMM plus a gather.
// Per (image, group), one batched MFMA GEMM forms
// Z[(m, kh, kw)][ih, iw] = sum_c W[c][m, kh, kw] * X[c][ih, iw]
// (the weights are read in place as the transposed operand), then each output
// element gathers the taps that land on it -- tap kh contributes when
// oh + pad - kh * dilation is a non-negative multiple of the stride inside
// the input -- adds the bias and is written once; no atomics. fp32 sums, as
// the reference's. Groups of fewer than 8 input channels, and problems whose
// Z would pass 2 GiB, keep the direct kernel: one thread per output gathering
// (channel, tap) pairs with double sums.

#include "common.hpp"
#include "gemm_engine.hpp"
#include "../../include/nert_hip.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace nert_hip {
namespace {

constexpr int kMaxLabels = 16;

struct EinsumArgs {
    int n_out;
    int n_sum;
    int two;
    int64_t out_size[kMaxLabels];
    int64_t out_sa[kMaxLabels];
    int64_t out_sb[kMaxLabels];
    int64_t sum_size[kMaxLabels];
    int64_t sum_sa[kMaxLabels];
    int64_t sum_sb[kMaxLabels];
    int64_t sum_total;
};

__global__ void EinsumKernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ y,
                             EinsumArgs e, int64_t n) {
#pragma clang fp contract(off)
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        int64_t rem = i;
        int64_t oa = 0;
        int64_t ob = 0;
        for (int d = e.n_out - 1; d >= 0; --d) {
            const int64_t c = rem % e.out_size[d];
            rem /= e.out_size[d];
            oa += c * e.out_sa[d];
            ob += c * e.out_sb[d];
        }
        int64_t coord[kMaxLabels];
        for (int d = 0; d < e.n_sum; ++d) {
            coord[d] = 0;
        }
        double acc = 0.0;
        for (int64_t step = 0; step < e.sum_total; ++step) {
            double prod = 1.0;
            prod = prod * static_cast<double>(a[oa]);
            if (e.two) {
                prod = prod * static_cast<double>(b[ob]);
            }
            acc += prod;
            for (int d = e.n_sum - 1; d >= 0; --d) {
                ++coord[d];
                oa += e.sum_sa[d];
                ob += e.sum_sb[d];
                if (coord[d] < e.sum_size[d]) {
                    break;
                }
                oa -= e.sum_sa[d] * e.sum_size[d];
                ob -= e.sum_sb[d] * e.sum_size[d];
                coord[d] = 0;
            }
        }
        y[i] = static_cast<float>(acc);
    }
}

struct ConvTArgs {
    int64_t batch, in_c, out_c, group, in_h, in_w, out_h, out_w, k_h, k_w;
    int64_t stride_h, stride_w, pad_h, pad_w, dil_h, dil_w;
};

__global__ void ConvTransposeKernel(const float* __restrict__ x, const float* __restrict__ w,
                                    const float* __restrict__ bias, float* __restrict__ y, ConvTArgs p, int64_t n) {
    const int64_t in_per_group = p.in_c / p.group;
    const int64_t out_per_group = p.out_c / p.group;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        const int64_t ow = i % p.out_w;
        const int64_t oh = (i / p.out_w) % p.out_h;
        const int64_t m = (i / (p.out_w * p.out_h)) % p.out_c;
        const int64_t b = i / (p.out_w * p.out_h * p.out_c);
        const int64_t g = m / out_per_group;
        const int64_t oc = m - g * out_per_group;
        double acc = 0.0;
        for (int64_t kh = 0; kh < p.k_h; ++kh) {
            const int64_t th = oh + p.pad_h - kh * p.dil_h;
            if (th < 0 || th % p.stride_h != 0) {
                continue;
            }
            const int64_t ih = th / p.stride_h;
            if (ih >= p.in_h) {
                continue;
            }
            for (int64_t kw = 0; kw < p.k_w; ++kw) {
                const int64_t tw = ow + p.pad_w - kw * p.dil_w;
                if (tw < 0 || tw % p.stride_w != 0) {
                    continue;
                }
                const int64_t iw = tw / p.stride_w;
                if (iw >= p.in_w) {
                    continue;
                }
                for (int64_t ic = 0; ic < in_per_group; ++ic) {
                    const int64_t c = g * in_per_group + ic;
                    const float xv = x[((b * p.in_c + c) * p.in_h + ih) * p.in_w + iw];
                    const float wv = w[((c * out_per_group + oc) * p.k_h + kh) * p.k_w + kw];
                    acc += static_cast<double>(xv) * static_cast<double>(wv);
                }
            }
        }
        const float init = bias != nullptr ? bias[m] : 0.0f;
        y[i] = static_cast<float>(static_cast<double>(init) + acc);
    }
}

struct Label {
    int64_t size, sa, sb;
};

// Merges labels (outer to inner) into one index of extent prod(size) whose
// stride in an operand is the innermost label's: each outer stride must equal
// the next inner one times its extent. `which` 0 checks the first operand's
// strides, 1 the second's.
bool Mergeable(const std::vector<Label>& g, int which) {
    for (size_t i = 0; i + 1 < g.size(); ++i) {
        const int64_t outer = which == 0 ? g[i].sa : g[i].sb;
        const int64_t inner = which == 0 ? g[i + 1].sa : g[i + 1].sb;
        if (outer != inner * g[i + 1].size) {
            return false;
        }
    }
    return true;
}

Label Merged(const std::vector<Label>& g) {
    Label m{1, 0, 0};
    for (const Label& l : g) {
        m.size *= l.size;
    }
    if (!g.empty()) {
        m.sa = g.back().sa;
        m.sb = g.back().sb;
    }
    return m;
}

// The batched-GEMM lowering; false when the equation does not fit it.
bool TryEinsumGemm(const float* a, const float* b, float* y, int n_out, const int64_t* out_size,
                   const int64_t* out_sa, const int64_t* out_sb, int n_sum, const int64_t* sum_size,
                   const int64_t* sum_sa, const int64_t* sum_sb, hipStream_t stream) {
    if (b == nullptr) {
        return false;
    }
    enum Kind { kBatch, kRow, kCol };
    std::vector<Label> batch, first, second;
    int first_kind = -1;
    bool in_second = false;
    for (int d = 0; d < n_out; ++d) {
        const Label l{out_size[d], out_sa[d], out_sb[d]};
        if (l.size == 1) {
            continue;
        }
        int kind;
        if (l.sa != 0 && l.sb != 0) {
            kind = kBatch;
        } else if (l.sa != 0) {
            kind = kRow;
        } else if (l.sb != 0) {
            kind = kCol;
        } else {
            return false; // output label present in neither operand
        }
        if (kind == kBatch) {
            if (first_kind >= 0) {
                return false; // batch labels must lead the output
            }
            batch.push_back(l);
            continue;
        }
        if (first_kind < 0) {
            first_kind = kind;
        }
        if (kind == first_kind) {
            if (in_second) {
                return false; // row and column labels interleave
            }
            first.push_back(l);
        } else {
            in_second = true;
            second.push_back(l);
        }
    }
    std::vector<Label> contracted;
    for (int d = 0; d < n_sum; ++d) {
        const Label l{sum_size[d], sum_sa[d], sum_sb[d]};
        if (l.size == 1) {
            continue;
        }
        if (l.sa == 0 || l.sb == 0) {
            return false; // summed in one operand only
        }
        contracted.push_back(l);
    }
    std::stable_sort(contracted.begin(), contracted.end(),
                     [](const Label& x, const Label& y) { return x.sa > y.sa; });
    // The GEMM's rows are the output's first non-batch group; when those are
    // the second operand's labels, the operands swap roles.
    const bool swap = first_kind == kCol;
    const std::vector<Label>& rows = first;
    const std::vector<Label>& cols = second;
    if (!Mergeable(rows, swap ? 1 : 0) || !Mergeable(cols, swap ? 0 : 1) || !Mergeable(contracted, 0) ||
        !Mergeable(contracted, 1)) {
        return false;
    }
    // Adjacent batch labels merge when both operands allow it; at most four remain.
    std::vector<std::vector<Label>> bgroups;
    for (const Label& l : batch) {
        if (!bgroups.empty()) {
            std::vector<Label> trial = bgroups.back();
            trial.push_back(l);
            if (Mergeable(trial, 0) && Mergeable(trial, 1)) {
                bgroups.back() = trial;
                continue;
            }
        }
        bgroups.push_back({l});
    }
    if (bgroups.size() > 4) {
        return false;
    }
    const Label m = Merged(rows);
    const Label n = Merged(cols);
    const Label k = Merged(contracted);
    GemmArgs p{};
    // Operand roles: A(m, k) from the rows' operand, B(k, n) from the other.
    p.a = swap ? b : a;
    p.b = swap ? a : b;
    p.y = y;
    p.m = m.size;
    p.n = n.size;
    p.k = k.size;
    p.a_sm = swap ? m.sb : m.sa;
    p.a_sk = swap ? k.sb : k.sa;
    p.b_sk = swap ? k.sa : k.sb;
    p.b_sn = swap ? n.sa : n.sb;
    // A unit extent has no stride of its own; give it the unit stride the
    // engine's layouts expect.
    if (p.m == 1 && p.a_sk != 1) {
        p.a_sm = 1;
    }
    if (p.k == 1) {
        if (p.a_sm != 1) {
            p.a_sk = 1;
        }
        if (p.b_sn != 1) {
            p.b_sk = 1;
        }
    }
    if (p.n == 1 && p.b_sk != 1) {
        p.b_sn = 1;
    }
    if ((p.a_sm != 1 && p.a_sk != 1) || (p.b_sk != 1 && p.b_sn != 1)) {
        return false;
    }
    p.alpha = 1.0f;
    p.beta = 0.0f;
    p.batch_rank = static_cast<int>(bgroups.size());
    int64_t batches = 1;
    for (size_t d = 0; d < bgroups.size(); ++d) {
        const Label l = Merged(bgroups[d]);
        p.bdims[d] = l.size;
        p.a_bs[d] = swap ? l.sb : l.sa;
        p.b_bs[d] = swap ? l.sa : l.sb;
        batches *= l.size;
    }
    if (batches > 65535) {
        return false;
    }
    // The lowered walk must span exactly the elements the label walk reads:
    // the largest offset into each operand agrees, so the GEMM stays inside
    // the operands whenever the equation's own strides do.
    int64_t reach_a = 0, reach_b = 0;
    for (int d = 0; d < n_out; ++d) {
        reach_a += (out_size[d] - 1) * out_sa[d];
        reach_b += (out_size[d] - 1) * out_sb[d];
    }
    for (int d = 0; d < n_sum; ++d) {
        reach_a += (sum_size[d] - 1) * sum_sa[d];
        reach_b += (sum_size[d] - 1) * sum_sb[d];
    }
    int64_t lowered_a = (p.m - 1) * p.a_sm + (p.k - 1) * p.a_sk;
    int64_t lowered_b = (p.k - 1) * p.b_sk + (p.n - 1) * p.b_sn;
    for (int d = 0; d < p.batch_rank; ++d) {
        lowered_a += (p.bdims[d] - 1) * p.a_bs[d];
        lowered_b += (p.bdims[d] - 1) * p.b_bs[d];
    }
    if (lowered_a != (swap ? reach_b : reach_a) || lowered_b != (swap ? reach_a : reach_b)) {
        return false;
    }
    LaunchGemm(p, batches, stream);
    return true;
}

// Output element i (row-major over [batch, out_c, out_h, out_w]) sums the
// Z entries of its valid taps. With unit dilation the valid kh are
// kh0, kh0 + stride, ... where kh0 = (oh + pad) mod stride.
__global__ __launch_bounds__(256) void ConvTransposeGatherKernel(const float* __restrict__ z,
                                                                 const float* __restrict__ bias, float* __restrict__ y,
                                                                 ConvTArgs p, FastDiv fw, FastDiv fh, FastDiv fc,
                                                                 uint32_t n) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) {
        return;
    }
    uint32_t ow, oh, m;
    uint32_t t = DivMod(fw, i, ow);
    t = DivMod(fh, t, oh);
    const uint32_t b = DivMod(fc, t, m);
    const int mg = static_cast<int>(p.out_c / p.group);
    const int g = static_cast<int>(m) / mg;
    const int ml = static_cast<int>(m) - g * mg;
    const int64_t plane = p.in_h * p.in_w;
    const float* zb = z + ((static_cast<int64_t>(b) * p.group + g) * mg + ml) * (p.k_h * p.k_w) * plane;
    const int sh = static_cast<int>(p.stride_h), sw = static_cast<int>(p.stride_w);
    const int dh = static_cast<int>(p.dil_h), dw = static_cast<int>(p.dil_w);
    const int kh_n = static_cast<int>(p.k_h), kw_n = static_cast<int>(p.k_w);
    const int ih_n = static_cast<int>(p.in_h), iw_n = static_cast<int>(p.in_w);
    const int th0 = static_cast<int>(oh) + static_cast<int>(p.pad_h);
    const int tw0 = static_cast<int>(ow) + static_cast<int>(p.pad_w);
    const int kh_first = dh == 1 ? (th0 % sh) : 0;
    const int kh_step = dh == 1 ? sh : 1;
    const int kw_first = dw == 1 ? (tw0 % sw) : 0;
    const int kw_step = dw == 1 ? sw : 1;
    float acc = 0.0f;
    for (int kh = kh_first; kh < kh_n; kh += kh_step) {
        const int th = th0 - kh * dh;
        if (th < 0) {
            break;
        }
        if (th % sh != 0) {
            continue;
        }
        const int ih = th / sh;
        if (ih >= ih_n) {
            continue;
        }
        for (int kw = kw_first; kw < kw_n; kw += kw_step) {
            const int tw = tw0 - kw * dw;
            if (tw < 0) {
                break;
            }
            if (tw % sw != 0) {
                continue;
            }
            const int iw = tw / sw;
            if (iw >= iw_n) {
                continue;
            }
            acc += zb[(kh * kw_n + kw) * plane + ih * iw_n + iw];
        }
    }
    y[i] = bias != nullptr ? bias[m] + acc : acc;
}

bool TryConvTransposeGemm(const float* x, const float* w, const float* bias, float* y, const ConvTArgs& p,
                          hipStream_t stream) {
    const int64_t cg = p.in_c / p.group;
    const int64_t mg = p.out_c / p.group;
    const int64_t rows = mg * p.k_h * p.k_w;
    const int64_t plane = p.in_h * p.in_w;
    const int64_t batches = p.batch * p.group;
    const int64_t outputs = p.batch * p.out_c * p.out_h * p.out_w;
    const int64_t z_bytes = batches * rows * plane * static_cast<int64_t>(sizeof(float));
    if (cg < 8 || batches > 65535 || z_bytes > (int64_t{1} << 31) || outputs >= (int64_t{1} << 31) ||
        plane <= 0 || rows <= 0 || p.pad_h < 0 || p.pad_w < 0 || p.dil_h < 1 || p.dil_w < 1) {
        return false;
    }
    float* z = static_cast<float*>(Workspace(z_bytes, stream, 1));
    GemmArgs g{};
    g.a = w; // A(r, c) = W[g*cg + c][r]
    g.b = x; // B(c, q) = X[b][g*cg + c][q]
    g.y = z;
    g.m = rows;
    g.n = plane;
    g.k = cg;
    g.a_sm = 1;
    g.a_sk = rows;
    g.b_sk = plane;
    g.b_sn = 1;
    g.alpha = 1.0f;
    g.beta = 0.0f;
    g.batch_rank = 2;
    g.bdims[0] = p.batch;
    g.a_bs[0] = 0;
    g.b_bs[0] = p.in_c * plane;
    g.bdims[1] = p.group;
    g.a_bs[1] = cg * rows;
    g.b_bs[1] = cg * plane;
    LaunchGemm(g, batches, stream);
    ConvTransposeGatherKernel<<<GridFor(outputs, 256, outputs), 256, 0, stream>>>(
        z, bias, y, p, FastDiv::Make(static_cast<uint32_t>(p.out_w)), FastDiv::Make(static_cast<uint32_t>(p.out_h)),
        FastDiv::Make(static_cast<uint32_t>(p.out_c)), static_cast<uint32_t>(outputs));
    CheckLaunch("conv_transpose gather launch");
    return true;
}

} // namespace
} // namespace nert_hip

using namespace nert_hip;

extern "C" {

int nert_hip_einsum_f32(const float* a, const float* b, float* y, int n_out, const int64_t* out_size,
                        const int64_t* out_stride_a, const int64_t* out_stride_b, int n_sum, const int64_t* sum_size,
                        const int64_t* sum_stride_a, const int64_t* sum_stride_b, void* stream) {
    return Guard([&] {
        if (n_out < 0 || n_out > kMaxLabels || n_sum < 0 || n_sum > kMaxLabels) {
            throw Error("einsum: at most 16 output and 16 summed labels");
        }
        EinsumArgs e{};
        e.n_out = n_out;
        e.n_sum = n_sum;
        e.two = b != nullptr ? 1 : 0;
        int64_t n = 1;
        for (int d = 0; d < n_out; ++d) {
            e.out_size[d] = out_size[d];
            e.out_sa[d] = out_stride_a[d];
            e.out_sb[d] = b != nullptr ? out_stride_b[d] : 0;
            n *= out_size[d];
        }
        e.sum_total = 1;
        for (int d = 0; d < n_sum; ++d) {
            e.sum_size[d] = sum_size[d];
            e.sum_sa[d] = sum_stride_a[d];
            e.sum_sb[d] = b != nullptr ? sum_stride_b[d] : 0;
            e.sum_total *= sum_size[d];
        }
        if (n <= 0) {
            return;
        }
        const char* exact = std::getenv("NERT_HIP_EINSUM_EXACT");
        const bool force_exact = exact != nullptr && std::strcmp(exact, "1") == 0;
        if (!force_exact && TryEinsumGemm(a, b, y, n_out, out_size, out_stride_a, out_stride_b, n_sum, sum_size,
                                          sum_stride_a, sum_stride_b, StreamOr(stream))) {
            return;
        }
        EinsumKernel<<<GridFor(n, 256, 16384), 256, 0, StreamOr(stream)>>>(a, b != nullptr ? b : a, y, e, n);
        CheckLaunch("einsum launch");
    });
}

int nert_hip_conv_transpose_f32(const float* x, const float* w, const float* bias, float* y, const int64_t* geom,
                                void* stream) {
    return Guard([&] {
        ConvTArgs p{};
        int64_t* f = &p.batch;
        for (int i = 0; i < 16; ++i) {
            f[i] = geom[i];
        }
        if (p.group <= 0 || p.in_c % p.group != 0 || p.out_c % p.group != 0 || p.stride_h <= 0 || p.stride_w <= 0) {
            throw Error("conv_transpose: bad geometry");
        }
        const int64_t n = p.batch * p.out_c * p.out_h * p.out_w;
        if (n <= 0) {
            return;
        }
        const char* exact = std::getenv("NERT_HIP_CONVT_EXACT");
        const bool force_exact = exact != nullptr && std::strcmp(exact, "1") == 0;
        if (!force_exact && TryConvTransposeGemm(x, w, bias, y, p, StreamOr(stream))) {
            return;
        }
        ConvTransposeKernel<<<GridFor(n, 256, 16384), 256, 0, StreamOr(stream)>>>(x, w, bias, y, p, n);
        CheckLaunch("conv_transpose launch");
    });
}

} // extern "C"
