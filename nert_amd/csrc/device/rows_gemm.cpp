// Gemm, MatMul and Conv rows: host validation mirroring the reference CPU
// rows, then one MFMA launch (plus a split-K reduction for small grids).

#include "rows.hpp"

#include <algorithm>

namespace nert_hip {
namespace rows {

using namespace seam;

// Validation follows src/kernels/gemm.cpp:59-117.
void Gemm(const Node& node, const Views& inputs, const Views& outputs) {
    const std::string context = "Gemm (node '" + node.name + "')";
    if (inputs.size() < 2 || inputs.size() > 3 || outputs.size() != 1) {
        throw InferenceException(context + ": expected two or three inputs and one output");
    }
    const TensorView& a = inputs[0];
    const TensorView& b = inputs[1];
    const TensorView& out = outputs[0];
    const bool has_c = inputs.size() == 3;
    if (a.dtype != DataType::Float32 || b.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (has_c && inputs[2].dtype != DataType::Float32) {
        throw InferenceException(context + ": bias tensor must be float32");
    }
    if (a.dims.size() != 2 || b.dims.size() != 2) {
        throw InferenceException(context + ": A and B must be rank-2");
    }
    (void)ElementCount(a.dims, context);
    (void)ElementCount(b.dims, context);
    const int64_t trans_a = IntAttr(node, "transA", 0, "Gemm");
    const int64_t trans_b = IntAttr(node, "transB", 0, "Gemm");
    const float alpha = FloatAttr(node, "alpha", 1.0f, "Gemm");
    const float beta = FloatAttr(node, "beta", 1.0f, "Gemm");
    const int64_t m = trans_a == 0 ? a.dims[0] : a.dims[1];
    const int64_t k = trans_a == 0 ? a.dims[1] : a.dims[0];
    const int64_t bk = trans_b == 0 ? b.dims[0] : b.dims[1];
    const int64_t n = trans_b == 0 ? b.dims[1] : b.dims[0];
    if (k != bk) {
        throw InferenceException(context + ": contraction dimension mismatch");
    }
    if (out.dims != std::vector<int64_t>{m, n}) {
        throw InferenceException(context + ": output shape does not match the operands");
    }
    (void)ElementCount(out.dims, context);
    const float* bias = nullptr;
    int bias_rank = 0;
    if (has_c) {
        const TensorView& c = inputs[2];
        const bool rank_one = c.dims.size() == 1 && c.dims[0] == n;
        const bool rank_two = c.dims.size() == 2 && c.dims[0] == m && c.dims[1] == n;
        if (!rank_one && !rank_two) {
            throw InferenceException(context + ": bias shape must be [N] or [M,N]");
        }
        (void)ElementCount(c.dims, context);
        bias = static_cast<const float*>(c.data);
        bias_rank = static_cast<int>(c.dims.size());
    }
    if (a.data == nullptr || b.data == nullptr || out.data == nullptr || (has_c && bias == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    CheckStatus(nert_hip_gemm_f32(static_cast<const float*>(a.data), static_cast<const float*>(b.data), bias,
                                  static_cast<float*>(out.data), m, n, k, trans_a != 0 ? 1 : 0, trans_b != 0 ? 1 : 0,
                                  alpha, beta, bias_rank, Stream()),
                context);
    AfterRow(outputs, context);
}

namespace {

std::vector<int64_t> BroadcastBatch(const std::vector<int64_t>& a, const std::vector<int64_t>& b,
                                    const std::string& context) {
    const size_t rank = std::max(a.size(), b.size());
    std::vector<int64_t> out(rank, 1);
    for (size_t i = 0; i < rank; ++i) {
        const int64_t da = i < rank - a.size() ? 1 : a[i - (rank - a.size())];
        const int64_t db = i < rank - b.size() ? 1 : b[i - (rank - b.size())];
        if (da != db && da != 1 && db != 1) {
            throw InferenceException(context + ": batch dimensions are not broadcast-compatible");
        }
        out[i] = std::max(da, db);
    }
    return out;
}

// Per-output-batch-axis element strides of one operand's batch (0 where the
// operand broadcasts), in units of whole matrices times `mat`.
std::vector<int64_t> BatchStrides(const std::vector<int64_t>& in, const std::vector<int64_t>& out, int64_t mat) {
    std::vector<int64_t> strides(out.size(), 0);
    int64_t s = mat;
    for (size_t j = out.size(); j-- > 0;) {
        const size_t off = out.size() - in.size();
        if (j < off) {
            continue;
        }
        const int64_t d = in[j - off];
        strides[j] = d == 1 ? 0 : s;
        s *= d;
    }
    return strides;
}

} // namespace

namespace {

// The MatMul row's work, shared with FusedMatMul: `scale`, `bias` (or null)
// and the activation go to the GEMM epilogue. Validation follows
// src/kernels/mat_mul.cpp:79-139.
void MatMulCore(const std::string& context, const TensorView& a, const TensorView& b, const TensorView& out,
                const Views& outputs, const float* bias, float scale, int act, const float* act_params) {
    if (a.dtype != DataType::Float32 || b.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (a.dims.empty() || b.dims.empty()) {
        throw InferenceException(context + ": operands must have at least one dimension");
    }
    std::vector<int64_t> a_dims = a.dims;
    std::vector<int64_t> b_dims = b.dims;
    const bool a_promoted = a_dims.size() == 1;
    const bool b_promoted = b_dims.size() == 1;
    if (a_promoted) {
        a_dims.insert(a_dims.begin(), 1);
    }
    if (b_promoted) {
        b_dims.push_back(1);
    }
    (void)ElementCount(a_dims, context);
    (void)ElementCount(b_dims, context);
    const size_t a_rank = a_dims.size();
    const size_t b_rank = b_dims.size();
    const int64_t m = a_dims[a_rank - 2];
    const int64_t k = a_dims[a_rank - 1];
    const int64_t bk = b_dims[b_rank - 2];
    const int64_t n = b_dims[b_rank - 1];
    if (k != bk) {
        throw InferenceException(context + ": contraction dimension mismatch");
    }
    const std::vector<int64_t> batch_a(a_dims.begin(), a_dims.end() - 2);
    const std::vector<int64_t> batch_b(b_dims.begin(), b_dims.end() - 2);
    const std::vector<int64_t> batch_out = BroadcastBatch(batch_a, batch_b, context);
    std::vector<int64_t> full = batch_out;
    full.push_back(m);
    full.push_back(n);
    std::vector<int64_t> expected = full;
    if (a_promoted) {
        expected.erase(expected.begin() + static_cast<std::ptrdiff_t>(batch_out.size()));
    }
    if (b_promoted) {
        const size_t n_index = a_promoted ? batch_out.size() : batch_out.size() + 1;
        expected.erase(expected.begin() + static_cast<std::ptrdiff_t>(n_index));
    }
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the operands");
    }
    (void)ElementCount(full, context);
    if (a.data == nullptr || b.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }

    const auto* ap = static_cast<const float*>(a.data);
    const auto* bp = static_cast<const float*>(b.data);
    auto* yp = static_cast<float*>(out.data);
    std::vector<int64_t> a_strides = BatchStrides(batch_a, batch_out, m * k);
    std::vector<int64_t> b_strides = BatchStrides(batch_b, batch_out, k * n);
    std::vector<int64_t> dims = batch_out;

    // A dense A batch against one shared B is a single tall GEMM: fold the
    // batch into M (the ViT projections [16,197,768] x [768,N]).
    bool b_shared = true;
    for (int64_t s : b_strides) {
        b_shared = b_shared && s == 0;
    }
    bool a_dense = true;
    {
        int64_t expect = m * k;
        for (size_t j = dims.size(); j-- > 0;) {
            if (dims[j] == 1) {
                continue;
            }
            a_dense = a_dense && a_strides[j] == expect;
            expect *= dims[j];
        }
    }
    int64_t batches = Count(dims);
    if (b_shared && a_dense && batches > 1) {
        CheckStatus(nert_hip_matmul_fused_f32(ap, bp, bias, yp, m * batches, n, k, 0, nullptr, nullptr, nullptr, scale,
                                              act, act_params, Stream()),
                    context);
        AfterRow(outputs, context);
        return;
    }
    // Drop unit batch axes; merge neighbours both operands walk densely.
    std::vector<int64_t> cd, ca, cb;
    for (size_t j = 0; j < dims.size(); ++j) {
        if (dims[j] == 1) {
            continue;
        }
        if (!cd.empty() && ca.back() == a_strides[j] * dims[j] && cb.back() == b_strides[j] * dims[j]) {
            cd.back() *= dims[j];
            ca.back() = a_strides[j];
            cb.back() = b_strides[j];
            continue;
        }
        if (!cd.empty() && ca.back() == 0 && a_strides[j] == 0 && cb.back() == b_strides[j] * dims[j]) {
            cd.back() *= dims[j];
            cb.back() = b_strides[j];
            continue;
        }
        if (!cd.empty() && cb.back() == 0 && b_strides[j] == 0 && ca.back() == a_strides[j] * dims[j]) {
            cd.back() *= dims[j];
            ca.back() = a_strides[j];
            continue;
        }
        cd.push_back(dims[j]);
        ca.push_back(a_strides[j]);
        cb.push_back(b_strides[j]);
    }
    if (cd.size() > 4) {
        throw InferenceException(context + ": more than four non-mergeable batch axes");
    }
    CheckStatus(nert_hip_matmul_fused_f32(ap, bp, bias, yp, m, n, k, static_cast<int>(cd.size()), cd.data(), ca.data(),
                                          cb.data(), scale, act, act_params, Stream()),
                context);
    AfterRow(outputs, context);
}

} // namespace

void MatMul(const Node& node, const Views& inputs, const Views& outputs) {
    const std::string context = "MatMul (node '" + node.name + "')";
    if (inputs.size() != 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected two inputs and one output");
    }
    MatMulCore(context, inputs[0], inputs[1], outputs[0], outputs, nullptr, 1.0f, 0, nullptr);
}

// Not a reference row: the runner's fusion of MatMul -> [Mul by a scalar]
// -> [Add of a [N] bias] -> [Div, Erf, Add, Mul, Mul: the erf Gelu chain].
// Inputs A, B, optional bias [N]; attributes alpha (the scalar, default 1),
// activation "" or "Gelu" with gelu_div, gelu_add, gelu_mul (the chain's
// constants). The epilogue rounds each step like the separate rows, so the
// output is bit-identical to the unfused chain.
void FusedMatMul(const Node& node, const Views& inputs, const Views& outputs) {
    const std::string context = "FusedMatMul (node '" + node.name + "')";
    if (inputs.size() < 2 || inputs.size() > 3 || outputs.size() != 1) {
        throw InferenceException(context + ": expected two or three inputs and one output");
    }
    const TensorView& out = outputs[0];
    const float* bias = nullptr;
    if (inputs.size() == 3 && inputs[2].data != nullptr) {
        const TensorView& c = inputs[2];
        if (c.dtype != DataType::Float32 || c.dims.size() != 1 || out.dims.empty() || c.dims[0] != out.dims.back()) {
            throw InferenceException(context + ": bias must be float32 [N]");
        }
        bias = static_cast<const float*>(c.data);
    }
    const float alpha = FloatAttrC(node, "alpha", 1.0f, context);
    const std::string activation = StringAttr(node, "activation", "", "FusedMatMul");
    float params[3] = {0.0f, 0.0f, 0.0f};
    int act = 0;
    if (activation == "Gelu") {
        act = 1;
        params[0] = FloatAttrC(node, "gelu_div", 0.0f, context);
        params[1] = FloatAttrC(node, "gelu_add", 0.0f, context);
        params[2] = FloatAttrC(node, "gelu_mul", 0.0f, context);
    } else if (!activation.empty()) {
        throw InferenceException(context + ": unsupported activation '" + activation + "'");
    }
    MatMulCore(context, inputs[0], inputs[1], out, outputs, bias, alpha, act, params);
}

// Not a reference row: the runner's fusion of a transformer encoder's
// attention block. Input: the packed QKV projection [B, S, 3 * H * D]
// (token-major, the Reshape to [B, S, 3, H, D] it replaces); attributes heads
// (H) and scale (the Mul's scalar). Output [B, S, H * D]: the heads of
// Softmax(scale * Q K^T) V side by side, as the Transpose + Reshape after the
// second MatMul lays them out. The reference runs MatMul, Mul, Softmax and
// MatMul (src/kernels/mat_mul.cpp, mul.cpp, softmax.cpp) plus the copies
// that split Q, K and V apart; the values agree within the fp32 parity bar.
void FusedAttention(const Node& node, const Views& inputs, const Views& outputs) {
    const std::string context = "FusedAttention (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input (packed QKV) and one output");
    }
    const TensorView& qkv = inputs[0];
    const TensorView& out = outputs[0];
    if (qkv.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (qkv.dims.size() != 3 || out.dims.size() != 3 || out.dims[0] != qkv.dims[0] || out.dims[1] != qkv.dims[1]) {
        throw InferenceException(context + ": expected QKV [B, S, 3*H*D] and output [B, S, H*D]");
    }
    const int64_t heads = IntAttrC(node, "heads", 0, context);
    const float scale = FloatAttrC(node, "scale", 1.0f, context);
    const int64_t width = out.dims[2];
    if (heads <= 0 || width % heads != 0 || qkv.dims[2] != 3 * width) {
        throw InferenceException(context + ": QKV width must be 3 * heads * head_dim and the output heads * head_dim");
    }
    const int64_t batch = qkv.dims[0];
    const int64_t seq = qkv.dims[1];
    const int64_t head_dim = width / heads;
    (void)ElementCount(qkv.dims, context);
    if (batch * seq * width == 0) {
        AfterRow(outputs, context);
        return;
    }
    if (qkv.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    const float* base = static_cast<const float*>(qkv.data);
    const int64_t in_strides[3] = {seq * 3 * width, 3 * width, head_dim};
    const int64_t out_strides[3] = {seq * width, width, head_dim};
    CheckStatus(nert_hip_attention_f32(base, base + width, base + 2 * width, static_cast<float*>(out.data), batch,
                                       heads, seq, head_dim, in_strides, out_strides, scale, Stream()),
                context);
    AfterRow(outputs, context);
}

namespace {

// src/kernels/conv.cpp:78-119.
void ResolvePads(const std::string& context, const std::string& auto_pad, const std::vector<int64_t>& in_spatial,
                 const std::vector<int64_t>& kernel, const std::vector<int64_t>& dilations,
                 const std::vector<int64_t>& strides, const std::vector<int64_t>& pads_attr,
                 std::vector<int64_t>& pad_begin, std::vector<int64_t>& pad_end) {
    const size_t rank = in_spatial.size();
    pad_begin.assign(rank, 0);
    pad_end.assign(rank, 0);
    if (auto_pad == "VALID") {
        return;
    }
    if (auto_pad == "SAME_UPPER" || auto_pad == "SAME_LOWER") {
        for (size_t i = 0; i < rank; ++i) {
            const int64_t out = (in_spatial[i] + strides[i] - 1) / strides[i];
            const int64_t effective = dilations[i] * (kernel[i] - 1) + 1;
            const int64_t total = std::max<int64_t>(0, (out - 1) * strides[i] + effective - in_spatial[i]);
            if (auto_pad == "SAME_UPPER") {
                pad_begin[i] = total / 2;
                pad_end[i] = total - pad_begin[i];
            } else {
                pad_end[i] = total / 2;
                pad_begin[i] = total - pad_end[i];
            }
        }
        return;
    }
    if (pads_attr.empty()) {
        return;
    }
    if (pads_attr.size() != 2 * rank) {
        throw InferenceException(context + ": pads must have two entries per spatial dimension");
    }
    for (size_t i = 0; i < rank; ++i) {
        pad_begin[i] = pads_attr[i];
        pad_end[i] = pads_attr[rank + i];
    }
}

} // namespace

void ResolveWindowPads(const std::string& context, const std::string& auto_pad, const std::vector<int64_t>& in_spatial,
                       const std::vector<int64_t>& kernel, const std::vector<int64_t>& dilations,
                       const std::vector<int64_t>& strides, const std::vector<int64_t>& pads_attr,
                       std::vector<int64_t>& pad_begin, std::vector<int64_t>& pad_end) {
    ResolvePads(context, auto_pad, in_spatial, kernel, dilations, strides, pads_attr, pad_begin, pad_end);
}

int64_t WindowOutput(const std::string& context, int64_t in, int64_t kernel, int64_t dilation, int64_t pad_begin,
                     int64_t pad_end, int64_t stride, bool ceil_mode) {
    const int64_t effective = dilation * (kernel - 1) + 1;
    const int64_t numer = in + pad_begin + pad_end - effective;
    if (numer < 0) {
        throw InferenceException(context + ": window is larger than the padded input");
    }
    const int64_t out = (ceil_mode ? (numer + stride - 1) / stride : numer / stride) + 1;
    if (out <= 0) {
        throw InferenceException(context + ": computes a non-positive output dimension");
    }
    return out;
}

namespace {

// The Conv row's work, shared with FusedConv: `residual` (or null) is added
// and the activation (0 none, 1 Relu, 2 SiLU) applied in the kernel epilogue
// when the fused row asks for them.
struct ConvCall {
    nert_conv_desc d;
    const float* bias;
    const float* residual;
};

// The checks of the Conv row and the kernel descriptor of its convolution.
ConvCall CheckConv(const Node& node, const std::string& context, const Views& inputs, bool has_bias,
                   const TensorView* residual, const Views& outputs) {
    const TensorView& x = inputs[0];
    const TensorView& w = inputs[1];
    const TensorView& out = outputs[0];
    if (x.dtype != DataType::Float32 || w.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (has_bias && inputs[2].dtype != DataType::Float32) {
        throw InferenceException(context + ": bias tensor must be float32");
    }
    const size_t rank = x.dims.size();
    if (rank < 3 || rank > 5) {
        throw InferenceException(context + ": input must be rank 3, 4, or 5 (1-D, 2-D, or 3-D convolution)");
    }
    if (w.dims.size() != rank) {
        throw InferenceException(context + ": weight rank must match the input rank");
    }
    (void)ElementCount(x.dims, context);
    (void)ElementCount(w.dims, context);
    (void)ElementCount(out.dims, context);
    const size_t spatial = rank - 2;
    const int64_t batch = x.dims[0];
    const int64_t in_channels = x.dims[1];
    const int64_t out_channels = w.dims[0];
    const int64_t group = IntAttr(node, "group", 1, "Conv");
    if (group <= 0) {
        throw InferenceException(context + ": group must be positive");
    }
    if (in_channels % group != 0) {
        throw InferenceException(context + ": input channels are not divisible by group");
    }
    if (w.dims[1] != in_channels / group) {
        throw InferenceException(context + ": weight channel dimension does not match input/group");
    }
    if (out_channels % group != 0) {
        throw InferenceException(context + ": output channels are not divisible by group");
    }
    std::vector<int64_t> strides = IntsAttr(node, "strides", "Conv");
    std::vector<int64_t> dilations = IntsAttr(node, "dilations", "Conv");
    if (strides.empty()) {
        strides.assign(spatial, 1);
    }
    if (dilations.empty()) {
        dilations.assign(spatial, 1);
    }
    if (strides.size() != spatial || dilations.size() != spatial) {
        throw InferenceException(context + ": stride and dilation must have one entry per spatial dimension");
    }
    const std::vector<int64_t> in_spatial(x.dims.begin() + 2, x.dims.end());
    const std::vector<int64_t> kernel(w.dims.begin() + 2, w.dims.end());
    for (size_t i = 0; i < spatial; ++i) {
        if (strides[i] <= 0 || dilations[i] <= 0) {
            throw InferenceException(context + ": stride and dilation must be positive");
        }
        if (kernel[i] <= 0) {
            throw InferenceException(context + ": kernel dimensions must be positive");
        }
    }
    std::vector<int64_t> pad_begin;
    std::vector<int64_t> pad_end;
    ResolvePads(context, StringAttr(node, "auto_pad", "NOTSET", "Conv"), in_spatial, kernel, dilations, strides,
                IntsAttr(node, "pads", "Conv"), pad_begin, pad_end);
    std::vector<int64_t> expected = {batch, out_channels};
    for (size_t i = 0; i < spatial; ++i) {
        expected.push_back(
            WindowOutput(context, in_spatial[i], kernel[i], dilations[i], pad_begin[i], pad_end[i], strides[i], false));
    }
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the convolution");
    }
    const float* bias = nullptr;
    if (has_bias) {
        const std::vector<int64_t>& bias_dims = inputs[2].dims;
        if (bias_dims.size() != 1 || bias_dims[0] != out_channels) {
            throw InferenceException(context + ": bias must be rank-1 of length M");
        }
        bias = static_cast<const float*>(inputs[2].data);
    }
    if (x.data == nullptr || w.data == nullptr || out.data == nullptr || (has_bias && bias == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    nert_conv_desc d{};
    d.batch = batch;
    d.in_channels = in_channels;
    d.out_channels = out_channels;
    d.group = group;
    const size_t lift = 3 - spatial;
    for (size_t i = 0; i < 3; ++i) {
        const bool real = i >= lift;
        const size_t s = real ? i - lift : 0;
        d.in[i] = real ? in_spatial[s] : 1;
        d.kernel[i] = real ? kernel[s] : 1;
        d.out[i] = real ? expected[2 + s] : 1;
        d.stride[i] = real ? strides[s] : 1;
        d.dilation[i] = real ? dilations[s] : 1;
        d.pad[i] = real ? pad_begin[s] : 0;
    }
    const float* res = nullptr;
    if (residual != nullptr) {
        if (residual->dtype != DataType::Float32 || residual->dims != out.dims) {
            throw InferenceException(context + ": the summed input must be float32 with the output's shape");
        }
        if (residual->data == nullptr) {
            throw InferenceException(context + ": null buffer");
        }
        res = static_cast<const float*>(residual->data);
    }
    return ConvCall{d, bias, res};
}

void ConvCore(const Node& node, const std::string& context, const Views& inputs, bool has_bias,
              const TensorView* residual, int act, const Views& outputs) {
    const ConvCall c = CheckConv(node, context, inputs, has_bias, residual, outputs);
    CheckStatus(nert_hip_conv_fused_f32(static_cast<const float*>(inputs[0].data),
                                        static_cast<const float*>(inputs[1].data), c.bias, c.residual,
                                        static_cast<float*>(outputs[0].data), &c.d, act, Stream()),
                context);
    AfterRow(outputs, context);
}

int ActivationCode(const Node& node, const std::string& context) {
    const std::string activation = StringAttr(node, "activation", "", "FusedConv");
    if (activation == "Relu") {
        return 1;
    }
    if (activation == "Silu") {
        return 2;
    }
    if (!activation.empty()) {
        throw InferenceException(context + ": unsupported activation '" + activation + "'");
    }
    return 0;
}

// The packed copy of W (FusedConv's seventh input): W's shape and dtype,
// C/group a multiple of 8 (the order is nert_hip_conv_packed_f32's).
const float* PackedWeights(const std::string& context, const TensorView& w, const TensorView& packed,
                           const nert_conv_desc& d) {
    if (packed.dtype != DataType::Float32 || packed.dims != w.dims) {
        throw InferenceException(context + ": the packed weights must be float32 with the weight's shape");
    }
    if ((d.in_channels / d.group) % 8 != 0) {
        throw InferenceException(context + ": packed weights need C / group to be a multiple of 8");
    }
    if (packed.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    return static_cast<const float*>(packed.data);
}

// FusedConv with a paired 1x1 convolution: inputs X, W, B, Z, W2, B2 (B, Z
// and B2 may be omitted) and optionally W packed, outputs Y and Y2.
void FusedConvPair(const Node& node, const std::string& context, const Views& inputs, const Views& outputs) {
    const int act = ActivationCode(node, context);
    const bool has_bias = inputs[2].dtype != DataType::Unknown;
    const TensorView* z = inputs[3].dtype != DataType::Unknown ? &inputs[3] : nullptr;
    Views main_inputs(inputs.begin(), inputs.begin() + (has_bias ? 3 : 2));
    const ConvCall c = CheckConv(node, context, main_inputs, has_bias, z, Views{outputs[0]});
    const float* packed = inputs.size() == 7 ? PackedWeights(context, inputs[1], inputs[6], c.d) : nullptr;
    const TensorView& w2 = inputs[4];
    const TensorView& b2 = inputs[5];
    const TensorView& y2 = outputs[1];
    const nert_conv_desc& d = c.d;
    const bool pad1 = d.kernel[0] == 1 && d.kernel[1] == 3 && d.kernel[2] == 3 && d.pad[1] == 1 && d.pad[2] == 1 &&
                      d.dilation[1] == 1 && d.dilation[2] == 1 && d.group == 1;
    if (!pad1) {
        throw InferenceException(context + ": a paired conv needs a 3x3 first conv with pad 1, dilation 1, group 1");
    }
    const std::vector<int64_t> w2_dims = {d.out_channels, d.in_channels, 1, 1};
    if (w2.dtype != DataType::Float32 || w2.dims != w2_dims) {
        throw InferenceException(context + ": the paired weight must be float32 [M, C, 1, 1]");
    }
    const bool has_b2 = b2.dtype != DataType::Unknown;
    if (has_b2 && (b2.dtype != DataType::Float32 || b2.dims != std::vector<int64_t>{d.out_channels})) {
        throw InferenceException(context + ": the paired bias must be float32 [M]");
    }
    if (y2.dtype != DataType::Float32 || y2.dims != outputs[0].dims) {
        throw InferenceException(context + ": the paired output must be float32 with the first output's shape");
    }
    if (w2.data == nullptr || y2.data == nullptr || (has_b2 && b2.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    if (packed != nullptr) {
        CheckStatus(nert_hip_conv_packed_f32(static_cast<const float*>(inputs[0].data),
                                             static_cast<const float*>(inputs[1].data), packed, c.bias, c.residual,
                                             static_cast<float*>(outputs[0].data),
                                             static_cast<const float*>(w2.data),
                                             has_b2 ? static_cast<const float*>(b2.data) : nullptr,
                                             static_cast<float*>(y2.data), &d, act, Stream()),
                    context);
    } else {
        CheckStatus(nert_hip_conv_pair_f32(static_cast<const float*>(inputs[0].data),
                                           static_cast<const float*>(inputs[1].data), c.bias, c.residual,
                                           static_cast<float*>(outputs[0].data), static_cast<const float*>(w2.data),
                                           has_b2 ? static_cast<const float*>(b2.data) : nullptr,
                                           static_cast<float*>(y2.data), &d, act, Stream()),
                    context);
    }
    AfterRow(outputs, context);
}

} // namespace

// Validation follows src/kernels/conv.cpp:138-231.
void Conv(const Node& node, const Views& inputs, const Views& outputs) {
    const std::string context = "Conv (node '" + node.name + "')";
    if (inputs.size() < 2 || inputs.size() > 3 || outputs.size() != 1) {
        throw InferenceException(context + ": expected two or three inputs and one output");
    }
    ConvCore(node, context, inputs, inputs.size() == 3, nullptr, 0, outputs);
}

// Not a reference row: Y = activation(Conv(X, W, B) + Z), the contract of
// the com.microsoft FusedConv contrib op (inputs X, W, optional B, optional
// Z; attribute `activation`, here "Relu", "Silu" or absent). "Silu" is this
// layer's addition to that contract: Y * Sigmoid(Y), the Sigmoid -> Mul pair
// of SiLU/Swish blocks. The nert_amd runner rewrites Conv -> [Add] -> [Relu]
// and Conv -> Sigmoid -> Mul chains into it; every step rounds as the
// separate rows do, so results are bit-identical to the unfused graph.
//
// With six inputs (X, W, B, Z, W2, B2; B, Z and B2 may be omitted) and two
// outputs it also computes Y2 = Conv(X, W2, B2) for a 1x1 W2 at the node's
// strides with pad 0, which the runner pairs with a 3x3 pad-1 conv of the
// same input (a ResNet block's downsampling shortcut): one launch for both
// (nert_hip_conv_pair_f32). A seventh input is W again in the packed order
// of nert_hip_conv_packed_f32 (the runner packs 3x3 initializer weights
// once); without a pair, W2 and B2 are then omitted and there is one output.
void FusedConv(const Node& node, const Views& inputs, const Views& outputs) {
    const std::string context = "FusedConv (node '" + node.name + "')";
    const bool paired = (inputs.size() == 6 || (inputs.size() == 7 && inputs[4].dtype != DataType::Unknown)) &&
                        outputs.size() == 2;
    if (paired) {
        FusedConvPair(node, context, inputs, outputs);
        return;
    }
    if (inputs.size() == 7 && outputs.size() == 1 && inputs[4].dtype == DataType::Unknown &&
        inputs[5].dtype == DataType::Unknown) {
        const int act = ActivationCode(node, context);
        const bool has_bias = inputs[2].dtype != DataType::Unknown;
        const TensorView* z = inputs[3].dtype != DataType::Unknown ? &inputs[3] : nullptr;
        Views conv_inputs(inputs.begin(), inputs.begin() + (has_bias ? 3 : 2));
        const ConvCall c = CheckConv(node, context, conv_inputs, has_bias, z, outputs);
        const float* packed = PackedWeights(context, inputs[1], inputs[6], c.d);
        CheckStatus(nert_hip_conv_packed_f32(static_cast<const float*>(inputs[0].data),
                                             static_cast<const float*>(inputs[1].data), packed, c.bias, c.residual,
                                             static_cast<float*>(outputs[0].data), nullptr, nullptr, nullptr, &c.d,
                                             act, Stream()),
                    context);
        AfterRow(outputs, context);
        return;
    }
    if (inputs.size() < 2 || inputs.size() > 4 || outputs.size() != 1) {
        throw InferenceException(context + ": expected two to four inputs and one output");
    }
    const int act = ActivationCode(node, context);
    const bool has_bias = inputs.size() >= 3 && inputs[2].dtype != DataType::Unknown;
    const TensorView* z = inputs.size() == 4 && inputs[3].dtype != DataType::Unknown ? &inputs[3] : nullptr;
    Views conv_inputs(inputs.begin(), inputs.begin() + (has_bias ? 3 : 2));
    ConvCore(node, context, conv_inputs, has_bias, z, act, outputs);
}

} // namespace rows
} // namespace nert_hip
