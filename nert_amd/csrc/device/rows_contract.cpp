// Resampling and contraction rows: Resize, GridSample, Einsum,
// ConvTranspose. Validation mirrors src/kernels/{resize,grid_sample,einsum,
// conv_transpose}.cpp; the Einsum equation front end (ellipsis expansion,
// implicit output, label binding) restates src/kernels/einsum.cpp:24-258
// and its nert::einsum helpers (:291-492) so that the same equations resolve to the
// same labels, sizes, strides and messages.

#include "rows.hpp"

#include <algorithm>
#include <cmath>
#include <map>

namespace nert_hip {
namespace rows {

using namespace seam;

// ---- Resize -----------------------------------------------------------------

// src/kernels/resize.cpp:162-255
NERT_HIP_ROW(Resize) {
    const std::string context = "Resize (node '" + node.name + "')";
    if (inputs.empty() || inputs.size() > 4 || outputs.size() != 1) {
        throw InferenceException(context + ": expected an input, roi, scales, and an optional sizes input");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    const std::string mode = StringAttr(node, "mode", "nearest", "Resize");
    if (mode != "nearest" && mode != "linear") {
        throw InferenceException(context + ": Resize 'mode' must be 'nearest' or 'linear' here");
    }
    const bool linear = mode == "linear";
    if (in.dtype != DataType::Float32 && !(in.dtype == DataType::Int64 && !linear)) {
        throw InferenceException(context + ": tensors must be float32 (or int64 for nearest)");
    }
    if (out.dtype != in.dtype) {
        throw InferenceException(context + ": output dtype must match the input dtype");
    }
    const std::string transform = StringAttr(node, "coordinate_transformation_mode", "half_pixel", "Resize");
    const std::string nearest = StringAttr(node, "nearest_mode", "round_prefer_floor", "Resize");
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    std::vector<double> scales(static_cast<size_t>(rank), 1.0);
    const bool has_scales =
        inputs.size() > 2 && inputs[2].dtype != DataType::Unknown && CountNonNeg(inputs[2].dims, context) > 0;
    const bool has_sizes = inputs.size() > 3 && inputs[3].dtype != DataType::Unknown;
    if (has_sizes && has_scales) {
        throw InferenceException(context + ": Resize takes exactly one of scales and sizes");
    }
    if (has_sizes) {
        const TensorView& sizes_view = inputs[3];
        if (sizes_view.dtype != DataType::Int64 || CountNonNeg(sizes_view.dims, context) != rank ||
            sizes_view.data == nullptr) {
            throw InferenceException(context + ": Resize sizes must be int64 with one entry per input axis");
        }
        const std::vector<int64_t> sizes = ReadInt64(sizes_view, rank, context);
        for (int64_t i = 0; i < rank; ++i) {
            const size_t u = static_cast<size_t>(i);
            if (out.dims.size() != static_cast<size_t>(rank) || out.dims[u] != sizes[u]) {
                throw InferenceException(context + ": output shape does not match the sizes input");
            }
            scales[u] = static_cast<double>(static_cast<float>(sizes[u]) / static_cast<float>(in.dims[u]));
        }
    } else {
        if (!has_scales || inputs[2].dtype != DataType::Float32) {
            throw InferenceException(context + ": Resize requires a scales or sizes input");
        }
        const TensorView& scales_view = inputs[2];
        if (CountNonNeg(scales_view.dims, context) != rank) {
            throw InferenceException(context + ": Resize scales rank must match the input rank");
        }
        if (scales_view.data == nullptr) {
            throw InferenceException(context + ": null scales buffer");
        }
        const std::vector<float> fs = ReadFloat(scales_view, rank, context);
        std::vector<int64_t> expected(static_cast<size_t>(rank), 0);
        for (int64_t i = 0; i < rank; ++i) {
            const size_t u = static_cast<size_t>(i);
            const int64_t dim =
                static_cast<int64_t>(std::floor(static_cast<double>(in.dims[u]) * static_cast<double>(fs[u])));
            if (dim <= 0) {
                throw InferenceException(context + ": Resize produces a non-positive output dim");
            }
            expected[u] = dim;
            scales[u] = static_cast<double>(fs[u]);
        }
        if (out.dims != expected) {
            throw InferenceException(context + ": output shape does not match the scaled input");
        }
    }
    const int64_t out_count = CountNonNeg(out.dims, context);
    (void)CountNonNeg(in.dims, context);
    if (out_count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    // The reference resolves the modes while building its per-axis tables,
    // i.e. only when some axis has output positions (resize.cpp:87-93).
    bool any_positions = false;
    for (const int64_t d : out.dims) {
        any_positions = any_positions || d > 0;
    }
    int transform_code = NERT_RESIZE_HALF_PIXEL;
    int nearest_code = NERT_RESIZE_ROUND_PREFER_FLOOR;
    if (any_positions) {
        if (transform == "half_pixel") {
            transform_code = NERT_RESIZE_HALF_PIXEL;
        } else if (transform == "pytorch_half_pixel") {
            transform_code = NERT_RESIZE_PYTORCH_HALF_PIXEL;
        } else if (transform == "align_corners") {
            transform_code = NERT_RESIZE_ALIGN_CORNERS;
        } else if (transform == "asymmetric") {
            transform_code = NERT_RESIZE_ASYMMETRIC;
        } else {
            throw InferenceException(context + ": unsupported coordinate_transformation_mode '" + transform + "'");
        }
        if (!linear) {
            if (nearest == "round_prefer_floor") {
                nearest_code = NERT_RESIZE_ROUND_PREFER_FLOOR;
            } else if (nearest == "round_prefer_ceil") {
                nearest_code = NERT_RESIZE_ROUND_PREFER_CEIL;
            } else if (nearest == "floor") {
                nearest_code = NERT_RESIZE_FLOOR;
            } else if (nearest == "ceil") {
                nearest_code = NERT_RESIZE_CEIL;
            } else {
                throw InferenceException(context + ": unsupported nearest_mode '" + nearest + "'");
            }
        }
    }
    if (out_count > 0) {
        CheckStatus(nert_hip_resize(DtypeCode(in.dtype), in.data, out.data, static_cast<int>(rank), in.dims.data(),
                                    out.dims.data(), scales.data(), linear ? 1 : 0, transform_code, nearest_code,
                                    Stream()),
                    context);
    }
    AfterRow(outputs, context);
}

// ---- GridSample -------------------------------------------------------------

// src/kernels/grid_sample.cpp:77-160
NERT_HIP_ROW(GridSample) {
    const std::string context = "GridSample (node '" + node.name + "')";
    if (inputs.size() != 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected two inputs and one output");
    }
    const std::string mode = StringAttr(node, "mode", "bilinear", "GridSample");
    const std::string padding = StringAttr(node, "padding_mode", "zeros", "GridSample");
    int64_t align = 0;
    if (const Attribute* attr = FindAttr(node, "align_corners")) {
        const int64_t* v = std::get_if<int64_t>(&attr->value);
        if (v == nullptr) {
            throw InferenceException("GridSample: attribute 'align_corners' must be an int (node '" + node.name +
                                     "')");
        }
        align = *v;
    }
    if (mode != "bilinear" && mode != "nearest") {
        throw InferenceException(context + ": unsupported mode '" + mode + "'");
    }
    if (padding != "zeros" && padding != "border" && padding != "reflection") {
        throw InferenceException(context + ": unsupported padding_mode '" + padding + "'");
    }
    if (align != 0 && align != 1) {
        throw InferenceException(context + ": align_corners must be 0 or 1");
    }
    const TensorView& x = inputs[0];
    const TensorView& grid = inputs[1];
    const TensorView& out = outputs[0];
    if (x.dtype != DataType::Float32 || grid.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (x.dims.size() != 4 || grid.dims.size() != 4 || grid.dims[3] != 2) {
        throw InferenceException(context + ": expected X [N,C,H,W] and grid [N,Ho,Wo,2]");
    }
    const int64_t n = x.dims[0];
    const int64_t c = x.dims[1];
    const int64_t h = x.dims[2];
    const int64_t w = x.dims[3];
    const int64_t ho = grid.dims[1];
    const int64_t wo = grid.dims[2];
    if (grid.dims[0] != n) {
        throw InferenceException(context + ": batch sizes of X and grid differ");
    }
    if (out.dims != std::vector<int64_t>({n, c, ho, wo})) {
        throw InferenceException(context + ": output shape does not match the operands");
    }
    if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || ho <= 0 || wo <= 0) {
        throw InferenceException(context + ": non-positive dimension");
    }
    if (x.data == nullptr || grid.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    const int pad_code =
        padding == "zeros" ? NERT_GRID_ZEROS : (padding == "border" ? NERT_GRID_BORDER : NERT_GRID_REFLECTION);
    CheckStatus(nert_hip_grid_sample_f32(static_cast<const float*>(x.data), static_cast<const float*>(grid.data),
                                         static_cast<float*>(out.data), n, c, h, w, ho, wo, mode == "nearest" ? 1 : 0,
                                         pad_code, static_cast<int>(align), Stream()),
                context);
    AfterRow(outputs, context);
}

// ---- Einsum -------------------------------------------------------------------

namespace {

bool IsLabel(char c) { return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z'); }

std::vector<std::string> SplitOperands(const std::string& lhs) {
    std::vector<std::string> subs;
    size_t start = 0;
    while (true) {
        const size_t comma = lhs.find(',', start);
        subs.push_back(lhs.substr(start, comma == std::string::npos ? std::string::npos : comma - start));
        if (comma == std::string::npos) {
            return subs;
        }
        start = comma + 1;
    }
}

// One subscript around its "...": false when the dots are not exactly one
// "..." group (nert::einsum SplitEllipsis, src/kernels/einsum.cpp:291-315).
bool SplitDots(const std::string& sub, std::string& left, std::string& right, bool& has) {
    has = false;
    left.clear();
    right.clear();
    size_t i = 0;
    while (i < sub.size() && sub[i] != '.') {
        left.push_back(sub[i++]);
    }
    if (i < sub.size()) {
        if (sub.compare(i, 3, "...") != 0) {
            return false;
        }
        has = true;
        i += 3;
        while (i < sub.size() && sub[i] != '.') {
            right.push_back(sub[i++]);
        }
        if (i < sub.size()) {
            return false;
        }
    }
    return true;
}

// An equation with every "..." replaced by fresh labels.
struct Expanded {
    std::string error;
    std::vector<std::string> inputs;
    std::string output;
    std::vector<char> fresh;
    std::vector<size_t> pads;
    std::vector<size_t> lefts;
    size_t width = 0;
};

// nert::einsum::EllipsisSyntaxError + ExpandEllipsis (src/kernels/einsum.cpp:317-459).
Expanded ExpandDots(const std::string& text, const std::vector<size_t>& ranks) {
    Expanded r;
    const size_t arrow = text.find("->");
    const std::string lhs = arrow == std::string::npos ? text : text.substr(0, arrow);
    const std::vector<std::string> subs = SplitOperands(lhs);
    std::vector<std::string> checked = subs;
    if (arrow != std::string::npos) {
        checked.push_back(text.substr(arrow + 2));
    }
    for (const std::string& sub : checked) {
        std::string left, right;
        bool has = false;
        if (!SplitDots(sub, left, right, has)) {
            r.error = "dots must form exactly one '...' per subscript";
            return r;
        }
        for (char c : left + right) {
            if (!IsLabel(c)) {
                r.error = "invalid character in the equation";
                return r;
            }
        }
    }
    if (subs.size() != ranks.size()) {
        r.error = "operand count does not match the equation";
        return r;
    }
    bool used[256] = {false};
    for (char c : text) {
        if (IsLabel(c)) {
            used[static_cast<unsigned char>(c)] = true;
        }
    }
    std::vector<std::string> lefts, rights;
    std::vector<size_t> counts;
    for (size_t i = 0; i < subs.size(); ++i) {
        std::string left, right;
        bool has = false;
        SplitDots(subs[i], left, right, has);
        if (ranks[i] < left.size() + right.size()) {
            r.error = "operand rank is smaller than its explicit labels";
            return r;
        }
        if (!has && ranks[i] != left.size() + right.size()) {
            r.error = "operand rank does not match its subscript";
            return r;
        }
        const size_t count = has ? ranks[i] - left.size() - right.size() : 0;
        r.width = std::max(r.width, count);
        lefts.push_back(left);
        rights.push_back(right);
        counts.push_back(count);
    }
    std::string pool;
    for (char c = 'a'; c <= 'z'; ++c) {
        if (!used[static_cast<unsigned char>(c)]) {
            pool.push_back(c);
        }
    }
    for (char c = 'A'; c <= 'Z'; ++c) {
        if (!used[static_cast<unsigned char>(c)]) {
            pool.push_back(c);
        }
    }
    if (pool.size() < r.width) {
        r.error = "equation leaves no fresh labels for the ellipsis";
        return r;
    }
    const std::string fresh = pool.substr(0, r.width);
    r.fresh.assign(fresh.begin(), fresh.end());
    for (size_t i = 0; i < subs.size(); ++i) {
        r.pads.push_back(r.width - counts[i]);
        r.lefts.push_back(lefts[i].size());
        r.inputs.push_back(lefts[i] + fresh + rights[i]);
    }
    if (arrow != std::string::npos) {
        std::string left, right;
        bool has = false;
        SplitDots(text.substr(arrow + 2), left, right, has);
        r.output = left + (has ? fresh : "") + right;
    } else {
        r.output = fresh;
    }
    return r;
}

struct Mapped {
    char label;
    int64_t dim;
    bool virtual_pad;
};

// nert::einsum::MapOperand (src/kernels/einsum.cpp:461-492).
bool MapDims(const std::string& sub, size_t left, size_t pad, size_t width, const std::vector<int64_t>& dims,
             std::vector<Mapped>& mapped) {
    mapped.clear();
    size_t d = 0;
    for (size_t q = 0; q < left && q < sub.size(); ++q) {
        if (d >= dims.size()) {
            return false;
        }
        mapped.push_back(Mapped{sub[q], dims[d++], false});
    }
    for (size_t p = 0; p < width; ++p) {
        const size_t q = left + p;
        if (q >= sub.size()) {
            return false;
        }
        if (p < pad) {
            mapped.push_back(Mapped{sub[q], 1, true});
        } else {
            if (d >= dims.size()) {
                return false;
            }
            mapped.push_back(Mapped{sub[q], dims[d++], false});
        }
    }
    for (size_t q = left + width; q < sub.size(); ++q) {
        if (d >= dims.size()) {
            return false;
        }
        mapped.push_back(Mapped{sub[q], dims[d++], false});
    }
    return d == dims.size();
}

} // namespace

// src/kernels/einsum.cpp:36-132 (equation), 134-258 (row)
NERT_HIP_ROW(Einsum) {
    const std::string context = "Einsum (node '" + node.name + "')";
    const Attribute* attr = nullptr;
    for (const Attribute& a : node.attributes) {
        if (a.name == "equation") {
            attr = &a;
        }
    }
    if (attr == nullptr) {
        throw InferenceException(context + ": missing 'equation' attribute");
    }
    const std::string* raw = std::get_if<std::string>(&attr->value);
    if (raw == nullptr) {
        throw InferenceException(context + ": attribute 'equation' must be a string");
    }
    std::string text;
    for (char c : *raw) {
        if (c != ' ') {
            text.push_back(c);
        }
    }
    std::string eq_text = text;
    std::vector<char> fresh;
    std::vector<size_t> pads, lefts;
    size_t width = 0;
    if (text.find('.') != std::string::npos) {
        if (text.find("->") == std::string::npos) {
            throw InferenceException(context + ": implicit output with ellipsis is not supported");
        }
        std::vector<size_t> ranks;
        for (const TensorView& in : inputs) {
            ranks.push_back(in.dims.size());
        }
        const Expanded ex = ExpandDots(text, ranks);
        if (!ex.error.empty()) {
            throw InferenceException(context + ": " + ex.error);
        }
        eq_text.clear();
        for (size_t i = 0; i < ex.inputs.size(); ++i) {
            if (i != 0) {
                eq_text.push_back(',');
            }
            eq_text += ex.inputs[i];
        }
        eq_text += "->" + ex.output;
        fresh = ex.fresh;
        pads = ex.pads;
        lefts = ex.lefts;
        width = ex.width;
    }
    const size_t arrow = eq_text.find("->");
    const bool explicit_output = arrow != std::string::npos;
    const std::vector<std::string> subs = SplitOperands(explicit_output ? eq_text.substr(0, arrow) : eq_text);
    std::map<char, int> counts;
    for (const std::string& sub : subs) {
        for (char c : sub) {
            if (!IsLabel(c)) {
                throw InferenceException(context + ": invalid character in the equation");
            }
            ++counts[c];
        }
    }
    std::string output;
    if (explicit_output) {
        output = eq_text.substr(arrow + 2);
        for (size_t i = 0; i < output.size(); ++i) {
            if (counts.find(output[i]) == counts.end()) {
                throw InferenceException(context + ": output label does not appear in the inputs");
            }
            if (output.find(output[i]) != i) {
                throw InferenceException(context + ": output label repeated");
            }
        }
    } else {
        for (const auto& entry : counts) {
            if (entry.second == 1) {
                output.push_back(entry.first);
            }
        }
    }
    if (subs.size() != inputs.size() || inputs.empty() || inputs.size() > 2 || outputs.size() != 1) {
        throw InferenceException(context + ": operand count does not match the equation");
    }
    const TensorView& out = outputs[0];
    if (out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    auto is_fresh = [&](char c) { return std::find(fresh.begin(), fresh.end(), c) != fresh.end(); };
    std::vector<std::vector<Mapped>> mapped(inputs.size());
    std::map<char, int64_t> sizes;
    for (size_t i = 0; i < inputs.size(); ++i) {
        if (inputs[i].dtype != DataType::Float32) {
            throw InferenceException(context + ": tensors must be float32");
        }
        if (inputs[i].data == nullptr) {
            throw InferenceException(context + ": null buffer");
        }
        const size_t left = i < lefts.size() ? lefts[i] : subs[i].size();
        const size_t pad = i < pads.size() ? pads[i] : 0;
        if (!MapDims(subs[i], left, pad, width, inputs[i].dims, mapped[i])) {
            throw InferenceException(context + ": operand rank does not match its subscript");
        }
        for (const Mapped& entry : mapped[i]) {
            if (entry.virtual_pad) {
                sizes.emplace(entry.label, 1);
                continue;
            }
            if (entry.dim <= 0) {
                throw InferenceException(context + ": non-positive dimension");
            }
            const auto inserted = sizes.emplace(entry.label, entry.dim);
            if (!inserted.second && inserted.first->second != entry.dim) {
                if (!is_fresh(entry.label) || (inserted.first->second != 1 && entry.dim != 1)) {
                    throw InferenceException(context + ": label bound to two different sizes");
                }
                inserted.first->second = std::max(inserted.first->second, entry.dim);
            }
        }
    }
    std::vector<int64_t> expected;
    for (char c : output) {
        expected.push_back(sizes.at(c));
    }
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the operands");
    }
    if (out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    // Per-label strides of each operand; repeated labels (diagonals) add up,
    // broadcast ellipsis planes contribute none.
    std::map<char, int64_t> stride_a, stride_b;
    for (size_t i = 0; i < inputs.size(); ++i) {
        std::map<char, int64_t>& st = i == 0 ? stride_a : stride_b;
        int64_t stride = 1;
        for (size_t k = mapped[i].size(); k-- > 0;) {
            const Mapped& entry = mapped[i][k];
            if (entry.virtual_pad || entry.dim != sizes.at(entry.label)) {
                if (!entry.virtual_pad && (!is_fresh(entry.label) || entry.dim != 1)) {
                    throw InferenceException(context + ": broadcast diagonal is not supported");
                }
            } else {
                st[entry.label] += stride;
            }
            stride *= entry.dim;
        }
    }
    auto at = [](const std::map<char, int64_t>& m, char c) {
        const auto it = m.find(c);
        return it == m.end() ? int64_t{0} : it->second;
    };
    std::vector<int64_t> out_size, out_sa, out_sb, sum_size, sum_sa, sum_sb;
    for (char c : output) {
        out_size.push_back(sizes.at(c));
        out_sa.push_back(at(stride_a, c));
        out_sb.push_back(at(stride_b, c));
    }
    for (const auto& entry : sizes) { // alphabetical, as the reference odometer
        if (output.find(entry.first) == std::string::npos) {
            sum_size.push_back(entry.second);
            sum_sa.push_back(at(stride_a, entry.first));
            sum_sb.push_back(at(stride_b, entry.first));
        }
    }
    if (out_size.size() > 16 || sum_size.size() > 16) {
        throw InferenceException(context + ": more than 16 output or summed labels");
    }
    CheckStatus(nert_hip_einsum_f32(static_cast<const float*>(inputs[0].data),
                                    inputs.size() == 2 ? static_cast<const float*>(inputs[1].data) : nullptr,
                                    static_cast<float*>(out.data), static_cast<int>(out_size.size()), out_size.data(),
                                    out_sa.data(), out_sb.data(), static_cast<int>(sum_size.size()), sum_size.data(),
                                    sum_sa.data(), sum_sb.data(), Stream()),
                context);
    AfterRow(outputs, context);
}

// ---- ConvTranspose ------------------------------------------------------------

// src/kernels/conv_transpose.cpp:76-158
NERT_HIP_ROW(ConvTranspose) {
    const std::string context = "ConvTranspose (node '" + node.name + "')";
    if (inputs.size() < 2 || inputs.size() > 3 || outputs.size() != 1) {
        throw InferenceException(context + ": expected input, weight, optional bias, and one output");
    }
    const TensorView& x = inputs[0];
    const TensorView& w = inputs[1];
    const TensorView* bias = inputs.size() == 3 && inputs[2].data != nullptr ? &inputs[2] : nullptr;
    const TensorView& out = outputs[0];
    if (x.dtype != DataType::Float32 || w.dtype != DataType::Float32 || out.dtype != DataType::Float32 ||
        (bias != nullptr && bias->dtype != DataType::Float32)) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (x.dims.size() != 4 || w.dims.size() != 4) {
        throw InferenceException(context + ": input and weight must be rank 4 (NCHW)");
    }
    (void)ElementCount(x.dims, context);
    (void)ElementCount(w.dims, context);
    (void)ElementCount(out.dims, context);
    const int64_t group = IntAttr(node, "group", 1, "ConvTranspose");
    const int64_t in_c = x.dims[1];
    if (group <= 0 || in_c % group != 0 || w.dims[0] != in_c) {
        throw InferenceException(context + ": weight channels do not match the input and group");
    }
    const int64_t out_c = w.dims[1] * group;
    std::vector<int64_t> strides = IntsAttr(node, "strides", "ConvTranspose");
    std::vector<int64_t> dilations = IntsAttr(node, "dilations", "ConvTranspose");
    std::vector<int64_t> out_pad = IntsAttr(node, "output_padding", "ConvTranspose");
    std::vector<int64_t> pads = IntsAttr(node, "pads", "ConvTranspose");
    if (strides.empty()) {
        strides = {1, 1};
    }
    if (dilations.empty()) {
        dilations = {1, 1};
    }
    if (out_pad.empty()) {
        out_pad = {0, 0};
    }
    if (pads.empty() || StringAttr(node, "auto_pad", "NOTSET", "ConvTranspose") == "VALID") {
        pads = {0, 0, 0, 0};
    }
    if (strides.size() != 2 || dilations.size() != 2 || out_pad.size() != 2 || pads.size() != 4) {
        throw InferenceException(context + ": strides, dilations, output_padding, and pads must be 2-D");
    }
    const int64_t k_h = w.dims[2];
    const int64_t k_w = w.dims[3];
    const int64_t out_h = strides[0] * (x.dims[2] - 1) + out_pad[0] + dilations[0] * (k_h - 1) + 1 - pads[0] - pads[2];
    const int64_t out_w = strides[1] * (x.dims[3] - 1) + out_pad[1] + dilations[1] * (k_w - 1) + 1 - pads[1] - pads[3];
    if (out.dims != std::vector<int64_t>{x.dims[0], out_c, out_h, out_w}) {
        throw InferenceException(context + ": output shape does not match the transposed window");
    }
    if (bias != nullptr && (bias->dims.size() != 1 || bias->dims[0] != out_c)) {
        throw InferenceException(context + ": bias must be rank-1 of length M");
    }
    if (x.data == nullptr || w.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    if (strides[0] <= 0 || strides[1] <= 0) {
        // The gather form needs a positive stride; the reference's scatter
        // would fold every input pixel onto one row.
        throw InferenceException(context + ": strides must be positive");
    }
    const int64_t geom[16] = {x.dims[0], in_c,       out_c,      group,      x.dims[2],    x.dims[3],
                              out_h,     out_w,      k_h,        k_w,        strides[0],   strides[1],
                              pads[0],   pads[1],    dilations[0], dilations[1]};
    CheckStatus(nert_hip_conv_transpose_f32(static_cast<const float*>(x.data), static_cast<const float*>(w.data),
                                            bias != nullptr ? static_cast<const float*>(bias->data) : nullptr,
                                            static_cast<float*>(out.data), geom, Stream()),
                context);
    AfterRow(outputs, context);
}

} // namespace rows
} // namespace nert_hip
